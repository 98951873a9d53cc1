"""FakeQuantize modules on MI355X kernels
(src/voyager_compiler/quantization/fake_quantize.py:101-495).

Same constructor arguments, buffers and state_dict behaviour as the
reference's ``FusedAmaxObsFakeQuantize``; the arithmetic runs in the HIP
kernels:

* per-tensor / per-channel / no qscheme: with the observer on, the device
  observer (``vqx_amax_observe_fake_quant``: scales from the amax history,
  then one pass that fake-quantizes and folds the input's amax into the
  history); otherwise the closed-form fake-quant kernel
  (``quantized_ops.fake_quant``), or the table path when ``qmap`` has been
  replaced or edited in place (as codebook fitting does);
* microscaling: one fused pass that computes the block scales, quantizes and
  multiplies back (``mx_fake_quantize``);
* group-wise affine: one fused pass over each block's min / max, scale, zero
  point and the affine fake-quant (``gwa_fake_quantize``).

Outliers (``outlier_pct`` / ``outlier_threshold``, fake_quantize.py:373-395)
stay on the device: the share's threshold and its running average come from
a radix select over |x| (``vqx_outlier_topk_threshold``); microscaling masks,
fake-quantizes, restores and counts in one pass
(``vqx_mx_fake_quant_outlier``); the other schemes run between a mask and a
restore pass.  The largest outlier fraction is kept on the device and read
when ``max_outlier_pct`` is.

Every autograd function passes gradients straight through to the input.
"""

import logging
from typing import Optional

import torch
from torch.ao.quantization import FakeQuantizeBase

from .. import _lib
from ..formats import get_quantization_map, parse_format
from ..ops import quantized as qops
from .qspec import QScheme

__all__ = [
    "FakeQuantizeFunction",
    "MXFakeQuantizeFunction",
    "GroupWiseAffineFakeQuantFunction",
    "ObservedFakeQuantizeFunction",
    "OutlierFakeQuantizeFunction",
    "FusedAmaxObsFakeQuantize",
    "_DerivedObserverOrFakeQuantize",
    "get_quantization_map",
]

logger = logging.getLogger(__name__)


def _per_tensor_fake_quant(x, qmap, scale, fmt):
    """vmap(x / s, qmap) * s with s = scale.to(x.dtype) (fake_quantize.py:114-115)."""
    if fmt is not None:
        y, _ = torch.ops.quantized_ops.fake_quant(x, fmt.dtype, scale, True, False)
        return y
    s = scale.to(device=x.device, dtype=x.dtype)
    desc, keep = qops._table_desc(qmap.to(x.device), x.device)
    xc = x.contiguous()
    m = qops._scale_map(xc, s.contiguous(), None, None)
    if m is None:
        s = s.expand(xc.shape).contiguous()
        m = _lib.VqxScaleMap(s.data_ptr(), None, xc.numel(), 1, 1, 0, 1, 0)
    y = torch.empty_like(xc)
    _lib.call("vqx_quantize_mapped", _lib.ptr(xc), _lib.dtype_tag(xc.dtype), xc.numel(),
              _lib.ctypes.byref(desc), _lib.ctypes.byref(m), 1, _lib.ptr(y), None, 0, _lib.stream_of(xc))
    del keep
    return y


class FakeQuantizeFunction(torch.autograd.Function):
    """Quantizes against an observed scale; straight-through gradient."""

    @staticmethod
    def forward(ctx, input, fake_quant_enabled, qmap, scale, fmt=None):
        if not fake_quant_enabled:
            return input
        return _per_tensor_fake_quant(input, qmap, scale, fmt)

    @staticmethod
    def backward(ctx, grad_output):
        return (grad_output,) + (None,) * 4


def _direct_scale(scale, input, axis, block_size):
    """The scale buffer resized to the block-scale shape, when the kernel can
    write it in place (fp32, on the input's device), else None."""
    if scale.dtype != torch.float32 or scale.device != input.device:
        return None
    shape = qops.mx_scale_shape(input.shape, axis, block_size)
    if list(scale.shape) != shape:
        scale.resize_(shape)
    return scale if scale.is_contiguous() else None


def _run(fn, x, *args):
    """fn.apply(x, *args), or fn's forward alone when no gradient can flow
    through it (grad mode off, or x not requiring one): the same output
    without an autograd node and without apply's per-call host cost.  The
    forwards here use no ctx."""
    if torch.is_grad_enabled() and x.requires_grad:
        return fn.apply(x, *args)
    return fn.forward(None, x, *args)


class MXFakeQuantizeFunction(torch.autograd.Function):
    """Microscaling fake-quant: block scales from the block amax, quantize,
    multiply back, all in one kernel pass; straight-through gradient."""

    @staticmethod
    def forward(ctx, input, fake_quant_enabled, scale, qmap, axes, block_size, quant_max,
                force_scale_power_of_two=False, scale_qmap=None, fmt=None):
        if not fake_quant_enabled:
            return input
        axis = qops._single_axis(axes)
        # scale.resize_(sf.shape).copy_(sf) (:152): an fp32 buffer on the
        # input's device takes the kernel's fp32 scale output directly
        direct = _direct_scale(scale, input, axis, block_size)
        if fmt is not None:
            sf, y = qops.mx_fake_quantize(input, fmt, axis, block_size, quant_max,
                                          force_scale_power_of_two, scale_qmap, scale_f32=direct)
        else:
            desc, keep = qops._table_desc(qmap.to(input.device), input.device)
            sf, _, y = qops._mx_call(input, axis, block_size, quant_max, force_scale_power_of_two,
                                     scale_qmap, desc, want_scale=direct is None, want_fq=True, scale_f32=direct)
            sf = direct if direct is not None else sf
            del keep
        if direct is None:
            scale.resize_(sf.shape).copy_(sf)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        return (grad_output,) + (None,) * 9


class ObservedFakeQuantizeFunction(torch.autograd.Function):
    """The observer step of a per-tensor / per-channel FusedAmaxObsFakeQuantize
    followed by FakeQuantizeFunction (fake_quantize.py:418-426), fused into
    one pass over the input on the device; straight-through gradient."""

    @staticmethod
    def forward(ctx, input, fake_quant_enabled, module, fmt=None):
        y = module._observe_fake_quant(input, fake_quant_enabled, fmt)
        return input if y is None else y

    @staticmethod
    def backward(ctx, grad_output):
        return (grad_output,) + (None,) * 3


class GroupWiseAffineFakeQuantFunction(torch.autograd.Function):
    """Group-wise affine fake-quant (fake_quantize.py:162-216): per block of
    block_size along the axis, scale and zero point from the block min / max,
    then (clamp(round(x / sf + zp)) - zp) * sf; scale and zero_point are
    written into the given buffers; straight-through gradient."""

    @staticmethod
    def forward(ctx, input, fake_quant_enabled, scale, zero_point, axes, block_size, quant_min, quant_max,
                scale_qmap=None):
        if not fake_quant_enabled:
            return input
        assert block_size > 0
        axis = qops._single_axis(axes)
        sf, zp, y = qops.gwa_fake_quantize(input, axis, block_size, quant_min, quant_max, scale_qmap)
        scale.resize_(sf.shape).copy_(sf)
        zero_point.resize_(zp.shape).copy_(zp)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        return (grad_output,) + (None,) * 8


class OutlierFakeQuantizeFunction(torch.autograd.Function):
    """FusedAmaxObsFakeQuantize.forward with outliers (fake_quantize.py:
    388-432): the outliers are masked out, the rest fake-quantized by the
    module's scheme, the outliers put back; the whole composite passes the
    gradient straight through (masked_fill's and where's gradients add up to
    the identity around the straight-through fake-quant)."""

    @staticmethod
    def forward(ctx, input, module, fake_quant_enabled, fmt=None):
        return module._outlier_forward(input, fake_quant_enabled, fmt)

    @staticmethod
    def backward(ctx, grad_output):
        return (grad_output,) + (None,) * 3


class _BufferFlags:
    """The enable flags of a FakeQuantizeBase read as the reference reads them
    on every forward (fake_quantize.py:373, :112, :138, :422).  Their values
    are cached and re-read only when a buffer changes: its version counter
    moves with the enable_ / disable_ methods, load_state_dict and in-place
    writes such as lcq.py's fake_quant_enabled.zero_() / .copy_(), and a moved
    buffer is a new tensor.  So a forward reads the device only after a
    change.  Buffers made under torch.inference_mode have no version counter
    and can be written in place there unseen, so they are read on every
    forward, as the reference reads them."""

    def _flag(self, name):
        cache = self.__dict__.setdefault("_flag_cache", {})
        buf = getattr(self, name)
        if buf.is_inference():
            return int(buf[0].item())
        key = (id(buf), buf.data_ptr(), buf.device, buf._version)
        hit = cache.get(name)
        if hit is not None and hit[0] == key:
            return hit[1]
        v = int(buf[0].item())
        cache[name] = (key, v)
        return v

    def _observer_on(self):
        return self._flag("observer_enabled") == 1

    def _fake_quant_on(self):
        return self._flag("fake_quant_enabled") != 0


class FusedAmaxObsFakeQuantize(_BufferFlags, FakeQuantizeBase):
    """Fake-quantize with an amax-history observer (fake_quantize.py:219-463)."""

    def __init__(self, dtype: str, qscheme: Optional[QScheme] = None, quant_min=None, quant_max=None,
                 amax_history_len: int = None, ch_axis=None, block_size=None, scale_dtype=None,
                 force_scale_power_of_two: bool = False, record_histogram: bool = False,
                 outlier_threshold: Optional[float] = None, outlier_pct: Optional[float] = None,
                 device=None, **kwargs):
        super().__init__()
        self.dtype = dtype
        self.qscheme = qscheme
        self.quant_min = quant_min
        self.quant_max = quant_max
        self.amax_history_len = amax_history_len
        self.ch_axis = ch_axis
        self.block_size = block_size
        self.scale_dtype = scale_dtype
        self.force_scale_power_of_two = force_scale_power_of_two
        self.record_histogram = record_histogram
        self.outlier_pct = outlier_pct
        assert outlier_pct is None or outlier_threshold is None, (
            "Only one of outlier_pct and outlier_threshold can be set.")
        self._fmt = parse_format(dtype)
        self.is_codebook_quantization = self._fmt.is_levels
        self._scale_fmt = parse_format(scale_dtype) if scale_dtype is not None else None

        fk = {"device": device, "dtype": torch.float}
        self.register_buffer("qmap", self._build_qmap(device), persistent=False)
        self.register_buffer("scale_qmap", self._build_scale_qmap(device), persistent=False)
        self.register_buffer("amax_history", torch.tensor([], **fk))
        self.register_buffer("scale", torch.tensor([1.0], **fk))
        self.register_buffer("zero_point", torch.tensor([1.0], **fk))
        if record_histogram:
            self.register_buffer("histogram", torch.zeros(254, **fk), persistent=False)
        self.observer_enabled[0] = self.qscheme is not None
        self._max_outlier_host = 0.0
        self._outlier_stats = None
        self._outlier_parity = 0
        self._topk_ws = None
        self.is_per_channel = self.qscheme == QScheme.PER_CHANNEL_SYMMETRIC
        if outlier_pct is not None:
            self.outlier_ema_decay = kwargs.get("outlier_ema_decay", 0.9)
            self.register_buffer("outlier_threshold", torch.tensor([], **fk))
        else:
            self.outlier_threshold = outlier_threshold

    # -- tables -------------------------------------------------------------
    @staticmethod
    def _gpu_ok(device):
        if device is not None and torch.device(device).type == "cuda":
            return True
        return torch.cuda.is_available()

    def _build_qmap(self, device):
        """bf16 value table; built lazily on the first GPU forward when no GPU
        is visible at construction."""
        if not self._gpu_ok(device):
            self._qmap_sig = None
            return torch.empty(0, dtype=torch.bfloat16)
        q = get_quantization_map(self.dtype, device)
        if isinstance(q, tuple):
            idx, vals = q
            q = vals[idx]
        self._qmap_sig = None
        return q

    def _build_scale_qmap(self, device):
        if self.scale_dtype is None:
            return None
        if not self._gpu_ok(device):
            return torch.empty(0, dtype=torch.bfloat16)
        q = get_quantization_map(self.scale_dtype, device)
        return q[1][q[0]] if isinstance(q, tuple) else q

    def _ensure_tables(self, device):
        if self.qmap.numel() == 0:
            self.qmap = self._build_qmap(device).to(device)
        elif self.qmap.device != device:
            self.qmap = self.qmap.to(device)
        if self.scale_dtype is not None and (self.scale_qmap is None or self.scale_qmap.numel() == 0):
            self.scale_qmap = self._build_scale_qmap(device).to(device)
        if self._qmap_sig is None:
            self._qmap_sig = (self.qmap.data_ptr(), _lib.version_of(self.qmap))

    def _closed_form(self):
        """The format's closed form applies while qmap is the table it built."""
        return self._qmap_sig == (self.qmap.data_ptr(), _lib.version_of(self.qmap))

    # max_outlier_pct: the largest fraction of outliers seen so far
    # (fake_quantize.py:389-391).  The kernels keep it on the device in a
    # stats buffer (count / numel in fp64, as Python divides), each forward
    # counting into the set after the previous one's, so the forward does not
    # synchronise; the host reads it when the value is read (convert reads it).
    @property
    def max_outlier_pct(self):
        st = self._outlier_stats
        if st is None:
            return self._max_outlier_host
        return max(self._max_outlier_host, qops.outlier_stats_fraction(st, self._outlier_parity ^ 1))

    @max_outlier_pct.setter
    def max_outlier_pct(self, value):
        self._max_outlier_host = float(value)
        if self._outlier_stats is not None:
            self._outlier_stats.zero_()

    def _stats_on(self, device):
        """(stats buffer on `device`, parity of this forward's set); a move
        folds the old buffer's fraction into the host value."""
        st = self._outlier_stats
        if st is not None and st.device != device:
            self._max_outlier_host = self.max_outlier_pct
            st = None
        if st is None:
            st = qops.outlier_stats(device)
            self._outlier_stats = st
            self._outlier_parity = 0
        parity = self._outlier_parity
        self._outlier_parity ^= 1
        return st, parity

    @torch.no_grad()
    def _update_outlier_threshold(self, x):
        """The outlier_pct threshold (fake_quantize.py:373-387): the top-k
        minimum of |x|, copied into outlier_threshold on the first call and
        folded in with the running average after."""
        first = self.outlier_threshold.numel() == 0
        if first:
            self.outlier_threshold.resize_(())
        t = self.outlier_threshold
        if t.dtype != torch.float32 or t.device != x.device:
            raise RuntimeError("FusedAmaxObsFakeQuantize: outlier_threshold must be float32 on the input's device")
        if self._topk_ws is None or self._topk_ws.device != x.device:
            self._topk_ws = qops.outlier_topk_workspace(x.device)
        qops.outlier_topk_threshold_(x, self.outlier_pct, t, not first, self.outlier_ema_decay, self._topk_ws)

    @torch.no_grad()
    def _outlier_forward(self, x, fake_quant, fmt):
        """fake_quantize.py:388-432 on the device: returns the output."""
        thr = self.outlier_threshold
        stats, parity = self._stats_on(x.device)
        xc = x.contiguous()
        if self.qscheme == QScheme.MICROSCALING and x.dtype in (torch.bfloat16, torch.float32):
            if not fake_quant:  # MXFakeQuantizeFunction returns its input: only the count
                qops.outlier_mask(xc, thr, stats, parity, masked=False)
                return x
            if fmt is not None:
                desc, keep = fmt.desc(xc.device), None
            else:
                desc, keep = qops._table_desc(self.qmap.to(xc.device), xc.device)
            axis = qops._single_axis(self.ch_axis)
            direct = _direct_scale(self.scale, xc, axis, self.block_size)
            sf, y = qops.mx_fake_quantize_outlier(xc, desc, axis, self.block_size, self.quant_max,
                                                  self.force_scale_power_of_two, self.scale_qmap, thr, stats,
                                                  parity, scale_f32=direct)
            del keep
            if direct is None:
                self.scale.resize_(sf.shape).copy_(sf)
            return y
        xm = qops.outlier_mask(xc, thr, stats, parity)
        if self.qscheme == QScheme.MICROSCALING:
            y = MXFakeQuantizeFunction.forward(None, xm, fake_quant, self.scale, self.qmap, self.ch_axis,
                                               self.block_size, self.quant_max, self.force_scale_power_of_two,
                                               self.scale_qmap, fmt)
        elif self.qscheme == QScheme.GROUP_WISE_AFFINE:
            y = GroupWiseAffineFakeQuantFunction.forward(None, xm, fake_quant, self.scale, self.zero_point,
                                                         self.ch_axis, self.block_size, self.quant_min,
                                                         self.quant_max, self.scale_qmap)
        elif self._observer_on():
            y = self._observe_fake_quant(xm, fake_quant, fmt)
            y = xm if y is None else y
        else:
            y = FakeQuantizeFunction.forward(None, xm, fake_quant, self.qmap, self.scale, fmt)
        if not y.is_contiguous() or y.data_ptr() == xc.data_ptr():
            y = y.contiguous() if y.data_ptr() != xc.data_ptr() else y.clone()
        return qops.outlier_restore_(xc, thr, y).view(x.shape)

    # -- observer -----------------------------------------------------------
    def _channel_geometry(self, x):
        """(channels, inner, keepdim shape of the amax) of the observed amax:
        one value per tensor, or per index of ch_axis (fake_quantize.py:318-324)."""
        if not self.is_per_channel:
            return 1, 1, ()
        ch_axis = self.ch_axis % x.ndim
        inner = 1
        for d in x.shape[ch_axis + 1:]:
            inner *= d
        shape = tuple(x.shape[ch_axis] if i == ch_axis else 1 for i in range(x.ndim))
        return x.shape[ch_axis], inner, shape

    @torch.no_grad()
    def _observe_fake_quant(self, x, fake_quant, fmt):
        """The observer step (:308-341) and, when fake_quant, the fake-quant
        at the new scale, in two launches that read x once: returns the
        fake-quantized tensor, or None when fake_quant is off."""
        C, inner, shape = self._channel_geometry(x)
        if self.amax_history.numel() == 0:
            self.amax_history.resize_((self.amax_history_len,) + shape).fill_(0.0)
            self.scale.resize_(shape).fill_(1.0)
        if (self.amax_history.device != x.device or self.amax_history.dtype != torch.float32
                or not self.amax_history.is_contiguous() or not self.scale.is_contiguous()
                or self.scale.dtype != torch.float32 or self.scale.device != x.device):
            raise RuntimeError("FusedAmaxObsFakeQuantize: amax_history / scale must be contiguous float32 on the "
                               "input's device")
        if self.amax_history.numel() != self.amax_history.shape[0] * C or self.scale.numel() != C:
            raise RuntimeError(f"FusedAmaxObsFakeQuantize: observed {C} channel(s), but amax_history is "
                               f"{tuple(self.amax_history.shape)} and scale {tuple(self.scale.shape)}")
        xc = x.contiguous()
        y = torch.empty_like(xc) if fake_quant else None
        if fmt is not None:
            desc, keep = fmt.desc(xc.device), None
        else:
            desc, keep = qops._table_desc(self.qmap.to(xc.device), xc.device)
        _lib.call("vqx_amax_observe_fake_quant", _lib.ptr(xc), _lib.dtype_tag(xc.dtype), xc.numel(), C, inner,
                  _lib.ctypes.byref(desc), _lib.ptr(self.amax_history), self.amax_history.shape[0],
                  _lib.ptr(self.scale), _lib.ctypes.c_float(self.quant_max),
                  1 if self.force_scale_power_of_two else 0, _lib.ptr(y), _lib.stream_of(xc))
        del keep
        return y

    @torch.jit.export
    def calculate_qparams(self):
        if self.qscheme == QScheme.GROUP_WISE_AFFINE:
            return self.scale, self.zero_point
        return self.scale

    @torch.jit.export
    def extra_repr(self):
        return (f"fake_quant_enabled={self.fake_quant_enabled}, observer_enabled={self.observer_enabled}, "
                f"dtype={self.dtype}, amax_history_len={self.amax_history_len}, quant_max={self.quant_max}, "
                f"qscheme={self.qscheme}, ch_axis={self.ch_axis}, block_size={self.block_size}, "
                f"force_scale_power_of_two={self.force_scale_power_of_two}, scale={self.scale}")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _lib.require_device(x, "FusedAmaxObsFakeQuantize")
        self._ensure_tables(x.device)
        if self.record_histogram:
            exp = torch.floor(torch.log2(torch.abs(x.detach().float())))
            self.histogram += torch.histc(exp, 254, min=-126, max=127)

        if self.outlier_pct is not None and self._observer_on():
            self._update_outlier_threshold(x)

        fmt = self._fmt if self._closed_form() else None
        fq_on = self._fake_quant_on()
        if self.outlier_threshold is not None:
            return _run(OutlierFakeQuantizeFunction, x, self, fq_on, fmt)
        if self.qscheme == QScheme.MICROSCALING:
            x = _run(MXFakeQuantizeFunction, x, fq_on, self.scale, self.qmap, self.ch_axis, self.block_size,
                     self.quant_max, self.force_scale_power_of_two, self.scale_qmap, fmt)
        elif self.qscheme == QScheme.GROUP_WISE_AFFINE:
            x = _run(GroupWiseAffineFakeQuantFunction, x, fq_on, self.scale, self.zero_point, self.ch_axis,
                     self.block_size, self.quant_min, self.quant_max, self.scale_qmap)
        elif self._observer_on():
            x = _run(ObservedFakeQuantizeFunction, x, fq_on, self, fmt)
        else:
            x = _run(FakeQuantizeFunction, x, fq_on, self.qmap, self.scale, fmt)
        return x

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        # scale / zero_point / amax_history start empty or size 1 and take
        # their observed shape on the first forward; resize before the copy.
        for name in ("scale", "zero_point", "amax_history"):
            key = prefix + name
            if key in state_dict:
                getattr(self, name).resize_(state_dict[key].shape)
            elif strict:
                missing_keys.append(key)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)


class _DerivedObserverOrFakeQuantize(_BufferFlags, FakeQuantizeBase):
    """A fake-quantizer whose scale is derived from other observers
    (fake_quantize.py:466-495), e.g. a bias quantized at input scale x weight
    scale: derive_qparams_fn(obs_or_fqs) gives the scale on every forward,
    and the tensor goes through FakeQuantizeFunction at that scale (int24 and
    other integer formats up to 31 bits in closed form).  It observes
    nothing."""

    def __init__(self, dtype: str, obs_or_fqs, derive_qparams_fn):
        super().__init__()
        self.obs_or_fqs = obs_or_fqs
        self.derive_qparams_fn = derive_qparams_fn
        self.dtype = dtype
        self._fmt = parse_format(dtype)
        self.register_buffer("qmap", torch.empty(0, dtype=torch.bfloat16), persistent=False)
        self.observer_enabled[0] = 0
        self.qscheme = obs_or_fqs[1].qscheme

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _lib.require_device(x, "_DerivedObserverOrFakeQuantize")
        devices = {p.device for p in self.buffers()}
        if len(devices) != 1 or next(iter(devices)) != x.device:
            self.to(x.device)
        if self.qmap.numel() == 0:
            q = get_quantization_map(self.dtype, x.device)
            self.qmap = (q[1][q[0]] if isinstance(q, tuple) else q).to(x.device)
        return _run(FakeQuantizeFunction, x, self._fake_quant_on(), self.qmap, self.calculate_qparams(), self._fmt)

    def calculate_qparams(self):
        return self.derive_qparams_fn(self.obs_or_fqs)
