"""FakeQuantize modules on MI355X kernels
(src/voyager_compiler/quantization/fake_quantize.py:101-495).

Same constructor arguments, buffers and state_dict behaviour as the
reference's ``FusedAmaxObsFakeQuantize``; the arithmetic runs in the HIP
kernels:

* per-tensor / per-channel / no qscheme: the closed-form fake-quant kernel
  (``quantized_ops.fake_quant``), or the table path when ``qmap`` has been
  replaced or edited in place (as codebook fitting does);
* microscaling: one fused pass that computes the block scales, quantizes and
  multiplies back (``mx_fake_quantize``);
* group-wise affine: one fused pass over each block's min / max, scale, zero
  point and the affine fake-quant (``gwa_fake_quantize``).

All three autograd functions pass gradients straight through to the input.
"""

import logging
import math
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
    "FusedAmaxObsFakeQuantize",
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


class MXFakeQuantizeFunction(torch.autograd.Function):
    """Microscaling fake-quant: block scales from the block amax, quantize,
    multiply back, all in one kernel pass; straight-through gradient."""

    @staticmethod
    def forward(ctx, input, fake_quant_enabled, scale, qmap, axes, block_size, quant_max,
                force_scale_power_of_two=False, scale_qmap=None, fmt=None):
        if not fake_quant_enabled:
            return input
        axis = qops._single_axis(axes)
        if fmt is not None:
            sf, y = qops.mx_fake_quantize(input, fmt, axis, block_size, quant_max,
                                          force_scale_power_of_two, scale_qmap)
        else:
            desc, keep = qops._table_desc(qmap.to(input.device), input.device)
            sf, _, y = qops._mx_call(input, axis, block_size, quant_max, force_scale_power_of_two,
                                     scale_qmap, desc, want_fq=True)
            del keep
        scale.resize_(sf.shape).copy_(sf)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        return (grad_output,) + (None,) * 9


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


class FusedAmaxObsFakeQuantize(FakeQuantizeBase):
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
        self.max_outlier_pct = 0.0
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
        self._observe = self.qscheme is not None
        self._fq_on = True
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
            self._qmap_sig = (self.qmap.data_ptr(), self.qmap._version)

    def _closed_form(self):
        """The format's closed form applies while qmap is the table it built."""
        return self._qmap_sig == (self.qmap.data_ptr(), self.qmap._version)

    # -- flags without device syncs -----------------------------------------
    def enable_fake_quant(self, enabled: bool = True):
        super().enable_fake_quant(enabled)
        self._fq_on = bool(enabled)
        return self

    def disable_fake_quant(self):
        return self.enable_fake_quant(False)

    def enable_observer(self, enabled: bool = True):
        super().enable_observer(enabled)
        self._observe = bool(enabled)
        return self

    def disable_observer(self):
        return self.enable_observer(False)

    # -- observer -----------------------------------------------------------
    @torch.no_grad()
    def _update_amax_scale(self, x: torch.Tensor) -> None:
        """Fold x's amax into the history and recompute scale (:308-341): the
        scale uses the history maximum from before this step's amax."""
        if self.is_per_channel:
            ch_axis = self.ch_axis % x.ndim
            dim = tuple(i for i in range(x.ndim) if i != ch_axis)
            amax_cur = torch.amax(torch.abs(x), dim=dim, keepdim=True)
        else:
            amax_cur = torch.amax(torch.abs(x))
        if self.amax_history.numel() == 0:
            size = (self.amax_history_len,) + amax_cur.shape
            self.amax_history.resize_(size).fill_(0.0)
            self.scale.resize_(amax_cur.shape).fill_(1.0)
        amax = torch.amax(self.amax_history, dim=0)
        self.amax_history.copy_(torch.roll(self.amax_history, -1, 0))
        self.amax_history[0] = amax_cur
        sf = amax / self.quant_max
        sf = torch.where(amax > 0.0, sf, self.scale)
        sf = torch.where(torch.isfinite(amax), sf, self.scale)
        if self.force_scale_power_of_two:
            sf = torch.pow(2, torch.ceil(torch.log2(sf)))
        self.scale.copy_(sf)

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

        if self.outlier_pct is not None and self._observe:
            flat = x.abs().flatten()
            k = max(1, math.ceil(self.outlier_pct * flat.numel()))
            threshold = torch.topk(flat, k, largest=True, sorted=False).values.min()
            if self.outlier_threshold.numel() == 0:
                self.outlier_threshold.resize_as_(threshold)
                self.outlier_threshold.copy_(threshold)
            else:
                self.outlier_threshold.mul_(self.outlier_ema_decay).add_(
                    threshold * (1.0 - self.outlier_ema_decay))

        skip = None
        if self.outlier_threshold is not None:
            skip = x.abs() >= self.outlier_threshold
            orig_x = x
            x = x.masked_fill(skip, 0.0)
            self.max_outlier_pct = max(skip.sum().item() / x.numel(), self.max_outlier_pct)

        fmt = self._fmt if self._closed_form() else None
        if self.qscheme == QScheme.MICROSCALING:
            x = MXFakeQuantizeFunction.apply(x, self._fq_on, self.scale, self.qmap, self.ch_axis,
                                             self.block_size, self.quant_max,
                                             self.force_scale_power_of_two, self.scale_qmap, fmt)
        elif self.qscheme == QScheme.GROUP_WISE_AFFINE:
            x = GroupWiseAffineFakeQuantFunction.apply(x, self._fq_on, self.scale, self.zero_point, self.ch_axis,
                                                       self.block_size, self.quant_min, self.quant_max,
                                                       self.scale_qmap)
        else:
            if self._observe:
                self._update_amax_scale(x)
            x = FakeQuantizeFunction.apply(x, self._fq_on, self.qmap, self.scale, fmt)

        if skip is not None:
            x = torch.where(skip, orig_x, x)
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
