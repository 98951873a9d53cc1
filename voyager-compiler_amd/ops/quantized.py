"""The ``quantized_ops`` torch library on MI355X kernels.

Same qualified names and schema strings as the reference library
(src/voyager_compiler/ops/quantized.py:12, :98, :124-128, :175-179, :286-292,
:363-368, :435-439, :502-506, :532-535, :633-639, :715-719, :809-813), so converted graphs and FakeQuantize modules
call into these kernels unchanged.  Every op has a kernel for the CUDA
dispatch key only (HIP tensors on ROCm dispatch there) plus a fake
implementation for tracing; CPU tensors raise, there is no CPU path.

Ops beyond the reference's (packed storage is this build's own):
``fake_quant``, ``quantize_mx_packed``, ``dequantize_mx_packed``,
``codebook_encode``, ``codebook_decode``, ``linear_nf4``.
"""

import ctypes
import math
import weakref
from typing import List, Optional, Tuple

import torch
from torch.library import Library
from torch.nn.modules.utils import _pair

from .. import _lib
from ..formats import Format, parse_format

quantized_ops_lib = Library("quantized_ops", "DEF")

_SCHEMAS = {
    "vmap": "vmap(Tensor self, Tensor other) -> Tensor",
    "quantize": (
        "quantize(Tensor input, Tensor scale, Tensor? zero_point=None, "
        "SymInt[]? axes=None, int? block_size=None, Tensor? qmap=None, "
        "Tensor? output_code=None) -> Tensor"),
    "dequantize": (
        "dequantize(Tensor input, Tensor scale, Tensor? zero_point=None, "
        "SymInt[]? axes=None, int? block_size=None, Tensor? input_qmap=None, "
        "Tensor? output_qmap=None) -> Tensor"),
    "linear_mx": (
        "linear_mx(Tensor input, Tensor weight, Tensor? bias=None, *, "
        "Tensor? input_scale=None, Tensor? weight_scale=None, "
        "int? block_size=None, Tensor? input_code=None, Tensor? weight_code=None, "
        "Tensor? A_data=None, Tensor? A_indices=None, Tensor? A_indptr=None, "
        'str weight_layout="kc") -> Tensor'),
    "matmul_mx": (
        "matmul_mx(Tensor self, Tensor other, *, Tensor? input_scale=None, "
        "Tensor? weight_scale=None, int? block_size=None, Tensor? input_code=None, "
        "Tensor? weight_code=None, Tensor? A_data=None, Tensor? A_indices=None, "
        'Tensor? A_indptr=None, str weight_layout="ck") -> Tensor'),
    "conv2d_mx": (
        "conv2d_mx(Tensor input, Tensor weight, Tensor? bias=None, "
        "SymInt[2] stride=1, SymInt[2] padding=0, SymInt[2] dilation=1, "
        "SymInt groups=1, *, Tensor? input_scale=None, Tensor? weight_scale=None, "
        "int? block_size=None, Tensor? input_code=None, "
        'Tensor? weight_code=None, str layout="nchw") -> Tensor'),
    "calculate_mx_qparam": (
        "calculate_mx_qparam(Tensor self, SymInt[] axes, int block_size, "
        "float quant_max, bool force_scale_power_of_two=False, "
        "Tensor scale_qmap=None) -> Tensor"),
    "quantize_mx": (
        "quantize_mx(Tensor self, Tensor qmap, SymInt[] axes, int block_size, "
        "float quant_max, bool force_scale_power_of_two=False, "
        "Tensor scale_qmap=None, Tensor output_code=None) -> (Tensor, Tensor)"),
    "filter_outlier": (
        "filter_outlier(Tensor input, float threshold, float max_pct=0.01) "
        "-> (Tensor, Tensor, Tensor, Tensor)"),
    "quantize_mx_outlier": (
        "quantize_mx_outlier(Tensor self, Tensor qmap, SymInt[] axes, "
        "int block_size, float quant_max, bool force_scale_power_of_two=False, "
        "Tensor scale_qmap=None, Tensor output_code=None, float? threshold=None, "
        "float max_pct=0.01, SymInt indptr_offset=0) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)"),
    "slice_csr_tensor": (
        "slice_csr_tensor(Tensor data, Tensor indices, Tensor indptr, int dim=0, "
        "SymInt? start=None, SymInt? end=None, float size_factor=1.0) "
        "-> (Tensor, Tensor, Tensor)"),
    "spmm_csr": (
        "spmm_csr(Tensor data, Tensor indices, Tensor indptr, Tensor B, "
        "Tensor? B_scale=None, Tensor? B_code=None, int? block_size=None, "
        'str weight_layout="kc") -> Tensor'),
    # this build's own
    "fake_quant": (
        "fake_quant(Tensor self, str dtype, Tensor? scale=None, bool mul_back=True, "
        "bool return_codes=False) -> (Tensor, Tensor)"),
    "quantize_mx_packed": (
        "quantize_mx_packed(Tensor self, str dtype, int axis, int block_size, "
        "bool force_scale_power_of_two=True, float? quant_max=None, "
        'str scale_dtype="e8m0") -> (Tensor, Tensor)'),
    "dequantize_mx_packed": (
        "dequantize_mx_packed(Tensor codes, Tensor scale, str dtype, int block_size, "
        "SymInt[] shape, ScalarType out_dtype=bfloat16) -> Tensor"),
    "codebook_encode": "codebook_encode(Tensor self, Tensor codebook) -> Tensor",
    "codebook_decode": (
        "codebook_decode(Tensor codes, Tensor codebook, ScalarType dtype=float) -> Tensor"),
    "linear_nf4": (
        "linear_nf4(Tensor input, Tensor codes, Tensor scale, Tensor? bias=None, int block_size=64, "
        'str dtype="nf4") -> Tensor'),
}
for _s in _SCHEMAS.values():
    quantized_ops_lib.define(_s)


def _impl(name):
    return torch.library.impl(quantized_ops_lib, name, "CUDA")


# ---------------------------------------------------------------------------
# Hardware-layout twins of aten ops (ops/layout.py:104-200): the same name and
# schema as the aten op, with operands stored in the layout the reference's
# layout passes choose.  linear / matmul take the weight (right matrix) with
# its last two dims swapped; conv2d takes NHWC activations and an HWIO weight
# (a grouped conv keeps OIHW) and returns NHWC.  They only permute around the
# aten op, so they are registered for every backend, as the reference's are.
# ---------------------------------------------------------------------------
_NHWC_TO_NCHW, _NCHW_TO_NHWC, _HWIO_TO_OIHW = (0, 3, 1, 2), (0, 2, 3, 1), (3, 2, 0, 1)
for _op in (torch.ops.aten.linear.default, torch.ops.aten.matmul.default, torch.ops.aten.conv2d.default):
    quantized_ops_lib.define(str(_op._schema).split("::", 1)[1])


def _swapped(t):
    # contiguous: batched bf16 products of transposed views are avoided
    return t.transpose(-2, -1).contiguous()


@torch.library.impl(quantized_ops_lib, "linear", "CompositeExplicitAutograd")
def linear_twin(input, weight, bias=None):
    return torch.ops.aten.linear(input, _swapped(weight), bias)


@torch.library.impl(quantized_ops_lib, "matmul", "CompositeExplicitAutograd")
def matmul_twin(self, other):
    return torch.ops.aten.matmul(self, _swapped(other))


@torch.library.impl(quantized_ops_lib, "conv2d", "CompositeExplicitAutograd")
def conv2d_twin(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    w = weight.permute(_HWIO_TO_OIHW) if groups == 1 else weight
    out = torch.ops.aten.conv2d(input.permute(_NHWC_TO_NCHW), w, bias, _pair(stride), _pair(padding),
                                _pair(dilation), groups)
    return out.permute(_NCHW_TO_NHWC)


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
_TABLE_FMT = {}  # data_ptr -> (weakref to table tensor, version, Format)


def register_table(t: torch.Tensor, fmt: Format):
    """Remember that table ``t`` is ``fmt``'s, so ops given ``t`` as a qmap
    can run the closed-form encoder instead of the table gather."""
    _TABLE_FMT[t.data_ptr()] = (weakref.ref(t), _lib.version_of(t), fmt)


def _format_of_table(qmap: torch.Tensor) -> Optional[Format]:
    ent = _TABLE_FMT.get(qmap.data_ptr())
    if ent is None:
        return None
    ref, ver, fmt = ent
    if ref() is not qmap or _lib.version_of(qmap) != ver:
        return None
    return fmt


_BF16_TABLES = {}


def _table_bf16(qmap: torch.Tensor) -> torch.Tensor:
    """A 65536-entry qmap as a contiguous bf16 table on its device."""
    if qmap.numel() != 65536:
        raise ValueError(f"qmap must have 65536 entries (one per bf16 pattern), got {qmap.numel()}")
    if qmap.dtype == torch.bfloat16 and qmap.is_contiguous():
        return qmap
    key = (qmap.data_ptr(), _lib.version_of(qmap), qmap.dtype)
    hit = _BF16_TABLES.get(key)
    if hit is not None and hit[0]() is qmap:
        return hit[1]
    t = qmap.reshape(-1).to(torch.bfloat16).contiguous()
    _BF16_TABLES[key] = (weakref.ref(qmap), t)
    return t


def _table_desc(qmap: torch.Tensor, device) -> Tuple[object, object]:
    """(vqx_format, keep-alive) for a qmap: closed form when it is a known
    format's table, else the table itself."""
    fmt = _format_of_table(qmap)
    if fmt is not None:
        return fmt.desc(device), None
    t = _table_bf16(qmap)
    d = _lib.VqxFormat()
    d.kind = _lib.FMT_TABLE
    d.code_bits = 16
    d.value_table = t.data_ptr()
    return d, t


def _axis_geometry(shape, axis):
    nd = len(shape)
    axis = axis + nd if axis < 0 else axis
    if not 0 <= axis < nd:
        raise ValueError(f"axis {axis} out of range for {nd}-d tensor")
    outer = math.prod(shape[:axis])
    inner = math.prod(shape[axis + 1:])
    return axis, outer, shape[axis], inner


def _single_axis(axes):
    if axes is None:
        raise ValueError("axes required")
    axes = [axes] if isinstance(axes, int) else list(axes)
    if len(axes) != 1:
        raise NotImplementedError(
            f"vqx: blocks along {len(axes)} axes are not implemented (one axis only)")
    return int(axes[0])


def _scale_map(x: torch.Tensor, scale: torch.Tensor, zp: Optional[torch.Tensor], block_size):
    """vqx_scale_map for a scale broadcast (block_size None) or expanded by
    ``expand`` (quantized.py:82-95) against x; None if the layout needs the
    general broadcast path."""
    nd = x.dim()
    s = scale
    while s.dim() < nd:
        s = s.unsqueeze(0)
    if s.dim() != nd:
        return None
    differ = [d for d in range(nd) if s.shape[d] != x.shape[d]]
    m = _lib.VqxScaleMap()
    m.scale = scale.data_ptr()
    m.zero_point = zp.data_ptr() if zp is not None else None
    if block_size is None:
        live = [d for d in range(nd) if s.shape[d] != 1]
        if any(s.shape[d] != x.shape[d] for d in live):
            return None
        if not live:
            m.L, m.inner, m.block, m.s_o, m.s_l, m.s_in = 1, 1, 1, 0, 0, 0
            return m
        if live != list(range(live[0], live[-1] + 1)):
            return None
        d0, d1 = live[0], live[-1]
        m.L = math.prod(x.shape[d0:d1 + 1])
        m.inner = math.prod(x.shape[d1 + 1:])
        m.block, m.s_o, m.s_l, m.s_in = 1, 0, 1, 0
        return m
    if len(differ) != 1:
        return None
    d = differ[0]
    L = x.shape[d]
    nblk = s.shape[d]
    if nblk != -(-L // block_size):
        return None
    m.L = L
    m.inner = math.prod(x.shape[d + 1:])
    m.block = block_size
    m.s_o, m.s_l, m.s_in = nblk * m.inner, m.inner, 1
    return m


def _expand(input, shape, block_size):
    """The reference's scale broadcast (quantized.py:82-95), for the rare
    layouts the scale map cannot describe."""
    while input.ndim < len(shape):
        input = input.unsqueeze(0)
    for dim in range(len(shape)):
        if input.shape[dim] != shape[dim]:
            input = torch.repeat_interleave(input, block_size, dim)
    if list(input.shape) != list(shape):
        input = input[[slice(0, x) for x in shape]]
    return input


# ---------------------------------------------------------------------------
# vmap  (quantized.py:98-121)
# ---------------------------------------------------------------------------
@_impl("vmap")
def vmap(input: torch.Tensor, qmap: torch.Tensor) -> torch.Tensor:
    _lib.require_device(input, "vmap")
    table = _table_bf16(qmap.to(input.device))
    dt = input.dtype
    x = input if dt in (torch.float32, torch.bfloat16, torch.float16) else input.to(torch.bfloat16)
    x = x.contiguous()
    y = torch.empty_like(x, memory_format=torch.contiguous_format)
    _lib.call("vqx_vmap", _lib.ptr(x), _lib.dtype_tag(x.dtype), x.numel(), _lib.ptr(table),
              _lib.ptr(y), _lib.stream_of(x))
    return y if y.dtype == dt else y.to(dt)


# ---------------------------------------------------------------------------
# quantize / dequantize  (quantized.py:124-227)
# ---------------------------------------------------------------------------
def _compute_dtype(*ts):
    dt = ts[0].dtype
    for t in ts[1:]:
        if t is not None:
            dt = torch.promote_types(dt, t.dtype)
    return dt


@_impl("quantize")
def quantize(input, scale, zero_point=None, axes=None, block_size=None, qmap=None, output_code=None):
    assert qmap is not None, "qmap must be provided for quantization"
    _lib.require_device(input, "quantize")
    cdt = _compute_dtype(input, scale, zero_point)
    if cdt not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"vqx: quantize computes in float32/bfloat16/float16, not {cdt}")
    x = input.to(cdt).contiguous()
    s = scale.to(device=x.device, dtype=cdt).contiguous()
    zp = zero_point.to(device=x.device, dtype=cdt).contiguous() if zero_point is not None else None
    m = _scale_map(x, s, zp, block_size)
    if m is None or (zp is not None and zp.shape != s.shape):
        # layouts outside the scale map: broadcast with torch, then one map
        s = (_expand(s, x.shape, block_size) if block_size is not None else s.expand(x.shape)).contiguous()
        zp = None if zp is None else (
            _expand(zp, x.shape, block_size) if block_size is not None else zp.expand(x.shape)).contiguous()
        m = _lib.VqxScaleMap(s.data_ptr(), zp.data_ptr() if zp is not None else None,
                             x.numel(), 1, 1, 0, 1, 0)
    desc, keep = _table_desc(qmap.to(x.device), x.device)
    y = torch.empty_like(x)
    _lib.call("vqx_quantize_mapped", _lib.ptr(x), _lib.dtype_tag(cdt), x.numel(), _lib.ctypes.byref(desc),
              _lib.ctypes.byref(m), 0, _lib.ptr(y), None, 0, _lib.stream_of(x))
    del keep
    return y


@_impl("dequantize")
def dequantize(input, scale, zero_point=None, axes=None, block_size=None, input_qmap=None,
               output_qmap=None):
    _lib.require_device(input, "dequantize")
    cdt = _compute_dtype(input, scale, zero_point)
    if cdt not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"vqx: dequantize computes in float32/bfloat16/float16, not {cdt}")
    if input_qmap is not None and input.dtype != cdt:
        input = vmap(input, input_qmap)
        input_qmap = None
    x = input.to(cdt).contiguous()
    s = scale.to(device=x.device, dtype=cdt).contiguous()
    zp = zero_point.to(device=x.device, dtype=cdt).contiguous() if zero_point is not None else None
    m = _scale_map(x, s, zp, block_size)
    if m is None or (zp is not None and zp.shape != s.shape):
        s = (_expand(s, x.shape, block_size) if block_size is not None else s.expand(x.shape)).contiguous()
        zp = None if zp is None else (
            _expand(zp, x.shape, block_size) if block_size is not None else zp.expand(x.shape)).contiguous()
        m = _lib.VqxScaleMap(s.data_ptr(), zp.data_ptr() if zp is not None else None,
                             x.numel(), 1, 1, 0, 1, 0)
    inm = _table_bf16(input_qmap.to(x.device)) if input_qmap is not None else None
    outm = _table_bf16(output_qmap.to(x.device)) if output_qmap is not None else None
    y = torch.empty_like(x)
    _lib.call("vqx_dequantize_mapped", _lib.ptr(x), _lib.dtype_tag(cdt), x.numel(), _lib.ptr(inm),
              _lib.ctypes.byref(m), _lib.ptr(outm), _lib.ptr(y), _lib.stream_of(x))
    return y


# ---------------------------------------------------------------------------
# calculate_mx_qparam / quantize_mx  (quantized.py:435-529)
# ---------------------------------------------------------------------------
_IDENTITY = None


def _identity_desc(device):
    global _IDENTITY
    if _IDENTITY is None:
        _IDENTITY = parse_format("bfloat16")
    return _IDENTITY.desc(device)


def _mx_call(x, axis, block_size, quant_max, force_pow2, scale_qmap, desc, want_scale=True,
             want_qvals=False, want_fq=False, scale_f32=None, e8m0=None, codes=None, code_layout=1):
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"vqx: block scales are computed for bfloat16/float32 inputs, not {x.dtype}")
    if block_size <= 0:
        raise AssertionError("block_size must be positive")
    x = x.contiguous()
    axis, outer, L, inner = _axis_geometry(list(x.shape), axis)
    sshape = list(x.shape)
    sshape[axis] = -(-L // block_size)
    scale = torch.empty(sshape, dtype=x.dtype, device=x.device) if want_scale else None
    qv = torch.empty_like(x) if want_qvals else None
    fq = torch.empty_like(x) if want_fq else None
    sq = _table_bf16(scale_qmap.to(x.device)) if (scale_qmap is not None and not force_pow2) else None
    shift = math.floor(math.log2(quant_max)) if force_pow2 else 0
    _lib.call("vqx_mx_quantize", _lib.ptr(x), _lib.dtype_tag(x.dtype), outer, L, inner, block_size,
              _lib.ctypes.byref(desc), 0 if force_pow2 else 1, shift, float(quant_max), _lib.ptr(sq),
              _lib.ptr(scale), _lib.ptr(scale_f32), _lib.ptr(e8m0), _lib.ptr(qv), _lib.ptr(fq),
              _lib.ptr(codes), code_layout, _lib.stream_of(x))
    return scale, qv, fq


@_impl("calculate_mx_qparam")
def calculate_mx_qparam(input, axes, block_size, quant_max, force_scale_power_of_two=False,
                        scale_qmap=None):
    _lib.require_device(input, "calculate_mx_qparam")
    axis = _single_axis(axes)
    scale, _, _ = _mx_call(input, axis, block_size, quant_max, force_scale_power_of_two, scale_qmap,
                           _identity_desc(input.device))
    return scale


@_impl("quantize_mx")
def quantize_mx(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                scale_qmap=None, output_code=None):
    _lib.require_device(input, "quantize_mx")
    axis = _single_axis(axes)
    desc, keep = _table_desc(qmap.to(input.device), input.device)
    scale, qv, _ = _mx_call(input, axis, block_size, quant_max, force_scale_power_of_two, scale_qmap,
                            desc, want_qvals=True)
    del keep
    return scale, qv


def mx_fake_quantize(input, fmt: Format, axis, block_size, quant_max, force_pow2, scale_qmap=None,
                     scale_f32=None):
    """MXFakeQuantizeFunction.forward's numerics (fake_quantize.py:143-153):
    (scale, quantize_mx values * expand(scale)) in one pass.  With scale_f32
    (a contiguous fp32 tensor of the scale shape) the scale is written there
    and returned as it, instead of a new tensor in x's dtype."""
    if scale_f32 is not None:
        _, _, fq = _mx_call(input, axis, block_size, quant_max, force_pow2, scale_qmap,
                            fmt.desc(input.device), want_scale=False, want_fq=True, scale_f32=scale_f32)
        return scale_f32, fq
    scale, _, fq = _mx_call(input, axis, block_size, quant_max, force_pow2, scale_qmap,
                            fmt.desc(input.device), want_fq=True)
    return scale, fq


def mx_scale_shape(shape, axis, block_size):
    """The block-scale shape of an MX quantization of `shape` along `axis`."""
    axis, _, L, _ = _axis_geometry(list(shape), axis)
    sshape = list(shape)
    sshape[axis] = -(-L // block_size)
    return sshape


def mx_fake_quantize_outlier(input, desc, axis, block_size, quant_max, force_pow2, scale_qmap, threshold, stats,
                             parity=0, scale_f32=None):
    """FakeQuantize's outlier masking around MXFakeQuantizeFunction.forward
    (fake_quantize.py:388-395 around :397-408) in one pass: the elements with
    |x| >= threshold (a float, or an fp32 device tensor) are zeros for the
    block scales and the fake-quant, come back unchanged in the output, and
    are counted into stats (outlier_stats(), set `parity`; see
    vqx_mx_fake_quant_outlier).  Returns (scale, output): the scale in x's
    dtype, or written into scale_f32 (a contiguous fp32 tensor of the scale
    shape) and returned as it."""
    if input.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"vqx: block scales are computed for bfloat16/float32 inputs, not {input.dtype}")
    if block_size <= 0:
        raise AssertionError("block_size must be positive")
    x = input.contiguous()
    axis, outer, L, inner = _axis_geometry(list(x.shape), axis)
    scale = None
    if scale_f32 is None:
        sshape = list(x.shape)
        sshape[axis] = -(-L // block_size)
        scale = torch.empty(sshape, dtype=x.dtype, device=x.device)
    y = torch.empty_like(x)
    sq = _table_bf16(scale_qmap.to(x.device)) if (scale_qmap is not None and not force_pow2) else None
    shift = math.floor(math.log2(quant_max)) if force_pow2 else 0
    thr_dev, thr = _threshold_args(threshold, x.device)
    _lib.call("vqx_mx_fake_quant_outlier", _lib.ptr(x), _lib.dtype_tag(x.dtype), outer, L, inner, block_size,
              _lib.ctypes.byref(desc), 0 if force_pow2 else 1, shift, float(quant_max), _lib.ptr(sq), thr_dev, thr,
              _lib.ptr(stats), int(parity), _lib.ptr(scale), _lib.ptr(scale_f32), _lib.ptr(y), _lib.stream_of(x))
    return (scale if scale_f32 is None else scale_f32), y


def _threshold_args(threshold, device):
    """(device pointer or None, host float) of an outlier threshold: a tensor
    is read on the device (its fp32 value), a number passes by value."""
    if isinstance(threshold, torch.Tensor):
        if threshold.dtype != torch.float32 or threshold.numel() != 1 or threshold.device != device:
            raise ValueError("vqx: an outlier threshold tensor must be one fp32 value on the input's device")
        return _lib.ptr(threshold), 0.0
    return None, float(threshold)


def outlier_mask(input, threshold, stats, parity=0, masked=True):
    """x.masked_fill(|x| >= threshold, 0) (fake_quantize.py:388-391), with the
    outliers counted into stats (set `parity`); masked=False only counts
    (returns None)."""
    x = input.contiguous()
    out = torch.empty_like(x) if masked else None
    thr_dev, thr = _threshold_args(threshold, x.device)
    _lib.call("vqx_outlier_mask", _lib.ptr(x), _lib.dtype_tag(x.dtype), x.numel(), thr_dev, thr, _lib.ptr(stats),
              int(parity), _lib.ptr(out), _lib.stream_of(x))
    return out


# The stats buffer's layout (include/vqx.h, vqx_outlier_stats_size): the fp64
# of the largest fraction folded so far at byte 0; set p at byte 256 + 2176 p,
# its numel there and 16 partial counts at 128-byte steps after it.
_STATS_SET0, _STATS_SET_BYTES, _STATS_STRIDE, _STATS_SLOTS = 256, 2176, 128, 16
_STATS_BYTES = None


def outlier_stats(device):
    """Zeroed device memory for the outlier counts (vqx_outlier_stats_size
    bytes, 256-byte aligned by the caching allocator)."""
    global _STATS_BYTES
    if _STATS_BYTES is None:
        n = ctypes.c_int64(0)
        _lib.call("vqx_outlier_stats_size", ctypes.byref(n))
        _STATS_BYTES = n.value
    return torch.zeros(_STATS_BYTES // 8, dtype=torch.int64, device=device)


def outlier_stats_fraction(stats, last_parity):
    """The largest fraction of outliers in a stats buffer (one host read):
    the folded maximum, or the last call's count / numel (set last_parity)
    when larger."""
    w = stats.cpu()
    best = float(w.view(torch.float64)[0])
    base = (_STATS_SET0 + last_parity * _STATS_SET_BYTES) // 8
    n = int(w[base])
    if n:
        c = sum(int(w[base + _STATS_STRIDE // 8 * (1 + s)]) for s in range(_STATS_SLOTS))
        best = max(best, c / n)
    return best


def outlier_restore_(input, threshold, y):
    """y = torch.where(|x| >= threshold, x, y) in place (fake_quantize.py:
    429-430); y contiguous, shaped and typed like x."""
    x = input.contiguous()
    if y.shape != x.shape or y.dtype != x.dtype or not y.is_contiguous():
        raise ValueError("vqx: outlier restore needs a contiguous output shaped and typed like the input")
    thr_dev, thr = _threshold_args(threshold, x.device)
    _lib.call("vqx_outlier_restore", _lib.ptr(x), _lib.dtype_tag(x.dtype), x.numel(), thr_dev, thr, _lib.ptr(y),
              _lib.stream_of(x))
    return y


_TOPK_WS_BYTES = None


def outlier_topk_threshold_(input, outlier_pct, threshold, ema, decay, workspace):
    """The outlier_pct threshold (fake_quantize.py:373-387) on the device:
    the k-th largest |x| (k = max(1, ceil(outlier_pct * numel)); NaN when x
    holds a NaN) stored into threshold (ema False) or folded into it as
    threshold * decay + value * (1 - decay) (ema True).  threshold: one fp32
    value on x's device; workspace: outlier_topk_workspace(device)."""
    x = input.contiguous()
    n = x.numel()
    k = max(1, math.ceil(outlier_pct * n))
    if k > n:
        raise RuntimeError(f"selected index k out of range: k = {k} for {n} elements (outlier_pct {outlier_pct})")
    _threshold_args(threshold, x.device)
    _lib.call("vqx_outlier_topk_threshold", _lib.ptr(x), _lib.dtype_tag(x.dtype), n, k, 1 if ema else 0,
              float(decay), float(1.0 - decay), _lib.ptr(threshold), _lib.ptr(workspace), workspace.numel(),
              _lib.stream_of(x))


def outlier_topk_workspace(device):
    """Zeroed device memory for outlier_topk_threshold_ (each call leaves it
    ready for the next; calls that share one must be ordered)."""
    global _TOPK_WS_BYTES
    if _TOPK_WS_BYTES is None:
        n = ctypes.c_int64(0)
        _lib.call("vqx_outlier_topk_workspace_size", ctypes.byref(n))
        _TOPK_WS_BYTES = n.value
    return torch.zeros(_TOPK_WS_BYTES, dtype=torch.uint8, device=device)


def gwa_fake_quantize(input, axis, block_size, quant_min, quant_max, scale_qmap=None):
    """GroupWiseAffineFakeQuantFunction.forward's numerics (fake_quantize.py:
    162-211): (scale, zero_point, fake-quantized input) in one pass, scale and
    zero_point shaped like the blocks (the axis becomes ceil(L / block_size))
    and in the input's dtype."""
    if input.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"vqx: group-wise affine fake-quant takes bfloat16/float32 inputs, not {input.dtype}")
    if block_size is None or block_size <= 0:
        raise AssertionError("block_size must be positive")
    _lib.require_device(input, "group_wise_affine fake-quant")
    x = input.contiguous()
    axis, outer, L, inner = _axis_geometry(list(x.shape), axis)
    sshape = list(x.shape)
    sshape[axis] = -(-L // block_size)
    scale = torch.empty(sshape, dtype=x.dtype, device=x.device)
    zero_point = torch.empty_like(scale)
    y = torch.empty_like(x)
    sq = _table_bf16(scale_qmap.to(x.device)) if scale_qmap is not None else None
    _lib.call("vqx_gwa_fake_quant", _lib.ptr(x), _lib.dtype_tag(x.dtype), outer, L, inner, block_size,
              float(quant_min), float(quant_max), _lib.ptr(sq), _lib.ptr(scale), _lib.ptr(zero_point),
              _lib.ptr(y), _lib.stream_of(x))
    return scale, zero_point, y


# ---------------------------------------------------------------------------
# linear_mx / matmul_mx  (quantized.py:286-432): a convert-format weight
# with up to 16 levels and blocks of 64 runs the fused dequant product;
# other operands decode on the GPU, then the dense product (hipBLASLt).
# ---------------------------------------------------------------------------
_CODE_LUTS = {}


def _code_lut(code: torch.Tensor) -> torch.Tensor:
    """65536-entry table sending each bf16 pattern x to code[x.long()] as the
    reference indexes it (quantized.py:313-320): x truncated toward zero, a
    negative index counting from the end.  Patterns whose index falls outside
    the table (and NaN / Inf) map to NaN, where the reference raises
    IndexError."""
    key = (code.data_ptr(), _lib.version_of(code), code.numel(), code.dtype)
    hit = _CODE_LUTS.get(key)
    if hit is not None and hit[0]() is code:
        return hit[1]
    K = code.numel()
    if K > 256:
        raise ValueError("code tables hold at most 256 entries")
    v = torch.arange(65536, dtype=torch.int32, device=code.device).to(torch.int16).view(torch.bfloat16).float()
    t = torch.trunc(v)
    ok = torch.isfinite(v) & (t >= -K) & (t < K)
    idx = torch.where(ok, t, torch.zeros_like(t)).to(torch.int64) % K
    lut = torch.where(ok, code.reshape(-1).to(torch.bfloat16)[idx], torch.full_like(v, float("nan")).to(torch.bfloat16))
    _CODE_LUTS[key] = (weakref.ref(code), lut)
    return lut


_BF16_EXACT = {}


def _bf16_exact(code: torch.Tensor) -> bool:
    """Whether every code value survives a round trip through bf16 (the
    65536-entry table the lookup uses holds bf16 values)."""
    key = (code.data_ptr(), _lib.version_of(code), code.numel(), code.dtype)
    hit = _BF16_EXACT.get(key)
    if hit is not None and hit[0]() is code:
        return hit[1]
    ok = code.dtype == torch.bfloat16 or bool(torch.equal(code.to(torch.bfloat16).to(code.dtype), code))
    _BF16_EXACT[key] = (weakref.ref(code), ok)
    return ok


def _decode_operand(t, code, scale, block_size):
    if code is None and scale is None:
        return t
    if code is not None and t.dtype != torch.bfloat16 and not _bf16_exact(code):
        # code values finer than bf16 in a wider operand: the reference's
        # gather by integer value (quantized.py:313-315), then the scales;
        # indices outside the table give NaN (the reference raises there)
        K = code.numel()
        tr = torch.trunc(t.float())
        ok = torch.isfinite(tr) & (tr >= -K) & (tr < K)
        idx = torch.where(ok, tr, torch.zeros_like(tr)).to(torch.long) % K
        t = torch.where(ok, code.to(t.device).reshape(-1)[idx].to(t.dtype), torch.full_like(t, float("nan")))
        code = None
        if scale is None:
            return t
    if code is not None:
        lut = _code_lut(code.to(t.device))
    else:
        lut = None
    if scale is None:
        return vmap(t, lut)
    return dequantize(t, scale, None, None, block_size, lut, None)


# The fused product.  A converted model's GEMM arrives as linear_mx /
# matmul_mx with the weight in convert format (quantize_pt2e.py:456-508, the
# rewrite at :592-645): integer-valued code indices in a bf16 tensor, at most
# 16 bf16 levels in weight_code, bf16 scales with blocks of 64 along K.  The
# reference decodes that into a dense bf16 weight, bf16(level * scale), and
# calls aten.linear / aten.matmul.  Here the operands are packed once per
# weight (4-bit codes, the scales widened exactly to fp32) and the decode runs
# inside the bf16 MFMA product (vqx_nf4_linear_ws), which computes the same
# bf16(level * scale) values.  The packing is cached per weight tensor and
# redone when any of the three operands changes (tensor version counters).
class _Packed:
    __slots__ = ("refs", "versions", "codes", "scale", "levels")


_PACKED = {}


def _release_packed(key):
    _PACKED.pop(key, None)


def _packed_weight(weight, weight_code, weight_scale, transposed):
    """Packed (codes, fp32 scales, 16 bf16 levels) of a convert-format weight,
    or None when an index is out of the code table's range (the unfused
    path then reproduces the reference's behaviour)."""
    key = (id(weight), bool(transposed))
    deps = (weight, weight_code, weight_scale)
    versions = tuple(None if t is None else (t.data_ptr(), _lib.version_of(t)) for t in deps)
    hit = _PACKED.get(key)
    if hit is not None and hit.versions == versions and all(
            (r is None and t is None) or (r is not None and r() is t) for r, t in zip(hit.refs, deps)):
        return None if hit.codes is None else (hit.codes, hit.scale, hit.levels)
    K, N = weight.shape if transposed else weight.shape[::-1]
    dev = weight.device
    w = weight.contiguous()
    s = None if weight_scale is None else weight_scale.to(dev).contiguous()
    ncode = weight_code.numel()
    codes = torch.empty(N, K // 2, dtype=torch.uint8, device=dev)
    scale32 = torch.empty(N, K // 64, dtype=torch.float32, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("vqx_nf4_pack_weight", _lib.ptr(w), _lib.dtype_tag(w.dtype), _lib.ptr(s),
              0 if s is None else _lib.dtype_tag(s.dtype), N, K, 1 if transposed else 0, ncode, _lib.ptr(codes),
              _lib.ptr(scale32), _lib.ptr(bad), _lib.stream_of(w))
    levels = torch.zeros(16, dtype=torch.bfloat16, device=dev)
    levels[:ncode] = weight_code.reshape(-1).to(device=dev, dtype=torch.bfloat16)
    entry = _Packed()
    entry.refs = tuple(None if t is None else weakref.ref(t) for t in deps)
    entry.versions = versions
    # one host read per packing (not per call): whether every index was valid
    if int(bad.item()):
        entry.codes = entry.scale = entry.levels = None
    else:
        entry.codes, entry.scale, entry.levels = codes, scale32, levels
    if hit is None:
        weakref.finalize(weight, _release_packed, key)
    _PACKED[key] = entry
    return None if entry.codes is None else (entry.codes, entry.scale, entry.levels)


def _fusable(x, weight, bias, weight_scale, block_size, weight_code, transposed):
    """Whether the product of x with this weight can run fused: bf16
    activations, a 2-D bf16 index weight with a code table of at most 16
    entries, bf16 scales in blocks of 64 along K (the reference's decoded
    weight is then bf16, as aten.linear needs), a bf16 bias, K % 64, and for
    more than 16 rows N % 128 (the tile kernel's column tiles)."""
    if weight_code is None or weight.dim() != 2 or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        return False
    if weight_code.dim() != 1 or not 1 <= weight_code.numel() <= 16 or weight_code.device != weight.device:
        return False
    K, N = weight.shape if transposed else weight.shape[::-1]
    if x.shape[-1] != K or K % 64 or not x.is_cuda or weight.device != x.device:
        return False
    if weight_scale is not None:
        want = (K // 64, N) if transposed else (N, K // 64)
        if block_size != 64 or weight_scale.dtype != torch.bfloat16 or tuple(weight_scale.shape) != want:
            return False
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (N,) or bias.device != x.device):
        return False
    M = x.numel() // K
    return M > 0 and (M <= 16 or N % 128 == 0)


def _nf4_product(x2d, codes, scale32, levels, bias, N):
    """out[M, N] = x2d . decode(codes, scale32, levels)^T (+ bias) through the
    fused kernel, launched on x's current stream."""
    M, K = x2d.shape
    out = torch.empty(M, N, dtype=torch.bfloat16, device=x2d.device)
    ws_bytes = _nf4_workspace_bytes(M, N, K, x2d.device)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x2d.device) if ws_bytes else None
    _lib.call("vqx_nf4_linear_ws", _lib.ptr(x2d), _lib.ptr(codes), _lib.ptr(scale32), _lib.ptr(levels),
              _lib.ptr(bias), _lib.ptr(out), M, N, K, _lib.ptr(ws), ws_bytes, _lib.stream_of(x2d))
    return out


def _fused_linear(x, weight, bias, weight_scale, weight_code, transposed):
    packed = _packed_weight(weight, weight_code, weight_scale, transposed)
    if packed is None:
        return None
    K = x.shape[-1]
    N = weight.shape[1] if transposed else weight.shape[0]
    # the kernel reads A in 16-byte and the bias in 8-byte units: a view
    # with an odd storage offset (a slice of a flat buffer) is copied first
    b = None if bias is None else bias.contiguous()
    if b is not None and b.data_ptr() % 8:
        b = b.clone()
    x2 = x.reshape(-1, K).contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    out = _nf4_product(x2, *packed, b, N)
    return out.reshape(*x.shape[:-1], N)


# The product with both operands decoded inside the kernel (vqx_mx_matmul):
# every other bf16 convert-format pair whose scales run along the contraction
# dim -- coded activations, code tables of up to 256 entries or none (int6,
# int8), power-of-two blocks from 8 up, batched right operands (the attention
# products), either storage layout of the right operand.
_BF16_CODES = {}


def _code_bf16(code: torch.Tensor, device) -> torch.Tensor:
    """The code table as the bf16 values the kernel reads (the reference casts
    the looked-up values to the operand's dtype, bf16 here), cached per code
    tensor and version."""
    key = (code.data_ptr(), _lib.version_of(code), code.numel(), code.dtype, str(device))
    hit = _BF16_CODES.get(key)
    if hit is not None and hit[0]() is code:
        return hit[1]
    t = code.reshape(-1).to(device=device, dtype=torch.bfloat16).contiguous()
    _BF16_CODES[key] = (weakref.ref(code), t)
    return t


def _mx_side_ok(t, code, scale, block_size, kdim):
    """Whether one operand fits vqx_mx_matmul: bf16 data, at most 256 code
    entries, bf16 scales with the operand's shape but ceil(K / block_size)
    along the contraction dim kdim, a power-of-two block size >= 8."""
    if t.dtype != torch.bfloat16 or not t.is_cuda or t.dim() < 2:
        return False
    if code is not None and (code.dim() != 1 or not 1 <= code.numel() <= 256):
        return False
    if scale is not None:
        if block_size is None or block_size < 8 or block_size & (block_size - 1) or scale.dtype != torch.bfloat16:
            return False
        want = list(t.shape)
        want[kdim] = -(-want[kdim] // block_size)
        if list(scale.shape) != want or scale.device != t.device:
            return False
    return True


def _coded(*parts):
    """Whether any operand carries a code table or scales (a product of two
    plain bf16 operands is the library GEMM's)."""
    return any(p is not None for p in parts)


def _aligned16(t):
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _mx_operand(data, code, scale, block_size, k_major, batch_stride, ld, scale_batch_stride, scale_ld):
    op = _lib.VqxMxOperand()
    op.data = data.data_ptr()
    op.scale = None if scale is None else scale.data_ptr()
    op.code = None if code is None else code.data_ptr()
    op.batch_stride, op.ld = batch_stride, ld
    op.scale_batch_stride, op.scale_ld = scale_batch_stride, scale_ld
    op.k_major = 1 if k_major else 0
    op.block_size = 0 if scale is None else int(block_size)
    op.code_len = 0 if code is None else code.numel()
    return op


def _right_operand(b, code, scale, block_size, stored_kn):
    """Descriptor pieces of the right operand [*, K, N] (stored_kn) or
    [*, N, K]: K-major when K is the contiguous dim in memory, else N-major;
    the scales laid out to match.  Returns (data, scale, k_major, ld, K, N)."""
    K, N = (b.shape[-2], b.shape[-1]) if stored_kn else (b.shape[-1], b.shape[-2])
    # the memory order: which of the last two dims is contiguous
    kn = b if stored_kn else b.transpose(-2, -1)   # logical [*, K, N]
    if kn.transpose(-2, -1).is_contiguous() and not kn.is_contiguous():
        k_major = True
    elif kn.is_contiguous():
        k_major = False
    else:
        k_major = not stored_kn
    if k_major:
        data = _aligned16(kn.transpose(-2, -1))    # [*, N, K]
        s = None if scale is None else (scale.transpose(-2, -1) if stored_kn else scale).contiguous()
        ld = K
    else:
        data = _aligned16(kn)                      # [*, K, N]
        s = None if scale is None else _aligned16(scale if stored_kn else scale.transpose(-2, -1))
        ld = N
    return data, s, k_major, ld, K, N


# An operand that many output tiles read is decoded once, by the vqx decode
# kernel (dequantize: about 4 bytes of HBM traffic per element), instead of
# in every tile that reads it (about 2.5 VALU per element per tile, which
# the product's VALU-bound staging pays in full); the kernel decodes the
# operands that at most this many 128-wide tiles read, such as the attention
# probabilities of P V (one column tile).
_FUSED_DECODE_MAX_TILES = 4
_DECODED = {}


def _release_decoded(key):
    _DECODED.pop(key, None)


def _mx_decoded(t, code, scale, block_size, kdim):
    """t (bf16, contraction dim kdim = -1 or -2, scales along it) decoded to
    dense bf16 by vqx_mx_operand_decode, in t's own memory layout; the reference's
    decode (quantized.py:313-326) through the decode-only pass of the product
    kernel.  Falls back to the general decode for layouts it does not take."""
    if t.dim() < 2:
        return _decode_operand(t, code, scale, block_size)
    lead = t.shape[:-2]
    # m: the operand as stored, [*, R, C] contiguous; k_major: K is C
    tt = t.transpose(-2, -1)
    if t.is_contiguous():
        m, flipped = t, False
    elif tt.is_contiguous():
        m, flipped = tt, True
    else:
        m, flipped = t.contiguous(), False
    k_major = (kdim == -1) != flipped
    R, C = m.shape[-2], m.shape[-1]
    K, cols = (C, R) if k_major else (R, C)
    if K % 8 or (not k_major and C % 8):
        return _decode_operand(t, code, scale, block_size)
    sm = None
    if scale is not None:
        sm = scale.transpose(-2, -1) if flipped else scale
        sm = _aligned16(sm)
    md = _aligned16(m)
    batch = math.prod(lead)
    op = _mx_operand(md, None if code is None else _code_bf16(code, t.device), sm, block_size, k_major,
                     R * C, C, 0 if sm is None else sm.shape[-2] * sm.shape[-1], 0 if sm is None else sm.shape[-1])
    out = torch.empty_like(md)
    _lib.call("vqx_mx_operand_decode", _lib.ctypes.byref(op), batch, cols, K, _lib.ptr(out), _lib.stream_of(t))
    return out.transpose(-2, -1) if flipped else out


def _activation_decoded(x, code, scale, block_size):
    """The left operand's decode ahead of the packed-weight product: the
    streaming decode pass when it takes the operand (bf16, scales along the
    last dim), else the general decode."""
    if (code is not None or scale is not None) and x.dim() >= 1 and x.shape[-1] % 8 == 0 and x.numel() > 0:
        x2 = x.reshape(-1, x.shape[-1])
        s2 = None
        if scale is not None and scale.dim() == x.dim() and tuple(scale.shape[:-1]) == tuple(x.shape[:-1]):
            s2 = scale.reshape(-1, scale.shape[-1])
        if (scale is None or s2 is not None) and _mx_side_ok(x2, code, s2, block_size, -1):
            return _mx_decoded(x2, code, s2, block_size, -1).reshape(x.shape)
    return _decode_operand(x, code, scale, block_size)


def _decoded_weight(weight, code, scale, block_size, kdim):
    """The bf16 decode of a convert-format weight, cached per weight tensor
    and rebuilt when the weight, its code or its scale change (version
    counters), as the packed NF4 weight is."""
    key = id(weight)
    deps = (weight, code, scale)
    versions = tuple(None if t is None else (t.data_ptr(), _lib.version_of(t)) for t in deps)
    hit = _DECODED.get(key)
    if hit is not None and hit[1] == versions and all(
            (r is None and t is None) or (r is not None and r() is t) for r, t in zip(hit[0], deps)):
        return hit[2]
    dense = _mx_decoded(weight, code, scale, block_size, kdim)
    if hit is None:
        weakref.finalize(weight, _release_decoded, key)
    _DECODED[key] = (tuple(None if t is None else weakref.ref(t) for t in deps), versions, dense)
    return dense


def _mx_product(a, a_code, a_scale, b, b_code, b_scale, block_size, b_stored_kn, bias, b_static=False):
    """A'[*, M, K] . B' through vqx_mx_matmul, or None when the operands fall
    outside it.  b: [*, K, N] when b_stored_kn, else [*, N, K]; batch dims
    equal, or one side without them.  b_static: b is a weight (its decode is
    cached when it is decoded ahead of the product)."""
    if not (_mx_side_ok(a, a_code, a_scale, block_size, -1)
            and _mx_side_ok(b, b_code, b_scale, block_size, -2 if b_stored_kn else -1)):
        return None
    N = b.shape[-1] if b_stored_kn else b.shape[-2]
    if (a_code is not None or a_scale is not None) and -(-N // 128) > _FUSED_DECODE_MAX_TILES:
        a, a_code, a_scale = _mx_decoded(a, a_code, a_scale, block_size, -1), None, None
    rows = a.shape[-2] * (math.prod(a.shape[:-2]) if b.dim() == 2 else 1)
    if (b_code is not None or b_scale is not None) and -(-rows // 128) > _FUSED_DECODE_MAX_TILES:
        kdim = -2 if b_stored_kn else -1
        b = _decoded_weight(b, b_code, b_scale, block_size, kdim) if b_static else \
            _mx_decoded(b, b_code, b_scale, block_size, kdim)
        b_code, b_scale = None, None
    M, K = a.shape[-2], a.shape[-1]
    Kb, N = (b.shape[-2], b.shape[-1]) if b_stored_kn else (b.shape[-1], b.shape[-2])
    if Kb != K or M < 1 or N < 1 or K < 1 or K % 8 or N % 4:
        return None
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (N,) or bias.device != a.device):
        return None
    ba, bb = tuple(a.shape[:-2]), tuple(b.shape[:-2])
    if ba == bb:
        batch_shape, a_shared, b_shared = ba, False, False
    elif len(bb) == 0:
        batch_shape, a_shared, b_shared = ba, False, True
    elif len(ba) == 0:
        batch_shape, a_shared, b_shared = bb, True, False
    else:
        return None
    batch = math.prod(batch_shape)
    if batch < 1:
        return None
    bd, bs_, bk_major, bld, _, _ = _right_operand(b, b_code, b_scale, block_size, b_stored_kn)
    if not bk_major and N % 8:
        return None
    nkb = 0 if a_scale is None else a_scale.shape[-1]
    if b_shared and not a_shared:
        # one right matrix for every item: the items' rows run as one product
        ad = _aligned16(a).reshape(-1, K)
        asc = None if a_scale is None else a_scale.contiguous().reshape(-1, nkb)
        rows, nbatch = ad.shape[0], 1
    else:
        ad = _aligned16(a)
        asc = None if a_scale is None else a_scale.contiguous()
        rows, nbatch = M, batch
    dev = a.device
    ac = None if a_code is None else _code_bf16(a_code, dev)
    bc = None if b_code is None else _code_bf16(b_code, dev)
    opa = _mx_operand(ad, ac, asc, block_size, True, 0 if (a_shared or nbatch == 1) else M * K, K,
                      0 if (asc is None or a_shared or nbatch == 1) else M * nkb, nkb)
    if bk_major:
        s_b = 0 if bs_ is None else bs_.shape[-1] * N
        s_ld = 0 if bs_ is None else bs_.shape[-1]
    else:
        s_b = 0 if bs_ is None else bs_.shape[-2] * N
        s_ld = N
    opb = _mx_operand(bd, bc, bs_, block_size, bk_major, 0 if b_shared else K * N, bld,
                      0 if (bs_ is None or b_shared) else s_b, s_ld)
    bias_c = None if bias is None else bias.contiguous()
    if bias_c is not None and bias_c.data_ptr() % 8:
        bias_c = bias_c.clone()
    out = torch.empty(nbatch, rows, N, dtype=torch.bfloat16, device=dev)
    _lib.call("vqx_mx_matmul", _lib.ctypes.byref(opa), _lib.ctypes.byref(opb), _lib.ptr(bias_c), _lib.ptr(out),
              nbatch, rows, N, K, _lib.stream_of(a))
    return out.reshape(*batch_shape, M, N)


@_impl("linear_mx")
def linear_mx(input, weight, bias=None, *, input_scale=None, weight_scale=None, block_size=None,
              input_code=None, weight_code=None, A_data=None, A_indices=None, A_indptr=None,
              weight_layout="kc"):
    """quantized.py:295-348.  A convert-format weight of up to 16 levels with
    blocks of 64 along K runs the packed-weight product (the activations
    decoded first); other bf16 convert-format operands run the product that
    decodes both inside the kernel; anything else decodes on the GPU and
    calls the library GEMM."""
    assert weight_layout in ("kc", "ck"), weight_layout
    _lib.require_device(input, "linear_mx")
    transposed = weight_layout == "ck"
    dense = None
    x = None
    if weight_code is not None and weight_code.numel() <= 16:
        x = _activation_decoded(input, input_code, input_scale, block_size)
        if _fusable(x, weight, bias, weight_scale, block_size, weight_code, transposed):
            dense = _fused_linear(x, weight, bias, weight_scale, weight_code, transposed)
    if dense is None and _coded(input_code, input_scale, weight_code, weight_scale) and input.dim() >= 1 \
            and weight.dim() == 2 and input.shape[-1] > 0 and (
                input_scale is None or tuple(input_scale.shape[:-1]) == tuple(input.shape[:-1])):
        # the activation's rows as one [M, K] product
        K = input.shape[-1]
        a = input.reshape(-1, K)
        s = None if input_scale is None else input_scale.reshape(a.shape[0], input_scale.shape[-1])
        dense = _mx_product(a, input_code, s, weight, weight_code, weight_scale, block_size, transposed, bias,
                            b_static=True)
        if dense is not None:
            dense = dense.reshape(*input.shape[:-1], dense.shape[-1])
    if dense is None:
        if x is None:
            x = _decode_operand(input, input_code, input_scale, block_size)
        w = _decode_operand(weight, weight_code, weight_scale, block_size)
        if weight_layout == "kc":
            dense = torch.nn.functional.linear(x, w, bias)
        else:
            dense = torch.ops.quantized_ops.linear(x, w, bias)
    if A_data is None:
        return dense
    return _spmm(A_data, A_indices, A_indptr, weight, weight_scale, weight_code, block_size, weight_layout,
                 addend=dense)


@_impl("matmul_mx")
def matmul_mx(self, other, *, input_scale=None, weight_scale=None, block_size=None, input_code=None,
              weight_code=None, A_data=None, A_indices=None, A_indptr=None, weight_layout="ck"):
    """quantized.py:371-421.  A 2-D convert-format right operand ([K, N] for
    "ck", [N, K] for "kc") of up to 16 levels with blocks of 64 runs the
    packed-weight product, as in linear_mx; other bf16 convert-format
    operands (both sides coded, batched, as the attention products are) run
    the product that decodes both inside the kernel; anything else decodes
    and calls the library GEMM."""
    assert weight_layout in ("kc", "ck"), weight_layout
    _lib.require_device(self, "matmul_mx")
    transposed = weight_layout == "ck"
    dense = None
    a = None
    if weight_code is not None and weight_code.numel() <= 16 and other.dim() == 2:
        a = _activation_decoded(self, input_code, input_scale, block_size)
        if a.dim() >= 1 and _fusable(a, other, None, weight_scale, block_size, weight_code, transposed):
            dense = _fused_linear(a, other, None, weight_scale, weight_code, transposed)
    if dense is None and _coded(input_code, input_scale, weight_code, weight_scale):
        dense = _mx_product(self, input_code, input_scale, other, weight_code, weight_scale, block_size,
                            transposed, None)
    if dense is None:
        if a is None:
            a = _decode_operand(self, input_code, input_scale, block_size)
        b = _decode_operand(other, weight_code, weight_scale, block_size)
        if weight_layout == "ck":
            dense = torch.matmul(a, b.contiguous())
        else:
            dense = torch.ops.quantized_ops.matmul(a, b)
    if A_data is None:
        return dense
    return _spmm(A_data, A_indices, A_indptr, other, weight_scale, weight_code, block_size, weight_layout,
                 addend=dense)


@_impl("conv2d_mx")
def conv2d_mx(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, *, input_scale=None,
              weight_scale=None, block_size=None, input_code=None, weight_code=None, layout="nchw"):
    """quantized.py:230-284: activations and weight decoded on the GPU as
    linear_mx decodes them (code lookup, then the product with the expanded
    block scales), then the convolution (MIOpen through aten), or its NHWC
    twin for ``layout="nhwc"`` (NHWC activations, HWIO weight)."""
    assert layout in ("nchw", "nhwc"), layout
    _lib.require_device(input, "conv2d_mx")
    x = _decode_operand(input, input_code, input_scale, block_size)
    w = _decode_operand(weight, weight_code, weight_scale, block_size)
    stride, padding, dilation = _pair(stride), _pair(padding), _pair(dilation)
    if layout == "nhwc":
        return torch.ops.quantized_ops.conv2d(x, w, bias, stride, padding, dilation, groups)
    return torch.ops.aten.conv2d(x, w, bias, stride, padding, dilation, groups)


# ---------------------------------------------------------------------------
# outliers as CSR: filter_outlier, quantize_mx_outlier, slice_csr_tensor,
# spmm_csr (quantized.py:532-895)
# ---------------------------------------------------------------------------
_FLOAT_TAGS = (torch.float32, torch.bfloat16, torch.float16)


def _float_tag(t, what):
    if t.dtype not in _FLOAT_TAGS:
        raise ValueError(f"vqx: {what} takes float32/bfloat16/float16 values, not {t.dtype}")
    return _lib.dtype_tag(t.dtype)


def _int32_index(t, what):
    if t.dtype != torch.int32:
        raise ValueError(f"vqx: {what} must be int32, not {t.dtype}")
    return t.contiguous()


def _outlier_csr(input, threshold, max_pct, indptr_offset):
    """filter_outlier (quantized.py:572-630) with the row pointers shifted by
    indptr_offset, on the GPU: (data, indices, indptr, inlier)."""
    _lib.require_device(input, "filter_outlier")
    if threshold is None:
        raise TypeError("filter_outlier: threshold must be a float, not None")
    if input.ndim < 2:
        raise ValueError(f"filter_outlier: input must have at least 2 dims, got {input.ndim}")
    x = input.contiguous()
    tag = _float_tag(x, "filter_outlier")
    batch_shape = x.shape[:-2]
    R, C = x.shape[-2:]
    max_nnz = int(math.prod(x.shape[-2:]) * max_pct)
    if max_nnz < 0:
        raise ValueError(f"filter_outlier: max_pct {max_pct} gives a negative capacity")
    if not -(1 << 31) <= indptr_offset < (1 << 31):
        raise ValueError(f"indptr_offset {indptr_offset} does not fit the int32 row pointers")
    # torch compares against the Python scalar cast to the tensor's dtype
    t = torch.tensor(float(threshold), dtype=x.dtype).item()
    nb = math.prod(batch_shape)
    dev = x.device
    data = torch.empty((*batch_shape, max_nnz), dtype=x.dtype, device=dev)
    indices = torch.empty((*batch_shape, max_nnz), dtype=torch.int32, device=dev)
    indptr = torch.empty((*batch_shape, R + 1), dtype=torch.int32, device=dev)
    inlier = torch.empty_like(x)
    ws = _outlier_workspace(tag, nb, R, C, max_nnz, dev)
    _lib.call("vqx_filter_outlier_ws", _lib.ptr(x), tag, nb, R, C, t, max_nnz, int(indptr_offset), _lib.ptr(data),
              _lib.ptr(indices), _lib.ptr(indptr), _lib.ptr(inlier), _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    return data, indices, indptr, inlier


def _outlier_workspace(tag, nb, R, C, max_nnz, dev):
    """Staging memory of the one-pass outlier split: each row's count and its
    first outliers (the library sizes it; the caching allocator keeps it)."""
    n = ctypes.c_int64(0)
    _lib.call("vqx_outlier_workspace_size", tag, nb, R, C, max_nnz, ctypes.byref(n))
    return torch.empty(max(n.value, 1), dtype=torch.uint8, device=dev)


@_impl("filter_outlier")
def filter_outlier(input, threshold, max_pct=0.01):
    """Outliers (|x| > threshold) as a per-matrix CSR over the last two dims,
    int32 indices, data/indices sized int(rows*cols*max_pct) and padded with
    0/-1 (the first entries in row-major order kept on overflow, row pointers
    clamped), plus the input with outliers zeroed (quantized.py:537-630)."""
    return _outlier_csr(input, threshold, max_pct, 0)


@_impl("quantize_mx_outlier")
def quantize_mx_outlier(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                        scale_qmap=None, output_code=None, threshold=None, max_pct=0.01, indptr_offset=0):
    """filter_outlier, row pointers + indptr_offset, then quantize_mx of the
    inliers (quantized.py:642-691): (data, indices, indptr, scale, inliers)."""
    seq = isinstance(axes, (list, tuple))
    ax = (axes[0] if len(axes) == 1 else None) if seq else axes
    if (ax in (-1, input.ndim - 1) and input.dtype == torch.bfloat16 and input.ndim >= 2 and threshold is not None
            and block_size in (8, 16, 32, 64) and input.shape[-1] % block_size == 0):
        return _quantize_mx_outlier_fused(input, qmap, block_size, quant_max, force_scale_power_of_two, scale_qmap,
                                          threshold, max_pct, indptr_offset)
    data, indices, indptr, inliers = _outlier_csr(input, threshold, max_pct, indptr_offset)
    scale, q = quantize_mx(inliers, qmap, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap)
    return data, indices, indptr, scale, q


def _quantize_mx_outlier_fused(input, qmap, block_size, quant_max, force_pow2, scale_qmap, threshold, max_pct,
                               indptr_offset):
    """quantize_mx_outlier for bf16 blocks along the last axis in one pass:
    the split writes the quantized inliers and their block scales directly."""
    _lib.require_device(input, "quantize_mx_outlier")
    x = input.contiguous()
    batch_shape = x.shape[:-2]
    R, C = x.shape[-2:]
    max_nnz = int(math.prod(x.shape[-2:]) * max_pct)
    if max_nnz < 0:
        raise ValueError(f"filter_outlier: max_pct {max_pct} gives a negative capacity")
    if not -(1 << 31) <= indptr_offset < (1 << 31):
        raise ValueError(f"indptr_offset {indptr_offset} does not fit the int32 row pointers")
    t = torch.tensor(float(threshold), dtype=x.dtype).item()
    nb = math.prod(batch_shape)
    dev = x.device
    data = torch.empty((*batch_shape, max_nnz), dtype=x.dtype, device=dev)
    indices = torch.empty((*batch_shape, max_nnz), dtype=torch.int32, device=dev)
    indptr = torch.empty((*batch_shape, R + 1), dtype=torch.int32, device=dev)
    scale = torch.empty((*x.shape[:-1], C // block_size), dtype=x.dtype, device=dev)
    values = torch.empty_like(x)
    table = _table_bf16(qmap.to(dev))
    sq = _table_bf16(scale_qmap.to(dev)) if (scale_qmap is not None and not force_pow2) else None
    shift = math.floor(math.log2(quant_max)) if force_pow2 else 0
    ws = _outlier_workspace(_lib.dtype_tag(x.dtype), nb, R, C, max_nnz, dev)
    _lib.call("vqx_quantize_mx_outlier_ws", _lib.ptr(x), nb, R, C, t, max_nnz, int(indptr_offset), block_size,
              0 if force_pow2 else 1, shift, float(quant_max), _lib.ptr(sq), _lib.ptr(table), _lib.ptr(data), _lib.ptr(indices), _lib.ptr(indptr), _lib.ptr(scale), _lib.ptr(values), _lib.ptr(ws),
              ws.numel(), _lib.stream_of(x))
    return data, indices, indptr, scale, values


@_impl("slice_csr_tensor")
def slice_csr_tensor(data, indices, indptr, dim=0, start=None, end=None, size_factor=1.0):
    """Rows (dim 0) or columns (dim 1) [start, end) of one CSR matrix, data and
    indices sized int(len(data) * size_factor) and padded like filter_outlier's
    (quantized.py:722-777)."""
    dim = dim + 2 if dim < 0 else dim
    if dim not in (0, 1):
        raise ValueError(f"Cannot slice sparse CSR matrix along dim {dim}")
    _lib.require_device(data, "slice_csr_tensor")
    if data.ndim != 1 or indices.ndim != 1 or indptr.ndim != 1:
        raise ValueError("slice_csr_tensor takes one CSR matrix: 1-D data, indices and indptr")
    if start is None or end is None:
        raise TypeError("slice_csr_tensor: start and end are required")
    tag = _float_tag(data, "slice_csr_tensor")
    data = data.contiguous()
    indices = _int32_index(indices, "slice_csr_tensor indices")
    indptr = _int32_index(indptr, "slice_csr_tensor indptr")
    rows = indptr.numel() - 1
    if rows < 0:
        raise ValueError("slice_csr_tensor: indptr is empty")
    max_nnz = int(data.shape[0] * size_factor)
    if max_nnz < 0:
        raise ValueError(f"slice_csr_tensor: size_factor {size_factor} gives a negative capacity")
    dev = data.device
    if dim == 0:
        L = rows + 1
        s = start + L if start < 0 else start
        e = end + L if end < 0 else end
        n_out = len(range(L)[start:end + 1])
        if not (0 <= s <= e <= rows) or n_out != e - s + 1:
            raise IndexError(f"slice_csr_tensor: rows [{start}, {end}) of a {rows}-row matrix")
        indptr_out = torch.empty(n_out, dtype=torch.int32, device=dev)
    else:
        if start < 0:
            raise ValueError("slice_csr_tensor: column slices start at a column >= 0")
        s, e = start, end
        indptr_out = torch.empty_like(indptr)
    data_out = torch.empty(max_nnz, dtype=data.dtype, device=dev)
    indices_out = torch.empty(max_nnz, dtype=torch.int32, device=dev)
    _lib.call("vqx_slice_csr", _lib.ptr(data), tag, _lib.ptr(indices), _lib.ptr(indptr), data.numel(), rows, dim,
              s, e, max_nnz, _lib.ptr(data_out), _lib.ptr(indices_out), _lib.ptr(indptr_out), _lib.stream_of(data))
    return data_out, indices_out, indptr_out


def _scale_index(scale, shape, block_size):
    """The element -> scale map of expand(scale, shape, block_size)
    (quantized.py:82-95) for a [.., rows, cols] operand:
    (batch stride, scale rows, scale cols, row block, col block)."""
    s = list(scale.shape)
    if len(s) > len(shape):
        raise ValueError(f"scale shape {tuple(scale.shape)} has more dims than {tuple(shape)}")
    s = [1] * (len(shape) - len(s)) + s
    div = []
    for a, b in zip(s, shape):
        if a == b:
            div.append(1)
        elif block_size is not None and a * block_size >= b:
            div.append(block_size)
        elif a == 1 and block_size == 1:
            div.append(max(b, 1))  # stays size 1 and broadcasts
        else:
            raise ValueError(f"scale shape {tuple(scale.shape)} does not expand to {tuple(shape)} "
                             f"with block_size {block_size}")
    sr, sc = s[-2], s[-1]
    lead = list(zip(s[:-2], shape[:-2], div[:-2]))
    if all(d == 1 for _, _, d in lead):
        sb = sr * sc
    elif all(b <= d for _, b, d in lead):
        sb = 0  # every batch maps to scale batch 0
    else:
        raise NotImplementedError("vqx: scales blocked across batch dims are not supported")
    return sb, sr, sc, div[-2], div[-1]


def _spmm(data, indices, indptr, B, B_scale=None, B_code=None, block_size=None, weight_layout="kc",
          addend=None):
    """spmm_csr (quantized.py:816-878) on the GPU; with an addend of the
    output's shape and dtype, addend + spmm in the same pass."""
    assert weight_layout in ("kc", "ck"), weight_layout
    _lib.require_device(B, "spmm_csr")
    if B.ndim < 2:
        raise ValueError("spmm_csr: B must have at least 2 dims")
    dev = B.device
    out_dtype = B.dtype if B_code is None else B_code.dtype
    if B_scale is not None:
        out_dtype = torch.promote_types(out_dtype, B_scale.dtype)
    if out_dtype not in _FLOAT_TAGS:
        raise ValueError(f"vqx: spmm_csr computes in float32/bfloat16/float16, not {out_dtype}")
    batch_shape = indptr.shape[:-1]
    nb = math.prod(batch_shape)
    R = indptr.shape[-1] - 1
    indptr2 = _int32_index(indptr, "spmm_csr indptr").reshape(nb, R + 1)
    indices2 = _int32_index(indices, "spmm_csr indices").reshape(nb, -1)
    data2 = data.contiguous().reshape(nb, -1)
    dtag = _float_tag(data2, "spmm_csr data")
    if indices2.shape[1] != data2.shape[1]:
        raise ValueError("spmm_csr: data and indices must have the same length")
    br, bc = B.shape[-2:]
    nbB = math.prod(B.shape[:-2]) if B.ndim > 2 else 1
    if B.ndim > 2 and nbB != nb:
        raise ValueError(f"spmm_csr: B holds {nbB} matrices for {nb} CSR batches")
    K, N = (bc, br) if weight_layout == "kc" else (br, bc)
    Bc = B.contiguous()
    if B_code is None and B_scale is None and weight_layout == "ck":
        Bt = Bc
    else:
        Bt = torch.empty((nbB, K, N), dtype=out_dtype, device=dev)
        code = None if B_code is None else B_code.reshape(-1).contiguous()
        scale = None if B_scale is None else B_scale.contiguous()
        sb, sr, sc, rdiv, cdiv = (0, 1, 1, 1, 1) if scale is None else _scale_index(scale, B.shape, block_size)
        if code is not None and code.dtype not in _FLOAT_TAGS:
            raise ValueError(f"vqx: B_code must be float32/bfloat16/float16, not {code.dtype}")
        if scale is not None and scale.dtype not in _FLOAT_TAGS:
            raise ValueError(f"vqx: B_scale must be float32/bfloat16/float16, not {scale.dtype}")
        _lib.call("vqx_csr_decode_weight", _lib.ptr(Bc), _lib.dtype_tag(Bc.dtype), nbB, br, bc,
                  1 if weight_layout == "kc" else 0, _lib.ptr(code),
                  _lib.dtype_tag(code.dtype) if code is not None else 0, 0 if code is None else code.numel(),
                  _lib.ptr(scale), _lib.dtype_tag(scale.dtype) if scale is not None else 0, sb, sr, sc, rdiv, cdiv,
                  _lib.ptr(Bt), _lib.dtype_tag(out_dtype), _lib.stream_of(Bc))
    out_shape = (*batch_shape, R, N)
    fuse = (addend is not None and addend.dtype == out_dtype and tuple(addend.shape) == out_shape
            and addend.is_contiguous() and addend.device == dev)
    out = torch.empty(out_shape, dtype=out_dtype, device=dev)
    _lib.call("vqx_spmm_csr", _lib.ptr(data2), dtag, _lib.ptr(indices2), _lib.ptr(indptr2), nb, R, data2.shape[1],
              _lib.ptr(Bt), _lib.dtype_tag(out_dtype), K * N if B.ndim > 2 else 0, K, N,
              _lib.ptr(addend) if fuse else None, _lib.ptr(out), _lib.stream_of(Bc))
    if addend is not None and not fuse:
        return addend + out
    return out


@_impl("spmm_csr")
def spmm_csr(data, indices, indptr, B, B_scale=None, B_code=None, block_size=None, weight_layout="kc"):
    """Per-batch CSR [rows, K] x decoded B [K, N] in fp32, cast to the decoded
    B's dtype (quantized.py:816-878)."""
    return _spmm(data, indices, indptr, B, B_scale, B_code, block_size, weight_layout)


# ---------------------------------------------------------------------------
# this build's own ops
# ---------------------------------------------------------------------------
def _codes_fit(fmt: Format):
    """Codes are at most 16 bits wide: int / uint formats beyond that (such as
    the int24 of a bias) have values but no code output."""
    if fmt.kind == _lib.FMT_INT and fmt.p0 > 16:
        raise ValueError(f"vqx: {fmt.dtype} values are supported, its codes are not (codes are at most 16 bits)")


@_impl("fake_quant")
def fake_quant(input, dtype, scale=None, mul_back=True, return_codes=False):
    """Closed-form FakeQuantizeFunction (fake_quantize.py:101-115) with an
    optional per-tensor or per-channel fp32 scale and optional codes."""
    _lib.require_device(input, "fake_quant")
    fmt = parse_format(dtype)
    x = input.contiguous()
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"vqx: fake_quant input must be float32/bfloat16/float16, not {x.dtype}")
    if return_codes:
        _codes_fit(fmt)
    y = torch.empty_like(x)
    cb = 1 if fmt.code_bits <= 8 else 2
    codes = (torch.empty(x.shape, dtype=torch.uint8 if cb == 1 else torch.int16, device=x.device)
             if return_codes else torch.empty(0, dtype=torch.uint8, device=x.device))
    s, sn, si = None, 1, 1
    if scale is not None:
        s = scale.to(device=x.device, dtype=torch.float32).contiguous()
        sn = s.numel()
        if sn > 1:
            m = _scale_map(x, s, None, None)
            if m is None or m.s_l != 1:
                raise ValueError("fake_quant: scale must be per-tensor or vary along one axis run")
            si = m.inner
    _lib.call("vqx_fake_quant", _lib.ptr(x), _lib.dtype_tag(x.dtype), x.numel(),
              _lib.ctypes.byref(fmt.desc(x.device)), _lib.ptr(s), sn, si, int(bool(mul_back)),
              _lib.ptr(y), _lib.ptr(codes) if return_codes else None, cb, _lib.stream_of(x))
    return y, codes


_SCALE_DTYPES = {"e8m0": torch.uint8, "float32": torch.float32, "bfloat16": torch.bfloat16}


@_impl("quantize_mx_packed")
def quantize_mx_packed(input, dtype, axis, block_size, force_scale_power_of_two=True, quant_max=None,
                       scale_dtype="e8m0"):
    """Block scales + packed codes (code_bits per element, element i at bits
    [cb*i, cb*i+cb) of a little-endian bitstream) along the last axis."""
    _lib.require_device(input, "quantize_mx_packed")
    fmt = parse_format(dtype)
    _codes_fit(fmt)
    if quant_max is None:
        from ..formats import quant_range
        quant_max = float(quant_range(dtype)[1])
    x = input.contiguous()
    ax, outer, L, inner = _axis_geometry(list(x.shape), axis)
    if inner != 1:
        raise ValueError("quantize_mx_packed blocks run along the last axis")
    if scale_dtype not in _SCALE_DTYPES:
        raise ValueError(f"scale_dtype must be one of {sorted(_SCALE_DTYPES)}")
    if scale_dtype == "e8m0" and not force_scale_power_of_two:
        raise ValueError("E8M0 scales need force_scale_power_of_two")
    if scale_dtype == "bfloat16" and x.dtype != torch.bfloat16:
        raise ValueError("bfloat16 scales need a bfloat16 input (scales come in the input dtype)")
    nbytes = x.numel() * fmt.code_bits // 8
    codes = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    sshape = list(x.shape)
    sshape[ax] = -(-L // block_size)
    sc = None
    if scale_dtype != "bfloat16":
        sc = torch.empty(sshape, dtype=_SCALE_DTYPES[scale_dtype], device=x.device)
    s_in, _, _ = _mx_call(x, ax, block_size, quant_max, force_scale_power_of_two, None, fmt.desc(x.device),
                          want_scale=scale_dtype == "bfloat16",
                          scale_f32=sc if scale_dtype == "float32" else None,
                          e8m0=sc if scale_dtype == "e8m0" else None,
                          codes=codes, code_layout=0)
    return (s_in if sc is None else sc), codes


@_impl("dequantize_mx_packed")
def dequantize_mx_packed(codes, scale, dtype, block_size, shape, out_dtype=torch.bfloat16):
    _lib.require_device(codes, "dequantize_mx_packed")
    fmt = parse_format(dtype)
    n = math.prod(shape)
    kind = {torch.float32: 0, torch.bfloat16: 1, torch.uint8: 2}.get(scale.dtype)
    if kind is None:
        raise ValueError(f"scale dtype {scale.dtype} not in float32/bfloat16/uint8(E8M0)")
    dtab = fmt.tables(codes.device)["decode"]
    out = torch.empty(list(shape), dtype=out_dtype, device=codes.device)
    _lib.call("vqx_mx_decode", _lib.ptr(codes.contiguous()), fmt.code_bits, _lib.ptr(dtab), dtab.numel(),
              _lib.ptr(scale.contiguous()), kind, n, block_size, _lib.ptr(out), _lib.dtype_tag(out_dtype),
              _lib.stream_of(codes))
    return out


@_impl("codebook_encode")
def codebook_encode(input, codebook):
    """Per-row nearest-entry codes against sorted per-row codebooks [rows, K]."""
    _lib.require_device(input, "codebook_encode")
    x = input.contiguous()
    rows = codebook.shape[0]
    cb = codebook.to(device=x.device, dtype=torch.float32).contiguous()
    if x.numel() % rows != 0:
        raise ValueError("input rows must match codebook rows")
    cols = x.numel() // rows
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    _lib.call("vqx_codebook_encode", _lib.ptr(x), _lib.dtype_tag(x.dtype), rows, cols, _lib.ptr(cb),
              cb.shape[1], _lib.ptr(codes), _lib.stream_of(x))
    return codes


@_impl("codebook_decode")
def codebook_decode(codes, codebook, dtype=torch.float32):
    _lib.require_device(codes, "codebook_decode")
    c = codes.contiguous()
    rows = codebook.shape[0]
    cb = codebook.to(device=c.device, dtype=torch.float32).contiguous()
    cols = c.numel() // rows
    out = torch.empty(c.shape, dtype=dtype, device=c.device)
    _lib.call("vqx_codebook_decode", _lib.ptr(c), rows, cols, _lib.ptr(cb), cb.shape[1], _lib.ptr(out),
              _lib.dtype_tag(dtype), _lib.stream_of(c))
    return out


@_impl("linear_nf4")
def linear_nf4(input, codes, scale, bias=None, block_size=64, dtype="nf4"):
    """linear_mx for an NF4 block-64 weight stored packed (quantize_mx_packed
    with fp32 scales): out = input . decode(codes, scale)^T + bias, the decode
    fused into the bf16 MFMA product.  input bf16 [..., K]; codes uint8
    [N * K / 2] or [N, K / 2]; scale fp32 [N, K / 64]."""
    _lib.require_device(input, "linear_nf4")
    if block_size != 64:
        raise ValueError("linear_nf4 is built for 64-element scale blocks")
    fmt = parse_format(dtype)
    if not fmt.is_levels or fmt.nlevels != 16:
        raise ValueError(f"linear_nf4 needs a 16-level NormalFloat format, not {dtype}")
    if input.dtype != torch.bfloat16:
        raise ValueError("linear_nf4 takes bfloat16 activations")
    K = input.shape[-1]
    x = input.reshape(-1, K).contiguous()
    M = x.shape[0]
    N = scale.shape[0]
    if scale.shape[-1] * 64 != K or codes.numel() * 2 != N * K:
        raise ValueError("codes / scale shapes do not match the input's K")
    lv = fmt.tables(x.device)["levels_bf16"]
    b = None if bias is None else bias.to(device=x.device, dtype=torch.bfloat16).contiguous()
    out = _nf4_product(x, codes.contiguous(), scale.to(torch.float32).contiguous(), lv, b, N)
    return out.reshape(*input.shape[:-1], N)


_NF4_WS = {}


def _nf4_workspace_bytes(M, N, K, device):
    """Workspace the NF4 tile kernel's balanced last round needs for this
    shape on ``device`` (0: whole tiles only), cached per shape."""
    key = (M, N, K, device.index)
    if key not in _NF4_WS:
        n = ctypes.c_int64(0)
        with torch.cuda.device(device):
            _lib.call("vqx_nf4_linear_workspace_size", M, N, K, ctypes.byref(n))
        _NF4_WS[key] = n.value
    return _NF4_WS[key]


# ---------------------------------------------------------------------------
# fake (meta) implementations for tracing
# ---------------------------------------------------------------------------
@torch.library.register_fake("quantized_ops::vmap")
def _(input, qmap):
    return torch.empty_like(input, memory_format=torch.contiguous_format)


@torch.library.register_fake("quantized_ops::quantize")
def _(input, scale, zero_point=None, axes=None, block_size=None, qmap=None, output_code=None):
    return torch.empty_like(input, dtype=_compute_dtype(input, scale, zero_point))


@torch.library.register_fake("quantized_ops::dequantize")
def _(input, scale, zero_point=None, axes=None, block_size=None, input_qmap=None, output_qmap=None):
    return torch.empty_like(input, dtype=_compute_dtype(input, scale, zero_point))


@torch.library.register_fake("quantized_ops::calculate_mx_qparam")
def _(input, axes, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None):
    shape = list(input.shape)
    for a in ([axes] if isinstance(axes, int) else axes):
        shape[a] = -(-shape[a] // block_size)
    return input.new_empty(shape)


@torch.library.register_fake("quantized_ops::quantize_mx")
def _(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None,
      output_code=None):
    shape = list(input.shape)
    for a in ([axes] if isinstance(axes, int) else axes):
        shape[a] = -(-shape[a] // block_size)
    return input.new_empty(shape), torch.empty_like(input, memory_format=torch.contiguous_format)


def _decoded_fake(t, scale):
    return t if scale is None else t.to(torch.promote_types(t.dtype, scale.dtype))


@torch.library.register_fake("quantized_ops::linear_mx")
def _(input, weight, bias=None, **kwargs):
    x = _decoded_fake(input, kwargs.get("input_scale"))
    w = _decoded_fake(weight, kwargs.get("weight_scale"))
    if kwargs.get("weight_layout", "kc") == "ck":
        return torch.ops.quantized_ops.linear(x, w, bias)
    return torch.nn.functional.linear(x, w, bias)


@torch.library.register_fake("quantized_ops::matmul_mx")
def _(self, other, **kwargs):
    a = _decoded_fake(self, kwargs.get("input_scale"))
    b = _decoded_fake(other, kwargs.get("weight_scale"))
    if kwargs.get("weight_layout", "ck") == "kc":
        return torch.ops.quantized_ops.matmul(a, b)
    return torch.matmul(a, b)


@torch.library.register_fake("quantized_ops::conv2d_mx")
def _(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, **kwargs):
    x = _decoded_fake(input, kwargs.get("input_scale"))
    w = _decoded_fake(weight, kwargs.get("weight_scale"))
    args = (bias, _pair(stride), _pair(padding), _pair(dilation), groups)
    if kwargs.get("layout", "nchw") == "nhwc":
        return torch.ops.quantized_ops.conv2d(x, w, *args)
    return torch.ops.aten.conv2d(x, w, *args)


def _csr_fake(input, max_pct):
    batch_shape = input.shape[:-2]
    max_nnz = int(math.prod(input.shape[-2:]) * max_pct)
    return (input.new_empty((*batch_shape, max_nnz)),
            input.new_empty((*batch_shape, max_nnz), dtype=torch.int32),
            input.new_empty((*batch_shape, input.shape[-2] + 1), dtype=torch.int32))


@torch.library.register_fake("quantized_ops::filter_outlier")
def _(input, threshold, max_pct=0.01):
    data, indices, indptr = _csr_fake(input, max_pct)
    return data, indices, indptr, torch.empty_like(input)


@torch.library.register_fake("quantized_ops::quantize_mx_outlier")
def _(input, qmap, axes, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None,
      output_code=None, threshold=None, max_pct=0.01, indptr_offset=0):
    data, indices, indptr = _csr_fake(input, max_pct)
    shape = list(input.shape)
    for a in ([axes] if isinstance(axes, int) else axes):
        shape[a] = -(-shape[a] // block_size)
    return (data, indices, indptr, input.new_empty(shape),
            torch.empty_like(input, memory_format=torch.contiguous_format))


@torch.library.register_fake("quantized_ops::slice_csr_tensor")
def _(data, indices, indptr, dim=0, start=None, end=None, size_factor=1.0):
    max_nnz = int(data.shape[0] * size_factor)
    rows = indptr.shape[0] if dim not in (0, -2) else len(range(indptr.shape[0])[start:end + 1])
    return (data.new_empty((max_nnz,)), indices.new_empty((max_nnz,)), indptr.new_empty((rows,)))


@torch.library.register_fake("quantized_ops::spmm_csr")
def _(data, indices, indptr, B, B_scale=None, B_code=None, block_size=None, weight_layout="kc"):
    dt = B.dtype if B_code is None else B_code.dtype
    if B_scale is not None:
        dt = torch.promote_types(dt, B_scale.dtype)
    N = B.shape[-2] if weight_layout == "kc" else B.shape[-1]
    return data.new_empty((*indptr.shape[:-1], indptr.shape[-1] - 1, N), dtype=dt)


@torch.library.register_fake("quantized_ops::fake_quant")
def _(input, dtype, scale=None, mul_back=True, return_codes=False):
    f = parse_format(dtype)
    cdt = torch.uint8 if f.code_bits <= 8 else torch.int16
    return torch.empty_like(input), input.new_empty(input.shape if return_codes else (0,), dtype=cdt)


@torch.library.register_fake("quantized_ops::quantize_mx_packed")
def _(input, dtype, axis, block_size, force_scale_power_of_two=True, quant_max=None, scale_dtype="e8m0"):
    f = parse_format(dtype)
    shape = list(input.shape)
    shape[axis] = -(-shape[axis] // block_size)
    return (input.new_empty(shape, dtype=_SCALE_DTYPES[scale_dtype]),
            input.new_empty((input.numel() * f.code_bits // 8,), dtype=torch.uint8))


@torch.library.register_fake("quantized_ops::dequantize_mx_packed")
def _(codes, scale, dtype, block_size, shape, out_dtype=torch.bfloat16):
    return codes.new_empty(list(shape), dtype=out_dtype)


@torch.library.register_fake("quantized_ops::codebook_encode")
def _(input, codebook):
    return input.new_empty(input.shape, dtype=torch.uint8)


@torch.library.register_fake("quantized_ops::codebook_decode")
def _(codes, codebook, dtype=torch.float32):
    return codes.new_empty(codes.shape, dtype=dtype)


@torch.library.register_fake("quantized_ops::linear_nf4")
def _(input, codes, scale, bias=None, block_size=64, dtype="nf4"):
    return input.new_empty((*input.shape[:-1], scale.shape[0]), dtype=torch.bfloat16)
