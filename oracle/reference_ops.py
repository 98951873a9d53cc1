"""CPU oracle, part 2: the reference's op sequences on CPU tensors.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Restates, on torch CPU
tensors, the operations of the reference's ``quantized_ops`` library and
FakeQuantize functions, with the same dtype semantics (every op rounds to its
tensor's dtype, bf16 log2 included).  The format tables come from
``oracle.formats`` (pinned to the golden tables).  Also the timed CPU baseline.

Citations: src/voyager_compiler = src/vc.
"""

import math

import numpy as np
import torch

from . import formats as F

__all__ = [
    "table_tensor",
    "vmap",
    "expand",
    "quantize",
    "dequantize",
    "calculate_mx_qparam",
    "quantize_mx",
    "mx_fake_quantize",
    "group_wise_affine_fake_quant",
    "fake_quantize_per_tensor",
    "codebook_encode_rows",
    "codebook_decode_rows",
    "linear_mx",
]


def table_tensor(u16):
    """uint16 bit patterns -> bf16 torch tensor."""
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).view(torch.bfloat16)


def vmap(x, qmap, chunk_size=1 << 20):
    """src/vc/ops/quantized.py:101-121: bf16 cast, then a chunked gather."""
    dt = x.dtype
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    idx = x.view(torch.int16).reshape(-1)
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    of = out.view(-1)
    for s in range(0, idx.numel(), chunk_size):
        e = min(s + chunk_size, idx.numel())
        of[s:e] = qmap[idx[s:e].to(torch.int32) & 0xFFFF]
    return out.to(dt)


def expand(t, shape, block_size):
    """src/vc/ops/quantized.py:82-95."""
    while t.ndim < len(shape):
        t = t.unsqueeze(0)
    for d in range(len(shape)):
        if t.shape[d] != shape[d]:
            t = torch.repeat_interleave(t, block_size, d)
    if list(t.shape) != list(shape):
        t = t[tuple(slice(0, x) for x in shape)]
    return t


def quantize(x, scale, zero_point=None, axes=None, block_size=None, qmap=None):
    """src/vc/ops/quantized.py:131-172."""
    if block_size is not None:
        scale = expand(scale, x.shape, block_size)
        if zero_point is not None:
            zero_point = expand(zero_point, x.shape, block_size)
    x = x / scale if zero_point is None else x / scale + zero_point
    return vmap(x, qmap)


def dequantize(x, scale, zero_point=None, axes=None, block_size=None, input_qmap=None, output_qmap=None):
    """src/vc/ops/quantized.py:182-227."""
    if input_qmap is not None:
        x = vmap(x, input_qmap)
    if block_size is not None:
        scale = expand(scale, x.shape, block_size)
        if zero_point is not None:
            zero_point = expand(zero_point, x.shape, block_size)
    y = x * scale if zero_point is None else (x - zero_point) * scale
    if output_qmap is not None:
        y = vmap(y, output_qmap)
    return y


def _to_blocks(x, axis, block_size):
    """src/vc/quantization/mx_utils.py:62-121 for one axis: unsqueeze, zero-pad
    the axis to a multiple of block_size, and split it into (blocks, block)."""
    axis = axis + x.ndim if axis < 0 else axis
    x = x.unsqueeze(axis + 1)
    L = x.shape[axis]
    if L % block_size:
        pad = [0, 0] * x.ndim
        pad[2 * (x.ndim - 1 - axis) + 1] = block_size - L % block_size
        x = torch.nn.functional.pad(x, pad, mode="constant")
    shape = list(x.shape)
    if shape[axis] >= block_size:
        shape[axis + 1] = block_size
        shape[axis] //= block_size
    else:
        shape[axis + 1] = shape[axis]
        shape[axis] = 1
    return x.view(shape), axis


def calculate_mx_qparam(x, axes, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None):
    """src/vc/ops/quantized.py:442-499 with mx_utils.py:16-59 (one axis)."""
    axis = axes[0] if isinstance(axes, (list, tuple)) else axes
    xb, axis = _to_blocks(x, axis, block_size)
    if force_scale_power_of_two:
        a = torch.abs(xb).amax(dim=axis + 1, keepdim=True)
        e = torch.floor(torch.log2(a + 2.0**-126 * (a == 0).type(a.dtype)))
        e = e - math.floor(math.log2(quant_max))
        e = e.squeeze(axis + 1)
        scale = 2 ** e
    else:
        amax = torch.amax(torch.abs(xb), dim=axis + 1)
        scale = amax / quant_max
        if scale_qmap is not None:
            scale = vmap(scale, scale_qmap)
    return torch.where(scale > 0.0, scale, 1.0)


def quantize_mx(x, qmap, axes, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None):
    """src/vc/ops/quantized.py:509-529."""
    scale = calculate_mx_qparam(x, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap)
    return scale, quantize(x, scale, None, axes, block_size, qmap)


def mx_fake_quantize(x, qmap, axes, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None):
    """MXFakeQuantizeFunction.forward (src/vc/quantization/fake_quantize.py:143-153)."""
    sf, q = quantize_mx(x, qmap, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap)
    return sf, q * expand(sf, q.shape, block_size)


def group_wise_affine_fake_quant(x, axes, block_size, quant_min, quant_max, scale_qmap=None):
    """GroupWiseAffineFakeQuantFunction.forward (src/vc/quantization/
    fake_quantize.py:162-211), one axis: block min / max of the zero-padded
    blocks, sf, zp, optional scale_qmap, then the affine fake-quant, every op
    on x's dtype.  Returns (scale, zero_point, y)."""
    axis = axes[0] if isinstance(axes, (list, tuple)) else axes
    xb, axis = _to_blocks(x, axis, block_size)
    mn = torch.amin(xb, dim=axis + 1)
    mx = torch.amax(xb, dim=axis + 1)
    sf = (mx - mn) / (quant_max - quant_min)
    sf = torch.where(sf > 0.0, sf, 1.0)
    zp = -mn / sf + quant_min
    if scale_qmap is not None:
        sf = vmap(sf, scale_qmap)
        zp = vmap(zp, scale_qmap)
    sfe = expand(sf, x.shape, block_size)
    zpe = expand(zp, x.shape, block_size)
    q = torch.clamp(torch.round(x / sfe + zpe), quant_min, quant_max)
    return sf, zp, (q - zpe) * sfe


def fake_quantize_per_tensor(x, qmap, scale):
    """FakeQuantizeFunction.forward (src/vc/quantization/fake_quantize.py:112-115)."""
    s = scale.to(x.dtype)
    return vmap(x / s, qmap) * s


def codebook_encode_rows(x, cb):
    """Per-row form of codebook_qmap + vmap (src/vc/quantization/lcq.py:286-291):
    bf16 value of x, clamped to the row's codebook range, nearest entry in
    fp32, first index on ties (torch.argmin); NaN -> 0."""
    v = x.to(torch.bfloat16).float()
    lo = cb.min(dim=1, keepdim=True).values
    hi = cb.max(dim=1, keepdim=True).values
    vc = torch.minimum(torch.maximum(v, lo), hi)
    out = torch.empty(v.shape, dtype=torch.int64)
    for r in range(v.shape[0]):
        d = (vc[r].unsqueeze(-1) - cb[r]).abs()
        out[r] = d.argmin(-1)
    out[torch.isnan(v)] = 0
    return out


def codebook_decode_rows(codes, cb):
    """Decode to the table value the reference stores: bf16 of the entry."""
    cbb = cb.to(torch.bfloat16).float()
    return torch.gather(cbb, 1, codes.long())


def linear_mx(x, weight, bias=None, weight_scale=None, block_size=None, weight_code=None):
    """src/vc/ops/quantized.py:295-331 (dense, "kc" layout)."""
    w = weight
    if weight_code is not None:
        w = weight_code[weight.to(torch.long)].to(weight.dtype)
    if weight_scale is not None:
        w = w * expand(weight_scale, weight.shape, block_size)
    return torch.nn.functional.linear(x, w, bias)
