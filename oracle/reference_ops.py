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
    "convert_weight",
    "AmaxObserverFakeQuantize",
    "OutlierFakeQuantize",
    "codebook_decode_rows",
    "linear_mx",
    "filter_outlier",
    "quantize_mx_outlier",
    "slice_csr_tensor",
    "spmm_csr",
    "csr_to_dense",
    "unit_scale",
    "lcq_histogram_add",
    "gptq_block",
    "gptq_compensate_weight",
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


class AmaxObserverFakeQuantize:
    """The per-tensor / per-channel branch of FusedAmaxObsFakeQuantize
    (src/vc/quantization/fake_quantize.py:219-463) on CPU tensors: state
    (amax_history, scale, the two enable flags) and forward (:404-432), with
    the observer step _update_amax_scale (:308-341) and FakeQuantizeFunction
    (:112-115).  The amax is taken over every axis, or every axis but ch_axis
    when per_channel; the scale comes from the history's maximum before this
    step's amax goes in."""

    def __init__(self, qmap, quant_max, amax_history_len, per_channel=False, ch_axis=None,
                 force_scale_power_of_two=False):
        self.qmap = qmap
        self.quant_max = quant_max
        self.amax_history_len = amax_history_len
        self.per_channel = per_channel
        self.ch_axis = ch_axis
        self.force_scale_power_of_two = force_scale_power_of_two
        self.amax_history = torch.tensor([], dtype=torch.float32)
        self.scale = torch.tensor([1.0], dtype=torch.float32)
        self.observer_enabled = True
        self.fake_quant_enabled = True

    @torch.no_grad()
    def update(self, x):
        """src/vc/quantization/fake_quantize.py:318-341."""
        if self.per_channel:
            ch_axis = self.ch_axis % x.ndim
            dim = tuple(i for i in range(x.ndim) if i != ch_axis)
            amax_cur = torch.amax(torch.abs(x), dim=dim, keepdim=True)
        else:
            amax_cur = torch.amax(torch.abs(x))
        if self.amax_history.numel() == 0:
            self.amax_history = torch.zeros((self.amax_history_len,) + amax_cur.shape, dtype=torch.float32)
            self.scale = torch.ones(amax_cur.shape, dtype=torch.float32)
        amax = torch.amax(self.amax_history, dim=0)
        self.amax_history = torch.roll(self.amax_history, -1, 0)
        self.amax_history[0] = amax_cur
        sf = amax / self.quant_max
        sf = torch.where(amax > 0.0, sf, self.scale)
        sf = torch.where(torch.isfinite(amax), sf, self.scale)
        if self.force_scale_power_of_two:
            sf = torch.pow(2, torch.ceil(torch.log2(sf)))
        self.scale = sf.clone()

    def __call__(self, x):
        """src/vc/quantization/fake_quantize.py:418-426."""
        if self.observer_enabled:
            self.update(x)
        if not self.fake_quant_enabled:
            return x
        return fake_quantize_per_tensor(x, self.qmap, self.scale)


class OutlierFakeQuantize:
    """FusedAmaxObsFakeQuantize.forward's outlier handling (src/vc/
    quantization/fake_quantize.py:373-395, :429-430) around a fake-quant
    step, on CPU tensors, over many forwards: with outlier_pct, the top-k
    threshold of |x| (k = max(1, ceil(pct * numel))) copied into the fp32
    outlier_threshold on the first observed forward, then folded in as
    threshold * decay + value * (1 - decay) (in-place ops on the fp32 buffer,
    the product in x's dtype); the outliers |x| >= threshold masked to 0
    before the fake-quant and put back after it; max_outlier_pct the largest
    count / numel seen.  fake_quant: a callable x -> y (the scheme's
    fake-quant of the masked input), or None when fake-quant is disabled."""

    def __init__(self, outlier_pct=None, outlier_threshold=None, decay=0.9):
        self.outlier_pct = outlier_pct
        self.outlier_ema_decay = decay
        self.outlier_threshold = torch.tensor([], dtype=torch.float32) if outlier_pct is not None \
            else outlier_threshold
        self.max_outlier_pct = 0
        self.observer_enabled = True

    def __call__(self, x, fake_quant):
        if self.outlier_pct is not None and self.observer_enabled:
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
            orig_x = x.clone()
            x = x.masked_fill(skip, 0.0)
            pct = skip.sum().item() / x.numel()
            self.max_outlier_pct = max(pct, self.max_outlier_pct)
        if fake_quant is not None:
            x = fake_quant(x)
        if skip is not None:
            x = torch.where(skip, orig_x, x)
        return x


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


def _decode_mx(t, code, scale, block_size):
    """The operand decode of linear_mx / matmul_mx / conv2d_mx
    (src/vc/ops/quantized.py:263-272, 313-326, 388-398): code lookup by the
    integer value in t's dtype, then the product with the expanded scales."""
    if code is not None:
        t = code[t.to(torch.long)].to(t.dtype)
    if scale is not None:
        t = t * expand(scale, t.shape, block_size)
    return t


def convert_weight(weight, table, axes, block_size, quant_max, force_scale_power_of_two=False, scale_qmap=None):
    """Convert-time quantization of a weight parameter with a codebook-style
    (NF) table, src/vc/quantization/quantize_pt2e.py:456-500: the table's
    distinct values become the code (``unique``), the table becomes an index
    table (``searchsorted``), the scale comes from calculate_mx_qparam and the
    stored weight is quantize() through the index table, i.e. integer-valued
    indices in the weight's dtype.  Returns (weight indices, scale, code)."""
    values = torch.unique(table)
    indices = torch.searchsorted(values, table).to(torch.int64)
    scale = calculate_mx_qparam(weight, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap)
    w = quantize(weight, scale, None, axes, block_size, indices)
    return w, scale, values


def linear_mx(x, weight, bias=None, weight_scale=None, block_size=None, weight_code=None, input_scale=None,
              input_code=None, weight_layout="kc"):
    """src/vc/ops/quantized.py:295-331 (the dense half).  "ck" is the layout
    twin (ops/layout.py:184-198): the weight's last two dims swapped."""
    x = _decode_mx(x, input_code, input_scale, block_size)
    w = _decode_mx(weight, weight_code, weight_scale, block_size)
    if weight_layout == "ck":
        w = w.transpose(-2, -1)
    return torch.nn.functional.linear(x, w, bias)


def matmul_mx(a, other, weight_scale=None, block_size=None, weight_code=None, input_scale=None, input_code=None,
              weight_layout="ck"):
    """src/vc/ops/quantized.py:371-406 (the dense half); "kc" is the layout
    twin with the right matrix's last two dims swapped."""
    a = _decode_mx(a, input_code, input_scale, block_size)
    b = _decode_mx(other, weight_code, weight_scale, block_size)
    if weight_layout == "kc":
        b = b.transpose(-2, -1)
    return torch.matmul(a, b)


def conv2d_mx(x, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, input_scale=None,
              weight_scale=None, block_size=None, input_code=None, weight_code=None, layout="nchw"):
    """src/vc/ops/quantized.py:239-284; "nhwc" is the layout twin
    (ops/layout.py:152-170): NHWC activations, HWIO weight (OIHW when
    grouped), NHWC result."""
    x = _decode_mx(x, input_code, input_scale, block_size)
    w = _decode_mx(weight, weight_code, weight_scale, block_size)
    if layout == "nhwc":
        x = x.permute(0, 3, 1, 2)
        w = w.permute(3, 2, 0, 1) if groups == 1 else w
    out = torch.nn.functional.conv2d(x, w, bias, stride, padding, dilation, groups)
    return out.permute(0, 2, 3, 1) if layout == "nhwc" else out


# ---------------------------------------------------------------------------
# outliers as CSR (src/vc/ops/quantized.py:532-895)
# ---------------------------------------------------------------------------
def _pad_csr(values, cols, crow, max_nnz):
    """src/vc/ops/quantized.py:537-569: pad to max_nnz with 0 / -1, or keep
    the first max_nnz entries and clamp the row pointers (in place)."""
    nse = int(crow[-1])
    if nse <= max_nnz:
        pad = max_nnz - nse
        return (torch.cat([values, values.new_zeros(pad)]),
                torch.cat([cols, cols.new_full((pad,), -1)]))
    crow.clamp_(max=max_nnz)
    return values[:max_nnz], cols[:max_nnz]


def filter_outlier(x, threshold, max_pct=0.01, indptr_offset=0):
    """src/vc/ops/quantized.py:572-630: outliers |x| > threshold (the Python
    scalar compared in x's dtype); per matrix of the last two dims, the CSR of
    the nonzero outliers in row-major order (numpy nonzero), int32 indices,
    padded by _pad_csr; inliers are x with outliers set to 0.  indptr_offset
    is quantize_mx_outlier's shift of the row pointers (:686-687)."""
    is_out = torch.abs(x) > threshold
    inlier = torch.where(is_out, 0, x)
    R, C = x.shape[-2:]
    batch = x.shape[:-2]
    max_nnz = int(math.prod((R, C)) * max_pct)
    xs = x.reshape(-1, R, C)
    keep = (is_out & (x != 0)).reshape(-1, R, C).numpy()
    datas, idxs, ptrs = [], [], []
    for b in range(xs.shape[0]):
        r, c = np.nonzero(keep[b])
        crow = np.zeros(R + 1, dtype=np.int64)
        crow[1:] = np.cumsum(np.bincount(r, minlength=R))
        vals = xs[b][torch.from_numpy(r), torch.from_numpy(c)]
        crow_t = torch.from_numpy(crow.astype(np.int32))
        d, i = _pad_csr(vals, torch.from_numpy(c.astype(np.int32)), crow_t, max_nnz)
        datas.append(d)
        idxs.append(i)
        ptrs.append(crow_t)
    data = torch.stack(datas).reshape(*batch, max_nnz)
    indices = torch.stack(idxs).reshape(*batch, max_nnz)
    indptr = torch.stack(ptrs).reshape(*batch, R + 1)
    if indptr_offset:
        indptr = indptr + indptr_offset
    return data, indices, indptr, inlier


def quantize_mx_outlier(x, qmap, axes, block_size, quant_max, force_scale_power_of_two=False,
                        scale_qmap=None, threshold=None, max_pct=0.01, indptr_offset=0):
    """src/vc/ops/quantized.py:642-691: filter_outlier, then quantize_mx of
    the inliers.  Returns (data, indices, indptr, scale, inliers)."""
    data, indices, indptr, inl = filter_outlier(x, threshold, max_pct, indptr_offset)
    scale, q = quantize_mx(inl, qmap, axes, block_size, quant_max, force_scale_power_of_two, scale_qmap)
    return data, indices, indptr, scale, q


def slice_csr_tensor(data, indices, indptr, dim=0, start=None, end=None, size_factor=1.0):
    """src/vc/ops/quantized.py:722-763 (numpy): rows [start, end) with the
    pointers rebased, or columns [start, end) with per-row counts of the kept
    entries and the indices rebased; then _pad_csr to int(len(data) * size_factor)."""
    dim = dim + 2 if dim < 0 else dim
    if dim not in (0, 1):
        raise ValueError(f"Cannot slice sparse CSR matrix along dim {dim}")
    p = indptr.numpy().astype(np.int64)
    d = data
    ix = indices.numpy()
    if dim == 0:
        s0, e0 = int(p[start]), int(p[end])
        new_ptr = (p[start:end + 1] - s0).astype(np.int32)
        vals = d[s0:e0]
        cols = torch.from_numpy(ix[s0:e0].copy())
    else:
        mask = (ix >= start) & (ix < end)
        nse = int(p[-1])
        counts = np.array([mask[p[r]:p[r + 1]].sum() for r in range(len(p) - 1)], dtype=np.int64)
        assert counts.sum() == mask[:nse].sum()
        new_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        vals = d[torch.from_numpy(mask)]
        cols = torch.from_numpy((ix[mask] - start).astype(ix.dtype))
    new_ptr = torch.from_numpy(new_ptr)
    max_nnz = int(data.shape[0] * size_factor)
    nd, ni = _pad_csr(vals, cols, new_ptr, max_nnz)
    return nd, ni, new_ptr


def csr_to_dense(data, indices, indptr, cols, dtype=None):
    """Dense [rows, cols] matrix of one CSR matrix (rows from indptr, entries
    at positions indptr[r] - indptr[0]); later duplicates overwrite."""
    p = indptr.numpy().astype(np.int64)
    p = p - p[0]
    R = len(p) - 1
    out = torch.zeros((R, cols), dtype=dtype or data.dtype)
    ix = indices.numpy()
    for r in range(R):
        for q in range(p[r], p[r + 1]):
            out[r, int(ix[q])] = data[q]
    return out


def spmm_csr(data, indices, indptr, B, B_scale=None, B_code=None, block_size=None, weight_layout="kc"):
    """src/vc/ops/quantized.py:816-878: decode B (B_code[B.long()], then times
    the expanded scale, in torch's dtypes), transpose a "kc" B to [K, N], then
    per batch the rebased CSR rows times B in fp32 (torch.sparse.mm), cast to
    the decoded B's dtype."""
    if B_code is not None:
        B = B_code[B.to(torch.long)]
    if B_scale is not None:
        B = B * expand(B_scale, B.shape, block_size)
    if weight_layout == "kc":
        B = B.mT
    batch = indptr.shape[:-1]
    nb = int(math.prod(batch))
    ip = indptr.reshape(-1, indptr.shape[-1])
    ix = indices.reshape(-1, indices.shape[-1])
    dt = data.reshape(-1, data.shape[-1])
    if B.ndim > 2:
        B = B.reshape(nb, B.shape[-2], B.shape[-1])
    outs = []
    for i in range(nb):
        Bi = B[i] if B.ndim == 3 else B
        base = int(ip[i][0])
        n = int(ip[i][-1]) - base
        csr = torch.sparse_csr_tensor(ip[i] - base, ix[i, :n], dt[i, :n], dtype=torch.float32,
                                      size=(ip[i].numel() - 1, Bi.shape[0]))
        outs.append(torch.sparse.mm(csr, Bi.to(torch.float32)).to(B.dtype))
    return torch.stack(outs).reshape(*batch, -1, B.shape[-1])


# ---------------------------------------------------------------------------
# learned-codebook calibration statistics (src/vc/quantization/lcq.py)
# ---------------------------------------------------------------------------
def unit_scale(x, block_size, quant_max):
    """src/vc/quantization/lcq.py:136-150: x / (max(block amax, 1e-12) / quant_max), fp32."""
    x = x.float()
    flat = x.reshape(-1, block_size)
    scale = flat.abs().amax(-1, keepdim=True).clamp_min(1e-12) / quant_max
    return (flat / scale).reshape(x.shape)


def lcq_histogram_add(values, weights, quant_min, quant_max, bins=4001, sums=None):
    """src/vc/quantization/lcq.py:77-109 on the CPU: bin by bucketize(right=True)
    over fp32 linspace edges, then fp64 sums of w, w v, (w v) v per bin.
    Returns (weight, total, square), added to ``sums`` when given."""
    if sums is None:
        sums = tuple(torch.zeros(bins, dtype=torch.float64) for _ in range(3))
    edges = torch.linspace(quant_min - 0.5, quant_max + 0.5, bins + 1, dtype=torch.float32)
    index = (torch.bucketize(values, edges, right=True) - 1).clamp_(0, bins - 1)
    v = values.double()
    w = weights.double().expand_as(v)
    sums[0].index_add_(0, index, w)
    sums[1].index_add_(0, index, w * v)
    sums[2].index_add_(0, index, w * v * v)
    return sums


# ---------------------------------------------------------------------------
# GPTQ compensation (src/vc/quantization/gptq.py)
# ---------------------------------------------------------------------------
def gptq_block(work, scale, hinv, qmap, start, end):
    """The column loop of src/vc/quantization/gptq.py:241-262 for one block on
    a private copy of work: returns (out[:, start:end], deltas)."""
    work = work.clone()
    out = torch.zeros(work.shape[0], end - start)
    deltas = torch.zeros(work.shape[0], end - start)
    for offset, column in enumerate(range(start, end)):
        values = work[:, column]
        quantized = vmap((values / scale).bfloat16(), qmap).float() * scale
        out[:, offset] = quantized
        delta = (values - quantized) / hinv[column, column].clamp_min(1e-12)
        deltas[:, offset] = delta
        if column + 1 < end:
            work[:, column + 1:end] -= delta.unsqueeze(1) * hinv[column, column + 1:end].unsqueeze(0)
    return out, deltas


def _hessian_inverse_chol(hessian, tokens, damping):
    """src/vc/quantization/gptq.py:32-71."""
    hessian = hessian / max(tokens, 1)
    damp = damping * hessian.diagonal().mean().clamp_min(1e-12)
    applied = 0
    for escalation in (1, 10, 100, 1000, 10000):
        hessian.diagonal().add_((escalation - applied) * damp)
        applied = escalation
        try:
            chol = torch.linalg.cholesky(hessian)
            return torch.linalg.cholesky(torch.cholesky_inverse(chol), upper=True)
        except torch.linalg.LinAlgError:
            continue
    raise torch.linalg.LinAlgError("Hessian not positive-definite")


def gptq_compensate_weight(weight, hessian, tokens, qmap, quant_max, block_size, damping, act_order=True,
                           within_block=True, scale_qmap=None):
    """src/vc/quantization/gptq.py:184-270 without the shrink search (scale =
    calculate_mx_qparam of the block, clamped at 1e-12), torch CPU fp32."""
    perm = None
    if act_order and weight.shape[1] % block_size == 0:
        blocks = weight.shape[1] // block_size
        diagonal = hessian.diagonal().reshape(blocks, block_size)
        block_order = torch.argsort(diagonal.mean(dim=1), descending=True)
        rank = (torch.argsort(diagonal, dim=1, descending=True) if within_block
                else torch.arange(block_size).expand(blocks, block_size))
        perm = (torch.arange(blocks).unsqueeze(1) * block_size + rank)[block_order].reshape(-1)
        hessian = hessian[perm][:, perm]
        weight = weight[:, perm]
    hinv = _hessian_inverse_chol(hessian, tokens, damping)
    out = gptq_compensate_with_factor(weight, hinv, qmap, quant_max, block_size, scale_qmap)
    if perm is None:
        return out
    restored = torch.empty_like(out)
    restored[:, perm] = out
    return restored


def gptq_compensate_with_factor(weight, hinv, qmap, quant_max, block_size, scale_qmap=None):
    """The block loop of src/vc/quantization/gptq.py:239-265 on columns in
    processing order, given the factor."""
    work = weight.float().clone()
    out = torch.zeros_like(work)
    for start in range(0, weight.shape[1], block_size):
        end = min(start + block_size, weight.shape[1])
        block = work[:, start:end]
        scale = calculate_mx_qparam(block, [-1], block.shape[-1], quant_max, False, scale_qmap).reshape(-1)
        scale = scale.clamp_min(1e-12)
        o, deltas = gptq_block(work, scale, hinv, qmap, start, end)
        out[:, start:end] = o
        if end < weight.shape[1]:
            work[:, end:] -= deltas @ hinv[start:end, end:]
    return out
