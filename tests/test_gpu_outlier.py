"""GPU parity of the outlier path against the CPU oracle (src/vc/ops/quantized.py
:286-895): filter_outlier, quantize_mx_outlier and slice_csr_tensor bit for bit
(CSR data / indices / row pointers, inliers, scales, quantized inliers);
spmm_csr and the dense + sparse linear_mx / matmul_mx within the tolerance of
an fp32 sum taken in another order.  Edge cases: overflowing and zero
capacity, negative / infinite / NaN thresholds, the threshold rounded to the
input dtype, NaN / Inf / signed zeros, odd widths (the element-wise path),
batch dims, row pointers offset into a longer array."""

import ctypes
import math

import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R

Q = torch.ops.quantized_ops


def rand_outliers(shape, dtype, seed, frac=0.03, scale=40.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    m = torch.rand(shape, generator=g) < frac
    return torch.where(m, x * scale, x).to(dtype)


def same(a, b):
    """Equal dtype, shape and bits (every NaN equal to every NaN)."""
    a, b = a.detach().cpu(), b.detach().cpu()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if not a.is_floating_point():
        return torch.equal(a, b)
    iv = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[a.dtype]
    return bool(((a.view(iv) == b.view(iv)) | (torch.isnan(a) & torch.isnan(b))).all())


def check_all(got, want, names):
    for g, w, n in zip(got, want, names):
        assert same(g, w), f"{n}: dtype {g.dtype}/{w.dtype} shape {tuple(g.shape)}/{tuple(w.shape)}"


CSR = ("data", "indices", "indptr", "inlier")


def with_specials(x):
    x = x.clone()
    f = x.reshape(-1)
    if f.numel() >= 6:
        f[:6] = torch.tensor([float("nan"), float("inf"), -float("inf"), -0.0, 0.0, -5000.0]).to(x.dtype)
    return x


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(64, 256), (3, 40, 72), (2, 2, 17, 33), (5, 3), (1, 1), (7, 1000), (4, 5000)])
@pytest.mark.parametrize("thr,pct", [(3.0, 0.01), (3.0, 0.5), (2.0, 0.0), (-1.0, 1.0)])
def test_filter_outlier_matches_oracle(vqx, dtype, shape, thr, pct):
    x = with_specials(rand_outliers(shape, dtype, seed=sum(shape)))
    got = Q.filter_outlier(x.cuda(), thr, pct)
    want = R.filter_outlier(x, thr, pct)
    check_all(got, want, CSR)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("thr", [float("inf"), float("nan"), 0.0, 1e30])
def test_filter_outlier_extreme_thresholds(vqx, dtype, thr):
    x = with_specials(rand_outliers((12, 64), dtype, seed=3))
    check_all(Q.filter_outlier(x.cuda(), thr, 0.25), R.filter_outlier(x, thr, 0.25), CSR)


@pytest.mark.gpu
def test_filter_outlier_threshold_rounds_to_input_dtype(vqx):
    # bf16(1.005) == 1.0078125, so 1.0078125 is not an outlier; a threshold a
    # hair above the bf16 midpoint 1.00390625 rounds through fp32 onto it and
    # then to 1.0 (ties to even), so it is
    x = torch.tensor([[1.0078125, -1.0078125, 1.0, 0.5] * 16], dtype=torch.bfloat16)
    for thr in (1.005, 1.00390625 + 2.0**-40, 1.0):
        check_all(Q.filter_outlier(x.cuda(), thr, 1.0), R.filter_outlier(x, thr, 1.0), CSR)
    d, i, p, _ = Q.filter_outlier(x.cuda(), 1.00390625 + 2.0**-40, 1.0)
    assert int(p[-1]) == 32


@pytest.mark.gpu
def test_filter_outlier_full_size_round_trip(vqx):
    # the bench shape: placing the CSR entries back into the inliers rebuilds
    # the input, per-row counts match a dense count, pointers are monotone
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(8192, 4096, device="cuda", generator=g).to(torch.bfloat16)
    x[torch.rand(8192, 4096, device="cuda", generator=g) < 0.005] *= 64
    thr = 6.0
    data, idx, ptr, inl = Q.filter_outlier(x, thr, 0.01)
    out = (x.abs() > thr) & (x != 0)
    counts = out.sum(1)
    assert int(counts.sum()) <= data.numel()
    assert torch.equal(ptr[1:] - ptr[:-1], counts.to(torch.int32))
    n = int(ptr[-1])
    rows = torch.repeat_interleave(torch.arange(8192, device="cuda"), counts)
    rec = inl.clone()
    rec[rows, idx[:n].long()] = data[:n]
    assert torch.equal(rec.view(torch.int16), x.view(torch.int16))
    assert bool((inl[out] == 0).all()) and bool((idx[n:] == -1).all())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,qmax", [("fp8_e4m3", 448.0), ("int8", 127.0), ("fp4_e2m1", 6.0)])
@pytest.mark.parametrize("pow2", [True, False])
@pytest.mark.parametrize("offset", [0, 1000])
def test_quantize_mx_outlier_matches_oracle(vqx, dtype, qmax, pow2, offset):
    x = rand_outliers((2, 32, 256), torch.bfloat16, seed=5)
    qm = vqx.get_quantization_map(dtype, "cuda")
    got = Q.quantize_mx_outlier(x.cuda(), qm, [-1], 32, qmax, pow2, None, None, 3.0, 0.02, offset)
    want = R.quantize_mx_outlier(x, R.table_tensor(F.quantization_table(dtype)), [-1], 32, qmax, pow2,
                                 threshold=3.0, max_pct=0.02, indptr_offset=offset)
    check_all(got, want, ("data", "indices", "indptr", "scale", "inliers"))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,start,end,sf", [(0, 0, 48, 1.0), (0, 8, 30, 1.0), (0, 5, 5, 1.0), (0, -20, -3, 0.5),
                                              (1, 16, 48, 1.0), (1, 0, 80, 0.25), (1, 70, 200, 2.0),
                                              (-1, 5, 6, 1.0)])
def test_slice_csr_matches_oracle(vqx, dtype, dim, start, end, sf):
    x = rand_outliers((48, 80), dtype, seed=6, frac=0.08)
    d, i, p, _ = R.filter_outlier(x, 2.5, max_pct=0.3)
    got = Q.slice_csr_tensor(d.cuda(), i.cuda(), p.cuda(), dim, start, end, sf)
    want = R.slice_csr_tensor(d, i, p, dim, start, end, sf)
    check_all(got, want, ("data", "indices", "indptr"))


@pytest.mark.gpu
def test_slice_csr_of_an_overflowed_csr(vqx):
    x = rand_outliers((40, 64), torch.bfloat16, seed=7, frac=0.3)
    d, i, p, _ = R.filter_outlier(x, 1.0, max_pct=0.05)     # truncated, pointers clamped
    for dim, s, e in ((0, 3, 33), (1, 10, 50)):
        check_all(Q.slice_csr_tensor(d.cuda(), i.cuda(), p.cuda(), dim, s, e, 1.0),
                  R.slice_csr_tensor(d, i, p, dim, s, e, 1.0), ("data", "indices", "indptr"))


def assert_spmm_close(got, want, bound, what):
    """|got - want| within two roundings of the output dtype plus the fp32
    order-of-summation error (bound = sum of |a * b| per output)."""
    eps = {torch.float32: 2.0**-24, torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11}[want.dtype]
    got, want, bound = got.cpu().double(), want.double(), bound.double()
    err = (got - want).abs()
    tol = 2 * eps * want.abs() + 64 * 2.0**-24 * bound + 2.0**-24
    assert bool((err <= tol).all()), f"{what}: max excess {float((err - tol).max())}"


def spmm_bound(data, idx, ptr, Bd, layout):
    """sum |a| |B| per output (float64), Bd the decoded B."""
    W = Bd.double().abs()
    W = W.mT if layout == "kc" else W
    nb = math.prod(ptr.shape[:-1])
    p2, i2, d2 = ptr.reshape(nb, -1), idx.reshape(nb, -1), data.reshape(nb, -1)
    outs = []
    for b in range(nb):
        A = R.csr_to_dense(d2[b], i2[b], p2[b], W.shape[-2], dtype=torch.float64).abs()
        outs.append(A @ (W[b] if W.ndim == 3 else W))
    return torch.stack(outs).reshape(*ptr.shape[:-1], -1, W.shape[-1])


@pytest.mark.gpu
@pytest.mark.parametrize("bdt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["kc", "ck"])
@pytest.mark.parametrize("N", [256, 40, 7, 4624])
def test_spmm_plain_matches_oracle(vqx, bdt, layout, N):
    x = rand_outliers((3, 24, 96), torch.bfloat16, seed=N, frac=0.1)
    d, i, p, _ = R.filter_outlier(x, 2.0, max_pct=0.3)
    g = torch.Generator().manual_seed(1)
    B = torch.randn((N, 96) if layout == "kc" else (96, N), generator=g).to(bdt)
    got = Q.spmm_csr(d.cuda(), i.cuda(), p.cuda(), B.cuda(), None, None, None, layout)
    want = R.spmm_csr(d, i, p, B, None, None, None, layout)
    assert got.dtype == want.dtype == bdt and got.shape == want.shape
    assert_spmm_close(got, want, spmm_bound(d, i, p, B, layout), f"{bdt} {layout} N={N}")


@pytest.mark.gpu
def test_spmm_more_items_than_resident_waves(vqx):
    """Rows x column slices well beyond the resident grid: each XCD's run of
    the slice-major item sequence is taken by its waves in several passes,
    and the runs' ends fall inside slices."""
    x = rand_outliers((1, 3000, 96), torch.bfloat16, seed=11, frac=0.1)
    d, i, p, _ = R.filter_outlier(x, 2.0, max_pct=0.3)
    g = torch.Generator().manual_seed(2)
    B = torch.randn(96, 4104, generator=g).to(torch.bfloat16)
    got = Q.spmm_csr(d.cuda(), i.cuda(), p.cuda(), B.cuda(), None, None, None, "ck")
    want = R.spmm_csr(d, i, p, B, None, None, None, "ck")
    assert_spmm_close(got, want, spmm_bound(d, i, p, B, "ck"), "3000 rows, N=4104")


@pytest.mark.gpu
@pytest.mark.parametrize("code_dt,scale_dt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                              (torch.bfloat16, torch.float32), (None, torch.bfloat16),
                                              (torch.float16, None)])
@pytest.mark.parametrize("layout", ["kc", "ck"])
def test_spmm_decoded_weight_matches_oracle(vqx, code_dt, scale_dt, layout):
    x = rand_outliers((2, 20, 128), torch.bfloat16, seed=9, frac=0.1)
    d, i, p, _ = R.filter_outlier(x, 2.0, max_pct=0.3)
    g = torch.Generator().manual_seed(2)
    N, K, bs = 72, 128, 32
    shape = (N, K) if layout == "kc" else (K, N)
    code = None if code_dt is None else torch.randn(16, generator=g).to(code_dt)
    B = torch.randint(0, 16, shape, generator=g).to(torch.bfloat16)
    if code is None:
        B = torch.randn(shape, generator=g).to(torch.bfloat16)
    scale = None
    if scale_dt is not None:
        sshape = (N, K // bs) if layout == "kc" else (K // bs, N)
        scale = torch.rand(sshape, generator=g).add(0.25).to(scale_dt)
    got = Q.spmm_csr(d.cuda(), i.cuda(), p.cuda(), B.cuda(), None if scale is None else scale.cuda(),
                     None if code is None else code.cuda(), bs, layout)
    want = R.spmm_csr(d, i, p, B, scale, code, bs, layout)
    assert got.dtype == want.dtype and got.shape == want.shape
    Bd = B if code is None else code[B.long()]
    if scale is not None:
        Bd = Bd * R.expand(scale, B.shape, bs)
    assert_spmm_close(got, want, spmm_bound(d, i, p, Bd, layout), f"code {code_dt} scale {scale_dt} {layout}")


@pytest.mark.gpu
def test_spmm_batched_weight_and_offset_rows(vqx):
    x = rand_outliers((4, 16, 64), torch.float32, seed=12, frac=0.1)
    d, i, p, _ = R.filter_outlier(x, 2.0, max_pct=0.3)
    g = torch.Generator().manual_seed(3)
    B = torch.randn(4, 64, 40, generator=g)
    got = Q.spmm_csr(d.cuda(), i.cuda(), p.cuda(), B.cuda(), weight_layout="ck")
    want = R.spmm_csr(d, i, p, B, weight_layout="ck")
    assert_spmm_close(got, want, spmm_bound(d, i, p, B, "ck"), "batched B")
    # the quantize_mx_outlier form: pointers offset, data holding only the span
    n = int(p[0, -1])
    got2 = Q.spmm_csr(d[0, :n].contiguous().cuda(), i[0, :n].contiguous().cuda(), (p[0] + 500).cuda(),
                      B[0].cuda(), weight_layout="ck")
    assert torch.equal(got2.cpu(), got[0].cpu())


@pytest.mark.gpu
def test_linear_mx_with_outliers(vqx):
    # dense inliers + CSR outliers through one linear_mx call, against the
    # oracle's dense linear plus spmm (the dense product is hipBLASLt's, so
    # the comparison allows the bf16 GEMM's rounding)
    g = torch.Generator().manual_seed(4)
    x = rand_outliers((2, 32, 128), torch.bfloat16, seed=13, frac=0.05)
    d, i, p, inl = R.filter_outlier(x, 3.0, max_pct=0.1)
    code = torch.linspace(-1, 1, 16).to(torch.bfloat16)
    W = torch.randint(0, 16, (64, 128), generator=g).to(torch.bfloat16)
    sc = torch.rand(64, 4, generator=g).add(0.5).to(torch.bfloat16)
    got = Q.linear_mx(inl.cuda(), W.cuda(), None, weight_scale=sc.cuda(), block_size=32, weight_code=code.cuda(),
                      A_data=d.cuda(), A_indices=i.cuda(), A_indptr=p.cuda())
    Wd = (code[W.long()] * R.expand(sc, W.shape, 32)).double()
    ref64 = x.double() @ Wd.T
    bound = x.double().abs() @ Wd.abs().T
    assert got.dtype == torch.bfloat16 and got.shape == (2, 32, 64)
    err = (got.cpu().double() - ref64).abs()
    assert bool((err <= 2.0**-6 * bound).all()), float((err - 2.0**-6 * bound).max())
    # the sparse half alone, through matmul_mx's "ck" form
    got_ck = Q.matmul_mx(torch.zeros_like(inl).cuda(), W.T.contiguous().cuda(), weight_scale=sc.T.contiguous().cuda(),
                         block_size=32, weight_code=code.cuda(), A_data=d.cuda(), A_indices=i.cuda(),
                         A_indptr=p.cuda())
    sp = R.spmm_csr(d, i, p, W.T.contiguous(), sc.T.contiguous(), code, 32, "ck")
    assert_spmm_close(got_ck, sp, spmm_bound(d, i, p, Wd.T, "ck"), "matmul_mx sparse half")


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [8, 16, 64])
@pytest.mark.parametrize("scale_dtype", [None, "fp8_e5m3"])
@pytest.mark.parametrize("pow2", [True, False])
def test_quantize_mx_outlier_fused_block_sizes(vqx, bs, scale_dtype, pow2):
    # the one-pass form (bf16, blocks along the last axis): every block size
    # it takes, scale codebook, special values in the input
    x = with_specials(rand_outliers((3, 24, 384), torch.bfloat16, seed=11 + bs))
    qm = vqx.get_quantization_map("fp8_e4m3", "cuda")
    sq = None if scale_dtype is None else vqx.get_quantization_map(scale_dtype, "cuda")
    got = Q.quantize_mx_outlier(x.cuda(), qm, [-1], bs, 448.0, pow2, sq, None, 4.0, 0.05, 7)
    sq_o = None if scale_dtype is None else R.table_tensor(F.quantization_table(scale_dtype))
    want = R.quantize_mx_outlier(x, R.table_tensor(F.quantization_table("fp8_e4m3")), [-1], bs, 448.0, pow2,
                                 scale_qmap=sq_o, threshold=4.0, max_pct=0.05, indptr_offset=7)
    check_all(got, want, ("data", "indices", "indptr", "scale", "inliers"))


@pytest.mark.gpu
def test_quantize_mx_outlier_fused_equals_two_pass_at_bench_size(vqx):
    # O2: the fused split against filter_outlier followed by quantize_mx
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4096, 11008, generator=g)
    x = torch.where(torch.rand(4096, 11008, generator=g) < 0.005, x * 32, x).to(torch.bfloat16).cuda()
    qm = vqx.get_quantization_map("fp8_e4m3", "cuda")
    fused = Q.quantize_mx_outlier(x, qm, [-1], 32, 448.0, True, None, None, 6.0, 0.01, 0)
    d, i, p, inl = vqx.ops.quantized._outlier_csr(x, 6.0, 0.01, 0)
    s, v = Q.quantize_mx(inl, qm, [-1], 32, 448.0, True)
    for a, b in zip(fused, (d, i, p, s, v)):
        assert same(a, b)


# ---------------------------------------------------------------------------
# one-pass entry points (staged outliers) against the two-pass ones, through
# the C ABI: default staging, none (every row with outliers read again) and
# three slots per row (some rows staged, some read again)
# ---------------------------------------------------------------------------
def _csr_buffers(x, max_nnz):
    nb = math.prod(x.shape[:-2])
    R = x.shape[-2]
    return (torch.full((nb, max_nnz), 7, dtype=x.dtype, device=x.device),
            torch.full((nb, max_nnz), 7, dtype=torch.int32, device=x.device),
            torch.full((nb, R + 1), 7, dtype=torch.int32, device=x.device))


def _workspace(vqx, x, max_nnz, slots):
    L = vqx._lib
    nb, (R, C) = math.prod(x.shape[:-2]), x.shape[-2:]
    if slots is None:
        n = ctypes.c_int64(0)
        L.call("vqx_outlier_workspace_size", L.dtype_tag(x.dtype), nb, R, C, max_nnz, ctypes.byref(n))
        size = n.value
    else:
        size = (nb * R * 4 + 255) // 256 * 256 + nb * R * slots * (4 + x.element_size())
    return torch.empty(max(size, 1), dtype=torch.uint8, device=x.device), size


def _filter(vqx, x, thr, max_nnz, offset, slots="two-pass"):
    L = vqx._lib
    nb, (R, C) = math.prod(x.shape[:-2]), x.shape[-2:]
    data, idx, ptr = _csr_buffers(x, max_nnz)
    inl = torch.full_like(x, 3.0)
    args = (L.ptr(x), L.dtype_tag(x.dtype), nb, R, C, thr, max_nnz, offset, L.ptr(data), L.ptr(idx), L.ptr(ptr),
            L.ptr(inl))
    if slots == "two-pass":
        L.call("vqx_filter_outlier", *args, L.stream_of(x))
    else:
        ws, size = _workspace(vqx, x, max_nnz, slots)
        L.call("vqx_filter_outlier_ws", *args, L.ptr(ws), size, L.stream_of(x))
    return data, idx, ptr, inl


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(3, 40, 72), (64, 256), (2, 7, 1001), (300, 96), (1, 5)])
@pytest.mark.parametrize("slots", [None, 0, 3])
def test_filter_outlier_one_pass_equals_two_pass(vqx, dtype, shape, slots):
    x = with_specials(rand_outliers(shape, dtype, seed=sum(shape) + 1, frac=0.05)).cuda()
    per = math.prod(shape[-2:])
    for pct, offset in [(0.01, 0), (0.5, 7), (0.0, 0), (1.0, -(1 << 31))]:
        max_nnz = int(per * pct)
        print(f"one-pass filter {dtype} {shape} slots={slots} max_nnz={max_nnz} offset={offset}", flush=True)
        want = _filter(vqx, x, 3.0, max_nnz, offset)
        got = _filter(vqx, x, 3.0, max_nnz, offset, slots)
        check_all(got, want, CSR)


@pytest.mark.gpu
def test_filter_outlier_one_pass_dense_rows_and_many_rows(vqx):
    # rows all outliers (more than the largest default staging); 16384 rows
    # per batch, the most the one-pass form takes (64-row chunks in its
    # second launch), and 17000, which the _ws entry point hands to the
    # two-pass form (its finalize reads would grow as rows^2)
    x = rand_outliers((2, 40, 3000), torch.bfloat16, seed=4)
    x[0, 5] = 100.0
    x[1, 39, 1000:] = -100.0
    x = x.cuda()
    for pct in (0.5, 0.02):
        max_nnz = int(40 * 3000 * pct)
        check_all(_filter(vqx, x, 3.0, max_nnz, 0, None), _filter(vqx, x, 3.0, max_nnz, 0), CSR)
    for rows in (16384, 17000):
        y = rand_outliers((2, rows, 64), torch.bfloat16, seed=6, frac=0.01).cuda()
        for slots in (None, 1):
            check_all(_filter(vqx, y, 3.0, int(rows * 64 * 0.01), 5, slots),
                      _filter(vqx, y, 3.0, int(rows * 64 * 0.01), 5), CSR)


def _qmx(vqx, x, qm, bs, pow2, sq, thr, max_nnz, offset, slots="two-pass"):
    L = vqx._lib
    nb, (R, C) = math.prod(x.shape[:-2]), x.shape[-2:]
    data, idx, ptr = _csr_buffers(x, max_nnz)
    scale = torch.full((*x.shape[:-1], C // bs), 3.0, dtype=x.dtype, device=x.device)
    values = torch.full_like(x, 3.0)
    args = (L.ptr(x), nb, R, C, thr, max_nnz, offset, bs, 0 if pow2 else 1, 8 if pow2 else 0, 448.0, L.ptr(sq),
            L.ptr(qm), L.ptr(data), L.ptr(idx), L.ptr(ptr), L.ptr(scale), L.ptr(values))
    if slots == "two-pass":
        L.call("vqx_quantize_mx_outlier", *args, L.stream_of(x))
    else:
        ws, size = _workspace(vqx, x, max_nnz, slots)
        L.call("vqx_quantize_mx_outlier_ws", *args, L.ptr(ws), size, L.stream_of(x))
    return data, idx, ptr, scale, values


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [8, 32, 64])
@pytest.mark.parametrize("slots", [None, 0, 2])
@pytest.mark.parametrize("fmt", ["fp8_e4m3", "fp4_e2m1", "int8"])
def test_quantize_mx_outlier_one_pass_equals_two_pass(vqx, bs, slots, fmt):
    x = with_specials(rand_outliers((3, 24, 384), torch.bfloat16, seed=21 + bs, frac=0.05)).cuda()
    qm = vqx.ops.quantized._table_bf16(vqx.get_quantization_map(fmt, "cuda"))
    for pow2, pct, offset in [(True, 0.02, 0), (False, 0.5, 11), (True, 0.0, 3)]:
        max_nnz = int(24 * 384 * pct)
        print(f"one-pass quantize_mx_outlier {fmt} bs={bs} slots={slots} pow2={pow2} max_nnz={max_nnz}", flush=True)
        want = _qmx(vqx, x, qm, bs, pow2, None, 4.0, max_nnz, offset)
        got = _qmx(vqx, x, qm, bs, pow2, None, 4.0, max_nnz, offset, slots)
        check_all(got, want, ("data", "indices", "indptr", "scale", "values"))
