"""Pins of the CSR oracle (filter_outlier, quantize_mx_outlier, slice_csr_tensor,
spmm_csr; src/vc/ops/quantized.py:532-895) on the CPU.

The reference's tests hold no vectors for these ops, so the oracle is pinned
by what the mathematics and torch's own sparse routines fix:
- filter_outlier's CSR equals torch's ``to_sparse_csr`` of the outlier matrix,
  and placing the entries back into the inliers rebuilds the input bit for bit;
- on overflow the entries are a prefix of the roomy CSR and the pointers the
  clamped roomy pointers;
- a row slice / column slice densifies to the dense slice, slices compose;
- spmm_csr agrees with a float64 dense product of the densified matrix, the
  weight decode with a per-element loop, and a CSR lifted out of a longer array
  (row pointers not starting at 0) gives the same product as the plain one.
"""

import math

import numpy as np
import pytest
import torch

from oracle import reference_ops as R


def rand_outliers(shape, dtype, seed, frac=0.03, scale=40.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    m = torch.rand(shape, generator=g) < frac
    return torch.where(m, x * scale, x).to(dtype)


def bits_equal(a, b):
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    iv = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[a.dtype]
    return bool(((a.view(iv) == b.view(iv)) | (torch.isnan(a) & torch.isnan(b))).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_filter_outlier_is_torch_to_sparse_csr(dtype):
    x = rand_outliers((3, 40, 70), dtype, seed=1)
    data, idx, ptr, inl = R.filter_outlier(x, 4.0, max_pct=0.5)
    assert data.dtype == dtype and idx.dtype == torch.int32 and ptr.dtype == torch.int32
    assert data.shape == (3, 1400) and ptr.shape == (3, 41)
    for b in range(3):
        csr = torch.where(torch.abs(x[b]) > 4.0, x[b], torch.zeros((), dtype=dtype)).to_sparse_csr()
        n = int(csr.crow_indices()[-1])
        assert n > 0
        assert torch.equal(ptr[b], csr.crow_indices().to(torch.int32))
        assert torch.equal(idx[b, :n], csr.col_indices().to(torch.int32))
        assert bits_equal(data[b, :n], csr.values())
        assert bool((idx[b, n:] == -1).all()) and bool((data[b, n:] == 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_filter_outlier_round_trip(dtype):
    x = rand_outliers((2, 33, 50), dtype, seed=2)
    x[0, 0, :4] = torch.tensor([float("nan"), float("inf"), -float("inf"), -0.0])
    data, idx, ptr, inl = R.filter_outlier(x, 3.0, max_pct=1.0)
    rec = inl.clone()
    for b in range(2):
        p = ptr[b].long()
        for r in range(33):
            for q in range(int(p[r]), int(p[r + 1])):
                assert inl[b, r, int(idx[b, q])] == 0
                rec[b, r, int(idx[b, q])] = data[b, q]
    assert bits_equal(rec, x)
    # NaN is never an outlier; +-Inf always is
    assert torch.isnan(inl[0, 0, 0]) and inl[0, 0, 1] == 0 and inl[0, 0, 2] == 0


def test_filter_outlier_overflow_keeps_a_prefix():
    x = rand_outliers((2, 30, 64), torch.bfloat16, seed=3, frac=0.1)
    big = R.filter_outlier(x, 2.0, max_pct=1.0)
    small = R.filter_outlier(x, 2.0, max_pct=0.02)
    cap = int(30 * 64 * 0.02)
    assert small[0].shape == (2, cap)
    assert int(big[2][:, -1].min()) > cap  # both matrices overflow
    assert bits_equal(small[0], big[0][:, :cap])
    assert torch.equal(small[1], big[1][:, :cap])
    assert torch.equal(small[2], big[2].clamp(max=cap))
    assert bits_equal(small[3], big[3])


def test_filter_outlier_negative_threshold_and_offset():
    x = torch.tensor([[0.0, -0.0, 1.0], [2.0, 0.0, -3.0]])
    data, idx, ptr, inl = R.filter_outlier(x, -1.0, max_pct=1.0, indptr_offset=7)
    # zeros compare as outliers but are not stored; their inliers become +0
    assert ptr.tolist() == [7, 8, 10]
    assert idx.tolist()[:3] == [2, 0, 2] and data.tolist()[:3] == [1.0, 2.0, -3.0]
    assert bool((inl == 0).all()) and not bool(torch.signbit(inl).any())


def dense_of(data, idx, ptr, cols):
    return R.csr_to_dense(data, idx, ptr, cols)


def test_slice_rows_and_cols_densify_to_dense_slices():
    x = rand_outliers((48, 80), torch.float32, seed=4, frac=0.08)
    data, idx, ptr, _ = R.filter_outlier(x, 2.5, max_pct=0.5)
    dense = dense_of(data, idx, ptr, 80)
    d0, i0, p0 = R.slice_csr_tensor(data, idx, ptr, 0, 8, 30)
    assert d0.shape == data.shape and p0.shape == (23,)
    assert torch.equal(dense_of(d0, i0, p0, 80), dense[8:30])
    d1, i1, p1 = R.slice_csr_tensor(data, idx, ptr, 1, 16, 48)
    assert p1.shape == ptr.shape
    assert torch.equal(dense_of(d1, i1, p1, 32), dense[:, 16:48])
    d01, i01, p01 = R.slice_csr_tensor(d0, i0, p0, -1, 16, 48)
    assert torch.equal(dense_of(d01, i01, p01, 32), dense[8:30, 16:48])
    # padding past the kept entries
    n = int(p1[-1])
    assert bool((i1[n:] == -1).all()) and bool((d1[n:] == 0).all())


def test_slice_overflow_truncates_and_clamps():
    x = rand_outliers((40, 64), torch.float32, seed=5, frac=0.2)
    data, idx, ptr, _ = R.filter_outlier(x, 1.0, max_pct=1.0)
    full = R.slice_csr_tensor(data, idx, ptr, 1, 0, 40, size_factor=1.0)
    cap = int(data.shape[0] * 0.05)
    assert int(full[2][-1]) > cap
    small = R.slice_csr_tensor(data, idx, ptr, 1, 0, 40, size_factor=0.05)
    assert torch.equal(small[0], full[0][:cap]) and torch.equal(small[1], full[1][:cap])
    assert torch.equal(small[2], full[2].clamp(max=cap))


def decode_loop(B, code, scale, bs):
    """decode of spmm_csr element by element: bf16(code[int(b)] * scale[n, k // bs])."""
    out = torch.empty(B.shape, dtype=torch.float64)
    for n in range(B.shape[0]):
        for k in range(B.shape[1]):
            v = float(code[int(B[n, k])]) * float(scale[n, k // bs])
            out[n, k] = float(torch.tensor(v, dtype=torch.float32).to(torch.bfloat16))
    return out


def test_spmm_matches_float64_dense_product_and_decode_loop():
    x = rand_outliers((2, 24, 40), torch.bfloat16, seed=6, frac=0.1)
    data, idx, ptr, _ = R.filter_outlier(x, 2.0, max_pct=0.5)
    g = torch.Generator().manual_seed(7)
    code = torch.linspace(-1, 1, 16).to(torch.bfloat16)
    Bc = torch.randint(0, 16, (30, 40), generator=g).to(torch.bfloat16)    # "kc": [N, K]
    scale = torch.rand(30, 5, generator=g).add(0.5).to(torch.bfloat16)
    out = R.spmm_csr(data, idx, ptr, Bc, scale, code, 8, "kc")
    assert out.shape == (2, 24, 30) and out.dtype == torch.bfloat16
    W = decode_loop(Bc, code, scale, 8)                                      # [N, K] float64
    for b in range(2):
        A = dense_of(data[b], idx[b], ptr[b], 40).double()
        want = A @ W.T
        tol = 2.0**-7 * want.abs() + 1e-6 * (A.abs() @ W.abs().T)
        assert bool(((out[b].double() - want).abs() <= tol).all())


def test_spmm_ck_layout_and_rebased_rows():
    x = rand_outliers((20, 32), torch.float32, seed=8, frac=0.15)
    data, idx, ptr, _ = R.filter_outlier(x, 2.0, max_pct=0.5)
    g = torch.Generator().manual_seed(9)
    B = torch.randn(32, 12, generator=g)                                     # "ck": [K, N]
    out = R.spmm_csr(data, idx, ptr, B, weight_layout="ck")
    A = dense_of(data, idx, ptr, 32).double()
    assert torch.allclose(out.double(), A @ B.double(), rtol=1e-5, atol=1e-5)
    # the same rows lifted out of a longer array: pointers start at 100
    n = int(ptr[-1])
    out2 = R.spmm_csr(data[:n], idx[:n], ptr + 100, B, weight_layout="ck")
    assert torch.equal(out2, out)
    # "kc" of the transposed weight is the same product
    out3 = R.spmm_csr(data, idx, ptr, B.T.contiguous(), weight_layout="kc")
    assert torch.equal(out3, out)


def test_quantize_mx_outlier_is_filter_then_quantize_mx():
    from oracle import formats as F

    x = rand_outliers((16, 64), torch.bfloat16, seed=10)
    qmap = R.table_tensor(F.int_table(8, True))
    d, i, p, s, q = R.quantize_mx_outlier(x, qmap, [-1], 32, 127.0, threshold=3.0, max_pct=0.1, indptr_offset=5)
    d0, i0, p0, inl = R.filter_outlier(x, 3.0, 0.1)
    assert torch.equal(p, p0 + 5) and torch.equal(i, i0) and bits_equal(d, d0)
    s2, q2 = R.quantize_mx(inl, qmap, [-1], 32, 127.0)
    assert bits_equal(s, s2) and bits_equal(q, q2)
    assert int(math.prod(q.shape)) == 16 * 64
