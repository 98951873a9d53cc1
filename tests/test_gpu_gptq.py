"""GPU GPTQ compensation (src/vc/quantization/gptq.py:184-270): the per-block
column loop bit for bit against the oracle; the whole block loop bit for bit
where the factor makes the later-column updates exact; and, with a dense
factor (a library GEMM on each side, summed in different orders), the
Hessian-weighted error of compensate_weight against the oracle's.  The
inverse-Hessian factor (a blockwise factorisation with HIP leaves) is checked
against the oracle's and against float64."""

import types

import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R


def qmap_of(dtype):
    return R.table_tensor(F.quantization_table(dtype))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["int4", "nf4", "fp4_e2m1"])
@pytest.mark.parametrize("rows,cols,start,end", [(300, 64, 0, 64), (257, 128, 64, 81), (64, 32, 31, 32)])
def test_gptq_block_matches_oracle(vqx, dtype, rows, cols, start, end):
    g = torch.Generator().manual_seed(rows + cols + start)
    work = torch.randn(rows, cols, generator=g)
    scale = torch.rand(rows, generator=g) * 0.5 + 0.05
    A = torch.randn(cols, cols, generator=g) * 0.1 + torch.eye(cols)
    hinv = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(A @ A.T + 0.1 * torch.eye(cols))),
                                 upper=True)
    q = qmap_of(dtype)
    want_out, want_d = R.gptq_block(work, scale, hinv, q, start, end)
    out = torch.zeros(rows, cols, device="cuda")
    d = torch.empty(rows, end - start, device="cuda")
    L = vqx._lib
    wk, sc, hv, qm = work.cuda(), scale.cuda(), hinv.contiguous().cuda(), q.cuda()
    L.call("vqx_gptq_block", L.ptr(wk), rows, cols, start, end - start, L.ptr(sc), 0.0, None, L.ptr(hv), cols,
           L.ptr(qm), L.ptr(out), L.ptr(d), end - start, L.stream_of(wk))
    assert torch.equal(out[:, start:end].cpu(), want_out)
    assert torch.equal(d.cpu(), want_d)
    assert torch.equal(wk.cpu(), work)       # the block's columns of work are left as they were


def make_problem(seed, out_f, in_f):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(4 * in_f, in_f, generator=g) @ (torch.randn(in_f, in_f, generator=g) * 0.3 + torch.eye(in_f))
    return (torch.randn(out_f, in_f, generator=g) * 0.05), X.T @ X, 4 * in_f


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,qmax", [("int4", 7.0), ("nf4", 1.0), ("fp4_e2m1", 6.0)])
def test_compensation_with_block_diagonal_factor_is_exact(vqx, dtype, qmax):
    # a factor with exact zeros between blocks makes every later-column update
    # an exact zero on both sides, so the whole compensation is bit-exact
    g = torch.Generator().manual_seed(7)
    # any upper-triangular factor with a positive diagonal will do
    blocks = [torch.triu(torch.randn(64, 64, generator=g) * 0.05, diagonal=1)
              + torch.diag(0.2 + torch.rand(64, generator=g)) for _ in range(3)]
    hinv = torch.block_diag(*blocks)
    w = torch.randn(96, 192, generator=g) * 0.05
    q = qmap_of(dtype)
    fq = types.SimpleNamespace(qmap=q.cuda(), scale_qmap=None, quant_max=qmax, block_size=64, ch_axis=-1)
    got = vqx.quantization.gptq.compensate_with_factor(w.cuda(), hinv.cuda(), hinv.diagonal().cuda(), fq).cpu()
    want = R.gptq_compensate_with_factor(w, hinv, q, qmax, 64)
    assert torch.equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,qmax", [("int4", 7.0), ("nf4", 1.0)])
@pytest.mark.parametrize("act_order", [True, False])
def test_compensate_weight_quality_matches_oracle(vqx, dtype, qmax, act_order):
    # with a dense factor the later-column updates are summed in different
    # orders (GPU and CPU GEMMs), and GPTQ amplifies any difference once a
    # rounding decision flips: compare what the compensation is for, the
    # Hessian-weighted error, against the oracle's and against plain rounding
    w, H, tokens = make_problem(3, 128, 256)
    q = qmap_of(dtype)
    fq = types.SimpleNamespace(qmap=q.cuda(), scale_qmap=None, quant_max=qmax, block_size=64, ch_axis=-1)
    got = vqx.quantization.compensate_weight(w.cuda(), H.cuda(), tokens, fq, 0.01, act_order=act_order).cpu()
    want = R.gptq_compensate_weight(w, H.clone(), tokens, q, qmax, 64, 0.01, act_order=act_order)
    assert got.shape == want.shape and got.dtype == torch.float32

    def err(o):
        e = (w - o).double()
        return torch.einsum("ij,jk,ik->", e, H.double() / tokens, e).item()

    s = R.calculate_mx_qparam(w, [-1], 64, qmax).repeat_interleave(64, dim=1)
    plain = R.vmap((w / s).bfloat16(), q).float() * s
    assert abs(err(got) - err(want)) <= 0.05 * err(want)
    assert err(got) < 0.9 * err(plain)


@pytest.mark.gpu
def test_compensate_weight_shrink_and_scale_codebook(vqx):
    w, H, tokens = make_problem(5, 64, 128)
    fq = types.SimpleNamespace(qmap=qmap_of("int4").cuda(), scale_qmap=qmap_of("fp8_e5m3").cuda(), quant_max=7.0,
                               block_size=64, ch_axis=-1)
    plain = vqx.quantization.compensate_weight(w.cuda(), H.cuda(), tokens, fq, 0.01, shrink=False)
    shrunk = vqx.quantization.compensate_weight(w.cuda(), H.cuda(), tokens, fq, 0.01, shrink=True)
    assert torch.isfinite(plain).all() and torch.isfinite(shrunk).all()

    def err(o):
        e = (w - o.cpu()).double()
        return torch.einsum("ij,jk,ik->", e, H.double() / tokens, e).item()

    assert err(shrunk) <= 1.05 * err(plain)


def hessian_of(seed, n):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(4 * n, n, generator=g) * (torch.rand(n, generator=g) * 2 + 0.1)
    return X.T @ X, 4 * n


@pytest.mark.gpu
@pytest.mark.parametrize("n", [40, 64, 128, 200, 1000])
def test_factor_matches_the_reference_sequence(vqx, n):
    # the factor is unique: the blockwise inverse factor of the reversed
    # Hessian must equal cholesky(cholesky_inverse(cholesky(H)), upper=True)
    H, tokens = hessian_of(n, n)
    got = vqx.quantization.gptq.hessian_inverse_chol(H.cuda(), tokens, 0.01).cpu()
    want = R._hessian_inverse_chol(H.double().clone(), tokens, 0.01)
    assert torch.equal(got, torch.triu(got))
    err = ((got.double() - want).abs().max() / want.abs().max()).item()
    assert err < 2e-5, err


@pytest.mark.gpu
def test_factor_escalates_the_damping_like_the_reference(vqx):
    # one negative diagonal entry: 1% damping leaves H indefinite, 10% does
    # not; both sides escalate to the same damping
    d = torch.ones(96)
    d[5] = -0.05
    H = torch.diag(d) * 50.0
    got = vqx.quantization.gptq.hessian_inverse_chol(H.cuda(), 50, 0.01).cpu()
    want = R._hessian_inverse_chol(H.clone(), 50, 0.01)
    assert torch.allclose(got, want, rtol=1e-6, atol=0)
    with pytest.raises(torch.linalg.LinAlgError):
        vqx.quantization.gptq.hessian_inverse_chol((-torch.eye(70)).cuda(), 1, 0.01)


@pytest.mark.gpu
def test_blocks_wider_than_the_column_loop(vqx):
    # 128-column blocks: one scale per block, the loop in two 64-column
    # pieces; the compensation's error matches the oracle's
    w, H, tokens = make_problem(6, 96, 256)
    q = qmap_of("int4")
    fq = types.SimpleNamespace(qmap=q.cuda(), scale_qmap=None, quant_max=7.0, block_size=128, ch_axis=-1)
    got = vqx.quantization.compensate_weight(w.cuda(), H.cuda(), tokens, fq, 0.01).cpu()
    want = R.gptq_compensate_weight(w, H.clone(), tokens, q, 7.0, 128, 0.01)

    def err(o):
        e = (w - o).double()
        return torch.einsum("ij,jk,ik->", e, H.double() / tokens, e).item()

    assert torch.isfinite(got).all()
    assert abs(err(got) - err(want)) <= 0.05 * err(want)


@pytest.mark.gpu
def test_compensate_weight_at_the_bench_size(vqx):
    # the G1 workload (4096 x 4096 weight, int4 blocks of 64, salience order,
    # Hessian of 16384 tokens): the Hessian-weighted error within 5% of the
    # oracle's and well below plain rounding's
    g = torch.Generator().manual_seed(11)
    C, T = 4096, 16384
    X = torch.randn(T, C, generator=g) * (torch.rand(C, generator=g) * 2 + 0.1)
    H = X.T @ X
    del X
    w = torch.randn(4096, C, generator=g) * 0.02
    q = qmap_of("int4")
    fq = types.SimpleNamespace(qmap=q.cuda(), scale_qmap=None, quant_max=7.0, block_size=64, ch_axis=-1)
    got = vqx.quantization.compensate_weight(w.cuda(), H.cuda(), T, fq, 0.01).cpu()
    want = R.gptq_compensate_weight(w, H.clone(), T, q, 7.0, 64, 0.01)
    Hd = H.double() / T

    def err(o):
        e = (w - o).double()
        return ((e @ Hd) * e).sum().item()

    s = R.calculate_mx_qparam(w, [-1], 64, 7.0).repeat_interleave(64, dim=1)
    plain = R.vmap((w / s).bfloat16(), q).float() * s
    assert torch.isfinite(got).all()
    assert abs(err(got) - err(want)) <= 0.05 * err(want)
    assert err(got) < 0.9 * err(plain)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["int4", "fp4_e2m1"])
def test_gptq_block_special_values(vqx, dtype):
    # NaN, +-Inf, signed zeros and huge values in the block: the column loop
    # propagates them as the reference's torch ops do (NaN compared as a class)
    g = torch.Generator().manual_seed(21)
    rows, cols = 70, 64
    work = torch.randn(rows, cols, generator=g)
    work[3, 5] = float("nan")
    work[7, 0] = float("inf")
    work[9, 63] = float("-inf")
    work[11, 10] = -0.0
    work[12, :] = 0.0
    work[13, 20] = 3e38
    scale = torch.rand(rows, generator=g) * 0.5 + 0.05
    A = torch.randn(cols, cols, generator=g) * 0.1 + torch.eye(cols)
    hinv = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(A @ A.T + 0.1 * torch.eye(cols))),
                                 upper=True)
    q = qmap_of(dtype)
    want_out, want_d = R.gptq_block(work, scale, hinv, q, 0, cols)
    out = torch.zeros(rows, cols, device="cuda")
    d = torch.empty(rows, cols, device="cuda")
    L = vqx._lib
    wk, sc, hv, qm = work.cuda(), scale.cuda(), hinv.contiguous().cuda(), q.cuda()
    L.call("vqx_gptq_block", L.ptr(wk), rows, cols, 0, cols, L.ptr(sc), 0.0, None, L.ptr(hv), cols, L.ptr(qm),
           L.ptr(out), L.ptr(d), cols, L.stream_of(wk))
    for got, want in ((out.cpu(), want_out), (d.cpu(), want_d)):
        same = (got.view(torch.int32) == want.view(torch.int32)) | (torch.isnan(got) & torch.isnan(want))
        assert bool(same.all()), int((~same).sum())


@pytest.mark.gpu
def test_compensate_weight_with_a_fake_quantize_module(vqx):
    # the weight's FakeQuantize module names the grid; one that has not run a
    # forward yet still has its tables built for the compensation
    w, H, tokens = make_problem(8, 64, 128)
    spec = vqx.quantization.QuantizationSpec.from_str("int4,qs=microscaling,bs=64,ax=-1")
    module = spec.make_fake_quantize()
    got = vqx.quantization.compensate_weight(w.cuda(), H.cuda(), tokens, module, 0.01).cpu()
    q = qmap_of("int4")
    fq = types.SimpleNamespace(qmap=q.cuda(), scale_qmap=None, quant_max=7.0, block_size=64, ch_axis=-1)
    want = vqx.quantization.compensate_weight(w.cuda(), H.cuda(), tokens, fq, 0.01).cpu()
    assert module.qmap.numel() == 65536 and module.quant_max == 7.0
    assert torch.equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,qmax", [("int4", 7.0), ("nf4", 1.0)])
@pytest.mark.parametrize("scale_dtype", [None, "fp8_e5m3"])
@pytest.mark.parametrize("rows,cols,start,end", [(300, 128, 64, 128), (70, 64, 0, 50)])
def test_gptq_block_forms_the_block_scale(vqx, dtype, qmax, scale_dtype, rows, cols, start, end):
    # scale NULL: the kernel forms block_scale's plain scale from the block
    # (calculate_mx_qparam of the block, clamped at 1e-12), NaN and zero rows
    # included; deltas written at a row stride wider than the block
    g = torch.Generator().manual_seed(rows + end)
    work = torch.randn(rows, cols, generator=g) * 0.3
    work[1, start + 3] = float("nan")
    work[2, start:end] = 0.0
    A = torch.randn(cols, cols, generator=g) * 0.1 + torch.eye(cols)
    hinv = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(A @ A.T + 0.1 * torch.eye(cols))),
                                 upper=True)
    q = qmap_of(dtype)
    sq = None if scale_dtype is None else qmap_of(scale_dtype)
    scale = R.calculate_mx_qparam(work[:, start:end], [-1], end - start, qmax, False, sq).reshape(-1).clamp_min(1e-12)
    want_out, want_d = R.gptq_block(work, scale, hinv, q, start, end)
    n, ldd = end - start, end - start + 9
    out = torch.zeros(rows, cols, device="cuda")
    dbuf = torch.full((rows, ldd), 7.0, device="cuda")
    L = vqx._lib
    wk, hv, qm = work.cuda(), hinv.contiguous().cuda(), q.cuda()
    sqc = None if sq is None else sq.cuda()
    L.call("vqx_gptq_block", L.ptr(wk), rows, cols, start, n, None, qmax, L.ptr(sqc), L.ptr(hv), cols, L.ptr(qm),
           L.ptr(out), L.ptr(dbuf), ldd, L.stream_of(wk))
    for got, want in ((out[:, start:end].cpu(), want_out), (dbuf[:, :n].cpu(), want_d)):
        same = (got.view(torch.int32) == want.view(torch.int32)) | (torch.isnan(got) & torch.isnan(want))
        assert bool(same.all()), int((~same).sum())
    assert bool((dbuf[:, n:] == 7.0).all())  # the stride's gap is not written
