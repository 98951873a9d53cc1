"""GPU: linear_mx / matmul_mx on the operands convert_pt2e writes
(src/vc/quantization/quantize_pt2e.py:456-508 and the rewrite at :592-645):
the weight as integer-valued code indices in a bf16 tensor, the 16 NF4 levels
as weight_code, bf16 scales per 64-element block along K.  These calls run
the fused dequant MFMA product (the packed operands are built once per weight
and cached); the result is compared with the oracle's linear_mx / matmul_mx
(the reference's decode, then torch CPU bf16 F.linear / matmul) within
relative tolerance 1e-2, as north_star states for GEMM outputs."""

import contextlib

import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R

Q = torch.ops.quantized_ops


def nf4_table():
    return R.table_tensor(F.quantization_table("nf4"))


def convert_format(N, K, seed, transposed=False):
    """A bf16 weight N(0, 0.02) [N, K] quantized as convert_pt2e does for
    "nf4,qs=microscaling,bs=64,ax=-1": (bf16 indices, bf16 scale, bf16 code).
    transposed: the same operands stored for the "ck" layout, [K, N] and
    [K/64, N]."""
    g = torch.Generator().manual_seed(seed)
    w = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16)
    idx, scale, code = R.convert_weight(w, nf4_table(), [-1], 64, 1.0)
    if transposed:
        idx, scale = idx.t().contiguous(), scale.t().contiguous()
    return idx, scale, code


def random_convert_format(N, K, seed, transposed=False):
    """Random operands of the same format at sizes where quantizing a real
    weight on the CPU would be slow: uniform indices 0..15, bf16 scales."""
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, 16, (N, K), generator=g).to(torch.bfloat16)
    scale = (torch.rand(N, K // 64, generator=g) * 0.05 + 0.001).to(torch.bfloat16)
    code = torch.unique(nf4_table())
    if transposed:
        idx, scale = idx.t().contiguous(), scale.t().contiguous()
    return idx, scale, code


def within_tolerance(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    assert got.shape == want.shape, (got.shape, want.shape)
    err = (got - want).abs()
    tol = 1e-2 * want.abs() + 1e-2 * want.abs().mean()
    rel = (err.norm() / want.norm()).item()
    frac_bad = (err > tol).float().mean().item()
    assert rel < 1e-2 and frac_bad < 1e-3, (rel, frac_bad)


@contextlib.contextmanager
def fused_only():
    """Make the unfused paths (decode + library GEMM) fail inside the block,
    so a passing call proves the fused kernel ran."""
    def refuse(*a, **k):
        raise AssertionError("the unfused decode + library GEMM path ran")
    saved = torch.nn.functional.linear, torch.matmul
    torch.nn.functional.linear, torch.matmul = refuse, refuse
    try:
        yield
    finally:
        torch.nn.functional.linear, torch.matmul = saved


def test_convert_weight_is_the_nf4_index_table():
    # the convert format's code and index table restate the reference's
    # unique + searchsorted of the nf4 table (quantize_pt2e.py:457-466)
    table = nf4_table()
    w, s, code = R.convert_weight(torch.tensor([[0.5, -1.0] * 32], dtype=torch.bfloat16), table, [-1], 64, 1.0)
    assert code.numel() == 16 and bool((code[1:] > code[:-1]).all())
    assert torch.equal(code, R.table_tensor(F.nf_levels(4)).sort().values)
    assert float(s) == 1.0
    # index k decodes to the level the fake-quant table gives
    assert torch.equal(code[w.long()].reshape(-1), R.vmap(torch.tensor([0.5, -1.0] * 32), table).to(torch.bfloat16))


@pytest.mark.gpu
def test_linear_mx_fused_c5_shape(vqx):
    """The drop-in check at the full C5 shape: a bf16 weight [11008, 4096]
    quantized to NF4 blocks of 64 as convert_pt2e writes it (index weight,
    weight_code, weight_scale; quantize_pt2e.py:456-508), then the
    reference's own op, torch.ops.quantized_ops.linear_mx, on A bf16
    [2048, 4096] through the fused kernel, against the oracle's linear_mx."""
    print("linear_mx fused M=2048 N=11008 K=4096 (convert-format weight)", flush=True)
    M, N, K = 2048, 11008, 4096
    g = torch.Generator().manual_seed(4)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    idx, scale, code = convert_format(N, K, 4)
    with fused_only():
        out = Q.linear_mx(A.cuda(), idx.cuda(), None, weight_scale=scale.cuda(), weight_code=code.cuda(), block_size=64)
    assert out.dtype == torch.bfloat16 and out.shape == (M, N)
    within_tolerance(out, R.linear_mx(A, idx, None, scale, 64, code))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(1, 11008, 4096), (16, 11008, 4096), (5, 200, 512), (300, 384, 1024),
                                   (256, 11008, 4096)])
def test_linear_mx_fused_matches_oracle(vqx, M, N, K):
    # M <= 16 runs the skinny kernel (any N), larger M the tile kernel, with
    # a partial row tile (300) or the stream-K split (256 x 11008)
    print(f"linear_mx fused M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + N)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    idx, scale, code = random_convert_format(N, K, M + K)
    with fused_only():
        out = Q.linear_mx(A.cuda(), idx.cuda(), None, weight_scale=scale.cuda(), weight_code=code.cuda(), block_size=64)
    within_tolerance(out, R.linear_mx(A, idx, None, scale, 64, code))


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["kc", "ck"])
def test_linear_mx_fused_real_weight_bias_batch(vqx, layout):
    # a weight quantized as convert_pt2e does, batched activations, a bias
    print(f"linear_mx fused real weight layout={layout}", flush=True)
    N, K = 512, 1024
    ck = layout == "ck"
    idx, scale, code = convert_format(N, K, 3, transposed=ck)
    g = torch.Generator().manual_seed(5)
    A = torch.randn(2, 96, K, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    with fused_only():
        out = Q.linear_mx(A.cuda(), idx.cuda(), bias.cuda(), weight_scale=scale.cuda(), weight_code=code.cuda(),
                          block_size=64, weight_layout=layout)
    assert out.shape == (2, 96, N)
    want = R.linear_mx(A, idx, bias, scale, 64, code, weight_layout=layout)
    within_tolerance(out, want)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["ck", "kc"])
@pytest.mark.parametrize("shape", [(64, 1024), (3, 40, 1024), (1024,)])
def test_matmul_mx_fused(vqx, layout, shape):
    # matmul_mx's right operand [K, N] ("ck", its default) or [N, K] ("kc");
    # 1-D, 2-D and batched left operands
    print(f"matmul_mx fused layout={layout} shape={shape}", flush=True)
    K, N = 1024, 384
    idx, scale, code = convert_format(N, K, 8, transposed=layout == "ck")
    a = torch.randn(*shape, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    with fused_only():
        out = Q.matmul_mx(a.cuda(), idx.cuda(), weight_scale=scale.cuda(), weight_code=code.cuda(), block_size=64,
                          weight_layout=layout)
    want = R.matmul_mx(a, idx, scale, 64, code, weight_layout=layout)
    assert out.shape == want.shape
    within_tolerance(out, want)


@pytest.mark.gpu
def test_linear_mx_fused_short_code_and_negative_indices(vqx):
    # a 9-entry code (fewer than 16 levels), indices as the reference reads
    # them: truncated toward zero, negative ones counting from the end
    N, K, M = 256, 256, 32
    g = torch.Generator().manual_seed(11)
    code = torch.linspace(-1, 1, 9).to(torch.bfloat16)
    raw = torch.randint(-9, 9, (N, K), generator=g).float()
    raw = raw + torch.where(raw >= 0, 0.25, -0.25) * (torch.rand(N, K, generator=g) < 0.3)
    idx = raw.to(torch.bfloat16)
    scale = (torch.rand(N, K // 64, generator=g) + 0.5).to(torch.bfloat16)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    with fused_only():
        out = Q.linear_mx(A.cuda(), idx.cuda(), None, weight_scale=scale.cuda(), weight_code=code.cuda(), block_size=64)
    within_tolerance(out, R.linear_mx(A, idx, None, scale, 64, code))


@pytest.mark.gpu
def test_linear_mx_out_of_range_index_takes_unfused_path(vqx):
    # the reference raises IndexError on an index past the code table; the
    # packing reports it and the call decodes without the fused kernel, the
    # bad entry as NaN (only the outputs that read it)
    N, K, M = 128, 128, 32
    idx, scale, code = random_convert_format(N, K, 12)
    idx[5, 7] = 16.0
    A = torch.randn(M, K, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    out = Q.linear_mx(A.cuda(), idx.cuda(), None, weight_scale=scale.cuda(), weight_code=code.cuda(), block_size=64)
    o = out.float().cpu()
    assert bool(torch.isnan(o[:, 5]).all())
    keep = torch.ones(N, dtype=torch.bool)
    keep[5] = False
    ok = idx.clone()
    ok[5, 7] = 0.0
    within_tolerance(o[:, keep], R.linear_mx(A, ok, None, scale, 64, code)[:, keep])


@pytest.mark.gpu
def test_linear_mx_fused_repacks_after_weight_update(vqx):
    # the packed operands are cached per weight and rebuilt when the weight,
    # its code or its scale change in place (version counters)
    N, K, M = 256, 512, 64
    idx, scale, code = random_convert_format(N, K, 13)
    A = torch.randn(M, K, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    w, s, c = idx.cuda(), scale.cuda(), code.cuda()
    with fused_only():
        first = Q.linear_mx(A, w, None, weight_scale=s, weight_code=c, block_size=64)
        assert torch.equal(first, Q.linear_mx(A, w, None, weight_scale=s, weight_code=c, block_size=64))
    w[:, :64] = 15.0
    s.mul_(2)
    with fused_only():
        second = Q.linear_mx(A, w, None, weight_scale=s, weight_code=c, block_size=64)
    idx2 = idx.clone()
    idx2[:, :64] = 15.0
    within_tolerance(second, R.linear_mx(A.cpu(), idx2, None, scale * 2, 64, code))


@pytest.mark.gpu
def test_linear_mx_unfusable_operands_still_match(vqx):
    # fp32 scales make the reference's decoded weight fp32: with fp32
    # activations the call runs (decode + library GEMM) and matches the
    # oracle; the fused kernel is not used
    N, K, M = 128, 128, 16
    idx, scale, code = random_convert_format(N, K, 14)
    A = torch.randn(M, K, generator=torch.Generator().manual_seed(3))
    out = Q.linear_mx(A.cuda(), idx.cuda(), None, weight_scale=scale.float().cuda(), weight_code=code.cuda(),
                      block_size=64)
    want = R.linear_mx(A, idx, None, scale.float(), 64, code)
    assert out.dtype == want.dtype == torch.float32
    assert torch.allclose(out.cpu(), want, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
def test_linear_mx_fused_offset_views(vqx):
    # activations cut from a flat buffer at an odd element offset and a bias
    # sliced at an offset that is not a multiple of 4 elements: contiguous
    # views whose storage is not 16- (A) or 8-byte (bias) aligned still run
    # fused and match the oracle
    N, K, M = 256, 512, 48
    idx, scale, code = random_convert_format(N, K, 15)
    g = torch.Generator().manual_seed(16)
    flat = torch.randn(M * K + 3, generator=g).to(torch.bfloat16).cuda()
    x = flat[3:].view(M, K)
    bflat = torch.randn(N + 5, generator=g).to(torch.bfloat16).cuda()
    bias = bflat[5:]
    assert x.data_ptr() % 16 and bias.data_ptr() % 8
    with fused_only():
        out = Q.linear_mx(x, idx.cuda(), bias, weight_scale=scale.cuda(), weight_code=code.cuda(), block_size=64)
    within_tolerance(out, R.linear_mx(x.cpu(), idx, bias.cpu(), scale, 64, code))


@pytest.mark.gpu
def test_linear_mx_fused_under_inference_mode(vqx):
    # operands made under torch.inference_mode carry no version counter; the
    # packed-weight cache keys them on their storage and the call runs fused,
    # twice (the second from the cache)
    N, K, M = 256, 512, 32
    idx, scale, code = random_convert_format(N, K, 17)
    A = torch.randn(M, K, generator=torch.Generator().manual_seed(18)).to(torch.bfloat16)
    with torch.inference_mode():
        w, s, c, a = idx.cuda(), scale.cuda(), code.cuda(), A.cuda()
        assert w.is_inference()
        with fused_only():
            first = Q.linear_mx(a, w, None, weight_scale=s, weight_code=c, block_size=64)
            second = Q.linear_mx(a, w, None, weight_scale=s, weight_code=c, block_size=64)
    assert torch.equal(first, second)
    within_tolerance(first, R.linear_mx(A, idx, None, scale, 64, code))
