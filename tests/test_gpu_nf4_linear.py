"""GPU: the NF4-dequant-fused linear (C5 shapes scaled down and full) against
the reference's linear_mx semantics (decode to bf16(level * scale), then a
bf16 product with fp32 accumulation), relative tolerance 1e-2."""

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R

Q = torch.ops.quantized_ops


def make_weight(N, K, seed=4):
    g = torch.Generator().manual_seed(seed)
    return (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16)


def decode_reference(codes_u8, scale_f32, N, K):
    lv = R.table_tensor(F.nf_levels(4))
    b = codes_u8.cpu().numpy()
    c = np.empty(N * K, np.int64)
    c[0::2] = b & 0xF
    c[1::2] = b >> 4
    idx = torch.from_numpy(c).reshape(N, K)
    return lv[idx] * R.expand(scale_f32.cpu().to(torch.bfloat16), (N, K), 64)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(256, 128, 64), (256, 128, 128), (256, 128, 192), (256, 256, 320),
                                   (256, 256, 512), (512, 384, 1024), (2048, 11008, 4096)])
def test_nf4_linear_matches_reference(vqx, M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = make_weight(N, K)
    sc, codes = Q.quantize_mx_packed(W.cuda(), "nf4", -1, 64, False, 1.0, "float32")
    out = Q.linear_nf4(A.cuda(), codes, sc, None, 64, "nf4")
    Wd = decode_reference(codes, sc, N, K).cuda()
    # the reference product: bf16 operands, fp32 accumulation (computed in fp32
    # on the GPU from the exact decoded weight), bf16 output
    ref = (A.cuda().float() @ Wd.float().t()).to(torch.bfloat16)
    err = (out.float() - ref.float()).abs()
    tol = 1e-2 * ref.float().abs() + 1e-2 * ref.float().abs().mean()
    frac_bad = (err > tol).float().mean().item()
    rel = (err.norm() / ref.float().norm()).item()
    assert rel < 1e-2 and frac_bad < 1e-3, (rel, frac_bad)


@pytest.mark.gpu
def test_nf4_linear_bias_and_batch(vqx):
    g = torch.Generator().manual_seed(7)
    A = torch.randn(2, 128, 256, generator=g).to(torch.bfloat16)
    W = make_weight(256, 256)
    bias = torch.randn(256, generator=g).to(torch.bfloat16)
    sc, codes = Q.quantize_mx_packed(W.cuda(), "nf4", -1, 64, False, 1.0, "float32")
    out = Q.linear_nf4(A.cuda(), codes, sc, bias.cuda(), 64, "nf4")
    assert out.shape == (2, 128, 256)
    Wd = decode_reference(codes, sc, 256, 256).cuda()
    ref = (A.cuda().float().reshape(-1, 256) @ Wd.float().t() + bias.cuda().float()).reshape(2, 128, 256)
    rel = ((out.float() - ref).norm() / ref.norm()).item()
    assert rel < 1e-2


def check_against_reference(A, W, bias=None):
    M, K = A.shape
    N = W.shape[0]
    sc, codes = Q.quantize_mx_packed(W.cuda(), "nf4", -1, 64, False, 1.0, "float32")
    out = Q.linear_nf4(A.cuda(), codes, sc, None if bias is None else bias.cuda(), 64, "nf4")
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    Wd = decode_reference(codes, sc, N, K).cuda()
    ref = A.cuda().float() @ Wd.float().t()
    if bias is not None:
        ref = ref + bias.cuda().float()
    ref = ref.to(torch.bfloat16).float()
    err = (out.float() - ref).abs()
    tol = 1e-2 * ref.abs() + 1e-2 * ref.abs().mean()
    frac_bad = (err > tol).float().mean().item()
    rel = (err.norm() / ref.norm()).item()
    assert rel < 1e-2 and frac_bad < 1e-3, (rel, frac_bad)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(1, 11008, 4096), (1, 64, 64), (2, 4096, 11008), (3, 200, 512), (4, 130, 256),
                                   (8, 1000, 1024), (16, 4096, 4096), (16, 64, 192), (1, 4096, 4096),
                                   (1, 1024, 4096), (5, 2048, 1984)])
def test_nf4_linear_skinny_matches_reference(vqx, M, N, K):
    # M <= 16: the skinny kernel (any N; K % 64), with 4, 8 or 16 waves per
    # workgroup as N leaves the CUs short of work
    g = torch.Generator().manual_seed(M * 7 + N + K)
    check_against_reference(torch.randn(M, K, generator=g).to(torch.bfloat16), make_weight(N, K, seed=M))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(17, 128, 64), (100, 256, 512), (300, 384, 256), (2047, 512, 1024)])
def test_nf4_linear_partial_row_tile(vqx, M, N, K):
    # M > 16 and not a multiple of 256: the MFMA kernel with a partial last row tile
    g = torch.Generator().manual_seed(M + N + K)
    check_against_reference(torch.randn(M, K, generator=g).to(torch.bfloat16), make_weight(N, K, seed=M))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 5, 33])
def test_nf4_linear_skinny_and_tail_bias(vqx, M):
    g = torch.Generator().manual_seed(M)
    A = torch.randn(M, 256, generator=g).to(torch.bfloat16)
    bias = torch.randn(256, generator=g).to(torch.bfloat16)
    check_against_reference(A, make_weight(256, 256, seed=9), bias)


@pytest.mark.gpu
def test_nf4_linear_rejects_unsupported_shape(vqx):
    # K must be a multiple of the 64-element scale block; N % 128 for M > 16
    A = torch.randn(100, 64).to(torch.bfloat16).cuda()
    W = make_weight(200, 64)
    sc, codes = Q.quantize_mx_packed(W.cuda(), "nf4", -1, 64, False, 1.0, "float32")
    with pytest.raises(RuntimeError, match="nf4_gemm"):
        Q.linear_nf4(A, codes, sc, None, 64, "nf4")


def _nf4_operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    sc, codes = Q.quantize_mx_packed(make_weight(N, K, seed).cuda(), "nf4", -1, 64, False, 1.0, "float32")
    return A, codes, sc


def _whole_tiles(vqx, A, codes, sc, N):
    """The product through the entry point without a workspace (whole tiles)."""
    L = vqx._lib
    M, K = A.shape
    lv = vqx.parse_format("nf4").tables(A.device)["levels_bf16"]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    L.call("vqx_nf4_linear", L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), None, L.ptr(out), M, N, K,
           L.stream_of(A))
    return out


# Shapes whose 256 x 128 tile count is not a multiple of the CU count, so
# linear_nf4 splits the last round's tiles along K (stream-K): 64 and 86
# tiles (no whole-tile launch, counters cleared by their own launch), 258
# full tiles plus a partial row tile, 344 tiles (256 whole, 88 split), and 24
# tiles of a long K.
SK_SHAPES = [(512, 4096, 4096), (256, 11008, 4096), (808, 11008, 4096), (1024, 11008, 4096), (768, 1024, 8192)]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", SK_SHAPES)
def test_nf4_linear_stream_k(vqx, M, N, K):
    print(f"stream-K NF4 linear M={M} N={N} K={K}", flush=True)
    L = vqx._lib
    import ctypes
    n = ctypes.c_int64(0)
    L.call("vqx_nf4_linear_workspace_size", M, N, K, ctypes.byref(n))
    assert n.value > 0  # these shapes do take the split path on a 256-CU device
    A, codes, sc = _nf4_operands(M, N, K, M + K)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(N)).to(torch.bfloat16).cuda()
    # a call on other activations of the same shape first: a workspace slot
    # read before its contributor wrote it would hold that call's sums
    Q.linear_nf4(torch.randn_like(A), codes, sc, bias, 64, "nf4")
    out = Q.linear_nf4(A, codes, sc, bias, 64, "nf4")
    again = Q.linear_nf4(A, codes, sc, bias, 64, "nf4")
    # fixed summation order: identical on every call
    assert torch.equal(out, again)
    Wd = decode_reference(codes, sc, N, K).cuda()
    ref = (A.float() @ Wd.float().t() + bias.float()).to(torch.bfloat16).float()
    err = (out.float() - ref).abs()
    tol = 1e-2 * ref.abs() + 1e-2 * ref.abs().mean()
    assert (err.norm() / ref.norm()).item() < 1e-2 and (err > tol).float().mean().item() < 1e-3
    # against whole tiles: only the grouping of the fp32 sums differs, so the
    # fp32 results are within 2 K u sum|a w| of each other (u = 2^-24) and
    # the bf16 outputs within that plus one bf16 spacing
    whole = _whole_tiles(vqx, A, codes, sc, N)
    out_nb = Q.linear_nf4(A, codes, sc, None, 64, "nf4")
    S = A.float().abs() @ Wd.float().abs().t()
    diff = (out_nb.float() - whole.float()).abs()
    bound = torch.maximum(whole.float().abs(), out_nb.float().abs()) * 2.0 ** -7 + 2 * K * 2.0 ** -24 * S
    assert bool((diff <= bound).all()), float((diff - bound).max())


@pytest.mark.gpu
def test_nf4_linear_ws_rejects_small_workspace(vqx):
    L = vqx._lib
    A, codes, sc = _nf4_operands(512, 4096, 4096, 1)
    lv = vqx.parse_format("nf4").tables(A.device)["levels_bf16"]
    out = torch.empty(512, 4096, dtype=torch.bfloat16, device=A.device)
    ws = torch.empty(1024, dtype=torch.uint8, device=A.device)
    with pytest.raises(ValueError, match="workspace"):
        L.call("vqx_nf4_linear_ws", L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), None, L.ptr(out), 512, 4096, 4096,
               L.ptr(ws), 1024, L.stream_of(A))
    with pytest.raises(ValueError, match="workspace"):
        L.call("vqx_nf4_linear_ws", L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), None, L.ptr(out), 512, 4096, 4096,
               None, 0, L.stream_of(A))
