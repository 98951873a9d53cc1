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
                                   (8, 1000, 1024), (16, 4096, 4096), (16, 64, 192)])
def test_nf4_linear_skinny_matches_reference(vqx, M, N, K):
    # M <= 16: the skinny kernel (any N; K % 64)
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
