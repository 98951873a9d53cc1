"""Pins of the oracle's linear_mx / matmul_mx / conv2d_mx restatements
(src/vc/ops/quantized.py:230-432, layout twins ops/layout.py:104-200) on the
CPU: the "ck" / "kc" forms equal the native ones on the transposed operand,
the NHWC conv equals the NCHW conv on permuted operands, a 1x1 conv equals a
per-pixel linear_mx, and the decode is the code lookup by integer value
followed by the product with the block-expanded scale (checked entry by
entry)."""

import torch

from oracle import reference_ops as R


def coded(shape, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, K, shape, generator=g).to(torch.float32)


def test_decode_is_lookup_then_scale():
    code = torch.tensor([-1.5, -0.25, 0.0, 0.5, 2.0])
    w = coded((6, 8), 5, 0)
    sc = torch.rand(6, 2, generator=torch.Generator().manual_seed(1)) + 0.5
    got = R._decode_mx(w, code, sc, 4)
    for r in range(6):
        for c in range(8):
            assert got[r, c] == code[int(w[r, c])] * sc[r, c // 4]


def test_linear_layouts_agree():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, 5, 16, generator=g)
    code = torch.linspace(-1, 1, 16)
    w = coded((12, 16), 16, 3)
    sc = torch.rand(12, 2, generator=g) + 0.5
    b = torch.randn(12, generator=g)
    kc = R.linear_mx(x, w, b, sc, 8, code)
    ck = R.linear_mx(x, w.T.contiguous(), b, sc.T.contiguous(), 8, code, weight_layout="ck")
    assert torch.allclose(kc, ck, atol=1e-6)
    mm_ck = R.matmul_mx(x, w.T.contiguous(), sc.T.contiguous(), 8, code)
    mm_kc = R.matmul_mx(x, w, sc, 8, code, weight_layout="kc")
    assert torch.allclose(mm_ck, kc - b, atol=1e-5) and torch.allclose(mm_kc, mm_ck, atol=1e-6)


def test_conv_layouts_agree_and_1x1_is_linear():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 8, 7, 9, generator=g)
    code = torch.linspace(-2, 2, 16)
    w = coded((6, 8, 3, 3), 16, 5)
    sc = torch.rand(6, 2, 3, 3, generator=g) + 0.5
    nchw = R.conv2d_mx(x, w, None, 1, 1, 1, 1, weight_scale=sc, block_size=4, weight_code=code)
    nhwc = R.conv2d_mx(x.permute(0, 2, 3, 1), w.permute(2, 3, 1, 0), None, 1, 1, 1, 1,
                       weight_scale=sc.permute(2, 3, 1, 0), block_size=4, weight_code=code, layout="nhwc")
    assert torch.allclose(nchw.permute(0, 2, 3, 1), nhwc, atol=1e-5)
    w1, s1 = coded((6, 8, 1, 1), 16, 6), torch.rand(6, 2, 1, 1, generator=g) + 0.5
    conv = R.conv2d_mx(x, w1, None, weight_scale=s1, block_size=4, weight_code=code)
    lin = R.linear_mx(x.permute(0, 2, 3, 1), w1[:, :, 0, 0], None, s1[:, :, 0, 0], 4, code)
    assert torch.allclose(conv.permute(0, 2, 3, 1), lin, atol=1e-5)
