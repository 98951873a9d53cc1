"""linear_mx / matmul_mx in both weight layouts and conv2d_mx in both
activation layouts on the GPU (src/vc/ops/quantized.py:230-432, layout twins
ops/layout.py:104-200).  The operand decode (code lookup, then the product
with the block-expanded scale) is compared bit for bit with the oracle's; the
product itself is a library GEMM / convolution, so it is compared with a
float64 product of the oracle's decoded operands, within 2^-6 (bf16) or 2^-18
(fp32) of the same product of magnitudes."""

import pytest
import torch

from oracle import reference_ops as R

Q = torch.ops.quantized_ops


def coded(shape, K, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, K, shape, generator=g).to(dtype)


def close(got, want64, bound64, dtype):
    tol = 2.0**-6 if dtype == torch.bfloat16 else 2.0**-18
    err = (got.cpu().double() - want64).abs()
    assert bool((err <= tol * bound64 + 1e-30).all()), float((err - tol * bound64).max())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["kc", "ck"])
@pytest.mark.parametrize("act", [False, True])
def test_linear_mx_layouts(vqx, dtype, layout, act):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 48, 128, generator=g).to(dtype)
    code = torch.linspace(-1, 1, 16).to(dtype)
    w = coded((96, 128), 16, 8, dtype)
    sc = (torch.rand(96, 4, generator=g) + 0.5).to(dtype)
    b = torch.randn(96, generator=g).to(dtype)
    xs, xc = None, None
    if act:  # coded, scaled activations too
        xc = torch.linspace(-3, 3, 256).to(dtype)
        x = coded((2, 48, 128), 256, 9, dtype)
        xs = (torch.rand(2, 48, 4, generator=g) + 0.5).to(dtype)
    wt, st = (w, sc) if layout == "kc" else (w.T.contiguous(), sc.T.contiguous())
    got = Q.linear_mx(x.cuda(), wt.cuda(), b.cuda(), input_scale=None if xs is None else xs.cuda(),
                      weight_scale=st.cuda(), block_size=32, input_code=None if xc is None else xc.cuda(),
                      weight_code=code.cuda(), weight_layout=layout)
    # the decode, bit for bit
    wd = R._decode_mx(wt, code, st, 32)
    dec = vqx.ops.quantized._decode_operand
    assert torch.equal(dec(wt.cuda(), code.cuda(), st.cuda(), 32).cpu(), wd)
    xd = R._decode_mx(x, xc, xs, 32)
    assert torch.equal(dec(x.cuda(), None if xc is None else xc.cuda(), None if xs is None else xs.cuda(),
                           32).cpu(), xd)
    wk = wd if layout == "kc" else wd.T
    want = xd.double() @ wk.double().T + b.double()
    bound = xd.double().abs() @ wk.double().abs().T + b.double().abs()
    assert got.shape == (2, 48, 96) and got.dtype == dtype
    close(got, want, bound, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["ck", "kc"])
def test_matmul_mx_layouts(vqx, dtype, layout):
    g = torch.Generator().manual_seed(11)
    a = torch.randn(3, 40, 64, generator=g).to(dtype)
    code = torch.linspace(-2, 2, 16).to(dtype)
    w = coded((64, 80), 16, 12, dtype)  # [K, N]
    sc = (torch.rand(2, 80, generator=g) + 0.5).to(dtype)
    wt, st = (w, sc) if layout == "ck" else (w.T.contiguous(), sc.T.contiguous())
    got = Q.matmul_mx(a.cuda(), wt.cuda(), weight_scale=st.cuda(), block_size=32, weight_code=code.cuda(),
                      weight_layout=layout)
    wd = R._decode_mx(w, code, sc, 32).double()
    want = a.double() @ wd
    close(got, want, a.double().abs() @ wd.abs(), dtype)
    assert got.shape == (3, 40, 80)


def conv64(x, w, stride, padding, dilation, groups):
    return torch.nn.functional.conv2d(x.double(), w.double(), None, stride, padding, dilation, groups)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
@pytest.mark.parametrize("groups,stride,padding,dilation", [(1, 1, 1, 1), (2, 2, 0, 1), (1, 1, 2, 2)])
def test_conv2d_mx(vqx, dtype, layout, groups, stride, padding, dilation):
    g = torch.Generator().manual_seed(13)
    C, O = 16, 12
    x = torch.randn(2, C, 11, 13, generator=g).to(dtype)
    code = torch.linspace(-1, 1, 16).to(dtype)
    w = coded((O, C // groups, 3, 3), 16, 14, dtype)
    sc = (torch.rand(O, C // groups // 4, 3, 3, generator=g) + 0.5).to(dtype)
    b = torch.randn(O, generator=g).to(dtype)
    if layout == "nchw":
        xin, win, sin = x, w, sc
    else:
        xin = x.permute(0, 2, 3, 1).contiguous()
        win, sin = (w.permute(2, 3, 1, 0).contiguous(), sc.permute(2, 3, 1, 0).contiguous()) if groups == 1 \
            else (w, sc)
    got = torch.ops.quantized_ops.conv2d_mx(xin.cuda(), win.cuda(), b.cuda(), [stride] * 2, [padding] * 2,
                                            [dilation] * 2, groups, weight_scale=sin.cuda(), block_size=4,
                                            weight_code=code.cuda(), layout=layout)
    wd = R._decode_mx(w, code, sc, 4)
    want = conv64(x, wd, stride, padding, dilation, groups) + b.double()[None, :, None, None]
    bound = conv64(x.abs(), wd.abs(), stride, padding, dilation, groups) + b.double().abs()[None, :, None, None]
    if layout == "nhwc":
        want, bound = want.permute(0, 2, 3, 1), bound.permute(0, 2, 3, 1)
    assert got.dtype == dtype and tuple(got.shape) == tuple(want.shape)
    close(got, want, bound, dtype)
