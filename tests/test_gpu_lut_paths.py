"""GPU: the compact-table kernels and the closed-form kernels agree bit for
bit (both are also checked against the oracle elsewhere), on random data and
on the edge cases the table path treats specially: signed zeros, quotients
that round to a bf16 zero, subnormal inputs, huge blocks, Inf/NaN."""

import math

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R
from tests.conftest import assert_bitexact

FORMATS = [("fp8_e4m3", 448.0), ("fp6_e3m2", 28.0), ("fp4_e2m1", 6.0), ("fp8_e5m2", 57344.0),
           ("int8", 127.0), ("int4", 7.0), ("posit8_1", 4096.0), ("nf4", 1.0), ("nf4_6", 31.0),
           ("e4m3", 448.0), ("uint8", 255.0)]


def tricky_rows(cols=256):
    g = torch.Generator().manual_seed(11)
    r = torch.randn(16, cols, generator=g) * torch.logspace(-3, 3, 16).unsqueeze(1)
    r[0, :] = 0.0
    r[0, 1::2] = -0.0
    r[1, 0] = 2.0**100
    r[1, 1:8] = torch.tensor([-2.0**-40, -2.0**-42, -2.0**-43, 2.0**-42, -3 * 2.0**-44, -2.0**-41, 1e-30])
    r[2, :] = 2.0**-130
    r[2, 5] = -2.0**-128
    r[3, 0] = 0.01
    r[3, 1:20] = -(2.0 ** -torch.arange(120, 139).float())
    r[4, 3] = float("nan")
    r[5, 9] = float("inf")
    r[6, 0] = 3.0e38
    r[7, :] = -(2.0**-126)
    r[8, 0] = 1.0
    r[8, 1:] = -(2.0**-10) * torch.rand(cols - 1, generator=g)
    # huge amax: absmax quotients of the small negatives run from fp32 normals
    # through fp32 subnormals to zero (sign of the rounded zero)
    r[9, :] = 0.0
    r[9, 0] = 2.0**60
    r[9, 1:60] = -(2.0 ** -torch.arange(70, 129).float())
    r[9, 64] = 2.0**60
    r[9, 65:124] = 2.0 ** -torch.arange(70, 129).float()
    return r.to(torch.bfloat16)


def run_mx(vqx, x, fmt, qmax, pow2, lut, bs):
    L = vqx._lib
    f = vqx.parse_format(fmt)
    desc = f.desc(x.device, lut=lut)
    rows, cols = x.shape
    sc = torch.empty(rows, cols // bs, dtype=torch.bfloat16, device=x.device)
    qv = torch.empty_like(x)
    fq = torch.empty_like(x)
    codes = torch.empty(x.numel() * f.code_bits // 8, dtype=torch.uint8, device=x.device)
    shift = math.floor(math.log2(qmax)) if pow2 else 0
    L.call("vqx_mx_quantize", L.ptr(x), L.BF16, rows, cols, 1, bs, L.ctypes.byref(desc), 0 if pow2 else 1,
           shift, float(qmax), None, L.ptr(sc), None, None, L.ptr(qv), L.ptr(fq), None, 1, L.stream_of(x))
    L.call("vqx_mx_quantize", L.ptr(x), L.BF16, rows, cols, 1, bs, L.ctypes.byref(desc), 0 if pow2 else 1,
           shift, float(qmax), None, None, None, None, None, None, L.ptr(codes), 0, L.stream_of(x))
    return sc, qv, fq, codes


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,qmax", FORMATS)
@pytest.mark.parametrize("pow2", [True, False])
@pytest.mark.parametrize("bs", [32, 64])
def test_mx_lut_equals_closed_form_and_oracle(vqx, fmt, qmax, pow2, bs):
    g = torch.Generator().manual_seed(5)
    x = torch.cat([(torch.randn(48, 256, generator=g) * 3).to(torch.bfloat16), tricky_rows()]).cuda()
    if vqx.parse_format(fmt).code_bits not in (4, 6, 8):
        pytest.skip("packed widths 4/6/8 only")
    a = run_mx(vqx, x, fmt, qmax, pow2, True, bs)
    b = run_mx(vqx, x, fmt, qmax, pow2, False, bs)
    for u, v, what in zip(a, b, ["scale", "values", "fake-quant", "codes"]):
        assert_bitexact(u.cpu() if u.dtype != torch.uint8 else u.cpu().float(),
                        v.cpu() if v.dtype != torch.uint8 else v.cpu().float(), f"{fmt} {what}")
    xc = x.cpu()
    qm = R.table_tensor(F.quantization_table(fmt))
    ws, wq = R.quantize_mx(xc, qm, [-1], bs, qmax, pow2)
    assert_bitexact(a[0].cpu(), ws, f"{fmt} oracle scale")
    assert_bitexact(a[1].cpu(), wq, f"{fmt} oracle values")
    assert_bitexact(a[2].cpu(), wq * R.expand(ws, wq.shape, bs), f"{fmt} oracle fake-quant")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["posit8_1", "fp8_e4m3", "int8", "nf4", "fp4_e2m1", "e5m2", "posit8_2"])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_fake_quant_lut_equals_closed_form(vqx, fmt, dt):
    L = vqx._lib
    f = vqx.parse_format(fmt)
    allp = torch.from_numpy(F.bf16_to_f32(F.ALL_BF16))
    g = torch.Generator().manual_seed(9)
    # fp32 values around the -2^-134 boundary between rounding to -0 and to
    # the smallest negative bf16 subnormal, and between bf16 neighbours
    t = 2.0**-134
    edge = torch.tensor([-t, -t * (1 + 2.0**-20), -t * (1 - 2.0**-20), -2 * t, -1e-45, t * (1 + 2.0**-20),
                         -1.5 * 2.0**-126, 1.0 + 2.0**-8, -(1.0 + 3 * 2.0**-9), 3.0e38, -3.3e38, 3.39e38])
    x = torch.cat([allp, torch.randn(4099, generator=g) * 10, edge]).to(dt).cuda()
    for scale in (None, torch.tensor([0.3], device="cuda"), torch.tensor([4.0], device="cuda")):
        outs = []
        for lut in (True, False):
            y = torch.empty_like(x)
            c = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
            L.call("vqx_fake_quant", L.ptr(x), L.dtype_tag(dt), x.numel(), L.ctypes.byref(f.desc(x.device, lut)),
                   L.ptr(scale), 1, 1, 1, L.ptr(y), L.ptr(c), 1, L.stream_of(x))
            outs.append((y.cpu(), c.cpu()))
        assert_bitexact(outs[0][0], outs[1][0], f"{fmt} {dt} values")
        assert torch.equal(outs[0][1], outs[1][1]), f"{fmt} {dt} codes"
        t = R.table_tensor(F.quantization_table(fmt))
        s = torch.tensor([1.0]) if scale is None else scale.cpu()
        assert_bitexact(outs[0][0], R.fake_quantize_per_tensor(x.cpu(), t, s), f"{fmt} {dt} oracle")
