"""GPU parity of the group-wise affine fake-quant (GroupWiseAffineFakeQuantFunction,
src/vc/quantization/fake_quantize.py:162-216) against the CPU oracle, bit for
bit: scale, zero point and output, bf16 and fp32 inputs, blocks along any
axis, short (zero-padded) last blocks, NaN / Inf, scale_qmap, and the
FakeQuantize module's group_wise_affine path."""

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R


def same(a, b):
    """Bit equality with NaN as a class."""
    a, b = a.cpu(), b.cpu()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    nan = torch.isnan(a) & torch.isnan(b)
    ai = a.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32)
    bi = b.view(torch.int16 if b.dtype == torch.bfloat16 else torch.int32)
    return bool(((ai == bi) | nan).all())


def gwa_inputs(shape, dt, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * torch.exp(torch.randn(*shape, generator=g))
    return x.to(dt)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape,axis,bs", [((64, 256), -1, 64), ((8, 100), -1, 32), ((4, 37, 6), 1, 8),
                                           ((33, 5), 0, 16), ((3, 7), -1, 64), ((16, 128), -1, 8),
                                           ((16, 96), -1, 16)])
@pytest.mark.parametrize("qrange", [(0, 3), (-8, 7), (0, 255)])
def test_gwa_fake_quant_matches_oracle(vqx, dt, shape, axis, bs, qrange):
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    x = gwa_inputs(shape, dt, seed=sum(shape) + bs)
    qmin, qmax = qrange
    sf, zp, y = qops.gwa_fake_quantize(x.cuda(), axis, bs, qmin, qmax)
    rsf, rzp, ry = R.group_wise_affine_fake_quant(x, axis, bs, qmin, qmax)
    assert same(sf, rsf) and same(zp, rzp), "scale / zero point"
    assert same(y, ry), f"{int((y.cpu() != ry).sum())} outputs differ"


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_gwa_special_values_and_scale_qmap(vqx, dt):
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    x = gwa_inputs((12, 64), dt, seed=5)
    x[0, 3] = float("nan")
    x[1, 0] = float("inf")
    x[2, 5] = -float("inf")
    x[3] = 2.5                                   # constant block: sf -> 1
    x[4, :32] = 0.0
    x[5] = torch.linspace(-1e-30, 1e-30, 64).to(dt)   # tiny range
    for sq in (None, R.table_tensor(F.quantization_table("fp8_e5m3"))):
        sf, zp, y = qops.gwa_fake_quantize(x.cuda(), -1, 32, 0, 3, None if sq is None else sq.cuda())
        rsf, rzp, ry = R.group_wise_affine_fake_quant(x, -1, 32, 0, 3, sq)
        assert same(sf, rsf) and same(zp, rzp) and same(y, ry)


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [32, 64])
def test_gwa_scale_qmap_rounding_scale_to_zero(vqx, bs):
    # blocks of exact zeros plus values below fp8_e5m3's subnormals: the
    # scale codebook rounds sf to 0, so a zero element gives 0 / 0 = NaN and
    # the output keeps it (torch.clamp propagates NaN), while the nonzero
    # elements give (qmax - zp) * 0.  Mixed with ordinary blocks in the same
    # waves, so the fast path of those waves must step aside too.
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    g = torch.Generator().manual_seed(23)
    rows = []
    for r in range(32):
        if r % 3 == 0:
            row = torch.zeros(128)
            row[torch.randint(0, 128, (5,), generator=g)] = torch.rand(5, generator=g) * 1e-6
        elif r % 3 == 1:
            row = torch.where(torch.rand(128, generator=g) < 0.5, 0.0, torch.rand(128, generator=g) * 3e-6)
        else:
            row = torch.randn(128, generator=g)
        rows.append(row)
    x = torch.stack(rows).to(torch.bfloat16)
    sq = R.table_tensor(F.quantization_table("fp8_e5m3"))
    sf, zp, y = qops.gwa_fake_quantize(x.cuda(), -1, bs, 0, 3, sq.cuda())
    rsf, rzp, ry = R.group_wise_affine_fake_quant(x, -1, bs, 0, 3, sq)
    assert bool(torch.isnan(ry).any()), "the case needs NaN outputs"
    assert same(sf, rsf) and same(zp, rzp), "scale / zero point"
    assert same(y, ry), f"{int((~((y.cpu() == ry) | (torch.isnan(y.cpu()) & torch.isnan(ry)))).sum())} outputs differ"


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [8, 64])
def test_gwa_quotients_near_and_below_the_normal_range(vqx, bs):
    # bf16 blocks whose quotients x / scale fall among the bf16 subnormals
    # (where rounding midpoints can be hit exactly), whose scale is itself
    # subnormal or infinite, and blocks of mixed magnitudes from 2^-140 to
    # 2^100, against the oracle's IEEE divisions
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    g = torch.Generator().manual_seed(17)
    sub = 2.0 ** -133
    rows = [
        torch.cat([torch.tensor([1.0]), torch.arange(1, 64) * sub]),              # subnormal quotients
        torch.cat([torch.tensor([3.0 * 2 ** -126]), torch.arange(1, 64) * sub]),  # ties near 2^-126
        torch.randint(-100, 100, (64,), generator=g) * sub,                      # subnormal scale
        torch.tensor([3e38, -3e38] * 32),                                          # range overflows
        torch.tensor([1.5 * 2 ** -120] + [float(k) * 2 ** -130 for k in range(63)]),
    ]
    for _ in range(27):
        e = torch.randint(-140, 100, (64,), generator=g).float()
        sgn = torch.where(torch.rand(64, generator=g) < 0.5, -1.0, 1.0)
        rows.append(sgn * torch.exp2(e) * (1 + torch.rand(64, generator=g)))
    x = torch.stack(rows).to(torch.bfloat16)
    sf, zp, y = qops.gwa_fake_quantize(x.cuda(), -1, bs, 0, 3)
    rsf, rzp, ry = R.group_wise_affine_fake_quant(x, -1, bs, 0, 3)
    assert same(sf, rsf) and same(zp, rzp), "scale / zero point"
    assert same(y, ry), f"{int((y.cpu().float() != ry.float()).sum())} outputs differ"


@pytest.mark.gpu
def test_gwa_fakequantize_module(vqx):
    """FusedAmaxObsFakeQuantize with qscheme group_wise_affine (uint2 KV-cache
    style, fake_quantize.py:409-420): output and the scale / zero_point buffers."""
    fq_mod = vqx.quantization.FusedAmaxObsFakeQuantize
    m = fq_mod("uint2", qscheme=vqx.quantization.QScheme.GROUP_WISE_AFFINE, quant_min=0, quant_max=3,
               ch_axis=-1, block_size=64, device="cuda")
    x = gwa_inputs((2, 8, 128), torch.bfloat16, seed=9)
    y = m(x.cuda())
    rsf, rzp, ry = R.group_wise_affine_fake_quant(x, -1, 64, 0, 3)
    assert same(y, ry)
    assert torch.equal(m.scale.cpu(), rsf.float()) and torch.equal(m.zero_point.cpu(), rzp.float())
    xg = x.cuda().requires_grad_(True)
    m(xg).sum().backward()
    assert torch.equal(xg.grad, torch.ones_like(xg))


@pytest.mark.gpu
def test_gwa_bench_shape_bit_exact(vqx):
    # the bench's F3 workload: C2's bf16 [4096, 11008] input, uint2, blocks of
    # 64 along the last axis (the coalesced last-axis kernel)
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    g = torch.Generator().manual_seed(1)
    x = (0.02 * torch.randn(4096, 11008, generator=g)).to(torch.bfloat16)
    sf, zp, y = qops.gwa_fake_quantize(x.cuda(), -1, 64, 0, 3)
    rsf, rzp, ry = R.group_wise_affine_fake_quant(x, -1, 64, 0, 3)
    assert same(sf.cpu(), rsf) and same(zp.cpu(), rzp) and same(y.cpu(), ry)
