"""GPU learned-codebook calibration histogram (Histogram.add and the fused
unit_scale + add of _accumulate, src/vc/quantization/lcq.py:44-150, 603-626)
against the CPU oracle: bin counts exact, fp64 moments to 1e-10 relative
(only the order of the fp64 additions differs)."""

import math

import pytest
import torch

from oracle import reference_ops as R


def assert_sums(got, want, what):
    for g, w, name in zip(got, want, ("weight", "total", "square")):
        g = g.cpu()
        assert g.dtype == torch.float64 and g.shape == w.shape, name
        nan = torch.isnan(w)
        assert torch.equal(torch.isnan(g), nan), f"{what} {name}: NaN bins differ"
        assert torch.allclose(g[~nan], w[~nan], rtol=1e-10, atol=1e-9), f"{what} {name}"


def hist(vqx, qmin, qmax, bins):
    return vqx.quantization.Histogram(qmin, qmax, bins)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bins", [11, 4001])
def test_histogram_add_matches_oracle(vqx, dtype, bins):
    g = torch.Generator().manual_seed(bins)
    edges = torch.linspace(-7.5, 7.5, bins + 1, dtype=torch.float32)
    v = torch.cat([torch.randn(200_000, generator=g) * 3, edges, edges.nextafter(torch.tensor(100.0)),
                   torch.tensor([float("inf"), -float("inf"), 1e6, -1e6, -0.0])]).to(dtype)
    w = torch.rand(v.numel(), generator=g)
    h = hist(vqx, -7.0, 7.0, bins)
    h.add(v.cuda(), w.cuda())
    want = R.lcq_histogram_add(v.float(), w, -7.0, 7.0, bins)
    assert torch.equal(h.weight.cpu() != 0, want[0] != 0)
    assert_sums((h.weight, h.total, h.square), want, f"{dtype} bins={bins}")
    # counts with unit weights are exact whatever the order
    h1 = hist(vqx, -7.0, 7.0, bins)
    h1.add(v.cuda(), torch.ones((), device="cuda"))
    assert torch.equal(h1.weight.cpu(), R.lcq_histogram_add(v.float(), torch.ones(()), -7.0, 7.0, bins)[0])


@pytest.mark.gpu
def test_histogram_nan_and_accumulation(vqx):
    v = torch.tensor([float("nan"), 0.5, 3.0, -9.0] * 64)
    h = hist(vqx, 0.0, 3.0, 7)
    h.add(v.cuda(), torch.ones(()))
    h.add(v.cuda() * 0.5, torch.full((), 2.0))
    want = R.lcq_histogram_add(v, torch.ones(()), 0.0, 3.0, 7)
    want = R.lcq_histogram_add(v * 0.5, torch.full((), 2.0), 0.0, 3.0, 7, sums=want)
    assert_sums((h.weight, h.total, h.square), want, "nan + two calls")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,bs,qmax", [((64, 256), 32, 7.0), ((4, 33, 64), 64, 15.0), ((8, 96), 16, 3.0)])
def test_fused_unit_scale_matches_oracle(vqx, dtype, shape, bs, qmax):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * torch.exp(torch.randn(shape, generator=g))).to(dtype)
    x.reshape(-1)[:bs] = 0.0                      # a zero block: the 1e-12 floor
    energy = torch.rand(shape[-1], generator=g)
    h = hist(vqx, -qmax, qmax, 4001)
    h.add_unit_scaled(x.cuda(), bs, qmax, energy.cuda())
    u = R.unit_scale(x, bs, qmax).reshape(-1)
    wts = energy.repeat(u.numel() // energy.numel())
    want = R.lcq_histogram_add(u, wts, -qmax, qmax, 4001)
    assert_sums((h.weight, h.total, h.square), want, f"{dtype} {shape} bs={bs}")
    # no energy: unit weights, exact counts
    h2 = hist(vqx, -qmax, qmax, 4001)
    h2.add_unit_scaled(x.cuda(), bs, qmax)
    assert torch.equal(h2.weight.cpu(), R.lcq_histogram_add(u, torch.ones(()), -qmax, qmax, 4001)[0])


@pytest.mark.gpu
def test_fused_unit_scale_full_size(vqx):
    # a 4096 x 4096 weight in blocks of 64: counts exact, moments to 1e-10
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4096, 4096, generator=g)
    h = hist(vqx, -7.0, 7.0, 4001)
    h.add_unit_scaled(x.cuda(), 64, 7.0)
    u = R.unit_scale(x, 64, 7.0).reshape(-1)
    want = R.lcq_histogram_add(u, torch.ones(()), -7.0, 7.0, 4001)
    assert torch.equal(h.weight.cpu(), want[0])
    assert_sums((h.weight, h.total, h.square), want, "full size")
    assert int(h.weight.sum().item()) == x.numel()
    assert math.isclose(h.square.sum().item(), (u.double() ** 2).sum().item(), rel_tol=1e-12)
