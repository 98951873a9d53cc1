"""Pins of the learned-codebook calibration oracle (src/vc/quantization/lcq.py:
44-150): bins against a brute-force edge count, moments against per-bin
numpy sums, unit_scale against its invariances."""

import numpy as np
import torch

from oracle import reference_ops as R


def brute_bins(values, quant_min, quant_max, bins):
    edges = torch.linspace(quant_min - 0.5, quant_max + 0.5, bins + 1, dtype=torch.float32).numpy()
    out = []
    for v in values.numpy():
        c = bins + 1 if np.isnan(v) else int(np.sum(edges <= v))
        out.append(min(max(c - 1, 0), bins - 1))
    return np.array(out)


def test_histogram_bins_are_the_edge_counts():
    g = torch.Generator().manual_seed(0)
    edges = torch.linspace(-7.5, 7.5, 12, dtype=torch.float32)
    v = torch.cat([torch.randn(500, generator=g) * 5, edges, edges + 1e-6, edges - 1e-6,
                   torch.tensor([float("nan"), float("inf"), -float("inf"), 100.0, -100.0, -0.0])])
    w, t, s = R.lcq_histogram_add(v, torch.ones(()), -7.0, 7.0, bins=11)
    counts = np.bincount(brute_bins(v, -7.0, 7.0, 11), minlength=11)
    assert np.array_equal(w.numpy(), counts.astype(np.float64))


def test_histogram_moments_are_per_bin_sums():
    g = torch.Generator().manual_seed(1)
    v = torch.randn(3000, generator=g) * 3
    wt = torch.rand(3000, generator=g)
    w, t, s = R.lcq_histogram_add(v, wt, -7.0, 7.0, bins=101)
    b = brute_bins(v, -7.0, 7.0, 101)
    vd, wd = v.double().numpy(), wt.double().numpy()
    for arr, want in ((w, wd), (t, wd * vd), (s, wd * vd * vd)):
        ref = np.zeros(101)
        np.add.at(ref, b, want)
        assert np.allclose(arr.numpy(), ref, rtol=1e-12, atol=1e-12)


def test_unit_scale_invariances():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(16, 128, generator=g)
    u = R.unit_scale(x, 32, 7.0)
    # a power-of-two multiple of the input normalizes identically
    assert torch.equal(R.unit_scale(x * 8.0, 32, 7.0), u)
    # every block's largest magnitude lands on quant_max (within an fp32 ulp)
    m = u.reshape(-1, 32).abs().amax(-1)
    assert torch.allclose(m, torch.full_like(m, 7.0), rtol=2**-22, atol=0)
    # an all-zero block divides by the 1e-12 floor and stays zero
    z = torch.zeros(2, 32)
    assert torch.equal(R.unit_scale(z, 32, 7.0), z)
