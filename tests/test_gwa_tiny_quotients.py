"""The group-wise affine kernel forms x / scale as x * rcp(scale) and skips
the IEEE division for quotients below 2^-124 in magnitude, where its bf16
rounding may differ from the division's.  This pins, on the CPU and with the
reference's own bf16 op sequence (fake_quantize.py:162-211:
clamp(round(x / s + zp), qmin, qmax), then (q - zp) * s), that the output does
not depend on such a quotient beyond its sign: every tiny quotient, perturbed
by a few fp32 ulps either way before its bf16 rounding, gives the same output
bits for every zero point (zero, tiny, moderate, either sign) and range."""

import pytest
import torch

bf = torch.bfloat16


def out_of(q32, zp, sf, qmin, qmax):
    """The reference's steps after the division, on bf16 tensors, from an
    fp32 quotient (rounded to bf16 first, as the division's result is)."""
    q = q32.to(bf)
    t = torch.clamp(torch.round(q + zp), qmin, qmax)
    return (t - zp) * sf


def tiny_quotients():
    # every bf16 magnitude below 2^-124 (subnormals included), both signs,
    # as fp32 values just around each (the exact quotient need not be bf16)
    mags = torch.arange(1, 0x0180, dtype=torch.int32)  # bf16 patterns below 2^-124
    base = (mags << 16).view(torch.float32)
    half = ((mags << 16) + 0x8000).view(torch.float32)  # bf16 rounding midpoints
    q = torch.cat([base, half, -base, -half, torch.tensor([0.0, -0.0])])
    return q


@pytest.mark.parametrize("qmin,qmax", [(0, 3), (-2, 1), (0, 15), (-8, 7)])
def test_tiny_quotient_output_depends_on_sign_only(qmin, qmax):
    q = tiny_quotients()
    assert float(q.abs().max()) < 2.0 ** -124
    zps = [0.0, -0.0, 2.0 ** -130, -(2.0 ** -130), 2.0 ** -117, -(2.0 ** -117), 1.5 * 2.0 ** -116, 2.0 ** -100,
           0.25, -0.75, 1.0, 2.5, -3.0, 7.0]
    sfs = [2.0 ** -120, 1e-3, 0.5, 3.0, 2.0 ** 60]
    for zpv in zps:
        zp = torch.tensor(zpv).to(bf)
        for sfv in sfs:
            sf = torch.tensor(sfv).to(bf)
            want = out_of(q, zp, sf, qmin, qmax).view(torch.int16)
            for rel in (1 + 2.0 ** -20, 1 - 2.0 ** -20, 1 + 2.0 ** -22, 1 - 2.0 ** -22):
                got = out_of(q * rel, zp, sf, qmin, qmax).view(torch.int16)
                assert torch.equal(got, want), (zpv, sfv, rel)


def test_the_check_has_power_outside_the_tiny_range():
    # the same perturbation of quotients that are not tiny (just around the
    # integer rounding points and the bf16 midpoints near them) does change
    # outputs, so the equality above is a property of the tiny range
    base = torch.tensor([0.5, 1.5, 2.5, -0.5, 0.25, 0.75], dtype=torch.float32)
    zp = torch.tensor(0.0).to(bf)
    sf = torch.tensor(1.0).to(bf)
    want = out_of(base, zp, sf, -8, 7).view(torch.int16)
    moved = out_of(base * (1 + 2.0 ** -7), zp, sf, -8, 7).view(torch.int16)
    assert not torch.equal(moved, want)
