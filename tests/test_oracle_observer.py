"""Pins of the oracle's amax-history observer (AmaxObserverFakeQuantize,
restating FusedAmaxObsFakeQuantize's per-tensor / per-channel branch,
src/vc/quantization/fake_quantize.py:308-341, :404-432) by what its definition
fixes independently of its code: the first forward uses scale 1 (history all
zeros); afterwards the scale used at step t is the maximum of the amaxes of
the previous amax_history_len steps divided by quant_max, or the previous
scale when that maximum is not positive or not finite; per-channel equals
per-tensor on each channel's slice; with the observer off nothing changes;
with fake-quant off the input comes back."""

import math

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R


def qmap(dtype="fp8_e4m3"):
    return R.table_tensor(F.quantization_table(dtype))


def with_amax(a, n=64, seed=0):
    """A tensor whose absolute maximum is exactly a (attained once, negative)."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(n, generator=g) * 2 - 1) * a * 0.75
    x[n // 3] = -a
    return x


def window_scales(amaxes, H, qmax, pow2=False):
    """The scale each step uses, from the definition: previous H amaxes."""
    out, prev = [], 1.0
    for t in range(len(amaxes)):
        win = amaxes[max(0, t - H):t]
        m = max(win) if win else 0.0
        if math.isfinite(m) and m > 0:
            prev = float(np.float32(np.float32(m) / np.float32(qmax)))
            if pow2:
                prev = 2.0 ** math.ceil(math.log2(prev))
        out.append(prev)
    return out


@pytest.mark.parametrize("H", [1, 2, 3, 16])
def test_scale_is_the_previous_window_maximum(H):
    amaxes = [3.0, 1.5, 7.25, 0.5, 2.0, 9.0, 0.25, 4.0, 1.0, 6.5, 0.75, 5.0] * 2
    obs = R.AmaxObserverFakeQuantize(qmap(), 448.0, H)
    for t, a in enumerate(amaxes):
        x = with_amax(a, seed=t)
        y = obs(x)
        want = window_scales(amaxes[:t + 1], H, 448.0)[-1]
        assert obs.scale.item() == np.float32(want), (t, obs.scale.item(), want)
        # the output is the fake-quant at the scale of this step
        assert torch.equal(y, R.fake_quantize_per_tensor(x, qmap(), torch.tensor(want)))
    # the history holds the last H amaxes
    assert sorted(obs.amax_history.tolist()) == sorted(amaxes[-H:])


def test_first_forward_uses_unit_scale():
    obs = R.AmaxObserverFakeQuantize(qmap("int8"), 127.0, 4)
    x = with_amax(300.0)
    y = obs(x)
    assert torch.equal(y, R.fake_quantize_per_tensor(x, qmap("int8"), torch.ones(())))
    assert obs.scale.item() == 1.0 and obs.amax_history[0].item() == 300.0


def test_non_positive_and_non_finite_windows_keep_the_scale():
    obs = R.AmaxObserverFakeQuantize(qmap(), 448.0, 2)
    obs(with_amax(4.0))
    obs(with_amax(8.0))                      # uses 4 / 448
    s = obs.scale.item()
    obs(torch.tensor([float("inf"), 1.0]))   # uses max(4, 8) / 448
    s2 = obs.scale.item()
    assert s2 == np.float32(np.float32(8.0) / np.float32(448.0)) and s2 != s
    obs(with_amax(2.0))                      # window holds inf: keep
    obs(with_amax(2.0))                      # window still holds inf: keep
    assert obs.scale.item() == s2
    obs(torch.zeros(8))                      # window max 2
    assert obs.scale.item() == np.float32(np.float32(2.0) / np.float32(448.0))
    z = R.AmaxObserverFakeQuantize(qmap(), 448.0, 1)
    z(torch.zeros(8))
    z(torch.zeros(8))                        # window max 0: keep 1
    assert z.scale.item() == 1.0
    n = R.AmaxObserverFakeQuantize(qmap(), 448.0, 1)
    n(torch.tensor([float("nan"), 1.0]))
    assert torch.isnan(n.amax_history).all()
    n(with_amax(3.0))                        # NaN window: keep
    assert n.scale.item() == 1.0


def test_power_of_two_scale():
    amaxes = [3.0, 100.0, 0.3, 50.0]
    obs = R.AmaxObserverFakeQuantize(qmap(), 448.0, 2, force_scale_power_of_two=True)
    for t, a in enumerate(amaxes):
        obs(with_amax(a, seed=t))
        assert obs.scale.item() == window_scales(amaxes[:t + 1], 2, 448.0, pow2=True)[-1]


@pytest.mark.parametrize("ch_axis", [0, 1, -1])
def test_per_channel_is_per_tensor_per_slice(ch_axis):
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(6, 5, 4, generator=g) * (t + 1) for t in range(5)]
    obs = R.AmaxObserverFakeQuantize(qmap("int8"), 127.0, 3, per_channel=True, ch_axis=ch_axis)
    C = xs[0].shape[ch_axis]
    per = [R.AmaxObserverFakeQuantize(qmap("int8"), 127.0, 3) for _ in range(C)]
    for x in xs:
        y = obs(x)
        for c in range(C):
            yc = per[c](x.select(ch_axis, c))
            assert torch.equal(y.select(ch_axis, c), yc)
            assert obs.scale.reshape(-1)[c].item() == per[c].scale.item()


def test_disabled_observer_and_fake_quant():
    obs = R.AmaxObserverFakeQuantize(qmap(), 448.0, 2)
    obs(with_amax(4.0))
    obs(with_amax(8.0))
    h, s = obs.amax_history.clone(), obs.scale.clone()
    obs.observer_enabled = False
    x = with_amax(100.0)
    y = obs(x)
    assert torch.equal(obs.amax_history, h) and torch.equal(obs.scale, s)
    assert torch.equal(y, R.fake_quantize_per_tensor(x, qmap(), s))
    obs.fake_quant_enabled = False
    assert obs(x) is x
