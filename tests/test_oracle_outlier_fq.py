"""CPU: the oracle's FakeQuantize outlier handling (OutlierFakeQuantize,
src/vc/quantization/fake_quantize.py:373-395) pinned by independent
restatements: the top-k threshold against a numpy sort of |x| (the k-th
largest, NaN when x holds a NaN, as torch.topk ranks NaN first and min
propagates it), the running average against numpy float32 arithmetic with
the product rounded to bf16 by the oracle's own bit-level rounding, the mask
and restore elementwise, and max_outlier_pct against count / numel."""

import math

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R


def kth_largest_abs(x, k):
    a = np.abs(x.float().numpy().reshape(-1))
    if np.isnan(a).any():
        return float("nan")
    return float(np.sort(a)[-k])


def bf16_round(v):
    return float(F.bf16_to_f32(F.f32_to_bf16(np.array([v], dtype=np.float32)))[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("pct", [0.01, 0.2, 1e-9])
def test_topk_threshold_and_running_average(dtype, pct):
    g = torch.Generator().manual_seed(3)
    ora = R.OutlierFakeQuantize(outlier_pct=pct)
    t = None
    for step in range(5):
        x = (torch.randn(37, 91, generator=g) * (1 + step)).to(dtype)
        x.view(-1)[5] = x.view(-1)[6]            # a tie
        ora(x, None)
        k = max(1, math.ceil(pct * x.numel()))
        v = kth_largest_abs(x, k)
        if t is None:
            t = np.float32(v)
        else:
            prod = np.float32(np.float32(v) * np.float32(1.0 - 0.9))
            if dtype == torch.bfloat16:
                prod = np.float32(bf16_round(prod))
            t = np.float32(np.float32(t * np.float32(0.9)) + prod)
        assert ora.outlier_threshold.dtype == torch.float32 and ora.outlier_threshold.dim() == 0
        assert ora.outlier_threshold.item() == float(t), (step, ora.outlier_threshold.item(), float(t))


def test_nan_makes_the_threshold_nan_and_masks_nothing():
    ora = R.OutlierFakeQuantize(outlier_pct=0.05)
    x = torch.randn(64, 32).to(torch.bfloat16)
    x[3, 4] = float("nan")
    y = ora(x, lambda xm: xm * 0)
    assert math.isnan(ora.outlier_threshold.item())
    assert ora.max_outlier_pct == 0
    # nothing is an outlier: every element takes the fake-quant (here 0, NaN * 0 = NaN)
    assert bool((y[~torch.isnan(x)] == 0).all())


@pytest.mark.parametrize("thr", [2.0, -1.0, 0.0])
def test_mask_restore_and_fraction(thr):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(50, 40, generator=g).to(torch.bfloat16)
    x[0, 0] = float("inf")
    x[0, 1] = -0.0
    ora = R.OutlierFakeQuantize(outlier_threshold=thr)
    seen = []
    y = ora(x, lambda xm: seen.append(xm.clone()) or xm + 1)
    a = x.float().numpy()
    t = bf16_round(thr)
    skip = np.abs(a) >= t
    assert np.array_equal(seen[0].float().numpy(), np.where(skip, 0.0, a))
    assert np.array_equal(y.float().numpy(), np.where(skip, a, (torch.from_numpy(np.where(skip, 0.0, a))
                                                                .to(torch.bfloat16) + 1).float().numpy()))
    assert ora.max_outlier_pct == skip.sum() / skip.size
