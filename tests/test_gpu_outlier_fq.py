"""GPU: FakeQuantize outlier masking on the device (src/vc/quantization/
fake_quantize.py:373-395) against the CPU oracle, bit for bit.

* vqx_outlier_topk_threshold: the k-th largest |x| (the top-k minimum) for
  bf16 / fp16 / fp32 inputs, ragged lengths, ties, signed zeros, infinities,
  subnormals, NaN (which makes it NaN), k from 1 to numel, and the running
  average over calls, against a numpy sort and numpy float32 arithmetic.
* FusedAmaxObsFakeQuantize with outlier_pct / outlier_threshold over many
  forwards: outputs, scale buffers, the threshold buffer and
  max_outlier_pct against the oracle's OutlierFakeQuantize around the
  scheme's fake-quant (microscaling on either axis, per-tensor with the
  observer, group-wise affine), fake-quant and observer switched off in
  between, and the straight-through gradient.
"""

import math

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R
from tests.conftest import assert_bitexact


def kth_largest_abs(x, k):
    a = np.abs(x.float().numpy().reshape(-1))
    if np.isnan(a).any():
        return float("nan")
    return float(np.sort(a)[-k])


def topk_call(vqx, x, k, thr, ws, ema=False, decay=0.9):
    L = vqx._lib
    L.call("vqx_outlier_topk_threshold", L.ptr(x), L.dtype_tag(x.dtype), x.numel(), k, 1 if ema else 0,
           float(decay), float(1.0 - decay), L.ptr(thr), L.ptr(ws), ws.numel(), L.stream_of(x))


def special_input(n, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * torch.exp(2 * torch.randn(n, generator=g))
    if n > 40:
        x[:8] = x[8]                    # ties
        x[10] = -0.0
        x[11] = 0.0
        x[12] = float("inf")
        x[13] = -float("inf")
        x[14] = 1e-40                   # subnormal in fp32 / zero in bf16
        x[15:25] = -x[15:25].abs()
    return x.to(dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 1000, 4099, 300000])
def test_topk_threshold_is_the_kth_largest(vqx, dtype, n):
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    ws = qops.outlier_topk_workspace("cuda")
    thr = torch.zeros((), dtype=torch.float32, device="cuda")
    x = special_input(n, dtype, seed=n)
    xd = x.cuda()
    ks = sorted({1, min(2, n), max(1, n // 100), max(1, n // 2), n})
    for k in ks:
        print(f"topk {dtype} n={n} k={k}", flush=True)
        topk_call(vqx, xd, k, thr, ws)
        want = kth_largest_abs(x, k)
        assert thr.item() == want, (k, thr.item(), want)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_topk_threshold_nan_and_all_equal(vqx, dtype):
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    ws = qops.outlier_topk_workspace("cuda")
    thr = torch.zeros((), dtype=torch.float32, device="cuda")
    x = torch.full((5000,), -2.5, dtype=dtype)
    topk_call(vqx, x.cuda(), 50, thr, ws)
    assert thr.item() == 2.5
    x[4321] = float("nan")
    topk_call(vqx, x.cuda(), 50, thr, ws)
    assert math.isnan(thr.item())
    # the state is clean again after a NaN call
    x[4321] = 7.0
    topk_call(vqx, x.cuda(), 1, thr, ws)
    assert thr.item() == 7.0
    topk_call(vqx, x.cuda(), 2, thr, ws)
    assert thr.item() == 2.5


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_topk_running_average_matches_torch(vqx, dtype):
    # the oracle's in-place fp32 running average, call by call
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    ws = qops.outlier_topk_workspace("cuda")
    thr = torch.zeros((), dtype=torch.float32, device="cuda")
    ora = R.OutlierFakeQuantize(outlier_pct=0.01, decay=0.85)
    g = torch.Generator().manual_seed(8)
    for step in range(8):
        x = (torch.randn(123, 456, generator=g) * 1.7 ** step).to(dtype)
        ora(x, None)
        topk_call(vqx, x.cuda(), max(1, math.ceil(0.01 * x.numel())), thr, ws, ema=step > 0, decay=0.85)
        assert thr.item() == ora.outlier_threshold.item(), step


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("pct", [1e-5, 0.01, 0.3])
def test_topk_running_average_window(vqx, dtype, pct):
    # calls after the first see the previous threshold: the first pass also
    # counts a window of magnitudes around it and finishes the select when
    # the k-th value falls inside (the same input again, scaled slightly),
    # else the second pass does (scaled by 4 and 1/16, or back); ties, +-Inf,
    # -0 and tiny values included
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    ws = qops.outlier_topk_workspace("cuda")
    thr = torch.zeros((), dtype=torch.float32, device="cuda")
    ora = R.OutlierFakeQuantize(outlier_pct=pct, decay=0.9)
    base = special_input(200003, torch.float32, seed=77)
    for step, f in enumerate([1.0, 1.0, 1.03, 0.97, 4.0, 4.0, 1.0 / 16, 1.0, 1.0]):
        x = (base * f).to(dtype)
        ora(x, None)
        topk_call(vqx, x.cuda(), max(1, math.ceil(pct * x.numel())), thr, ws, ema=step > 0, decay=0.9)
        assert thr.item() == ora.outlier_threshold.item(), (step, f, thr.item(), ora.outlier_threshold.item())


def spec_module(vqx, s):
    return vqx.quantization.QuantizationSpec.from_str(s).make_fake_quantize("cuda").cuda()


def table(dtype):
    return R.table_tensor(F.quantization_table(dtype))


def activations(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    x = torch.where(torch.rand(shape, generator=g) < 0.01, x * 20, x)
    return x.to(dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("spec,shape,dtype", [
    ("nf4_6,qs=microscaling,bs=64,ax=-1,scale=fp8_e5m3,opct=0.01", (4, 96, 256), torch.bfloat16),
    ("nf4_6,qs=microscaling,bs=64,ax=-2,scale=fp8_e5m3,othr=6.0", (2, 4, 128, 64), torch.bfloat16),
    ("nf4_6,qs=microscaling,bs=64,ax=-1,scale=fp8_e5m3,opct=0.01", (64, 320), torch.float32),
    ("int6,qs=microscaling,bs=32,ax=-1,opct=0.02", (3, 50, 64), torch.bfloat16),
    ("fp8_e4m3,qs=microscaling,bs=32,ax=-1,opct=0.005", (256, 1024), torch.bfloat16),
])
def test_outlier_microscaling_module_over_forwards(vqx, spec, shape, dtype):
    print(f"outlier module {spec} {shape} {dtype}", flush=True)
    fq = spec_module(vqx, spec)
    parts = dict(p.split("=") for p in spec.split(",")[1:] if "=" in p)
    dtype_s = spec.split(",")[0]
    axis = int(parts["ax"])
    bs = int(parts["bs"])
    sq = table(parts["scale"]) if "scale" in parts else None
    ora = R.OutlierFakeQuantize(outlier_pct=float(parts["opct"]) if "opct" in parts else None,
                                outlier_threshold=float(parts["othr"]) if "othr" in parts else None)
    sf_box = []

    def mx(xm):
        sf, y = R.mx_fake_quantize(xm, table(dtype_s), [axis], bs, fq.quant_max, False, sq)
        sf_box.append(sf)
        return y

    for step in range(7):
        x = activations(shape, dtype, seed=step, scale=1.0 + 0.5 * step)
        if step == 4:
            x.view(-1)[3] = float("nan")        # a NaN threshold (opct) masks nothing
        if step == 5:
            fq.disable_fake_quant()
            got = fq(x.cuda()).cpu()
            want = ora(x, None)
            assert_bitexact(got, want, f"{spec} step {step} (fake-quant off)")
            fq.enable_fake_quant()
            continue
        if step == 6:
            fq.disable_observer()
            ora.observer_enabled = False
        got = fq(x.cuda()).cpu()
        want = ora(x, mx)
        assert_bitexact(got, want, f"{spec} step {step}")
        assert_bitexact(fq.scale.cpu(), sf_box[-1].float(), f"{spec} step {step} scale")
        if ora.outlier_pct is not None:
            assert_bitexact(fq.outlier_threshold.cpu(), ora.outlier_threshold, f"{spec} step {step} threshold")
        assert fq.max_outlier_pct == ora.max_outlier_pct, (step, fq.max_outlier_pct, ora.max_outlier_pct)


@pytest.mark.gpu
def test_outlier_other_schemes(vqx):
    # per-tensor with the amax-history observer (the observer sees the masked
    # input), and group-wise affine, each between the mask and the restore
    g = torch.Generator().manual_seed(12)
    fq = spec_module(vqx, "int8,qs=per_tensor_symmetric,ahl=3,opct=0.01")
    obs = R.AmaxObserverFakeQuantize(table("int8"), fq.quant_max, 3)
    ora = R.OutlierFakeQuantize(outlier_pct=0.01)
    for step in range(5):
        x = activations((70, 130), torch.bfloat16, seed=20 + step, scale=1 + step)
        got = fq(x.cuda()).cpu()
        want = ora(x, obs)
        assert_bitexact(got, want, f"per-tensor step {step}")
        assert_bitexact(fq.scale.cpu(), obs.scale, f"per-tensor step {step} scale")
    assert fq.max_outlier_pct == ora.max_outlier_pct

    m = vqx.quantization.FusedAmaxObsFakeQuantize("uint2", qscheme=vqx.quantization.QScheme.GROUP_WISE_AFFINE,
                                                  quant_min=0, quant_max=3, ch_axis=-1, block_size=64,
                                                  outlier_threshold=2.5, device="cuda")
    ora = R.OutlierFakeQuantize(outlier_threshold=2.5)
    for step in range(3):
        x = activations((2, 8, 128), torch.bfloat16, seed=30 + step)
        got = m(x.cuda()).cpu()
        want = ora(x, lambda xm: R.group_wise_affine_fake_quant(xm, -1, 64, 0, 3)[2])
        assert_bitexact(got, want, f"group-wise affine step {step}")
    assert m.max_outlier_pct == ora.max_outlier_pct
    m.max_outlier_pct = 0.75
    assert m.max_outlier_pct == 0.75
    m(activations((2, 8, 128), torch.bfloat16, seed=40).cuda())
    assert m.max_outlier_pct == 0.75


@pytest.mark.gpu
def test_outlier_threshold_edge_values(vqx):
    # a negative threshold makes every non-NaN element an outlier (the
    # output is the input); one above every |x| none; the same and zero /
    # mid thresholds for blocks along -2; table (edited qmap) path of the
    # microscaling kernel
    x = activations((16, 256), torch.bfloat16, seed=50)
    for thr in (-1.0, 1e30):
        fq = spec_module(vqx, f"nf4,qs=microscaling,bs=64,ax=-1,othr={thr}")
        got = fq(x.cuda()).cpu()
        ora = R.OutlierFakeQuantize(outlier_threshold=thr)
        want = ora(x, lambda xm: R.mx_fake_quantize(xm, table("nf4"), [-1], 64, 1.0, False)[1])
        assert_bitexact(got, want, f"othr={thr}")
        assert fq.max_outlier_pct == ora.max_outlier_pct
    # blocks along -2 (the column kernel), with NaN, +-Inf and -0 elements
    xc = activations((2, 128, 64), torch.bfloat16, seed=51)
    flat = xc.view(-1)
    flat[5], flat[700], flat[9000], flat[12345] = float("nan"), float("inf"), float("-inf"), -0.0
    for thr in (-1.0, 0.0, 2.0, 1e30):
        fq = spec_module(vqx, f"nf4_6,qs=microscaling,bs=64,ax=-2,scale=fp8_e5m3,othr={thr}")
        got = fq(xc.cuda()).cpu()
        ora = R.OutlierFakeQuantize(outlier_threshold=thr)
        want = ora(xc, lambda xm: R.mx_fake_quantize(xm, table("nf4_6"), [-2], 64, fq.quant_max, False,
                                                     table("fp8_e5m3"))[1])
        assert_bitexact(got, want, f"ax=-2 othr={thr}")
        assert fq.max_outlier_pct == ora.max_outlier_pct
    fq = spec_module(vqx, "int8,qs=microscaling,bs=32,ax=-1,othr=3.0")
    fq.qmap.mul_(1.0)  # an in-place edit: the kernels take the table path
    got = fq(x.cuda()).cpu()
    want = R.OutlierFakeQuantize(outlier_threshold=3.0)(
        x, lambda xm: R.mx_fake_quantize(xm, table("int8"), [-1], 32, fq.quant_max, False)[1])
    assert_bitexact(got, want, "table path")


@pytest.mark.gpu
def test_outlier_straight_through_gradient(vqx):
    fq = spec_module(vqx, "nf4_6,qs=microscaling,bs=64,ax=-1,scale=fp8_e5m3,opct=0.01")
    x = activations((8, 256), torch.bfloat16, seed=60).cuda().requires_grad_(True)
    fq(x).float().sum().backward()
    assert torch.equal(x.grad, torch.ones_like(x))
