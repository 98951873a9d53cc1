"""GPU: FusedAmaxObsFakeQuantize with the per-tensor and per-channel amax-
history observer (src/vc/quantization/fake_quantize.py:308-341, :404-432) over
several forwards, bit for bit against the oracle's restatement: outputs,
amax_history and scale after every step, including the first forward (scale
1), zero / NaN / Inf inputs, power-of-two scales near the CPU log2's rounding
steps, state_dict round trips in the middle of the history, the enable flags
as buffers (loaded, or written in place as lcq.py does), the outlier
fraction, and the straight-through gradients of every fake-quant function."""

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R
from tests.conftest import assert_bitexact


def spec_module(vqx, s):
    return vqx.quantization.QuantizationSpec.from_str(s).make_fake_quantize("cuda").cuda()


def oracle_for(fq, dtype):
    return R.AmaxObserverFakeQuantize(R.table_tensor(F.quantization_table(dtype)), fq.quant_max,
                                      fq.amax_history_len, per_channel=fq.is_per_channel, ch_axis=fq.ch_axis,
                                      force_scale_power_of_two=fq.force_scale_power_of_two)


def check_state(fq, ora, what):
    assert_bitexact(fq.amax_history.cpu(), ora.amax_history, f"{what}: amax_history")
    assert_bitexact(fq.scale.cpu(), ora.scale, f"{what}: scale")


def steps(shape, dtype, n, seed, edge=True):
    """n inputs with amaxes that rise and fall; with edge, a zero tensor, an
    input holding NaN and one holding Inf among them."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for t in range(n):
        x = torch.randn(*shape, generator=g) * float(2.0 ** ((t * 5) % 7 - 3))
        if edge and t == 3:
            x = torch.zeros(*shape)
        if edge and t == 5:
            x.view(-1)[7] = float("nan")
        if edge and t == 7:
            x.view(-1)[11] = float("-inf")
        out.append(x.to(dtype))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("spec,fmt", [("fp8_e4m3,qs=per_tensor_symmetric", "fp8_e4m3"),
                                      ("int8,qs=per_tensor_symmetric,ahl=3", "int8"),
                                      ("posit8_1,qs=per_tensor_symmetric,ahl=1", "posit8_1")])
def test_per_tensor_observer(vqx, dtype, spec, fmt):
    print(f"observer {spec} {dtype}", flush=True)
    fq = spec_module(vqx, spec)
    ora = oracle_for(fq, fmt)
    for t, x in enumerate(steps((96, 130), dtype, 24, 1)):
        y = fq(x.cuda())
        want = ora(x)
        assert_bitexact(y.cpu(), want, f"step {t} output")
        check_state(fq, ora, f"step {t}")


@pytest.mark.gpu
@pytest.mark.parametrize("shape,ax", [((256, 1024), 0), ((64, 96), -1), ((4, 24, 40), 1), ((6, 10, 33), 0)])
def test_per_channel_observer(vqx, shape, ax):
    print(f"per-channel observer shape={shape} ax={ax}", flush=True)
    fq = spec_module(vqx, f"int8,qs=per_channel_symmetric,ax={ax},ahl=4")
    ora = oracle_for(fq, "int8")
    for t, x in enumerate(steps(shape, torch.bfloat16, 10, 2)):
        y = fq(x.cuda())
        assert_bitexact(y.cpu(), ora(x), f"step {t} output")
        check_state(fq, ora, f"step {t}")


@pytest.mark.gpu
def test_observer_power_of_two_near_log2_steps(vqx):
    # amaxes whose scale amax / quant_max lands on 2^p (1 + d 2^-23) for small
    # d, where the CPU's fp32 log2 rounds down to p for the first few d
    fq = spec_module(vqx, "fp8_e4m3,qs=per_tensor_symmetric,ahl=1")
    fq.force_scale_power_of_two = True
    fq.quant_max = 256.0  # a power of two, so amax / quant_max is exactly the scale built below
    ora = oracle_for(fq, "fp8_e4m3")
    xs = []
    for p in (4, 9, 20, 40, 70, 100, -5, -12, -30, -70, -120, -130):
        for d in (0, 1, 2, 3, 6, 12, 23):
            sf = np.array([((p + 127) << 23) | d if p >= -126 else (1 << (p + 149)) | d], np.uint32).view(np.float32)
            amax = np.float32(sf[0]) * np.float32(256.0)
            x = torch.full((1024,), float(amax) / 2)
            x[100] = float(amax)
            xs.append(x)
    xs.append(torch.ones(1024))
    for t, x in enumerate(xs):
        y = fq(x.cuda())
        assert_bitexact(y.cpu(), ora(x), f"step {t} output")
        check_state(fq, ora, f"step {t}")


@pytest.mark.gpu
def test_observer_state_dict_round_trip_mid_history(vqx):
    spec = "fp8_e4m3,qs=per_tensor_symmetric,ahl=4"
    fq = spec_module(vqx, spec)
    ora = oracle_for(fq, "fp8_e4m3")
    xs = steps((128, 64), torch.bfloat16, 9, 3, edge=False)
    for x in xs[:3]:
        fq(x.cuda())
        ora(x)
    sd = {k: v.clone() for k, v in fq.state_dict().items()}
    fresh = spec_module(vqx, spec)
    fresh.load_state_dict(sd)
    check_state(fresh, ora, "loaded")
    for t, x in enumerate(xs[3:]):
        y = fresh(x.cuda())
        assert_bitexact(y.cpu(), ora(x), f"after load, step {t}")
        check_state(fresh, ora, f"after load, step {t}")


@pytest.mark.gpu
def test_loaded_flags_are_honoured(vqx):
    spec = "int8,qs=per_tensor_symmetric,ahl=2"
    fq = spec_module(vqx, spec)
    for x in steps((64, 64), torch.float32, 3, 4, edge=False):
        fq(x.cuda())
    sd = {k: v.clone() for k, v in fq.state_dict().items()}
    sd["observer_enabled"].zero_()
    sd["fake_quant_enabled"].zero_()
    other = spec_module(vqx, spec)
    other.load_state_dict(sd)
    h, s = other.amax_history.clone(), other.scale.clone()
    x = torch.randn(64, 64).cuda() * 50
    y = other(x)
    assert torch.equal(y, x)
    assert torch.equal(other.amax_history, h) and torch.equal(other.scale, s)
    # fake-quant back on through an in-place write (as lcq.py does), observer
    # still off: the stored scale is used and nothing is updated
    other.fake_quant_enabled.copy_(torch.ones_like(other.fake_quant_enabled))
    y = other(x)
    want = R.fake_quantize_per_tensor(x.cpu(), R.table_tensor(F.quantization_table("int8")), s.cpu())
    assert_bitexact(y.cpu(), want, "stored-scale fake-quant")
    assert torch.equal(other.amax_history, h) and torch.equal(other.scale, s)
    other.fake_quant_enabled.zero_()
    assert torch.equal(other(x), x)


@pytest.mark.gpu
def test_outlier_fraction_without_host_sync(vqx):
    fq = spec_module(vqx, "int8,qs=per_tensor_symmetric,ahl=2,othr=2.5")
    g = torch.Generator().manual_seed(5)
    fracs = []
    for t in range(3):
        x = torch.randn(200, 100, generator=g) * (1 + t)
        fq(x.cuda())
        fracs.append((x.abs() >= 2.5).sum().item() / x.numel())
    assert fq.max_outlier_pct == max(fracs)
    fq.max_outlier_pct = 0.5
    assert fq.max_outlier_pct == 0.5


@pytest.mark.gpu
def test_straight_through_gradients(vqx):
    Fn = vqx.quantization.fake_quantize
    g = torch.Generator().manual_seed(6)
    x = torch.randn(64, 128, generator=g).to(torch.bfloat16).cuda().requires_grad_(True)
    up = torch.randn(64, 128, generator=g).to(torch.bfloat16).cuda()
    qm = vqx.get_quantization_map("fp8_e4m3", "cuda")
    cases = {
        "per-tensor": lambda: Fn.FakeQuantizeFunction.apply(x, True, qm, torch.ones(1, device="cuda"), None),
        "mx": lambda: Fn.MXFakeQuantizeFunction.apply(x, True, torch.ones(1, device="cuda"), qm, -1, 32, 448.0,
                                                      True, None, None),
        "group-wise affine": lambda: Fn.GroupWiseAffineFakeQuantFunction.apply(
            x, True, torch.ones(1, device="cuda"), torch.zeros(1, device="cuda"), -1, 64, 0.0, 3.0, None),
        "observed": lambda: spec_module(vqx, "fp8_e4m3,qs=per_tensor_symmetric")(x),
        "disabled": lambda: Fn.FakeQuantizeFunction.apply(x, False, qm, torch.ones(1, device="cuda"), None),
    }
    for name, f in cases.items():
        x.grad = None
        y = f()
        assert y.shape == x.shape, name
        y.backward(up)
        assert torch.equal(x.grad, up), name


@pytest.mark.gpu
def test_int24_table_all_patterns(vqx):
    # get_quantization_map("int24") (fake_quantize.py:42-46): the reference's
    # expression on all bf16 patterns, evaluated by torch on the CPU
    vals = torch.arange(2**16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    want = torch.clamp(torch.round(vals), -(2**23), 2**23 - 1)
    got = vqx.get_quantization_map("int24", "cuda")
    assert_bitexact(got.cpu(), want, "int24 table")
    assert_bitexact(got.cpu(), R.table_tensor(F.int_table(24)), "int24 table vs oracle")


@pytest.mark.gpu
@pytest.mark.parametrize("weight_spec", ["int8,qs=per_tensor_symmetric", "int8,qs=per_channel_symmetric,ax=0"])
def test_derived_bias_scale(vqx, weight_spec):
    # the INT8 scheme's int24 bias (test/run_ci.py:61-65): scale = input scale
    # x weight scale (quantize_pt2e.py:163-175), fake-quantized through the
    # int24 table with FakeQuantizeFunction (fake_quantize.py:466-495)
    Qz = vqx.quantization
    act = spec_module(vqx, "int8,qs=per_tensor_symmetric")
    wfq = spec_module(vqx, weight_spec)
    g = torch.Generator().manual_seed(8)
    w = torch.randn(96, 64, generator=g) * 0.05
    for t in range(3):  # let both observers see a few tensors
        act(torch.randn(32, 64, generator=g).cuda() * (1 + t))
        wfq(w.cuda())
    spec = Qz.DerivedQuantizationSpec(derived_from=["x", "w"], derive_qparams_fn=Qz.derive_bias_qparams_fn,
                                      dtype="int24")
    bfq = spec.make_fake_quantize({"x": act, "w": wfq})
    bias = torch.randn(96, generator=g) * 0.3
    y = bfq(bias.cuda())
    scale = act.scale.cpu() * wfq.scale.cpu().flatten()
    assert_bitexact(bfq.calculate_qparams().cpu(), scale, "derived scale")
    want = R.fake_quantize_per_tensor(bias, R.table_tensor(F.int_table(24)), scale)
    assert_bitexact(y.cpu(), want, "int24 bias")
    assert not bfq._observer_on()
    bfq.disable_fake_quant()
    assert bfq(bias.cuda()).equal(bias.cuda())


@pytest.mark.gpu
def test_module_built_and_run_under_inference_mode(vqx):
    # a module made and run under torch.inference_mode: its buffers carry no
    # version counter, so the enable flags are read on every forward and an
    # in-place write to them (disable_observer) takes effect at once
    print("observer under inference_mode", flush=True)
    xs = steps((64, 96), torch.bfloat16, 7, 3, edge=False)
    with torch.inference_mode():
        fq = spec_module(vqx, "int8,qs=per_tensor_symmetric,ahl=2")
        assert fq.observer_enabled.is_inference()
        ora = oracle_for(fq, "int8")
        for t, x in enumerate(xs[:5]):
            assert_bitexact(fq(x.cuda()).cpu(), ora(x), f"step {t} output")
            check_state(fq, ora, f"step {t}")
        fq.disable_observer()
        ora.observer_enabled = False
        assert_bitexact(fq(xs[5].cuda()).cpu(), ora(xs[5]), "observer off")
        check_state(fq, ora, "observer off")
        mx = spec_module(vqx, "nf4_6,qs=microscaling,bs=64,ax=-1,scale=fp8_e5m3")
        x = xs[6]
        want = R.mx_fake_quantize(x, R.table_tensor(F.quantization_table("nf4_6")), [-1], 64, 31.0, False,
                                  R.table_tensor(F.quantization_table("fp8_e5m3")))[1]
        assert_bitexact(mx(x.cuda()).cpu(), want, "microscaling under inference_mode")
