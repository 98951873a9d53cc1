"""Host-side logic without a GPU: the C-ABI library loads and exports every
entry point include/vqx.h declares, spec strings parse as the reference's
grammar does, dtype strings route as get_quantization_map does, and CPU
tensors are refused (no CPU path)."""

import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "vqx.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(vqx_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol(vqx):
    lib = vqx._lib.load()
    names = declared_symbols()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(vqx._lib.exported_symbols()) == names
    assert lib.vqx_version().decode().startswith("vqx")


def declared_arity():
    """Parameter count of every prototype in include/vqx.h."""
    text = open(os.path.join(ROOT, "include", "vqx.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(vqx_\w+)\s*\(([^;{]*?)\)\s*;", text, re.S):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_signatures_match_the_header(vqx):
    # the binding passes exactly the arguments each C prototype declares
    arity = declared_arity()
    assert sorted(arity) == declared_symbols()
    for name, (args, _) in vqx._lib._SIGNATURES.items():
        assert len(args) == arity[name], (name, len(args), arity[name])


def test_spec_parsing(vqx):
    from voyager_compiler_amd.quantization import QScheme, QuantizationSpec, parse_spec_fields

    p = parse_spec_fields("int8,qs=microscaling,bs=16,ax=-1,scale=fp8_e5m3")
    assert p == {"dtype": "int8", "qscheme": QScheme.MICROSCALING, "block_size": 16, "ch_axis": -1,
                 "scale_dtype": "fp8_e5m3", "quant_min": -128.0, "quant_max": 127.0}
    p = parse_spec_fields("posit8_1")
    assert p == {"dtype": "posit8_1"}
    p = parse_spec_fields("fp8_e4m3,qs=per_tensor_symmetric")
    assert p["quant_max"] == 448.0 and p["amax_history_len"] == 16
    p = parse_spec_fields("nf4_6,qs=microscaling,bs=64,ax=(2,3)")
    assert p["ch_axis"] == (2, 3) and p["quant_max"] == 31.0
    assert parse_spec_fields("posit8_1,qs=per_channel_symmetric")["quant_max"] == 4096.0
    assert parse_spec_fields("fp6_e3m2,qs=microscaling,bs=32")["quant_max"] == 28.0
    assert parse_spec_fields("fp4_e2m1,qs=microscaling,bs=32")["quant_max"] == 6.0
    with pytest.raises(ValueError, match="empty"):
        parse_spec_fields("")
    with pytest.raises(ValueError, match="key=value"):
        parse_spec_fields("int8,bogus")
    with pytest.raises(ValueError, match="Unknown argument"):
        parse_spec_fields("int8,foo=1")
    with pytest.raises(ValueError, match="block_size is required"):
        QuantizationSpec.from_str("int8,qs=microscaling")
    with pytest.raises(ValueError, match="quant_max is required"):
        QuantizationSpec(dtype="int8", qscheme=QScheme.PER_TENSOR_SYMMETRIC)


@pytest.mark.parametrize("dtype,kind,p0,p1", [
    ("int8", 2, 8, 1), ("UINT4", 2, 4, 0), ("e4m3", 4, 4, 0), ("fp8.e5m2", 4, 5, 0),
    ("fp8_e4m3", 3, 4, 3), ("fp6_e3m2", 3, 3, 2), ("fp4_e2m1", 3, 2, 1), ("fp8_e5m3", 3, 5, 3),
    ("posit8_1", 5, 8, 1), ("posit16_1", 5, 16, 1), ("nf4", 6, 0, 0), ("bfloat16", 0, 0, 0),
    ("float16", 1, 0, 0)])
def test_format_routing(vqx, dtype, kind, p0, p1):
    f = vqx.parse_format(dtype)
    assert (f.kind, f.p0, f.p1) == (kind, p0, p1)


def test_format_details(vqx):
    assert vqx.parse_format("fp8_e4m3").max_norm == 448.0
    assert vqx.parse_format("fp8_e5m2").max_norm == 57344.0
    assert vqx.parse_format("fp6_e3m2").code_bits == 6
    assert vqx.parse_format("fp8_e5m3").flags == 1
    assert vqx.parse_format("nf4").code_bits == 4 and vqx.parse_format("nf4").nlevels == 16
    with pytest.raises(ValueError, match="Unsupported dtype"):
        vqx.parse_format("mxfoo")
    with pytest.raises(AssertionError):
        vqx.parse_format("fp8_e2m2")


def test_cpu_tensors_are_refused(vqx):
    x = torch.randn(8)
    with pytest.raises(NotImplementedError):
        torch.ops.quantized_ops.vmap(x, torch.zeros(65536, dtype=torch.bfloat16))
    with pytest.raises(NotImplementedError):
        torch.ops.quantized_ops.fake_quant(x, "posit8_1", None, True, False)
    with pytest.raises(NotImplementedError):
        torch.ops.quantized_ops.quantize_mx(x.reshape(1, 8), torch.zeros(65536, dtype=torch.bfloat16),
                                            [-1], 8, 448.0, True)


def test_fake_impls_trace(vqx):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(4, 64, dtype=torch.bfloat16)
        s, q = torch.ops.quantized_ops.quantize_mx(x, torch.empty(65536, dtype=torch.bfloat16), [-1],
                                                   32, 448.0, True)
        assert s.shape == (4, 2) and q.shape == (4, 64)
        sc, codes = torch.ops.quantized_ops.quantize_mx_packed(x, "fp4_e2m1", -1, 32)
        assert sc.shape == (4, 2) and sc.dtype == torch.uint8 and codes.numel() == 128
        # both weight layouts of the GEMM ops, both activation layouts of conv2d_mx
        w = torch.empty(48, 64, dtype=torch.bfloat16)
        ws = torch.empty(48, 2, dtype=torch.bfloat16)
        assert torch.ops.quantized_ops.linear_mx(x, w, weight_scale=ws, block_size=32).shape == (4, 48)
        assert torch.ops.quantized_ops.linear_mx(x, w.T, weight_scale=ws.T, block_size=32,
                                                 weight_layout="ck").shape == (4, 48)
        assert torch.ops.quantized_ops.matmul_mx(x, w.T).shape == (4, 48)
        assert torch.ops.quantized_ops.matmul_mx(x, w, weight_layout="kc").shape == (4, 48)
        img = torch.empty(2, 8, 10, 12, dtype=torch.bfloat16)
        k = torch.empty(6, 8, 3, 3, dtype=torch.bfloat16)
        out = torch.ops.quantized_ops.conv2d_mx(img, k, None, [2, 2], [1, 1])
        assert out.shape == (2, 6, 5, 6)
        out = torch.ops.quantized_ops.conv2d_mx(img.permute(0, 2, 3, 1), k.permute(2, 3, 1, 0), None, [2, 2],
                                                [1, 1], layout="nhwc")
        assert out.shape == (2, 5, 6, 6)


def test_fake_quantize_module_state_on_cpu(vqx):
    from voyager_compiler_amd.quantization import FusedAmaxObsFakeQuantize, QuantizationSpec

    fq = QuantizationSpec.from_str("fp8_e4m3,qs=per_tensor_symmetric").make_fake_quantize()
    assert bool(fq.observer_enabled[0]) and fq.amax_history_len == 16
    sd = {"scale": torch.tensor([2.0]), "amax_history": torch.ones(16, 1), "fake_quant_enabled": torch.tensor([1], dtype=torch.uint8),
          "observer_enabled": torch.tensor([1], dtype=torch.uint8), "zero_point": torch.tensor([1.0])}
    fq.load_state_dict(sd)
    assert fq.amax_history.shape == (16, 1) and fq.scale.item() == 2.0
    fq2 = FusedAmaxObsFakeQuantize("posit8_1")
    assert not bool(fq2.observer_enabled[0])


def test_fake_quantize_flags_follow_the_buffers(vqx):
    # the enable flags are buffers: a loaded state_dict, an in-place write
    # (lcq.py writes fake_quant_enabled.zero_() / .copy_()) and the enable /
    # disable methods all take effect on the next forward
    from voyager_compiler_amd.quantization import QuantizationSpec

    spec = QuantizationSpec.from_str("int8,qs=per_tensor_symmetric,ahl=2")
    fq = spec.make_fake_quantize()
    assert fq._observer_on() and fq._fake_quant_on()
    sd = {k: v.clone() for k, v in fq.state_dict().items()}
    sd["observer_enabled"].zero_()
    sd["fake_quant_enabled"].zero_()
    fq.load_state_dict(sd)
    assert not fq._observer_on() and not fq._fake_quant_on()
    fq.fake_quant_enabled.copy_(torch.ones(1, dtype=torch.uint8))
    assert fq._fake_quant_on() and not fq._observer_on()
    fq.observer_enabled[0] = 1
    assert fq._observer_on()
    fq.disable_observer()
    fq.fake_quant_enabled.zero_()
    assert not fq._observer_on() and not fq._fake_quant_on()
    fq.enable_fake_quant()
    assert fq._fake_quant_on()


def _stream_k_bytes(M, N, K, cus=256):
    """The NF4 tile kernel's balanced-last-round plan, restated: split the
    tiles of the last partly filled round along K when each CU's share is at
    least max(16, nk / 4) steps and at least 24 steps shorter than a tile,
    with at most 6 ranges meeting one tile."""
    if M <= 16 or N % 128 or K % 64:
        return 0
    tiles, nk = (M // 256) * (N // 128), K // 64
    rem = tiles % cus
    if rem == 0:
        return 0
    U = rem * nk
    g = min(cus, U // max(16, nk // 4))
    if g < 1 or -(-U // g) + 24 > nk or -(-nk // (U // g)) + 1 > 6:
        return 0
    return -(-rem * 4 // 256) * 256 + 2 * g * 256 * 128 * 4


def test_nf4_linear_workspace_size(vqx):
    # without a GPU the library assumes MI355X's 256 CUs
    import ctypes
    L = vqx._lib
    for shape in [(2048, 11008, 4096), (4096, 4096, 4096), (512, 4096, 4096), (16, 4096, 4096), (300, 512, 2048),
                  (256, 11008, 4096), (808, 11008, 4096), (768, 1024, 8192), (256, 128, 64), (4096, 11008, 128)]:
        n = ctypes.c_int64(-1)
        L.call("vqx_nf4_linear_workspace_size", *shape, ctypes.byref(n))
        assert n.value == _stream_k_bytes(*shape), shape
    assert _stream_k_bytes(2048, 11008, 4096) == 0  # C5: 688 tiles, whole tiles
    assert _stream_k_bytes(256, 11008, 4096) == 512 + 2 * 256 * 131072
