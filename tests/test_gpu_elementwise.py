"""GPU parity of the elementwise path: FakeQuantizeFunction in closed form
(C1: posit(8,1) of a 4096x4096 fp32 N(0,1) tensor), codes, vmap, and the
reference's quantize / dequantize ops, against the CPU oracle."""

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R
from tests.conftest import assert_bitexact

Q = torch.ops.quantized_ops


def oracle_fq_f32(x, dtype):
    """y = table[bf16(x)] as fp32 (scale 1), numpy-fast."""
    t = F.quantization_table(dtype)
    h = F.f32_to_bf16(x.numpy())
    return torch.from_numpy(F.bf16_to_f32(t[h]))


@pytest.mark.gpu
def test_c1_posit8_1_fake_quant_and_codes(vqx):
    torch.manual_seed(0)
    x = torch.randn(4096, 4096, dtype=torch.float32)
    y, codes = Q.fake_quant(x.cuda(), "posit8_1", None, True, True)
    torch.cuda.synchronize()
    assert_bitexact(y.cpu(), oracle_fq_f32(x, "posit8_1"), "C1 values")
    h = F.f32_to_bf16(x.numpy())
    want = (F.posit_codes(h, 8, 1) & 0xFF).astype(np.uint8)
    assert np.array_equal(codes.cpu().numpy(), want)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["posit8_1", "fp8_e4m3", "fp6_e3m2", "fp4_e2m1", "e4m3", "int8", "nf4",
                                   "posit16_1", "uint4", "fp16_e5m10"])
def test_fake_quant_all_patterns(vqx, dtype):
    # every bf16 pattern through the fp32, bf16 and fp16 entry dtypes
    allp = torch.from_numpy(F.bf16_to_f32(F.ALL_BF16))
    t = R.table_tensor(F.quantization_table(dtype))
    for dt in (torch.float32, torch.bfloat16):
        x = allp.to(dt)
        y, _ = Q.fake_quant(x.cuda(), dtype, None, True, False)
        assert_bitexact(y.cpu(), R.fake_quantize_per_tensor(x, t, torch.tensor([1.0])), f"{dtype} {dt}")
    x = torch.randn(5003).to(torch.float16)
    y, _ = Q.fake_quant(x.cuda(), dtype, None, True, False)
    assert_bitexact(y.cpu(), R.fake_quantize_per_tensor(x, t, torch.tensor([1.0])), f"{dtype} fp16")


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [0.37, 0.125, 3.0, 1e-3])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_fake_quant_scaled(vqx, scale, dt):
    torch.manual_seed(1)
    x = (torch.randn(257, 129) * 4).to(dt)
    s = torch.tensor([scale])
    for dtype in ("posit8_1", "fp8_e4m3", "int8"):
        t = R.table_tensor(F.quantization_table(dtype))
        y, _ = Q.fake_quant(x.cuda(), dtype, s.cuda(), True, False)
        assert_bitexact(y.cpu(), R.fake_quantize_per_tensor(x, t, s), f"{dtype} s={scale}")
        yq, _ = Q.fake_quant(x.cuda(), dtype, s.cuda(), False, False)
        assert_bitexact(yq.cpu(), R.vmap(x / s.to(dt), t), f"{dtype} quantize s={scale}")


@pytest.mark.gpu
def test_fake_quant_per_channel(vqx):
    torch.manual_seed(2)
    x = torch.randn(64, 33, 7)
    s = torch.rand(1, 33, 1) + 0.1
    t = R.table_tensor(F.quantization_table("fp8_e4m3"))
    y, _ = Q.fake_quant(x.cuda(), "fp8_e4m3", s.cuda(), True, False)
    assert_bitexact(y.cpu(), R.vmap(x / s, t) * s, "per-channel")


@pytest.mark.gpu
@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 1 << 16, (1 << 20) + 3])
def test_vmap_sizes_and_tables(vqx, n):
    g = torch.Generator().manual_seed(n)
    table = torch.randint(-32768, 32767, (65536,), generator=g, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = torch.randn(n, generator=g)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        xx = x.to(dt)
        y = Q.vmap(xx.cuda(), table.cuda())
        assert y.dtype == dt
        assert_bitexact(y.cpu(), R.vmap(xx, table), f"vmap n={n} {dt}")


@pytest.mark.gpu
def test_vmap_unaligned_view_and_int_table(vqx):
    x = torch.randn(1000)
    xv = x.cuda()[3:]  # misaligned start
    t = torch.arange(65536, dtype=torch.int64)  # an index table (convert's codebook qmap)
    y = Q.vmap(xv, t.cuda())
    assert_bitexact(y.cpu(), R.vmap(x[3:], t), "unaligned")


@pytest.mark.gpu
def test_quantize_dequantize_ops_block_scale(vqx):
    torch.manual_seed(3)
    x = torch.randn(6, 100, 5, dtype=torch.bfloat16)
    scale = (torch.rand(6, 4, 5) + 0.05).to(torch.bfloat16)  # blocks of 32 along dim 1 (last short)
    qmap = R.table_tensor(F.quantization_table("fp6_e3m2"))
    got = Q.quantize(x.cuda(), scale.cuda(), None, [1], 32, qmap.cuda(), None)
    want = R.quantize(x, scale, None, [1], 32, qmap)
    assert_bitexact(got.cpu(), want, "quantize")
    back = Q.dequantize(got, scale.cuda(), None, [1], 32, None, None)
    assert_bitexact(back.cpu(), R.dequantize(want, scale, None, [1], 32), "dequantize")
    outq = R.table_tensor(F.quantization_table("posit8_1"))
    back2 = Q.dequantize(got, scale.cuda(), None, [1], 32, qmap.cuda(), outq.cuda())
    assert_bitexact(back2.cpu(), R.dequantize(want, scale, None, [1], 32, qmap, outq), "dequantize maps")


@pytest.mark.gpu
def test_quantize_promotes_like_torch(vqx):
    x = torch.randn(40, 16, dtype=torch.bfloat16)
    s = torch.rand(40, 1) + 0.5  # fp32 scale: bf16 / fp32 computes in fp32
    qmap = R.table_tensor(F.quantization_table("int8"))
    got = Q.quantize(x.cuda(), s.cuda(), None, None, None, qmap.cuda(), None)
    want = R.quantize(x, s, None, None, None, qmap)
    assert got.dtype == want.dtype == torch.float32
    assert_bitexact(got.cpu(), want, "promote")
    zp = torch.full((40, 1), 3.0)
    got = Q.quantize(x.cuda(), s.cuda(), zp.cuda(), None, None, qmap.cuda(), None)
    assert_bitexact(got.cpu(), R.quantize(x, s, zp, None, None, qmap), "zero point")
