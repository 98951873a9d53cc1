"""GPU: the closed-form encoders tabulated over all 65536 bf16 patterns on the
MI355X (get_quantization_map) equal the golden tables from the reference."""

import numpy as np
import pytest
import torch

from oracle import formats as F
from tests.conftest import assert_bitexact

GOLDEN = ["posit8_1", "posit8_0", "posit8_2", "posit6_1", "posit16_1", "fp8_e4m3", "fp8_e5m2", "fp6_e3m2",
          "fp6_e2m3", "fp4_e2m1", "fp8_e5m3", "fp8_e8m0", "fp16_e5m10", "e4m3", "e5m2", "nf4", "nf4_6",
          "nf3", "int8", "int4", "uint8", "uint4"]


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", GOLDEN)
def test_gpu_table_equals_golden(vqx, golden, dtype):
    q = vqx.get_quantization_map(dtype, "cuda")
    if isinstance(q, tuple):
        idx, vals = q
        assert np.array_equal(idx.cpu().numpy(), golden["nf_index_" + dtype].astype(np.int64))
        assert np.array_equal(u16(vals), golden["nf_values_" + dtype])
        q = vals[idx]
    g = torch.from_numpy(golden["t_" + dtype].view(np.int16)).view(torch.bfloat16)
    assert_bitexact(q.cpu(), g, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("n,es", [(8, 1), (8, 0), (8, 2), (16, 1)])
def test_gpu_posit_codes(vqx, n, es):
    f = vqx.parse_format(f"posit{n}_{es}")
    codes = f.tables("cuda")["codes"].cpu().numpy().view(np.uint16).astype(np.int64)
    assert np.array_equal(codes, F.posit_codes(F.ALL_BF16, n, es) & ((1 << n) - 1))


@pytest.mark.gpu
def test_gpu_level_boundaries_monotone(vqx):
    for d in ["nf4", "nf4_6", "nf3"]:
        t = vqx.parse_format(d).tables("cuda")
        assert t["monotone"], d


@pytest.mark.gpu
def test_gpu_codebook_table_matches_oracle(vqx):
    rng = np.random.default_rng(3)
    for K in (16, 256):
        cb = np.sort(rng.standard_normal(K).astype(np.float32))
        cb[3] = cb[4]  # a duplicate entry: the lower index wins
        f = vqx.codebook_format(cb)
        t = f.tables("cuda")
        assert np.array_equal(t["index_table"].cpu().numpy().astype(np.int64), F.codebook_index_table(cb))


@pytest.mark.gpu
def test_gpu_decode_tables(vqx):
    for d in ["fp8_e4m3", "fp6_e3m2", "fp4_e2m1", "posit8_1", "nf4", "int8"]:
        f = vqx.parse_format(d)
        t = f.tables("cuda")
        vals, codes, dtab = t["values"].cpu(), t["codes"].cpu().long() & ((1 << f.code_bits) - 1), t["decode"].cpu()
        fin = torch.isfinite(vals.float()) & torch.isfinite(F_to(F.ALL_BF16))
        got, want = dtab[codes[fin]], vals[fin]
        if d.startswith("int"):
            # int codes carry no sign of zero: code 0 decodes to +0
            got, want = got.float() + 0.0, want.float() + 0.0
        assert_bitexact(got, want, d)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["fp8_e4m3", "fp6_e3m2", "fp4_e2m1", "fp8_e5m2", "e4m3", "posit8_1",
                                   "posit8_2", "int8", "uint8", "int4", "nf4", "nf4_6", "fp8_e5m3"])
def test_gpu_lut_matches_full_table(vqx, dtype):
    """The compact table, read the way the kernels read it, reproduces the
    full 65536-entry table for every pattern below its special threshold."""
    f = vqx.parse_format(dtype)
    t = f.tables("cuda")
    assert "lut" in t, f"{dtype}: no compact table"
    blob = t["lut"].cpu().numpy().view(np.uint32)
    valid, t0m1, t1, S, ln, zsign = blob[:6]
    assert valid == 1
    pos = blob[16:16 + ln]
    neg = blob[16 + ln:16 + 2 * ln]
    full = blob[16 + 2 * 8192:16 + 2 * 8192 + 65536]
    h = np.arange(65536, dtype=np.int64)
    a = h & 0x7FFF
    sel = a < S
    c = np.clip(a, t0m1, t1) - t0m1
    negf = ((a != 0) | (zsign == 1)) & (h >> 15 == 1)
    e = np.where(negf, neg[c], pos[c])
    assert np.array_equal(e[sel], full[sel])
    vals = t["values"].cpu().view(torch.int16).numpy().view(np.uint16).astype(np.uint32)
    assert np.array_equal(full & 0xFFFF, vals)


def F_to(u):
    return torch.from_numpy(F.bf16_to_f32(u))
