"""The device encoders of vqx_formats.h, compiled for the host with g++, over
all 65536 bf16 inputs against the oracle (no GPU needed).  The same header
is what the HIP kernels run."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import formats as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
P = ctypes.c_void_p


@pytest.fixture(scope="module")
def host(tmp_path_factory):
    out = tmp_path_factory.mktemp("host") / "formats_host.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
                    "-I", os.path.join(ROOT, "voyager-compiler_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "formats_host.cpp"), "-o", str(out)],
                   check=True)
    return ctypes.CDLL(str(out))


def enc(lib, kind, p0=0, p1=0, mx=0.0, flags=0, b=None, lv=None):
    n = 65536
    code = np.zeros(n, np.uint32)
    val = np.zeros(n, np.uint16)
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    ll = None if lv is None else np.ascontiguousarray(lv, np.uint16)
    rc = lib.vqx_host_encode(kind, p0, p1, ctypes.c_float(mx), flags,
                             None if bb is None else bb.ctypes.data_as(P),
                             None if ll is None else ll.ctypes.data_as(P), 0 if lv is None else len(lv),
                             F.ALL_BF16.ctypes.data_as(P), ctypes.c_int64(n), code.ctypes.data_as(P),
                             val.ctypes.data_as(P))
    assert rc == 0
    return code, val


def same(a, b):
    fa, fb = F.bf16_to_f32(a), F.bf16_to_f32(b)
    return (a == b) | (np.isnan(fa) & np.isnan(fb))


def test_log2floor(host):
    out = np.zeros(65536, np.int32)
    host.vqx_host_log2floor(F.ALL_BF16.ctypes.data_as(P), ctypes.c_int64(65536), out.ctypes.data_as(P))
    a = F.ALL_BF16 & 0x7FFF
    m = (a != 0) & (a < 0x7F80)
    assert np.array_equal(out[m], F.log2floor_bf16(F.ALL_BF16)[m])


@pytest.mark.parametrize("n,es", [(8, 1), (8, 0), (8, 2), (6, 1), (16, 1), (10, 2), (4, 0)])
def test_posit(host, n, es):
    c, v = enc(host, 5, n, es)
    assert same(v, F.posit_table(n, es)).all()
    assert np.array_equal(c, F.posit_codes(F.ALL_BF16, n, es) & ((1 << n) - 1))


@pytest.mark.parametrize("dtype", ["fp8_e4m3", "fp8_e5m2", "fp6_e3m2", "fp6_e2m3", "fp4_e2m1",
                                   "fp8_e5m3", "fp8_e8m0", "fp16_e5m10", "fp8_e3m4", "fp5_e2m2"])
def test_fp_core(host, dtype):
    eb, mb, mx, uns = F.fp_core_params(dtype)
    c, v = enc(host, 3, eb, mb, mx, int(uns))
    assert same(v, F.fp_core_table(eb, mb, mx, uns)).all()


@pytest.mark.parametrize("dtype", ["fp8_e4m3", "fp6_e3m2", "fp4_e2m1", "fp6_e2m3"])
def test_fp_codes_decode_to_values(host, dtype):
    # OCP element decode of the code reproduces the value (finite inputs)
    eb, mb, mx, uns = F.fp_core_params(dtype)
    c, v = enc(host, 3, eb, mb, mx, int(uns))
    nb = eb + mb + (0 if uns else 1)
    emin = 2 - 2 ** (eb - 1)
    vals = F.bf16_to_f32(v).astype(np.float64)
    fin = np.isfinite(vals)
    s = (c >> (eb + mb)) & 1 if not uns else np.zeros_like(c)
    e = (c >> mb) & ((1 << eb) - 1)
    m = c & ((1 << mb) - 1)
    dec = np.where(e == 0, m / 2.0**mb * 2.0**emin, (1 + m / 2.0**mb) * 2.0 ** (e.astype(np.int64) - 1 + emin))
    dec = np.where(s == 1, -dec, dec)
    assert np.all(dec[fin] == vals[fin])
    assert np.all(c < (1 << nb))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_nv_fp8(host, fmt):
    c, v = enc(host, 4, 4 if fmt == "e4m3" else 5)
    assert same(v, F.nv_fp8_table(fmt)).all()


@pytest.mark.parametrize("n,signed", [(8, 1), (4, 1), (8, 0), (4, 0), (2, 1)])
def test_int(host, n, signed):
    c, v = enc(host, 2, n, signed)
    assert same(v, F.int_table(n, bool(signed))).all()


@pytest.mark.parametrize("k,ib", [(4, None), (4, 6), (3, None), (2, None)])
def test_levels_boundaries(host, k, ib):
    lv = F.nf_levels(k, ib)
    idx = F.nf_index_table(lv)
    x = F.bf16_to_f32(F.ALL_BF16)
    fin = ~np.isnan(x)
    b = np.array([x[fin][idx[fin] >= j].min() for j in range(1, len(lv))], np.float32)
    c, v = enc(host, 6, b=b, lv=lv)
    assert np.array_equal(c, idx)
    assert np.array_equal(v, lv[idx])


def pow2_ceil_inputs():
    """fp32 patterns around every power of two: the lowest and highest 64
    mantissas of every binade, random mantissas, subnormals near each power of
    two, zeros, negatives, Inf and NaN."""
    g = np.random.default_rng(5)
    E = np.arange(1, 255, dtype=np.int64)[:, None] << 23
    low = (E | np.arange(64)).reshape(-1)
    high = (E | (0x7FFFFF - np.arange(64))).reshape(-1)
    rnd = (E | g.integers(0, 1 << 23, (254, 8))).reshape(-1)
    sub = np.concatenate([(1 << k) + np.arange(min(64, 1 << k)) for k in range(23)])
    special = np.array([0, 0x80000000, 0xBF800000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F7FFFFF], np.int64)
    return np.concatenate([low, high, rnd, sub, special]).astype(np.uint32)


def test_pow2_ceil_log2_matches_torch_cpu(host):
    # the observer's force_scale_power_of_two (fake_quantize.py:339-340):
    # torch.pow(2, torch.ceil(torch.log2(sf))) on the CPU, both through
    # torch's vectorised path (a long tensor) and its scalar path (1 element)
    import torch

    bits = pow2_ceil_inputs()
    out = np.zeros_like(bits)
    host.vqx_host_pow2_ceil_log2(bits.ctypes.data_as(P), ctypes.c_int64(bits.size), out.ctypes.data_as(P))
    x = torch.from_numpy(bits.view(np.int32)).view(torch.float32)
    want = torch.pow(2, torch.ceil(torch.log2(x))).numpy().view(np.uint32)
    got_f, want_f = out.view(np.float32), want.view(np.float32)
    ok = (out == want) | (np.isnan(got_f) & np.isnan(want_f))
    assert ok.all(), [(hex(b), hex(o), hex(w)) for b, o, w in zip(bits[~ok][:8], out[~ok][:8], want[~ok][:8])]
    one = np.array([torch.pow(2, torch.ceil(torch.log2(x[i:i + 1])))[0].item() for i in range(0, x.numel(), 7)],
                   np.float32)
    sel = got_f[::7]
    assert ((sel.view(np.uint32) == one.view(np.uint32)) | (np.isnan(sel) & np.isnan(one))).all()
    # the rule keeps 2^p for the first mantissas above 2^p at larger |p|
    # (e.g. 16 * (1 + 2^-23)), where the exact ceiling would be 2^(p+1)
    assert out[np.where(bits == ((4 + 127) << 23 | 1))[0][0]] == (4 + 127) << 23
