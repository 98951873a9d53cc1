"""CPU oracle, part 1: the reference's element formats as 65536-entry tables.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``voyager-compiler_amd/``)
may import this package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker.

Every reference quantizer is a lookup table indexed by the bf16 bit pattern of
its input (``get_quantization_map``, src/voyager_compiler/quantization/
fake_quantize.py:30-98).  This module restates each format's table in numpy,
in closed form on the bit pattern, with every bf16 rounding step of the
reference's own arithmetic emulated explicitly.  Parity of every table here is
pinned exhaustively (all 2^16 patterns) against ``tests/golden/tables.npz``,
which was written from the reference's leaf format functions, and by the
textbook checks in ``tests/test_oracle.py`` (posit decode, OCP FP grids,
brute-force argmin, floor(log2) margins).

Array conventions: ``u16`` = bf16 bit patterns (np.uint16), ``f32`` = float32.
"""

import math
import re

import numpy as np

__all__ = [
    "ALL_BF16",
    "bf16_to_f32",
    "f32_to_bf16",
    "bf16_round",
    "log2floor_bf16",
    "posit_table",
    "posit_codes",
    "posit_decode",
    "fp_core_table",
    "fp_core_params",
    "nv_fp8_table",
    "int_table",
    "nf_levels",
    "nf_index_table",
    "codebook_index_table",
    "quantization_table",
]

ALL_BF16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)


# ----------------------------------------------------------------------------
# bf16 <-> fp32
# ----------------------------------------------------------------------------
def bf16_to_f32(u16):
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f32):
    """Round-to-nearest-even fp32 -> bf16 bit pattern; NaN -> 0x7FC0.

    Matches c10::BFloat16's conversion, which torch uses for ``.to(bfloat16)``
    and for the result of every bf16 CPU arithmetic op.
    """
    f = np.ascontiguousarray(f32, dtype=np.float32)
    b = f.view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    out = (r & 0xFFFF).astype(np.uint16)
    return np.where(np.isnan(f), np.uint16(0x7FC0), out)


def bf16_round(f32):
    """The fp32 value of ``f32`` rounded to bf16 (RNE)."""
    return bf16_to_f32(f32_to_bf16(f32))


def _round_f64_to_bf16(x):
    """RNE of float64 values to 8 significant bits (normal bf16 range only)."""
    x = np.asarray(x, dtype=np.float64)
    m, e = np.frexp(x)  # x = m * 2**e, 0.5 <= |m| < 1
    return np.ldexp(np.rint(m * 256.0), e - 8)


# ----------------------------------------------------------------------------
# floor(log2(a)) evaluated in bf16
# ----------------------------------------------------------------------------
def log2floor_bf16(u16):
    """``floor(bf16(log2(|a|)))`` for bf16 patterns with |a| > 0 finite.

    torch evaluates ``log2`` of a bf16 tensor in fp32 and rounds the result to
    bf16 (mx_utils.py:43-47 and fp8.py:193-197 both call it on bf16 data), so
    for mantissas close to 2 the floor lands one above the true exponent
    (31.75 -> 5).  Here the true log2 is taken in float64 and rounded to bf16;
    ``tests/test_oracle.py`` shows every value lies far enough from a bf16
    rounding boundary that fp32-accurate log2 rounds the same way, and pins
    the result against torch's own table.  Zero/NaN/Inf inputs return
    -32768 (callers handle them).
    """
    u = np.asarray(u16, dtype=np.uint16) & np.uint16(0x7FFF)
    with np.errstate(invalid="ignore"):
        v = bf16_to_f32(u).astype(np.float64)
    out = np.full(u.shape, -32768, dtype=np.int32)
    ok = (u != 0) & (u < 0x7F80)
    with np.errstate(divide="ignore"):
        lg = np.log2(np.where(ok, v, 1.0))
    out[ok] = np.floor(_round_f64_to_bf16(lg[ok])).astype(np.int32)
    return out


# ----------------------------------------------------------------------------
# posit(n, es)   (dtypes/posit.py:8-73, routed from fake_quantize.py:84-88)
# ----------------------------------------------------------------------------
def _posit_threshold_exp(nbits, es):
    # posit.py:54-56: |x| below 2^floor(-(n-1)*2^es + 2^(es-1)) flushes to 0
    return math.floor(-(nbits - 1) * (1 << es) + 2.0 ** (es - 1))


def posit_codes(u16, nbits, es):
    """Posit code (two's complement, nbits wide) of each bf16 input.

    The code is the bit-string round-to-nearest-even of the posit encoding
    (sign, regime run + terminator, es exponent bits, fraction), which is what
    the reference's lb/gb/sb rounding on ``pt_bits`` computes (posit.py:28-49),
    together with its three special rules: |x| < 2^floor(-(n-1)2^es + 2^(es-1))
    flushes to zero (posit.py:52-57), a regime longer than the word saturates
    to maxpos / minpos (posit.py:20-21, :37, :42), and non-finite inputs give
    NaR (posit.py:61).  Both zeros give code 0.
    """
    u = np.asarray(u16, dtype=np.uint16).astype(np.int64)
    neg = (u >> 15) & 1
    a = u & 0x7FFF
    E = a >> 7
    f = a & 0x7F
    scale = E - 127
    maxs = (nbits - 2) << es
    useed_mask = (1 << es) - 1

    k = scale >> es  # floor division
    e = scale & useed_mask
    kp = np.maximum(k, 0)
    reg = np.where(k >= 0, ((np.int64(1) << (kp + 1)) - 1) << 1, 1)
    rlen = np.where(k >= 0, k + 2, -k + 1)
    body = (((reg << es) | e) << 7) | f
    blen = rlen + es + 7
    cut = blen - (nbits - 1)
    cpos = np.maximum(cut, 0)
    c = np.where(cut <= 0, body << np.maximum(-cut, 0), body >> cpos)
    g = np.where(cut > 0, (body >> np.maximum(cut - 1, 0)) & 1, 0)
    st = np.where(cut > 1, (body & ((np.int64(1) << np.maximum(cut - 1, 0)) - 1)) != 0, False)
    c = c + (g & (st | (c & 1)))

    c = np.where(scale > maxs, (1 << (nbits - 1)) - 1, c)
    c = np.where(scale < -maxs, 1, c)
    t = _posit_threshold_exp(nbits, es)
    thr_bits = (t + 127) << 7 if t >= -126 else (1 << max(t + 133, 0))
    c = np.where(a < thr_bits, 0, c)
    c = np.where(a == 0, 0, c)
    mod = 1 << nbits
    c = np.where(neg == 1, (mod - c) % mod, c)
    c = np.where(E == 255, 1 << (nbits - 1), c)
    return c.astype(np.int64)


def posit_decode(codes, nbits, es):
    """Textbook decode of posit(n, es) codes to float64 (NaR -> nan)."""
    c = np.asarray(codes, dtype=np.int64) & ((1 << nbits) - 1)
    out = np.zeros(c.shape, dtype=np.float64)
    for i, ci in np.ndenumerate(c):
        ci = int(ci)
        if ci == 0:
            continue
        if ci == 1 << (nbits - 1):
            out[i] = np.nan
            continue
        neg = ci >> (nbits - 1)
        if neg:
            ci = (1 << nbits) - ci
        bits = [(ci >> (nbits - 2 - j)) & 1 for j in range(nbits - 1)]
        first = bits[0]
        run = 1
        while run < len(bits) and bits[run] == first:
            run += 1
        k = run - 1 if first == 1 else -run
        rest = bits[run + 1:]
        ebits = rest[:es] + [0] * max(0, es - len(rest))
        e = 0
        for b in ebits:
            e = (e << 1) | b
        frac = rest[es:]
        fv = 1.0
        for j, b in enumerate(frac):
            fv += b * 2.0 ** -(j + 1)
        v = 2.0 ** (k * (1 << es) + e) * fv
        out[i] = -v if neg else v
    return out


def posit_table(nbits, es):
    """bf16 table of posit(n, es) fake-quant values (the reference's LUT)."""
    codes = posit_codes(ALL_BF16, nbits, es)
    dec = posit_decode(np.arange(1 << nbits), nbits, es)
    vals = dec[codes]
    return f32_to_bf16(vals.astype(np.float32))


# ----------------------------------------------------------------------------
# fpN_eXmY via the microscaling element core (dtypes/fp8.py:160-225)
# ----------------------------------------------------------------------------
def fp_core_params(dtype):
    """(ebits, mbits, max_norm, unsigned) as fake_quantize.py:63-80 derives them."""
    m = re.fullmatch(r"fp(\d+)_e(\d+)m(\d+)", dtype)
    if m is None:
        raise ValueError(dtype)
    nbits, ebits, mbits = map(int, m.groups())
    assert nbits == ebits + mbits + 1 or nbits == ebits + mbits
    unsigned = nbits == ebits + mbits
    emax = 2 ** (ebits - 1) - 1 if ebits > 4 else 2 ** (ebits - 1)
    if dtype != "fp8_e4m3":
        max_norm = 2**emax * float(2 ** (mbits + 1) - 1) / 2**mbits
    else:
        max_norm = 2**emax * 1.75
    return ebits, mbits, max_norm, unsigned


def _bf(x):
    return bf16_round(np.asarray(x, dtype=np.float32))


def fp_core_table(ebits, mbits, max_norm, unsigned=False, u16=None):
    """bf16 table of ``_quantize_elemwise_core(A, mbits+2, ebits, max_norm,
    "even", saturate_normals=True)`` on bf16 ``A`` (fp8.py:160-225).

    Each step is evaluated as torch evaluates it on a bf16 tensor: the exact
    fp32 result of the step, rounded to bf16.
    """
    if u16 is None:
        u16 = ALL_BF16
    A = bf16_to_f32(u16)
    if unsigned:  # fake_quantize.py:68-69
        A = np.abs(A)
    A = _bf(A)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        absA0 = np.abs(A)
        arg = _bf(absA0 + (A == 0).astype(np.float32))
        pe = log2floor_bf16(f32_to_bf16(arg)).astype(np.float64)
        pe = np.where(np.isnan(A), np.nan, pe)
        pe = np.where(np.isinf(A), np.inf, pe)
        min_exp = -(2 ** (ebits - 1)) + 2
        pe = np.maximum(pe, min_exp)  # .clip keeps NaN
        pe = np.where(np.isnan(A), np.nan, pe)
        p2 = _bf(np.exp2(pe).astype(np.float32))  # 2**private_exp in bf16
        out = _bf(A / p2)
        out = _bf(out * np.float32(2.0**mbits))
        # _round_mantissa(..., "even")
        absA = np.abs(out)
        t1 = _bf(absA - np.float32(0.5))
        # torch's % is a floored remainder; only equality with 0 matters here
        mask = (t1 - 2.0 * np.floor(t1 / 2.0)) == 0
        mask = mask.astype(np.float32)
        t2 = np.floor(_bf(absA + np.float32(0.5)))
        sgn = np.sign(out).astype(np.float32)
        sgn = np.where(out == 0, np.float32(0.0), sgn)
        q = _bf(sgn * _bf(t2 - mask))
        out = _bf(q / np.float32(2.0**mbits))
        out = _bf(out * p2)
        mn = np.float32(_bf(np.float32(max_norm)))
        out = np.where(np.isnan(out), out, np.clip(out, -mn, mn))
        out = np.where(A == np.inf, np.float32(np.inf), out)
        out = np.where(A == -np.inf, np.float32(-np.inf), out)
    return f32_to_bf16(out.astype(np.float32))


# ----------------------------------------------------------------------------
# NVIDIA-style e4m3 / e5m2 (dtypes/fp8.py:13-74; fake_quantize.py:55-60)
# ----------------------------------------------------------------------------
def nv_fp8_table(fmt, u16=None):
    """Round-to-nearest-even onto the e4m3 (max 448, min normal 2^-6) or e5m2
    (max 57344, min normal 2^-14) grid with subnormals, saturating; inputs at or
    below half the smallest subnormal, and both zeros, give +0; non-finite
    inputs give NaN."""
    if u16 is None:
        u16 = ALL_BF16
    mbits, fmax, emin = (3, 448.0, -6) if fmt == "e4m3" else (2, 57344.0, -14)
    x = bf16_to_f32(u16).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        ax = np.abs(x)
        ex = np.floor(np.log2(np.where(ax > 0, ax, 1.0)))
        ex = np.maximum(ex, emin)
        ulp = np.exp2(ex - mbits)
        q = np.rint(ax / ulp) * ulp  # rint = half-to-even
        q = np.minimum(q, fmax)
        q = np.where(ax <= 2.0**emin * 2.0 ** -(mbits + 1), 0.0, q)
        v = np.where(x < 0, -q, q)
        v = np.where(x == 0, 0.0, v)
        v = np.where(np.isfinite(x), v, np.nan)
        v = np.where(v == 0, 0.0, v)  # torch.where(..., 0, ...) gives +0
    return f32_to_bf16(v.astype(np.float32))


# ----------------------------------------------------------------------------
# int / uint (fake_quantize.py:43-52)
# ----------------------------------------------------------------------------
def int_table(nbits, signed=True, u16=None):
    if u16 is None:
        u16 = ALL_BF16
    if signed:
        lo, hi = -(2 ** (nbits - 1)), 2 ** (nbits - 1) - 1
    else:
        lo, hi = 0, 2**nbits - 1
    x = bf16_to_f32(u16)
    with np.errstate(invalid="ignore"):
        r = np.rint(x)  # torch.round: half to even; keeps -0.0
    lo_b = _bf(np.float32(lo))
    hi_b = _bf(np.float32(hi))
    # torch.clamp is max-then-min with strict comparisons: -0.0 is not below
    # a lower bound of 0, so rounding a small negative to -0.0 survives it.
    with np.errstate(invalid="ignore"):
        r = np.where(r < lo_b, lo_b, r)
        r = np.where(r > hi_b, hi_b, r)
    return f32_to_bf16(r.astype(np.float32))


# ----------------------------------------------------------------------------
# NormalFloat (dtypes/normal_float.py:4-62)
# ----------------------------------------------------------------------------
def nf_levels(k=4, int_bits=None, offset=0.9677083, use_extra_value=True):
    """bf16 bit patterns of the sorted NF levels (normal_float.py:4-29, :54-58)."""
    from scipy.stats import norm

    n = 2 ** (k - 1)

    def lin(num):  # torch.linspace in fp32
        return np.linspace(offset, 0.5, num, dtype=np.float64).astype(np.float32)

    if use_extra_value:
        v = list(norm.ppf(lin(n + 1)[:-1].astype(np.float64))) + [0.0] + \
            list(-norm.ppf(lin(n)[:-1].astype(np.float64)))
    else:
        v = list(norm.ppf(lin(n)[:-1].astype(np.float64))) + [0.0, 0.0] + \
            list(-norm.ppf(lin(n)[:-1].astype(np.float64)))
    vals = np.sort(np.asarray(v, dtype=np.float32))
    vals = (vals / vals.max()).astype(np.float32)
    if int_bits is not None:
        vals = np.rint(vals * np.float32(2 ** (int_bits - 1) - 1)).astype(np.float32)
    return f32_to_bf16(vals)


def nf_index_table(levels_u16, u16=None):
    """argmin_k |level_k - clamp(x)| evaluated in bf16, first index on ties
    (normal_float.py:58-60).  NaN inputs give index 0 (argmin sees the NaN
    distances first)."""
    if u16 is None:
        u16 = ALL_BF16
    lv = bf16_to_f32(levels_u16)
    x = bf16_to_f32(u16)
    with np.errstate(invalid="ignore"):
        xc = np.where(np.isnan(x), x, np.clip(x, lv.min(), lv.max()))
        d = np.abs(_bf(lv[None, :] - xc[:, None]))
    d = np.where(np.isnan(d), -np.inf, d)
    return np.argmin(d, axis=1).astype(np.int64)


# ----------------------------------------------------------------------------
# Codebook (quantization/lcq.py:270-291)
# ----------------------------------------------------------------------------
def codebook_index_table(codebook_f32, u16=None):
    """argmin_k |clamp(x) - cb_k| in fp32, lowest index on ties (lcq.py:286-291)."""
    if u16 is None:
        u16 = ALL_BF16
    cb = np.asarray(codebook_f32, dtype=np.float32)
    x = bf16_to_f32(u16)
    with np.errstate(invalid="ignore"):
        xc = np.where(np.isnan(x), x, np.clip(x, cb.min(), cb.max()))
        d = np.abs((xc[:, None] - cb[None, :]).astype(np.float32))
    d = np.where(np.isnan(d), -np.inf, d)
    return np.argmin(d, axis=1).astype(np.int64)


# ----------------------------------------------------------------------------
# get_quantization_map routing (fake_quantize.py:30-98)
# ----------------------------------------------------------------------------
def quantization_table(dtype):
    """The 65536-entry bf16 table for a dtype string, as uint16 patterns.

    For ``nf*`` dtypes the reference returns (indices, values); FakeQuantize
    turns that into ``values[indices]`` (fake_quantize.py:274-277), which is
    what this returns.
    """
    if dtype in ("float32", "bfloat16"):
        return ALL_BF16.copy()
    if dtype == "float16":
        x = bf16_to_f32(ALL_BF16).astype(np.float16).astype(np.float32)
        return f32_to_bf16(x)
    if m := re.fullmatch(r"int(\d+)", dtype, re.IGNORECASE):
        return int_table(int(m.group(1)), True)
    if m := re.fullmatch(r"uint(\d+)", dtype, re.IGNORECASE):
        return int_table(int(m.group(1)), False)
    if m := re.fullmatch(r"(?:fp8\.)?(e4m3|e5m2)", dtype, re.IGNORECASE):
        return nv_fp8_table(m.group(1).lower())
    if re.fullmatch(r"fp(\d+)_e(\d+)m(\d+)", dtype):
        eb, mb, mx, uns = fp_core_params(dtype)
        return fp_core_table(eb, mb, mx, uns)
    if m := re.fullmatch(r"posit(\d+)_(\d+)", dtype):
        return posit_table(int(m.group(1)), int(m.group(2)))
    if m := re.fullmatch(r"nf(\d+)(?:_(\d+))?", dtype):
        lv = nf_levels(int(m.group(1)), int(m.group(2)) if m.group(2) else None)
        return lv[nf_index_table(lv)]
    raise ValueError(f"Unsupported dtype: {dtype}")
