"""The CPU oracle pinned: against the golden tables written from the
reference's own leaf functions, and against textbook facts that a dropped
term, wrong sign or off-by-one in the oracle would break."""

import math
import re

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R

GOLDEN_DTYPES = ["posit8_1", "posit8_0", "posit8_2", "posit6_1", "posit16_1", "fp8_e4m3", "fp8_e5m2",
                 "fp6_e3m2", "fp6_e2m3", "fp4_e2m1", "fp8_e5m3", "fp8_e8m0", "fp16_e5m10", "e4m3",
                 "e5m2", "nf4", "nf4_6", "nf3", "int8", "int4", "uint8", "uint4"]


def same_bits(a, b):
    fa, fb = F.bf16_to_f32(a), F.bf16_to_f32(b)
    return (a == b) | (np.isnan(fa) & np.isnan(fb))


@pytest.mark.parametrize("dtype", GOLDEN_DTYPES)
def test_table_matches_golden(dtype, golden):
    t = F.quantization_table(dtype)
    ok = same_bits(t, golden["t_" + dtype])
    assert ok.all(), f"{dtype}: {int((~ok).sum())} patterns differ"


@pytest.mark.parametrize("name,k,ib", [("nf4", 4, None), ("nf4_6", 4, 6), ("nf3", 3, None)])
def test_nf_levels_and_index(name, k, ib, golden):
    lv = F.nf_levels(k, ib)
    assert np.array_equal(lv, golden["nf_values_" + name])
    assert np.array_equal(F.nf_index_table(lv), golden["nf_index_" + name].astype(np.int64))


def test_nf4_levels_are_the_published_constants():
    # QLoRA / bitsandbytes NF4 levels; after the bf16 cast they pin the map.
    pub = np.array([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
                    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], np.float32)
    assert np.array_equal(F.nf_levels(4), F.f32_to_bf16(pub))


def test_log2floor_matches_torch(golden):
    a = F.ALL_BF16
    m = ((a & 0x7FFF) != 0) & ((a & 0x7FFF) < 0x7F80)
    assert np.array_equal(F.log2floor_bf16(a)[m], golden["log2floor"].astype(np.int32)[m])


def test_log2floor_margin_and_quirk():
    # every bf16 log2 lies >= 8 fp32 ulps from a bf16 rounding boundary, so any
    # fp32 log2 within a few ulps floors the same way
    a = np.arange(1, 0x7F80, dtype=np.uint32).astype(np.uint16)
    v = F.bf16_to_f32(a).astype(np.float64)
    lg = np.log2(v)
    m, e = np.frexp(lg)
    frac = m * 256 - np.floor(m * 256)
    dist = np.abs(frac - 0.5) * np.exp2(e - 8)
    nz = lg != 0
    assert (dist[nz] / np.abs(lg[nz])).min() > 8 * 2.0**-24
    # the reference quirk: 31.75 floors to 5 in bf16, 7.96875 to 3
    for x, want in [(31.75, 5), (7.96875, 3), (1.9921875, 0), (0.5, -1), (2.0**-126, -126)]:
        assert F.log2floor_bf16(F.f32_to_bf16(np.float32([x])))[0] == want


def test_posit_decode_is_the_textbook_bijection():
    for n, es in [(8, 1), (8, 0), (8, 2), (6, 1)]:
        vals = F.posit_decode(np.arange(1 << n), n, es)
        assert vals[0] == 0 and np.isnan(vals[1 << (n - 1)])
        pos = vals[1:1 << (n - 1)]
        assert np.all(np.diff(pos) > 0), "positive codes decode in increasing order"
        assert pos[0] == 2.0 ** (-(n - 2) * (1 << es))  # minpos
        assert pos[-1] == 2.0 ** ((n - 2) * (1 << es))  # maxpos
        neg = vals[(1 << (n - 1)) + 1:]
        assert np.array_equal(neg, -pos[::-1]), "two's complement negation"
    # posit8 es=1 spot values: 0x40 = 1, 0x50 = 2, 0x48 = 1.5, 0x30 = 0.5
    v = F.posit_decode(np.array([0x40, 0x50, 0x48, 0x30, 0x7F, 0x01]), 8, 1)
    assert list(v) == [1.0, 2.0, 1.5, 0.5, 4096.0, 2.0**-12]


def test_posit_codes_decode_to_table_values():
    for n, es in [(8, 1), (8, 0), (8, 2), (6, 1)]:
        codes = F.posit_codes(F.ALL_BF16, n, es)
        table = F.bf16_to_f32(F.posit_table(n, es))
        dec = F.posit_decode(np.arange(1 << n), n, es)[codes]
        both = np.isnan(dec) & np.isnan(table)
        assert np.all((dec.astype(np.float32) == table) | both)


def test_posit_rounding_brute_force():
    # nearest posit in log-free arithmetic with ties to the even code, on
    # inputs between minpos and maxpos (the reference's special rules aside)
    n, es = 8, 1
    dec = F.posit_decode(np.arange(1, 1 << (n - 1)), n, es)
    xs = F.bf16_to_f32(np.arange(0x3980, 0x4580, dtype=np.uint32).astype(np.uint16)).astype(np.float64)
    codes = F.posit_codes(F.f32_to_bf16(xs.astype(np.float32)), n, es)
    for x, c in zip(xs, codes):
        # candidates: the posits bracketing x
        hi = np.searchsorted(dec, x)
        lo = hi - 1
        if dec[min(hi, len(dec) - 1)] == x:
            want = hi + 1
        else:
            # bit-string RNE compares x with the midpoint of the two codes'
            # real-valued bit strings; within a binade that is the arithmetic
            # midpoint, across a regime/exponent boundary the geometric one
            a, b = dec[lo], dec[hi]
            mid = (a + b) / 2 if (b / a) <= 2 and math.floor(math.log2(a)) == math.floor(math.log2(b) - 1e-12) \
                else math.sqrt(a * b)
            if x < mid:
                want = lo + 1
            elif x > mid:
                want = hi + 1
            else:
                want = lo + 1 if (lo + 1) % 2 == 0 else hi + 1
        assert c == want, (x, c, want)


@pytest.mark.parametrize("dtype,grid_max,sub", [("fp8_e4m3", 448.0, 2.0**-9), ("fp6_e3m2", 28.0, 2.0**-4),
                                                ("fp4_e2m1", 6.0, 0.5), ("fp6_e2m3", 7.5, 2.0**-3)])
def test_fp_tables_follow_ocp_grids(dtype, grid_max, sub):
    eb, mb, mx, _ = F.fp_core_params(dtype)
    assert mx == grid_max
    # OCP MX v1.0 element grid: subnormal spacing, normals with mb bits, max
    emin = 2 - 2 ** (eb - 1)
    grid = {0.0}
    for e in range(emin, 40):
        for k in range(1 << mb):
            v = 2.0**e * (1 + k / 2**mb)
            if v <= grid_max:
                grid.add(v)
    for k in range(1, 1 << mb):
        grid.add(2.0**emin * k / 2**mb)
    grid = np.array(sorted(grid))
    assert grid[1] == sub
    t = F.bf16_to_f32(F.quantization_table(dtype)).astype(np.float64)
    x = F.bf16_to_f32(F.ALL_BF16).astype(np.float64)
    fin = np.isfinite(x) & (np.abs(x) < 2.0**127 * 1.6875)
    assert set(np.unique(np.abs(t[fin]))) <= set(grid)
    # nearest grid value (ties to even mantissa) for in-range magnitudes,
    # saturation above
    ax = np.abs(x[fin])
    i = np.clip(np.searchsorted(grid, ax), 1, len(grid) - 1)
    lo, hi = grid[i - 1], grid[i]
    near = np.where(ax - lo < hi - ax, lo, hi)
    tie = (ax - lo) == (hi - ax)
    inr = ax <= grid_max
    sel = inr & ~tie
    # the reference's one bf16 quirk: (0.5 - 2^-9) of the smallest subnormal
    # step rounds up (floor(bf16(0.498046875 + 0.5)) = 1)
    quirk = ax / sub == 0.5 - 2.0**-9
    assert np.all(np.abs(t[fin])[sel & ~quirk] == near[sel & ~quirk])
    assert np.all(np.abs(t[fin])[ax > grid_max] == grid_max)


def test_int_tables_are_round_half_even_and_clamp():
    t = F.bf16_to_f32(F.int_table(8)).astype(np.float64)
    x = F.bf16_to_f32(F.ALL_BF16).astype(np.float64)
    fin = np.isfinite(x)
    assert np.array_equal(t[fin], np.clip(np.round(x[fin]), -128, 127))
    assert F.bf16_to_f32(F.int_table(8, u16=F.f32_to_bf16(np.float32([2.5, 3.5, -2.5]))))[:3].tolist() == [2, 4, -2]


def test_nf_index_is_brute_force_argmin():
    lv = F.nf_levels(4)
    lvf = F.bf16_to_f32(lv).astype(np.float64)
    x = F.bf16_to_f32(F.ALL_BF16)
    idx = F.nf_index_table(lv)
    fin = np.isfinite(x) & (np.abs(x) <= 1)
    # exact-arithmetic argmin agrees except where bf16-rounded distances tie
    d = np.abs(lvf[None, :] - x[fin, None].astype(np.float64))
    exact = d.argmin(1)
    ok = idx[fin] == exact
    close = np.sort(d, 1)[:, 1] - np.sort(d, 1)[:, 0] < 2.0**-7 * np.sort(d, 1)[:, 0] + 1e-30
    assert np.all(ok | close)
    assert (ok | close).sum() == fin.sum()


def test_codebook_index_brute_force():
    rng = np.random.default_rng(0)
    cb = np.sort(rng.standard_normal(16).astype(np.float32))
    idx = F.codebook_index_table(cb)
    x = F.bf16_to_f32(F.ALL_BF16)
    fin = np.isfinite(x)
    xc = np.clip(x[fin], cb[0], cb[-1])
    for j in range(0, fin.sum(), 997):
        d = np.abs((xc[j] - cb).astype(np.float32))
        assert idx[fin][j] == int(np.flatnonzero(d == d.min())[0])


def test_mx_scale_oracle_against_closed_form():
    # calculate_mx_qparam on one block per bf16 amax value, pow2 mode:
    # 2^(floor(bf16 log2 amax) - floor(log2 qmax)), zero -> 2^(-126-shift),
    # bf16 underflow to 0 -> 1
    a = np.arange(0, 0x7F80, 37, dtype=np.uint32).astype(np.uint16)
    x = R.table_tensor(a).reshape(-1, 1)
    for qmax, shift in [(448.0, 8), (28.0, 4), (6.0, 2)]:
        s = R.calculate_mx_qparam(x, [-1], 1, qmax, True).float().reshape(-1).numpy()
        e = np.where(a == 0, -126, F.log2floor_bf16(a)) - shift
        want = np.where(e >= -133, np.exp2(e.astype(np.float64)), 0.0)
        want = np.where(want > 0, want, 1.0)
        assert np.array_equal(s, want.astype(np.float32))


def test_oracle_vmap_chunks_and_dtypes():
    t = R.table_tensor(F.posit_table(8, 1))
    x = torch.randn(3 * (1 << 20) + 5)
    y = R.vmap(x, t, chunk_size=1 << 20)
    h = F.f32_to_bf16(x.numpy())
    assert np.array_equal(y.numpy().view(np.uint32), F.bf16_to_f32(F.posit_table(8, 1)[h]).view(np.uint32))


# ---------------------------------------------------------------------------
# group-wise affine fake-quant (fake_quantize.py:162-211)
# ---------------------------------------------------------------------------
GWA = R.group_wise_affine_fake_quant


def test_gwa_identity_on_the_grid():
    """Blocks whose min is 0 and max is qmax - qmin hold sf = 1, zp = 0, so
    integer inputs come back unchanged (a wrong sign in zp, a dropped qmin
    or a swapped min / max would move them)."""
    x = torch.tensor([[0.0, 1.0, 2.0, 3.0, 3.0, 0.0, 1.0, 2.0]])
    sf, zp, y = GWA(x, -1, 4, 0, 3)
    assert torch.equal(sf, torch.ones(1, 2)) and torch.equal(zp, torch.zeros(1, 2))
    assert torch.equal(y, x)
    x2 = torch.tensor([[-8.0, -3.0, 0.0, 7.0]])
    sf, zp, y = GWA(x2, -1, 4, -8, 7)  # int4: sf = 15 / 15 = 1, zp = 8 - 8 = 0
    assert torch.equal(sf, torch.ones(1, 1)) and torch.equal(zp, torch.zeros(1, 1)) and torch.equal(y, x2)


def test_gwa_constant_block_and_shift():
    """A constant block has max - min = 0, so sf becomes 1 and zp = qmin - c:
    the block is reproduced exactly; shifting a grid block by an integer
    shifts only zp."""
    x = torch.full((1, 4), 5.0)
    sf, zp, y = GWA(x, -1, 4, 0, 3)
    assert sf.item() == 1.0 and zp.item() == -5.0 and torch.equal(y, x)
    base = torch.tensor([[0.0, 1.0, 2.0, 3.0]])
    sf, zp, y = GWA(base + 10.0, -1, 4, 0, 3)
    assert sf.item() == 1.0 and zp.item() == -10.0 and torch.equal(y, base + 10.0)


def test_gwa_short_block_is_zero_padded():
    """mx_utils.py:62-108 pads a short last block with zeros before min / max:
    the result equals that of the explicitly padded tensor, trimmed."""
    g = torch.Generator().manual_seed(11)
    x = torch.rand(3, 10, generator=g) + 2.0          # all positive: the padding zero becomes the min
    xp = torch.cat([x, torch.zeros(3, 2)], dim=1)
    for dt in (torch.float32, torch.bfloat16):
        sf, zp, y = GWA(x.to(dt), -1, 4, 0, 3)
        sfp, zpp, yp = GWA(xp.to(dt), -1, 4, 0, 3)
        assert torch.equal(sf, sfp) and torch.equal(zp, zpp) and torch.equal(y, yp[:, :10])
        assert (zp[:, -1] == 0).all()                  # min = 0 in the padded block


def test_gwa_levels_and_error_bound():
    """Each block's outputs take at most qmax - qmin + 1 distinct values, and
    in fp32 every output is within sf / 2 (plus rounding) of its input."""
    g = torch.Generator().manual_seed(12)
    x = torch.randn(16, 256, generator=g)
    for qmin, qmax in ((0, 3), (-8, 7), (0, 255)):
        sf, zp, y = GWA(x, 1, 64, qmin, qmax)
        for b in range(4):
            yb = y[:, 64 * b:64 * (b + 1)]
            for r in range(16):
                assert yb[r].unique().numel() <= qmax - qmin + 1
        err = (y - x).abs()
        bound = R.expand(sf, x.shape, 64) * (0.5 + 1e-4)
        assert (err <= bound).all()


def test_gwa_matches_a_per_block_loop():
    """The vectorised oracle against a per-block scalar loop over another axis
    (blocks along dim 0 of a 3-d tensor), bf16 arithmetic step by step."""
    g = torch.Generator().manual_seed(13)
    x = (torch.randn(10, 3, 5, generator=g) * 4).to(torch.bfloat16)
    sf, zp, y = GWA(x, 0, 4, 0, 3)
    bf = torch.bfloat16
    for j in range(3):
        for k in range(5):
            for b in range(3):                            # blocks of rows 0-3, 4-7, 8-9 (+2 zero rows)
                col = x[4 * b:4 * b + 4, j, k]
                vals = col.tolist() + [0.0] * (4 - col.numel())
                mn, mx = min(vals), max(vals)
                s = ((torch.tensor(mx, dtype=bf) - torch.tensor(mn, dtype=bf)) / 3)
                s = s if s.item() > 0 else torch.tensor(1.0, dtype=bf)
                z = (-torch.tensor(mn, dtype=bf)) / s + 0
                assert sf[b, j, k] == s and zp[b, j, k] == z
                for i in range(col.numel()):
                    q = torch.clamp(torch.round(col[i] / s + z), 0, 3)
                    assert y[4 * b + i, j, k] == (q - z) * s


def test_int_table_wide_formats_match_the_reference_expression():
    # get_quantization_map for int<n> / uint<n> (fake_quantize.py:42-52) is
    # torch.clamp(torch.round(values), qmin, qmax) on the bf16 patterns; the
    # golden tables hold 4 and 8 bits, this covers the bias widths
    import torch

    vals = torch.arange(2**16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    def same(got_u16, want_bf16):
        w = want_bf16.view(torch.int16).numpy().view(np.uint16)
        nan = np.isnan(F.bf16_to_f32(got_u16)) & torch.isnan(want_bf16).numpy()  # NaN as a class
        return bool(((got_u16 == w) | nan).all())

    for n in (12, 16, 24, 31):
        assert same(F.int_table(n), torch.clamp(torch.round(vals), -(2 ** (n - 1)), 2 ** (n - 1) - 1)), n
        assert same(F.int_table(n, signed=False), torch.clamp(torch.round(vals), 0, 2**n - 1)), n


def test_bf16_quotients_stay_clear_of_bf16_midpoints():
    # The absmax kernels compute x / s for bf16 x and s as x * rcp(s), whose
    # error (v_rcp_f32's 1 ulp plus the product's rounding) stays below 2^-22
    # relative; that rounds like the reference's fp32 division to bf16 only
    # because an exact quotient of two 8-bit significands is never within
    # 2^-17 (relative) of a bf16 rounding midpoint.  Exhaustive over the
    # significands (1..255 covers the subnormals' shorter ones).
    from fractions import Fraction

    worst = Fraction(1)
    for X in range(1, 256):
        for S in range(1, 256):
            r = Fraction(X, S)
            e = math.floor(math.log2(X) - math.log2(S))
            m = r / Fraction(2) ** e
            while m >= 2:
                m /= 2
            while m < 1:
                m *= 2
            k = math.floor((m - 1) * 128)  # the bf16 value below m is 1 + k / 128
            for mid in (1 + Fraction(2 * k + 1, 256), 1 + Fraction(2 * k - 1, 256)):
                worst = min(worst, abs(m - mid) / m)
    assert worst > Fraction(1, 2**17), float(worst)
