"""CPU check of the decision-threshold construction that the GPU codebook
encoder (csrc/vqx_codebook.hip: exact_gap, code_threshold, the breadth-first
tree) relies on, restated here in numpy float32: for rows that pass the gap
condition, "number of thresholds <= v" must equal the reference's nearest
entry (clamp, argmin of fp32 |v - c|, lowest index on ties, NaN -> 0) for
every one of the 65536 bf16 patterns; rows that fail it take the exact
per-element search on the GPU (and the last test shows why they must).  The GPU kernel itself is checked against the
oracle in tests/test_gpu_codebook.py."""

import warnings

import numpy as np
import pytest

f32 = np.float32


def _u2f(u):
    return np.array([u], dtype=np.uint32).view(np.float32)[0]


def _f2u(x):
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def _bf2f(h):
    return _u2f(h << 16)


def _f2bf(x):
    u = _f2u(x)
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return (u >> 16) | 0x40
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def _key(h):
    return (h ^ 0xFFFF) if h & 0x8000 else (h | 0x8000)


def _unkey(k):
    return (k & 0x7FFF) if k & 0x8000 else (k ^ 0xFFFF)


def _exact_gap(lo, hi):
    r = f32(hi - lo)
    if not (r < np.inf):
        return np.inf
    e = _f2u(r) >> 23
    ulp = _u2f((e - 23) << 23) if e > 23 else _u2f(1 << (e - 1 if e > 0 else 0))
    return f32(4) * ulp


def _threshold(cb, i, gap, state):
    K = len(cb)
    a = cb[i]
    j = i + 1
    while j < K and not (cb[j] > a):
        j += 1
    if j == K:
        return None
    b = cb[j]
    if not (f32(b - a) >= gap):
        state["exact"] = False
    vmin, vmax = cb[0], cb[-1]

    def closer_to_b(k):
        v = _bf2f(_unkey(k))
        v = vmin if v < vmin else (vmax if v > vmax else v)
        return abs(f32(b - v)) < abs(f32(v - a))

    km = _key(_f2bf(f32(f32(0.5) * a + f32(0.5) * b)))
    if km - 2 >= 0x7F and km + 2 <= 0xFF80 and not closer_to_b(km - 2) and closer_to_b(km + 2):
        lo, hi = km - 2, km + 2
    else:
        lo = max(_key(_f2bf(a)) - 2, 0x7F)
        hi = min(_key(_f2bf(b)) + 2, 0xFF80)
    while lo + 1 < hi:
        mid = (lo + hi) >> 1
        if closer_to_b(mid):
            hi = mid
        else:
            lo = mid
    return _bf2f(_unkey(hi))


def _codebooks():
    rng = np.random.default_rng(5)
    n01 = np.sort(rng.standard_normal(64)).astype(np.float32)
    sym = np.sort(np.concatenate([n01[:8], -n01[:8]])).astype(np.float32)
    dup = np.sort(rng.standard_normal(17)).astype(np.float32)
    dup[5:9] = dup[5]
    dup[-3:] = dup[-3]
    sub = (np.sort(rng.standard_normal(16)) * np.float32(2.0 ** -130)).astype(np.float32)
    # entries spread over 40 binades (|c| from 5e-8 to 5e8): values near 258
    # are 258 away from several entries at once, and in fp32 those distances tie
    wide = np.array([-4.5617120e+08, -1.7806498e+04, -4.6088116e+02, -4.8019073e+01, -4.9426060e-02,
                     -6.8074833e-03, -2.1707090e-03, -9.7630935e-04, -5.2784779e-04, -8.3647523e-05,
                     -2.4869628e-06, -1.9292422e-07, -5.5566971e-08, 4.8861853e-06, 1.9638399e-05,
                     4.0374794e-05, 7.8944244e+02], dtype=np.float32)
    near = np.sort(rng.standard_normal(16)).astype(np.float32)
    near[1] = np.nextafter(near[0], np.float32(np.inf))
    return {"n01_64": n01, "symmetric_16": sym, "duplicates_17": dup, "subnormal_16": sub,
            "wide_range_17": wide, "ulp_apart_16": near, "single": np.array([0.5], np.float32)}


@pytest.mark.parametrize("name", list(_codebooks()))
def test_threshold_count_equals_nearest_entry(name):
    cb = _codebooks()[name]
    gap = _exact_gap(cb[0], cb[-1])
    state = {"exact": True}
    thr = [_threshold(cb, i, gap, state) for i in range(len(cb) - 1)]
    vals = (np.arange(0x10000, dtype=np.uint32) << 16).view(np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        want = np.abs(np.clip(vals, cb[0], cb[-1])[:, None] - cb[None, :]).argmin(1)
    want[np.isnan(vals)] = 0
    if name in ("wide_range_17", "ulp_apart_16"):
        assert not state["exact"], "rows with tying rounded distances must take the exact search"
        return
    assert state["exact"]
    t = np.array([np.float32(np.nan) if v is None else v for v in thr], dtype=np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        got = (t[None, :] <= vals[:, None]).sum(1) if len(t) else np.zeros_like(want)
    bad = np.nonzero(got != want)[0]
    assert len(bad) == 0, [hex(int(b)) for b in bad[:8]]


def test_wide_range_row_breaks_pairwise_thresholds():
    """The reason for the gap condition: in the wide-range row several
    entries round to the same distance from some values, and counting the
    pairwise decisions d_b < d_a then misses the first index of the tied
    minimum, so the thresholds alone would encode those values wrongly."""
    cb = _codebooks()["wide_range_17"]
    state = {"exact": True}
    t = np.array([np.float32(np.nan) if v is None else v
                  for v in (_threshold(cb, i, np.float32(0), state) for i in range(len(cb) - 1))],
                 dtype=np.float32)
    vals = (np.arange(0x10000, dtype=np.uint32) << 16).view(np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        want = np.abs(np.clip(vals, cb[0], cb[-1])[:, None] - cb[None, :]).argmin(1)
        got = (t[None, :] <= vals[:, None]).sum(1)
    want[np.isnan(vals)] = 0
    assert (got != want).any()
