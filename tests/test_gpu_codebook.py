"""GPU parity of per-channel codebook encode/decode (C4): nearest entry in
fp32 with lowest-index ties, against a brute-force argmin oracle."""

import numpy as np
import pytest
import torch

from oracle import reference_ops as R

Q = torch.ops.quantized_ops


def c4_codebooks(rows, K, seed=3):
    g = torch.Generator().manual_seed(seed)
    from scipy.stats import norm

    q = torch.tensor(norm.ppf((np.arange(K) + 0.5) / K), dtype=torch.float32)
    spacing = torch.diff(q, prepend=q[:1] - (q[1] - q[0]))
    jit = (torch.rand(rows, K, generator=g) - 0.5) * 0.5 * spacing
    return torch.sort(q + jit, dim=1).values


@pytest.mark.gpu
@pytest.mark.parametrize("K", [16, 256])
def test_c4_codebook_encode_decode(vqx, K):
    g = torch.Generator().manual_seed(3)
    rows, cols = 256, 4096
    x = torch.randn(rows, cols, generator=g)
    cb = c4_codebooks(rows, K)
    # ties: inputs exactly on codebook entries and on bf16 midpoints
    x[0, :K] = cb[0]
    mids = ((cb[1, :-1] + cb[1, 1:]) / 2).to(torch.bfloat16).float()
    x[1, :K - 1] = mids
    cb[2, 5] = cb[2, 4]  # duplicate entry
    x[3, 0] = float("nan")
    x[3, 1] = float("inf")
    x[3, 2] = -float("inf")
    codes = Q.codebook_encode(x.cuda(), cb.cuda())
    want = R.codebook_encode_rows(x, cb)
    assert torch.equal(codes.cpu().long(), want)
    dec = Q.codebook_decode(codes, cb.cuda(), torch.float32)
    assert torch.equal(dec.cpu(), R.codebook_decode_rows(want, cb))


@pytest.mark.gpu
def test_codebook_bf16_input(vqx):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(64, 512, generator=g).to(torch.bfloat16)
    cb = c4_codebooks(64, 16)
    codes = Q.codebook_encode(x.cuda(), cb.cuda())
    assert torch.equal(codes.cpu().long(), R.codebook_encode_rows(x.float(), cb))


def random_codebooks(rows, K, g):
    """Sorted rows with repeated entries, including runs at the top (which
    leave the later decision thresholds empty) and at the bottom; rows with
    entries one fp32 ulp apart, and rows spanning 40 binades, where rounded
    distances tie (encoded by the exact per-element search)."""
    cb = torch.sort(torch.randn(rows, K, generator=g), dim=1).values
    if K >= 3:
        for r in range(0, rows, 7):
            n = 1 + r % (K - 1)
            cb[r, K - n:] = cb[r, K - n]        # top run
        for r in range(3, rows, 11):
            n = 1 + r % (K - 1)
            cb[r, :n] = cb[r, n - 1]            # bottom run
    if K >= 2:
        for r in range(5, rows, 13):
            cb[r, 1] = torch.nextafter(cb[r, 0], torch.tensor(float("inf")))
            cb[r] = torch.sort(cb[r]).values
        for r in range(6, rows, 17):
            mag = torch.exp(torch.empty(K).uniform_(-20, 20, generator=g))
            cb[r] = torch.sort(torch.randn(K, generator=g) * mag).values
    return cb


@pytest.mark.gpu
@pytest.mark.parametrize("K", [1, 2, 3, 5, 17, 100, 129, 255, 256])
@pytest.mark.parametrize("rows,cols", [(3000, 16), (40, 1040), (9, 2064)])
def test_codebook_sizes_and_shapes(vqx, K, rows, cols):
    """Every search depth (codebook sizes 1 .. 256), rows beyond the resident
    grid, row lengths below, at and past the 1024-element chunk, fp32 and
    bf16 outputs."""
    g = torch.Generator().manual_seed(1000 * K + cols)
    cb = random_codebooks(rows, K, g)
    x = torch.randn(rows, cols, generator=g) * 1.5
    n = min(K, cols)
    x[0, :n] = cb[0, :n]
    codes = Q.codebook_encode(x.cuda(), cb.cuda())
    want = R.codebook_encode_rows(x, cb)
    assert torch.equal(codes.cpu().long(), want)
    for dt in (torch.float32, torch.bfloat16):
        dec = Q.codebook_decode(codes, cb.cuda(), dt)
        assert torch.equal(dec.cpu().float(), R.codebook_decode_rows(want, cb))


@pytest.mark.gpu
@pytest.mark.parametrize("K,rows,cols", [(16, 5, 4112), (100, 5, 4112), (256, 5, 4112), (256, 700, 3088),
                                         (16, 4500, 2064)])
def test_codebook_rows_shared_by_waves(vqx, K, rows, cols):
    """Rows split over 2 or 4 waves (each taking every 2nd or 4th chunk and
    building its own tree), the tail past the last whole chunk, and more
    split rows than resident waves (each wave then takes several rows)."""
    g = torch.Generator().manual_seed(77 + K + rows)
    cb = random_codebooks(rows, K, g)
    x = torch.randn(rows, cols, generator=g) * 1.5
    x[:, -3:] = cb[:, :3]
    codes = Q.codebook_encode(x.cuda(), cb.cuda())
    assert torch.equal(codes.cpu().long(), R.codebook_encode_rows(x, cb))


@pytest.mark.gpu
@pytest.mark.parametrize("K", [2, 16, 256])
def test_codebook_subnormals_and_signed_zeros(vqx, K):
    """Codebooks whose entries straddle zero at subnormal magnitudes, and
    inputs that round to bf16 subnormals, signed zeros, huge values and
    NaNs: the fp32 -> bf16 rounding of the input and the threshold
    comparisons must stay exact down to the smallest subnormal."""
    g = torch.Generator().manual_seed(77 + K)
    rows, cols = 24, 2048
    tiny = 2.0 ** -130
    base = torch.sort(torch.randn(rows, K, generator=g), dim=1).values
    cb = base * tiny                                  # all entries subnormal
    cb[rows // 2:] = base[rows // 2:]                 # ordinary rows for contrast
    cb[1] = torch.linspace(-3 * tiny, 3 * tiny, K)    # evenly spaced across zero
    x = torch.randn(rows, cols, generator=g) * tiny * 4
    x[:, :8] = torch.tensor([0.0, -0.0, tiny, -tiny, 2.0 ** -149, -(2.0 ** -149), 3e38, -3e38])
    x[:, 8] = float("nan")
    # fp32 values just around bf16 rounding boundaries among subnormals
    m = torch.randint(0, 1 << 23, (rows, 64), generator=g, dtype=torch.int64)
    x[:, 64:128] = (m | 0x8000).to(torch.int32).view(torch.float32)
    x[:, 128:192] = -((m & ~0xFFFF) | 0x8000).to(torch.int32).view(torch.float32)
    codes = Q.codebook_encode(x.cuda(), cb.cuda())
    want = R.codebook_encode_rows(x, cb)
    assert torch.equal(codes.cpu().long(), want)


@pytest.mark.gpu
def test_codebook_tied_distances_row_all_patterns(vqx):
    """A row whose entries span 40 binades: values near 258 are equally far
    (in fp32) from several entries, so the decision-threshold count would be
    wrong there; the kernel must notice and encode the row exactly.  Every
    bf16 pattern is encoded, next to an ordinary row."""
    wide = torch.tensor([-4.5617120e+08, -1.7806498e+04, -4.6088116e+02, -4.8019073e+01, -4.9426060e-02,
                         -6.8074833e-03, -2.1707090e-03, -9.7630935e-04, -5.2784779e-04, -8.3647523e-05,
                         -2.4869628e-06, -1.9292422e-07, -5.5566971e-08, 4.8861853e-06, 1.9638399e-05,
                         4.0374794e-05, 7.8944244e+02], dtype=torch.float32)
    cb = torch.stack([wide, torch.linspace(-2, 2, 17)])
    pats = (torch.arange(0x10000, dtype=torch.int32) << 16).view(torch.float32)
    x = torch.stack([pats, pats])
    codes = Q.codebook_encode(x.cuda(), cb.cuda())
    assert torch.equal(codes.cpu().long(), R.codebook_encode_rows(x, cb))


def deep_codebooks():
    """Codebooks of the deep search trees (K = 32 .. 256): quantile rows of
    every deep size, evenly spaced rows whose decision thresholds sit on
    integers (range 1024), the same all <= 0, a row within one binade,
    a row with three thresholds within 0.0004 of its range, and a row with
    a duplicate entry (two equal thresholds)."""
    rows = []
    for K in (32, 64, 128, 256):
        rows.append(c4_codebooks(2, K, seed=K)[:, :].tolist())
    flat = [r for pair in rows for r in pair]
    out = [torch.tensor(r) for r in flat]
    edges = torch.arange(256, dtype=torch.float32) * 4.0
    edges[-1] = 1024.0                                                  # thresholds 2, 6, ..., 1018, 1020
    out.append(edges)
    out.append(edges - 1024.0)                                          # the same, all <= 0
    out.append(torch.linspace(-3.0, 3.0, 200))
    out.append(torch.linspace(0.5, 0.75, 100))
    crowded = c4_codebooks(1, 256, seed=9)[0].clone()
    w = float(crowded[-1] - crowded[0]) / 1024
    for i in (1, 2, 3):                                                  # crowded thresholds
        crowded[99 + i] = crowded[99] + 0.2 * i * w
    out.append(torch.sort(crowded).values)
    dup = c4_codebooks(1, 128, seed=10)[0].clone()
    dup[40] = dup[39]
    out.append(dup)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_codebook_deep_trees_all_patterns(vqx, dtype):
    """Every bf16 bit pattern (NaNs, infinities, subnormals, signed zeros)
    encoded against the deep-tree codebooks, equal to the brute-force argmin;
    one call per codebook size."""
    pats = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    cbs = deep_codebooks()
    for K in sorted({len(c) for c in cbs}):
        cb = torch.stack([c for c in cbs if len(c) == K])
        x = pats.float().expand(cb.shape[0], -1).contiguous()
        print(f"deep tree K={K} rows={cb.shape[0]} {dtype}", flush=True)
        codes = Q.codebook_encode(x.to(dtype).cuda(), cb.cuda())
        want = R.codebook_encode_rows(x, cb)
        assert torch.equal(codes.cpu().long(), want), K
