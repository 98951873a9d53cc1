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
    leave the later decision thresholds empty) and at the bottom."""
    cb = torch.sort(torch.randn(rows, K, generator=g), dim=1).values
    if K >= 3:
        for r in range(0, rows, 7):
            n = 1 + r % (K - 1)
            cb[r, K - n:] = cb[r, K - n]        # top run
        for r in range(3, rows, 11):
            n = 1 + r % (K - 1)
            cb[r, :n] = cb[r, n - 1]            # bottom run
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
