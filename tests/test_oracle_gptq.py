"""Pins of the GPTQ oracle (src/vc/quantization/gptq.py:32-270): with an
identity factor the column loop is plain rounding, a two-column case by hand,
the compensation lowering the Hessian-weighted error of plain rounding, and
the factor checked against its definition in float64; plus the library's
host-side salience order against the oracle's (CPU tensors)."""

import numpy as np
import torch

from oracle import formats as F
from oracle import reference_ops as R


def int4_qmap():
    return R.table_tensor(F.int_table(4, True))


def test_identity_factor_is_plain_rounding():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(40, 64, generator=g)
    s = torch.rand(40, generator=g) + 0.1
    q = int4_qmap()
    out, deltas = R.gptq_block(w, s, torch.eye(64), q, 0, 64)
    plain = R.vmap((w / s[:, None]).bfloat16(), q).float() * s[:, None]
    assert torch.equal(out, plain)
    assert torch.equal(deltas, w - plain)


def test_two_columns_by_hand():
    q = int4_qmap()
    w = torch.tensor([[0.30, 0.45]])
    s = torch.tensor([0.1])
    h = torch.tensor([[2.0, 0.5], [0.0, 4.0]])
    out, deltas = R.gptq_block(w, s, h, q, 0, 2)
    f32 = np.float32
    q0 = f32(round(float(f32(0.30) / f32(0.1)))) * f32(0.1)       # 3 * 0.1 (int4 grid, RNE)
    d0 = (f32(0.30) - f32(q0)) / f32(2.0)
    w1 = f32(0.45) - f32(d0 * f32(0.5))
    assert out[0, 0].item() == float(f32(q0)) and deltas[0, 0].item() == float(f32(d0))
    q1 = f32(np.round(float(f32(w1 / f32(0.1))))) * f32(0.1)
    assert out[0, 1].item() == float(f32(q1))
    assert deltas[0, 1].item() == float(f32((w1 - f32(q1)) / f32(4.0)))


def test_compensation_beats_plain_rounding():
    g = torch.Generator().manual_seed(1)
    X = torch.randn(2048, 128, generator=g) @ (torch.randn(128, 128, generator=g) * 0.3 + torch.eye(128))
    H = X.T @ X
    w = torch.randn(64, 128, generator=g) * 0.05
    q = int4_qmap()
    out = R.gptq_compensate_weight(w, H.clone(), 2048, q, 7.0, 64, damping=0.01)
    s = R.calculate_mx_qparam(w, [-1], 64, 7.0).repeat_interleave(64, dim=1)
    plain = R.vmap((w / s).bfloat16(), q).float() * s

    def err(o):
        e = w - o
        return torch.einsum("ij,jk,ik->", e, H / 2048, e).item()

    assert err(out) < 0.9 * err(plain)


def _hessian(seed, n):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(4 * n, n, generator=g) * (torch.rand(n, generator=g) * 2 + 0.1)
    return X.T @ X, 4 * n


def test_factor_is_the_cholesky_of_the_damped_inverse():
    # U^T U = inv(H / tokens + damping * mean(diag)), U upper with a positive
    # diagonal (the definition the compensation relies on), checked in float64
    H, tokens = _hessian(2, 96)
    U = R._hessian_inverse_chol(H.clone(), tokens, 0.01).double()
    Hd = H.double() / tokens
    Hd.diagonal().add_(0.01 * Hd.diagonal().mean())
    assert torch.equal(U, torch.triu(U)) and bool((U.diagonal() > 0).all())
    assert torch.allclose(U.T @ U @ Hd, torch.eye(96, dtype=torch.float64), atol=1e-4)


def test_salience_order_matches_the_oracle_permutation(vqx):
    H, _ = _hessian(4, 256)
    for within in (True, False):
        perm = vqx.quantization.gptq.salience_order(H, 256, within, 64)
        blocks = 4
        diagonal = H.diagonal().reshape(blocks, 64)
        order = torch.argsort(diagonal.mean(dim=1), descending=True)
        # whole blocks, most salient first; inside a block by salience or in place
        assert sorted(perm.tolist()) == list(range(256))
        for b in range(blocks):
            chunk = perm[b * 64:(b + 1) * 64]
            assert set((chunk // 64).tolist()) == {int(order[b])}
            d = H.diagonal()[chunk]
            if within:
                assert bool((d[:-1] >= d[1:]).all())
            else:
                assert torch.equal(chunk, torch.arange(64) + 64 * int(order[b]))
