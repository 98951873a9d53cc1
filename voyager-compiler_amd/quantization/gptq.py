"""GPTQ weight compensation against the deployed microscaling grid, on the
MI355X (src/voyager_compiler/quantization/gptq.py:32-270).

The per-block column loop -- quantize a column, charge its rounding error to
the block's later columns through the inverse-Hessian factor -- is one HIP
kernel launch per block (``vqx_gptq_block``, each output row on a quad of
lanes with the row's block in registers) instead of a few small torch
launches per column.  The inverse-Hessian factor is a blockwise
factor-and-invert of the reversed Hessian whose 64-row diagonal blocks run in
a HIP kernel (``vqx_chol_inverse_block``).  The block scale uses the
library's ``calculate_mx_qparam`` and ``vmap``; the permutation and the GEMMs
(the factor's off-diagonal blocks, the update of the later columns) are
torch calls.
"""

import logging

import torch

from .. import _lib
from ..ops import quantized as Q

logger = logging.getLogger(__name__)

#: Floor of scales and of the factor's diagonal (lcq.py:35).
EPS = 1e-12

#: Columns whose deltas are subtracted from the later columns in one GEMM.
OUTER_COLUMNS = 512

#: Columns the HIP column loop walks per launch (its registers hold them).
LOOP_COLUMNS = 64

#: Rows of the diagonal blocks the HIP kernel factors and inverts.
FACTOR_LEAF = 64

#: Scale factors tried below ``amax / quant_max`` (gptq.py:75).
SHRINK_GRID = (1.0, 0.93, 0.86, 0.79, 0.72)


def _inverse_factor(a, li, info):
    """li <- inverse of the lower Cholesky factor of the symmetric positive
    definite ``a`` (its lower triangle; ``a`` is overwritten), blockwise:
    with a = [[A11, .], [A21, A22]] and L11^-1 from the first half,
    L21 = A21 L11^-T, the second half factors S = A22 - L21 L21^T, and the
    inverse's lower-left block is -L22^-1 L21 L11^-1.  The diagonal blocks
    of at most FACTOR_LEAF rows run in the HIP kernel, everything else is
    library GEMMs.  ``info`` (int32, device) becomes 1 on a non-positive
    pivot."""
    n = a.shape[0]
    if n == 0:
        return
    if n <= FACTOR_LEAF:
        _lib.call("vqx_chol_inverse_block", _lib.ptr(a), a.stride(0), n, _lib.ptr(li), li.stride(0),
                  _lib.ptr(info), _lib.stream_of(a))
        return
    h = (n // 2 + FACTOR_LEAF - 1) // FACTOR_LEAF * FACTOR_LEAF
    _inverse_factor(a[:h, :h], li[:h, :h], info)
    l21 = a[h:, :h] @ li[:h, :h].T
    a[h:, h:].addmm_(l21, l21.T, alpha=-1.0)
    _inverse_factor(a[h:, h:], li[h:, h:], info)
    li[h:, :h].addmm_(li[h:, h:], l21 @ li[:h, :h], beta=0.0, alpha=-1.0)


def hessian_inverse_chol(hessian, tokens, damping):
    """Upper Cholesky factor U of inv(H / tokens + damping) (U^T U = inv(H)),
    the damping raised tenfold up to 10^4x while H stays indefinite
    (gptq.py:32-71).

    The reference factors H, forms inv(H) and factors that.  Here the same
    (unique) factor comes from one blockwise factorisation that also inverts:
    with J the order reversal and J H J = L L^T, H = (J L J)(J L J)^T where
    J L J is upper triangular, so U = (J L J)^-1 = J L^-1 J.  inv(H) is never
    formed in fp32.
    """
    _lib.require_device(hessian, "hessian_inverse_chol")
    hessian = hessian.float() / max(tokens, 1)
    damp = damping * hessian.diagonal().mean().clamp_min(EPS)
    applied = 0
    for escalation in (1, 10, 100, 1000, 10000):
        hessian.diagonal().add_((escalation - applied) * damp)
        applied = escalation
        work = hessian.flip(0, 1).contiguous()
        li = torch.zeros_like(work)
        info = torch.zeros(1, dtype=torch.int32, device=work.device)
        _inverse_factor(work, li, info)
        if int(info.item()) == 0 and bool(torch.isfinite(li).all()):
            if escalation > 1:
                logger.warning("Hessian needed %dx the requested damping to invert", escalation)
            return li.flip(0, 1)
    raise torch.linalg.LinAlgError("Hessian not positive-definite")


def block_scale(block, weights, fake_quant, shrink):
    """Each row's scale for one block: amax / quant_max through the scale
    codebook, or the best of the shrink grid by salience-weighted error
    (gptq.py:84-137)."""
    qmap, scale_qmap = fake_quant.qmap, fake_quant.scale_qmap
    base = Q.calculate_mx_qparam(block, [-1], block.shape[-1], fake_quant.quant_max, False,
                                 scale_qmap).reshape(-1).clamp_min(EPS)
    if not shrink:
        return base
    chosen, lowest = base, None
    for factor in SHRINK_GRID:
        scale = base if factor == 1.0 else Q.vmap((base * factor).bfloat16(), scale_qmap).float().clamp_min(EPS)
        quantized = Q.vmap((block / scale[:, None]).bfloat16(), qmap).float() * scale[:, None]
        error = ((block - quantized).pow(2) * weights).sum(dim=1)
        if lowest is None:
            chosen, lowest = scale, error
            continue
        better = error < lowest
        chosen = torch.where(better, scale, chosen)
        lowest = torch.where(better, error, lowest)
    return chosen


def salience_order(hessian, columns, within_block, block_size):
    """Column permutation putting the most salient blocks first, whole blocks
    kept together (gptq.py:140-181); None when columns is not a whole number
    of blocks."""
    if columns % block_size:
        return None
    blocks = columns // block_size
    diagonal = hessian.diagonal().reshape(blocks, block_size)
    block_order = torch.argsort(diagonal.mean(dim=1), descending=True)
    if within_block:
        rank = torch.argsort(diagonal, dim=1, descending=True)
    else:
        rank = torch.arange(block_size, device=hessian.device).expand(blocks, block_size)
    base = torch.arange(blocks, device=hessian.device).unsqueeze(1)
    return (base * block_size + rank)[block_order].reshape(-1)


def compensate_weight(weight, hessian, tokens, fake_quant, damping, act_order=True, within_block=True,
                      shrink=False):
    """The GPTQ-compensated reconstruction of ``weight`` ([out, in]) on the
    grid of ``fake_quant`` (its qmap, scale_qmap, quant_max, block_size and
    ch_axis), in the original column order (gptq.py:184-270)."""
    _lib.require_device(weight, "compensate_weight")
    ensure = getattr(fake_quant, "_ensure_tables", None)
    if ensure is not None:  # this library's FakeQuantize builds its tables on first use
        ensure(weight.device)
    block_size = fake_quant.block_size
    axis = fake_quant.ch_axis
    axis = axis[0] if isinstance(axis, (tuple, list)) else axis
    if axis not in (-1, weight.dim() - 1):
        raise ValueError(f"weight blocks run along axis {axis}, but the compensation walks the input channels of a "
                         f"{tuple(weight.shape)} weight")
    perm = salience_order(hessian, weight.shape[1], within_block, block_size) if act_order else None
    if act_order and perm is None:
        logger.warning("%d input channels is not a whole number of %d-channel blocks, so the salience ordering "
                       "would split one and is skipped", weight.shape[1], block_size)
    if perm is not None:
        hessian = hessian[perm][:, perm]
        weight = weight[:, perm]
    salience = hessian.diagonal().clone()
    hinv = hessian_inverse_chol(hessian, tokens, damping)
    out = compensate_with_factor(weight, hinv, salience, fake_quant, shrink)
    if perm is None:
        return out
    restored = torch.empty_like(out)
    restored[:, perm] = out
    return restored


def compensate_with_factor(weight, hinv, salience, fake_quant, shrink=False):
    """The block loop of compensate_weight (gptq.py:239-265) on columns
    already in processing order, given the upper Cholesky factor of the
    inverse Hessian: each block's scale from the current weights, the
    block's column loop on the GPU, then the later columns updated by the
    block's deltas (library GEMMs).

    The reference subtracts each block's deltas from every later column at
    once.  Here the columns up to the end of the current span of
    ``OUTER_COLUMNS`` are brought up to date after each block, and the
    span's deltas are subtracted from the columns after it in one GEMM with
    a contraction of ``OUTER_COLUMNS`` (K = 64 GEMMs run at a fifth of the
    rate).  Every block still starts from fully updated columns; only the
    grouping of the fp32 sums differs.  Blocks wider than ``LOOP_COLUMNS``
    keep one scale per block and run their column loop in pieces."""
    _lib.require_device(weight, "compensate_with_factor")
    block_size = fake_quant.block_size
    hinv = hinv.to(device=weight.device, dtype=torch.float32).contiguous()
    qmap = Q._table_bf16(fake_quant.qmap.to(weight.device))
    sq = fake_quant.scale_qmap
    sq = None if sq is None else Q._table_bf16(sq.to(weight.device))
    work = weight.float().contiguous().clone()
    out = torch.zeros_like(work)
    R, C = work.shape
    # the kernel forms the plain block scale itself from the block it loads
    in_kernel = not shrink and block_size <= LOOP_COLUMNS
    span = max(block_size, OUTER_COLUMNS // block_size * block_size)
    for outer in range(0, C, span):
        stop = min(outer + span, C)
        deltas = torch.empty(R, stop - outer, dtype=torch.float32, device=work.device)
        for start in range(outer, stop, block_size):
            end = min(start + block_size, stop)
            scale = None if in_kernel else \
                block_scale(work[:, start:end], salience[start:end], fake_quant, shrink).float().contiguous()
            # the kernel walks at most LOOP_COLUMNS columns; a wider block's
            # later pieces get the earlier pieces' deltas through the GEMM
            for lo in range(start, end, LOOP_COLUMNS):
                hi = min(lo + LOOP_COLUMNS, end)
                d = deltas[:, lo - outer:hi - outer]  # written in place, row stride stop - outer
                _lib.call("vqx_gptq_block", _lib.ptr(work), R, C, lo, hi - lo, _lib.ptr(scale),
                          float(fake_quant.quant_max), _lib.ptr(sq), _lib.ptr(hinv), hinv.shape[1], _lib.ptr(qmap),
                          _lib.ptr(out), _lib.ptr(d), deltas.stride(0), _lib.stream_of(work))
                if hi < stop:
                    work[:, hi:stop].addmm_(d, hinv[lo:hi, hi:stop], alpha=-1.0)
        if stop < C:
            work[:, stop:].addmm_(deltas, hinv[outer:stop, stop:], alpha=-1.0)
    return out
