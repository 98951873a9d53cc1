"""GPU: linear_mx / matmul_mx on convert-format operands outside the packed
NF4 weight's format, which run vqx_mx_matmul (both operands decoded inside
the kernel): the attention products of the reference's LLaMA configs with
int6 / nf4_6 operands coded on both sides, blocks of 64 along the
contraction dim (src/voyager_compiler/ops/quantized.py:371-406;
test/test_codegen.py:126-152), MXINT8 linears with blocks of 16
(test/run_ci.py:66-70), coded activations with weights of more than 16
levels, ragged shapes, broadcast batches, both storage layouts of the right
operand, and indices outside the code table.  Results are compared with the
oracle's linear_mx / matmul_mx (the reference's decode, then torch's bf16
product) within relative tolerance 1e-2, as north_star states for GEMM
outputs; the library GEMM is made to fail inside the calls, so a pass
proves the HIP kernel ran."""

import pytest
import torch

from oracle import formats as F
from oracle import reference_ops as R
from tests.conftest import assert_bitexact
from tests.test_gpu_linear_mx_fused import fused_only, within_tolerance

Q = torch.ops.quantized_ops


def gen(seed):
    return torch.Generator().manual_seed(seed)


def int_operand(shape, lo, hi, seed):
    """Integer-valued bf16 operand in [lo, hi) (int6: -32..31, int8)."""
    return torch.randint(lo, hi, shape, generator=gen(seed)).to(torch.bfloat16)


def e5m3_scales(shape, seed):
    """bf16 scales on the fp8_e5m3 grid: 2^e (1 + m / 8)."""
    g = gen(seed)
    e = torch.randint(-10, 1, shape, generator=g).float()
    m = torch.randint(0, 8, shape, generator=g).float()
    return (torch.exp2(e) * (1 + m / 8)).to(torch.bfloat16)


def pow2_scales(shape, seed):
    return torch.exp2(torch.randint(-12, -4, shape, generator=gen(seed)).float()).to(torch.bfloat16)


def blocks(n, bs):
    return -(-n // bs)


def nf4_6_code():
    """The code convert_pt2e builds for an nf4_6 quantizer: the table's
    distinct values (quantize_pt2e.py:457-466)."""
    return torch.unique(R.table_tensor(F.quantization_table("nf4_6"))).to(torch.bfloat16)


def cuda(*ts):
    return [None if t is None else t.cuda() for t in ts]


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,S,D", [(1, 32, 2048, 128), (2, 3, 200, 64)])
def test_attention_int6_both_sides(vqx, B, H, S, D):
    """Q K^T and P V of the LLaMA attention with the reference's int6 specs:
    the left operand blocked along -1, the right along -2 (the contraction
    dim of both products), bf16 scales on the fp8_e5m3 grid."""
    print(f"attention int6 B={B} H={H} S={S} D={D}", flush=True)
    bs = 64
    q = int_operand((B, H, S, D), -32, 32, 1)
    qs = e5m3_scales((B, H, S, blocks(D, bs)), 2)
    kt = int_operand((B, H, D, S), -32, 32, 3)           # K^T, quantized along -2
    ks = e5m3_scales((B, H, blocks(D, bs), S), 4)
    with fused_only():
        scores = Q.matmul_mx(*cuda(q, kt), input_scale=qs.cuda(), weight_scale=ks.cuda(), block_size=bs)
    within_tolerance(scores, R.matmul_mx(q, kt, ks, bs, None, qs, None))
    p = int_operand((B, H, S, S), -32, 32, 5)
    ps = e5m3_scales((B, H, S, blocks(S, bs)), 6)
    v = int_operand((B, H, S, D), -32, 32, 7)
    vs = e5m3_scales((B, H, blocks(S, bs), D), 8)
    with fused_only():
        out = Q.matmul_mx(*cuda(p, v), input_scale=ps.cuda(), weight_scale=vs.cuda(), block_size=bs)
    within_tolerance(out, R.matmul_mx(p, v, vs, bs, None, ps, None))


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,S,D", [(1, 32, 2048, 128), (1, 2, 136, 128)])
def test_attention_nf4_6_codes_both_sides(vqx, B, H, S, D):
    """The MXNF4 config's attention products: nf4_6 indices on both sides
    with the 16-entry code, blocks of 64 along the contraction dim."""
    print(f"attention nf4_6 B={B} H={H} S={S} D={D}", flush=True)
    bs, code = 64, nf4_6_code()
    q = int_operand((B, H, S, D), 0, 16, 11)
    qs = e5m3_scales((B, H, S, blocks(D, bs)), 12)
    kt = int_operand((B, H, D, S), 0, 16, 13)
    ks = e5m3_scales((B, H, blocks(D, bs), S), 14)
    with fused_only():
        got = Q.matmul_mx(*cuda(q, kt), input_scale=qs.cuda(), weight_scale=ks.cuda(), block_size=bs,
                          input_code=code.cuda(), weight_code=code.cuda())
    within_tolerance(got, R.matmul_mx(q, kt, ks, bs, code, qs, code))


@pytest.mark.gpu
def test_attention_from_quantize_mx(vqx):
    """Operands as the converted model makes them at run time: quantize_mx of
    bf16 activations with the int6 spec (values and fp8_e5m3 scales), the
    right operand quantized along -2, then matmul_mx on the results."""
    print("attention from quantize_mx", flush=True)
    g = gen(21)
    qmap = R.table_tensor(F.quantization_table("int6"))
    smap = R.table_tensor(F.quantization_table("fp8_e5m3"))
    a = torch.randn(2, 4, 96, 128, generator=g).to(torch.bfloat16)
    b = torch.randn(2, 4, 128, 80, generator=g).to(torch.bfloat16)
    qmax = 31.0                         # int6 quant_max
    sa, qa = Q.quantize_mx(a.cuda(), qmap.cuda(), [-1], 64, qmax, False, smap.cuda())
    sb, qb = Q.quantize_mx(b.cuda(), qmap.cuda(), [-2], 64, qmax, False, smap.cuda())
    with fused_only():
        got = Q.matmul_mx(qa, qb, input_scale=sa, weight_scale=sb, block_size=64)
    want = R.matmul_mx(qa.cpu(), qb.cpu(), sb.cpu(), 64, None, sa.cpu(), None)
    within_tolerance(got, want)
    # and the quantization itself is the reference's
    rs, rq = R.quantize_mx(a, qmap, [-1], 64, qmax, False, smap)
    assert torch.equal(qa.cpu(), rq) and torch.equal(sa.cpu(), rs)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(2048, 11008, 4096), (77, 300, 200), (5, 64, 16)])
def test_mxint8_linear(vqx, M, N, K):
    """The MXINT8 CI scheme's linears: int8 activations and weights, blocks
    of 16 along K, power-of-two scales, a bias; ragged M, N and a K that is
    not a multiple of 64."""
    print(f"mxint8 linear M={M} N={N} K={K}", flush=True)
    bs = 16
    x = int_operand((M, K), -127, 128, 31)
    xs = pow2_scales((M, blocks(K, bs)), 32)
    w = int_operand((N, K), -127, 128, 33)
    ws = pow2_scales((N, blocks(K, bs)), 34)
    bias = torch.randn(N, generator=gen(35)).to(torch.bfloat16)
    with fused_only():
        got = Q.linear_mx(*cuda(x, w, bias), input_scale=xs.cuda(), weight_scale=ws.cuda(), block_size=bs)
    within_tolerance(got, R.linear_mx(x, w, bias, ws, bs, None, xs, None))


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["kc", "ck"])
def test_linear_coded_activation_wide_code_weight(vqx, layout):
    """input_code / input_scale on the activation (nf4_6 indices) with a
    weight of a 40-entry code table and blocks of 32 along K: both decoded in
    the kernel, batched activations, either weight layout."""
    print(f"linear coded activation layout={layout}", flush=True)
    N, K, bs = 384, 512, 32
    code_w = torch.linspace(-3, 3, 40).to(torch.bfloat16)
    x = int_operand((2, 50, K), 0, 16, 41)
    xs = e5m3_scales((2, 50, blocks(K, bs)), 42)
    w = int_operand((N, K), 0, 40, 43)
    ws = e5m3_scales((N, blocks(K, bs)), 44)
    if layout == "ck":
        w, ws = w.t().contiguous(), ws.t().contiguous()
    with fused_only():
        got = Q.linear_mx(*cuda(x, w), None, input_scale=xs.cuda(), weight_scale=ws.cuda(), block_size=bs,
                          input_code=nf4_6_code().cuda(), weight_code=code_w.cuda(), weight_layout=layout)
    assert got.shape == (2, 50, N)
    within_tolerance(got, R.linear_mx(x, w, None, ws, bs, code_w, xs, nf4_6_code(), weight_layout=layout))


@pytest.mark.gpu
def test_linear_coded_activation_nf4_weight_runs_packed_path(vqx):
    """A coded activation with a 16-level weight with blocks of 64: the
    activation is decoded by the vqx decode kernel and the product runs the
    packed-weight kernel; the result still matches."""
    N, K, M, bs = 256, 512, 40, 64
    code = nf4_6_code()
    x = int_operand((M, K), 0, 16, 51)
    xs = e5m3_scales((M, blocks(K, bs)), 52)
    w = int_operand((N, K), 0, 16, 53)
    ws = e5m3_scales((N, blocks(K, bs)), 54)
    with fused_only():
        got = Q.linear_mx(*cuda(x, w), None, input_scale=xs.cuda(), weight_scale=ws.cuda(), block_size=bs,
                          input_code=code.cuda(), weight_code=code.cuda())
    within_tolerance(got, R.linear_mx(x, w, None, ws, bs, code, xs, code))


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["b_2d", "a_2d", "kc", "kt_view", "kc_view", "codes_only", "scale_only_b"])
def test_matmul_mx_layouts_and_broadcast(vqx, case):
    """Right operands stored [K, N] or [N, K] (and transposed views of
    either), one side without batch dims, code without scale and scale
    without code."""
    print(f"matmul_mx case={case}", flush=True)
    bs, code = 32, nf4_6_code()
    M, K, N = 70, 192, 136
    a = int_operand((3, M, K), -32, 32, 61)
    a_s = e5m3_scales((3, M, blocks(K, bs)), 62)
    a_code = None
    layout = "ck"
    if case == "b_2d":
        b = int_operand((K, N), -32, 32, 63)
        b_s = e5m3_scales((blocks(K, bs), N), 64)
    elif case == "a_2d":
        a, a_s = a[0], a_s[0]
        b = int_operand((3, K, N), -32, 32, 65)
        b_s = e5m3_scales((3, blocks(K, bs), N), 66)
    elif case == "kc":
        layout = "kc"
        b = int_operand((3, N, K), -32, 32, 67)
        b_s = e5m3_scales((3, N, blocks(K, bs)), 68)
    elif case == "kt_view":
        # [K, N] right operand that is the transpose of a [N, K] tensor
        b = int_operand((3, N, K), -32, 32, 69).transpose(-2, -1)
        b_s = e5m3_scales((3, N, blocks(K, bs)), 70).transpose(-2, -1)
    elif case == "kc_view":
        layout = "kc"
        b = int_operand((3, K, N), -32, 32, 71).transpose(-2, -1)
        b_s = e5m3_scales((3, blocks(K, bs), N), 72).transpose(-2, -1)
    elif case == "codes_only":
        a, a_s, a_code = int_operand((3, M, K), 0, 16, 73), None, code
        b = int_operand((3, K, N), 0, 16, 74)
        b_s = None
    else:
        a_s = None
        b = int_operand((3, K, N), -32, 32, 75)
        b_s = e5m3_scales((3, blocks(K, bs), N), 76)
    b_code = code if case == "codes_only" else None
    with fused_only():
        got = Q.matmul_mx(*cuda(a, b), input_scale=None if a_s is None else a_s.cuda(),
                          weight_scale=None if b_s is None else b_s.cuda(), block_size=bs,
                          input_code=None if a_code is None else a_code.cuda(),
                          weight_code=None if b_code is None else b_code.cuda(), weight_layout=layout)
    want = R.matmul_mx(a, b, b_s, bs, b_code, a_s, a_code, weight_layout=layout)
    assert got.shape == want.shape, (got.shape, want.shape)
    within_tolerance(got, want)


@pytest.mark.gpu
def test_code_indices_truncate_wrap_and_out_of_range(vqx):
    """Indices as the reference reads them: fractions truncated toward zero,
    negative ones counting from the end of the table, |x| < 1 as index 0;
    an index past the table decodes to NaN (the reference raises), so only
    the outputs that read it are NaN."""
    bs, L = 16, 20
    code = torch.linspace(-2, 2, L).to(torch.bfloat16)
    M, K, N = 40, 64, 48
    g = gen(81)
    raw = torch.randint(-L, L, (M, K), generator=g).float()
    raw = raw + torch.where(raw >= 0, 0.5, -0.5) * (torch.rand(M, K, generator=g) < 0.3)
    raw[0, :4] = torch.tensor([0.75, -0.75, -0.0, 19.9])
    a = raw.to(torch.bfloat16)
    a_s = e5m3_scales((M, blocks(K, bs)), 82)
    b = int_operand((K, N), -32, 32, 83)
    b_s = e5m3_scales((blocks(K, bs), N), 84)
    with fused_only():
        got = Q.matmul_mx(*cuda(a, b), input_scale=a_s.cuda(), weight_scale=b_s.cuda(), block_size=bs,
                          input_code=code.cuda())
    within_tolerance(got, R.matmul_mx(a, b, b_s, bs, None, a_s, code))
    bad = a.clone()
    bad[7, 9] = 20.0          # past the 20-entry table
    bad[11, 3] = -21.0
    with fused_only():
        got = Q.matmul_mx(*cuda(bad, b), input_scale=a_s.cuda(), weight_scale=b_s.cuda(), block_size=bs,
                          input_code=code.cuda()).float().cpu()
    assert bool(torch.isnan(got[7]).all()) and bool(torch.isnan(got[11]).all())
    keep = torch.ones(M, dtype=torch.bool)
    keep[[7, 11]] = False
    within_tolerance(got[keep], R.matmul_mx(a, b, b_s, bs, None, a_s, code)[keep])


@pytest.mark.gpu
def test_mx_matmul_c_abi_rejects_bad_shapes(vqx):
    """The entry point's own checks: K % 8, an N-major right operand with
    N % 8, a block size that is not a power of two."""
    L = vqx._lib
    a = torch.zeros(16, 24, dtype=torch.bfloat16, device="cuda")
    b = torch.zeros(24, 12, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(16, 12, dtype=torch.bfloat16, device="cuda")

    def op(t, k_major, ld, scale=None, bs=0, sld=0):
        o = L.VqxMxOperand()
        o.data, o.k_major, o.ld = t.data_ptr(), k_major, ld
        o.scale = None if scale is None else scale.data_ptr()
        o.block_size, o.scale_ld = bs, sld
        return o

    def run(oa, ob, M, N, K):
        L.call("vqx_mx_matmul", L.ctypes.byref(oa), L.ctypes.byref(ob), None, out.data_ptr(), 1, M, N, K,
               L.stream_of(a))

    with pytest.raises(ValueError, match="N-major"):
        run(op(a, 1, 24), op(b, 0, 12), 16, 12, 24)
    with pytest.raises(ValueError, match="multiple of 8"):
        run(op(a, 1, 24), op(b.t().contiguous(), 1, 24), 16, 12, 20)
    s = torch.ones(16, 3, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="block_size"):
        run(op(a, 1, 24, s, 12, 3), op(b.t().contiguous(), 1, 24), 16, 12, 24)
    run(op(a, 1, 24), op(b.t().contiguous(), 1, 24), 16, 12, 24)
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["kmajor_code_scale", "nmajor_scale", "kt_view_code", "kc_view_scale_bs16",
                                  "code_only", "scale_only_wide"])
def test_mx_decode_is_the_reference_decode_bit_for_bit(vqx, case):
    """vqx_mx_operand_decode (the decode the host runs ahead of the product for an
    operand that many tiles read) against the oracle's decode of
    linear_mx / matmul_mx, bit for bit: code lookup by truncated index
    (negative from the end, out of range NaN), then bf16(value * scale)."""
    from importlib import import_module

    qops = import_module(vqx.__name__ + ".ops.quantized")
    code = torch.linspace(-2, 2, 20).to(torch.bfloat16)
    g = gen(91)
    bs, kdim, use_code, use_scale = 32, -1, True, True
    if case == "kmajor_code_scale":
        shape = (3, 40, 96)
    elif case == "nmajor_scale":
        shape, kdim, use_code = (2, 96, 48), -2, False
    elif case == "kt_view_code":
        shape, kdim = (2, 48, 96), -2            # logical [*, K, N], stored as [*, N, K]
    elif case == "kc_view_scale_bs16":
        shape, bs, use_code = (2, 96, 40), 16, False   # logical [*, N, K], stored [*, K, N]
    elif case == "code_only":
        shape, use_scale = (5, 64), False
    else:
        shape, bs, use_code = (4, 4096), 64, False
    raw = torch.randint(-20, 20, shape, generator=g).float()
    raw = raw + 0.5 * (torch.rand(shape, generator=g) < 0.2)
    if use_code:
        raw.view(-1)[7] = 20.0                   # past the table: NaN
    t = raw.to(torch.bfloat16)
    sshape = list(shape)
    sshape[kdim] = -(-shape[kdim] // bs)
    scale = e5m3_scales(tuple(sshape), 92) if use_scale else None
    if case == "kt_view_code":
        t = t.transpose(-2, -1).contiguous().transpose(-2, -1)
        scale = scale.transpose(-2, -1).contiguous().transpose(-2, -1)
    if case == "kc_view_scale_bs16":
        t = t.transpose(-2, -1).contiguous().transpose(-2, -1)
        scale = scale.transpose(-2, -1).contiguous().transpose(-2, -1)
    if use_code:
        # the reference raises IndexError on the index past the table; the
        # decode gives NaN there and the reference's values elsewhere
        bad = t.float().trunc() >= 20
        want = R._decode_mx(torch.where(bad, torch.zeros_like(t), t), code, scale, bs)
        want = torch.where(bad, torch.full_like(want, float("nan")), want)
    else:
        want = R._decode_mx(t, None, scale, bs)
    got = qops._mx_decoded(t.cuda(), code.cuda() if use_code else None, None if scale is None else scale.cuda(), bs,
                           kdim)
    assert got.shape == want.shape and got.dtype == torch.bfloat16
    assert_bitexact(got, want, case)


@pytest.mark.gpu
def test_short_k_ragged_many_tiles(vqx):
    """K = 72 (a partial second k-step) with blocks of 8, ragged M and N over
    576 tiles, both operands decoded in the kernel (each read by at most 3
    tiles)."""
    print("short-K ragged", flush=True)
    bs = 8
    a = int_operand((64, 300, 72), -32, 32, 101)
    a_s = e5m3_scales((64, 300, 9), 102)
    b = int_operand((64, 72, 264), -32, 32, 103)
    b_s = e5m3_scales((64, 9, 264), 104)
    with fused_only():
        got = Q.matmul_mx(*cuda(a, b), input_scale=a_s.cuda(), weight_scale=b_s.cuda(), block_size=bs)
    within_tolerance(got, R.matmul_mx(a, b, b_s, bs, None, a_s, None))
