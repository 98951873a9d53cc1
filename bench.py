"""Benchmark of the Voyager quantization hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c2] [--no-cpu]

A step is one pass of a hot-path kernel over one batch of synthetic, seeded
input already resident in HBM.  The headline (``value``) is BASELINE.json
NF4 block-64 encode of a bf16 4096x11008 weight (C2), in
quantized elements per second over the whole timed region (K back-to-back
launches between two synchronisations); every other config is reported in
``configs``.  A bandwidth-bound config cycles its launches through several
copies of its buffers, more than twice the 256 MiB MALL together, so every
launch streams from HBM (the cold figure, which every fraction uses); the
warm figure (one buffer set, input left in the MALL by the launch before) is
reported beside it.  ``roofline.achieved`` divides the algorithmic bytes of a
launch by the kernel's average launch duration, from HIP events around the
launches on the launch stream (the kernels launch on torch's current stream,
so torch.cuda.Event sees them); ``roofline.traffic`` is the HBM bytes per launch
measured by rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/
hbm_traffic.json).  ``cpu_baseline`` times the CPU oracle (a restatement of
the reference's PyTorch CPU path) on this host's cores.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time
from types import SimpleNamespace

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default=None, help="comma list of config keys to run")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-iters", type=int, default=3)
    ap.add_argument("--no-warm", action="store_true",
                    help="skip the warm-MALL timing pass (one buffer set re-launched), so that a profiler's "
                         "average over every launch of a kernel is the cold figure the bench reports")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only measure what HBM sustains on this box for each traffic mix, with 1 GiB working sets "
                         "(beyond the 256 MiB MALL): torch's own copy, fill and read kernels, and the C3 e4m3 "
                         "kernel on a 1 GiB input")
    ap.add_argument("--build-probe", action="store_true",
                    help="only compile bench_hbm_probe.hip (the --hbm-ceiling probe) into bench_hbm_probe.so")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device-to-device copy of 512 MiB (5 times), the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# CPU oracle timings: each returns a callable that times the reference's
# torch-CPU op sequence (the oracle) on a bounded sample of the config and
# returns (seconds for the whole config, what the sample was)
# ---------------------------------------------------------------------------
CPU_WARMUP, CPU_RUNS = 2, 5


def _timed(f):
    """Median seconds of CPU_RUNS runs of f after CPU_WARMUP untimed ones."""
    for _ in range(CPU_WARMUP):
        f()
    ts = []
    for _ in range(CPU_RUNS):
        t0 = time.perf_counter()
        f()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_c1(torch, xc):
    def run():
        from oracle import formats as F
        from oracle import reference_ops as R
        q = R.table_tensor(F.posit_table(8, 1))
        return _timed(lambda: R.fake_quantize_per_tensor(xc, q, torch.ones(()))), \
            "full input: FakeQuantizeFunction.forward (vmap of x / 1 through the posit8_1 table)"
    return run


def cpu_c2_decode(torch, xc):
    def run():
        from oracle import formats as F
        from oracle import reference_ops as R
        xs = xc[:512]
        s, q = R.quantize_mx(xs, R.table_tensor(F.quantization_table("nf4")), [-1], 64, 1.0, False)
        return _timed(lambda: R.dequantize(q, s, None, [-1], 64)) * 8, \
            "rows 0-511 (1/8), scaled: dequantize (values x expand(scale))"
    return run


def cpu_c3(torch, xc, dtype, qmax, fake):
    def run():
        from oracle import formats as F
        from oracle import reference_ops as R
        xs = xc[:1024]
        q = R.table_tensor(F.quantization_table(dtype))
        f = R.mx_fake_quantize if fake else R.quantize_mx
        return _timed(lambda: f(xs, q, [-1], 32, qmax, True)) * 8, \
            f"rows 0-1023 (1/8), scaled: {'MXFakeQuantizeFunction.forward' if fake else 'quantize_mx'}"
    return run


def cpu_c4(torch, xc, cbc, decode):
    def run():
        from oracle import reference_ops as R
        xs, cs = xc[:128], cbc[:128]
        if decode:
            codes = R.codebook_encode_rows(xs, cs)
            return _timed(lambda: R.codebook_decode_rows(codes, cs)) * 32, "rows 0-127 (1/32), scaled: decode"
        return _timed(lambda: R.codebook_encode_rows(xs, cs)) * 32, \
            "rows 0-127 (1/32), scaled: per-row argmin over the codebook"
    return run


def cpu_c5(torch, Ac, N):
    def run():
        from oracle import formats as F
        from oracle import reference_ops as R
        M, K = Ac.shape
        g = torch.Generator().manual_seed(4)
        codes = torch.randint(0, 16, (N, K), generator=g).to(torch.bfloat16)   # weight codes as floats
        scale = (torch.rand(N, K // 64, generator=g) * 0.05).to(torch.bfloat16)
        nf = R.table_tensor(F.nf_levels(4))
        rows = min(M, 256)
        full = _timed(lambda: R.linear_mx(Ac[:rows], codes, None, scale, 64, nf))
        if rows == M:
            return full, "full M: linear_mx (weight_code[w] * expand(scale), then F.linear in bf16)"
        dec = _timed(lambda: nf[codes.to(torch.long)] * R.expand(scale, codes.shape, 64))
        return dec + (full - dec) * (M / rows), \
            f"rows 0-{rows - 1}: the weight decode timed once, the product scaled to M = {M}"
    return run


# ---------------------------------------------------------------------------
# configs: setup() -> (list of launch callables, info)
#
# An HBM-bound config builds several sets of its input and output buffers and
# the timed loop cycles through them, so that the sets together exceed twice
# the 256 MiB MALL (MI355X's last-level cache) and no launch finds its input
# still cached from the launch before: its time is the time to stream from
# HBM.  The first set is the one the parity tests check.
# ---------------------------------------------------------------------------
ROTATE_BYTES = 640 << 20
MIN_SETS = 3


def rotate(make, set_bytes):
    """[launch] and [buffers] of n buffer sets, make(i) -> (launch, buffers),
    n = the sets whose bytes reach ROTATE_BYTES, at least MIN_SETS."""
    n = max(MIN_SETS, -(-ROTATE_BYTES // max(int(set_bytes), 1)))
    made = [make(i) for i in range(n)]
    return [m[0] for m in made], [m[1] for m in made]


def cpu_f3(torch, xc):
    def run():
        from oracle import reference_ops as R
        rows = 512
        dt = _timed(lambda: R.group_wise_affine_fake_quant(xc[:rows], [-1], 64, 0.0, 3.0))
        return dt * xc.shape[0] / rows, \
            f"rows 0-{rows - 1} (1/{xc.shape[0] // rows}), scaled: GroupWiseAffineFakeQuantFunction.forward"
    return run


def setup_f3(vqx, torch, L):
    """Group-wise affine fake-quant (uint2, blocks of 64 along the last
    axis, as for a KV cache) of C2's bf16 input."""
    xc = c2_input(torch)
    rows, cols = xc.shape
    n = xc.numel()
    fn = L.load().vqx_gwa_fake_quant

    def make(i):
        x = xc.cuda()
        y = torch.empty_like(x)
        sc = torch.empty(rows, cols // 64, dtype=x.dtype, device="cuda")
        zp = torch.empty_like(sc)
        args = (L.ptr(x), L.BF16, rows, cols, 1, 64, 0.0, 3.0, None, L.ptr(sc), L.ptr(zp), L.ptr(y),
                L.stream_of(x))
        return (lambda: fn(*args)), (x, y, sc, zp)

    algo = 4 * n + 2 * 2 * (n // 64)
    launches, bufs = rotate(make, algo)
    return launches, dict(
        name="F3 group-wise affine fake-quant, uint2 (0..3), blocks of 64 along the last axis: bf16 [4096,11008] "
             "-> bf16 values + bf16 scale and zero point per block",
        elements=n, bytes=algo, bound="hbm", dtype="bf16", keep=bufs, cpu=cpu_f3(torch, xc))


def setup_c1(vqx, torch, L):
    torch.manual_seed(0)
    xc = torch.randn(4096, 4096, dtype=torch.float32)
    n = xc.numel()
    desc = vqx.parse_format("posit8_1").desc(torch.device("cuda"))
    fn = L.load().vqx_fake_quant

    def make(i):
        x = xc.cuda()
        y = torch.empty_like(x)
        codes = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
        args = (L.ptr(x), L.F32, n, L.ctypes.byref(desc), None, 1, 1, 1, L.ptr(y), L.ptr(codes), 1,
                L.stream_of(x))
        return (lambda: fn(*args)), (x, y, codes)

    launches, bufs = rotate(make, 9 * n)
    return launches, dict(
        name="C1 posit8_1 fake-quant + uint8 codes, fp32 4096x4096 N(0,1) seed 0",
        elements=n, bytes=9 * n, bound="hbm", dtype="f32->u8", cpu=cpu_c1(torch, xc),
        check=dict(x=xc, out=bufs[0][1], codes=bufs[0][2]), keep=(bufs, desc))


def c2_input(torch, rows=4096, cols=11008, seed=1):
    g = torch.Generator().manual_seed(seed)
    w = 0.02 * torch.randn(rows, cols, generator=g)
    n = round(0.001 * w.numel())
    idx = torch.randperm(w.numel(), generator=g)[:n]
    sign = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
    w.view(-1)[idx] = sign * 8 * 0.02
    return w.to(torch.bfloat16)


def setup_c2(vqx, torch, L, decode=False):
    xc = c2_input(torch)
    n = xc.numel()
    fmt = vqx.parse_format("nf4")
    desc = fmt.desc(torch.device("cuda"))
    dtab = fmt.tables(torch.device("cuda"))["decode"]
    enc = L.load().vqx_mx_quantize
    dec = L.load().vqx_mx_decode
    algo = n * 2 + n // 2 + n // 64 * 4

    def make(i):
        x = xc.cuda()
        codes = torch.empty(n // 2, dtype=torch.uint8, device="cuda")
        scale = torch.empty(4096, 11008 // 64, dtype=torch.float32, device="cuda")
        st = L.stream_of(x)
        eargs = (L.ptr(x), L.BF16, 4096, 11008, 1, 64, L.ctypes.byref(desc), 1, 0, L.ctypes.c_float(1.0), None,
                 None, L.ptr(scale), None, None, None, L.ptr(codes), 0, st)
        if not decode:
            return (lambda: enc(*eargs)), (x, codes, scale)
        enc(*eargs)
        del x
        out = torch.empty(4096, 11008, dtype=torch.bfloat16, device="cuda")
        dargs = (L.ptr(codes), 4, L.ptr(dtab), dtab.numel(), L.ptr(scale), 0, n, 64, L.ptr(out), L.BF16, st)
        return (lambda: dec(*dargs)), (None, codes, scale, out)

    launches, bufs = rotate(make, algo)
    if not decode:
        return launches, dict(
            name="C2 NF4 block-64 absmax encode, bf16 4096x11008 N(0,0.02)+0.1% outliers seed 1 "
                 "-> packed 4-bit codes + fp32 scales",
            elements=n, bytes=algo, bound="hbm", dtype="bf16->u4", cpu_input=xc,
            check=dict(x=xc, codes=bufs[0][1], scale=bufs[0][2]), keep=(bufs, desc))
    return launches, dict(
        name="C2 NF4 block-64 decode: packed codes + fp32 scales -> bf16 4096x11008",
        elements=n, bytes=algo, bound="hbm", dtype="u4->bf16", cpu=cpu_c2_decode(torch, xc),
        check=dict(x=xc, codes=bufs[0][1], scale=bufs[0][2], out=bufs[0][3]), keep=(bufs, dtab, desc))


def c3_input(torch, rows=8192, cols=8192, seed=2):
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(rows, cols, generator=g) - 0.5
    lap = -torch.sign(u) * torch.log1p(-2 * u.abs())
    mult = 10 ** (torch.rand(cols, generator=g) * 2 - 1)
    return (lap * mult).to(torch.bfloat16)


_C3_X = {}


def _c3_inputs(torch, nsets):
    """C3's bf16 input on the device, nsets copies (kept across the C3
    configs, which all read it)."""
    if "xc" not in _C3_X:
        _C3_X["xc"] = c3_input(torch)
        _C3_X["x"] = []
    while len(_C3_X["x"]) < nsets:
        _C3_X["x"].append(_C3_X["xc"].cuda())
    return _C3_X["x"]


def setup_c3(vqx, torch, L, dtype, qmax, fake=False):
    n = 8192 * 8192
    fmt = vqx.parse_format(dtype)
    desc = fmt.desc(torch.device("cuda"))
    shift = math.floor(math.log2(qmax))
    fn = L.load().vqx_mx_quantize
    cb = fmt.code_bits
    algo = n * 4 + n // 32 * 2 if fake else n * 2 + n * cb // 8 + n // 32
    xs = _c3_inputs(torch, max(MIN_SETS, -(-ROTATE_BYTES // algo)))
    cpu = cpu_c3(torch, _C3_X["xc"], dtype, qmax, fake)

    def make(i):
        x = xs[i]
        st = L.stream_of(x)
        if fake:
            y = torch.empty_like(x)
            sc = torch.empty(8192, 256, dtype=torch.bfloat16, device="cuda")
            args = (L.ptr(x), L.BF16, 8192, 8192, 1, 32, L.ctypes.byref(desc), 0, shift, L.ctypes.c_float(qmax),
                    None, L.ptr(sc), None, None, None, L.ptr(y), None, 1, st)
            return (lambda: fn(*args)), (y, sc)
        codes = torch.empty(n * cb // 8, dtype=torch.uint8, device="cuda")
        e8 = torch.empty(8192, 256, dtype=torch.uint8, device="cuda")
        args = (L.ptr(x), L.BF16, 8192, 8192, 1, 32, L.ctypes.byref(desc), 0, shift, L.ctypes.c_float(qmax),
                None, None, None, L.ptr(e8), None, None, L.ptr(codes), 0, st)
        return (lambda: fn(*args)), (codes, e8)

    launches, bufs = rotate(make, algo)
    if fake:
        return launches, dict(
            name=f"C3 MX block-32 {dtype} fake-quant (bf16 values + bf16 scales), bf16 8192x8192 Laplace seed 2",
            elements=n, bytes=algo, bound="hbm", dtype="bf16", cpu=cpu,
            check=dict(x=_C3_X["xc"], out=bufs[0][0], scale=bufs[0][1]), keep=(bufs, desc))
    return launches, dict(
        name=f"C3 MX block-32 {dtype} + E8M0 scales, bf16 8192x8192 Laplace x 10^U(-1,1) seed 2 -> packed codes",
        elements=n, bytes=algo, bound="hbm", dtype=f"bf16->{dtype}", cpu=cpu,
        check=dict(x=_C3_X["xc"], codes=bufs[0][0], scale=bufs[0][1]), keep=(bufs, desc))


def c4_codebooks(torch, rows, K, seed=3):
    import numpy as np
    from scipy.stats import norm

    g = torch.Generator().manual_seed(seed)
    q = torch.tensor(norm.ppf((np.arange(K) + 0.5) / K), dtype=torch.float32)
    spacing = torch.diff(q, prepend=q[:1] - (q[1] - q[0]))
    jit = (torch.rand(rows, K, generator=g) - 0.5) * 0.5 * spacing
    return torch.sort(q + jit, dim=1).values


def setup_c4(vqx, torch, L, K, decode=False):
    g = torch.Generator().manual_seed(3)
    xc = torch.randn(4096, 4096, generator=g)
    cbc = c4_codebooks(torch, 4096, K)
    n = xc.numel()
    algo = 5 * n + cbc.numel() * 4
    enc = L.load().vqx_codebook_encode
    dec = L.load().vqx_codebook_decode

    def make(i):
        x = xc.cuda()
        cb = cbc.cuda()
        codes = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
        st = L.stream_of(x)
        eargs = (L.ptr(x), L.F32, 4096, 4096, L.ptr(cb), K, L.ptr(codes), st)
        if not decode:
            return (lambda: enc(*eargs)), (x, cb, codes)
        enc(*eargs)
        del x
        out = torch.empty(4096, 4096, dtype=torch.float32, device="cuda")
        dargs = (L.ptr(codes), 4096, 4096, L.ptr(cb), K, L.ptr(out), L.F32, st)
        return (lambda: dec(*dargs)), (None, cb, codes, out)

    launches, bufs = rotate(make, algo)
    if not decode:
        return launches, dict(
            name=f"C4 per-channel codebook encode K={K}, fp32 4096x4096 N(0,1) seed 3 -> uint8 indices",
            elements=n, bytes=algo, bound="hbm", dtype="f32->u8", cpu=cpu_c4(torch, xc, cbc, False),
            check=dict(x=xc, codebooks=cbc, codes=bufs[0][2]), keep=bufs)
    return launches, dict(
        name=f"C4 per-channel codebook decode K={K}: uint8 indices -> fp32 4096x4096",
        elements=n, bytes=algo, bound="hbm", dtype="u8->f32", cpu=cpu_c4(torch, xc, cbc, True),
        check=dict(x=xc, codebooks=cbc, codes=bufs[0][2], out=bufs[0][3]), keep=bufs)


def setup_c5(vqx, torch, L, whole_tiles=False, M=2048):
    g = torch.Generator().manual_seed(4)
    N, K = 11008, 4096
    Ac = torch.randn(M, K, generator=g).to(torch.bfloat16)
    A = Ac.cuda()
    W = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).cuda()
    Q = torch.ops.quantized_ops
    sc, codes = Q.quantize_mx_packed(W, "nf4", -1, 64, False, 1.0, "float32")
    del W
    lv = vqx.parse_format("nf4").tables(A.device)["levels_bf16"]
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    st = L.stream_of(A)
    if whole_tiles:
        fn = L.load().vqx_nf4_linear
        args = (L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), None, L.ptr(out), M, N, K, st)
        how, launches, keep = "whole 256x128 tiles only", 1, (A, codes, sc, lv, out)
    else:
        import ctypes
        n = ctypes.c_int64(0)
        L.call("vqx_nf4_linear_workspace_size", M, N, K, ctypes.byref(n))
        ws = torch.empty(n.value, dtype=torch.uint8, device="cuda")
        fn = L.load().vqx_nf4_linear_ws
        args = (L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), None, L.ptr(out), M, N, K, L.ptr(ws), n.value, st)
        if n.value:
            how, launches = "whole tiles in full rounds of the CUs, the last round's tiles split along K (stream-K)", 2
        else:
            how, launches = "whole 256x128 tiles (the last round is too full for a K split to pay)", 1
        keep = (A, codes, sc, lv, out, ws)
    return [lambda: fn(*args)], dict(
        name=f"C5 NF4-dequant linear: A bf16 [{M},4096] x W NF4 block-64 [11008,4096]^T -> bf16, fp32 accumulate; "
             + how,
        elements=M * N, flops=2 * M * N * K, bytes=M * K * 2 + N * K // 2 + N * K // 64 * 4 + M * N * 2,
        bound="mfma", dtype="bf16", cpu=cpu_c5(torch, Ac, N), launches=launches, keep=keep)


def setup_c5_linear_mx(vqx, torch, L, M=2048):
    """C5 through the reference's own op: quantized_ops::linear_mx with the
    operands convert_pt2e writes (bf16 code indices [11008, 4096], the 16 NF4
    levels as weight_code, bf16 scales [11008, 64]).  The first call packs the
    weight (cached); each step is one torch op call, whose fused kernel is
    what the HIP events time (with the op's host dispatch hidden behind the
    previous launch)."""
    g = torch.Generator().manual_seed(4)
    N, K = 11008, 4096
    Ac = torch.randn(M, K, generator=g).to(torch.bfloat16)
    A = Ac.cuda()
    idx = torch.randint(0, 16, (N, K), generator=g).to(torch.bfloat16).cuda()
    scale = (torch.rand(N, K // 64, generator=g) * 0.05 + 0.001).to(torch.bfloat16).cuda()
    # the 16 NF4 levels, ascending, as convert_pt2e's weight_code
    code = vqx.parse_format("nf4").tables(A.device)["levels_bf16"].clone()
    Q = torch.ops.quantized_ops

    def launch():
        Q.linear_mx(A, idx, None, weight_scale=scale, weight_code=code, block_size=64)
        return 0

    launch()  # packs the weight once
    return [launch], dict(
        name=f"C5 via quantized_ops::linear_mx on convert-format operands: A bf16 [{M},4096], weight = bf16 NF4 "
             f"indices [11008,4096] + weight_code (16 bf16 levels) + bf16 weight_scale [11008,64], block 64 -> bf16; "
             f"the fused dequant MFMA kernel (weight packed once, cached)",
        elements=M * N, flops=2 * M * N * K, bytes=M * K * 2 + N * K // 2 + N * K // 64 * 4 + M * N * 2,
        bound="mfma", dtype="bf16", cpu=cpu_c5(torch, Ac, N), keep=(A, idx, scale, code))


def setup_c5_linear_mx_skinny(vqx, torch, L, M=1, N=11008):
    """The decode-time call as a converted model makes it: one
    torch.ops.quantized_ops.linear_mx per step on convert-format operands
    (bf16 indices, weight_code, bf16 weight_scale) with an [M, 4096]
    activation, host dispatch included: the step time is the rate at which
    the op can be called back to back (the weight is packed once, cached)."""
    g = torch.Generator().manual_seed(4)
    K = 4096
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    idx = torch.randint(0, 16, (N, K), generator=g).to(torch.bfloat16).cuda()
    scale = (torch.rand(N, K // 64, generator=g) * 0.05 + 0.001).to(torch.bfloat16).cuda()
    code = vqx.parse_format("nf4").tables(A.device)["levels_bf16"].clone()
    Q = torch.ops.quantized_ops

    def launch():
        Q.linear_mx(A, idx, None, weight_scale=scale, weight_code=code, block_size=64)
        return 0

    launch()  # packs the weight once
    return [launch], dict(
        name=f"C5 decode-time call: quantized_ops::linear_mx per step, A bf16 [{M},4096] x convert-format NF4 weight "
             f"[{N},4096] (bf16 indices + weight_code + bf16 weight_scale, block 64) -> bf16; host dispatch included",
        elements=M * N, bytes=N * K // 2 + N * K // 64 * 4 + M * K * 2 + M * N * 2, flops=2 * M * N * K,
        bound="hbm", dtype="bf16", keep=(A, idx, scale, code))


def setup_c5_skinny(vqx, torch, L, M, N=11008):
    """C5's weight with a decode-time batch of M rows (the skinny kernel,
    bound by the 4-bit weight's bytes); N = 4096 is a 7B attention
    projection."""
    g = torch.Generator().manual_seed(4)
    K = 4096
    Ac = torch.randn(M, K, generator=g).to(torch.bfloat16)
    A = Ac.cuda()
    W = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).cuda()
    Q = torch.ops.quantized_ops
    sc, codes = Q.quantize_mx_packed(W, "nf4", -1, 64, False, 1.0, "float32")
    del W
    lv = vqx.parse_format("nf4").tables(A.device)["levels_bf16"]
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    fn = L.load().vqx_nf4_linear
    args = (L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), None, L.ptr(out), M, N, K, L.stream_of(A))
    return [lambda: fn(*args)], dict(
        name=f"C5 skinny NF4-dequant linear: A bf16 [{M},4096] x W NF4 block-64 [{N},4096]^T -> bf16",
        elements=M * N, bytes=N * K // 2 + N * K // 64 * 4 + M * K * 2 + M * N * 2, flops=2 * M * N * K,
        bound="hbm", dtype="bf16", keep=(A, codes, sc, lv, out), cpu=cpu_c5(torch, Ac, N))


def _e5m3_scales(torch, g, shape):
    e = torch.randint(-10, 1, shape, generator=g).float()
    m = torch.randint(0, 8, shape, generator=g).float()
    return (torch.exp2(e) * (1 + m / 8)).to(torch.bfloat16).cuda()


def _graph_of(torch, op):
    """One call of `op` captured in a HIP graph (after a warm-up call that
    fills the host caches), replayed once per step: the step is exactly the
    GPU work the op launches, without its host dispatch."""
    op()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = op()
    torch.cuda.synchronize()

    def launch():
        g.replay()
        return 0

    return launch, (g, out)


def setup_c6_attention(vqx, torch, L, which, coded=False):
    """The LLaMA-7B attention products of a converted model (B 1, 32 heads,
    2048 positions, head dim 128) with the reference's attention specs:
    int6 operands (or nf4_6 indices with the 16-entry code), the left one
    blocked along -1 and the right one along -2 (the contraction dim), bf16
    scales on the fp8_e5m3 grid, through quantized_ops::matmul_mx (graph
    replay of one call: the decode of the operands that many tiles read, then
    vqx_mx_matmul).  qk: [1,32,2048,128] x [1,32,128,2048]; pv:
    [1,32,2048,2048] x [1,32,2048,128]."""
    g = torch.Generator().manual_seed(6)
    H, S, D, bs = 32, 2048, 128, 64
    hi, lo = (16, 0) if coded else (32, -32)
    M, N, K = (S, S, D) if which == "qk" else (S, D, S)
    a = torch.randint(lo, hi, (1, H, M, K), generator=g).to(torch.bfloat16).cuda()
    b = torch.randint(lo, hi, (1, H, K, N), generator=g).to(torch.bfloat16).cuda()
    a_s = _e5m3_scales(torch, g, (1, H, M, K // bs))
    b_s = _e5m3_scales(torch, g, (1, H, K // bs, N))
    code = None
    if coded:
        code = torch.tensor([-31., -22., -16., -12., -9., -6., -3., 0., 2., 5., 8., 10., 14., 17., 22., 31.],
                            dtype=torch.bfloat16, device="cuda")
    Q = torch.ops.quantized_ops
    launch, keep = _graph_of(torch, lambda: Q.matmul_mx(a, b, input_scale=a_s, weight_scale=b_s, block_size=bs,
                                                        input_code=code, weight_code=code))
    fmt = "nf4_6 indices + 16-entry code" if coded else "int6"
    nbytes = 2 * H * (M * K + K * N + M * (K // bs) + (K // bs) * N + M * N)
    return [launch], dict(
        name=f"C6 attention {which.upper()} of LLaMA-7B through quantized_ops::matmul_mx: [1,32,{M},{K}] x "
             f"[1,32,{K},{N}] ({fmt}, bf16 fp8_e5m3-grid scales per 64 along K on both sides) -> bf16; one call "
             f"replayed from a HIP graph",
        elements=H * M * N, flops=2 * H * M * N * K, bytes=nbytes, bound="hbm", dtype="bf16",
        keep=(a, b, a_s, b_s, code, keep))


def setup_c6_mxnf4_linear(vqx, torch, L, M=2048, N=11008, K=4096):
    """The MXNF4 CI scheme's linear at the LLaMA-7B MLP shape through
    quantized_ops::linear_mx: nf4_6 activation indices with input_code and
    fp8_e5m3-grid input_scale per 64 along K, a convert-format nf4_6 weight
    (16-entry weight_code, weight_scale per 64): the activation's decode pass,
    then the packed-weight product (graph replay of one call; the weight is
    packed once, cached)."""
    g = torch.Generator().manual_seed(8)
    bs = 64
    code = torch.tensor([-31., -22., -16., -12., -9., -6., -3., 0., 2., 5., 8., 10., 14., 17., 22., 31.],
                        dtype=torch.bfloat16, device="cuda")
    x = torch.randint(0, 16, (M, K), generator=g).to(torch.bfloat16).cuda()
    w = torch.randint(0, 16, (N, K), generator=g).to(torch.bfloat16).cuda()
    xs = _e5m3_scales(torch, g, (M, K // bs))
    ws = _e5m3_scales(torch, g, (N, K // bs))
    Q = torch.ops.quantized_ops
    launch, keep = _graph_of(torch, lambda: Q.linear_mx(x, w, None, input_scale=xs, weight_scale=ws, block_size=bs,
                                                        input_code=code, weight_code=code))
    return [launch], dict(
        name=f"C6 MXNF4 linear through quantized_ops::linear_mx: nf4_6 A indices [{M},{K}] + input_code + "
             f"input_scale, nf4_6 W [{N},{K}] convert format, blocks of 64 -> bf16; one call replayed from a HIP graph",
        elements=M * N, flops=2 * M * N * K, bytes=2 * M * K + N * K // 2 + 2 * (M + N) * (K // bs) + 2 * M * N,
        bound="mfma", dtype="bf16", keep=(x, w, xs, ws, code, keep))


def setup_c6_mxint8_linear(vqx, torch, L, M=2048, N=11008, K=4096):
    """The MXINT8 CI scheme's linear at the LLaMA-7B MLP shape through
    quantized_ops::linear_mx: int8 activations and weights (integer-valued
    bf16, as convert writes them), power-of-two bf16 scales per 16 along K on
    both sides (graph replay of one call: the activation's decode, the
    product; the weight's decode is cached per weight)."""
    g = torch.Generator().manual_seed(7)
    bs = 16
    x = torch.randint(-127, 128, (M, K), generator=g).to(torch.bfloat16).cuda()
    w = torch.randint(-127, 128, (N, K), generator=g).to(torch.bfloat16).cuda()
    xs = torch.exp2(torch.randint(-12, -4, (M, K // bs), generator=g).float()).to(torch.bfloat16).cuda()
    ws = torch.exp2(torch.randint(-12, -4, (N, K // bs), generator=g).float()).to(torch.bfloat16).cuda()
    Q = torch.ops.quantized_ops
    launch, keep = _graph_of(torch, lambda: Q.linear_mx(x, w, None, input_scale=xs, weight_scale=ws, block_size=bs))
    return [launch], dict(
        name=f"C6 MXINT8 linear through quantized_ops::linear_mx: int8 A [{M},{K}] x int8 W [{N},{K}]^T, bf16 "
             f"power-of-two scales per 16 along K on both sides -> bf16; one call replayed from a HIP graph",
        elements=M * N, flops=2 * M * N * K, bytes=2 * (M * K + N * K + (M + N) * (K // bs) + M * N),
        bound="mfma", dtype="bf16", keep=(x, w, xs, ws, keep))


def setup_c6_dense_library(vqx, torch, L, which):
    """Comparison point, not this build's code: the C6 products on operands
    already decoded to dense bf16, through torch.matmul / F.linear
    (hipBLASLt): the GEMM half of the reference's decode-then-product, with
    the decode not counted."""
    g = torch.Generator().manual_seed(6)
    if which == "linear":
        M, N, K = 2048, 11008, 4096
        a = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
        b = torch.randn(N, K, generator=g).to(torch.bfloat16).cuda()
        F = torch.nn.functional
        fn, H = (lambda: F.linear(a, b)), 1
    else:
        H, S, D = 32, 2048, 128
        M, N, K = (S, S, D) if which == "qk" else (S, D, S)
        a = torch.randn(H, M, K, generator=g).to(torch.bfloat16).cuda()
        b = torch.randn(H, K, N, generator=g).to(torch.bfloat16).cuda()
        fn = lambda: torch.matmul(a, b)

    def launch():
        fn()
        return 0

    return [launch], dict(
        name=f"comparison: library bf16 GEMM on pre-decoded operands, [{H}] x [{M},{K}] x [{K},{N}] (hipBLASLt)",
        elements=H * M * N, flops=2 * H * M * N * K, bytes=2 * H * (M * K + K * N + M * N),
        bound="mfma" if which == "linear" else "hbm", dtype="bf16", keep=(a, b))


def setup_c5_dense_library(vqx, torch, L, N=11008, M=2048):
    """Comparison point, not this build's code: C5's product with an already
    dense bf16 weight through torch.nn.functional.linear (hipBLASLt), i.e. the
    GEMM half of the reference's own linear_mx (decode, then F.linear), with
    the decode not counted."""
    g = torch.Generator().manual_seed(4)
    K = 4096
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    W = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).cuda()
    F = torch.nn.functional

    def launch():
        F.linear(A, W)
        return 0

    return [launch], dict(
        name=f"comparison: dense bf16 A [{M},4096] x W [{N},4096]^T through torch F.linear (hipBLASLt), the GEMM "
             f"the reference's linear_mx runs after its decode (decode not counted)",
        elements=M * N, flops=2 * M * N * K, bytes=M * K * 2 + N * K * 2 + M * N * 2, bound="mfma", dtype="bf16",
        keep=(A, W))


def setup_l1(vqx, torch, L):
    """Learned-codebook calibration statistics of a 4096x4096 fp32 weight:
    unit_scale in blocks of 64 (quant_max 7) fused with the 4001-bin fp64
    histogram of Histogram.add, unit weights."""
    g = torch.Generator().manual_seed(9)
    xc = torch.randn(4096, 4096, generator=g)
    n = xc.numel()
    h = vqx.quantization.Histogram(-7.0, 7.0, 4001)
    edges = h._prepare(torch.device("cuda"))
    fn = L.load().vqx_lcq_histogram

    def make(i):
        # every set adds into the one histogram (its 96 KB of bins stay
        # cached either way); the inputs rotate
        x = xc.cuda()
        args = (L.ptr(x), L.F32, n, 64, L.ctypes.c_float(7.0), None, 1, L.ptr(edges), 4001, L.ptr(h.weight),
                L.ptr(h.total), L.ptr(h.square), L.stream_of(x))
        return (lambda: fn(*args)), x

    algo = n * 4 + 3 * 4001 * 8
    launches, bufs = rotate(make, algo)
    return launches, dict(
        name="L1 LCQ calibration histogram: unit_scale (blocks of 64, quant_max 7) + 4001-bin fp64 moments of a "
             "fp32 4096x4096 N(0,1) seed 9",
        elements=n, bytes=algo, bound="hbm", dtype="f32->f64", cpu_input=xc, keep=(h, edges, bufs))


def setup_g1(vqx, torch, L):
    """GPTQ compensation of a 4096x4096 fp32 weight (a 7B-class attention
    projection) onto int4 blocks of 64, salience ordering on, damping 0.01,
    from the Hessian of 16384 synthetic tokens.  One step is the whole
    compensate_weight: permutation, Cholesky factor of the inverse Hessian,
    64 block launches and the 63 trailing fp32 GEMM updates."""
    g = torch.Generator().manual_seed(11)
    C, Rw, T = 4096, 4096, 16384
    X = torch.randn(T, C, generator=g) * (torch.rand(C, generator=g) * 2 + 0.1)
    Hc = X.T @ X
    wc = torch.randn(Rw, C, generator=g) * 0.02
    w, H = wc.cuda(), Hc.cuda()
    fq = SimpleNamespace(qmap=vqx.quantization.get_quantization_map("int4", "cuda"), scale_qmap=None, quant_max=7.0, block_size=64, ch_axis=-1)
    comp = vqx.quantization.compensate_weight

    def launch():
        comp(w, H, T, fq, 0.01)
        return 0

    nb = C // 64
    # the trailing updates: sum over blocks of 2 * rows * 64 * (columns after the block)
    flops = sum(2 * Rw * 64 * (C - 64 * (b + 1)) for b in range(nb))

    def cpu():
        from oracle import formats as F
        from oracle import reference_ops as R

        q = R.table_tensor(F.quantization_table("int4"))
        return _timed(lambda: R.gptq_compensate_weight(wc, Hc.clone(), T, q, 7.0, 64, 0.01)), \
            "the oracle's compensate_weight on the full 4096x4096 weight"

    return [launch], dict(
        name="G1 GPTQ compensate_weight: fp32 4096x4096 weight N(0,0.02) seed 11 onto int4 blocks of 64 "
             "(act_order, damping 0.01), Hessian of 16384 synthetic tokens; one step = the whole compensation "
             "(many launches: the block kernel, Cholesky, trailing GEMMs)",
        elements=w.numel(), bytes=0, flops=flops, bound="fp32", dtype="f32", cpu=cpu, multi_launch=True,
        keep=(w, H))


def outlier_input(torch, rows=4096, cols=11008, seed=5):
    """Activation-like bf16 [tokens, features]: N(0,1) with 0.5% of the
    entries scaled by 32, the outliers the CSR path splits off (|x| > 6)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g)
    m = torch.rand(rows, cols, generator=g) < 0.005
    return torch.where(m, x * 32, x).to(torch.bfloat16)


OUTLIER_THRESHOLD, OUTLIER_PCT = 6.0, 0.01


def _outlier_csr(torch, L, x):
    R, C = x.shape
    max_nnz = int(R * C * OUTLIER_PCT)
    bufs = dict(data=torch.empty(max_nnz, dtype=torch.bfloat16, device="cuda"),
                idx=torch.empty(max_nnz, dtype=torch.int32, device="cuda"),
                ptr=torch.empty(R + 1, dtype=torch.int32, device="cuda"),
                inl=torch.empty_like(x))
    args = (L.ptr(x), L.BF16, 1, R, C, L.ctypes.c_float(OUTLIER_THRESHOLD), max_nnz, 0, L.ptr(bufs["data"]),
            L.ptr(bufs["idx"]), L.ptr(bufs["ptr"]), L.ptr(bufs["inl"]), L.stream_of(x))
    return bufs, args, max_nnz


def setup_o1(vqx, torch, L, mx=False):
    xc = outlier_input(torch)
    R, C = xc.shape
    n = xc.numel()
    max_nnz = int(R * C * OUTLIER_PCT)
    # the one-pass entry points: x read once, the outliers staged in a
    # workspace and placed by a second, small launch
    wsz = L.ctypes.c_int64(0)
    L.call("vqx_outlier_workspace_size", L.BF16, 1, R, C, max_nnz, L.ctypes.byref(wsz))
    filt = L.load().vqx_filter_outlier_ws
    fused = L.load().vqx_quantize_mx_outlier_ws
    table = vqx.get_quantization_map("fp8_e4m3", "cuda")
    csr_bytes = 6 * max_nnz + 4 * (R + 1)
    algo = 4 * n + n // 32 * 2 + csr_bytes if mx else 4 * n + csr_bytes

    def make(i):
        x = xc.cuda()
        bufs, fargs, _ = _outlier_csr(torch, L, x)
        ws = torch.empty(max(wsz.value, 1), dtype=torch.uint8, device="cuda")
        fargs = fargs[:-1] + (L.ptr(ws), wsz.value, fargs[-1])
        if not mx:
            L.call("vqx_filter_outlier_ws", *fargs)
            return (lambda: filt(*fargs)), (x, bufs, ws)
        # the one-pass form: the split writes the quantized inliers and their
        # block scales instead of the inliers
        sc = torch.empty(R, C // 32, dtype=torch.bfloat16, device="cuda")
        qv = torch.empty_like(x)
        margs = (L.ptr(x), 1, R, C, L.ctypes.c_float(OUTLIER_THRESHOLD), max_nnz, 0, 32, 0, 8,
                 L.ctypes.c_float(448.0), None, L.ptr(table), L.ptr(bufs["data"]), L.ptr(bufs["idx"]),
                 L.ptr(bufs["ptr"]), L.ptr(sc), L.ptr(qv), L.ptr(ws), wsz.value, L.stream_of(x))
        L.call("vqx_quantize_mx_outlier_ws", *margs)
        return (lambda: fused(*margs)), (x, bufs, ws, sc, qv)

    launches, sets = rotate(make, algo)
    torch.cuda.synchronize()
    nnz = int(sets[0][1]["ptr"][-1])
    common = dict(elements=n, bound="hbm", dtype="bf16", nnz=nnz, bytes=algo,
                  cpu_input=(xc, OUTLIER_THRESHOLD, OUTLIER_PCT), keep=(sets, table))
    if not mx:
        return launches, dict(
            name=f"O1 filter_outlier, bf16 4096x11008 N(0,1) with 0.5% x32 seed 5, |x| > {OUTLIER_THRESHOLD}, "
                 f"capacity 1% -> CSR ({nnz} outliers) + inliers", **common)
    return launches, dict(
        name=f"O2 quantize_mx_outlier: O1's CSR and, in the same split pass, MX block-32 fp8_e4m3 power-of-two "
             f"scales and quantized values of the inliers -> CSR + bf16 scales + bf16 quantized inliers", **common)


def setup_o3(vqx, torch, L):
    x = outlier_input(torch).cuda()
    R, K = x.shape
    N = 4096
    bufs, fargs, max_nnz = _outlier_csr(torch, L, x)
    L.load().vqx_filter_outlier(*fargs)
    torch.cuda.synchronize()
    nnz = int(bufs["ptr"][-1])
    del x
    g = torch.Generator().manual_seed(6)
    Bc = (0.02 * torch.randn(K, N, generator=g)).to(torch.bfloat16)
    fn = L.load().vqx_spmm_csr
    algo = nnz * 6 + 4 * (R + 1) + K * N * 2 + R * N * 2

    def make(i):
        # the CSR (a few MB) is shared; B and the output rotate
        B = Bc.cuda()
        out = torch.empty(R, N, dtype=torch.bfloat16, device="cuda")
        args = (L.ptr(bufs["data"]), L.BF16, L.ptr(bufs["idx"]), L.ptr(bufs["ptr"]), 1, R, max_nnz, L.ptr(B),
                L.BF16, 0, K, N, None, L.ptr(out), L.stream_of(B))
        return (lambda: fn(*args)), (B, out)

    launches, sets = rotate(make, algo)
    cpu = (bufs["data"].cpu(), bufs["idx"].cpu(), bufs["ptr"].cpu(), Bc)
    return launches, dict(
        name=f"O3 spmm_csr: O1's CSR [4096 x 11008] ({nnz} entries) x bf16 [11008, 4096] ('ck') -> bf16, "
             f"fp32 accumulate",
        elements=R * N, bytes=algo, gathered_bytes=nnz * N * 2,
        flops=2 * nnz * N, bound="hbm", dtype="bf16", nnz=nnz, cpu_input=cpu, keep=(bufs, sets))


def setup_f1(vqx, torch, L, spec, shape, seed=13):
    """FusedAmaxObsFakeQuantize forward with outliers, as the reference's
    LLaMA outlier configs quantize a Linear's activation (opct: the top 1%
    by magnitude, with the threshold's running average) or the attention's
    value operand (othr: |x| >= 6), on bf16 activations N(0,1) with 1% of
    the entries scaled by 20.  One step is one module forward: the top-k
    threshold passes (opct) and the fused mask / MX fake-quant / restore /
    count pass, all on the device."""
    g = torch.Generator().manual_seed(seed)
    xc = torch.randn(*shape, generator=g)
    xc = torch.where(torch.rand(shape, generator=g) < 0.01, xc * 20, xc).to(torch.bfloat16)
    fq = vqx.quantization.QuantizationSpec.from_str(spec).make_fake_quantize("cuda").cuda()
    n = xc.numel()

    def make(i):
        x = xc.cuda()
        return (lambda: (fq(x), 0)[1]), x

    # the fused pass reads x and writes y and the scales; the opct threshold
    # needs x read once more before it (the select's minimum)
    algo = 4 * n + n // 64 * 2 + (2 * n if "opct" in spec else 0)
    launches, bufs = rotate(make, 4 * n)
    launches[0]()
    torch.cuda.synchronize()
    return launches, dict(
        name=f"F1 FusedAmaxObsFakeQuantize('{spec}') forward, bf16 {list(shape)} N(0,1) with 1% x20 outliers seed "
             f"{seed}: every kernel on the device, no host synchronisation",
        elements=n, bytes=algo, bound="hbm", dtype="bf16", multi_launch=True, keep=(fq, bufs))


CONFIGS = {
    "c2": lambda v, t, L: setup_c2(v, t, L),
    "c1": lambda v, t, L: setup_c1(v, t, L),
    "c2_decode": lambda v, t, L: setup_c2(v, t, L, decode=True),
    "c3_e4m3": lambda v, t, L: setup_c3(v, t, L, "fp8_e4m3", 448.0),
    "c3_e3m2": lambda v, t, L: setup_c3(v, t, L, "fp6_e3m2", 28.0),
    "c3_e2m1": lambda v, t, L: setup_c3(v, t, L, "fp4_e2m1", 6.0),
    "c3_e4m3_fq": lambda v, t, L: setup_c3(v, t, L, "fp8_e4m3", 448.0, fake=True),
    "c4_k16": lambda v, t, L: setup_c4(v, t, L, 16),
    "c4_k256": lambda v, t, L: setup_c4(v, t, L, 256),
    "c4_k16_decode": lambda v, t, L: setup_c4(v, t, L, 16, decode=True),
    "c5": lambda v, t, L: setup_c5(v, t, L),
    "c5_linear_mx": lambda v, t, L: setup_c5_linear_mx(v, t, L),
    "c5_m256": lambda v, t, L: setup_c5(v, t, L, M=256),
    "c5_m1": lambda v, t, L: setup_c5_skinny(v, t, L, 1),
    "c5_m16": lambda v, t, L: setup_c5_skinny(v, t, L, 16),
    "c5_m1_n4096": lambda v, t, L: setup_c5_skinny(v, t, L, 1, N=4096),
    "c5_linear_mx_m1": lambda v, t, L: setup_c5_linear_mx_skinny(v, t, L, 1),
    "f3_gwa": lambda v, t, L: setup_f3(v, t, L),
    "o1_filter": lambda v, t, L: setup_o1(v, t, L),
    "o2_quantize_mx_outlier": lambda v, t, L: setup_o1(v, t, L, mx=True),
    "o3_spmm": lambda v, t, L: setup_o3(v, t, L),
    "l1_histogram": lambda v, t, L: setup_l1(v, t, L),
    "f1_outlier_opct": lambda v, t, L: setup_f1(v, t, L, "nf4_6,qs=microscaling,bs=64,ax=-1,scale=fp8_e5m3,opct=0.01",
                                                (2048, 4096)),
    "f1_outlier_othr_ax2": lambda v, t, L: setup_f1(v, t, L, "nf4_6,qs=microscaling,bs=64,ax=-2,scale=fp8_e5m3,othr=6.0",
                                                    (1, 32, 2048, 128)),
    "g1_gptq": lambda v, t, L: setup_g1(v, t, L),
    "c6_attn_qk_int6": lambda v, t, L: setup_c6_attention(v, t, L, "qk"),
    "c6_attn_pv_int6": lambda v, t, L: setup_c6_attention(v, t, L, "pv"),
    "c6_mxint8_linear": lambda v, t, L: setup_c6_mxint8_linear(v, t, L),
}
HEADLINE = "c2"


def _check_rc(rc):
    if rc != 0:
        raise RuntimeError(f"launch failed: {rc}")


def time_config(torch, launches, steps, warmup, warm=True):
    """Time a config's launches, each step one C-ABI call that launches one
    kernel, cycling through the config's buffer sets (launches[i % n]):

    (1) the whole region of `steps` back-to-back launches between two HIP
        events on the launch stream, after `warmup` untimed ones; region /
        steps is the kernel's average duration (plus the back-to-back launch
        gap), and every figure the bench reports uses it.  With n > 1 sets
        the inputs come from HBM (cold MALL).
    (2) each launch between its own pair of events, queued behind a GPU spin
        so that the host has enqueued every pair before the GPU reaches it
        (otherwise a pair also spans the host's launch latency); the median.
    (3) with `warm` and n > 1: (1) again on the first set only, so that every
        launch after the first finds its input in the MALL (the warm time)."""
    n = len(launches)

    def region(seq):
        for i in range(warmup):
            _check_rc(seq(i)())
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        t0.record()
        for i in range(steps):
            seq(i)()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1), time.perf_counter() - w0

    region_ms, wall = region(lambda i: launches[i % n])
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    try:
        torch.cuda._sleep(20_000_000)  # ~10 ms of GPU spin while the pairs are enqueued
    except (AttributeError, RuntimeError):
        pass
    for i in range(steps):
        starts[i].record()
        launches[i % n]()
        ends[i].record()
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    out = {"kernel_ms_avg": region_ms / steps, "kernel_ms_isolated_median": statistics.median(per),
           "region_ms": region_ms, "wall_s": wall, "buffer_sets": n}
    if warm and n > 1:
        warm_ms, _ = region(lambda i: launches[0])
        out["kernel_ms_warm"] = warm_ms / steps
    return out


def cpu_baseline_c2(torch, x):
    """The reference's CPU path for C2 (calculate_mx_qparam absmax + quantize
    with the NF index table), timed on this host."""
    import numpy as np

    from oracle import formats as F
    from oracle import reference_ops as R

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    lv = F.nf_levels(4)
    idx_q = torch.from_numpy(F.nf_index_table(lv).astype(np.float32)).to(torch.bfloat16)
    # the full C2 tensor, repeated until about 10 s of CPU work is timed
    xs = x.contiguous()

    def run():
        s = R.calculate_mx_qparam(xs, [-1], 64, 1.0, False)
        return R.quantize(xs, s, None, [-1], 64, idx_q)

    for _ in range(2):  # warm-up
        run()
    ts = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < 10.0 or len(ts) < 3:
        t = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t)
    med = statistics.median(ts)
    return {"value": xs.numel() / med, "unit": "elements/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"full C2 tensor (45,088,768 bf16 elements), 2 warm-ups + {len(ts)} timed runs "
                      f"(~10 s), median {med:.3f} s; torch-CPU restatement of calculate_mx_qparam + quantize "
                      f"with the NF4 index table",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count()}


def cpu_oracle_time(torch, k, info, kernel_ms):
    """One run of the CPU oracle (the reference's torch-CPU op sequence) on a
    config's input, or a bounded sample of it scaled to the whole config,
    timed beside the GPU figure."""
    from oracle import formats as F
    from oracle import reference_ops as R

    torch.set_num_threads(os.cpu_count() or 1)
    if "cpu" in info:
        dt, sample = info["cpu"]()
        return {"seconds": dt, "cores": torch.get_num_threads(), "kind": "port",
                "gpu_speedup": dt / (kernel_ms * 1e-3), "elements_per_s": info["elements"] / dt, "sample": sample,
                "timing": f"each timed piece: {CPU_WARMUP} warm-up runs, then the median of {CPU_RUNS}"}
    if k == "l1_histogram":
        x = info["cpu_input"]

        def fn():
            u = R.unit_scale(x, 64, 7.0).reshape(-1)
            return R.lcq_histogram_add(u, torch.ones(()), -7.0, 7.0, 4001)
    elif k == "o3_spmm":
        d, i, p, B = info["cpu_input"]

        def fn():
            return R.spmm_csr(d, i, p, B, weight_layout="ck")
    else:
        x, t, pct = info["cpu_input"]
        if k == "o1_filter":
            def fn():
                return R.filter_outlier(x, t, pct)
        else:
            qmap = R.table_tensor(F.quantization_table("fp8_e4m3"))

            def fn():
                return R.quantize_mx_outlier(x, qmap, [-1], 32, 448.0, True, threshold=t, max_pct=pct)
    dt = _timed(fn)
    return {"seconds": dt, "cores": torch.get_num_threads(), "kind": "port", "gpu_speedup": dt / (kernel_ms * 1e-3),
            "elements_per_s": info["elements"] / dt, "sample": "the config's full input",
            "timing": f"{CPU_WARMUP} warm-up runs, then the median of {CPU_RUNS}"}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# Kernel that dominates each config's launch (rocprofv3 names it this way).
# configs run only when named with --only: comparison points that would
# share a kernel name with a default config in a rocprof run of all of them
ON_REQUEST = {
    "c5_m256_whole_tiles": lambda v, t, L: setup_c5(v, t, L, whole_tiles=True, M=256),
    "c5_dense_library": lambda v, t, L: setup_c5_dense_library(v, t, L),
    "c5_dense_library_n8192": lambda v, t, L: setup_c5_dense_library(v, t, L, N=8192),
    "c6_attn_qk_nf4_6": lambda v, t, L: setup_c6_attention(v, t, L, "qk", coded=True),
    "c6_mxnf4_linear": lambda v, t, L: setup_c6_mxnf4_linear(v, t, L),
    "c6_qk_dense_library": lambda v, t, L: setup_c6_dense_library(v, t, L, "qk"),
    "c6_pv_dense_library": lambda v, t, L: setup_c6_dense_library(v, t, L, "pv"),
    "c6_linear_dense_library": lambda v, t, L: setup_c6_dense_library(v, t, L, "linear"),
}

DOMINANT = {
    "c1": "fq_lut_kernel<float, 1>",
    "c2": "mx_lut_kernel<4, 4, true, 0, true>",
    "c2_decode": "decode_group_kernel<unsigned short, 4, 4>",
    "c3_e4m3": "mx_lut_kernel<8, 2, false, 0, true>",
    "c3_e3m2": "mx_lut_kernel<6, 2, false, 0, false>",
    "c3_e2m1": "mx_lut_kernel<4, 2, false, 0, true>",
    "c3_e4m3_fq": "mx_lut_kernel<0, 2, false, 2, false>",
    "c4_k16": "cb_encode_kernel<float, 4>",
    "c4_k256": "cb_encode_kernel<float, 8>",
    "c4_k16_decode": "cb_decode_kernel<float>",
    "c5": "nf4_gemm_kernel",
    "c5_linear_mx": "nf4_gemm_kernel",
    "c5_m256": "nf4_gemm_sk_kernel",
    "c5_m256_whole_tiles": "nf4_gemm_kernel",
    "c5_m1": "nf4_skinny_kernel",
    "c5_m16": "nf4_skinny_kernel",
    "c5_m1_n4096": "nf4_skinny_kernel",
    "c5_linear_mx_m1": "nf4_skinny_kernel",
    "f3_gwa": "gwa_fq_rows_kernel<unsigned short, 8>",
    "o1_filter": "outlier_split_kernel<1, 8, false, 1, true>",
    "o2_quantize_mx_outlier": "outlier_split_kernel<1, 8, true, 4, true>",
    "o3_spmm": "spmm_csr_kernel<1, 8>",
    "l1_histogram": "lcq_hist_kernel<0, true, false>",
    "g1_gptq": "gptq_block_kernel",
    "f1_outlier_opct": "mx_lut_kernel<0, 4, true, 2, false, true>",
    "f1_outlier_othr_ax2": "mx_cols_lut_kernel<true, 4, true>",
    "c6_attn_qk_int6": "mx_gemm_kernel<0, 0, false, 128, 128>",
    "c6_attn_pv_int6": "mx_gemm_kernel<1, 0, false, 128, 128>",
    "c6_mxint8_linear": "mx_gemm_kernel<0, 0, true, 256, 128>",
}
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")


def measured_traffic(key):
    """HBM bytes per launch of a config's dominant kernel, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE passes summarised in profiles/hbm_traffic.json
    (already scaled by the copy-kernel calibration), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t["configs"][key]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError, TypeError):
        return None


def hbm_ceiling(steps, warmup):
    """HBM bandwidth by traffic mix with 1 GiB working sets, which the 256 MiB
    MALL cannot hold: read only (torch amax and sum reductions), write only
    (torch fill_), 1:1 (torch copy_), and two
    passes of this library's MX kernel over a bf16 16384x32768 input: E8M0
    scales only (read-mostly: 2 B read, 1/32 B written per element) and the
    C3 e4m3 quantize (2:1 read:write).  One JSON line."""
    import torch

    import __graft_entry__

    n = 1 << 28  # 1 GiB of fp32
    a = torch.empty(n, dtype=torch.float32, device="cuda").uniform_()
    b = torch.empty_like(a)
    res = {}

    def run(name, fn, nbytes):
        tm = time_config(torch, [lambda: (fn(), 0)[1]], steps, warmup)
        ms = tm["kernel_ms_avg"]
        res[name] = {"bytes": nbytes, "ms": ms, "GBps": nbytes / (ms * 1e-3) / 1e9,
                     "frac_of_8TBps": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        print(f"[bench] hbm ceiling {name}: {ms * 1e3:.1f} us, {res[name]['GBps']:.0f} GB/s", file=sys.stderr,
              flush=True)

    run("read_1GiB (torch amax)", lambda: torch.amax(a), 4 * n)
    run("read_1GiB (torch sum)", lambda: a.sum(), 4 * n)
    run("write_1GiB (torch fill_)", lambda: b.fill_(1.0), 4 * n)
    run("copy_1GiB_to_1GiB (torch copy_)", lambda: b.copy_(a), 8 * n)
    del a, b
    torch.cuda.empty_cache()
    # the probe library's streaming kernel at fixed read:write mixes, each
    # stream 512 MiB (16-byte accesses, 1 KiB per wave instruction; stores
    # non-temporal, loads non-temporal or plain), with a one-shot grid (a
    # workgroup per 256 units) and with a persistent grid of 2048 workgroups
    import ctypes

    if not os.path.exists(PROBE_LIB):
        sys.exit(f"bench.py --hbm-ceiling: {PROBE_LIB} is missing; build it first with python bench.py --build-probe")
    probe = ctypes.CDLL(PROBE_LIB)
    fn = probe.vqx_probe_hbm_mix_loads
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    units = 1 << 25
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    big = torch.empty(4 * units * 16, dtype=torch.uint8, device="cuda").random_()
    out = torch.empty(4 * units * 16, dtype=torch.uint8, device="cuda")
    sink = torch.empty(max(units // 256, 2048) * 256, dtype=torch.int32, device="cuda")
    for r, w in ((1, 0), (0, 1), (1, 1), (2, 1), (4, 1), (1, 2), (1, 4)):
        for grid, how in ((units // 256, "one-shot grid"), (2048, "persistent grid")):
            for nt, kind in ((1, "non-temporal loads"), (0, "plain loads")):
                if r == 0 and nt == 0:
                    continue
                args = (big.data_ptr(), out.data_ptr(), units, r, w, sink.data_ptr(), grid, nt, st)
                run(f"probe read:write {r}:{w} ({how}, {kind})", lambda: fn(*args), (r + w) * units * 16)
    del big, out, sink
    torch.cuda.empty_cache()
    vqx = __graft_entry__.load_package()
    L = vqx._lib
    rows, cols = 16384, 32768
    x = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda").normal_()
    fmt = vqx.parse_format("fp8_e4m3")
    desc = fmt.desc(x.device)
    codes = torch.empty(rows * cols, dtype=torch.uint8, device="cuda")
    e8 = torch.empty(rows, cols // 32, dtype=torch.uint8, device="cuda")
    fn = L.load().vqx_mx_quantize
    sargs = (L.ptr(x), L.BF16, rows, cols, 1, 32, L.ctypes.byref(desc), 0, 8, L.ctypes.c_float(448.0), None,
             None, None, L.ptr(e8), None, None, None, 0, L.stream_of(x))
    run("read_mostly_1GiB (vqx MX scales only)", lambda: fn(*sargs), rows * cols * 2 + e8.numel())
    args = (L.ptr(x), L.BF16, rows, cols, 1, 32, L.ctypes.byref(desc), 0, 8, L.ctypes.c_float(448.0), None, None,
            None, L.ptr(e8), None, None, L.ptr(codes), 0, L.stream_of(x))
    run("c3_e4m3_kernel_1GiB_input", lambda: fn(*args), rows * cols * 3 + e8.numel())
    print(json.dumps({"hbm_ceiling": res, "note": "1 GiB working sets, beyond the 256 MiB MALL"}))


PROBE_SRC = os.path.join(ROOT, "bench_hbm_probe.hip")
PROBE_LIB = os.path.join(ROOT, "bench_hbm_probe.so")


def build_probe():
    """Compile the HBM traffic-mix probe (bench_hbm_probe.hip) for gfx950, on
    the host, before a GPU run of --hbm-ceiling."""
    import subprocess

    tmp = PROBE_LIB + ".tmp"
    subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", PROBE_SRC, "-o", tmp], check=True)
    os.replace(tmp, PROBE_LIB)
    print(PROBE_LIB)


def calibrate_copy():
    import torch

    n = 512 << 20
    x = torch.ones(n // 4, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "launches": 5}))


def main():
    a = parse()
    if a.build_probe:
        build_probe()
        return
    if a.calibrate_copy:
        calibrate_copy()
        return
    if a.hbm_ceiling:
        hbm_ceiling(a.steps, a.warmup)
        return
    if a.gpus != 1:
        print(json.dumps({"error": "bench.py runs on one GPU only: this build has no multi-GPU path "
                                   f"(asked for --gpus {a.gpus})"}))
        sys.exit(2)
    import torch

    import __graft_entry__

    vqx = __graft_entry__.load_package()
    L = vqx._lib
    keys = list(CONFIGS) if a.only is None else a.only.split(",")
    for k in keys:
        if k not in CONFIGS and k not in ON_REQUEST:
            sys.exit(f"bench.py: unknown config {k!r}")
    if HEADLINE not in keys:
        keys = [HEADLINE] + keys
    results = {}
    info_head = None
    for k in keys:
        print(f"[bench] {k}: setup", file=sys.stderr, flush=True)
        launches, info = {**CONFIGS, **ON_REQUEST}[k](vqx, torch, L)
        tm = time_config(torch, launches, a.steps, a.warmup, warm=not a.no_warm)
        ms = tm["kernel_ms_avg"]
        gbs = info["bytes"] / (ms * 1e-3) / 1e9
        region = tm["region_ms"] / a.steps
        results[k] = {
            "workload": info["name"], "elements_per_s": info["elements"] / (region * 1e-3),
            "kernel_ms": ms, "kernel_ms_isolated_median": tm["kernel_ms_isolated_median"],
            "region_ms_per_step": region, "kernel": DOMINANT.get(k),
            "hbm_traffic_bytes": measured_traffic(k),
            "algorithmic_bytes": info["bytes"], "achieved_GBps": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
            "dtype": info["dtype"], "buffer_sets": tm["buffer_sets"]}
        if tm["buffer_sets"] > 1:
            results[k]["buffer_set_bytes"] = info["bytes"]
            results[k]["timing"] = (f"cold MALL: the timed launches cycle through {tm['buffer_sets']} sets of "
                                    f"input and output buffers (> 512 MiB together)")
        if "kernel_ms_warm" in tm:
            mw = tm["kernel_ms_warm"]
            results[k]["kernel_ms_warm"] = mw
            results[k]["hbm_frac_warm"] = info["bytes"] / (mw * 1e-3) / 1e9 / HBM_PEAK_GBS
        if info.get("launches", 1) > 1:
            results[k]["launches_per_step"] = info["launches"]
        if info.get("multi_launch"):
            # one step is a whole host routine of many launches: the
            # bandwidth fields of a single kernel do not apply to it
            for key in ("kernel_ms", "kernel_ms_isolated_median", "hbm_traffic_bytes", "algorithmic_bytes",
                        "achieved_GBps", "hbm_frac"):
                results[k].pop(key)
            results[k].update({"step_is_many_launches": True, "step_ms": ms})
            if "flops" in info:
                tf = info["flops"] / (ms * 1e-3) / 1e12
                results[k].update({"trailing_update_flops": info["flops"], "trailing_update_TFLOPs_over_step": tf})
                print(f"[bench] {k}: {ms:.2f} ms/step (many launches), trailing updates at {tf:.1f} TFLOP/s over "
                      f"the step", file=sys.stderr, flush=True)
            else:
                gbs = info["bytes"] / (ms * 1e-3) / 1e9
                results[k].update({"algorithmic_bytes": info["bytes"], "step_GBps": gbs,
                                   "step_hbm_frac": gbs / HBM_PEAK_GBS})
                print(f"[bench] {k}: {ms * 1e3:.1f} us/step (many launches), {gbs:.0f} GB/s of algorithmic bytes "
                      f"over the step ({gbs / HBM_PEAK_GBS:.1%} of HBM peak)", file=sys.stderr, flush=True)
        elif info["bound"] == "mfma":
            tf = info["flops"] / (ms * 1e-3) / 1e12
            results[k].update({"algorithmic_flops": info["flops"], "achieved_TFLOPs": tf,
                               "mfma_frac": tf / BF16_PEAK_TFLOPS})
            print(f"[bench] {k}: {ms * 1e3:.1f} us/launch, {tf:.0f} TFLOP/s ({tf / BF16_PEAK_TFLOPS:.1%} of bf16 "
                  f"MFMA peak)", file=sys.stderr, flush=True)
        else:
            warm_txt = ""
            if "kernel_ms_warm" in results[k]:
                warm_txt = (f"; warm MALL {results[k]['kernel_ms_warm'] * 1e3:.1f} us "
                            f"({results[k]['hbm_frac_warm']:.1%})")
            print(f"[bench] {k}: {ms * 1e3:.1f} us/launch, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM peak, "
                  f"{tm['buffer_sets']} buffer sets){warm_txt}", file=sys.stderr, flush=True)
        if "nnz" in info:
            results[k]["nnz"] = info["nnz"]
        if "gathered_bytes" in info:
            results[k]["gathered_bytes"] = info["gathered_bytes"]
            results[k]["gathered_GBps"] = info["gathered_bytes"] / (ms * 1e-3) / 1e9
            results[k]["spmm_TFLOPs"] = info["flops"] / (ms * 1e-3) / 1e12
        if not a.no_cpu and ("cpu" in info or k.startswith("o") or k.startswith("l")):
            results[k]["cpu_oracle"] = cpu_oracle_time(torch, k, info, ms)
            print(f"[bench] {k}: CPU oracle {results[k]['cpu_oracle']['seconds'] * 1e3:.1f} ms "
                  f"({results[k]['cpu_oracle']['sample']})", file=sys.stderr, flush=True)
        if k == HEADLINE:
            info_head = info
        del launches
        info.pop("keep", None)
        torch.cuda.empty_cache()
    head = results[HEADLINE]
    cpu = None
    if not a.no_cpu:
        print("[bench] cpu baseline (C2 sample)", file=sys.stderr, flush=True)
        cpu = cpu_baseline_c2(torch, info_head["cpu_input"])
    out = {
        "metric": "quantized elements/sec",
        "value": head["elements_per_s"],
        "unit": "elements/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": head["region_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE.json configs)",
        "config": {"workload": head["workload"], "block_size": 64, "format": "nf4", "shape": [4096, 11008]},
        "roofline": {"bound": "hbm", "achieved": head["achieved_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["hbm_frac"], "traffic": head["hbm_traffic_bytes"],
                     "kernel": DOMINANT[HEADLINE],
                     "algorithmic_bytes_per_launch": head["algorithmic_bytes"],
                     "kernel_ms_avg": head["kernel_ms"], "mall": "cold",
                     "buffer_sets": head["buffer_sets"], "kernel_ms_warm": head.get("kernel_ms_warm")},
        "cpu_baseline": cpu,
        "configs": results,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
