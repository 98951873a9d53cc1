"""GPU parity at the benchmark's full shapes, on bench.py's own inputs (the
same generators and seeds) through the same launches the benchmark times:
C1 posit8_1 fake-quant + codes (fp32 4096x4096), C2 NF4 block-64 encode and
decode (bf16 4096x11008), C3 MX block-32 e4m3 / e3m2 / e2m1 packed codes +
E8M0 scales and the e4m3 fake-quant (bf16 8192x8192), C4 per-channel
codebook encode (K = 16, 256) and decode (fp32 4096x4096).  Every output is
compared bit for bit with the CPU oracle."""

import numpy as np
import pytest
import torch

import bench
from oracle import formats as F
from oracle import reference_ops as R
from tests.conftest import assert_bitexact
from tests.test_gpu_mx import ocp_code, unpack


def assert_codes_equal(got, want, x, what):
    """Integer codes equal; on a mismatch, name the count and the first
    differing elements with their inputs."""
    if np.array_equal(got, want):
        return
    bad = np.nonzero(got != want)[0]
    xs = x.reshape(-1)
    first = ", ".join(f"[{i}] got {got[i]:#x} want {want[i]:#x} x={float(xs[i])!r}" for i in bad[:8])
    raise AssertionError(f"{what}: {bad.size} of {got.size} codes differ; {first}")


def run_config(vqx, key):
    print(f"bench shape {key}: setup", flush=True)
    # one buffer set: the bench's cold-MALL rotation copies are for timing only
    saved = bench.ROTATE_BYTES, bench.MIN_SETS
    bench.ROTATE_BYTES, bench.MIN_SETS = 0, 1
    try:
        launches, info = bench.CONFIGS[key](vqx, torch, vqx._lib)
    finally:
        bench.ROTATE_BYTES, bench.MIN_SETS = saved
    assert len(launches) == 1 and launches[0]() == 0
    torch.cuda.synchronize()
    print(f"bench shape {key}: launched, checking against the oracle", flush=True)
    return info["check"]


@pytest.mark.gpu
def test_c1_full_shape(vqx):
    c = run_config(vqx, "c1")
    h = F.f32_to_bf16(c["x"].numpy())
    want = F.bf16_to_f32(F.posit_table(8, 1)[h])
    assert_bitexact(c["out"].cpu(), torch.from_numpy(want), "C1 posit8_1 fake-quant")
    want_codes = (F.posit_codes(h, 8, 1) & 0xFF).astype(np.uint8)
    assert np.array_equal(c["codes"].cpu().numpy(), want_codes)


def c2_oracle(x):
    ws = R.calculate_mx_qparam(x, [-1], 64, 1.0, False)
    idx_q = torch.from_numpy(F.nf_index_table(F.nf_levels(4)).astype(np.float32)).to(torch.bfloat16)
    return ws, R.quantize(x, ws, None, [-1], 64, idx_q)


@pytest.mark.gpu
def test_c2_encode_full_shape(vqx):
    c = run_config(vqx, "c2")
    ws, wq = c2_oracle(c["x"])
    assert_bitexact(c["scale"].cpu(), ws.float(), "C2 scales")
    got = unpack(c["codes"], 4, c["x"].numel())
    assert_codes_equal(got, wq.float().reshape(-1).numpy().astype(np.int64), c["x"], "C2 codes")


@pytest.mark.gpu
def test_c2_decode_full_shape(vqx):
    c = run_config(vqx, "c2_decode")
    ws, wq = c2_oracle(c["x"])
    want = R.table_tensor(F.nf_levels(4))[wq.long()] * R.expand(ws, c["x"].shape, 64)
    assert_bitexact(c["out"].cpu(), want, "C2 decode")


@pytest.mark.gpu
@pytest.mark.parametrize("key,dtype,qmax", [("c3_e4m3", "fp8_e4m3", 448.0), ("c3_e3m2", "fp6_e3m2", 28.0),
                                            ("c3_e2m1", "fp4_e2m1", 6.0)])
def test_c3_full_shape(vqx, key, dtype, qmax):
    c = run_config(vqx, key)
    ws, wq = R.quantize_mx(c["x"], R.table_tensor(F.quantization_table(dtype)), [-1], 32, qmax, True)
    want_e8 = ((ws.float().view(torch.int32) >> 23) & 0xFF).to(torch.uint8)
    assert torch.equal(c["scale"].cpu(), want_e8), f"{key} E8M0 scales"
    eb, mb, _, _ = F.fp_core_params(dtype)
    got = unpack(c["codes"], eb + mb + 1, c["x"].numel())
    # the generator's inverse-CDF Laplace draw gives -inf where rand() hits
    # 0 exactly (twice at this size): the reference then fake-quantizes
    # -inf / inf = NaN in that block, a value the element formats encode as
    # the all-ones magnitude with the input element's sign (the reference's
    # value is NaN whatever its sign; the code's sign is this library's rule)
    v = wq.float().reshape(-1).numpy()
    nan = np.isnan(v)
    assert nan.sum() >= 2, "the C3 input holds the two infinities this check covers"
    want = ocp_code(np.where(nan, 0.0, v), eb, mb)
    mag = (1 << (eb + mb)) - 1
    xsign = (c["x"].reshape(-1).view(torch.int16).numpy() < 0).astype(np.int64)
    want[nan] = (xsign[nan] << (eb + mb)) | mag
    assert_codes_equal(got, want, c["x"], f"{key} codes")


@pytest.mark.gpu
def test_c3_fake_quant_full_shape(vqx):
    c = run_config(vqx, "c3_e4m3_fq")
    ws, wy = R.mx_fake_quantize(c["x"], R.table_tensor(F.quantization_table("fp8_e4m3")), [-1], 32, 448.0, True)
    assert_bitexact(c["scale"].cpu(), ws, "C3 fake-quant scales")
    assert_bitexact(c["out"].cpu(), wy, "C3 fake-quant values")


@pytest.mark.gpu
@pytest.mark.parametrize("key", ["c4_k16", "c4_k256", "c4_k16_decode"])
def test_c4_full_shape(vqx, key):
    c = run_config(vqx, key)
    want = R.codebook_encode_rows(c["x"], c["codebooks"])
    assert torch.equal(c["codes"].cpu().long(), want), f"{key} codes"
    if "out" in c:
        assert torch.equal(c["out"].cpu(), R.codebook_decode_rows(want, c["codebooks"])), f"{key} decode"
