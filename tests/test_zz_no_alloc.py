"""GPU: the allocation-free NF4 linear (vqx_nf4_linear_noalloc, its workspace
a device array of the library) against the same product with a caller-owned
workspace (vqx_nf4_linear_ws), through the C ABI: bit-identical, since both
run the same stream-K plan.  Two calls in a row, the second on a smaller
input, so the second reuses the array with the first call's contents."""

import ctypes

import pytest
import torch

Q = torch.ops.quantized_ops


def operands(vqx, M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    W = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).cuda()
    sc, codes = Q.quantize_mx_packed(W, "nf4", -1, 64, False, 1.0, "float32")
    bias = torch.randn(N, generator=g).to(torch.bfloat16).cuda()
    return A, codes, sc, bias


def with_workspace(vqx, A, codes, sc, lv, bias, N):
    L = vqx._lib
    M, K = A.shape
    n = ctypes.c_int64(0)
    L.call("vqx_nf4_linear_workspace_size", M, N, K, ctypes.byref(n))
    ws = torch.empty(max(n.value, 1), dtype=torch.uint8, device=A.device)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    L.call("vqx_nf4_linear_ws", L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), L.ptr(bias), L.ptr(out), M, N, K,
           L.ptr(ws) if n.value else None, n.value, L.stream_of(A))
    return out, n.value


def no_alloc(vqx, A, codes, sc, lv, bias, N):
    L = vqx._lib
    M, K = A.shape
    out = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    L.call("vqx_nf4_linear_noalloc", L.ptr(A), L.ptr(codes), L.ptr(sc), L.ptr(lv), L.ptr(bias), L.ptr(out), M, N, K,
           L.stream_of(A))
    return out


@pytest.mark.gpu
def test_no_alloc_matches_workspace_entry_point(vqx):
    lv = vqx.parse_format("nf4").tables(torch.device("cuda"))["levels_bf16"]
    # first: 86 tiles, all split along K (the array's counters and slots in
    # use); second: smaller, 32 tiles, split too; third: whole tiles only
    for i, (M, N, K) in enumerate([(256, 11008, 4096), (256, 4096, 4096), (2048, 1024, 1024)]):
        print(f"no-alloc NF4 linear call {i}: M={M} N={N} K={K}", flush=True)
        A, codes, sc, bias = operands(vqx, M, N, K, 100 + i)
        want, ws_bytes = with_workspace(vqx, A, codes, sc, lv, bias, N)
        assert (ws_bytes > 0) == (i < 2), ws_bytes
        got = no_alloc(vqx, A, codes, sc, lv, bias, N)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: {int((got != want).sum())} outputs differ"
        # once more on the same array: identical
        assert torch.equal(no_alloc(vqx, A, codes, sc, lv, bias, N), want)
