"""ctypes binding of libvqx.so (the C ABI declared in include/vqx.h).

Loading fails loudly: there is no CPU fallback for any kernel.  Every call
checks the status and raises ``ValueError`` (bad argument) or
``RuntimeError`` (HIP failure) with the library's message.
"""

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("VQX_LIB", os.path.join(HERE, "libvqx.so"))

F32, BF16, F16, U8 = 0, 1, 2, 3
FMT_IDENTITY, FMT_FP16, FMT_INT, FMT_FP, FMT_NV_FP8, FMT_POSIT, FMT_LEVELS, FMT_TABLE = range(8)
FLAG_UNSIGNED = 1

_DTYPE_TAG = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.uint8: U8}


class VqxFormat(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("p0", ctypes.c_int32),
        ("p1", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("max_norm", ctypes.c_float),
        ("code_bits", ctypes.c_int32),
        ("boundaries", ctypes.c_void_p),
        ("levels", ctypes.c_void_p),
        ("code_table", ctypes.c_void_p),
        ("value_table", ctypes.c_void_p),
        ("lut", ctypes.c_void_p),
        ("lut_len", ctypes.c_int32),
    ]


class VqxScaleMap(ctypes.Structure):
    _fields_ = [
        ("scale", ctypes.c_void_p),
        ("zero_point", ctypes.c_void_p),
        ("L", ctypes.c_int64),
        ("inner", ctypes.c_int64),
        ("block", ctypes.c_int64),
        ("s_o", ctypes.c_int64),
        ("s_l", ctypes.c_int64),
        ("s_in", ctypes.c_int64),
    ]


class VqxMxOperand(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("code", ctypes.c_void_p),
        ("batch_stride", ctypes.c_int64),
        ("ld", ctypes.c_int64),
        ("scale_batch_stride", ctypes.c_int64),
        ("scale_ld", ctypes.c_int64),
        ("k_major", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("code_len", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float

_SIGNATURES = {
    "vqx_version": ([], ctypes.c_char_p),
    "vqx_last_error": ([], ctypes.c_char_p),
    "vqx_device_cus": ([], ctypes.c_int),
    "vqx_vmap": ([_P, _I32, _I64, _P, _P, _P], ctypes.c_int),
    "vqx_fake_quant": ([_P, _I32, _I64, ctypes.POINTER(VqxFormat), _P, _I64, _I64, _I32, _P, _P,
                        _I32, _P], ctypes.c_int),
    "vqx_amax_observe_fake_quant": ([_P, _I32, _I64, _I64, _I64, ctypes.POINTER(VqxFormat), _P, _I32, _P, _F, _I32,
                                     _P, _P], ctypes.c_int),
    "vqx_quantize_mapped": ([_P, _I32, _I64, ctypes.POINTER(VqxFormat), ctypes.POINTER(VqxScaleMap),
                             _I32, _P, _P, _I32, _P], ctypes.c_int),
    "vqx_dequantize_mapped": ([_P, _I32, _I64, _P, ctypes.POINTER(VqxScaleMap), _P, _P, _P],
                              ctypes.c_int),
    "vqx_build_table": ([ctypes.POINTER(VqxFormat), _P, _P, _P], ctypes.c_int),
    "vqx_lut_bytes": ([], ctypes.c_int64),
    "vqx_build_lut": ([ctypes.POINTER(VqxFormat), _P, _P], ctypes.c_int),
    "vqx_level_tables": ([_P, _I32, _I32, _P, _P, _P, _P, _P], ctypes.c_int),
    "vqx_mx_quantize": ([_P, _I32, _I64, _I64, _I64, _I64, ctypes.POINTER(VqxFormat), _I32, _I32,
                         _F, _P, _P, _P, _P, _P, _P, _P, _I32, _P], ctypes.c_int),
    "vqx_mx_decode": ([_P, _I32, _P, _I32, _P, _I32, _I64, _I64, _P, _I32, _P], ctypes.c_int),
    "vqx_outlier_topk_workspace_size": ([ctypes.POINTER(_I64)], ctypes.c_int),
    "vqx_outlier_topk_threshold": ([_P, _I32, _I64, _I64, _I32, _F, _F, _P, _P, _I64, _P], ctypes.c_int),
    "vqx_mx_fake_quant_outlier": ([_P, _I32, _I64, _I64, _I64, _I64, ctypes.POINTER(VqxFormat), _I32, _I32, _F, _P,
                                   _P, _F, _P, _I32, _P, _P, _P, _P], ctypes.c_int),
    "vqx_outlier_stats_size": ([ctypes.POINTER(_I64)], ctypes.c_int),
    "vqx_outlier_mask": ([_P, _I32, _I64, _P, _F, _P, _I32, _P, _P], ctypes.c_int),
    "vqx_outlier_restore": ([_P, _I32, _I64, _P, _F, _P, _P], ctypes.c_int),
    "vqx_decode_table": ([ctypes.POINTER(VqxFormat), _P, _I32, _P], ctypes.c_int),
    "vqx_gwa_fake_quant": ([_P, _I32, _I64, _I64, _I64, _I64, _F, _F, _P, _P, _P, _P, _P], ctypes.c_int),
    "vqx_codebook_encode": ([_P, _I32, _I64, _I64, _P, _I32, _P, _P], ctypes.c_int),
    "vqx_codebook_decode": ([_P, _I64, _I64, _P, _I32, _P, _I32, _P], ctypes.c_int),
    "vqx_nf4_linear": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P], ctypes.c_int),
    "vqx_nf4_linear_workspace_size": ([_I64, _I64, _I64, ctypes.POINTER(_I64)], ctypes.c_int),
    "vqx_nf4_linear_ws": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _P], ctypes.c_int),
    "vqx_mx_matmul": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P], ctypes.c_int),
    "vqx_mx_operand_decode": ([_P, _I64, _I64, _I64, _P, _P], ctypes.c_int),
    "vqx_nf4_linear_noalloc": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P], ctypes.c_int),
    "vqx_nf4_pack_weight": ([_P, _I32, _P, _I32, _I64, _I64, _I32, _I32, _P, _P, _P, _P], ctypes.c_int),
    "vqx_filter_outlier": ([_P, _I32, _I64, _I64, _I64, _F, _I64, _I32, _P, _P, _P, _P, _P], ctypes.c_int),
    "vqx_outlier_workspace_size": ([_I32, _I64, _I64, _I64, _I64, ctypes.POINTER(_I64)], ctypes.c_int),
    "vqx_filter_outlier_ws": ([_P, _I32, _I64, _I64, _I64, _F, _I64, _I32, _P, _P, _P, _P, _P, _I64, _P],
                              ctypes.c_int),
    "vqx_quantize_mx_outlier_ws": ([_P, _I64, _I64, _I64, ctypes.c_float, _I64, _I32, _I64, _I32, _I32,
                                    ctypes.c_float, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P], ctypes.c_int),
    "vqx_slice_csr": ([_P, _I32, _P, _P, _I64, _I64, _I32, _I64, _I64, _I64, _P, _P, _P, _P], ctypes.c_int),
    "vqx_csr_decode_weight": ([_P, _I32, _I64, _I64, _I64, _I32, _P, _I32, _I64, _P, _I32, _I64, _I64, _I64,
                               _I64, _I64, _P, _I32, _P], ctypes.c_int),
    "vqx_spmm_csr": ([_P, _I32, _P, _P, _I64, _I64, _I64, _P, _I32, _I64, _I64, _I64, _P, _P, _P], ctypes.c_int),
    "vqx_lcq_histogram": ([_P, _I32, _I64, _I64, _F, _P, _I64, _P, _I32, _P, _P, _P, _P], ctypes.c_int),
    "vqx_quantize_mx_outlier": ([_P, _I64, _I64, _I64, ctypes.c_float, _I64, _I32, _I64, _I32, _I32, ctypes.c_float,
                                 _P, _P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "vqx_gptq_block": ([_P, _I64, _I64, _I64, _I32, _P, ctypes.c_float, _P, _P, _I64, _P, _P, _P, _I64, _P],
                       ctypes.c_int),
    "vqx_chol_inverse_block": ([_P, _I64, _I32, _P, _I64, _P, _P], ctypes.c_int),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load libvqx.so once; raises ImportError if it is missing or broken."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"vqx: {LIB_PATH} is not built; run __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950). There is no CPU fallback.")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def _check(rc, what):
    if rc == 0:
        return
    msg = load().vqx_last_error().decode(errors="replace")
    if rc == -1:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


_FNS = {}


def call(name, *args):
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        _check(rc, name)


def ptr(t):
    """Device pointer of a tensor (None -> NULL), as the int ctypes passes
    for a void* argument."""
    if t is None:
        return None
    return t.data_ptr()


def dtype_tag(dt):
    try:
        return _DTYPE_TAG[dt]
    except KeyError:
        raise ValueError(f"vqx: dtype {dt} not supported") from None


def stream_of(t):
    """The current torch stream of t's device, as a hipStream_t (the raw
    handle, without building a torch Stream object on every call)."""
    idx = t.device.index
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device() if idx is None else idx)


def require_device(t, what):
    if not t.is_cuda:
        raise RuntimeError(
            f"vqx: {what} runs on the MI355X only (got a {t.device} tensor); there is no CPU path")


INFERENCE = "inference"


def version_of(t):
    """t's version counter, the key the host-side caches use to notice an
    in-place write.  Tensors made under torch.inference_mode carry no
    counter (reading it raises); they give INFERENCE instead, so a cache
    keyed on them relies on their storage (data_ptr) alone."""
    return INFERENCE if t.is_inference() else t._version
