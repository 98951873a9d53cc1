"""Write the golden 65536-entry format tables from the reference's own leaf code.

Every reference quantizer is a table over all bf16 bit patterns
(``get_quantization_map``, src/voyager_compiler/quantization/fake_quantize.py:30-98),
so a dtype's whole behaviour is one 65536-entry bf16 vector.  This script builds
those vectors by calling the reference's leaf format functions, loaded by file
path from ``/root/reference`` (the package itself does not import here: it
needs torchao/peft/wandb).  It runs only in the build container; the GPU box
never sees the reference.  Output: ``tests/golden/tables.npz`` holding, for
each dtype, the uint16 bit patterns of the table (key ``t_<dtype>``), plus

* ``nf_values_<dtype>``: the NF level vector ``quantize_to_nf`` returns,
* ``log2floor``: int16 ``floor(log2(x))`` evaluated in bf16 the way
  ``_shared_exponents`` does (src/voyager_compiler/quantization/mx_utils.py:43-47),
  for every bf16 pattern (torch's own CPU kernel; no reference code).

The dtype routing below restates ``get_quantization_map``'s regex dispatch
(fake_quantize.py:37-98) with the same arguments it passes.

Usage: python tests/golden/make_golden.py [--ref /root/reference]
"""

import argparse
import importlib.util
import math
import os
import re

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

DTYPES = [
    # posit(n, es)  -> quantize_to_posit(values, n, es, round_to_even=True)
    "posit8_1", "posit8_0", "posit8_2", "posit6_1", "posit16_1",
    # fpN_eXmY      -> _quantize_elemwise_core(values, m+2, e, max_norm, "even", True)
    "fp8_e4m3", "fp8_e5m2", "fp6_e3m2", "fp6_e2m3", "fp4_e2m1",
    "fp8_e5m3", "fp8_e8m0", "fp16_e5m10",
    # NVIDIA-style  -> quantize_to_fp8_e4m3/e5m2(values)
    "e4m3", "e5m2",
    # NormalFloat   -> quantize_to_nf(values, k, int_bits=b) -> (indices, values)
    "nf4", "nf4_6", "nf3",
    # integers      -> clamp(round(values), qmin, qmax)
    "int8", "int4", "uint8", "uint4",
]


def _load(path, name):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--out", default=os.path.join(HERE, "tables.npz"))
    args = ap.parse_args()

    dt = os.path.join(args.ref, "src/voyager_compiler/quantization/dtypes")
    posit = _load(os.path.join(dt, "posit.py"), "_ref_posit")
    fp8 = _load(os.path.join(dt, "fp8.py"), "_ref_fp8")
    nf = _load(os.path.join(dt, "normal_float.py"), "_ref_nf")

    values = torch.arange(2**16, dtype=torch.int16).view(torch.bfloat16)
    out = {}
    for dtype in DTYPES:
        if m := re.fullmatch(r"posit(\d+)_(\d+)", dtype):
            t = posit.quantize_to_posit(values, int(m.group(1)), int(m.group(2)),
                                        round_to_even=True)
        elif m := re.fullmatch(r"fp(\d+)_e(\d+)m(\d+)", dtype):
            nbits, ebits, mbits = map(int, m.groups())
            v = values
            if nbits == ebits + mbits:
                v = torch.abs(values)
            mbits = mbits + 2
            emax = 2 ** (ebits - 1) - 1 if ebits > 4 else 2 ** (ebits - 1)
            if dtype != "fp8_e4m3":
                max_norm = 2**emax * float(2 ** (mbits - 1) - 1) / 2 ** (mbits - 2)
            else:
                max_norm = 2**emax * 1.75
            t = fp8._quantize_elemwise_core(v, mbits, ebits, max_norm,
                                            round="even", saturate_normals=True)
        elif dtype in ("e4m3", "e5m2"):
            fn = fp8.quantize_to_fp8_e4m3 if dtype == "e4m3" else fp8.quantize_to_fp8_e5m2
            t = fn(values)
        elif m := re.fullmatch(r"nf(\d+)(?:_(\d+))?", dtype):
            k = int(m.group(1))
            ib = int(m.group(2)) if m.group(2) else None
            idx, lv = nf.quantize_to_nf(values, k, int_bits=ib)
            out[f"nf_index_{dtype}"] = idx.to(torch.uint8).numpy()
            out[f"nf_values_{dtype}"] = lv.view(torch.int16).numpy().view(np.uint16)
            t = lv[idx]
        elif m := re.fullmatch(r"(u?)int(\d+)", dtype):
            nbits = int(m.group(2))
            if m.group(1):
                lo, hi = 0, 2**nbits - 1
            else:
                lo, hi = -(2 ** (nbits - 1)), 2 ** (nbits - 1) - 1
            t = torch.clamp(torch.round(values), lo, hi)
        else:
            raise ValueError(dtype)
        assert t.dtype == torch.bfloat16 and t.numel() == 2**16, dtype
        out[f"t_{dtype}"] = t.view(torch.int16).numpy().view(np.uint16).copy()

    # floor(log2(a + 2^-126 [a == 0])) in bf16, as _shared_exponents computes it
    a = values.abs()
    fmn = 2.0 ** -126
    le = torch.floor(torch.log2(a + fmn * (a == 0).to(a.dtype)))
    le = le.float()
    le = torch.where(torch.isfinite(le), le, torch.full_like(le, -32768.0))
    out["log2floor"] = le.to(torch.int16).numpy()

    out["torch_version"] = np.frombuffer(torch.__version__.encode(), dtype=np.uint8)
    np.savez_compressed(args.out, **out)
    print("wrote", args.out, len(out), "arrays",
          os.path.getsize(args.out), "bytes")


if __name__ == "__main__":
    main()
