"""Element formats: dtype strings -> kernel format descriptors and device tables.

``parse_format`` routes a dtype string exactly as the reference's
``get_quantization_map`` does (src/voyager_compiler/quantization/
fake_quantize.py:37-98); ``get_quantization_map`` returns the same 65536-entry
bf16 table (or ``(indices, values)`` for NormalFloat), computed on the GPU by
the closed-form encoders instead of by a table-building torch program.

Device tables (value table, code table, NF/codebook index tables, decode
table) are built once per (format, device) and cached.
"""

import math
import re
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from . import _lib

__all__ = [
    "Format",
    "parse_format",
    "codebook_format",
    "get_quantization_map",
    "create_normal_map",
    "quant_range",
]


def create_normal_map(offset=0.9677083, use_extra_value=True, k=4):
    """NormalFloat levels, sorted and scaled to max 1 (normal_float.py:4-29).

    Half the levels are standard-normal quantiles of an evenly spaced grid
    from ``offset`` to 0.5 (one extra on the positive side when
    ``use_extra_value``), mirrored, plus zero.  Host-side constants (scipy),
    as in the reference.
    """
    from scipy.stats import norm

    n = 2 ** (k - 1)
    pos = norm.ppf(torch.linspace(offset, 0.5, n + 1 if use_extra_value else n)[:-1].numpy())
    neg = -norm.ppf(torch.linspace(offset, 0.5, n)[:-1].numpy())
    mid = [0.0] if use_extra_value else [0.0, 0.0]
    vals = torch.tensor(list(pos) + mid + list(neg), dtype=torch.float32).sort().values
    vals = vals / vals.max()
    assert vals.numel() == 2**k
    return vals


def quant_range(dtype: str):
    """(quant_min, quant_max) a qscheme implies for a dtype (qspec.py:64-105)."""
    if m := re.fullmatch(r"int(\d+)", dtype, re.IGNORECASE):
        n = int(m.group(1))
        return -(2 ** (n - 1)), 2 ** (n - 1) - 1
    if m := re.fullmatch(r"uint(\d+)", dtype, re.IGNORECASE):
        return 0, 2 ** int(m.group(1)) - 1
    if m := re.fullmatch(r"fp(\d+)_e(\d+)m(\d+)", dtype, re.IGNORECASE):
        e, mb = int(m.group(2)), int(m.group(3)) + 2
        emax = 2 ** (e - 1) - 1 if e > 4 else 2 ** (e - 1)
        if dtype.lower() == "fp8_e4m3":
            mx = 2**emax * 1.75
        else:
            mx = 2**emax * (2 ** (mb - 1) - 1) / 2 ** (mb - 2)
        return -mx, mx
    if m := re.fullmatch(r"posit(\d+)_(\d+)", dtype, re.IGNORECASE):
        n, es = int(m.group(1)), int(m.group(2))
        mx = (2 ** (2**es)) ** (n - 2)
        return -mx, mx
    if m := re.fullmatch(r"nf(\d+)(?:_(\d+))?", dtype, re.IGNORECASE):
        mx = 2 ** (int(m.group(2)) - 1) - 1 if m.group(2) is not None else 1
        return -mx, mx
    raise ValueError(f"Unsupported dtype: {dtype}")


def _code_bits(n):
    return 4 if n <= 4 else 6 if n <= 6 else 8 if n <= 8 else 16


@dataclass
class Format:
    """A parsed dtype string.  ``kind``/``p0``/``p1``/``flags``/``max_norm``
    follow ``vqx_format`` in include/vqx.h."""

    dtype: str
    kind: int
    p0: int = 0
    p1: int = 0
    flags: int = 0
    max_norm: float = 0.0
    code_bits: int = 16
    # level sets (NormalFloat: bf16 arithmetic; codebook: fp32 arithmetic)
    levels: Optional[torch.Tensor] = None
    level_mode: int = 0
    _dev: dict = field(default_factory=dict, repr=False)

    @property
    def is_levels(self):
        return self.kind == _lib.FMT_LEVELS

    @property
    def nlevels(self):
        return 0 if self.levels is None else self.levels.numel()

    # -- device tables ------------------------------------------------------
    def tables(self, device):
        """Device tables for this format on ``device`` (built once)."""
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError(f"vqx: format tables live on the GPU, not {device}")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        key = str(device)
        if key in self._dev:
            return self._dev[key]
        t = {}
        with torch.cuda.device(device):
            st = torch.cuda.current_stream(device)
            sptr = _lib.ctypes.c_void_p(st.cuda_stream)
            if self.is_levels:
                lv = self.levels.to(device=device, dtype=torch.float32).contiguous()
                K = lv.numel()
                idx = torch.empty(65536, dtype=torch.uint8, device=device)
                bnd = torch.empty(max(K - 1, 1), dtype=torch.float32, device=device)
                work = torch.empty(max(K, 1), dtype=torch.int32, device=device)
                bad = torch.zeros(1, dtype=torch.int32, device=device)
                _lib.call("vqx_level_tables", _lib.ptr(lv), K, self.level_mode, _lib.ptr(idx),
                          _lib.ptr(bnd), _lib.ptr(work), _lib.ptr(bad), sptr)
                t["levels_f32"] = lv
                t["levels_bf16"] = lv.to(torch.bfloat16).contiguous()
                t["index_table"] = idx
                t["boundaries"] = bnd
                t["monotone"] = int(bad.item()) == 0
            desc = self._desc_from(t)
            t["desc_closed"] = desc
            if self.code_bits <= 8:
                # compact code/value table for the streaming kernels
                blob = torch.empty(int(_lib.load().vqx_lut_bytes()) // 4, dtype=torch.int32, device=device)
                _lib.call("vqx_build_lut", _lib.ctypes.byref(desc), _lib.ptr(blob), sptr)
                hdr = blob[:16].cpu()
                if int(hdr[0]) == 1:
                    t["lut"] = blob
                    t["lut_len"] = int(hdr[4])
                    desc = self._desc_from(t)
            vals = torch.empty(65536, dtype=torch.bfloat16, device=device)
            codes = torch.empty(65536, dtype=torch.int16, device=device)
            _lib.call("vqx_build_table", _lib.ctypes.byref(desc), _lib.ptr(vals), _lib.ptr(codes), sptr)
            ntab = 1 << min(self.code_bits, 16)
            dtab = torch.zeros(ntab, dtype=torch.bfloat16, device=device)
            if self.code_bits <= 8:
                _lib.call("vqx_decode_table", _lib.ctypes.byref(desc), _lib.ptr(dtab), ntab, sptr)
            t["values"] = vals
            t["codes"] = codes
            t["decode"] = dtab
            t["desc"] = desc
        self._dev[key] = t
        return t

    def _desc_from(self, t):
        d = _lib.VqxFormat()
        d.kind, d.p0, d.p1, d.flags = self.kind, self.p0, self.p1, self.flags
        d.max_norm, d.code_bits = float(self.max_norm), self.code_bits
        if self.is_levels:
            d.boundaries = t["boundaries"].data_ptr()
            d.levels = t["levels_bf16"].data_ptr()
            d.code_table = t["index_table"].data_ptr()
        if "lut" in t:
            d.lut = t["lut"].data_ptr()
            d.lut_len = t["lut_len"]
        return d

    def desc(self, device, lut=True):
        """ctypes ``vqx_format`` for kernels on ``device``; ``lut=False`` gives
        the closed-form-only descriptor (the table path's cross-check)."""
        t = self.tables(device)
        return t["desc"] if lut else t["desc_closed"]


_CACHE = {}


def parse_format(dtype: str) -> Format:
    """Route a dtype string to a format (fake_quantize.py:37-98)."""
    if dtype in _CACHE:
        return _CACHE[dtype]
    f = _parse(dtype)
    _CACHE[dtype] = f
    return f


def _parse(dtype):
    if dtype in ("float32", "bfloat16"):
        return Format(dtype, _lib.FMT_IDENTITY, code_bits=16)
    if dtype == "float16":
        return Format(dtype, _lib.FMT_FP16, code_bits=16)
    if m := re.fullmatch(r"int(\d+)", dtype, re.IGNORECASE):
        n = int(m.group(1))
        return Format(dtype, _lib.FMT_INT, n, 1, code_bits=_code_bits(n))
    if m := re.fullmatch(r"uint(\d+)", dtype, re.IGNORECASE):
        n = int(m.group(1))
        return Format(dtype, _lib.FMT_INT, n, 0, code_bits=_code_bits(n))
    if m := re.fullmatch(r"(?:fp8\.)?(e4m3|e5m2)", dtype, re.IGNORECASE):
        return Format(dtype, _lib.FMT_NV_FP8, 4 if m.group(1).lower() == "e4m3" else 5, code_bits=8)
    if m := re.fullmatch(r"fp(\d+)_e(\d+)m(\d+)", dtype):
        nbits, ebits, mbits = map(int, m.groups())
        if not (nbits == ebits + mbits + 1 or nbits == ebits + mbits):
            raise AssertionError(f"{dtype}: N must be E + M + 1 (signed) or E + M (unsigned)")
        emax = 2 ** (ebits - 1) - 1 if ebits > 4 else 2 ** (ebits - 1)
        if dtype != "fp8_e4m3":
            max_norm = 2**emax * float(2 ** (mbits + 1) - 1) / 2**mbits
        else:
            max_norm = 2**emax * 1.75
        flags = _lib.FLAG_UNSIGNED if nbits == ebits + mbits else 0
        return Format(dtype, _lib.FMT_FP, ebits, mbits, flags, max_norm, _code_bits(nbits))
    if m := re.fullmatch(r"posit(\d+)_(\d+)", dtype):
        n, es = int(m.group(1)), int(m.group(2))
        return Format(dtype, _lib.FMT_POSIT, n, es, code_bits=_code_bits(n))
    if m := re.fullmatch(r"nf(\d+)(?:_(\d+))?", dtype):
        k = int(m.group(1))
        lv = create_normal_map(k=k)
        if m.group(2):
            lv = torch.round(lv * (2 ** (int(m.group(2)) - 1) - 1))
        lv = lv.to(torch.bfloat16).float()
        return Format(dtype, _lib.FMT_LEVELS, code_bits=_code_bits(max(1, math.ceil(math.log2(lv.numel())))),
                      levels=lv, level_mode=0)
    raise ValueError(f"Unsupported dtype: {dtype}")


def codebook_format(entries: Sequence[float], name: str = "codebook") -> Format:
    """A per-tensor codebook as a level format (lcq.py:270-291): nearest entry
    under fp32 distance, lowest index on ties."""
    lv = torch.as_tensor(entries, dtype=torch.float32).flatten().cpu()
    K = lv.numel()
    if not 1 <= K <= 256:
        raise ValueError(f"codebook must have 1..256 entries, got {K}")
    return Format(name, _lib.FMT_LEVELS, code_bits=_code_bits(max(1, math.ceil(math.log2(K)))),
                  levels=lv, level_mode=1)


def _resolve_device(device):
    if device is None or torch.device(device).type != "cuda":
        if not torch.cuda.is_available():
            raise RuntimeError("vqx: get_quantization_map builds tables on the GPU; no GPU is available")
        return torch.device("cuda", torch.cuda.current_device()), device
    return torch.device(device), device


def get_quantization_map(dtype, device=None):
    """The 65536-entry bf16 table of a dtype (fake_quantize.py:30-98).

    ``None`` gives every bf16 pattern itself.  ``nf*`` dtypes return
    ``(indices, values)`` like the reference.  Tables are computed on the GPU
    and moved to ``device`` when that is not a GPU.
    """
    gdev, want = _resolve_device(device)
    if dtype is None:
        t = torch.arange(2**16, dtype=torch.int32, device=gdev).to(torch.int16).view(torch.bfloat16)
        return t if want is None or torch.device(want).type == "cuda" else t.to(want)
    f = parse_format(dtype)
    tb = f.tables(gdev)
    move = (lambda x: x) if (want is not None and torch.device(want).type == "cuda") else \
        (lambda x: x.to(want if want is not None else "cpu"))
    if f.is_levels:
        return move(tb["index_table"].to(torch.int64)), move(tb["levels_bf16"].clone())
    return move(tb["values"].clone())
