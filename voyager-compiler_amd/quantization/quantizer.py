"""QuantizationSpec and DerivedQuantizationSpec
(src/voyager_compiler/quantization/quantizer/quantizer.py:18-71), with the
bias derivation of quantize_pt2e.py:163-175."""

from dataclasses import dataclass
from typing import Any, Callable, List, Optional, Union

from torch.ao.quantization.quantizer import QuantizationSpecBase

from .fake_quantize import FusedAmaxObsFakeQuantize, _DerivedObserverOrFakeQuantize
from .qspec import QScheme, parse_spec_fields

__all__ = ["QuantizationSpec", "DerivedQuantizationSpec", "derive_bias_qparams_fn"]


@dataclass(eq=True)
class QuantizationSpec(QuantizationSpecBase):
    """How to quantize one tensor: dtype string, qscheme, range, block layout."""

    dtype: str
    observer_or_fake_quant_ctr: type = FusedAmaxObsFakeQuantize
    quant_min: Optional[float] = None
    quant_max: Optional[float] = None
    qscheme: Optional[QScheme] = None
    amax_history_len: Optional[int] = None
    ch_axis: Optional[Union[int, List[int]]] = None
    block_size: Optional[Union[int, List[int]]] = None
    scale_dtype: Optional[str] = None
    outlier_threshold: Optional[float] = None
    outlier_pct: Optional[float] = None
    is_dynamic: bool = False

    @staticmethod
    def from_str(s):
        """Build a spec from a comma-separated spec string."""
        return QuantizationSpec(**parse_spec_fields(s))

    def __post_init__(self):
        if self.qscheme is not None and self.quant_max is None:
            raise ValueError("quant_max is required for quantization.")
        if self.qscheme in (QScheme.MICROSCALING, QScheme.GROUP_WISE_AFFINE) and self.block_size is None:
            raise ValueError("block_size is required for microscaling.")

    def make_fake_quantize(self, device=None):
        """The FakeQuantize module this spec configures."""
        return self.observer_or_fake_quant_ctr(
            dtype=self.dtype, qscheme=self.qscheme, quant_min=self.quant_min,
            quant_max=self.quant_max, amax_history_len=self.amax_history_len,
            ch_axis=self.ch_axis, block_size=self.block_size, scale_dtype=self.scale_dtype,
            outlier_threshold=self.outlier_threshold, outlier_pct=self.outlier_pct, device=device)


@dataclass(eq=True)
class DerivedQuantizationSpec(QuantizationSpecBase):
    """A tensor whose quantization parameters come from other tensors'
    observers (a bias: input scale x weight scale).  derived_from names those
    tensors (graph edges or nodes); derive_qparams_fn maps their observers
    to the scale."""

    derived_from: List[Any]
    derive_qparams_fn: Callable
    dtype: str
    quant_min: Optional[int] = None
    quant_max: Optional[int] = None
    qscheme: Optional[QScheme] = None

    def make_fake_quantize(self, obs_or_fq_map):
        """The fake-quantizer of this spec, given the observers of the tensors
        it derives from (keyed as in derived_from), as convert_pt2e builds it
        (quantize_pt2e.py:60-68)."""
        obs_or_fqs = [obs_or_fq_map[k] for k in self.derived_from]
        return _DerivedObserverOrFakeQuantize(self.dtype, obs_or_fqs, self.derive_qparams_fn)


def derive_bias_qparams_fn(obs_or_fqs):
    """The bias scale of a quantized GEMM: the activation's scale times the
    weight's (per-channel weight scales flattened to one per output channel)."""
    assert len(obs_or_fqs) == 2, (
        "Expecting two obs/fqs, one for activation and one for weight, got: {}".format(len(obs_or_fqs)))
    act_scale = obs_or_fqs[0].calculate_qparams()
    weight_scale = obs_or_fqs[1].calculate_qparams()
    return act_scale * weight_scale.flatten()
