"""QuantizationSpec (src/voyager_compiler/quantization/quantizer/quantizer.py:18-55)."""

from dataclasses import dataclass
from typing import List, Optional, Union

from torch.ao.quantization.quantizer import QuantizationSpecBase

from .fake_quantize import FusedAmaxObsFakeQuantize
from .qspec import QScheme, parse_spec_fields

__all__ = ["QuantizationSpec"]


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
