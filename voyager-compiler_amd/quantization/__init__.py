"""QuantizationSpec / FakeQuantize API of the hot path."""

from .fake_quantize import (  # noqa: F401
    FakeQuantizeFunction,
    FusedAmaxObsFakeQuantize,
    MXFakeQuantizeFunction,
    get_quantization_map,
)
from .qspec import QScheme, parse_spec_fields  # noqa: F401
from .quantizer import QuantizationSpec  # noqa: F401
