"""QuantizationSpec / FakeQuantize API of the hot path, and the calibration
consumers: the learned-codebook histogram and GPTQ weight compensation."""

from .fake_quantize import (  # noqa: F401
    FakeQuantizeFunction,
    FusedAmaxObsFakeQuantize,
    MXFakeQuantizeFunction,
    _DerivedObserverOrFakeQuantize,
    get_quantization_map,
)
from .gptq import compensate_weight  # noqa: F401
from .lcq import HISTOGRAM_BINS, Histogram  # noqa: F401
from .qspec import QScheme, parse_spec_fields  # noqa: F401
from .quantizer import DerivedQuantizationSpec, QuantizationSpec, derive_bias_qparams_fn  # noqa: F401
