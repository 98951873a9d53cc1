"""voyager-compiler_amd: the Voyager quantization hot path on MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (``include/vqx.h``, ``libvqx.so``),
registered as the ``quantized_ops`` torch library with the reference's schemas,
plus the QuantizationSpec / FakeQuantize API that drives them.

This directory is loaded under the importable name ``voyager_compiler_amd``
(see ``load_package`` in ``__graft_entry__.py``).
"""

__version__ = "0.1.0"

from . import _lib  # noqa: F401,E402
from . import formats  # noqa: F401,E402
from . import ops  # noqa: F401,E402  (registers torch.ops.quantized_ops)
from .formats import codebook_format, get_quantization_map, parse_format  # noqa: F401,E402
from . import quantization  # noqa: F401,E402
