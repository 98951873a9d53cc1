"""``torch.ops.quantized_ops`` on MI355X kernels (see ``quantized.py``)."""

from .quantized import (  # noqa: F401
    calculate_mx_qparam,
    dequantize,
    linear_mx,
    matmul_mx,
    mx_fake_quantize,
    quantize,
    quantize_mx,
    quantized_ops_lib,
    register_table,
    vmap,
)
