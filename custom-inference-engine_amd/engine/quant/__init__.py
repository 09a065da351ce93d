"""INT8 weight path: the drop-in for the reference's ``engine.quant`` and its
``kernels.int8_matmul`` kernel."""

from engine.quant.calibrate import calibrate_weight
from engine.quant.int8_linear import Int8Linear, quantize_linear
from engine.quant.int8_matmul import int8_matmul, int8_matmul_workspace_bytes

__all__ = ["Int8Linear", "quantize_linear", "calibrate_weight", "int8_matmul", "int8_matmul_workspace_bytes"]
