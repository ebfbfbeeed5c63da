"""MI355X (gfx950) implementation of fusor-ai's quantized matrix product (crates/kernels).

The names follow the reference crate's public API (kernels/src/lib.rs:22-31): DType, Tensor,
Table, Matrix, Vector, QuantFormat, QuantizedRows, Quantized, Input, quantize_rows, matmul,
Linear, project, project_input, project_residual, project_residual_input, conv.project_rows,
QuantizedMatrix and the constants, and the blocks crate's int8 attention (attention::attend). Every computation runs in the
HIP library libfusor_gpu.so through its C ABI (include/fusor_gpu.h); there is no CPU fallback.
"""

from ._lib import Error, FormatError, GpuError, ShapeError, lib
from .attention import Call, Exponentials, Operand, attend
from .bundle import IntegrityError, Store
from .conv import Patches, project_rows
from .linear import (COLUMN_ALIGN, NARROW_COLUMN_ALIGN, Ctx, Linear, SharedRows, project, project_input,
                     project_residual, project_residual_input)
from .matmul import (ROWS_PER_CALL, Input, Quantized, QuantizedMatrix, QuantizedRows, matmul, matmul_dots,
                     quantize_rows)
from .qwen2 import Qwen2, Shape
from .tensor import BLOCK, QUAD, TERNARY_GROUP, DType, Matrix, QuantFormat, Table, TableUpload, Tensor, Vector, byte_len

__all__ = [
    "BLOCK", "QUAD", "TERNARY_GROUP", "ROWS_PER_CALL", "COLUMN_ALIGN", "NARROW_COLUMN_ALIGN",
    "DType", "QuantFormat", "Tensor", "Table", "TableUpload", "Matrix", "Vector", "byte_len", "Store",
    "IntegrityError",
    "QuantizedRows", "QuantizedMatrix", "Quantized", "Input", "quantize_rows", "matmul", "matmul_dots",
    "Linear", "Ctx", "SharedRows", "project", "project_input", "project_residual", "project_residual_input",
    "Patches", "project_rows", "Qwen2", "Shape", "Call", "Operand", "Exponentials", "attend",
    "Error", "FormatError", "ShapeError", "GpuError", "lib",
]
