"""Products over many rows (conv.rs:563-606), on the GPU.

The reference splits the rows (or, for few rows, the output columns) over a team's threads and
walks each thread's share in chunks of 64 rows, quantizing every chunk before its product. Rows
are independent and each output's group order is unchanged, so one launch over a thread's whole
share gives the same bits; `Patches` keeps the quantization scratch the reference keeps there.
"""

from .linear import COLUMN_ALIGN
from .matmul import Input, QuantizedRows
from .tensor import QUAD

CHUNK_ROWS = 64  # conv.rs: rows quantized and projected at a time on the CPU


class Patches:
    """conv.rs:114-118: per-thread scratch of the row products."""

    def __init__(self):
        self.quant = QuantizedRows()


def project_rows(ctx, linear, rows, patches, out):
    """conv.rs:563-575: out[row, col] = input[row]·W[col] + b[col] for this thread's share of
    `rows` = (input, count) rows of the linear's width (a device f32 tensor) and every output
    column; `out` is a device f32 tensor [count, outputs]. Split by rows when there are at least
    as many rows as outputs or the outputs are not whole COLUMN_ALIGN units, else by columns
    (conv.rs:584-589)."""
    x, count = rows
    matrix = linear.matrix()
    outputs, width = matrix.rows, matrix.cols
    by_rows = count >= outputs or outputs % COLUMN_ALIGN != 0
    if by_rows:
        mine, cols = ctx.split(count, 1), range(0, outputs)
    else:
        mine, cols = range(0, count), ctx.split(outputs, COLUMN_ALIGN)
    if len(mine) == 0 or len(cols) == 0:
        return
    flat = x.reshape(-1)[mine.start * width:mine.stop * width]
    inp = patches.quant.input(matrix, flat) if len(mine) > 4 else Input(f32=flat)
    quads = range(cols.start // QUAD * QUAD, (cols.stop + QUAD - 1) // QUAD * QUAD)
    res = linear.project_quads(inp, quads)
    out[mine.start:mine.stop, cols.start:cols.stop] = res[:, cols.start - quads.start:cols.stop - quads.start]
