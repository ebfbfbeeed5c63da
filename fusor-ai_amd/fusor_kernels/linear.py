"""A linear layer and the team-split projections (linear.rs), on the GPU.

The reference calls these from every thread of a team with its share of the output columns
(Ctx::split). `Ctx` mirrors that split so that a caller's per-thread ranges map one to one; a
single full-range call (Ctx(0, 1)) is the natural GPU use.
"""

from ._lib import FormatError, ShapeError
from .matmul import matmul
from .tensor import QUAD

COLUMN_ALIGN = 16        # linear.rs:12-13
NARROW_COLUMN_ALIGN = 8  # linear.rs:14-15


class Ctx:
    """team::Ctx's split (team/src/team.rs:86-93)."""

    def __init__(self, index=0, count=1):
        self.index, self.count = index, count

    def split(self, total, align):
        units = total // align
        return range(units * self.index // self.count * align, units * (self.index + 1) // self.count * align)

    def is_first(self):
        return self.index == 0


class Linear:
    """linear.rs:17-98"""

    def __init__(self, weight, bias=None):
        outputs = weight.rows
        if bias is not None and len(bias.values()) != outputs:
            raise FormatError(f"bias of {len(bias.values())} for {outputs} outputs")
        self.weight, self.bias = weight, bias

    def matrix(self):
        return self.weight.matrix()

    def _bias(self):
        return self.bias.device if self.bias is not None else None

    def project_quads(self, x, cols, store=None, out=None, accumulate=False):
        """store(row, first, x[row]·W[first + lane] + b[first + lane]) per row and quad of `cols`
        (whole quads); returns the device results [rows, len(cols)]."""
        if cols.start % QUAD or cols.stop % QUAD:
            raise ShapeError("whole quads of output columns")
        return matmul(self.matrix(), x, cols, store, bias=self._bias(), out=out, accumulate=accumulate)

    def project(self, x, cols, store=None):
        """The columns `cols` exactly (any range within the outputs), over whole quads."""
        quads = range(cols.start // QUAD * QUAD, (cols.stop + QUAD - 1) // QUAD * QUAD)
        res = self.project_quads(x, quads)
        sub = res[:, cols.start - quads.start:cols.stop - quads.start]
        if store is not None:
            host = sub.cpu().numpy()
            for r in range(host.shape[0]):
                for c, v in zip(cols, host[r]):
                    store(r, c, float(v))
        return sub

    def apply(self, x, quant):
        """out = x·Wᵀ + b for every row and output (linear.rs:89-97)."""
        inp = quant.input(self.matrix(), x)
        return self.project(inp, range(0, self.matrix().rows))


class SharedRows:
    """linear.rs:22-27: the first `rows` rows of a shared activation buffer (a device f32
    tensor)."""

    def __init__(self, values, rows):
        self.values, self.rows = values, rows


def _prepare(linear, rows, quant):
    """linear.rs:145-153: the rows as the linear's input, quantized when its weights are."""
    m = linear.matrix()
    return quant.input(m, rows.values.reshape(-1)[:rows.rows * m.cols])


def project(ctx, linear, rows, quant, out):
    """linear.rs:100-111: this thread's share of the columns of rows·Wᵀ + b into out [rows,
    outputs], the rows quantized into `quant` (a QuantizedRows)."""
    project_input(ctx, linear, _prepare(linear, rows, quant), out)


def project_residual(ctx, linear, rows, residual, quant):
    """linear.rs:121-132: residual[:, cols] += rows·Wᵀ + b for this thread's share."""
    project_residual_input(ctx, linear, _prepare(linear, rows, quant), residual)


def project_input(ctx, linear, x, out):
    """This thread's share of the columns of x·Wᵀ + b into out [rows, outputs] (linear.rs:112-119)."""
    outputs = linear.matrix().rows
    cols = ctx.split(outputs, COLUMN_ALIGN)
    if len(cols) == 0:
        return
    quads = range(cols.start // QUAD * QUAD, (cols.stop + QUAD - 1) // QUAD * QUAD)
    res = linear.project_quads(x, quads)
    out[:, cols.start:cols.stop] = res[:, cols.start - quads.start:cols.stop - quads.start]


def project_residual_input(ctx, linear, x, residual):
    """residual[:, cols] += x·Wᵀ + b for this thread's share (linear.rs:133-143)."""
    outputs = linear.matrix().rows
    cols = ctx.split(outputs, COLUMN_ALIGN)
    if len(cols) == 0:
        return
    view = residual.reshape(-1, outputs)[:, cols.start:cols.stop]
    linear.project_quads(x, range(cols.start, cols.stop), out=view, accumulate=True)
