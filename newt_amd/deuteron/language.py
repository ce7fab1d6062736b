"""deuteron.language - the tile DSL surface (`import deuteron as dt`).

Behaviour follows the reference (deuteron/language.py:1-144): every function
has an eager PyTorch meaning, so a @dt.kernel function called with full-size
tiles runs as plain PyTorch - that is the correctness oracle the autotuner
checks candidate configurations against, and the DEUTERON_INTERPRET mode. The
tracer (tracer.py) maps the same names onto nl.* for compiled kernels.
"""

import torch

float32 = torch.float32
float16 = torch.float16
bfloat16 = torch.bfloat16
int32 = torch.int32
int64 = torch.int64


class Tile:
    """One tile of an iteration dimension. Eagerly it spans the whole
    dimension; compiled, it is BLOCK_<NAME> offsets plus a bounds mask."""

    def __init__(self, size, name=None):
        self.size = int(size)
        self.name = name

    def as_slice(self):
        return slice(0, self.size)

    def __repr__(self):
        return f"Tile({self.name or '?'}, {self.size})"


def _eager_index(idx):
    idx = idx if isinstance(idx, tuple) else (idx,)
    return tuple(i.as_slice() if isinstance(i, Tile) else i for i in idx)


class EagerTensor:
    """A kernel argument during eager execution: Tile indices act as full
    slices, reads give plain tensors, writes go to the wrapped tensor."""

    def __init__(self, t):
        self._t = t

    def __getitem__(self, idx):
        return self._t[_eager_index(idx)]

    def __setitem__(self, idx, value):
        self._t[_eager_index(idx)] = value

    @property
    def shape(self):
        return self._t.shape

    @property
    def dtype(self):
        return self._t.dtype

    def size(self, d=None):
        return self._t.size() if d is None else self._t.size(d)


def tile(sizes):
    """Iterate over tiles of one or more dimensions. The outermost loop of a
    kernel is its launch grid, inner ones sequential loops. Eagerly: one
    full-size tile (or a tuple of them)."""
    if isinstance(sizes, (list, tuple)):
        yield tuple(Tile(s) for s in sizes)
    else:
        yield Tile(sizes)


def _sizes(shape):
    return [s.size if isinstance(s, Tile) else int(s) for s in shape]


def zeros(shape, dtype=torch.float32):
    return torch.zeros(*_sizes(shape), dtype=dtype, device="cuda")


def full(shape, value, dtype=torch.float32):
    return torch.full(_sizes(shape), value, dtype=dtype, device="cuda")


exp = torch.exp
log = torch.log
sqrt = torch.sqrt
rsqrt = torch.rsqrt
sigmoid = torch.sigmoid
tanh = torch.tanh
erf = torch.erf
abs = torch.abs
maximum = torch.maximum
minimum = torch.minimum
where = torch.where


def relu(x):
    return torch.clamp_min(x, 0)


# dt.<name>(args) -> newt expression (positional placeholders)
NL_CALLS = {
    "exp": "nl.exp({0})",
    "log": "nl.log({0})",
    "sqrt": "nl.sqrt({0})",
    "rsqrt": "nl.rsqrt({0})",
    "sigmoid": "nl.sigmoid({0})",
    "tanh": "nl.tanh({0})",
    "erf": "nl.erf({0})",
    "abs": "nl.abs({0})",
    "maximum": "nl.maximum({0}, {1})",
    "minimum": "nl.minimum({0}, {1})",
    "where": "nl.where({0}, {1}, {2})",
    "relu": "nl.maximum({0}, 0.0)",
}

# value.<method>(axis) reductions -> (nl function, identity for masked lanes)
REDUCE_METHODS = {
    "sum": ("nl.sum", "0.0"),
    "max": ("nl.max", "float('-inf')"),
    "amax": ("nl.max", "float('-inf')"),
    "min": ("nl.min", "float('inf')"),
    "amin": ("nl.min", "float('inf')"),
}

NL_DTYPES = {
    torch.float32: "nl.float32",
    torch.float16: "nl.float16",
    torch.bfloat16: "nl.bfloat16",
    torch.int32: "nl.int32",
    torch.int64: "nl.int64",
}
