"""deuteron on MI355X - a PyTorch-like tile DSL compiled to newt kernels with
correctness-gated autotuning (the reference's nano-Helion, deuteron/__init__.py).

    import deuteron as dt

    @dt.kernel
    def matmul(x, y, out):
        for tile_m, tile_n in dt.tile([x.shape[0], y.shape[1]]):
            acc = dt.zeros([tile_m, tile_n], dtype=dt.float32)
            for tile_k in dt.tile(x.shape[1]):
                acc += x[tile_m, tile_k] @ y[tile_k, tile_n]
            out[tile_m, tile_n] = acc

    matmul(x, y, out)          # traces, autotunes, caches, launches (HIP, gfx950)
    matmul.ref(x, y, out)      # eager PyTorch reference (the oracle)
    print(matmul.to_newt_source(x, y, out))
"""

from .language import (EagerTensor, Tile, abs, bfloat16, erf, exp, float16, float32,  # noqa: F401
                       full, int32, int64, log, maximum, minimum, relu, rsqrt, sigmoid,
                       sqrt, tanh, tile, where, zeros)
from .runtime import Config, Kernel, kernel  # noqa: F401
from .tracer import TraceError  # noqa: F401

__version__ = "0.1.0"
