"""newt_amd - newt's block-programming DSL on AMD Instinct MI355X (gfx950).

    import newt                      # (the `newt` package re-exports newt_amd)
    import newt.language as nl

    @newt.jit
    def add_kernel(x_ptr, y_ptr, out_ptr, n, BLOCK: nl.constexpr):
        pid = nl.program_id(0)
        offs = pid * BLOCK + nl.arange(0, BLOCK)
        mask = offs < n
        x = nl.load(x_ptr + offs, mask=mask)
        y = nl.load(y_ptr + offs, mask=mask)
        nl.store(out_ptr + offs, x + y, mask=mask)

    add_kernel[(newt.cdiv(n, 1024),)](x, y, out, n, BLOCK=1024)

Kernels compile to HIP C++ for gfx950 (hipRTC) and launch through
hipModuleLaunchKernel on torch-ROCm's current stream.
"""

from . import language, testing
from .compiler import CompileError
from .runtime.autotuner import Autotuner, Config, Heuristics, autotune, heuristics
from .runtime.jit import JITFunction, jit

__version__ = "0.1.0"


def cdiv(a, b):
    return -(-a // b)


def next_power_of_2(n):
    n = int(n)
    if n <= 1:
        return 1
    return 1 << (n - 1).bit_length()


__all__ = ["Autotuner", "CompileError", "Config", "Heuristics", "JITFunction", "__version__",
           "autotune", "cdiv", "heuristics", "jit", "language", "next_power_of_2", "testing"]
