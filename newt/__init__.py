"""`import newt` on MI355X: the public surface of newt_amd under the
reference's package name, so existing kernels run unchanged."""

from newt_amd import *  # noqa: F401,F403
from newt_amd import (Autotuner, CompileError, Config, Heuristics, JITFunction,  # noqa: F401
                      __version__, autotune, cdiv, heuristics, jit, next_power_of_2)
from . import language, testing  # noqa: F401
