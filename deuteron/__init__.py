"""`import deuteron` on MI355X: the tile DSL of newt_amd.deuteron under the
reference's package name, so existing deuteron kernels run unchanged."""

from newt_amd.deuteron import *  # noqa: F401,F403
from newt_amd.deuteron import (Config, EagerTensor, Kernel, Tile, TraceError,  # noqa: F401
                               __version__, kernel)
from newt_amd.deuteron import language  # noqa: F401
