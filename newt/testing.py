"""`newt.testing`: re-export of newt_amd.testing."""
from newt_amd.testing import assert_close, do_bench  # noqa: F401
