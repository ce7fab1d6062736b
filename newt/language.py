"""`newt.language` (nl): re-export of newt_amd.language."""
from newt_amd.language import *  # noqa: F401,F403
from newt_amd.language import constexpr  # noqa: F401
