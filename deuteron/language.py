"""`deuteron.language`: re-export of newt_amd.deuteron.language."""
from newt_amd.deuteron.language import *  # noqa: F401,F403
