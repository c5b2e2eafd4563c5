"""CPU restatement of the tagged-op path: test infrastructure only (see oracle.py)."""
from .oracle import *  # noqa: F401,F403
from .oracle import build, lib  # noqa: F401
