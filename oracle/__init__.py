"""CPU oracle for DeLS-Spec's draft-token selection path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory: only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline
leg of ``bench.py`` use it, and only to test results against (or as the timed CPU
baseline), never as a fallback for the HIP path.
"""

from .dels_oracle import *  # noqa: F401,F403
from . import sampling  # noqa: F401
from . import domino  # noqa: F401
from . import bounds  # noqa: F401
