"""CPU oracle for quantized-KV GQA attention (test infrastructure only).

This package checks the product and is never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  ``rec_amd`` never imports it and has no CPU fallback.
"""

from .oracle import *  # noqa: F401,F403
from .oracle import __all__  # noqa: F401
