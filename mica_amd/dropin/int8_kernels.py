"""Top-level ``int8_kernels`` for the reference's serving code (akivet/Mica v0.5/serving/lib).

The reference imports its kernel launcher by its bare module name, ``import int8_kernels as aot``
(int8_runtime.py:78, 222, 262, 278, 551; fast_runtime.py:67), in the server process and again in the
self-test child that int8_runtime._spawn starts (int8_runtime.py:292, 501-524).  That child rebuilds
``sys.path`` from the parent's list before any import, so a directory placed ahead of the reference's
``lib/`` on the parent's ``sys.path`` is searched first in both processes.  This directory is meant to
be that one: importing ``int8_kernels`` from it binds the name to ``mica_amd.int8_kernels`` itself (the
same module object, so ``STATS`` and ``ATTN`` are shared with every other user of mica_amd).
"""
import sys
from pathlib import Path

_ROOT = str(Path(__file__).resolve().parents[2])   # the checkout that holds the mica_amd package
if _ROOT not in sys.path:
    sys.path.append(_ROOT)

from mica_amd import int8_kernels as _impl  # noqa: E402

# the import system returns whatever sys.modules holds under the name once this file has run
sys.modules[__name__] = _impl
