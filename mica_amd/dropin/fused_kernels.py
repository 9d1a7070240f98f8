"""Top-level ``fused_kernels`` for the reference's serving code (akivet/Mica v0.5/serving/lib).

The reference imports its fused RMSNorm / SwiGLU module by its bare name, ``import fused_kernels as ffk``
(fork.py:181, fast_runtime.py:127).  With this directory ahead of the reference's ``lib/`` on
``sys.path``, that name binds to ``mica_amd.fused_kernels`` itself (the same module object).
"""
import sys
from pathlib import Path

_ROOT = str(Path(__file__).resolve().parents[2])   # the checkout that holds the mica_amd package
if _ROOT not in sys.path:
    sys.path.append(_ROOT)

from mica_amd import fused_kernels as _impl  # noqa: E402

# the import system returns whatever sys.modules holds under the name once this file has run
sys.modules[__name__] = _impl
