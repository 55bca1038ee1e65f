"""breeze_amd -- Breeze's quantized linear path on AMD MI355X (gfx950).

Modules mirror the reference's public surface for this path:
``hip_backend`` (for breeze/cpu_backend.py), ``quant`` (breeze/quant.py) and
``linear`` (breeze/linear.py, imported on demand since it pulls in torch).
The compute lives in ``libbreeze_qmm.so``, hand-written HIP behind a C ABI
(include/breeze_qmm.h).
"""
from . import hip_backend, quant  # noqa: F401

__all__ = ["hip_backend", "quant", "linear"]
