"""breeze_amd -- Breeze's quantized linear path on AMD MI355X (gfx950).

Modules mirror the reference's public surface for this path:

- ``hip_backend`` for breeze/cpu_backend.py;
- ``quant`` for breeze/quant.py;
- ``linear`` for breeze/linear.py (imported on demand since it pulls in torch);
- ``ops`` for the MatMulNBits operator and weight cache of breeze/ops.py and
  breeze/graph_session.py;
- ``loader`` for the external-data mapping of breeze/loader.py (weights go
  from the mapped file to the GPU without a host copy).

The compute lives in ``libbreeze_qmm.so``, hand-written HIP behind a C ABI
(include/breeze_qmm.h).
"""
from . import hip_backend, loader, ops, quant  # noqa: F401

__all__ = ["hip_backend", "loader", "ops", "quant", "linear"]
