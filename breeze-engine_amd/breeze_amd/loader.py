"""MatMulNBits initializers from ONNX external data, mapped without host copies.

breeze-engine's loader maps every external initializer of a model straight
from its ``.data`` file (breeze/loader.py:69-95, ``mmap_external=True``) so a
graph session can prepack the quantized projections without reading the
weights into host buffers first.  ``external_tensor`` is that per-tensor
step with the same checks and errors: the location must stay inside the
model directory, the element type must be one the loader knows, the byte
range must lie inside the file, and an empty tensor is an empty array.  It
returns a read-only ``numpy.memmap``; ``hip_backend.prepack`` passes such a
map's pages to the library, which copies the packed weight bytes to the GPU
and repacks them there, so the bulk of every weight goes file -> device with
no host-side copy.

Tensors are described by the fields ONNX's ``TensorProto`` carries (``name``,
``data_type``, ``dims``, ``data_location``, ``external_data`` key/value
entries), so an ``onnx`` ``TensorProto`` works as it is; ``load_external``
reads a model file with the ``onnx`` package when it is installed.
"""
from pathlib import Path

import numpy as np

# ONNX TensorProto.DataType codes (the ONNX specification) -> numpy, the subset
# breeze/loader.py:11-20 maps.
FLOAT, UINT8, INT8, INT32, INT64, BOOL, FLOAT16, DOUBLE = 1, 2, 3, 6, 7, 9, 10, 11
ONNX_TO_NP = {
    FLOAT: np.float32,
    FLOAT16: np.float16,
    DOUBLE: np.float64,
    INT64: np.int64,
    INT32: np.int32,
    INT8: np.int8,
    UINT8: np.uint8,
    BOOL: np.bool_,
}
EXTERNAL = 1  # TensorProto.DataLocation.EXTERNAL


def _entries(tensor):
    out = {}
    for e in tensor.external_data:
        key, value = (e.key, e.value) if hasattr(e, "key") else e
        out[key] = value
    return out


def external_tensor(base, tensor):
    """Map one external initializer (breeze/loader.py:73-91): a read-only
    little-endian ``numpy.memmap`` of the tensor's bytes in its data file,
    located relative to the model directory ``base``."""
    info = _entries(tensor)
    location = Path(info["location"])
    if location.is_absolute() or ".." in location.parts:
        raise ValueError(f"External tensor escapes model directory: {tensor.name}")
    external = Path(base) / location
    if tensor.data_type not in ONNX_TO_NP:
        raise ValueError(f"Unsupported external tensor dtype {tensor.data_type}: {tensor.name}")
    dtype = np.dtype(ONNX_TO_NP[tensor.data_type]).newbyteorder("<")
    offset = int(info.get("offset", 0))
    dims = tuple(int(d) for d in tensor.dims)
    count = int(np.prod(dims, dtype=np.int64))
    if offset < 0 or offset + count * dtype.itemsize > external.stat().st_size:
        raise ValueError(f"Truncated external tensor: {tensor.name}")
    if count == 0:
        return np.empty(dims, dtype=dtype)
    return np.memmap(external, dtype=dtype, mode="r", offset=offset, shape=dims)


def load_tensor(base, tensor, to_array=None):
    """An initializer as breeze/loader.py:73-75 loads it: mapped when it is
    external, else converted by ``to_array`` (``onnx.numpy_helper.to_array``
    for ONNX tensors)."""
    if tensor.data_location != EXTERNAL:
        if to_array is None:
            raise ValueError(f"{tensor.name}: in-model tensor data needs a converter")
        return to_array(tensor)
    return external_tensor(base, tensor)


def load_external(path):
    """``{name: array}`` for a model's initializers, external ones mapped
    (breeze/loader.py:69-95).  Needs the ``onnx`` package."""
    try:
        import onnx
        from onnx import numpy_helper
    except ImportError as e:
        raise RuntimeError("reading .onnx files needs the onnx package") from e
    base = Path(path).absolute().parent
    graph = onnx.load(path, load_external_data=False).graph
    return {t.name: load_tensor(base, t, numpy_helper.to_array) for t in graph.initializer}
