"""The MatMulNBits operator of breeze-engine's graph session on the GPU path.

breeze-engine prepacks every ``MatMulNBits`` node of a graph once
(breeze/graph_session.py:47-64) into a weight cache whose entries are
``("i4", handle, N)`` for the compiled kernel, or ``("linear", w, N)`` /
``("dense", W_fp32[K, N], N)`` for the float fallbacks, and the operator body
(breeze/ops.py:118-130) reshapes the activation to 2-D, multiplies and
restores the leading shape.  This module keeps that cache format and
operator contract with ``hip_backend`` in place of ``cpu_backend``, so a
graph session can route its quantized projections to the GPU by swapping the
backend module.

Nodes are described by the attributes the session reads: ``name``,
``inputs`` (initializer names: activation, qweight, scales, optional
qzeros) and ``attrs`` (``N``, ``K``, ``bits``, ``block_size``).  The
reference session prepacks with the default 4 bits; here ``bits`` and
``block_size`` come from the node, so 8-bit nodes prepack correctly too.
"""
import numpy as np

from . import hip_backend


def _qzeros(node, initializers):
    # graph_session.py:57-58: an absent or empty fourth input means no zeros.
    if len(node.inputs) > 3 and node.inputs[3] != "":
        return initializers[node.inputs[3]]
    return None


def prepack_nodes(nodes, initializers, backend=hip_backend):
    """Prepack the ``MatMulNBits`` nodes into a weight cache
    ``{node name: ("i4", handle, N)}`` (graph_session.py:53-64)."""
    cache = {}
    try:
        for node in nodes:
            if getattr(node, "op_type", "MatMulNBits") != "MatMulNBits":
                continue
            attrs = node.attrs
            N, K = int(attrs["N"]), int(attrs["K"])
            handle = backend.prepack(
                initializers[node.inputs[1]],
                initializers[node.inputs[2]],
                _qzeros(node, initializers),
                K, N,
                bits=int(attrs.get("bits", 4)),
                block_size=int(attrs.get("block_size", 32)))
            cache[node.name] = ("i4", handle, N)
    except BaseException:
        free_cache(cache, backend)
        raise
    return cache


def matmul_nbits(weight_cache, node_name, a, backend=hip_backend):
    """The operator body (ops.py:118-130): ``a[..., K]`` times the cached
    weight, returning ``[..., N]`` float32.  A NumPy input gives NumPy out; a
    GPU torch tensor stays on the device (the backend's stream semantics)."""
    kind, w, N = weight_cache[node_name]
    if hip_backend._is_torch(a):
        a2d = a.reshape(-1, a.shape[-1])
        if kind != "i4":
            raise TypeError("the float fallbacks take NumPy activations")
        return backend.matmul(w, a2d, N).reshape(*a.shape[:-1], N)
    a = np.asarray(a, dtype=np.float32)
    a2d = a.reshape(-1, a.shape[-1])
    if kind == "i4":
        out2d = backend.matmul(w, a2d, N)
    elif kind == "dense":
        out2d = a2d @ w
    else:
        from . import linear

        out2d = linear.linear(a2d, w)
    return out2d.reshape(*a.shape[:-1], N)


def free_cache(weight_cache, backend=hip_backend):
    """Release every ``"i4"`` handle of a weight cache and empty it."""
    for kind, w, _ in list(weight_cache.values()):
        if kind == "i4":
            backend.free(w)
    weight_cache.clear()
