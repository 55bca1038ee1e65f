"""The MatMulNBits operator module without a GPU: the weight-cache format and
prepack arguments of breeze/graph_session.py:47-64 and the operator body of
breeze/ops.py:118-130 (reshape to 2-D, multiply, restore the leading shape),
driven through a stub backend whose matmul is the oracle."""
import types

import numpy as np
import pytest

from conftest import bits_equal, rng_weights


class StubBackend:
    def __init__(self, orc, fail_at=None):
        self.orc = orc
        self.calls = []
        self.freed = []
        self.fail_at = fail_at

    def prepack(self, qw, sc, qz, K, N, bits=4, block_size=32):
        if self.fail_at is not None and len(self.calls) == self.fail_at:
            raise ValueError("contract")
        self.calls.append(dict(K=K, N=N, bits=bits, block_size=block_size, qz=qz is not None))
        return (len(self.calls), qw, sc, qz, K, N, bits)

    def matmul(self, h, a2d, N):
        _, qw, sc, qz, K, N2, bits = h
        assert N2 == N and a2d.ndim == 2
        return self.orc.matmul(qw, sc, qz, N, K, bits, a2d, True)

    def free(self, h):
        self.freed.append(h[0])


def _node(name, inputs, **attrs):
    return types.SimpleNamespace(name=name, op_type="MatMulNBits", inputs=inputs, attrs=attrs)


def _graph(rng):
    qw4, sc4, qz4 = rng_weights(rng, 32, 64, 4, np.float32, True)
    qw8, sc8, _ = rng_weights(rng, 48, 96, 8)
    inits = {"w4": qw4, "s4": sc4, "z4": qz4, "w8": qw8, "s8": sc8}
    nodes = [
        _node("proj4", ["x", "w4", "s4", "z4"], K=64, N=32, bits=4, block_size=32),
        _node("proj8", ["x", "w8", "s8", ""], K=96, N=48, bits=8, block_size=32),
        types.SimpleNamespace(name="norm", op_type="SimplifiedLayerNormalization", inputs=[], attrs={}),
    ]
    return nodes, inits


def test_prepack_nodes_builds_the_session_cache(orc):
    from breeze_amd import ops

    nodes, inits = _graph(np.random.default_rng(0))
    be = StubBackend(orc)
    cache = ops.prepack_nodes(nodes, inits, backend=be)
    assert sorted(cache) == ["proj4", "proj8"]
    assert [e[0] for e in cache.values()] == ["i4", "i4"]
    assert cache["proj4"][2] == 32 and cache["proj8"][2] == 48
    assert be.calls == [dict(K=64, N=32, bits=4, block_size=32, qz=True),
                        dict(K=96, N=48, bits=8, block_size=32, qz=False)]
    ops.free_cache(cache, backend=be)
    assert cache == {} and sorted(be.freed) == [1, 2]


def test_prepack_nodes_releases_handles_on_failure(orc):
    from breeze_amd import ops

    nodes, inits = _graph(np.random.default_rng(1))
    be = StubBackend(orc, fail_at=1)
    with pytest.raises(ValueError):
        ops.prepack_nodes(nodes, inits, backend=be)
    assert be.freed == [1]


def test_matmul_nbits_restores_the_leading_shape(orc):
    from breeze_amd import ops

    rng = np.random.default_rng(2)
    nodes, inits = _graph(rng)
    be = StubBackend(orc)
    cache = ops.prepack_nodes(nodes, inits, backend=be)
    a = rng.normal(size=(2, 3, 96)).astype(np.float32)
    out = ops.matmul_nbits(cache, "proj8", a, backend=be)
    assert out.shape == (2, 3, 48) and out.dtype == np.float32
    want = orc.matmul(inits["w8"], inits["s8"], None, 48, 96, 8, a.reshape(6, 96), True)
    assert bits_equal(out.reshape(6, 48), want)


def test_matmul_nbits_float_fallbacks():
    from breeze_amd import linear, ops

    rng = np.random.default_rng(3)
    w = rng.normal(size=(64, 24)).astype(np.float32)
    a = rng.normal(size=(5, 64)).astype(np.float32)
    cache = {"d": ("dense", w, 24), "l": ("linear", linear.prepare_weight(w), 24)}
    assert np.array_equal(ops.matmul_nbits(cache, "d", a), a @ w)
    out = ops.matmul_nbits(cache, "l", a[None])
    assert out.shape == (1, 5, 24)
    if linear.backend() == "numpy-fp32":
        assert np.allclose(out[0], a @ w, rtol=1e-5, atol=1e-5)
