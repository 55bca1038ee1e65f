"""MatMulNBits weights from ONNX external data (breeze/loader.py:69-95,
``mmap_external=True``): the per-tensor mapping and its checks, that prepack
hands the mapped pages to the library without a host copy, and (GPU) that
weights prepacked from a data file give bit-exact results through the
MatMulNBits operator."""
import types

import numpy as np
import pytest

from conftest import bits_equal, rng_weights


def _tensor(name, data_type, dims, location, offset, external=True):
    ext = [("location", location), ("offset", str(offset)),
           ("length", str(int(np.prod(dims)) * np.dtype(_np(data_type)).itemsize))]
    return types.SimpleNamespace(name=name, data_type=data_type, dims=list(dims),
                                 data_location=1 if external else 0, external_data=ext)


def _np(code):
    from breeze_amd import loader
    return loader.ONNX_TO_NP[code]


def _write_model(tmp_path, arrays):
    """Writes arrays back to back (each 64-byte aligned) into model.data and
    returns TensorProto-like descriptions of them."""
    from breeze_amd import loader
    codes = {np.dtype(v): k for k, v in loader.ONNX_TO_NP.items()}
    blob, tensors, off = bytearray(), {}, 0
    for name, arr in arrays.items():
        arr = np.ascontiguousarray(arr)
        pad = (-off) % 64
        blob += b"\0" * pad
        off += pad
        tensors[name] = _tensor(name, codes[arr.dtype], arr.shape, "model.data", off)
        blob += arr.astype(arr.dtype.newbyteorder("<")).tobytes()
        off += arr.nbytes
    (tmp_path / "model.data").write_bytes(bytes(blob))
    return tensors


def _matmulnbits_graph(rng):
    qw4, sc4, qz4 = rng_weights(rng, 48, 128, 4, np.float16, True)
    qw8, sc8, _ = rng_weights(rng, 32, 96, 8, np.float32)
    arrays = {"w4": qw4, "s4": sc4, "z4": qz4, "w8": qw8, "s8": sc8}
    nodes = [
        types.SimpleNamespace(name="p4", op_type="MatMulNBits", inputs=["x", "w4", "s4", "z4"],
                              attrs=dict(K=128, N=48, bits=4, block_size=32)),
        types.SimpleNamespace(name="p8", op_type="MatMulNBits", inputs=["x", "w8", "s8", ""],
                              attrs=dict(K=96, N=32, bits=8, block_size=32)),
    ]
    return arrays, nodes


def test_external_tensors_map_the_file_bytes(tmp_path):
    from breeze_amd import loader

    arrays, _ = _matmulnbits_graph(np.random.default_rng(1))
    tensors = _write_model(tmp_path, arrays)
    for name, arr in arrays.items():
        got = loader.load_tensor(tmp_path, tensors[name])
        assert isinstance(got, np.memmap) and not got.flags.writeable
        assert got.dtype.byteorder in ("<", "=", "|") and got.shape == arr.shape
        np.testing.assert_array_equal(got, arr)


def test_external_tensor_checks_follow_the_reference_loader(tmp_path):
    from breeze_amd import loader

    (tmp_path / "model.data").write_bytes(bytes(256))
    ok = _tensor("t", loader.FLOAT, (4, 4), "model.data", 0)
    assert loader.external_tensor(tmp_path, ok).shape == (4, 4)
    for bad in ("../model.data", "sub/../../x.data", str(tmp_path / "model.data")):
        with pytest.raises(ValueError, match="escapes model directory"):
            loader.external_tensor(tmp_path, _tensor("t", loader.FLOAT, (4,), bad, 0))
    bf16 = types.SimpleNamespace(**{**vars(ok), "data_type": 16})
    with pytest.raises(ValueError, match="Unsupported external tensor dtype 16"):
        loader.external_tensor(tmp_path, bf16)
    with pytest.raises(ValueError, match="Truncated external tensor"):
        loader.external_tensor(tmp_path, _tensor("t", loader.FLOAT, (8, 8), "model.data", 64))
    with pytest.raises(ValueError, match="Truncated external tensor"):
        loader.external_tensor(tmp_path, _tensor("t", loader.FLOAT, (4,), "model.data", -4))
    empty = loader.external_tensor(tmp_path, _tensor("t", loader.UINT8, (0, 16), "model.data", 0))
    assert empty.shape == (0, 16) and empty.dtype == np.uint8
    inline = _tensor("t", loader.FLOAT, (2,), "model.data", 0, external=False)
    with pytest.raises(ValueError, match="needs a converter"):
        loader.load_tensor(tmp_path, inline)
    assert loader.load_tensor(tmp_path, inline, lambda t: np.ones(2)).tolist() == [1.0, 1.0]


def test_prepack_hands_the_mapped_pages_to_the_library(tmp_path, hb, monkeypatch):
    """The packed weights, scales and zero points reach the native prepack as
    the mapped file pages themselves (no host copy)."""
    from breeze_amd import loader, ops

    arrays, nodes = _matmulnbits_graph(np.random.default_rng(2))
    tensors = _write_model(tmp_path, arrays)
    inits = {name: loader.load_tensor(tmp_path, t) for name, t in tensors.items()}
    seen = []

    def fake_prepack(qw, sc, qz, N, K, bits, scale_bits):
        seen.append((qw.value, sc.value, qz.value if qz is not None else None, N, K, bits, scale_bits))
        return 1000 + len(seen)

    monkeypatch.setattr(hb, "_native_prepack", fake_prepack)
    cache = ops.prepack_nodes(nodes, inits, backend=hb)
    assert cache == {"p4": ("i4", 1001, 48), "p8": ("i4", 1002, 32)}
    addr = {k: v.ctypes.data for k, v in inits.items()}
    assert seen[0] == (addr["w4"], addr["s4"], addr["z4"], 48, 128, 4, 16)
    assert seen[1] == (addr["w8"], addr["s8"], None, 32, 96, 8, 32)


@pytest.mark.gpu
def test_external_data_weights_bit_exact(tmp_path, gpu, hb, orc, hi_prec):
    from breeze_amd import loader, ops

    rng = np.random.default_rng(3)
    arrays, nodes = _matmulnbits_graph(rng)
    tensors = _write_model(tmp_path, arrays)
    inits = {name: loader.load_tensor(tmp_path, t) for name, t in tensors.items()}
    cache = ops.prepack_nodes(nodes, inits)
    try:
        for hp in (False, True):
            hb.set_hi_prec(hp)
            for node in nodes:
                K, N, bits = node.attrs["K"], node.attrs["N"], node.attrs["bits"]
                qz = arrays["z4"] if bits == 4 else None
                sc = arrays["s4"] if bits == 4 else arrays["s8"]
                qw = arrays["w4"] if bits == 4 else arrays["w8"]
                a = rng.normal(size=(2, 3, K)).astype(np.float32)
                got = ops.matmul_nbits(cache, node.name, a)
                want = orc.matmul(qw, sc, qz, N, K, bits, a.reshape(-1, K), hp).reshape(2, 3, N)
                assert bits_equal(got, want), (node.name, hp)
    finally:
        ops.free_cache(cache)
