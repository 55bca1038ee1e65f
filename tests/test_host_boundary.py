"""The drop-in boundary on a machine without a GPU: the C-ABI library loads
and exports every entry point include/breeze_qmm.h declares, the Python
bridge keeps the reference's validation and exception contract
(breeze/cpu_backend.py:119-168, tests/test_cpu_packing.py:171-190), the
native entry points reject contract violations before touching a device,
and the host-built legacy layout carries exactly the MatMulNBits weights.
No test here launches device work.
"""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT, rng_weights

HEADER = os.path.join(ROOT, "include", "breeze_qmm.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(i4_\w+)\s*\(", text)))


def test_header_declares_the_reference_abi_and_gpu_additions():
    names = _declared_functions()
    for ref_name in ("i4_set_threads", "i4_set_numa_split", "i4_set_hi_prec", "i4_prepack_onnx",
                     "i4_prepack", "i4_free", "i4_matmul", "i4_matmul_region"):
        assert ref_name in names
    for gpu_name in ("i4_last_error", "i4_device_ok", "i4_matmul_dev", "i4_matmul_argmax_dev"):
        assert gpu_name in names


def test_library_loads_and_exports_every_declared_symbol(hb):
    assert hb.available(), f"library failed to load: {hb._SO}"
    lib = ctypes.CDLL(hb._SO)
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_native_prepack_rejects_contract_violations_without_a_device(hb):
    lib = hb._lib
    qw = np.zeros(64 * 16, np.uint8)
    sc = np.ones(64, np.float32)
    for N, K, bits, sbits in ((15, 32, 4, 32), (16, 33, 4, 32), (0, 32, 4, 32), (16, 32, 5, 32),
                              (16, 32, 4, 8), (-16, 32, 8, 32)):
        assert not lib.i4_prepack_onnx(hb._p(qw), hb._p(sc), None, N, K, bits, sbits)
        assert hb.last_error()
    zeros = np.full(16, 128, np.uint8)
    assert not lib.i4_prepack_onnx(hb._p(qw), hb._p(sc), hb._p(zeros), 16, 32, 8, 32)
    assert "zero" in hb.last_error()


def test_native_prepack_refuses_weights_past_the_kernels_cursors(hb):
    """The decode kernels address weights with 32-bit cursors over 16-byte
    chunks: a handle of 64 GiB or more is refused before any buffer is read
    (the tiny buffers here are never touched), by both packers."""
    lib = hb._lib
    qw = np.zeros(16, np.uint8)
    sc = np.ones(16, np.float32)
    # INT4: N * K / 2 bytes; 2^20 x 2^17 is exactly 64 GiB, one 32-block less fits.
    assert not lib.i4_prepack_onnx(hb._p(qw), hb._p(sc), None, 1 << 20, 1 << 17, 4, 32)
    assert "2^32" in hb.last_error()
    # INT8: N * K bytes; 2^20 x 2^16 is 64 GiB.
    assert not lib.i4_prepack_onnx(hb._p(qw), hb._p(sc), None, 1 << 20, 1 << 16, 8, 32)
    assert "2^32" in hb.last_error()
    corr = np.zeros(16, np.int32)
    assert not lib.i4_prepack(hb._p(qw), hb._p(sc), None, hb._p(corr), 1 << 20, 1 << 16, 1 << 11, 8)
    assert "2^32" in hb.last_error()


def test_native_calls_reject_a_foreign_handle(hb):
    bogus = np.zeros(64, np.uint8)
    A = np.zeros((1, 32), np.float32)
    C = np.zeros((1, 16), np.float32)
    hb._lib.i4_matmul(hb._p(bogus), hb._p(A), 1, hb._p(C))
    assert "invalid handle" in hb.last_error()
    assert hb._lib.i4_matmul_dev(hb._p(bogus), hb._p(A), 1, hb._p(C), None) != 0
    hb._lib.i4_free(None)  # NULL is ignored, as in the reference


@pytest.mark.parametrize("fault", ["weights", "scales", "zeros", "zero_dtype", "fractional_dim",
                                   "overflow_dim", "bool_dim", "bits", "block_size", "n_mod16",
                                   "k_mod32", "weight_dtype", "int8_zero_point"])
def test_prepack_validation_matches_reference_contract(hb, fault):
    rng = np.random.default_rng(1)
    qw, sc, qz = rng_weights(rng, 16, 32, 4, np.float32, True)
    K, N, bits, bs = 32, 16, 4, 32
    if fault == "weights":
        qw = qw.reshape(-1)[:-1]
    elif fault == "scales":
        sc = sc.reshape(-1)[:-1]
    elif fault == "zeros":
        qz = qz.reshape(-1)[:-1]
    elif fault == "zero_dtype":
        qz = qz.astype(np.int16)
    elif fault == "fractional_dim":
        K = 32.0
    elif fault == "overflow_dim":
        N = 2 ** 40
    elif fault == "bool_dim":
        N = True
    elif fault == "bits":
        bits = 3
    elif fault == "block_size":
        bs = 64
    elif fault == "n_mod16":
        N = 24
    elif fault == "k_mod32":
        K = 48
    elif fault == "weight_dtype":
        qw = qw.astype(np.int8)
    elif fault == "int8_zero_point":
        bits = 8
        qw = np.zeros((16, 1, 32), np.uint8)
        qz = np.full((16, 1), 127, np.uint8)
    with pytest.raises(ValueError):
        hb.prepack(qw, sc, qz, K, N, bits=bits, block_size=bs)


def test_prepack_without_library_raises_runtime_error(hb, monkeypatch):
    rng = np.random.default_rng(2)
    qw, sc, _ = rng_weights(rng, 16, 32, 4)
    monkeypatch.setattr(hb, "_lib", None)
    with pytest.raises(RuntimeError):
        hb.prepack(qw, sc, None, 32, 16)
    with pytest.raises(RuntimeError):
        hb.matmul(1, np.zeros((1, 32), np.float32), 16)


def test_prepack_null_handle_raises_memory_error(hb, monkeypatch):
    rng = np.random.default_rng(3)
    qw, sc, _ = rng_weights(rng, 16, 32, 8)
    monkeypatch.setattr(hb, "_native_prepack", lambda *a: None)
    with pytest.raises(MemoryError):
        hb.prepack(qw, sc, None, 32, 16, bits=8)


@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
def test_legacy_layout_carries_the_matmulnbits_weights(hb, orc, bits, explicit_zeros):
    """The host-built legacy layout, read back by the oracle's restatement of
    the reference tile kernels, gives the MatMulNBits weights, scales and a
    corr with no delta."""
    N, K = 48, 160
    rng = np.random.default_rng(4 + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float16, explicit_zeros)
    B, scale, zp, corr = hb._legacy_layout(qw, sc, qz, K, N, bits)
    b, sb, delta = orc.unpack_legacy(B, scale, zp, corr, N, K, bits)
    b_ref, sb_ref = orc.unpack_nbits(qw, sc, qz, N, K, bits)
    assert np.array_equal(b, b_ref)
    assert np.array_equal(sb.view(np.uint32), sb_ref.view(np.uint32))
    assert not delta.any()


def test_dequant_contract_matches_oracle():
    from breeze_amd import quant
    from oracle import oracle

    rng = np.random.default_rng(5)
    for bits in (4, 8):
        N, K = 32, 192
        qw, sc, qz = rng_weights(rng, N, K, bits, np.float16, bits == 4)
        a = quant.dequantize_matmul_nbits(qw, sc, qz, bits=bits, block_size=32, K=K, N=N)
        b = oracle.dequantize_matmul_nbits(qw, sc, qz, bits=bits, block_size=32, K=K, N=N)
        assert a.shape == (K, N)
        assert np.array_equal(a, b)


def test_dequant_equals_the_oracles_unpacked_weights_times_scales(orc):
    """breeze/quant.py:9-58 against the C oracle's unpacking (the one the
    golden vectors pin through every matmul): W[k, n] = b[n, k] * s[n, k/32]
    exactly, with b = nibble - zero point (explicit packed INT4 zero points,
    low nibble first, odd block counts so the last zero-point byte is half
    used) or byte - 128, fp16 and fp32 scales.  (q - zp) is an exact small
    integer in float, so both sides round once."""
    from breeze_amd import quant

    rng = np.random.default_rng(15)
    for bits, explicit in ((4, True), (4, False), (8, False)):
        for dtype in (np.float16, np.float32):
            N, K = 48, 32 * 7
            qw, sc, qz = rng_weights(rng, N, K, bits, dtype, explicit)
            W = quant.dequantize_matmul_nbits(qw, sc, qz, bits=bits, block_size=32, K=K, N=N)
            b, sb = orc.unpack_nbits(qw, sc, qz, N, K, bits)
            want = (b.astype(np.float32) * np.repeat(sb, 32, axis=1)).T
            assert W.dtype == np.float32 and W.shape == (K, N)
            assert np.array_equal(W.view(np.uint32), np.ascontiguousarray(want).view(np.uint32)), (bits, explicit)


def test_linear_api_on_cpu():
    from breeze_amd import linear

    rng = np.random.default_rng(6)
    w = rng.normal(size=(64, 48)).astype(np.float32)
    a = rng.normal(size=(2, 3, 64)).astype(np.float32)
    pw = linear.prepare_weight(w)
    out = linear.linear(a, pw)
    assert out.shape == (2, 3, 48) and out.dtype == np.float32
    if linear.backend() == "numpy-fp32":
        assert np.allclose(out, a @ w, rtol=1e-5, atol=1e-5)


def test_workload_generator_is_pinned():
    """The seeded benchmark inputs (seeds 1..5, fixed draw order) and the
    algorithmic byte counts stay what the benchmark specification fixes."""
    from breeze_amd import workloads

    assert workloads.algorithmic_bytes("w8_gemv") == 16_826_368
    assert workloads.algorithmic_bytes("w4_gemv") == 26_804_224
    assert workloads.algorithmic_bytes("w4_decode", 1) == 26_804_224
    assert workloads.algorithmic_bytes("w4_decode", 8) == 27_262_976
    assert workloads.algorithmic_bytes("w8_lmhead") == 779_148_288
    assert workloads.algorithmic_ops("w8_prefill") == 182_536_110_080
    import hashlib

    digests = {"w8_gemv": "eea57793c08833d1", "w4_gemv": "7f1653f2c34d5f1b",
               "w4_decode": "396772d7c47415b0"}
    for name, want in digests.items():
        d = workloads.make_config(name)
        h = hashlib.sha256()
        for k in ("qweight", "scales", "A"):
            h.update(np.ascontiguousarray(d[k]).tobytes())
        assert h.hexdigest()[:16] == want, name
    d = workloads.make_config("w8_gemv")
    assert d["qweight"].shape == (4096, 128, 32) and d["A"].shape == (1, 4096)
    d4 = workloads.make_config("w4_decode", 2)
    assert d4["A"].shape == (2, 12288) and np.max(np.abs(d4["A"])) > 20.0  # outliers present
    assert np.all(d4["scales"].reshape(4096, 96, 4) == d4["scales"].reshape(4096, 96, 4)[:, :, :1])


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "8"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
