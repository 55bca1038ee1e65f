"""The oracle against the reference kernel's own outputs.

tests/golden/ref_vectors.npz holds inputs and outputs of the reference CPU
kernel (kernel/quantized_matmul.cpp, compiled from its source into
oracle/_ref by oracle/Makefile; fixture written by tests/golden/gen_golden.py).
Both the C restatement and the independent NumPy twin must reproduce every
output bit-for-bit, in both activation modes.  Where the compiled reference
is present, fresh random cases are compared against it directly as well.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits_equal

FIXTURE = os.path.join(GOLDEN, "ref_vectors.npz")


def _cases():
    z = np.load(FIXTURE)
    meta = json.loads(bytes(z["meta"]).decode())
    return z, meta


Z, META = _cases()


def _get(name, key):
    k = f"{name}_{key}"
    return Z[k] if k in Z.files else None


@pytest.mark.parametrize("name", sorted(n for n in META if not n.startswith("legacy")))
def test_c_oracle_matches_reference_outputs(orc, name):
    m = META[name]
    for hp in (1, 0):
        want = _get(name, f"C_hp{hp}")
        if want is None:
            continue
        got = orc.matmul(_get(name, "qweight"), _get(name, "scales"), _get(name, "qzeros"),
                         m["N"], m["K"], m["bits"], _get(name, "A"), bool(hp))
        assert bits_equal(got, want), (name, hp)
    row0 = _get(name, "C_hp1_row0")
    if row0 is not None:
        got = orc.matmul(_get(name, "qweight"), _get(name, "scales"), _get(name, "qzeros"),
                         m["N"], m["K"], m["bits"], _get(name, "A")[:1], True)
        assert bits_equal(got, row0)


@pytest.mark.parametrize("name", sorted(n for n in META if n.startswith("legacy")))
def test_c_oracle_legacy_layout_matches_reference(orc, name):
    m = META[name]
    for hp in (1, 0):
        got = orc.matmul_legacy(_get(name, "B"), _get(name, "scale"), _get(name, "zp"),
                                _get(name, "corr"), m["N"], m["K"], m["bits"], _get(name, "A"), bool(hp))
        assert bits_equal(got, _get(name, f"C_hp{hp}")), (name, hp)


@pytest.mark.parametrize("name", sorted(n for n in META if n.startswith(("pack", "edge", "nonfinite"))))
def test_numpy_twin_matches_reference_outputs(name):
    from oracle import oracle

    m = META[name]
    for hp in (1, 0):
        want = _get(name, f"C_hp{hp}")
        got = oracle.matmul_np(_get(name, "qweight"), _get(name, "scales"), _get(name, "qzeros"),
                               m["N"], m["K"], m["bits"], _get(name, "A"), bool(hp))
        assert bits_equal(got, want), (name, hp)


def test_fixture_covers_the_contract():
    """The fixture exercises both widths, both scale dtypes, explicit zero
    points, rows beyond the reference's 8-row chunk and non-finite inputs."""
    bits = {META[n]["bits"] for n in META}
    dtypes = {str(_get(n, "scales").dtype) for n in META if n.startswith("pack")}
    assert bits == {4, 8}
    assert dtypes == {"float16", "float32"}
    assert any(_get(n, "qzeros") is not None for n in META)
    assert any(_get(n, "A").shape[0] > 8 for n in META)
    assert any(not np.all(np.isfinite(_get(n, "A"))) for n in META)


needs_ref = pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref",
                                                                "libref_qmm.so")),
                               reason="reference kernel not built (make -C oracle ref)")


@needs_ref
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("hp", [True, False])
def test_c_oracle_matches_compiled_reference_random(orc, bits, hp):
    from oracle import oracle

    ref = oracle.Ref(threads=2)
    rng = np.random.default_rng(100 + bits + 2 * hp)
    for N, K, rows in ((32, 64, 1), (80, 160, 5), (16, 1024, 12)):
        qw = rng.integers(0, 256, (N, K // 32, 4 * bits), dtype=np.uint8)
        sc = rng.uniform(1e-4, 3e-2, (N, K // 32)).astype(np.float32)
        qz = rng.integers(0, 256, (N, (K // 32 + 1) // 2), dtype=np.uint8) if bits == 4 else None
        A = (rng.normal(size=(rows, K)) * rng.choice([1e-3, 1.0, 100.0], size=(rows, 1))).astype(np.float32)
        want = ref.run(qw, sc, qz, N, K, bits, A, hp)
        assert bits_equal(orc.matmul(qw, sc, qz, N, K, bits, A, hp), want), (N, K, rows)


NATIVE = os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref", "libref_qmm_native.so")
NATIVE_HOST = os.path.join(os.path.dirname(NATIVE), "native_host.txt")


def _this_cpu():
    with open("/proc/cpuinfo") as f:
        for line in f:
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    return None


def _native_usable():
    # The -march=native build runs only on the CPU it was built for.
    return os.path.exists(NATIVE) and os.path.exists(NATIVE_HOST) and \
        open(NATIVE_HOST).read().strip() == _this_cpu()


@pytest.mark.skipif(not _native_usable(), reason="no -march=native reference build for this CPU "
                                                 "(make -C oracle ref-native)")
@pytest.mark.parametrize("name", sorted(META))
def test_native_flag_build_gives_the_golden_bits(name):
    """The golden vectors come from the reference built with an explicit ISA
    level (-march=x86-64-v4 -mavx512vnni -mavx512vbmi -mf16c).  The
    reference's own build line says -march=native (build_kernel.py:17); built
    that way on this host, the same source gives the same bits on every
    golden case: both activation modes, the quantizer's edge blocks, the
    non-finite activations (the q = 0 rule) and the legacy layout."""
    from oracle import oracle

    ref = oracle.Ref(path=NATIVE, threads=2)
    m = META[name]
    N, K, bits = m["N"], m["K"], m["bits"]
    A = _get(name, "A")
    if name.startswith("legacy"):
        B, scale, zp, corr = (_get(name, k) for k in ("B", "scale", "zp", "corr"))
        h = ref.lib.i4_prepack(B.ctypes.data, scale.ctypes.data, None if zp is None else zp.ctypes.data,
                               corr.ctypes.data, N, K, K // 32, bits)
        assert h
    else:
        h = ref.prepack(_get(name, "qweight"), _get(name, "scales"), _get(name, "qzeros"), N, K, bits)
    try:
        for hp in (True, False):
            want = _get(name, f"C_hp{int(hp)}")
            if want is not None:
                assert bits_equal(ref.matmul(h, A, N, hi_prec=hp), want), (name, hp)
        want = _get(name, "C_hp1_row0")
        if want is not None:
            assert bits_equal(ref.matmul(h, A[:1], N, hi_prec=True), want), name
    finally:
        ref.free(h)
