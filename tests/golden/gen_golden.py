"""Writes tests/golden/ref_vectors.npz: inputs and outputs of the reference
CPU kernel (kernel/quantized_matmul.cpp of breeze-engine, compiled from its
own source by `make -C oracle ref` into oracle/_ref/libref_qmm.so) on small
seeded cases.  Run in a checkout where that library is built:

    python tests/golden/gen_golden.py

The fixture holds only data.  Cases:
  pack_*    MatMulNBits weights in the shapes, dtypes and zero-point
            options of the reference's packing tests
            (tests/test_cpu_packing.py:33-53, 70-96), edge bytes forced,
            rows 1 and 9, both activation modes;
  proj_*    the projection widths and seed of tests/test_qwen35_cpu.py:196-208
            (three rows, high-precision mode);
  edge_*    activation blocks that hit the quantizer's special cases: all
            zero, constant, exact .5 ties, subnormal, mixed magnitudes,
            values near FLT_MAX, negative maxima, and (in their own case)
            NaN and infinity;
  legacy_*  the pre-transformed layout entry point i4_prepack with random
            corr (kernel/benchmark_matmul.cpp:28 passes it).
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402

OUT = os.path.join(HERE, "ref_vectors.npz")


def fixture_weights(N, K, bits, dtype, explicit_zeros):
    """Seeded weights with forced edge bytes (same recipe as the packing
    tests of the reference: seed N+K+bits, first bytes 0,1,7,15,127,128,254,255)."""
    rng = np.random.default_rng(N + K + bits)
    blocks = K // 32
    qw = rng.integers(0, 256, (N, blocks, 4 * bits), dtype=np.uint8)
    qw.reshape(-1)[:8] = [0, 1, 7, 15, 127, 128, 254, 255]
    scales = rng.uniform(0.0001, 0.02, (N, blocks)).astype(dtype)
    zeros = None
    if explicit_zeros and bits == 4:
        zeros = rng.integers(0, 256, (N, (blocks + 1) // 2), dtype=np.uint8)
    return qw, scales, zeros


def edge_activations(K, rows, finite=True):
    """Rows of 32-blocks that each exercise one quantizer case."""
    rng = np.random.default_rng(77)
    A = rng.normal(size=(rows, K)).astype(np.float32)
    nblk = K // 32
    for r in range(rows):
        for j in range(nblk):
            kind = (r * nblk + j) % 9
            blk = A[r, 32 * j:32 * j + 32]
            if kind == 0:
                blk[:] = 0.0
            elif kind == 1:
                blk[:] = np.float32(3.0) * (1 if r % 2 == 0 else -1)
            elif kind == 2:
                # amax 32767 (hi-prec scale exactly 1) and 127 in the same
                # row-block family: .5 products round to even.
                blk[:] = np.arange(32, dtype=np.float32) - np.float32(15.5)
                blk[0] = np.float32(32767.0 if r % 2 == 0 else 127.0)
            elif kind == 3:
                blk[:] = rng.uniform(-1, 1, 32).astype(np.float32) * np.float32(1e-40)
            elif kind == 4:
                blk[:] = rng.normal(size=32).astype(np.float32) * np.float32(1e-30)
                blk[5] = np.float32(1e30)
            elif kind == 5:
                blk[:] = rng.uniform(-1, 1, 32).astype(np.float32) * np.float32(3.0e38)
            elif kind == 6:
                blk[:] = rng.uniform(-1, 0.5, 32).astype(np.float32)
                blk[7] = np.float32(-2.75)
            elif kind == 7:
                blk[:] = np.float32(1.0) / np.float32(3.0) * (np.arange(32) % 3 - 1)
            # kind 8: keep the random normals
            if not finite and kind in (2, 6):
                blk[3] = np.nan if kind == 2 else np.inf
                blk[9] = -np.inf if kind == 6 else blk[9]
    return A


def main():
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libref_qmm.so is missing: run `make -C oracle ref` first")
    ref = oracle.Ref(threads=1)
    out = {}
    meta = {}

    def put(prefix, **arrays):
        for k, v in arrays.items():
            if v is not None:
                out[f"{prefix}_{k}"] = np.ascontiguousarray(v)

    i = 0
    for N, K in ((16, 32), (48, 96), (64, 512)):
        for bits in (4, 8):
            for dtype in (np.float16, np.float32):
                for zeros in ((False, True) if bits == 4 else (False,)):
                    qw, sc, qz = fixture_weights(N, K, bits, dtype, zeros)
                    rng = np.random.default_rng(1000 + i)
                    A = rng.normal(size=(9, K)).astype(np.float32)
                    h = ref.prepack(qw, sc, qz, N, K, bits)
                    try:
                        c1 = ref.matmul(h, A, N, hi_prec=True)
                        c0 = ref.matmul(h, A, N, hi_prec=False)
                        c1r = ref.matmul(h, A[:1], N, hi_prec=True)
                    finally:
                        ref.free(h)
                    name = f"pack{i}"
                    put(name, qweight=qw, scales=sc, qzeros=qz, A=A, C_hp1=c1, C_hp0=c0, C_hp1_row0=c1r)
                    meta[name] = dict(N=N, K=K, bits=bits)
                    i += 1

    for j, (K, N, bits) in enumerate(((5120, 48, 8), (17408, 16, 4), (6144, 64, 8), (4096, 32, 4))):
        rng = np.random.default_rng(3)
        qw = rng.integers(0, 256, (N, K // 32, 32 * bits // 8), dtype=np.uint8)
        sc = rng.uniform(0.001, 0.005, (N, K // 32)).astype(np.float32)
        A = rng.normal(size=(3, K)).astype(np.float32)
        name = f"proj{j}"
        put(name, qweight=qw, scales=sc, A=A, C_hp1=ref.run(qw, sc, None, N, K, bits, A, True))
        meta[name] = dict(N=N, K=K, bits=bits)

    for j, (bits, finite) in enumerate(((4, True), (8, True), (4, False), (8, False))):
        N, K = 32, 288
        qw, sc, _ = fixture_weights(N, K, bits, np.float32, False)
        A = edge_activations(K, 4, finite)
        name = f"edge{j}" if finite else f"nonfinite{j}"
        put(name, qweight=qw, scales=sc, A=A, C_hp1=ref.run(qw, sc, None, N, K, bits, A, True),
            C_hp0=ref.run(qw, sc, None, N, K, bits, A, False))
        meta[name] = dict(N=N, K=K, bits=bits)

    for j, bits in enumerate((4, 8)):
        N, K = 32, 128
        nblk = K // 32
        rng = np.random.default_rng(21 + j)
        gb = 64 if bits == 8 else 32
        B = rng.integers(0, 256, (N // 16, nblk, 8, gb), dtype=np.uint8)
        scale = rng.uniform(0.001, 0.02, (N // 16, nblk, 16)).astype(np.float32)
        zp = rng.integers(0, 16, (N // 16, nblk, 16), dtype=np.int8) if bits == 4 else None
        corr = rng.integers(-5000, 5000, (N // 16, nblk, 16), dtype=np.int32)
        A = rng.normal(size=(5, K)).astype(np.float32)
        zp_p = zp.ctypes.data if zp is not None else None
        h = ref.lib.i4_prepack(B.ctypes.data, scale.ctypes.data, zp_p, corr.ctypes.data, N, K, nblk, bits)
        assert h
        try:
            c1 = ref.matmul(h, A, N, hi_prec=True)
            c0 = ref.matmul(h, A, N, hi_prec=False)
        finally:
            ref.free(h)
        name = f"legacy{j}"
        put(name, B=B, scale=scale, zp=zp, corr=corr, A=A, C_hp1=c1, C_hp0=c0)
        meta[name] = dict(N=N, K=K, bits=bits)

    out["meta"] = np.frombuffer(json.dumps(meta, sort_keys=True).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(meta)} cases, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
