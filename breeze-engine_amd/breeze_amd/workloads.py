"""Seeded synthetic inputs of the five benchmark workloads (and a W4
prefill of the same shape as the W8 one).

MatMulNBits weights and activations drawn exactly as the benchmark
specification prescribes (one ``numpy.random.default_rng(seed)`` stream per
workload, drawn in a fixed order), plus the algorithmic byte and operation
counts the roofline figures are quoted on.  Shared by ``bench.py`` (the
measured GPU leg) and the parity tests.
"""
import numpy as np

# name: (bits, M, K, N, scale group in 32-blocks (None = per column), seed, outliers)
CONFIGS = {
    "w8_gemv": (8, 1, 4096, 4096, None, 1, False),
    "w4_gemv": (4, 1, 4096, 12288, 4, 2, False),
    "w4_decode": (4, 8, 12288, 4096, 4, 3, True),
    "w8_prefill": (8, 512, 5120, 17408, None, 4, False),
    "w8_lmhead": (8, 1, 5120, 151936, None, 5, False),
    # Not benchmark workloads: the W4 counterpart of the prefill GEMM; two
    # tall-skinny decode shapes (few column tiles over a long K: a 64-column
    # projection of the MLP's 17408-wide activation, a 48-column one of a
    # 12288-wide activation, and a W8 64-column one over K = 32768, long
    # enough for split-K); and the decoder MLP's gate/up and down widths.
    "w4_prefill": (4, 512, 5120, 17408, 4, 6, False),
    "w4_skinny_k17408": (4, 1, 17408, 64, 4, 7, False),
    "w4_skinny_k12288": (4, 1, 12288, 48, 4, 8, False),
    "w4_mlp_up": (4, 1, 5120, 17408, 4, 9, False),
    "w4_mlp_down": (4, 1, 17408, 5120, 4, 10, False),
    "w8_skinny_k32768": (8, 1, 32768, 64, None, 11, False),
}

LABELS = {
    "w8_gemv": "W8 GEMV M=1 K=4096 N=4096, per-channel scales",
    "w4_gemv": "W4 GEMV M=1 K=4096 N=12288, group-128 scales",
    "w4_decode": "W4 decode M={M} K=12288 N=4096, group-128 scales, 1% x20 outliers",
    "w8_prefill": "W8 prefill M={M} K=5120 N=17408, per-channel scales",
    "w8_lmhead": "W8 LM head M=1 K=5120 N=151936 + argmax, per-channel scales",
    "w4_prefill": "W4 prefill M={M} K=5120 N=17408, group-128 scales",
    "w4_skinny_k17408": "W4 tall-skinny M={M} K=17408 N=64, group-128 scales",
    "w4_skinny_k12288": "W4 tall-skinny M={M} K=12288 N=48, group-128 scales",
    "w4_mlp_up": "W4 MLP gate/up width M={M} K=5120 N=17408, group-128 scales",
    "w4_mlp_down": "W4 MLP down width M={M} K=17408 N=5120, group-128 scales",
    "w8_skinny_k32768": "W8 tall-skinny M={M} K=32768 N=64 (split-K), per-channel scales",
}


def make_weights(rng, bits, N, K, group):
    """Seeded MatMulNBits weights and fp32 [N, K/32] scales.

    W8: w uniform in [-127,127] stored as uint8 w+128 (zero point 128);
        scales |N(0,0.02)|/127 per column, repeated over the K/32 blocks.
    W4: w uniform in [-8,7] stored as nibbles w+8, low nibble = even k;
        scales |N(0,0.02)|/7 per (column, group of `group` blocks)."""
    nblk = K // 32
    if bits == 8:
        w = rng.integers(-127, 128, (N, K), dtype=np.int16)
        qweight = (w + 128).astype(np.uint8).reshape(N, nblk, 32)
        s = (np.abs(rng.normal(0.0, 0.02, N)) / 127).astype(np.float32)
        scales = np.ascontiguousarray(np.repeat(s[:, None], nblk, axis=1))
    else:
        w = rng.integers(-8, 8, (N, K), dtype=np.int16)
        nib = (w + 8).astype(np.uint8)
        qweight = np.ascontiguousarray((nib[:, 0::2] | (nib[:, 1::2] << 4)).reshape(N, nblk, 16))
        if group is None:
            g = (np.abs(rng.normal(0.0, 0.02, N)) / 7).astype(np.float32)
            scales = np.ascontiguousarray(np.repeat(g[:, None], nblk, axis=1))
        else:
            g = (np.abs(rng.normal(0.0, 0.02, (N, nblk // group))) / 7).astype(np.float32)
            scales = np.ascontiguousarray(np.repeat(g, group, axis=1))
    return qweight, scales


def make_config(name, rows=None):
    """Inputs of one workload: dict(qweight, scales, qzeros=None, A, bits, K, N).

    The W4 decode workload draws 8 rows (and its 1% x20 outliers) once and
    keeps the first `rows`; the one-row shapes below the benchmark workloads
    draw `rows` rows."""
    bits, M, K, N, group, seed, outliers = CONFIGS[name]
    if rows is not None and rows > M:
        M = rows
    rng = np.random.default_rng(seed)
    qweight, scales = make_weights(rng, bits, N, K, group)
    A = rng.standard_normal((M, K), dtype=np.float32)
    if outliers:
        mask = rng.random((M, K)) < 0.01
        A[mask] *= np.float32(20)
    if rows is not None:
        A = np.ascontiguousarray(A[:rows])
    return dict(qweight=qweight, scales=scales, qzeros=None, A=A, bits=bits, K=K, N=N)


def algorithmic_bytes(name, M=None):
    """Bytes one call must move at least: packed weights, one fp32 per
    distinct scale, fp32 activations in, fp32 outputs out."""
    bits, M0, K, N, group, _, _ = CONFIGS[name]
    M = M0 if M is None else M
    scales = N if group is None else N * (K // 32 // group)
    return N * K * bits // 8 + 4 * scales + 4 * M * K + 4 * M * N


def algorithmic_ops(name, M=None):
    """Integer operations of one call in the two-pass INT16 mode: two int8
    passes (high and low activation bytes) of 2*M*N*K each."""
    _, M0, K, N, _, _, _ = CONFIGS[name]
    M = M0 if M is None else M
    return 2 * 2 * M * N * K
