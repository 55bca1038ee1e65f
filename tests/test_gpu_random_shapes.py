"""Seeded random shapes through the device entry points against the oracle,
bit for bit (outputs and argmax).

The kernel a call reaches depends on the rows (decode row groups of 4, 2 or
1 rows, up to 8 of them; the prefill GEMM's 32-, 64- and 128-row
workgroups), K (whether a row group's activation records fit the decode
kernel's staged copy), the column tiles (the routing limit and the GEMM's
width) and the handle (INT4 or INT8, scale grouping, explicit zero points).
Each case draws all of these, so the cases cross those boundaries in
combinations the targeted tests do not spell out.  The seed is fixed: a
failure names its case and reproduces.
"""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu

N_CASES = 128


def _case(i):
    rng = np.random.default_rng(1000 + i)
    bits = int(rng.choice([4, 8]))
    nblk = int(rng.choice([1, 2, 3, 7, 33, 64, 160, 385, 544, 640]))
    K = 32 * nblk
    ntiles = int(rng.choice([1, 3, 16, 20, 64, 129]))
    N = 16 * ntiles
    # Rows: mostly around the routing boundaries.
    M = int(rng.choice([1, 2, 3, 4, 5, 8, 9, 12, 13, 16, 17, 24, 25, 32, 33, 40, 64, 65, 100, 130]))
    group = int(rng.choice([0, 1, 2, 4]))  # 0: one scale per column; g: groups of g blocks
    zeros = bits == 4 and bool(rng.integers(0, 2))
    hp = bool(rng.integers(0, 4))  # mostly the two-pass mode
    return rng, bits, K, N, M, group, zeros, hp


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape_bit_exact(gpu, hb, orc, hi_prec, i):
    rng, bits, K, N, M, group, zeros, hp = _case(i)
    nblk = K // 32
    qw, sc, qz = rng_weights(rng, N, K, bits, explicit_zeros=zeros)
    if group == 0:
        sc = np.repeat(sc[:, :1], nblk, axis=1)
    elif group > 1:
        sc = np.repeat(sc[:, ::group], group, axis=1)[:, :nblk]
    sc = np.ascontiguousarray(sc)
    A = rng.normal(size=(M, K)).astype(np.float32)
    A[rng.random(A.shape) < 0.01] *= 20.0
    case = dict(i=i, bits=bits, K=K, N=N, M=M, group=group, zeros=zeros, hp=hp)
    print(f"random shape {case}", flush=True)
    hb.set_hi_prec(hp)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
        got, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
        gpu.cuda.synchronize()
        assert bits_equal(got.cpu().numpy(), want), case
        assert idx.cpu().numpy().tolist() == np.argmax(want, axis=1).tolist(), case
    finally:
        hb.free(h)
