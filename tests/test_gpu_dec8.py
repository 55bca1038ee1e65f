"""The five-to-eight-row decode kernel (one workgroup per tile range for all
eight rows, records through the register ring, the two-pass bias term
128 * sum(b) summed in the lane) against the oracle, bit for bit, and against
the row-group kernel it replaces for those rows (BREEZE_HIP_DEC8=0).

Shapes cover a padded last chunk (nblk not a multiple of the chunk's
blocks), a tile's K in exactly one phase and in a short last phase, several
tiles per workgroup (more tiles than CUs, so the idle loads of a short last
phase warm the next tile), per-column and grouped scales, INT4 and INT8
weights, both activation modes, and weight bytes at the ends of their ranges
(every column of a tile at -128 / +127, or nibbles at 0 / 15), which put the
bias sums at their extremes.
"""
import os

import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu

# (K, N), all with more than 128 blocks (fewer go to the row-group kernel,
# which quantizes in its prologue): a padded last chunk at both chunk sizes
# (145 blocks); phases that are all full (168 blocks: 42 INT4 or 84 INT8
# chunks, a multiple of 14) on one tile and on three; the C3 shape; more
# tiles than CUs (544 tiles); a long K (the eight rows' scale rows past one
# uint4 per thread).
SHAPES = [(4640, 272), (5376, 16), (5376, 48), (12288, 4096), (5120, 8704), (24576, 64)]


def _run(hb, torch, h, A, N):
    c = hb.matmul(h, torch.from_numpy(A).cuda(), N)
    torch.cuda.synchronize()
    return c.cpu().numpy()


@pytest.mark.parametrize("K,N", SHAPES)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("hp", [True, False])
def test_dec8_bit_exact(gpu, hb, orc, hi_prec, K, N, bits, hp):
    rng = np.random.default_rng(K * 7 + N + bits + (100 if hp else 0))
    nblk = K // 32
    qw, sc, _ = rng_weights(rng, N, K, bits)
    if K >= 4096 and bits == 4:
        sc = np.ascontiguousarray(np.repeat(sc[:, ::4], 4, axis=1)[:, :nblk])  # group 128
    else:
        sc = np.ascontiguousarray(np.repeat(sc[:, :1], nblk, axis=1))  # per column
    # Extreme weight bytes in the first tile: bias sums at both ends.
    if bits == 8:
        qw[0:8] = 0      # raw 0 -> b = -128
        qw[8:16] = 255   # b = +127
    else:
        qw[0:8] = 0x00
        qw[8:16] = 0xFF
    A8 = rng.normal(size=(8, K)).astype(np.float32)
    A8[rng.random(A8.shape) < 0.01] *= 20.0
    hb.set_hi_prec(hp)
    h = hb.prepack(qw, sc, None, K, N, bits=bits)
    try:
        for M in (5, 6, 7, 8):
            if K * N > 4096 * 4096 and M in (6, 7):
                continue  # the large shapes at 5 and 8 rows only
            A = np.ascontiguousarray(A8[:M])
            case = dict(K=K, N=N, bits=bits, hp=hp, M=M)
            print(f"dec8 {case}", flush=True)
            want = orc.matmul(qw, sc, None, N, K, bits, A, hp)
            got = _run(hb, gpu, h, A, N)
            assert bits_equal(got, want), case
            os.environ["BREEZE_HIP_DEC8"] = "0"
            try:
                old = _run(hb, gpu, h, A, N)
            finally:
                del os.environ["BREEZE_HIP_DEC8"]
            assert bits_equal(old, want), case
    finally:
        hb.free(h)


def test_dec8_then_fewer_rows(gpu, hb, orc, hi_prec):
    """Eight rows, then five: rows past M in the shared record buffer are
    rewritten as zeros, so the second call's results do not see the first's."""
    rng = np.random.default_rng(77)
    K, N = 4096, 512
    qw, sc, _ = rng_weights(rng, N, K, 4)
    hb.set_hi_prec(True)
    h = hb.prepack(qw, sc, None, K, N, bits=4)
    try:
        for M in (8, 5, 8):
            A = rng.normal(size=(M, K)).astype(np.float32)
            want = orc.matmul(qw, sc, None, N, K, 4, A, True)
            assert bits_equal(_run(hb, gpu, h, A, N), want), M
    finally:
        hb.free(h)


@pytest.mark.parametrize("K,N", [(4640, 272), (5120, 8704), (12288, 4096), (17408, 80)])
@pytest.mark.parametrize("bits", [4, 8])
def test_dec8_row_groups_bit_exact(gpu, hb, orc, hi_prec, K, N, bits):
    """Up to four row groups of eight rows, their workgroups on one XCD per
    tile range (512 tiles) or not (17, 5 tiles); a partial last group at 9,
    17 and 27 rows; K = 17408, whose records the four-row groups cannot hold
    past 16 rows."""
    rng = np.random.default_rng(K + N + bits)
    nblk = K // 32
    qw, sc, _ = rng_weights(rng, N, K, bits)
    sc = np.ascontiguousarray(np.repeat(sc[:, :1], nblk, axis=1))
    A32 = rng.normal(size=(32, K)).astype(np.float32)
    A32[rng.random(A32.shape) < 0.01] *= 20.0
    h = hb.prepack(qw, sc, None, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for M in (9, 16, 17, 27, 32):
                A = np.ascontiguousarray(A32[:M])
                case = dict(K=K, N=N, bits=bits, hp=hp, M=M)
                print(f"dec8 row groups {case}", flush=True)
                want = orc.matmul(qw, sc, None, N, K, bits, A, hp)
                assert bits_equal(_run(hb, gpu, h, A, N), want), case
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("hp", [True, False])
def test_dec8_argmax(gpu, hb, orc, hi_prec, bits, hp):
    """The in-kernel argmax at 5-12 rows (LM-head batches), several tiles
    per workgroup: outputs bit-exact and indices equal to the first maximum,
    with two identical columns (5 and 9000) holding every row's maximum, so
    the tie must resolve to the lower index across workgroups.  Calls repeat
    on one stream, so the re-armed keys and ticket are exercised."""
    rng = np.random.default_rng(31 + bits + (10 if hp else 0))
    K, N = 5120, 16 * 600
    nblk = K // 32
    qw, sc, _ = rng_weights(rng, N, K, bits)
    sc = np.ascontiguousarray(np.repeat(sc[:, :1], nblk, axis=1))
    top = 0xFF if bits == 4 else 255  # nibbles 15 / raw 255: the largest weights
    qw[5] = top
    qw[9000] = top
    sc[5] = sc[9000] = 0.02
    h = hb.prepack(qw, sc, None, K, N, bits=bits)
    hb.set_hi_prec(hp)
    try:
        for M in (5, 8, 12, 8):
            A = np.abs(rng.normal(size=(M, K))).astype(np.float32)
            want = orc.matmul(qw, sc, None, N, K, bits, A, hp)
            got, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
            gpu.cuda.synchronize()
            case = dict(bits=bits, hp=hp, M=M)
            assert bits_equal(got.cpu().numpy(), want), case
            assert (want[:, 5] == want[:, 9000]).all() and np.argmax(want, axis=1).tolist() == [5] * M, case
            assert idx.cpu().numpy().tolist() == [5] * M, case
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits,rows", [(8, 16), (4, 32)])
def test_dec8_wide_limit(gpu, hb, orc, hi_prec, bits, rows):
    """The widths where the eight-row groups take more rows than the
    four-row groups did before the GEMM: W8 at 1088 tiles up to 16 rows, W4
    at 1088 tiles up to 32."""
    rng = np.random.default_rng(50 + bits)
    K, N = 5120, 17408
    nblk = K // 32
    qw, sc, _ = rng_weights(rng, N, K, bits)
    sc = np.ascontiguousarray(np.repeat(sc[:, :1], nblk, axis=1))
    A = rng.normal(size=(rows, K)).astype(np.float32)
    hb.set_hi_prec(True)
    h = hb.prepack(qw, sc, None, K, N, bits=bits)
    try:
        want = orc.matmul(qw, sc, None, N, K, bits, A, True)
        assert bits_equal(_run(hb, gpu, h, A, N), want)
    finally:
        hb.free(h)


@pytest.mark.parametrize("kind", ["zeros", "group2", "legacy4", "legacy8"])
def test_dec8_per_block_metadata(gpu, hb, orc, hi_prec, kind):
    """Handles with per-block metadata through the eight-row groups (K past
    4096, 5 to 32 rows): explicit INT4 zero points (the block's zero point
    times -sum(q) of the row), INT4 scales per two blocks (smaller than a
    chunk, so per-block scales), and legacy handles whose corr disagrees with
    the weights (the corr delta, 256 per unit in the two-pass mode), INT4
    with zero points and INT8.  600 tiles, so workgroups hold several tiles
    and copy their records into LDS.  Both activation modes, against the
    oracle and against the four-row groups (BREEZE_HIP_DEC8=0)."""
    rng = np.random.default_rng(sum(map(ord, kind)))
    N, K = 16 * 600, 4640
    nblk = K // 32
    if kind in ("zeros", "group2"):
        bits = 4
        qw, sc, qz = rng_weights(rng, N, K, 4, explicit_zeros=kind == "zeros")
        if kind == "group2":
            sc = np.ascontiguousarray(np.repeat(sc[:, ::2], 2, axis=1)[:, :nblk])
        h = hb.prepack(qw, sc, qz, K, N, bits=4)
        want_of = lambda A, hp: orc.matmul(qw, sc, qz, N, K, 4, A, hp)
    else:
        bits = 4 if kind == "legacy4" else 8
        gb = 64 if bits == 8 else 32
        B = rng.integers(0, 256, (N // 16, nblk, 8, gb), dtype=np.uint8)
        scale = rng.uniform(0.001, 0.02, (N // 16, nblk, 16)).astype(np.float32)
        zp = rng.integers(0, 16, (N // 16, nblk, 16), dtype=np.int8) if bits == 4 else None
        corr = rng.integers(-5000, 5000, (N // 16, nblk, 16), dtype=np.int32)
        h = hb._lib.i4_prepack(hb._p(B), hb._p(scale), hb._p(zp), hb._p(corr), N, K, nblk, bits)
        assert h, hb.last_error()
        want_of = lambda A, hp: orc.matmul_legacy(B, scale, zp, corr, N, K, bits, A, hp)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for M in (5, 8, 17, 32):
                A = rng.normal(size=(M, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                case = dict(kind=kind, hp=hp, M=M)
                want = want_of(A, hp)
                assert bits_equal(_run(hb, gpu, h, A, N), want), case
                os.environ["BREEZE_HIP_DEC8"] = "0"
                try:
                    assert bits_equal(_run(hb, gpu, h, A, N), want), case
                finally:
                    del os.environ["BREEZE_HIP_DEC8"]
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits,K", [(8, 5120), (4, 4640)])
def test_dec8_records_in_lds(gpu, hb, orc, hi_prec, bits, K):
    """Workgroups with several tiles copy their records into LDS once
    (where they fit: W8 up to K = 5120, W4 K = 4640): outputs and argmax
    bit-exact against the oracle and against the records read from L2 per
    tile (BREEZE_HIP_DEC8_LREC=0), at 5, 8 and 24 rows (three row groups),
    and through the gate/up pair."""
    rng = np.random.default_rng(K + bits)
    N = 16 * 700  # 700 tiles: 2-3 per workgroup at one row group, more with three
    nblk = K // 32
    qw, sc, _ = rng_weights(rng, N, K, bits)
    sc = np.ascontiguousarray(np.repeat(sc[:, :1], nblk, axis=1))
    qu, su, _ = rng_weights(rng, N, K, bits)
    su = np.ascontiguousarray(np.repeat(su[:, :1], nblk, axis=1))
    h = hb.prepack(qw, sc, None, K, N, bits=bits)
    hu = hb.prepack(qu, su, None, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for M in (5, 8, 24):
                A = rng.normal(size=(M, K)).astype(np.float32)
                want = orc.matmul(qw, sc, None, N, K, bits, A, hp)
                case = dict(bits=bits, K=K, hp=hp, M=M)
                got, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
                pair = hb.matmul_silu_mul(h, hu, gpu.from_numpy(A).cuda(), N)
                os.environ["BREEZE_HIP_DEC8_LREC"] = "0"
                try:
                    got_l2, idx_l2 = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
                    pair_l2 = hb.matmul_silu_mul(h, hu, gpu.from_numpy(A).cuda(), N)
                finally:
                    del os.environ["BREEZE_HIP_DEC8_LREC"]
                gpu.cuda.synchronize()
                assert bits_equal(got.cpu().numpy(), want), case
                assert idx.cpu().numpy().tolist() == np.argmax(want, axis=1).tolist(), case
                assert bits_equal(got_l2.cpu().numpy(), want), case
                assert idx_l2.cpu().numpy().tolist() == idx.cpu().numpy().tolist(), case
                assert bits_equal(pair.cpu().numpy(), pair_l2.cpu().numpy()), case
    finally:
        hb.free(h)
        hb.free(hu)


@pytest.mark.parametrize("bits", [4, 8])
def test_dec8_argmax_long_k(gpu, hb, orc, hi_prec, bits):
    """24 rows over K = 17408 with the argmax: the eight-row groups take the
    call (four rows of records would not fit the four-row groups), and the
    index is the one their in-kernel merge writes (no second argmax launch
    follows the eight-row kernel)."""
    K, N, M = 17408, 16 * 40, 24
    assert hb.plan(bits, M, K, N, argmax=True)["route"] == "decode8"
    rng = np.random.default_rng(90 + bits)
    qw, sc, _ = rng_weights(rng, N, K, bits)
    h = hb.prepack(qw, sc, None, K, N, bits=bits)
    try:
        hb.set_hi_prec(True)
        A = rng.normal(size=(M, K)).astype(np.float32)
        want = orc.matmul(qw, sc, None, N, K, bits, A, True)
        c, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
        gpu.cuda.synchronize()
        assert bits_equal(c.cpu().numpy(), want)
        assert idx.cpu().tolist() == np.argmax(want, axis=1).tolist()
    finally:
        hb.free(h)
