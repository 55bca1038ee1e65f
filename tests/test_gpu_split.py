"""Split-K decode (a tile's K range spread over several workgroups, the last
one to finish folding every block in order) against the oracle and the
unsplit kernel, bit for bit.

The reference folds a column's per-block values in block order on one core
(kernel/quantized_matmul.cpp:311-315, acc = fma(sa, f, acc)); the split
launch computes the same per-block values on several CUs and folds them in
the same order, so every output keeps the reference's bits.  Cases: the
tall-skinny widths (3 and 4 tiles over K = 12288 and 17408, split where
forced; the default route's own cases at K = 18432 to 40960), one to four
rows, both activation modes, INT8, explicit zero points (per-block
metadata), padded last chunks, forced piece counts (two pieces, one phase
per piece, and counts that leave pieces of unequal length), repeated calls
(the tickets re-arm) and a captured HIP graph replayed between eager calls.
"""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def _acts(rng, M, K):
    A = rng.normal(size=(M, K)).astype(np.float32)
    A[rng.random(A.shape) < 0.01] *= 20.0  # outliers that need the lo byte
    return A


@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
@pytest.mark.parametrize("M,K,N", [(1, 17408, 64), (2, 17408, 64), (1, 12288, 48), (3, 5120, 256),
                                   (4, 12288, 48), (2, 4000, 1024), (1, 4064, 16)])
def test_split_matches_oracle_and_unsplit(gpu, hb, orc, hi_prec, monkeypatch, bits, explicit_zeros, M, K, N):
    torch = gpu
    monkeypatch.setenv("BREEZE_HIP_SPLIT", "1")
    plan = hb.plan(bits, M, K, N, extra=explicit_zeros)
    assert plan["split"] >= 2 and plan["quant"] is None, plan
    rng = np.random.default_rng(M * 131 + K + N + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            A = _acts(rng, M, K)
            dA = torch.from_numpy(A).cuda()
            got = hb.matmul(h, dA, N).cpu().numpy()
            assert bits_equal(got, orc.matmul(qw, sc, qz, N, K, bits, A, hp)), (M, K, N, hp)
            monkeypatch.setenv("BREEZE_HIP_SPLIT", "0")
            assert hb.plan(bits, M, K, N, extra=explicit_zeros)["split"] == 0
            unsplit = hb.matmul(h, dA, N).cpu().numpy()
            monkeypatch.setenv("BREEZE_HIP_SPLIT", "1")
            assert bits_equal(got, unsplit), (M, K, N, hp)
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("pieces", [2, 3, 4, 7, 64])
def test_split_piece_counts(gpu, hb, orc, hi_prec, monkeypatch, bits, pieces):
    """Forced piece counts over one K: two pieces, counts that do not divide
    the phases (pieces of unequal length) and one phase per piece (64 asks
    for more pieces than phases and gets one per phase)."""
    torch = gpu
    M, K, N = 2, 13344, 32  # 417 blocks: a padded last chunk for both widths
    monkeypatch.setenv("BREEZE_HIP_SPLIT", str(pieces))
    plan = hb.plan(bits, M, K, N)
    nbg = -(-417 // (2 if bits == 8 else 4))  # chunks of the 417 blocks
    npw = -(-nbg // 15)  # phases of 15 chunks
    assert plan["split"] == min(pieces, npw), plan
    rng = np.random.default_rng(pieces * 10 + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        hb.set_hi_prec(True)
        A = _acts(rng, M, K)
        got = hb.matmul(h, torch.from_numpy(A).cuda(), N).cpu().numpy()
        assert bits_equal(got, orc.matmul(qw, sc, qz, N, K, bits, A, True)), pieces
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits,M,K,N", [(8, 1, 24576, 64), (8, 2, 32768, 128), (4, 1, 40960, 64), (8, 4, 18432, 16)])
def test_split_default_route(gpu, hb, orc, hi_prec, bits, M, K, N):
    """Tall-skinny calls that split-K takes without any override."""
    torch = gpu
    plan = hb.plan(bits, M, K, N)
    assert plan["split"] >= 20, plan
    rng = np.random.default_rng(K + N + M)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            A = _acts(rng, M, K)
            got = hb.matmul(h, torch.from_numpy(A).cuda(), N).cpu().numpy()
            assert bits_equal(got, orc.matmul(qw, sc, qz, N, K, bits, A, hp)), hp
    finally:
        hb.free(h)


def test_split_repeated_calls_rearm_the_tickets(gpu, hb, orc, hi_prec, monkeypatch):
    """Back-to-back calls without a host synchronization between them, on
    shapes of different tile counts sharing the tickets: each call's last
    workgroup per tile must see only its own call's pieces."""
    torch = gpu
    monkeypatch.setenv("BREEZE_HIP_SPLIT", "1")
    rng = np.random.default_rng(77)
    shapes = [(4, 17408, 64), (4, 12288, 48), (8, 17408, 32)]
    handles = []
    try:
        for bits, K, N in shapes:
            assert hb.plan(bits, 1, K, N)["split"] >= 2
            qw, sc, qz = rng_weights(rng, N, K, bits, np.float32)
            handles.append((hb.prepack(qw, sc, qz, K, N, bits=bits), qw, sc, qz, bits, K, N))
        hb.set_hi_prec(True)
        calls = []
        for rep in range(4):
            for h, qw, sc, qz, bits, K, N in handles:
                A = _acts(rng, 1, K)
                calls.append((hb.matmul(h, torch.from_numpy(A).cuda(), N), A, qw, sc, qz, bits, K, N))
        torch.cuda.synchronize()
        for out, A, qw, sc, qz, bits, K, N in calls:
            assert bits_equal(out.cpu().numpy(), orc.matmul(qw, sc, qz, N, K, bits, A, True)), (bits, K, N)
    finally:
        for h, *_ in handles:
            hb.free(h)


def test_split_in_a_captured_graph(gpu, hb, orc, hi_prec, monkeypatch):
    """A split call captured in a HIP graph (after one eager call sized the
    scratch) replays bit-exact, with eager split calls of another shape
    between the replays."""
    torch = gpu
    monkeypatch.setenv("BREEZE_HIP_SPLIT", "1")
    rng = np.random.default_rng(5)
    K, N, K2, N2 = 17408, 64, 12288, 48
    qw, sc, qz = rng_weights(rng, N, K, 4, np.float32)
    qw2, sc2, qz2 = rng_weights(rng, N2, K2, 4, np.float32)
    h = hb.prepack(qw, sc, qz, K, N, bits=4)
    h2 = hb.prepack(qw2, sc2, qz2, K2, N2, bits=4)
    try:
        hb.set_hi_prec(True)
        dA = torch.from_numpy(_acts(rng, 1, K)).cuda()
        hb.matmul(h, dA, N)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            hb.matmul(h, dA, N)  # sizes the side stream's scratch before capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out = hb.matmul(h, dA, N)
        for rep in range(4):
            A = _acts(rng, 1, K)
            dA.copy_(torch.from_numpy(A))
            graph.replay()
            torch.cuda.synchronize()
            assert bits_equal(out.cpu().numpy(), orc.matmul(qw, sc, qz, N, K, 4, A, True)), rep
            A2 = _acts(rng, 1, K2)
            got2 = hb.matmul(h2, torch.from_numpy(A2).cuda(), N2).cpu().numpy()
            assert bits_equal(got2, orc.matmul(qw2, sc2, qz2, N2, K2, 4, A2, True)), rep
    finally:
        hb.free(h)
        hb.free(h2)
