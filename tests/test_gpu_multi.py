"""Several projections of one activation in one launch (i4_matmul_multi_dev)
against the oracle, bit for bit: the Qwen3.5-27B decoder's in_qkv, in_z,
in_b, in_a (kernel/qwen35_decoder.cpp:285-288; K = 5120, N = 10240, 6144,
48, 48) and q, k, v (334-336; N = 12288, 1024, 1024), odd widths whose
segment boundaries fall inside workgroups, a partial last chunk, one to
thirty-two rows (row groups of four up to 16 rows, of eight from 5), and the
shapes that fall back to one launch per projection (mixed bits, explicit
zero points, more than 16 rows that only the four-row groups could take)."""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def _w4_group128(rng, N, K):
    qw, sc, _ = rng_weights(rng, N, K, 4)
    sc = np.ascontiguousarray(np.repeat(sc[:, ::4], 4, axis=1)[:, :K // 32])
    return qw, sc, None


def _w8_channel(rng, N, K):
    qw, sc, _ = rng_weights(rng, N, K, 8)
    return qw, np.ascontiguousarray(np.repeat(sc[:, :1], K // 32, axis=1)), None


@pytest.mark.parametrize("shape", ["linear_attn", "full_attn", "odd"])
@pytest.mark.parametrize("bits", [4, 8])
def test_multi_projection_bit_exact(gpu, hb, orc, hi_prec, shape, bits):
    torch = gpu
    K, Ns = {"linear_attn": (5120, [10240, 6144, 48, 48]),
             "full_attn": (5120, [12288, 1024, 1024]),
             "odd": (4640, [16, 272, 4096, 48])}[shape]
    rng = np.random.default_rng(len(Ns) * 10 + bits)
    make = _w4_group128 if bits == 4 else _w8_channel
    ws = [make(rng, N, K) for N in Ns]
    hs = [hb.prepack(qw, sc, qz, K, N, bits=bits) for (qw, sc, qz), N in zip(ws, Ns)]
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for M in (1, 2, 3, 5, 8, 12, 16, 24, 32):
                A = rng.normal(size=(M, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                print(f"multi {shape} bits={bits} hp={hp} M={M}", flush=True)
                outs = hb.matmul_multi(hs, torch.from_numpy(A).cuda(), Ns)
                torch.cuda.synchronize()
                for i, ((qw, sc, qz), N) in enumerate(zip(ws, Ns)):
                    want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
                    assert bits_equal(outs[i].cpu().numpy(), want), (shape, hp, M, i)
    finally:
        for h in hs:
            hb.free(h)


@pytest.mark.parametrize("case", ["mixed_bits", "explicit_zeros", "rows_20", "single"])
def test_multi_projection_fallbacks(gpu, hb, orc, hi_prec, case):
    """Shapes one decode launch does not take run one launch per projection
    and give the same bits."""
    torch = gpu
    K = 1024
    rng = np.random.default_rng(sum(map(ord, case)))
    if case == "mixed_bits":
        specs = [(4, 256, False), (8, 128, False)]
    elif case == "explicit_zeros":
        specs = [(4, 256, True), (4, 64, True)]
    elif case == "single":
        specs = [(4, 512, False)]
    else:
        specs = [(8, 256, False), (8, 96, False), (8, 32, False)]
    M = 20 if case == "rows_20" else 4
    ws = [rng_weights(rng, N, K, b, np.float32, z) for b, N, z in specs]
    hs = [hb.prepack(qw, sc, qz, K, N, bits=b) for (qw, sc, qz), (b, N, _) in zip(ws, specs)]
    try:
        hb.set_hi_prec(True)
        A = rng.normal(size=(M, K)).astype(np.float32)
        outs = hb.matmul_multi(hs, torch.from_numpy(A).cuda(), [N for _, N, _ in specs])
        torch.cuda.synchronize()
        for i, ((qw, sc, qz), (b, N, _)) in enumerate(zip(ws, specs)):
            assert bits_equal(outs[i].cpu().numpy(), orc.matmul(qw, sc, qz, N, K, b, A, True)), (case, i)
    finally:
        for h in hs:
            hb.free(h)


def test_multi_projection_rejects_bad_calls(gpu, hb, hi_prec):
    torch = gpu
    rng = np.random.default_rng(3)
    qw, sc, _ = rng_weights(rng, 64, 256, 8)
    qw2, sc2, _ = rng_weights(rng, 64, 512, 8)
    h1 = hb.prepack(qw, sc, None, 256, 64, bits=8)
    h2 = hb.prepack(qw2, sc2, None, 512, 64, bits=8)
    try:
        A = torch.zeros((1, 256), device="cuda")
        with pytest.raises(ValueError):
            hb.matmul_multi([], A, [])
        with pytest.raises(ValueError):
            hb.matmul_multi([h1] * 5, A, [64] * 5)
        with pytest.raises(RuntimeError, match="one K"):
            hb.matmul_multi([h1, h2], A, [64, 64])
    finally:
        hb.free(h1)
        hb.free(h2)
