"""Seeded random shapes through the decoder's fused calls against the oracle.

- i4_matmul_multi_dev: every projection bit for bit equal to the oracle's
  matmul of the one activation;
- i4_rmsnorm_matmul_multi_dev: hn and every projection of hn bit for bit
  equal to the oracle's rmsnorm then matmul (kernel/qwen35_decoder.cpp:
  134-140, 285-288);
- i4_matmul_silu_mul_dev: bit for bit the oracle's silu(gate) * up of its
  two projections, formed with the host C library's expf as the reference
  forms it (qwen35_decoder.cpp:128, 406-408).

Each case draws the kind, bits, K, the number of handles and their widths,
the rows, the scale grouping and the activation mode, so the cases cross
the one-launch limits (rows, row-blocks the prologue quantizes, the staged
record sizes) and the fallbacks in combinations the targeted tests do not
spell out.  The seed is fixed: a failure names its case and reproduces.
"""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu

N_CASES = 96
F = np.float32


def _case(i):
    rng = np.random.default_rng(5000 + i)
    kind = ("multi", "norm", "pair")[i % 3]
    bits = int(rng.choice([4, 8]))
    nblk = int(rng.choice([1, 3, 7, 33, 64, 128, 160, 385]))
    K = 32 * nblk
    n = 2 if kind == "pair" else int(rng.integers(1, 5))
    tiles = [int(rng.choice([1, 3, 16, 64, 129])) for _ in range(n)]
    if kind == "pair":
        tiles[1] = tiles[0]
    Ns = [16 * t for t in tiles]
    M = int(rng.choice([1, 2, 3, 4, 5, 8, 9, 12, 16, 17, 20]))
    group = int(rng.choice([0, 1, 4]))  # 0: one scale per column; g: groups of g blocks
    hp = bool(rng.integers(0, 4))  # mostly the two-pass mode
    return rng, kind, bits, K, Ns, M, group, hp


def _weights(rng, bits, N, K, group):
    qw, sc, _ = rng_weights(rng, N, K, bits)
    nblk = K // 32
    if group == 0:
        sc = np.repeat(sc[:, :1], nblk, axis=1)
    elif group > 1:
        sc = np.repeat(sc[:, ::group], group, axis=1)[:, :nblk]
    return qw, np.ascontiguousarray(sc)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_fused_call(gpu, hb, orc, hi_prec, i):
    torch = gpu
    rng, kind, bits, K, Ns, M, group, hp = _case(i)
    case = dict(i=i, kind=kind, bits=bits, K=K, Ns=Ns, M=M, group=group, hp=hp)
    print(f"random fused {case}", flush=True)
    ws = [_weights(rng, bits, N, K, group) for N in Ns]
    hb.set_hi_prec(hp)
    hs = [hb.prepack(qw, sc, None, K, N, bits=bits) for (qw, sc), N in zip(ws, Ns)]
    try:
        A = (rng.standard_normal((M, K)) * 2).astype(F)
        A[rng.random(A.shape) < 0.01] *= 20.0
        dA = torch.from_numpy(A).cuda()
        if kind == "multi":
            outs = hb.matmul_multi(hs, dA, Ns)
            torch.cuda.synchronize()
            for k, ((qw, sc), N) in enumerate(zip(ws, Ns)):
                assert bits_equal(outs[k].cpu().numpy(), orc.matmul(qw, sc, None, N, K, bits, A, hp)), (case, k)
        elif kind == "norm":
            ln = (1 + 0.1 * rng.standard_normal(K)).astype(F)
            outs, hn = hb.rmsnorm_matmul_multi(dA, torch.from_numpy(ln).cuda(), 1e-6, hs, Ns, want_hn=True)
            torch.cuda.synchronize()
            hn_ref = orc.rmsnorm(A, ln, F(1e-6))
            assert bits_equal(hn.cpu().numpy(), hn_ref), (case, "hn")
            for k, ((qw, sc), N) in enumerate(zip(ws, Ns)):
                assert bits_equal(outs[k].cpu().numpy(), orc.matmul(qw, sc, None, N, K, bits, hn_ref, hp)), (case, k)
        else:
            (qg, sg), (qu, su) = ws
            got = hb.matmul_silu_mul(hs[0], hs[1], dA, Ns[0]).cpu().numpy()
            g = orc.matmul(qg, sg, None, Ns[0], K, bits, A, hp)
            u = orc.matmul(qu, su, None, Ns[0], K, bits, A, hp)
            assert bits_equal(got, orc.silu_mul(g, u)), case
    finally:
        for h in hs:
            hb.free(h)
