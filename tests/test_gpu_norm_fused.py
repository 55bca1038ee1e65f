"""The decoder's RMSNorm in the prologue of the projection launch
(i4_rmsnorm_matmul_multi_dev) against the oracle's two steps, bit for bit:
hn = rmsnorm(x, w, eps) (kernel/qwen35_decoder.cpp:134-140) and each
projection of hn.  The Qwen3.5-27B in_qkv/in_z/in_b/in_a shapes (K = 5120)
at one and two rows take the fused launch, three, four and eight rows the
norm-then-projections fallback (past 384 row-blocks the norm runs as its
own launch); rows from the RMSNorm parity set
(ties, vanishing terms, outliers, denormals, a mean on a float rounding
midpoint that the bound leaves to the in-order sum) at K = 4096 one at a
time, and all together at K = 3072 (row groups of 4 x 96 blocks, fused);
each case as shipped and with BREEZE_HIP_NORM_EXACT=1 (every row through
the in-order sum)."""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights
from test_gpu_rmsnorm import _rows, _same

pytestmark = pytest.mark.gpu

F = np.float32


def _weights(rng, bits, N, K):
    qw, sc, _ = rng_weights(rng, N, K, bits)
    if bits == 4:
        sc = np.repeat(sc[:, ::4], 4, axis=1)[:, :K // 32]
    return qw, np.ascontiguousarray(sc)


@pytest.mark.parametrize("mode", ["auto", "exact"])
@pytest.mark.parametrize("bits", [4, 8])
def test_norm_then_projections_bit_exact(gpu, hb, orc, hi_prec, monkeypatch, mode, bits):
    torch = gpu
    if mode == "exact":
        monkeypatch.setenv("BREEZE_HIP_NORM_EXACT", "1")
    K, Ns = 5120, [10240, 6144, 48, 48]
    rng = np.random.default_rng(bits)
    ws = [_weights(rng, bits, N, K) for N in Ns]
    hs = [hb.prepack(qw, sc, None, K, N, bits=bits) for (qw, sc), N in zip(ws, Ns)]
    ln = (1 + 0.1 * rng.standard_normal(K)).astype(F)
    try:
        hb.set_hi_prec(True)
        for M in (1, 2, 3, 4, 8):
            x = (rng.standard_normal((M, K)) * 3).astype(F)
            x[rng.random(x.shape) < 0.01] *= 20
            print(f"norm+multi bits={bits} mode={mode} M={M}", flush=True)
            outs, hn = hb.rmsnorm_matmul_multi(torch.from_numpy(x).cuda(), torch.from_numpy(ln).cuda(), 1e-6, hs,
                                               Ns, want_hn=True)
            torch.cuda.synchronize()
            hn_ref = orc.rmsnorm(x, ln, F(1e-6))
            assert bits_equal(hn.cpu().numpy(), hn_ref), (M, "hn")
            for i, ((qw, sc), N) in enumerate(zip(ws, Ns)):
                assert bits_equal(outs[i].cpu().numpy(), orc.matmul(qw, sc, None, N, K, bits, hn_ref, True)), (M, i)
    finally:
        for h in hs:
            hb.free(h)


@pytest.mark.parametrize("mode", ["auto", "exact"])
def test_norm_in_prologue_adversarial_rows(gpu, hb, orc, hi_prec, monkeypatch, mode):
    """Each row of the RMSNorm parity set alone (one row: the fused
    launch) at K = 4096, and the whole set at once at K = 3072 (row groups
    of four, fused), one W4 and one W8 projection, three eps values.  hn
    and the projections match the oracle outside NaNs, which appear at the
    same places (non-finite rows)."""
    torch = gpu
    if mode == "exact":
        monkeypatch.setenv("BREEZE_HIP_NORM_EXACT", "1")
    K = 4096
    rng = np.random.default_rng(5)
    w4, w8 = _weights(rng, 4, 64, K), _weights(rng, 8, 32, K)
    h4 = hb.prepack(*w4, None, K, 64, bits=4)
    h8 = hb.prepack(*w8, None, K, 32, bits=8)
    ln = rng.standard_normal(K).astype(F)
    K2 = 3072
    v4, v8 = _weights(rng, 4, 64, K2), _weights(rng, 8, 32, K2)
    g4 = hb.prepack(*v4, None, K2, 64, bits=4)
    g8 = hb.prepack(*v8, None, K2, 32, bits=8)
    ln2 = rng.standard_normal(K2).astype(F)
    rows2 = _rows(K2, K2)
    try:
        hb.set_hi_prec(True)
        rows = _rows(K, K)
        for eps in (F(1e-6), F(0.0), F(1e-2)):
            for r in range(rows.shape[0]):
                x = rows[r:r + 1]
                with np.errstate(all="ignore"):
                    hn_ref = orc.rmsnorm(x, ln, eps)
                outs, hn = hb.rmsnorm_matmul_multi(torch.from_numpy(x).cuda(), torch.from_numpy(ln).cuda(),
                                                   float(eps), [h4, h8], [64, 32], want_hn=True)
                torch.cuda.synchronize()
                assert _same(hn.cpu().numpy(), hn_ref), (r, eps)
                if np.all(np.isfinite(hn_ref)):
                    assert bits_equal(outs[0].cpu().numpy(), orc.matmul(*w4, None, 64, K, 4, hn_ref, True)), (r, eps)
                    assert bits_equal(outs[1].cpu().numpy(), orc.matmul(*w8, None, 32, K, 8, hn_ref, True)), (r, eps)
            # All the rows at once at K = 3072: four row groups of 4 (4 x 96
            # row-blocks each), each normalizing its own rows in the
            # prologue of the one launch.
            with np.errstate(all="ignore"):
                hn_ref = orc.rmsnorm(rows2, ln2, eps)
            outs, hn = hb.rmsnorm_matmul_multi(torch.from_numpy(rows2).cuda(), torch.from_numpy(ln2).cuda(),
                                               float(eps), [g4, g8], [64, 32], want_hn=True)
            torch.cuda.synchronize()
            assert _same(hn.cpu().numpy(), hn_ref), ("all rows", eps)
            fin = np.all(np.isfinite(hn_ref), axis=1)
            assert bits_equal(outs[0].cpu().numpy()[fin], orc.matmul(*v4, None, 64, K2, 4, hn_ref[fin], True)), eps
            assert bits_equal(outs[1].cpu().numpy()[fin], orc.matmul(*v8, None, 32, K2, 8, hn_ref[fin], True)), eps
    finally:
        for h in (h4, h8, g4, g8):
            hb.free(h)


def test_norm_fused_without_hn_output(gpu, hb, orc, hi_prec):
    torch = gpu
    K, N = 2048, 256
    rng = np.random.default_rng(9)
    qw, sc = _weights(rng, 4, N, K)
    h = hb.prepack(qw, sc, None, K, N, bits=4)
    try:
        hb.set_hi_prec(False)
        x = rng.standard_normal((2, K)).astype(F)
        ln = rng.standard_normal(K).astype(F)
        outs = hb.rmsnorm_matmul_multi(torch.from_numpy(x).cuda(), torch.from_numpy(ln).cuda(), 1e-5, [h], [N])
        torch.cuda.synchronize()
        hn_ref = orc.rmsnorm(x, ln, F(1e-5))
        assert bits_equal(outs[0].cpu().numpy(), orc.matmul(qw, sc, None, N, K, 4, hn_ref, False))
    finally:
        hb.free(h)
