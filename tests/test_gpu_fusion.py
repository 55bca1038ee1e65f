"""The fused gate/up projection of a decoder MLP (i4_matmul_silu_mul_dev),
replacing kernel/qwen35_decoder.cpp:406-408: g1 = i4_matmul(gate), g2 =
i4_matmul(up), g1 = siluf(g1) * g2 with siluf(x) = x / (1 + exp(-x)).

Both projections are the exact path (bit-identical to the oracle), so the
result is compared with the oracle's projections through float32 SiLU and
product: the only difference allowed is exp's last-place rounding (the
device expf against numpy's), bounded here at 1e-6 relative.  The one-launch
path (handles of the same layout; up to 16 rows on the four-row groups, 32 on
the eight-row groups) and the two-launch fallback use the same device
arithmetic and must agree bit for bit."""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def _silu_mul(g, u):
    g = g.astype(np.float32)
    return (g / (np.float32(1) + np.exp(-g))) * u.astype(np.float32)


def _group4(s):
    """One scale per 4 blocks (128-element groups): the layout without
    per-block metadata."""
    g = np.repeat(s[:, ::4], 4, axis=1)[:, : s.shape[1]]
    return np.ascontiguousarray(g)


def _pair(hb, rng, N, K, bits, explicit_zeros, same_layout=True, grouped=False):
    qg, sg, zg = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    qu, su, zu = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    if grouped:
        sg, su = _group4(sg), _group4(su)
    if not same_layout:
        su = np.repeat(su[:, :1], su.shape[1], axis=1)  # per-column scales: another device layout
    return (qg, sg, zg), (qu, su, zu), hb.prepack(qg, sg, zg, K, N, bits=bits), hb.prepack(qu, su, zu, K, N, bits=bits)


@pytest.mark.parametrize("bits,explicit_zeros,grouped", [(4, False, True), (8, False, True),
                                                         (4, False, False), (4, True, False), (8, False, False)])
@pytest.mark.parametrize("N,K", [(64, 224), (16 * 1029, 768), (512, 4096), (16 * 100, 5120)])
def test_fused_gate_up_matches_the_composition(gpu, hb, orc, hi_prec, monkeypatch, bits, explicit_zeros, grouped,
                                               N, K):
    torch = gpu
    rng = np.random.default_rng(N + K + bits)
    (qg, sg, zg), (qu, su, zu), hg, hu = _pair(hb, rng, N, K, bits, explicit_zeros, grouped=grouped)
    try:
        if grouped:
            assert hb.handle_info(hg)["scale_group"] == 4
        for hp in (False, True):
            hb.set_hi_prec(hp)
            A = (rng.normal(size=(20, K)) * 2).astype(np.float32)
            g = orc.matmul(qg, sg, zg, N, K, bits, A, hp)
            u = orc.matmul(qu, su, zu, N, K, bits, A, hp)
            want = _silu_mul(g, u)
            fused = {}
            for rows in (1, 2, 3, 5, 8, 12, 16):
                got = hb.matmul_silu_mul(hg, hu, torch.from_numpy(A[:rows]).cuda(), N).cpu().numpy()
                np.testing.assert_allclose(got, want[:rows], rtol=1e-6, atol=1e-30, err_msg=f"{rows} rows")
                fused[rows] = got
            # Twenty rows: one launch where the eight-row groups take the
            # call (K past 4096, no per-block metadata), else the two-launch
            # fallback, which BREEZE_HIP_DEC8=0 forces; every way gives the
            # bits of the one-launch rows.
            got20 = hb.matmul_silu_mul(hg, hu, torch.from_numpy(A).cuda(), N).cpu().numpy()
            monkeypatch.setenv("BREEZE_HIP_DEC8", "0")
            two = hb.matmul_silu_mul(hg, hu, torch.from_numpy(A).cuda(), N).cpu().numpy()
            monkeypatch.delenv("BREEZE_HIP_DEC8")
            torch.cuda.synchronize()
            assert bits_equal(got20[:16], fused[16]), hp
            assert bits_equal(got20[:1], fused[1]), hp
            assert bits_equal(two, got20), hp
            np.testing.assert_allclose(got20, want, rtol=1e-6, atol=1e-30)
    finally:
        hb.free(hg)
        hb.free(hu)


def test_fused_gate_up_with_different_layouts_and_bad_shapes(gpu, hb, orc, hi_prec):
    torch = gpu
    rng = np.random.default_rng(9)
    N, K = 128, 512
    (qg, sg, zg), (qu, su, zu), hg, hu = _pair(hb, rng, N, K, 4, False, same_layout=False)
    other = hb.prepack(*rng_weights(rng, 2 * N, K, 4)[:2], None, K, 2 * N, bits=4)
    try:
        hb.set_hi_prec(True)
        A = rng.normal(size=(2, K)).astype(np.float32)
        got = hb.matmul_silu_mul(hg, hu, torch.from_numpy(A).cuda(), N).cpu().numpy()
        want = _silu_mul(orc.matmul(qg, sg, zg, N, K, 4, A, True), orc.matmul(qu, su, zu, N, K, 4, A, True))
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-30)
        with pytest.raises(RuntimeError, match="differ in shape"):
            hb.matmul_silu_mul(hg, other, torch.from_numpy(A).cuda(), N)
    finally:
        for h in (hg, hu, other):
            hb.free(h)
