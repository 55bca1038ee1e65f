"""The fused gate/up projection of a decoder MLP (i4_matmul_silu_mul_dev),
replacing kernel/qwen35_decoder.cpp:406-408: g1 = i4_matmul(gate), g2 =
i4_matmul(up), g1 = siluf(g1) * g2 with siluf(x) = x / (1 + exp(-x)).

Both projections are the exact path (bit-identical to the oracle), and the
SiLU and product are the reference's bit for bit: the expected values are
the oracle's projections through the oracle's silu * u, which forms
g / (1 + expf(-g)) * u with the host C library's expf, the function the
reference's siluf calls.  The one-launch path (handles of the same layout; up
to 16 rows on the four-row groups, 32 on the eight-row groups), the
two-launch fallback and the elementwise entry point (i4_silu_mul_dev) are all
held to those bits."""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def _silu_mul(g, u):
    from oracle import oracle
    return oracle.c_oracle().silu_mul(g, u)


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
                assert bits_equal(got, want[:rows]), f"{rows} rows"
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
            assert bits_equal(got20, want), hp
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
        assert bits_equal(got, want)
        with pytest.raises(RuntimeError, match="differ in shape"):
            hb.matmul_silu_mul(hg, other, torch.from_numpy(A).cuda(), N)
    finally:
        for h in (hg, hu, other):
            hb.free(h)


def _same(got, want):
    """Bitwise equality, any NaN matching any NaN."""
    nan = np.isnan(got) & np.isnan(want)
    return np.array_equal(np.isnan(got), np.isnan(want)) and \
        np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])


def test_silu_mul_entry_point_is_the_reference_on_a_sweep_of_floats(gpu, hb, orc):
    """i4_silu_mul_dev against the oracle (the C library's expf) on one in
    16 float bit patterns (268 million gate values over all signs and
    exponents, so the overflow and underflow branches and the subnormal
    results too), each with a random up value, and on edge values."""
    torch = gpu
    rng = np.random.default_rng(12)
    for start in range(0, 64, 16):
        g = (np.arange(start, 1 << 32, 64, dtype=np.uint64) + rng.integers(0, 64)).astype(np.uint32).view(np.float32)
        u = rng.normal(0, 1, g.size).astype(np.float32)
        got = hb.silu_mul(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()).cpu().numpy()
        assert _same(got, orc.silu_mul(g, u)), start
    hexes = ["0x1.62e42ep6", "0x1.62e430p6", "-0x1.9fe368p6", "-0x1.9fe36ap6", "0x1.60p6", "-0x1.60p6"]
    edge = np.array([0.0, -0.0, 1e-45, -1e-45, 88.72, -88.72, 103.97, -103.97, 3.4e38, -3.4e38, np.inf, -np.inf,
                     np.nan] + [float.fromhex(h) for h in hexes], np.float32)
    ones = np.ones_like(edge)
    got = hb.silu_mul(torch.from_numpy(edge).cuda(), torch.from_numpy(ones).cuda()).cpu().numpy()
    assert _same(got, orc.silu_mul(edge, ones))
