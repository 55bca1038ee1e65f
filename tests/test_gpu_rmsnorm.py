"""GPU parity of the decoder's RMSNorm (kernel/qwen35_decoder.cpp:134-140).

i4_rmsnorm_dev takes (float)(ss / H) from a tree sum and its error bound
when the bound decides it, and otherwise rebuilds the reference's in-order
double sum of squares in parallel; every output must equal the oracle's bit
for bit (both NaN where the oracle gives NaN).  Each case runs twice: as
shipped, and with BREEZE_HIP_NORM_EXACT=1, which always takes the in-order
rebuild.  The rows stress what that rebuild depends on: exact ties of both
parities, terms that round away, binade crossings, zeros, leading zeros,
outliers, denormal and non-finite inputs, a row whose partial sums hug a
power of two (the one-wave fallback), and a row whose mean is a float
rounding midpoint (the bound cannot decide it).  Widths straddle the
kernel's one-to-two terms per thread step (1024/1025) and its staged /
unstaged switch (8192/8193).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32


def _same(a, b):
    a, b = np.asarray(a, F), np.asarray(b, F)
    nan = np.isnan(b)
    return np.array_equal(np.isnan(a), nan) and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))


def _rows(H, seed):
    rng = np.random.default_rng(seed)
    rows = [rng.standard_normal(H).astype(F)]
    r = rng.standard_normal(H).astype(F)
    r[rng.random(H) < 0.01] *= 20
    rows.append(r)
    rows.append(np.ones(H, F))
    r = np.full(H, 2.0 ** -30, F)
    r[0] = 1.0
    rows.append(r)
    ties = np.where(rng.random(H) < 0.5, F(2.0 ** -26), F(3 * 2.0 ** -26)).astype(F)
    r = ties.copy()
    r[0] = 1.5
    rows.append(r)
    r = ties.copy()
    r[::97] = rng.standard_normal(len(r[::97]))
    rows.append(r)
    r = ties.copy()
    r[0], r[1 % H] = 1.5, F((2 ** 23 + 5) * 2.0 ** -28)
    rows.append(r)
    rows.append(np.zeros(H, F))
    r = np.zeros(H, F)
    r[(3 * H) // 4:] = rng.standard_normal(H - (3 * H) // 4)
    rows.append(r)
    rows.append((rng.standard_normal(H) * np.exp(rng.uniform(-40, 40, H))).astype(F))
    r = rng.standard_normal(H).astype(F)
    r[H // 2] = 1e18
    rows.append(r)
    r = rng.standard_normal(H).astype(F)
    r[rng.random(H) < 0.3] = F(1e-42)  # denormal floats
    rows.append(r)
    r = rng.standard_normal(H).astype(F) * F(3e38)
    rows.append(r.astype(F))
    # Mean exactly between two floats when H is a power of two: x0^2 =
    # 1 + 2^-11 + 2^-24.
    r = np.zeros(H, F)
    r[0] = F(1 + 2.0 ** -12)
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("mode", ["auto", "exact"])
@pytest.mark.parametrize("H", [1, 4, 7, 255, 256, 257, 1000, 1024, 1025, 2048, 5120, 8192, 8193, 12288])
def test_rmsnorm_bit_exact(gpu, hb, orc, monkeypatch, H, mode):
    import torch

    if mode == "exact":
        monkeypatch.setenv("BREEZE_HIP_NORM_EXACT", "1")

    x = _rows(H, H)
    rng = np.random.default_rng(H + 1)
    w = rng.standard_normal(H).astype(F)
    for eps in (F(1e-6), F(0.0), F(1e-2)):
        print(f"rmsnorm H={H} rows={x.shape[0]} eps={eps}", flush=True)
        got = hb.rmsnorm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), float(eps))
        torch.cuda.synchronize()
        want = orc.rmsnorm(x, w, eps)
        got = got.cpu().numpy()
        for i in range(x.shape[0]):
            assert _same(got[i], want[i]), f"row {i} H={H} eps={eps}"


def test_rmsnorm_non_finite_rows(gpu, hb, orc):
    import torch

    H = 300
    x = np.ones((4, H), F)
    x[0, 5] = np.inf
    x[1, 7] = np.nan
    x[2, 9], x[2, 11] = np.inf, np.nan
    x[3, 299] = -np.inf
    w = np.linspace(-1, 1, H, dtype=F)
    got = hb.rmsnorm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), 1e-6)
    torch.cuda.synchronize()
    assert _same(got.cpu().numpy(), orc.rmsnorm(x, w, F(1e-6)))


def test_rmsnorm_rejects_bad_shapes(gpu, hb):
    import torch

    x = torch.ones((2, 64), device="cuda")
    with pytest.raises(ValueError):
        hb.rmsnorm(x, torch.ones(63, device="cuda"), 1e-6)
    assert hb.rmsnorm(torch.ones((0, 64), device="cuda"), torch.ones(64, device="cuda"), 1e-6).shape == (0, 64)


@pytest.mark.parametrize("bits", [4, 8])
def test_rmsnorm_then_projection(gpu, hb, orc, hi_prec, bits):
    """The decoder step hn = rmsnorm(h); y = hn @ W (qwen35_decoder.cpp:405-408)
    on the GPU equals the same two steps of the oracle, bit for bit."""
    import torch

    rng = np.random.default_rng(bits)
    M, K, N = 3, 5120, 256
    h = (rng.standard_normal((M, K)) * 3).astype(F)
    ln = (1 + 0.1 * rng.standard_normal(K)).astype(F)
    qw = rng.integers(0, 256, (N, K // 32, 4 * bits), dtype=np.uint8)
    sc = rng.uniform(1e-3, 2e-2, (N, K // 32)).astype(F)
    hb.set_hi_prec(True)
    handle = hb.prepack(qw, sc, None, K, N, bits=bits)
    try:
        hn = hb.rmsnorm(torch.from_numpy(h).cuda(), torch.from_numpy(ln).cuda(), 1e-6)
        y = hb.matmul(handle, hn, N)
        torch.cuda.synchronize()
        y = y.cpu().numpy()
    finally:
        hb.free(handle)
    hn_ref = orc.rmsnorm(h, ln, F(1e-6))
    want = orc.matmul(qw, sc, None, N, K, bits, hn_ref, True)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
