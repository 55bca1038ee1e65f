"""The no-allocation entry point (i4_matmul_noalloc_dev) against the
allocating device entry points, through the C ABI, bit for bit: each case
makes two calls in a row, the second with a smaller input, so the second
runs on the scratch contents the first left behind.  Cases cover every
kernel route that uses scratch: the decode kernels with staged activation
records (four-row groups, and eight-row groups at 24 then 9 rows), the
decode argmax state, split-K's tickets and block values (cleared and
overwritten on every call), the prefill GEMM's records, the rows
kernel (legacy corr) and the argmax partials after it; plus a shape that
needs no scratch and one too large for the fixed scratch, which is refused.
"""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def _noalloc(hb, torch, h, A, N, argmax):
    dA = torch.from_numpy(A).cuda()
    M = A.shape[0]
    c = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    idx = torch.full((M,), -1, dtype=torch.int64, device="cuda") if argmax else None
    st = hb._vp(torch.cuda.current_stream().cuda_stream)
    rc = hb._lib.i4_matmul_noalloc_dev(hb._vp(h), hb._vp(dA.data_ptr()), M, hb._vp(c.data_ptr()),
                                       hb._vp(idx.data_ptr()) if argmax else None, st)
    assert rc == 0, hb.last_error()
    torch.cuda.synchronize()
    return c.cpu().numpy(), (idx.cpu().numpy() if argmax else None)


def _reference_call(hb, torch, h, A, N, argmax):
    dA = torch.from_numpy(A).cuda()
    if argmax:
        c, idx = hb.matmul_argmax(h, dA, N)
        torch.cuda.synchronize()
        return c.cpu().numpy(), idx.cpu().numpy()
    c = hb.matmul(h, dA, N)
    torch.cuda.synchronize()
    return c.cpu().numpy(), None


@pytest.mark.parametrize("case", ["fused", "staged", "argmax", "row_groups_argmax", "eight_row_groups", "split",
                                  "prefill", "prefill_argmax"])
@pytest.mark.parametrize("bits", [4, 8])
def test_noalloc_matches_allocating_entry(gpu, hb, hi_prec, monkeypatch, case, bits):
    torch = gpu
    if case == "split":
        monkeypatch.setenv("BREEZE_HIP_SPLIT", "1")
    K, N, rows, argmax = {
        "fused": (512, 256, (3, 1), False),
        "staged": (4608, 256, (8, 4), False),
        "argmax": (1024, 16 * 600, (2, 1), True),
        "row_groups_argmax": (1024, 16 * 320, (16, 12), True),
        "eight_row_groups": (4608, 256, (24, 9), True),
        "split": (17408, 64, (2, 1), False),
        "prefill": (1056, 304, (130, 20), False),
        "prefill_argmax": (640, 16 * 300, (40, 17), True),
    }[case]
    if case == "split":
        assert all(hb.plan(bits, m, K, N, extra=bits == 4)["split"] >= 2 for m in rows)
    rng = np.random.default_rng(sum(map(ord, case)) + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, bits == 4)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for m in rows:
                A = rng.normal(size=(m, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                got, gi = _noalloc(hb, torch, h, A, N, argmax)
                want, wi = _reference_call(hb, torch, h, A, N, argmax)
                assert bits_equal(got, want), (case, hp, m)
                if argmax:
                    assert gi.tolist() == wi.tolist(), (case, hp, m)
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits", [4, 8])
def test_noalloc_legacy_corr_rows_kernel(gpu, hb, orc, hi_prec, bits):
    """A legacy handle whose corr disagrees with its weights takes the rows
    kernel past the decode kernel's 32 rows (staged records in the fixed
    scratch)."""
    torch = gpu
    N, K, nblk = 48, 384, 12
    rng = np.random.default_rng(31 + bits)
    gb = 64 if bits == 8 else 32
    B = rng.integers(0, 256, (N // 16, nblk, 8, gb), dtype=np.uint8)
    scale = rng.uniform(0.001, 0.02, (N // 16, nblk, 16)).astype(np.float32)
    zp = rng.integers(0, 16, (N // 16, nblk, 16), dtype=np.int8) if bits == 4 else None
    corr = rng.integers(-5000, 5000, (N // 16, nblk, 16), dtype=np.int32)
    h = hb._lib.i4_prepack(hb._p(B), hb._p(scale), hb._p(zp), hb._p(corr), N, K, nblk, bits)
    assert h, hb.last_error()
    try:
        hb.set_hi_prec(True)
        for m in (40, 33):
            A = rng.normal(size=(m, K)).astype(np.float32)
            got, _ = _noalloc(hb, torch, h, A, N, False)
            want, _ = _reference_call(hb, torch, h, A, N, False)
            assert bits_equal(got, want), m
            assert bits_equal(got, orc.matmul_legacy(B, scale, zp, corr, N, K, bits, A, True)), m
    finally:
        hb.free(h)


def test_noalloc_refuses_what_does_not_fit(gpu, hb, hi_prec):
    """Prefill records of 2048 rows x K = 17408 (about 150 MB) exceed the
    16 MiB scratch: the call returns an error and launches nothing; the next
    call that fits works."""
    torch = gpu
    N, K = 32, 17408
    rng = np.random.default_rng(5)
    qw, sc, _ = rng_weights(rng, N, K, 8)
    h = hb.prepack(qw, sc, None, K, N, bits=8)
    try:
        hb.set_hi_prec(True)
        big = torch.zeros((2048, K), dtype=torch.float32, device="cuda")
        out = torch.zeros((2048, N), dtype=torch.float32, device="cuda")
        st = hb._vp(torch.cuda.current_stream().cuda_stream)
        rc = hb._lib.i4_matmul_noalloc_dev(hb._vp(h), hb._vp(big.data_ptr()), 2048, hb._vp(out.data_ptr()),
                                           None, st)
        assert rc == -4
        assert "scratch" in hb.last_error()
        A = rng.normal(size=(3, K)).astype(np.float32)
        got, _ = _noalloc(hb, torch, h, A, N, False)
        want, _ = _reference_call(hb, torch, h, A, N, False)
        assert bits_equal(got, want)
    finally:
        hb.free(h)


def test_noalloc_inside_graph_capture(gpu, hb, hi_prec):
    """Captured without any uncaptured call first (nothing to allocate),
    replayed several times with eager work between the replays: every
    replay equals the allocating entry point's result."""
    torch = gpu
    N, K = 16 * 300, 4608
    rng = np.random.default_rng(17)
    qw, sc, _ = rng_weights(rng, N, K, 8)
    h = hb.prepack(qw, sc, None, K, N, bits=8)
    try:
        hb.set_hi_prec(True)
        inputs = [rng.normal(size=(6, K)).astype(np.float32) for _ in range(3)]
        want = [hb.matmul(h, x, N) for x in inputs]
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        x_static = torch.from_numpy(inputs[0]).cuda()
        c_static = torch.zeros((6, N), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            rc = hb._lib.i4_matmul_noalloc_dev(hb._vp(h), hb._vp(x_static.data_ptr()), 6,
                                               hb._vp(c_static.data_ptr()), None,
                                               hb._vp(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, hb.last_error()
        for i in range(4):
            x_static.copy_(torch.from_numpy(inputs[i % 3]).cuda())
            graph.replay()
            torch.cuda.synchronize()
            assert bits_equal(c_static.cpu().numpy(), want[i % 3]), i
            _noalloc(hb, torch, h, inputs[(i + 1) % 3][:2], N, False)  # eager work on the same scratch
    finally:
        hb.free(h)
