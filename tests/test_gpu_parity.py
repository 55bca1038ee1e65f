"""GPU parity: the HIP path against the C restatement of the reference.

Bar: bit-exact FP32 outputs and bit-exact per-block INT32 integers on the
same seeded inputs (the oracle is itself pinned bit-for-bit against the
compiled reference kernel, tests/test_oracle_*.py).  Cases follow the
reference's own tests: tests/test_cpu_packing.py:70-96 (shapes, bits,
fp16/fp32 scales, explicit zero points, rows 1 and 9, both activation modes),
tests/test_qwen35_cpu.py:196-208 (projection widths), plus the benchmark
workloads.
"""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def _run_both(hb, torch, h, A, N):
    """Host-pointer entry point and device-pointer entry point."""
    c_host = hb.matmul(h, A, N)
    c_dev = hb.matmul(h, torch.from_numpy(A).cuda(), N)
    torch.cuda.synchronize()
    return c_host, c_dev.cpu().numpy()


@pytest.mark.parametrize("N,K", [(16, 32), (48, 96), (64, 512), (32, 4096)])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
def test_matmul_bit_exact(gpu, hb, orc, hi_prec, N, K, bits, dtype, explicit_zeros):
    rng = np.random.default_rng(N + K + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, dtype, explicit_zeros)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (False, True):
            hb.set_hi_prec(hp)
            for rows in (1, 2, 3, 8, 9, 17):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
                c_host, c_dev = _run_both(hb, gpu, h, A, N)
                assert bits_equal(c_host, want), (hp, rows, np.max(np.abs(c_host - want)))
                assert bits_equal(c_dev, want), (hp, rows)
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
def test_block_integers_exact(gpu, hb, orc, hi_prec, bits, explicit_zeros):
    N, K = 64, 1024
    rng = np.random.default_rng(11 + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    A = (rng.normal(size=(9, K)) * rng.choice([1e-3, 1.0, 50.0], size=(9, 1))).astype(np.float32)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (False, True):
            hb.set_hi_prec(hp)
            _, cs_want = orc.matmul(qw, sc, qz, N, K, bits, A, hp, want_cs=True)
            cs = hb.block_dots(h, gpu.from_numpy(A).cuda(), N, K).cpu().numpy()
            np.testing.assert_array_equal(cs, cs_want)
    finally:
        hb.free(h)


@pytest.mark.parametrize("K,N,bits", [(5120, 48, 8), (17408, 16, 4), (6144, 64, 8), (4096, 32, 4)])
def test_projection_widths(gpu, hb, orc, hi_prec, K, N, bits):
    """tests/test_qwen35_cpu.py:196-208 shapes and seed, HP mode, bit-exact."""
    rng = np.random.default_rng(3)
    qw = rng.integers(0, 256, (N, K // 32, 32 * bits // 8), dtype=np.uint8)
    scales = rng.uniform(0.001, 0.005, (N, K // 32)).astype(np.float32)
    a = rng.normal(size=(3, K)).astype(np.float32)
    hb.set_hi_prec(True)
    h = hb.prepack(qw, scales, None, K, N, bits=bits)
    try:
        got = hb.matmul(h, a, N)
    finally:
        hb.free(h)
    assert bits_equal(got, orc.matmul(qw, scales, None, N, K, bits, a, True))


@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
def test_decode_with_staged_activation_records(gpu, hb, orc, hi_prec, bits, explicit_zeros):
    """Decode shapes whose activation records come from the stand-alone
    quantizer (more than 512 row-blocks per row group: K = 4608 with 4 or
    more rows; K = 17408 with one row), beside a shape quantized inside the
    decode kernel (2 rows), in both activation modes, bit-exact."""
    rng = np.random.default_rng(11 + bits)
    # K = 4640: 145 blocks, a partial last chunk of the records (1 of 4 or
    # 1 of 2 blocks); 3 rows quantize inside the kernel, 4 and 8 stage.
    for K, rows_list in ((4608, (2, 4, 5, 8)), (4640, (3, 4, 8)), (17408, (1,))):
        N = 64
        qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
        h = hb.prepack(qw, sc, qz, K, N, bits=bits)
        try:
            for hp in (False, True):
                hb.set_hi_prec(hp)
                for rows in rows_list:
                    A = rng.normal(size=(rows, K)).astype(np.float32)
                    want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
                    c_host, c_dev = _run_both(hb, gpu, h, A, N)
                    assert bits_equal(c_host, want), (K, hp, rows)
                    assert bits_equal(c_dev, want), (K, hp, rows)
        finally:
            hb.free(h)


@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
@pytest.mark.parametrize("K", [224, 672, 2080])
def test_single_row_decode_several_tiles_per_workgroup(gpu, hb, orc, hi_prec, bits, explicit_zeros, K):
    """One activation row with 4 or 5 tiles per decode workgroup
    (N = 16 * 1029, uneven split), K with short last phases and padded last
    chunks.  Outputs bit-exact, argmax first-max across workgroups."""
    rng = np.random.default_rng(K + bits)
    N = 16 * 1029
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (False, True):
            hb.set_hi_prec(hp)
            A = rng.normal(size=(1, K)).astype(np.float32)
            want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
            c_host, c_dev = _run_both(hb, gpu, h, A, N)
            assert bits_equal(c_host, want), (K, hp)
            assert bits_equal(c_dev, want), (K, hp)
            c_arg, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
            gpu.cuda.synchronize()
            assert bits_equal(c_arg.cpu().numpy(), want), (K, hp)
            assert idx.cpu().tolist() == np.argmax(want, axis=1).tolist(), (K, hp)
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits", [4, 8])
def test_legacy_layout_entry_point(gpu, hb, orc, hi_prec, bits):
    """i4_prepack of the NumPy-built legacy layout == i4_prepack_onnx."""
    N, K = 48, 96
    rng = np.random.default_rng(7)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float16, bits == 4)
    fast = hb.prepack(qw, sc, qz, K, N, bits=bits)
    old = hb._prepack_numpy(qw, sc, qz, K, N, bits=bits)
    try:
        uf, uo = hb.unpack(fast), hb.unpack(old)
        for key in ("qweight", "scales", "zp", "corr_delta"):
            np.testing.assert_array_equal(uf[key], uo[key])
        for hp in (False, True):
            hb.set_hi_prec(hp)
            for rows in (1, 9):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                assert bits_equal(hb.matmul(fast, A, N), hb.matmul(old, A, N))
    finally:
        hb.free(fast)
        hb.free(old)


@pytest.mark.parametrize("bits", [4, 8])
def test_legacy_corr_is_honoured(gpu, hb, orc, hi_prec, bits):
    """A corr that disagrees with the weights (kernel/benchmark_matmul.cpp
    passes zeros) changes the result exactly as the reference's hp_combine."""
    N, K, nblk = 32, 128, 4
    rng = np.random.default_rng(21)
    gb = 64 if bits == 8 else 32
    B = rng.integers(0, 256, (N // 16, nblk, 8, gb), dtype=np.uint8)
    scale = rng.uniform(0.001, 0.02, (N // 16, nblk, 16)).astype(np.float32)
    zp = rng.integers(0, 16, (N // 16, nblk, 16), dtype=np.int8) if bits == 4 else None
    corr = rng.integers(-5000, 5000, (N // 16, nblk, 16), dtype=np.int32)
    corr.reshape(-1)[:8] = 0
    h = hb._lib.i4_prepack(hb._p(B), hb._p(scale), hb._p(zp), hb._p(corr), N, K, nblk, bits)
    assert h, hb.last_error()
    try:
        for hp in (False, True):
            hb.set_hi_prec(hp)
            # 5, 9 and 17 rows: the decode kernel (up to 32 rows here); 33
            # and 40: the rows kernel's corr delta in row chunks of 8
            # (quantized_matmul.cpp:542-550).
            for rows in (5, 9, 17, 33, 40):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                want = orc.matmul_legacy(B, scale, zp, corr, N, K, bits, A, hp)
                assert bits_equal(hb.matmul(h, A, N), want), (hp, rows)
    finally:
        hb.free(h)


@pytest.mark.parametrize("zp_lo,zp_hi", [(-112, 0), (-112, 16), (-5, 3), (100, 128)])
def test_legacy_int4_signed_zero_points(gpu, hb, orc, hi_prec, zp_lo, zp_hi):
    """Legacy INT4 handles keep signed int8 zero points from -112 up
    (b = nibble - zp never wraps there) with a consistent corr, so they stay
    INT4 with explicit zero points: the decode kernel (1, 3, 8, 9, 17 rows)
    and the prefill GEMM's in-LDS nibble expansion (33, 130 rows), whose per-byte
    n - zp must not borrow across bytes for negative zp.  33 blocks: a
    partial last 4-block chunk."""
    N, K = 64, 1056
    nblk = K // 32
    rng = np.random.default_rng(zp_lo + 1000)
    B = rng.integers(0, 256, (N // 16, nblk, 8, 32), dtype=np.uint8)
    scale = rng.uniform(0.001, 0.02, (N // 16, nblk, 16)).astype(np.float32)
    zp = rng.integers(zp_lo, zp_hi, (N // 16, nblk, 16)).astype(np.int8)
    # corr = 128 * sum(b): the oracle's delta against a zero corr.
    _, _, full = orc.unpack_legacy(B, scale, zp, np.zeros_like(scale, dtype=np.int32), N, K, 4)
    corr = np.ascontiguousarray(full.reshape(N // 16, 16, nblk).transpose(0, 2, 1)).astype(np.int32)
    h = hb._lib.i4_prepack(hb._p(B), hb._p(scale), hb._p(zp), hb._p(corr), N, K, nblk, 4)
    assert h, hb.last_error()
    try:
        info = hb.handle_info(h)
        assert info["bits"] == 4 and not info["has_corr_delta"], info
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for rows in (1, 3, 8, 9, 17, 33, 130):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                want = orc.matmul_legacy(B, scale, zp, corr, N, K, 4, A, hp)
                got = hb.matmul(h, gpu.from_numpy(A).cuda(), N)
                gpu.cuda.synchronize()
                assert bits_equal(got.cpu().numpy(), want), (hp, rows)
    finally:
        hb.free(h)


@pytest.mark.parametrize("bits", [4, 8])
def test_matmul_region_entry_point(gpu, hb, orc, hi_prec, bits):
    """i4_matmul_region (quantized_matmul.cpp:558-572) with the caller's
    scratch (2*M*K bytes) and ascale (M*K/32 floats) buffers, M <= 8 as the
    reference allows: the same outputs as the oracle, bit for bit."""
    N, K = 96, 640
    rng = np.random.default_rng(40 + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, bits == 4)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (False, True):
            hb.set_hi_prec(hp)
            for rows in (1, 3, 8):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                C = np.full((rows, N), np.nan, np.float32)
                scratch = np.zeros(2 * rows * K, np.uint8)
                ascale = np.zeros(rows * (K // 32), np.float32)
                hb._lib.i4_matmul_region(hb._vp(h), hb._p(A), rows, hb._p(C), hb._p(scratch), hb._p(ascale))
                assert hb.last_error() == "", hb.last_error()
                assert bits_equal(C, orc.matmul(qw, sc, qz, N, K, bits, A, hp)), (hp, rows)
    finally:
        hb.free(h)


def test_linear_fp16_backend_values(gpu):
    """breeze_amd.linear on the GPU (fp16 weight and activation, fp32
    accumulate): within fp16 input rounding of the fp32 product."""
    from breeze_amd import linear

    assert linear.backend() == "torch-hip-fp16"
    rng = np.random.default_rng(6)
    w = rng.normal(size=(512, 96)).astype(np.float32)
    a = rng.normal(size=(2, 3, 512)).astype(np.float32)
    out = linear.linear(a, linear.prepare_weight(w))
    assert out.shape == (2, 3, 96) and out.dtype == np.float32
    ref = a.astype(np.float64) @ w.astype(np.float64)
    # Each input rounds to fp16 (relative 2^-11); the products' errors add
    # up over K = 512 terms of typical size |a||w| ~ 1.
    err = np.max(np.abs(out - ref)) / np.max(np.abs(ref))
    assert err < 2e-3, err


@pytest.mark.parametrize("bits", [4, 8])
def test_unpack_round_trip(gpu, hb, bits):
    """The device layout holds exactly the MatMulNBits inputs."""
    N, K = 80, 160
    rng = np.random.default_rng(5)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float16, bits == 4)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        u = hb.unpack(h)
        np.testing.assert_array_equal(u["qweight"], qw)
        np.testing.assert_array_equal(u["scales"], sc.astype(np.float32))
        if bits == 4:
            zpf = np.empty((N, 2 * qz.shape[1]), np.uint8)
            zpf[:, 0::2] = qz & 15
            zpf[:, 1::2] = qz >> 4
            np.testing.assert_array_equal(u["zp"], zpf[:, :K // 32])
        assert not u["corr_delta"].any()
    finally:
        hb.free(h)


def test_row_slices_match_single_rows(gpu, hb, orc, hi_prec):
    """Row m of an M-row call equals a 1-row call (reference property,
    tests/test_cpu_packing.py:155-168)."""
    N, K = 64, 768
    rng = np.random.default_rng(9)
    qw, sc, _ = rng_weights(rng, N, K, 4)
    h = hb.prepack(qw, sc, None, K, N, bits=4)
    hb.set_hi_prec(True)
    try:
        A = rng.normal(size=(19, K)).astype(np.float32)
        full = hb.matmul(h, A, N)
        for m in (0, 7, 8, 18):
            assert bits_equal(hb.matmul(h, A[m:m + 1], N)[0], full[m])
    finally:
        hb.free(h)


def test_argmax_first_max_semantics(gpu, hb, hi_prec):
    """Ties, -0/+0 and NaN follow numpy.argmax on the computed logits."""
    N, K = 4096, 64
    rng = np.random.default_rng(4)
    # Identical weight columns produce exact ties.
    col = rng.integers(0, 256, (1, 2, 32), dtype=np.uint8)
    qw = np.repeat(col, N, axis=0)
    sc = np.full((N, 2), 0.01, np.float32)
    sc[::7] = 0.02
    h = hb.prepack(qw, sc, None, K, N, bits=8)
    hb.set_hi_prec(True)
    try:
        A = gpu.from_numpy(rng.normal(size=(3, K)).astype(np.float32)).cuda()
        logits, idx = hb.matmul_argmax(h, A, N)
        gpu.cuda.synchronize()
        np.testing.assert_array_equal(idx.cpu().numpy(), np.argmax(logits.cpu().numpy(), axis=1))
    finally:
        hb.free(h)


# Prefill workgroup shapes (row pairs : column tiles), as instantiated.
PF_CFGS = ["auto", "4:17", "4:16", "4:13", "4:12", "4:9", "4:8", "4:5", "4:4", "2:16", "2:8", "2:4", "1:16", "1:8"]
PF_ROWS = (9, 33, 70, 130, 300)


def _force_pf(monkeypatch, cfg):
    # Rows 9-16 would take the decode kernel: keep them on the GEMM here.
    monkeypatch.setenv("BREEZE_HIP_DEC_ROWS", "8")
    if cfg != "auto":
        rp, ct = cfg.split(":")
        monkeypatch.setenv("BREEZE_HIP_PREFILL_RP", rp)
        monkeypatch.setenv("BREEZE_HIP_PREFILL_CT", ct)


@pytest.mark.parametrize("scales", ["channel", "group", "block"])
@pytest.mark.parametrize("cfg", PF_CFGS)
def test_prefill_gemm_bit_exact(gpu, hb, orc, hi_prec, monkeypatch, scales, cfg):
    """The M > 8 INT8 GEMM against the oracle: per-column, per-group (4 blocks)
    and per-block scales; every workgroup shape (32, 64 or 128 rows, every
    column-tile width), with a partial last column group (19 tiles); an odd
    block count (33, so the last chunk and the last scale group are
    partial); row counts around the 32-, 64- and 128-row workgroups; and
    activations with x20 outliers for the hi/lo split."""
    _force_pf(monkeypatch, cfg)
    N, K = 304, 1056
    rng = np.random.default_rng(11)
    qw, sc, _ = rng_weights(rng, N, K, 8)
    if scales == "channel":
        sc = np.repeat(sc[:, :1], K // 32, axis=1)
    elif scales == "group":
        sc = np.repeat(sc[:, ::4], 4, axis=1)[:, :K // 32]
    h = hb.prepack(qw, sc, None, K, N, bits=8)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for rows in PF_ROWS:
                A = rng.normal(size=(rows, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                want = orc.matmul(qw, sc, None, N, K, 8, A, hp)
                got = hb.matmul(h, gpu.from_numpy(A).cuda(), N)
                gpu.cuda.synchronize()
                assert bits_equal(got.cpu().numpy(), want), (hp, rows)
    finally:
        hb.free(h)


@pytest.mark.parametrize("scales", ["channel", "group4", "group8", "block", "zeros"])
@pytest.mark.parametrize("cfg", PF_CFGS)
def test_prefill_gemm_int4_bit_exact(gpu, hb, orc, hi_prec, monkeypatch, scales, cfg):
    """The M > 8 GEMM on INT4 weights (nibbles expanded to signed bytes
    n - zp in LDS) against the oracle: per-column scales, groups of one and
    two 4-block chunks, per-block scales (default zero point 8) and explicit
    zero points 0..15; every workgroup shape with a partial last column
    group (19 tiles); 33 and 35 blocks, so the last 4-block chunk holds one
    or three blocks."""
    _force_pf(monkeypatch, cfg)
    N = 304
    rng = np.random.default_rng(12)
    for K in (1056, 1120):
        qw, sc, qz = rng_weights(rng, N, K, 4, explicit_zeros=scales == "zeros")
        nblk = K // 32
        if scales == "channel":
            sc = np.repeat(sc[:, :1], nblk, axis=1)
        elif scales.startswith("group"):
            g = int(scales[5:])
            sc = np.repeat(sc[:, ::g], g, axis=1)[:, :nblk]
        sc = np.ascontiguousarray(sc)
        h = hb.prepack(qw, sc, qz, K, N, bits=4)
        try:
            info = hb.handle_info(h)
            assert info["scale_group"] == {"channel": 0, "group4": 4, "group8": 8, "block": 1, "zeros": 1}[scales], info
            for hp in (True, False):
                hb.set_hi_prec(hp)
                for rows in PF_ROWS:
                    A = rng.normal(size=(rows, K)).astype(np.float32)
                    A[rng.random(A.shape) < 0.01] *= 20.0
                    want = orc.matmul(qw, sc, qz, N, K, 4, A, hp)
                    got = hb.matmul(h, gpu.from_numpy(A).cuda(), N)
                    gpu.cuda.synchronize()
                    assert bits_equal(got.cpu().numpy(), want), (K, hp, rows)
        finally:
            hb.free(h)


def test_matmulnbits_operator_routes_to_the_gpu(gpu, hb, orc, hi_prec):
    """breeze_amd.ops with the real backend: the session cache prepacks an
    INT4 node with explicit zeros and an INT8 node, and the operator body
    matches the oracle for a 3-D NumPy activation and a GPU tensor."""
    import types

    from breeze_amd import ops

    rng = np.random.default_rng(12)
    qw4, sc4, qz4 = rng_weights(rng, 64, 256, 4, np.float16, True)
    qw8, sc8, _ = rng_weights(rng, 32, 320, 8)
    inits = {"w4": qw4, "s4": sc4, "z4": qz4, "w8": qw8, "s8": sc8}
    nodes = [types.SimpleNamespace(name="p4", op_type="MatMulNBits", inputs=["x", "w4", "s4", "z4"],
                                   attrs=dict(K=256, N=64, bits=4, block_size=32)),
             types.SimpleNamespace(name="p8", op_type="MatMulNBits", inputs=["x", "w8", "s8"],
                                   attrs=dict(K=320, N=32, bits=8, block_size=32))]
    cache = ops.prepack_nodes(nodes, inits)
    try:
        hb.set_hi_prec(True)
        a4 = rng.normal(size=(2, 5, 256)).astype(np.float32)
        out4 = ops.matmul_nbits(cache, "p4", a4)
        assert out4.shape == (2, 5, 64)
        assert bits_equal(out4.reshape(10, 64), orc.matmul(qw4, sc4, qz4, 64, 256, 4, a4.reshape(10, 256), True))
        a8 = rng.normal(size=(3, 320)).astype(np.float32)
        out8 = ops.matmul_nbits(cache, "p8", gpu.from_numpy(a8[None]).cuda())
        gpu.cuda.synchronize()
        assert tuple(out8.shape) == (1, 3, 32)
        assert bits_equal(out8[0].cpu().numpy(), orc.matmul(qw8, sc8, None, 32, 320, 8, a8, True))
    finally:
        ops.free_cache(cache)


def _nan_aware_equal(a, b):
    """NaN at the same places, bit-identical elsewhere.  A NaN output comes
    from inf * 0 in the fold, and its sign and payload are the machine's:
    x86 makes the negative default NaN, the GPU the positive one."""
    a, b = np.asarray(a), np.asarray(b)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _special_rows(rng, K):
    """One N(0,1) row per pattern, the pattern planted in block 1 (k 32..63):
    a quiet NaN, signaling NaNs, an all-NaN block, +inf, -inf, a block of
    denormals, signed zeros only, values near the float maximum, and tiny
    normals whose block scale is denormal (its reciprocal overflows)."""
    snan = np.array([0x7F800001, 0xFFA00000, 0x7FBFFFFF], np.uint32).view(np.float32)
    rows = []

    def row():
        return rng.normal(size=K).astype(np.float32)

    r = row(); r[40] = np.nan; rows.append(r)
    r = row(); r[33], r[50], r[63] = snan; rows.append(r)
    r = row(); r[32:64] = np.nan; r[36:39] = snan; rows.append(r)
    r = row(); r[45] = np.inf; rows.append(r)
    r = row(); r[45] = -np.inf; rows.append(r)
    r = row(); r[32:64] = (rng.uniform(-1, 1, 32) * 1e-39).astype(np.float32); rows.append(r)
    r = row(); r[32:64] = 0.0; r[32:64:3] = -0.0; rows.append(r)
    r = row(); r[32:64] = (rng.uniform(-1, 1, 32) * 3.4e38).astype(np.float32); rows.append(r)
    r = row(); r[32:64] = (rng.uniform(-1, 1, 32) * 1e-34).astype(np.float32); rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
def test_non_finite_and_extreme_activations(gpu, hb, orc, hi_prec, monkeypatch, bits, explicit_zeros):
    """Activation blocks with NaNs (quiet and signaling: skipped by the block
    max), infinities (the row becomes NaN), denormals, signed zeros, values
    near the float maximum and tiny normals, through every quantizer: the
    decode kernel's own (one row; 16 and 256 row-blocks), the stand-alone
    decode quantizer (4 rows of K = 4608), the decode kernel's row groups
    (all nine rows at once) and the prefill GEMM's records (the nine rows
    again with the decode kernel held to 8 rows).  Outputs match the oracle
    bit for bit outside NaNs."""
    rng = np.random.default_rng(91 + bits)
    N = 48
    for K, groups in ((512, "single"), (8192, "single"), (4608, "four"), (512, "all"), (512, "gemm")):
        if groups == "gemm":
            monkeypatch.setenv("BREEZE_HIP_DEC_ROWS", "8")
        qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
        h = hb.prepack(qw, sc, qz, K, N, bits=bits)
        try:
            A = _special_rows(rng, K)
            batches = {"single": [A[i:i + 1] for i in range(len(A))],
                       "four": [A[0:4], A[4:8]],
                       "all": [A], "gemm": [A]}[groups]
            for hp in (False, True):
                hb.set_hi_prec(hp)
                for x in batches:
                    want = orc.matmul(qw, sc, qz, N, K, bits, x, hp)
                    c_host, c_dev = _run_both(hb, gpu, h, x, N)
                    assert _nan_aware_equal(c_host, want), (K, groups, hp, x.shape)
                    assert _nan_aware_equal(c_dev, want), (K, groups, hp, x.shape)
        finally:
            hb.free(h)


@pytest.mark.parametrize("dec8", ["on", "off"])
@pytest.mark.parametrize("bits", [4, 8])
def test_decode_staged_rows_with_argmax(gpu, hb, orc, hi_prec, monkeypatch, bits, dec8):
    """Four to eight rows whose records come from the stand-alone quantizers
    (K = 4640: 145 blocks, a partial last chunk; five to eight rows in one
    eight-row workgroup per tile range, or with BREEZE_HIP_DEC8=0 in two
    four-row ones): outputs bit-exact and the argmax of every row first-max
    exact, several tiles per workgroup (N = 16 * 600)."""
    if dec8 == "off":
        monkeypatch.setenv("BREEZE_HIP_DEC8", "0")
    N, K = 16 * 600, 4640
    rng = np.random.default_rng(60 + bits)
    qw, sc, _ = rng_weights(rng, N, K, bits)
    h = hb.prepack(qw, sc, None, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for rows in (4, 5, 7, 8):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                want = orc.matmul(qw, sc, None, N, K, bits, A, hp)
                c, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
                gpu.cuda.synchronize()
                assert bits_equal(c.cpu().numpy(), want), (hp, rows)
                assert idx.cpu().tolist() == np.argmax(want, axis=1).tolist(), (hp, rows)
    finally:
        hb.free(h)


@pytest.mark.parametrize("dec8", ["on", "off"])
@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
def test_decode_row_groups(gpu, hb, orc, hi_prec, monkeypatch, bits, explicit_zeros, dec8):
    """9 to 32 rows through the decode kernels' row groups (two to four
    workgroups of 8 rows, or with BREEZE_HIP_DEC8=0 or explicit zero points
    three to eight of 4 rows, per tile range, on one XCD when the range
    count allows; the limit forced to 32), outputs and argmax against the
    oracle: K = 4608 (staged records, 40 tiles: row groups placed on one
    XCD) and K = 96 (the four-row groups quantize in their prologue up to 20
    rows, the eight-row groups take 25 and 32; 20 tiles: the plain block
    order)."""
    monkeypatch.setenv("BREEZE_HIP_DEC_ROWS", "32")
    if dec8 == "off":
        monkeypatch.setenv("BREEZE_HIP_DEC8", "0")
    rng = np.random.default_rng(31)
    for K, N in ((4608, 640), (96, 320)):
        qw, sc, qz = rng_weights(rng, N, K, bits, explicit_zeros=explicit_zeros)
        h = hb.prepack(qw, sc, qz, K, N, bits=bits)
        try:
            for hp in (True, False):
                hb.set_hi_prec(hp)
                for rows in (9, 12, 13, 16, 20, 25, 32):
                    A = rng.normal(size=(rows, K)).astype(np.float32)
                    A[rng.random(A.shape) < 0.01] *= 20.0
                    want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
                    got, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
                    gpu.cuda.synchronize()
                    assert bits_equal(got.cpu().numpy(), want), (K, hp, rows)
                    assert idx.cpu().numpy().tolist() == np.argmax(want, axis=1).tolist(), (K, hp, rows)
        finally:
            hb.free(h)


@pytest.mark.parametrize("dec8", ["on", "off"])
@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
def test_decode_two_row_groups_long_k(gpu, hb, orc, hi_prec, monkeypatch, bits, explicit_zeros, dec8):
    """K = 17408 (544 blocks, the MLP down projection at decode batch sizes):
    four rows of records exceed the four-row kernel's staged copy, so 3 to 16
    rows run as its workgroups of 2 rows, except 5-16 rows of handles
    without per-block metadata, which take the eight-row groups unless
    BREEZE_HIP_DEC8=0.  Outputs and argmax against the oracle."""
    if dec8 == "off":
        monkeypatch.setenv("BREEZE_HIP_DEC8", "0")
    rng = np.random.default_rng(37)
    K, N = 17408, 320
    qw, sc, qz = rng_weights(rng, N, K, bits, explicit_zeros=explicit_zeros)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for rows in (3, 4, 7, 8, 12, 16):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
                got, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
                gpu.cuda.synchronize()
                assert bits_equal(got.cpu().numpy(), want), (hp, rows)
                assert idx.cpu().numpy().tolist() == np.argmax(want, axis=1).tolist(), (hp, rows)
    finally:
        hb.free(h)


@pytest.mark.parametrize("dec8", ["on", "off"])
@pytest.mark.parametrize("bits", [4, 8])
def test_decode_one_row_groups_longer_k(gpu, hb, orc, hi_prec, monkeypatch, bits, dec8):
    """K = 26624 (832 blocks): even two rows of records exceed the four-row
    kernel's staged copy, so 2 to 4 rows run as its workgroups of one row;
    5 to 9 rows take the eight-row groups (with BREEZE_HIP_DEC8=0: one-row
    workgroups up to 8 rows, the GEMM at 9).  Outputs and argmax against
    the oracle."""
    if dec8 == "off":
        monkeypatch.setenv("BREEZE_HIP_DEC8", "0")
    rng = np.random.default_rng(41)
    K, N = 26624, 160
    qw, sc, qz = rng_weights(rng, N, K, bits)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            for rows in (1, 2, 3, 8, 9):
                A = rng.normal(size=(rows, K)).astype(np.float32)
                A[rng.random(A.shape) < 0.01] *= 20.0
                want = orc.matmul(qw, sc, qz, N, K, bits, A, hp)
                got, idx = hb.matmul_argmax(h, gpu.from_numpy(A).cuda(), N)
                gpu.cuda.synchronize()
                assert bits_equal(got.cpu().numpy(), want), (hp, rows)
                assert idx.cpu().numpy().tolist() == np.argmax(want, axis=1).tolist(), (hp, rows)
    finally:
        hb.free(h)


# The decode prologue quantizes up to 768 row-blocks of one or two rows
# itself (three passes of 256 over its sixteen waves) and up to 512 of more
# rows; BREEZE_HIP_FUSED_MAX_BLOCKS raises the limit to the prologue's six
# passes (1536 row-blocks), which the routing does not use by default, so the
# longer prologues are checked here too.  Row counts and K cover every pass
# count from one to six, partial last passes and padded last chunks.
@pytest.mark.parametrize("bits,explicit_zeros", [(4, False), (4, True), (8, False)])
@pytest.mark.parametrize("M,K,limit", [(1, 17408, None), (1, 24576, None), (2, 12288, None), (2, 8224, None),
                                       (3, 12288, 1536), (4, 12288, 1536), (4, 10272, 1536), (1, 49120, 1536)])
def test_decode_prologue_passes(gpu, hb, orc, hi_prec, monkeypatch, bits, explicit_zeros, M, K, limit):
    torch = gpu
    if limit:
        monkeypatch.setenv("BREEZE_HIP_FUSED_MAX_BLOCKS", str(limit))
    N = 64
    assert hb.plan(bits, M, K, N, extra=explicit_zeros)["quant"] is None  # the prologue quantizes
    rng = np.random.default_rng(M * 7 + K + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        for hp in (True, False):
            hb.set_hi_prec(hp)
            A = (rng.normal(size=(M, K)) * rng.choice([1e-3, 1.0, 50.0], size=(M, 1))).astype(np.float32)
            A[0, 5] = np.float32(0.0)
            got = hb.matmul(h, torch.from_numpy(A).cuda(), N).cpu().numpy()
            assert bits_equal(got, orc.matmul(qw, sc, qz, N, K, bits, A, hp)), (M, K, hp)
    finally:
        hb.free(h)


# Non-temporal weight loads (the decode kernel's stream mode) change only how
# the weight chunks are fetched: with the mode forced on and off, on shapes it
# takes by default and shapes it does not, every output is the oracle's.
@pytest.mark.parametrize("bits,M,K,N,explicit_zeros", [(4, 1, 12288, 256, False), (4, 3, 12288, 256, True),
                                                       (8, 1, 5120, 512, False), (8, 2, 4096, 256, False),
                                                       (4, 4, 4096, 512, False), (4, 8, 12288, 256, False),
                                                       (8, 12, 5120, 512, False), (4, 16, 12288, 256, True)])
def test_stream_loads_are_the_same_bits(gpu, hb, orc, hi_prec, monkeypatch, bits, M, K, N, explicit_zeros):
    torch = gpu
    rng = np.random.default_rng(M * 11 + K + N + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        hb.set_hi_prec(True)
        A = (rng.normal(size=(M, K)) * 3).astype(np.float32)
        want = orc.matmul(qw, sc, qz, N, K, bits, A, True)
        for mode in ("1", "0"):
            monkeypatch.setenv("BREEZE_HIP_STREAM", mode)
            assert hb.plan(bits, M, K, N, extra=explicit_zeros)["stream"] == int(mode)
            got = hb.matmul(h, torch.from_numpy(A).cuda(), N).cpu().numpy()
            assert bits_equal(got, want), mode
    finally:
        hb.free(h)


# Phases across tile boundaries (the decode kernel's flow mode): a
# workgroup's tiles form one stream of chunks, a tile ending inside a phase.
# Forced on and off, with and without non-temporal loads, over shapes with
# two to three tiles a workgroup (tiles of 15 chunks, ending on a phase
# boundary, among them), one to three rows, zero points and the argmax:
# every output is the oracle's and every index its first maximum.
@pytest.mark.parametrize("bits,M,K,N,explicit_zeros,argmax", [(4, 1, 4096, 16 * 600, False, False),
                                                              (4, 2, 4096, 16 * 520, True, False),
                                                              (8, 1, 5120, 16 * 700, False, True),
                                                              (8, 3, 2432, 16 * 300, False, True),
                                                              (4, 3, 1920, 16 * 513, False, False)])
def test_flow_phases_are_the_same_bits(gpu, hb, orc, hi_prec, monkeypatch, bits, M, K, N, explicit_zeros, argmax):
    torch = gpu
    rng = np.random.default_rng(M * 13 + K + N + bits)
    qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, explicit_zeros)
    h = hb.prepack(qw, sc, qz, K, N, bits=bits)
    try:
        hb.set_hi_prec(True)
        A = (rng.normal(size=(M, K)) * 2).astype(np.float32)
        want = orc.matmul(qw, sc, qz, N, K, bits, A, True)
        for flow, stream in (("1", "0"), ("1", "1"), ("0", "0")):
            monkeypatch.setenv("BREEZE_HIP_FLOW", flow)
            monkeypatch.setenv("BREEZE_HIP_STREAM", stream)
            p = hb.plan(bits, M, K, N, extra=explicit_zeros, argmax=argmax)
            assert (p["flow"], p["stream"]) == (int(flow), int(stream)), p
            dA = torch.from_numpy(A).cuda()
            if argmax:
                c, idx = hb.matmul_argmax(h, dA, N)
                assert idx.cpu().tolist() == np.argmax(want, axis=1).tolist(), (flow, stream)
            else:
                c = hb.matmul(h, dA, N)
            assert bits_equal(c.cpu().numpy(), want), (flow, stream)
    finally:
        hb.free(h)
