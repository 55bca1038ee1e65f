"""Known answers and invariants that pin the oracle independently of the
reference binary: closed forms, special cases and exact brute force.

Each check is chosen so that a plausible slip in a restatement (a dropped
term, a wrong rounding mode, a swapped index or operand) fails it.
"""
from fractions import Fraction

import numpy as np
import pytest

from conftest import bits_equal


# ---------------------------------------------------------------- fp16 scales

def test_fp16_to_fp32_is_exact_for_every_non_nan_half(orc):
    """quantized_matmul.cpp:157 (_cvtsh_ss): exact for normals, subnormals,
    signed zeros and infinities; NaNs stay NaN with the quiet bit set."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = np.array([orc.half_to_float(int(x)) for x in h], np.float32)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))
    assert np.all(got[nan].view(np.uint32) & 0x00400000)


# ---------------------------------------------------------------- quantizer

@pytest.mark.parametrize("hp,qmax", [(True, 32767), (False, 127)])
def test_quantizer_special_blocks(orc, hp, qmax):
    """quantize_A_i16 / quantize_A (quantized_matmul.cpp:215-258)."""
    A = np.zeros((1, 32 * 5), np.float32)
    A[0, 32:64] = 3.0                                     # constant block
    A[0, 64:96] = np.linspace(-1, 1, 32)                  # max element at both ends
    A[0, 96:128] = np.arange(32) - 15.5                   # .5 products with scale 1
    A[0, 96] = qmax                                       # amax = qmax -> s = 1, inv = 1
    A[0, 128:160] = -np.linspace(0, 2, 32)                # negative maximum
    q, sa, sq = orc.quantize(A, hp)
    assert sa[0, 0] == 0 and not q[0, :32].any() and sq[0, 0] == 0
    assert np.all(q[0, 32:64] == qmax)
    assert q[0, 64] == -qmax and q[0, 95] == qmax
    assert sa[0, 3] == np.float32(1.0)
    ties = A[0, 97:128]
    assert np.array_equal(q[0, 97:128], np.rint(ties).astype(np.int16))  # ties to even
    assert q[0, 97 + 13] == -2 and q[0, 97 + 14] == 0                   # -2.5 -> -2, -0.5 -> 0
    assert q[0, 159] == -qmax
    assert np.array_equal(sq[0], q[0].reshape(5, 32).astype(np.int64).sum(axis=1))


def test_quantizer_closed_form_on_random_blocks(orc):
    """s = amax/qmax and inv = 1/s rounded once each (float32 division),
    q = round-half-even(a*inv) clamped; checked against float64 arithmetic
    rounded to float32 step by step."""
    rng = np.random.default_rng(3)
    A = (rng.normal(size=(4, 32 * 64)) * rng.choice([1e-6, 1.0, 1e4], size=(4, 1))).astype(np.float32)
    for hp, qmax in ((True, 32767), (False, 127)):
        q, sa, _ = orc.quantize(A, hp)
        blk = A.reshape(4, 64, 32).astype(np.float64)
        amax = np.abs(blk).max(axis=2)
        s = (amax / qmax).astype(np.float32)
        inv = (1.0 / s.astype(np.float64)).astype(np.float32)
        prod = (blk * inv[:, :, None].astype(np.float64)).astype(np.float32)
        want = np.clip(np.rint(prod), -qmax, qmax).astype(np.int16).reshape(4, -1)
        assert bits_equal(sa, s)
        assert np.array_equal(q, want)


def test_hi_lo_split_reassembles_q(orc):
    """hi = (q+32768) >> 8, lo = (q+32768) & 255, so q = 256*hi + lo - 32768
    (quantized_matmul.cpp:249-252) for every INT16 value the quantizer makes."""
    q = np.arange(-32767, 32768, dtype=np.int16)
    hi, lo = orc.split_hilo(q)
    assert np.array_equal(256 * hi.astype(np.int32) + lo - 32768, q.astype(np.int32))


# ---------------------------------------------------------------- weights

@pytest.mark.parametrize("bits", [4, 8])
def test_unpack_follows_matmulnbits(orc, bits):
    """b = q - zp with the low nibble first and default zp 8 (INT4) / 128 (INT8)
    (breeze/quant.py:9-58), explicit INT4 zero points packed two per byte."""
    rng = np.random.default_rng(9)
    N, K = 16, 96
    qw = rng.integers(0, 256, (N, K // 32, 4 * bits), dtype=np.uint8)
    sc = rng.uniform(0.001, 0.01, (N, K // 32)).astype(np.float16)
    qz = rng.integers(0, 256, (N, 2), dtype=np.uint8) if bits == 4 else None
    b, sb = orc.unpack_nbits(qw, sc, qz, N, K, bits)
    if bits == 8:
        want = qw.reshape(N, K).astype(np.int16) - 128
    else:
        nib = np.stack([qw & 15, qw >> 4], axis=-1).reshape(N, K // 32, 32).astype(np.int16)
        zp = np.stack([qz & 15, qz >> 4], axis=-1).reshape(N, 4)[:, :K // 32].astype(np.int16)
        want = (nib - zp[:, :, None]).reshape(N, K)
    assert np.array_equal(b, want)
    assert bits_equal(sb, sc.astype(np.float32))


# ---------------------------------------------------------------- integer dots and chain

def test_block_dots_brute_force(orc):
    """cs[m,n,j] = sum_k q*b over block j, exact in int64."""
    rng = np.random.default_rng(4)
    q = rng.integers(-32767, 32768, (3, 128), dtype=np.int16)
    b = rng.integers(-128, 128, (5, 128), dtype=np.int16)
    cs = orc.block_dots(q, b)
    for m in range(3):
        for n in range(5):
            for j in range(4):
                want = sum(int(q[m, 32 * j + k]) * int(b[n, 32 * j + k]) for k in range(32))
                assert cs[m, n, j] == want


def _fma_exact(a, b, c):
    """Round-to-nearest-even float32 of the exact a*b + c."""
    x = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if x == 0:
        return np.float32(0.0) if (float(a) * float(b) >= 0 and float(c) >= 0) else np.float32(-0.0)
    f = np.float32(float(x))  # within an ulp of x
    lo, hi = (np.nextafter(f, np.float32(-np.inf)), f) if Fraction(float(f)) > x else \
             (f, np.nextafter(f, np.float32(np.inf)))
    dlo, dhi = x - Fraction(float(lo)), Fraction(float(hi)) - x
    if dlo < dhi:
        return lo
    if dhi < dlo:
        return hi
    return lo if (lo.view(np.uint32) & 1) == 0 else hi


def test_chain_is_fma_in_block_order(orc):
    """C = fold over j ascending of fma(sa, f32(cs)*sb, acc) from +0
    (quantized_matmul.cpp:311-315), checked against exact rational
    arithmetic with one rounding per step."""
    rng = np.random.default_rng(6)
    M, N, nblk = 2, 3, 40
    cs = rng.integers(-(1 << 22), 1 << 22, (M, N, nblk), dtype=np.int32)
    sa = rng.uniform(1e-5, 1e-1, (M, nblk)).astype(np.float32)
    sb = rng.uniform(1e-4, 1e-2, (N, nblk)).astype(np.float32)
    C = orc.chain(cs, sa, sb)
    for m in range(M):
        for n in range(N):
            acc = np.float32(0.0)
            for j in range(nblk):
                f = np.float32(np.float32(cs[m, n, j]) * sb[n, j])
                acc = _fma_exact(sa[m, j], f, acc)
            assert C[m, n].view(np.uint32) == acc.view(np.uint32), (m, n)


def test_numpy_fma_emulation_is_exact():
    rng = np.random.default_rng(8)
    from oracle import oracle

    a = (rng.normal(size=400) * 10.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    b = (rng.normal(size=400) * 10.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    c = (rng.normal(size=400) * 10.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    got = oracle.fma_f32(a, b, c)
    want = np.array([_fma_exact(x, y, z) for x, y, z in zip(a, b, c)], np.float32)
    assert bits_equal(got, want)


# ---------------------------------------------------------------- end to end

@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("hp", [True, False])
def test_exact_known_answer(orc, bits, hp):
    """All weights w = 1 (nibble 9 / byte 129), scale 1/8, activations
    k * 2^e with one exponent e per row and a maximum of qmax * 2^e in every
    block, so each block scale is exactly 2^e.  Quantization, the integer
    dot and every step of the FP32 chain are then exact (all partial sums
    are multiples of 2^e below 2^22 * 2^e), so
    C[m, n] = sum_k a[m, k] / 8 with no rounding at all."""
    N, K = 16, 128
    qmax = 32767 if hp else 127
    qw = np.full((N, K // 32, 4 * bits), 0x99 if bits == 4 else 129, np.uint8)
    sc = np.full((N, K // 32), 0.125, np.float32)
    rng = np.random.default_rng(12)
    A = np.zeros((3, K), np.float32)
    for m in range(3):
        e = int(rng.integers(-8, 4))
        for j in range(K // 32):
            ints = rng.integers(-qmax, qmax + 1, 32)
            ints[0] = qmax                       # amax = qmax * 2^e -> s = 2^e exactly
            A[m, 32 * j:32 * j + 32] = (ints * 2.0 ** e).astype(np.float32)
    C = orc.matmul(qw, sc, None, N, K, bits, A, hp)
    want = (A.astype(np.float64).sum(axis=1) / 8.0).astype(np.float32)
    assert np.array_equal(C, np.repeat(want[:, None], N, axis=1))


def test_cosine_against_float_dequant(orc):
    """tests/test_qwen35_cpu.py:196-208 of the reference: projection widths,
    seed 3, cosine >= 0.999999 against the float MatMulNBits dequant."""
    from oracle import oracle

    for K, N, bits in ((5120, 48, 8), (17408, 16, 4), (6144, 64, 8), (4096, 32, 4)):
        rng = np.random.default_rng(3)
        qw = rng.integers(0, 256, (N, K // 32, 32 * bits // 8), dtype=np.uint8)
        sc = rng.uniform(0.001, 0.005, (N, K // 32)).astype(np.float32)
        a = rng.normal(size=(3, K)).astype(np.float32)
        W = oracle.dequantize_matmul_nbits(qw, sc, None, bits=bits, block_size=32, K=K, N=N)
        got = orc.matmul(qw, sc, None, N, K, bits, a, True)
        assert oracle.compare_logits(got, a.astype(np.float64) @ W, 0.999999) >= 0.999999


def test_rows_are_independent(orc):
    """Row m of an M-row call equals the row alone (test_cpu_packing.py:155-168)."""
    rng = np.random.default_rng(14)
    N, K = 32, 256
    qw = rng.integers(0, 256, (N, K // 32, 16), dtype=np.uint8)
    sc = rng.uniform(0.001, 0.01, (N, K // 32)).astype(np.float32)
    A = rng.normal(size=(11, K)).astype(np.float32)
    full = orc.matmul(qw, sc, None, N, K, 4, A, True)
    for m in (0, 7, 8, 10):
        assert bits_equal(orc.matmul(qw, sc, None, N, K, 4, A[m:m + 1], True)[0], full[m])


def test_numpy_twin_agrees_with_c_oracle_including_block_integers(orc):
    from oracle import oracle

    rng = np.random.default_rng(15)
    for bits in (4, 8):
        N, K = 48, 320
        qw = rng.integers(0, 256, (N, K // 32, 4 * bits), dtype=np.uint8)
        qw.reshape(-1)[:8] = [0, 1, 7, 15, 127, 128, 254, 255]
        sc = rng.uniform(1e-4, 0.02, (N, K // 32)).astype(np.float16)
        qz = rng.integers(0, 256, (N, 5), dtype=np.uint8) if bits == 4 else None
        A = rng.normal(size=(6, K)).astype(np.float32)
        for hp in (True, False):
            c1, cs1 = orc.matmul(qw, sc, qz, N, K, bits, A, hp, want_cs=True)
            c2, cs2 = oracle.matmul_np(qw, sc, qz, N, K, bits, A, hp, want_cs=True)
            assert np.array_equal(cs1, cs2)
            assert bits_equal(c1, c2)
