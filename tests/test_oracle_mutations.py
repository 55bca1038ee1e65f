"""The checks that pin the oracle have teeth.

Plausible mistakes are planted in a copy of the NumPy restatement (never in
the product): each mutant must disagree with the reference kernel's golden
outputs (tests/golden/ref_vectors.npz) on at least one case, while the
unmutated restatement agrees with all of them.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits_equal

Z = np.load(os.path.join(GOLDEN, "ref_vectors.npz"))
META = json.loads(bytes(Z["meta"]).decode())
CASES = sorted(n for n in META if n.startswith(("pack", "edge")))


def _twin(qweight, scales, qzeros, N, K, bits, A, hp, mut=None):
    """The NumPy restatement with an optional planted mistake."""
    from oracle import oracle

    b, sb = oracle.unpack_nbits_np(qweight, scales, qzeros, N, K, bits)
    if mut == "nibble_order" and bits == 4:
        qw = np.ascontiguousarray(qweight).reshape(N, K // 32, 16)
        nib = np.empty((N, K // 32, 32), np.int16)
        nib[:, :, 0::2] = qw >> 4
        nib[:, :, 1::2] = qw & 15
        b = (nib - 8).reshape(N, K) if qzeros is None else b
    if mut == "int4_zero_point_7" and bits == 4 and qzeros is None:
        b = b + 1
    if mut == "int8_zero_point_127" and bits == 8:
        b = b + 1
    qmax = 32767 if hp else 127
    blk = np.ascontiguousarray(A, np.float32).reshape(A.shape[0], K // 32, 32)
    mag = np.abs(blk)
    amax = np.max(np.where(np.isnan(mag), np.float32(0), mag), axis=2, initial=np.float32(0))
    sa = (amax / np.float32(qmax)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        if mut == "inverse_in_one_division":
            inv = np.where(amax > 0, np.float32(qmax) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
        else:
            inv = np.where(sa > 0, np.float32(1) / np.where(sa > 0, sa, 1), 0).astype(np.float32)
        p = (blk * inv[:, :, None]).astype(np.float32)
    p = np.where(np.isfinite(p), p, np.float32(0))
    if mut == "round_half_away":
        r = np.sign(p) * np.floor(np.abs(p) + np.float32(0.5))
    else:
        r = np.rint(p)
    q = np.clip(r, -qmax, qmax).astype(np.int64)
    if mut == "drop_low_byte" and hp:
        q = ((q + 32768) >> 8 << 8) - 32768 + 128
    cs = oracle.block_dots_np(q.reshape(A.shape[0], K).astype(np.int16), b).astype(np.int64)
    if mut == "sign_flip_weights":
        cs = -cs
    M = A.shape[0]
    acc = np.zeros((M, N), np.float32)
    order = range(K // 32 - 1, -1, -1) if mut == "reverse_block_order" else range(K // 32)
    for j in order:
        f = (cs[:, :, j].astype(np.float32) * sb[None, :, j]).astype(np.float32)
        s = np.broadcast_to(sa[:, j:j + 1], (M, N))
        if mut == "mul_then_add":
            acc = (acc + (s * f).astype(np.float32)).astype(np.float32)
        elif mut == "activation_scale_of_row0":
            acc = oracle.fma_f32(np.broadcast_to(sa[:1, j:j + 1], (M, N)), f, acc)
        else:
            acc = oracle.fma_f32(s, f, acc)
    return acc


def _agrees(mut):
    for name in CASES:
        m = META[name]
        for hp in (1, 0):
            got = _twin(Z[f"{name}_qweight"], Z[f"{name}_scales"],
                        Z[f"{name}_qzeros"] if f"{name}_qzeros" in Z.files else None,
                        m["N"], m["K"], m["bits"], Z[f"{name}_A"], bool(hp), mut)
            if not bits_equal(got, Z[f"{name}_C_hp{hp}"]):
                return False
    return True


def test_unmutated_restatement_agrees():
    assert _agrees(None)


@pytest.mark.parametrize("mut", [
    "mul_then_add", "reverse_block_order", "round_half_away", "inverse_in_one_division",
    "drop_low_byte", "nibble_order", "int4_zero_point_7", "int8_zero_point_127",
    "sign_flip_weights", "activation_scale_of_row0",
])
def test_planted_mistake_is_caught(mut):
    assert not _agrees(mut), f"golden vectors do not detect the planted mistake {mut!r}"
