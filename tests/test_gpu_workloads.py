"""GPU parity at the benchmark workloads' full sizes.

Each workload's seeded inputs (oracle.make_config) go through the device
entry point and are compared bit-for-bit with the C restatement of the
reference arithmetic, in the reference's high-precision (two-pass INT16)
activation mode that the workloads specify.  The LM head also checks the
fused argmax index exactly; the prefill workloads compare all 512 rows (the
oracle computes its outputs on every core, one output per task, which
changes no bit).
"""
import numpy as np
import pytest

from conftest import bits_equal

pytestmark = pytest.mark.gpu


def _device_matmul(hb, torch, h, A, N, argmax=False):
    dA = torch.from_numpy(A).cuda()
    if argmax:
        c, idx = hb.matmul_argmax(h, dA, N)
        torch.cuda.synchronize()
        return c.cpu().numpy(), idx.cpu().numpy()
    c = hb.matmul(h, dA, N)
    torch.cuda.synchronize()
    return c.cpu().numpy()


@pytest.mark.parametrize("name,rows", [
    ("w8_gemv", None),
    ("w4_gemv", None),
    ("w4_decode", 1),
    ("w4_decode", 2),
    ("w4_decode", 4),
    ("w4_decode", 8),
])
def test_decode_workloads_bit_exact(gpu, hb, orc, hi_prec, name, rows):
    from oracle import oracle
    d = oracle.make_config(name, rows)
    N, K, bits = d["N"], d["K"], d["bits"]
    hb.set_hi_prec(True)
    h = hb.prepack(d["qweight"], d["scales"], None, K, N, bits=bits)
    try:
        got = _device_matmul(hb, gpu, h, d["A"], N)
    finally:
        hb.free(h)
    want = orc.matmul(d["qweight"], d["scales"], None, N, K, bits, d["A"], True)
    assert bits_equal(got, want), (name, rows, float(np.max(np.abs(got - want))))


def test_lm_head_logits_and_argmax(gpu, hb, orc, hi_prec):
    from oracle import oracle
    d = oracle.make_config("w8_lmhead")
    N, K = d["N"], d["K"]
    hb.set_hi_prec(True)
    h = hb.prepack(d["qweight"], d["scales"], None, K, N, bits=8)
    try:
        logits, idx = _device_matmul(hb, gpu, h, d["A"], N, argmax=True)
    finally:
        hb.free(h)
    want = orc.matmul(d["qweight"], d["scales"], None, N, K, 8, d["A"], True)
    assert bits_equal(logits, want)
    assert idx.tolist() == np.argmax(want, axis=1).tolist()


@pytest.mark.parametrize("name,rows", [("w8_prefill", None), ("w4_prefill", None), ("w8_prefill", 16),
                                       ("w4_prefill", 100)])
def test_prefill_rows_bit_exact(gpu, hb, orc, hi_prec, name, rows):
    """All 512 rows, and the first 16 or 100 rows alone (32-row workgroups,
    and 128-row workgroups at another column width)."""
    from oracle import oracle
    d = oracle.make_config(name, rows)
    N, K, bits = d["N"], d["K"], d["bits"]
    hb.set_hi_prec(True)
    h = hb.prepack(d["qweight"], d["scales"], None, K, N, bits=bits)
    try:
        got = _device_matmul(hb, gpu, h, d["A"], N)
    finally:
        hb.free(h)
    want = orc.matmul(d["qweight"], d["scales"], None, N, K, bits, d["A"], True)
    bad = np.nonzero(np.any(got.view(np.uint32) != want.view(np.uint32), axis=1))[0]
    assert bad.size == 0, (name, rows, bad[:10].tolist())
