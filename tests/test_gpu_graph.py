"""The GPU path inside a captured HIP graph: the per-layer sequence of the
decoder's MLP (qwen35_decoder.cpp:405-409: gate and up projections, SiLU
times up, down projection) and the LM head's argmax, captured once after one
uncaptured call per shape on the capturing stream (which sizes that
stream's device scratch) and replayed.  Every replay is checked bit for bit
against the same sequence run eagerly on the same inputs, with eager work and
synchronisations between the replays."""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def _mlp(hb, torch, hg, hu, hd, x, inter, H):
    g = hb.matmul(hg, x, inter)
    u = hb.matmul(hu, x, inter)
    return hb.matmul(hd, torch.nn.functional.silu(g) * u, H)


# Hidden sizes past 4096 put the gate and up projections on the stand-alone
# quantizer and the eight-row groups (8 rows: one group, W4 with zero points;
# 16 rows: two, W8).
@pytest.mark.parametrize("rows,bits,H,inter", [(1, 4, 512, 1024), (4, 4, 512, 1024), (64, 8, 512, 1024),
                                               (8, 4, 5120, 1024), (16, 8, 4640, 2048)])
def test_captured_mlp_block_replays_bit_exact(gpu, hb, hi_prec, rows, bits, H, inter):
    torch = gpu
    rng = np.random.default_rng(rows + bits)
    hs = []
    for K, N in ((H, inter), (H, inter), (inter, H)):
        qw, sc, qz = rng_weights(rng, N, K, bits, np.float32, bits == 4)
        hs.append(hb.prepack(qw, sc, qz, K, N, bits=bits))
    try:
        hb.set_hi_prec(True)
        inputs = [torch.from_numpy(rng.normal(size=(rows, H)).astype(np.float32)).cuda() for _ in range(4)]
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            want = [_mlp(hb, torch, *hs, x, inter, H) for x in inputs]  # also the uncaptured first calls
        torch.cuda.synchronize()

        x_static = inputs[0].clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            y_static = _mlp(hb, torch, *hs, x_static, inter, H)
        for i, x in enumerate(inputs):
            x_static.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            assert bits_equal(y_static.cpu().numpy(), want[i].cpu().numpy()), (rows, bits, i)
            # Eager work between replays.
            again = _mlp(hb, torch, *hs, inputs[(i + 1) % len(inputs)], inter, H)
            torch.cuda.synchronize()
            assert bits_equal(again.cpu().numpy(), want[(i + 1) % len(inputs)].cpu().numpy())
    finally:
        for h in hs:
            hb.free(h)


def test_captured_argmax_replays_exact(gpu, hb, hi_prec):
    torch = gpu
    K, N = 1024, 16 * 600
    rng = np.random.default_rng(5)
    qw, sc, _ = rng_weights(rng, N, K, 8)
    h = hb.prepack(qw, sc, None, K, N, bits=8)
    try:
        hb.set_hi_prec(True)
        inputs = [torch.from_numpy(rng.normal(size=(1, K)).astype(np.float32)).cuda() for _ in range(3)]
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            want = [hb.matmul_argmax(h, x, N) for x in inputs]
        torch.cuda.synchronize()
        x_static = inputs[0].clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            logits, idx = hb.matmul_argmax(h, x_static, N)
        for i, x in enumerate(inputs):
            x_static.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            assert bits_equal(logits.cpu().numpy(), want[i][0].cpu().numpy()), i
            assert idx.cpu().tolist() == want[i][1].cpu().tolist(), i
            _ = hb.matmul_argmax(h, inputs[(i + 2) % len(inputs)], N)  # eager call between replays
            torch.cuda.synchronize()
    finally:
        hb.free(h)
