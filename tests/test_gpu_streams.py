"""Device scratch under concurrency and graph capture.

The library keeps its device scratch (stand-alone quantizer records,
prefill records, argmax state) per (device, stream).  Calls on two streams
of one device therefore never share it; a buffer that has to grow is
replaced without freeing the old one, so a graph captured earlier keeps
valid addresses; and a call that would have to allocate while its stream is
capturing fails with an error instead of breaking the capture.  Every value
is checked against the oracle or the eager result, bit for bit.
"""
import numpy as np
import pytest

from conftest import bits_equal, rng_weights

pytestmark = pytest.mark.gpu


def test_two_streams_on_one_device(gpu, hb, orc, hi_prec):
    """Interleaved calls on two streams, each shape using scratch: staged
    decode records (4 rows of K = 4608 on the four-row groups, 8 and 20 rows
    on the eight-row groups), prefill records (130 rows) and the decode
    argmax state (1 row, and 8 rows on the eight-row groups).  Each stream's
    outputs equal the oracle's."""
    torch = gpu
    N, K = 256, 4608
    rng = np.random.default_rng(77)
    qw, sc, _ = rng_weights(rng, N, K, 8)
    h = hb.prepack(qw, sc, None, K, N, bits=8)
    hb.set_hi_prec(True)
    try:
        main = torch.cuda.current_stream()
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        cases = []
        for rows, am in ((4, False), (8, False), (20, False), (130, False), (1, True), (8, True)):
            for s in streams:
                A = rng.normal(size=(rows, K)).astype(np.float32)
                cases.append((s, A, torch.from_numpy(A).cuda(), am))
        for s in streams:
            s.wait_stream(main)
        outs = []
        for _ in range(2):
            for s, A, dA, am in cases:
                with torch.cuda.stream(s):
                    if am:
                        outs.append(hb.matmul_argmax(h, dA, N))
                    else:
                        outs.append((hb.matmul(h, dA, N), None))
        torch.cuda.synchronize()
        for i, (c, idx) in enumerate(outs):
            A = cases[i % len(cases)][1]
            want = orc.matmul(qw, sc, None, N, K, 8, A, True)
            assert bits_equal(c.cpu().numpy(), want), i
            if idx is not None:
                assert idx.cpu().tolist() == np.argmax(want, axis=1).tolist(), i
    finally:
        hb.free(h)


def test_capture_that_would_allocate_raises(gpu, hb, hi_prec):
    """A shape whose scratch the capturing stream does not hold yet raises a
    clear error; nothing is allocated inside the capture."""
    torch = gpu
    N, K = 64, 4608
    rng = np.random.default_rng(78)
    qw, sc, _ = rng_weights(rng, N, K, 8)
    h = hb.prepack(qw, sc, None, K, N, bits=8)
    hb.set_hi_prec(True)
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        x = torch.from_numpy(rng.normal(size=(8, K)).astype(np.float32)).cuda()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="capturing"):
            with torch.cuda.graph(graph, stream=s):
                hb.matmul(h, x, N)
        torch.cuda.synchronize()
        # The stream works normally afterwards.
        with torch.cuda.stream(s):
            y = hb.matmul(h, x, N)
        torch.cuda.synchronize()
        assert bits_equal(y.cpu().numpy(), hb.matmul(h, x.cpu().numpy(), N))
    finally:
        hb.free(h)


def test_graph_survives_scratch_growth(gpu, hb, hi_prec):
    """A graph captured with 4-row staged records keeps replaying bit-exact
    after eager calls on its stream grew that scratch (8 rows, then 130
    rows through the prefill records)."""
    torch = gpu
    N, K = 128, 4608
    rng = np.random.default_rng(79)
    qw, sc, _ = rng_weights(rng, N, K, 4)
    h = hb.prepack(qw, sc, None, K, N, bits=4)
    hb.set_hi_prec(True)
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        inputs = [torch.from_numpy(rng.normal(size=(4, K)).astype(np.float32)).cuda() for _ in range(3)]
        big = [torch.from_numpy(rng.normal(size=(r, K)).astype(np.float32)).cuda() for r in (8, 130)]
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            want = [hb.matmul(h, x, N) for x in inputs]  # also sizes the stream's scratch for 4 rows
        torch.cuda.synchronize()
        x_static = inputs[0].clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            y_static = hb.matmul(h, x_static, N)
        for i in range(4):
            x_static.copy_(inputs[i % 3])
            graph.replay()
            torch.cuda.synchronize()
            assert bits_equal(y_static.cpu().numpy(), want[i % 3].cpu().numpy()), i
            if i < 2:
                with torch.cuda.stream(s):
                    grown = hb.matmul(h, big[i], N)
                torch.cuda.synchronize()
                assert bits_equal(grown.cpu().numpy(), hb.matmul(h, big[i].cpu().numpy(), N)), i
    finally:
        hb.free(h)
