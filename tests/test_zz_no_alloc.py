"""qp_dispatch_noalloc: the prefill matmul through the entry point that allocates nothing (its workspace is the
library's fixed device scratch array) gives exactly qp_dispatch's results, on two calls in a row (the second with
fewer tokens), with split-K and with the 256-token tiles; a call whose workspace would not fit fails with
QP_E_ARG; and the call can be captured in a HIP graph, whose replays (fresh inputs uploaded between them) match the
eager calls."""
import numpy as np
import pytest

from quipullm_amd import capi, synth

pytestmark = pytest.mark.gpu


def raw_matrix(fmt, N, K, seed):
    return np.frombuffer(synth.gen_blocks(np.random.default_rng(seed), fmt, N * K, "w"), np.uint8)


class Bufs:
    def __init__(self, q):
        self.q, self.hs = q, []

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        h = self.q.alloc(arr.nbytes)
        self.q.upload(h, arr)
        self.hs.append(h)
        return h

    def matrix(self, fmt, N, K, seed):
        h = self.q.upload_matrix(fmt, raw_matrix(fmt, N, K, seed), N, K)
        self.hs.append(h)
        return h

    def close(self):
        for h in self.hs:
            self.q.free(h)


def matmul(q, b, fmt, w, N, K, T, x, noalloc):
    y = b.put(np.zeros((T, N), np.float32))
    q.dispatch("matmul_%s_t" % capi.FMT_NAME[fmt], [("u", N), ("u", K), ("u", 0), ("u", 0)],
               [b.put(np.array([T, 0, 0, 0], np.uint32)), w, b.put(x), y], ((N + 63) // 64, 1, (T + 31) // 32),
               noalloc=noalloc)
    return q.download(y, (T, N))


@pytest.mark.parametrize("fmt,N,K,Ts", [(capi.Q4_K, 300, 2048, (200, 70)), (capi.Q6_K, 512, 1024, (300, 64))])
def test_noalloc_matches_dispatch(quipu, fmt, N, K, Ts):
    b = Bufs(quipu)
    try:
        w = b.matrix(fmt, N, K, 3)
        for i, T in enumerate(Ts):  # two calls in a row, the second smaller
            x = np.random.default_rng(10 + i).standard_normal((T, K)).astype(np.float32)
            want = matmul(quipu, b, fmt, w, N, K, T, x, False)
            got = matmul(quipu, b, fmt, w, N, K, T, x, True)
            assert np.isfinite(got).all()
            np.testing.assert_array_equal(got, want)
    finally:
        b.close()


def test_noalloc_rejects_a_workspace_past_the_scratch(quipu):
    b = Bufs(quipu)
    try:
        N, K, T = 256, 14336, 1024  # split planes alone: 4 * 1024 * 14336 bytes = 56 MiB
        w = b.matrix(capi.Q4_K, N, K, 4)
        x = np.zeros((T, K), np.float32)
        with pytest.raises(capi.QuipuError) as e:
            matmul(quipu, b, capi.Q4_K, w, N, K, T, x, True)
        assert "scratch" in str(e.value)
    finally:
        b.close()


def test_noalloc_matmul_in_a_captured_graph(quipu):
    fmt, N, K, T = capi.Q4_K, 300, 2048, 200
    b = Bufs(quipu)
    try:
        w = b.matrix(fmt, N, K, 5)
        paso = b.put(np.array([T, 0, 0, 0], np.uint32))
        xb = b.put(np.zeros((T, K), np.float32))
        yb = b.put(np.zeros((T, N), np.float32))
        u = [("u", N), ("u", K), ("u", 0), ("u", 0)]
        grid = ((N + 63) // 64, 1, (T + 31) // 32)
        quipu.graph_begin()
        try:
            quipu.dispatch("matmul_q4k_t", u, [paso, w, xb, yb], grid, noalloc=True)
        finally:
            g = quipu.graph_end()
        try:
            for r in range(3):
                x = np.random.default_rng(20 + r).standard_normal((T, K)).astype(np.float32)
                quipu.upload(xb, x)
                quipu.graph_launch(g)
                got = quipu.download(yb, (T, N))
                want = matmul(quipu, b, fmt, w, N, K, T, x, True)  # eager, between the replays
                np.testing.assert_array_equal(got, want)
        finally:
            quipu.graph_free(g)
    finally:
        b.close()
