"""qp_dispatch_noalloc: the prefill matmul through the entry point that allocates nothing (its workspace is the
library's fixed device scratch array) gives exactly qp_dispatch's results, on two calls in a row (the second with
fewer tokens), with split-K and with the 256-token tiles; where qp_dispatch's split-K partials would not fit the
scratch (the 8B model's 4096 x 14336 and 4096 x 4096 matmuls from 64 tokens on), it splits K fewer times and stays
within the matmul's error bound of the float64 product (2e-5 sum |w x|); a call whose input planes alone would not
fit fails with QP_E_ARG; and the calls can be captured in a HIP graph, whose replays (fresh inputs uploaded
between them) match the eager calls: the plain matmul, the fused gate/up/SwiGLU matmul, and a matmul asked to
reuse the previous call's input planes (P[4] = 1), which a capture must not take from eager state."""
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


def glu(q, b, fmt, wg, wu, N, K, T, x, noalloc):
    y = b.put(np.zeros((T, N), np.float32))
    q.dispatch("matmul_%s_t_swiglu" % capi.FMT_NAME[fmt], [("u", N), ("u", K)],
               [b.put(np.array([T, 0, 0, 0], np.uint32)), wg, wu, b.put(x), y], ((N + 63) // 64, 1, (T + 31) // 32),
               noalloc=noalloc)
    return q.download(y, (T, N))


@pytest.mark.parametrize("N,K,T", [(4096, 14336, 256), (4096, 4096, 64), (4096, 14336, 64)])
def test_noalloc_splits_k_less_where_the_partials_do_not_fit(quipu, oracle, N, K, T):
    """The 8B model's wo / down shapes, whose split-K partials qp_dispatch keeps in a larger workspace: through the
    fixed scratch the K range is split fewer times, and both results stay within 2e-5 sum |w x| of the float64
    product."""
    fmt = capi.Q4_K
    b = Bufs(quipu)
    try:
        raw = raw_matrix(fmt, N, K, 6)
        w = b.matrix(fmt, N, K, 6)
        x = np.random.default_rng(7).standard_normal((T, K)).astype(np.float32)
        want = matmul(quipu, b, fmt, w, N, K, T, x, False)
        got = matmul(quipu, b, fmt, w, N, K, T, x, True)
        W = oracle.dequant(fmt, raw, N * K).reshape(N, K).astype(np.float64)
        exact = x.astype(np.float64) @ W.T
        bound = 2e-5 * (np.abs(x).astype(np.float64) @ np.abs(W).T)
        for r in (want, got):
            assert np.isfinite(r).all()
            assert np.all(np.abs(r - exact) <= bound), float(np.max(np.abs(r - exact) - bound))
    finally:
        b.close()


def test_noalloc_fused_swiglu_matmul_eager_and_captured(quipu):
    """matmul_q4k_t_swiglu (gate, up and SwiGLU in one matrix-core launch) through qp_dispatch_noalloc: bit for bit
    qp_dispatch's result on two calls in a row (the second smaller), and inside a captured graph replayed three
    times with fresh inputs."""
    fmt, N, K = capi.Q4_K, 512, 2048
    b = Bufs(quipu)
    try:
        wg, wu = b.matrix(fmt, N, K, 11), b.matrix(fmt, N, K, 12)
        for i, T in enumerate((300, 256)):
            x = np.random.default_rng(30 + i).standard_normal((T, K)).astype(np.float32)
            want = glu(quipu, b, fmt, wg, wu, N, K, T, x, False)
            got = glu(quipu, b, fmt, wg, wu, N, K, T, x, True)
            assert np.isfinite(got).all()
            np.testing.assert_array_equal(got, want)
        T = 256
        paso = b.put(np.array([T, 0, 0, 0], np.uint32))
        xb = b.put(np.zeros((T, K), np.float32))
        yb = b.put(np.zeros((T, N), np.float32))
        quipu.graph_begin()
        try:
            quipu.dispatch("matmul_q4k_t_swiglu", [("u", N), ("u", K)], [paso, wg, wu, xb, yb],
                           ((N + 63) // 64, 1, T // 32), noalloc=True)
        finally:
            g = quipu.graph_end()
        try:
            for r in range(3):
                x = np.random.default_rng(40 + r).standard_normal((T, K)).astype(np.float32)
                quipu.upload(xb, x)
                quipu.graph_launch(g)
                got = quipu.download(yb, (T, N))
                want = glu(quipu, b, fmt, wg, wu, N, K, T, x, False)
                np.testing.assert_array_equal(got, want)
        finally:
            quipu.graph_free(g)
    finally:
        b.close()


def test_noalloc_reuse_of_input_planes_is_not_taken_from_eager_state_while_capturing(quipu):
    """P[4] = 1 asks a matmul to reuse the input planes of the previous prefill matmul when they are still there.
    An eager call leaves the planes of x in the scratch; a capture that then asks for reuse must still record the
    split, since the replays run later, after other calls have overwritten the scratch."""
    fmt, N, K, T = capi.Q4_K, 300, 2048, 200
    b = Bufs(quipu)
    try:
        w = b.matrix(fmt, N, K, 13)
        paso = b.put(np.array([T, 0, 0, 0], np.uint32))
        xb = b.put(np.random.default_rng(50).standard_normal((T, K)).astype(np.float32))
        yb = b.put(np.zeros((T, N), np.float32))
        u = [("u", N), ("u", K), ("u", 0), ("u", 0)]
        grid = ((N + 63) // 64, 1, (T + 31) // 32)
        quipu.dispatch("matmul_q4k_t", u, [paso, w, xb, yb], grid, noalloc=True)  # planes of xb in the scratch
        quipu.graph_begin()
        try:
            quipu.dispatch("matmul_q4k_t", u + [("u", 1)], [paso, w, xb, yb], grid, noalloc=True)
        finally:
            g = quipu.graph_end()
        try:
            for r in range(3):
                other = np.random.default_rng(60 + r).standard_normal((T, K)).astype(np.float32)
                matmul(quipu, b, fmt, w, N, K, T, other, True)  # overwrites the scratch's planes
                x = np.random.default_rng(70 + r).standard_normal((T, K)).astype(np.float32)
                quipu.upload(xb, x)
                quipu.graph_launch(g)
                got = quipu.download(yb, (T, N))
                np.testing.assert_array_equal(got, matmul(quipu, b, fmt, w, N, K, T, x, True))
        finally:
            quipu.graph_free(g)
    finally:
        b.close()


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
