"""Op-level parity of the gfx950 kernels against the CPU oracle, through the C ABI (ctypes).

Bars: dequantization, embedding rows, KV appends and argmax are bit-exact; the dot products follow their own
summation order on the GPU, so they are held to an absolute bound proportional to sum |x_k w_k| (float32
rounding of a K-term sum in any order); the other float kernels to small relative bounds stated per test.

Every dispatch here uses buffers sized exactly as the kernel indexes them (shapes are checked by the op table
on the host before any launch).
"""
import numpy as np
import pytest

import refs
from quipullm_amd import capi, synth

pytestmark = pytest.mark.gpu

FMTS = [capi.Q2_K, capi.Q3_K, capi.Q4_K, capi.Q5_K, capi.Q6_K, capi.Q8_0, capi.F32, capi.IQ4_NL]
PLANAR = (capi.Q8_0, capi.IQ4_NL)  # bound as two buffers: quants, then the f16 scales after them


def raw_matrix(fmt, N, K, seed, centered=False):
    if fmt == capi.F32:
        return np.random.default_rng(seed).standard_normal(N * K).astype(np.float32).view(np.uint8)
    return np.frombuffer(synth.gen_blocks(np.random.default_rng(seed), fmt, N * K, "w", centered), np.uint8)


def dot_bound(W, x, rel=2e-5):
    """Absolute error allowed for y = W x in float32: rel * sum_k |w_k x_k| per row."""
    return rel * (np.abs(W.astype(np.float64)) @ np.abs(np.asarray(x, np.float64))) + 1e-30


class Dev:
    """Tracks device buffers of one test and frees them."""

    def __init__(self, q):
        self.q, self.hs = q, []

    def buf(self, arr):
        h = self.q.buffer_from(np.ascontiguousarray(arr))
        self.hs.append(h)
        return h

    def zeros(self, nbytes):
        h = self.q.alloc(nbytes)
        self.q.upload(h, np.zeros(nbytes, np.uint8))
        self.hs.append(h)
        return h

    def matrix(self, fmt, raw, N, K):
        h = self.q.upload_matrix(fmt, raw, N, K)
        self.hs.append(h)
        return h

    def paso(self, T, pos0):
        return self.buf(np.array([T, pos0, 0, 0], np.uint32))

    def get(self, h, shape, dtype=np.float32):
        self.q.sync()
        return self.q.download(h, shape, dtype)

    def close(self):
        for h in self.hs:
            self.q.free(h)


@pytest.fixture
def dev(quipu):
    d = Dev(quipu)
    yield d
    d.close()


def test_info(quipu):
    i = quipu.info()
    assert i["arch"].startswith("gfx950") and i["cus"] >= 200


# ------------------------------------------------------------------------------------------------ dequant / embed
@pytest.mark.parametrize("fmt", [capi.Q4_K, capi.Q6_K, capi.Q8_0, capi.IQ4_NL])
@pytest.mark.parametrize("centered", [False, True])
def test_dequant_bit_exact(quipu, dev, oracle, fmt, centered):
    N, K = 96, 1024
    raw = raw_matrix(fmt, N, K, 11, centered)
    h = dev.matrix(fmt, raw, N, K)
    got = quipu.dequant(fmt, h, N * K, K)
    want = oracle.dequant(fmt, raw, N * K)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", FMTS)
def test_embed_rows_bit_exact(quipu, dev, oracle, fmt):
    V, D = 300, 512
    raw = raw_matrix(fmt, V, D, 12)
    w = dev.matrix(fmt, raw, V, D)
    ids = np.array([0, 299, 17, 17, 150], np.uint32)
    T = len(ids)
    y = dev.zeros(T * D * 4)
    nm = "embed_" + capi.FMT_NAME[fmt]
    wb = [w, capi.scale_plane(fmt, w, V, D)] if fmt in PLANAR else [w]
    quipu.dispatch(nm, [("u", D), ("u", V)], [dev.paso(T, 0)] + wb + [dev.buf(ids), y], ((T * D + 255) // 256,))
    got = dev.get(y, (T, D))
    np.testing.assert_array_equal(got.view(np.uint32), oracle.embed(fmt, raw, D, ids).view(np.uint32))


# ------------------------------------------------------------------------------------------------ GEMV
@pytest.mark.parametrize("fmt,N,K", [(capi.Q4_K, 1000, 4096), (capi.Q6_K, 513, 2048), (capi.Q8_0, 700, 1536),
                                     (capi.IQ4_NL, 700, 1536), (capi.F32, 130, 1024), (capi.Q4_K, 64, 14336),
                                     (capi.Q6_K, 40, 14336),
                                     (capi.Q6_K, 700, 9216), (capi.Q4_K, 4100, 15360),
                                     # the planar formats' edges: an odd number of 32-weight blocks per row (a
                                     # partial slot of 64), the input staged in a second round (K > 8192), and
                                     # several passes per workgroup whose item count is not a multiple of two
                                     (capi.Q8_0, 37, 288), (capi.F32, 33, 80), (capi.IQ4_NL, 130, 2080),
                                     (capi.IQ4_NL, 300, 9248), (capi.Q8_0, 100, 12320), (capi.IQ4_NL, 40000, 256),
                                     (capi.Q8_0, 40000, 96)])
def test_matmul_1_reference_op(quipu, dev, oracle, fmt, N, K):
    raw = raw_matrix(fmt, N, K, 13)
    w = dev.matrix(fmt, raw, N, K)
    x = np.random.default_rng(1).standard_normal(K).astype(np.float32)
    y0 = np.random.default_rng(2).standard_normal(N).astype(np.float32)
    W = oracle.dequant(fmt, raw, N * K).reshape(N, K) if fmt != capi.F32 else raw.view(np.float32).reshape(N, K)
    wb = [w, capi.scale_plane(fmt, w, N, K)] if fmt in PLANAR else [w]
    for acc in (0, 1):
        y = dev.buf(y0)
        quipu.dispatch("matmul_%s_1" % capi.FMT_NAME[fmt], [("u", N), ("u", K), ("u", acc), ("u", 0)],
                       [dev.paso(1, 0)] + wb + [dev.buf(x), y], capi.dim2((N + 7) // 8))
        got = dev.get(y, (N,))
        want = oracle.matmul(fmt, raw, N, K, x, y=y0 if acc else None, acc=bool(acc))[0]
        assert np.all(np.abs(got - want) <= dot_bound(W, x) + (2e-7 * np.abs(y0) if acc else 0)), acc


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("R", [1, 2, 4, 8])
def test_gemv_segments_norm_and_persistent_grid(quipu, dev, oracle, fmt, R):
    """Three segments (like Q, K, V) over one RMS-normalized input, the middle one a row window of a larger
    matrix; the grid capped at 5 workgroups so each strides over many row groups."""
    K = 2048
    shapes = [(260, 0, 260), (72, 40, 150), (33, 0, 33)]  # (n, row_base, rows_total)
    x = (np.random.default_rng(3).standard_normal(K) * 2).astype(np.float32)
    nw = (1 + 0.2 * np.random.default_rng(4).standard_normal(K)).astype(np.float32)
    eps = 1e-5
    xn = oracle.rmsnorm(x[None], nw, eps)[0]
    segs, bufs, want, bounds, outs = [], [], [], [], []
    for i, (n, rb, rt) in enumerate(shapes):
        raw = raw_matrix(fmt, rt, K, 20 + i)
        W = (oracle.dequant(fmt, raw, rt * K) if fmt != capi.F32 else raw.view(np.float32)).reshape(rt, K)
        h = dev.matrix(fmt, raw, rt, K)
        y = dev.zeros(n * 4)
        segs.append((capi.STORE, n, rb, rt))
        bufs += [h, 0, y]
        want.append(oracle.matmul(fmt, raw, rt, K, xn)[0][rb:rb + n])
        bounds.append(dot_bound(W[rb:rb + n], xn, 3e-5))
        outs.append((y, n))
    u = capi.gemv_uniform(3, K, eps=eps, R=R, max_wg=5, fmt=fmt, segs=segs)
    quipu.dispatch("gemv", u, [dev.paso(1, 0), dev.buf(x), dev.buf(nw), 0] + bufs)
    for (y, n), w_, b in zip(outs, want, bounds):
        got = dev.get(y, (n,))
        assert np.all(np.abs(got - w_) <= b)


@pytest.mark.parametrize("K", [1024, 4096, 12288])
def test_gemv_mixed_k_quant_segments(quipu, dev, oracle, K):
    """Q, K (Q4_K) and V (Q6_K) of the Q4_K_M models in one launch over one RMS-normalized input."""
    x = (np.random.default_rng(14).standard_normal(K) * 2).astype(np.float32)
    nw = (1 + 0.2 * np.random.default_rng(15).standard_normal(K)).astype(np.float32)
    eps = 1e-5
    xn = oracle.rmsnorm(x[None], nw, eps)[0]
    segs, bufs, checks = [], [], []
    for i, (fmt, n) in enumerate([(capi.Q4_K, 200), (capi.Q4_K, 72), (capi.Q6_K, 72)]):
        raw = raw_matrix(fmt, n, K, 80 + i)
        W = oracle.dequant(fmt, raw, n * K).reshape(n, K)
        y = dev.zeros(n * 4)
        segs.append((capi.STORE, n, 0, n, fmt))
        bufs += [dev.matrix(fmt, raw, n, K), 0, y]
        checks.append((y, n, oracle.matmul(fmt, raw, n, K, xn)[0], dot_bound(W, xn, 3e-5)))
    u = capi.gemv_uniform(3, K, eps=eps, fmt=capi.Q4_K, segs=segs)
    quipu.dispatch("gemv", u, [dev.paso(1, 0), dev.buf(x), dev.buf(nw), 0] + bufs)
    for y, n, want, bound in checks:
        assert np.all(np.abs(dev.get(y, (n,)) - want) <= bound)


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_acc_last_row(quipu, dev, oracle, fmt):
    """ACC mode (the residual add of wo / ffn_down) reading the last of T = 3 input rows."""
    N, K, T = 300, 1024, 3
    raw = raw_matrix(fmt, N, K, 30)
    W = (oracle.dequant(fmt, raw, N * K) if fmt != capi.F32 else raw.view(np.float32)).reshape(N, K)
    x = np.random.default_rng(5).standard_normal((T, K)).astype(np.float32)
    y0 = np.random.default_rng(6).standard_normal(N).astype(np.float32)
    y = dev.buf(y0)
    u = capi.gemv_uniform(1, K, last_row=1, fmt=fmt, segs=[(capi.ACC, N, 0, N)])
    quipu.dispatch("gemv", u, [dev.paso(T, 0), dev.buf(x), 0, 0, dev.matrix(fmt, raw, N, K), 0, y])
    got = dev.get(y, (N,))
    want = oracle.matmul(fmt, raw, N, K, x[-1], y=y0, acc=True)[0]
    assert np.all(np.abs(got - want) <= dot_bound(W, x[-1]) + 2e-7 * np.abs(y0))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("R", [2, 4, 8])
def test_gemv_swiglu_pairs(quipu, dev, oracle, fmt, R):
    N, K = 333, 1024
    rg, ru = raw_matrix(fmt, N, K, 40), raw_matrix(fmt, N, K, 41)
    Wg = (oracle.dequant(fmt, rg, N * K) if fmt != capi.F32 else rg.view(np.float32)).reshape(N, K)
    Wu = (oracle.dequant(fmt, ru, N * K) if fmt != capi.F32 else ru.view(np.float32)).reshape(N, K)
    x = np.random.default_rng(7).standard_normal(K).astype(np.float32)
    y = dev.zeros(N * 4)
    u = capi.gemv_uniform(1, K, R=R, fmt=fmt, segs=[(capi.SWIGLU, N, 0, N)])
    quipu.dispatch("gemv", u, [dev.paso(1, 0), dev.buf(x), 0, 0, dev.matrix(fmt, rg, N, K),
                               dev.matrix(fmt, ru, N, K), y])
    got = dev.get(y, (N,))
    g, uu = oracle.matmul(fmt, rg, N, K, x)[0], oracle.matmul(fmt, ru, N, K, x)[0]
    want = oracle.swiglu(g, uu)
    silu = np.abs(g / (1 + np.exp(-g.astype(np.float64))))
    bound = 1.1 * np.abs(uu) * dot_bound(Wg, x) + silu * dot_bound(Wu, x) + 1e-6 * np.abs(want)
    assert np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("fmt", [capi.Q6_K, capi.Q4_K, capi.Q8_0])
def test_gemv_argmax_fused(quipu, dev, oracle, fmt):
    """Output GEMV with the fused device argmax: partial maxima per workgroup, then argmax_fin.  Rows 7 and 900
    are copies of the largest row, so the greedy choice is the lowest index holding that value (strict '>'
    scan)."""
    V, K, maxwg = 1200, 1024, 37
    raw = bytearray(raw_matrix(fmt, V, K, 50).tobytes())
    x = np.random.default_rng(8).standard_normal(K).astype(np.float32)
    W = oracle.dequant(fmt, bytes(raw), V * K).reshape(V, K)
    best = int(np.argmax(W @ x))
    rb = capi.gguf_bytes(fmt, 1, K)
    for dst in (7, 900):
        raw[dst * rb:(dst + 1) * rb] = raw[best * rb:(best + 1) * rb]
    raw = np.frombuffer(bytes(raw), np.uint8)
    W = oracle.dequant(fmt, raw, V * K).reshape(V, K)
    y = dev.zeros(V * 4)
    amax = dev.zeros(8 * maxwg)
    ids = dev.zeros(16)
    toks = dev.zeros(4 * 8)
    step = dev.zeros(16)
    paso = dev.paso(1, 5)
    u = capi.gemv_uniform(1, K, R=2, max_wg=maxwg, fmt=fmt, segs=[(capi.ARGMAX, V, 0, V)])
    fin = [("u", maxwg), ("u", 1), ("u", 8)]
    quipu.dispatch("gemv", u, [paso, dev.buf(x), 0, amax, dev.matrix(fmt, raw, V, K), 0, y])
    quipu.dispatch("argmax_fin", fin, [paso, amax, ids, toks, step])
    logits = dev.get(y, (V,))
    top = min(best, 7)
    assert int(dev.get(ids, (1,), np.uint32)[0]) == top == oracle.argmax(logits)
    assert dev.get(amax, (maxwg,), np.uint64).sum() == 0  # partials cleared for the next launch
    assert list(dev.get(step, (1,), np.uint32)) == [1] and list(dev.get(paso, (2,), np.uint32)) == [1, 6]
    assert dev.get(toks, (1,), np.uint32)[0] == top
    want = oracle.matmul(fmt, raw, V, K, x)[0]
    assert np.all(np.abs(logits - want) <= dot_bound(W, x))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,op", [(3, "4"), (9, "4"), (40, "t"), (70, "t")])
def test_matmul_multi_token(quipu, dev, oracle, fmt, T, op):
    """Prefill matmuls (matmul_<fmt>_4 and the tiled _t), acc on, T rows of x."""
    N, K = 200, 1024
    raw = raw_matrix(fmt, N, K, 60)
    W = (oracle.dequant(fmt, raw, N * K) if fmt != capi.F32 else raw.view(np.float32)).reshape(N, K)
    x = np.random.default_rng(9).standard_normal((T, K)).astype(np.float32)
    y0 = np.random.default_rng(10).standard_normal((T, N)).astype(np.float32)
    y = dev.buf(y0)
    wb = [dev.matrix(fmt, raw, N, K)]
    if fmt in PLANAR:
        wb.append(capi.scale_plane(fmt, wb[0], N, K))
    grid = ((N + 63) // 64, 1, (T + 31) // 32) if op == "t" else capi.dim2((N + 7) // 8) + ((T + 3) // 4,)
    quipu.dispatch("matmul_%s_%s" % (capi.FMT_NAME[fmt], op), [("u", N), ("u", K), ("u", 1), ("u", 0)],
                   [dev.paso(T, 0)] + wb + [dev.buf(x), y], grid)
    got = dev.get(y, (T, N))
    want = oracle.matmul(fmt, raw, N, K, x, T, y=y0, acc=True, mode=1)
    for t in range(T):
        assert np.all(np.abs(got[t] - want[t]) <= dot_bound(W, x[t]) + 2e-7 * np.abs(y0[t])), t


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,N,K,acc", [(200, 300, 2048, 1), (128, 256, 1024, 0), (64, 77, 512, 0),
                                        (300, 500, 256, 1), (128, 1024, 5632, 1), (512, 4096, 1024, 0),
                                        (1000, 700, 4864, 1), (256, 130, 2048, 0)])
def test_matmul_prefill_mfma(quipu, dev, oracle, fmt, T, N, K, acc):
    """The matrix-core prefill path (T >= 64): bf16 hi/lo products stay within the float32 dot bound, with
    partial token and row tiles, and tile counts that are not a multiple of the 8 XCDs (3 x 4 = 12 tiles).  For
    K-quants the input is split into bf16 planes once and small tile grids split K (K = 5632: 15 splits, the last
    one partial), partials summed in order; from T = 256 on they take the 256-token tiles."""
    if fmt in PLANAR and K % 64:
        K += 32
    raw = raw_matrix(fmt, N, K, 61)
    W = (oracle.dequant(fmt, raw, N * K) if fmt != capi.F32 else raw.view(np.float32)).reshape(N, K)
    x = (np.random.default_rng(12).standard_normal((T, K)) * 3).astype(np.float32)
    y0 = np.random.default_rng(13).standard_normal((T, N)).astype(np.float32)
    y = dev.buf(y0)
    wb = [dev.matrix(fmt, raw, N, K)]
    if fmt in PLANAR:
        wb.append(capi.scale_plane(fmt, wb[0], N, K))
    quipu.dispatch("matmul_%s_t" % capi.FMT_NAME[fmt], [("u", N), ("u", K), ("u", acc), ("u", 0)],
                   [dev.paso(T, 0)] + wb + [dev.buf(x), y], ((N + 63) // 64, 1, (T + 31) // 32))
    got = dev.get(y, (T, N))
    want = (W.astype(np.float64) @ x.astype(np.float64).T).T + (y0 if acc else 0)
    bound = (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)).T).T * 2e-5 + 2e-7 * np.abs(y0) + 1e-30
    assert np.all(np.abs(got - want) <= bound)


KQ_FMTS = [capi.Q2_K, capi.Q3_K, capi.Q4_K, capi.Q5_K, capi.Q6_K]


@pytest.mark.parametrize("fmt", KQ_FMTS)
@pytest.mark.parametrize("tiles", ["wide", "narrow"])
@pytest.mark.parametrize("T,N,K,acc", [(256, 300, 2048, 1), (512, 520, 1024, 0), (300, 700, 4864, 1),
                                        (768, 256, 512, 0)])
def test_matmul_prefill_tile_kinds(quipu, dev, oracle, monkeypatch, fmt, tiles, T, N, K, acc):
    """Both K-quant tile kinds from 256 tokens on, forced (QP_GEMM_TILES): 256 x 256 tiles (8 wavefronts of 128
    tokens x 64 rows, each thread staging two weight rows) and 256 x 128 tiles, at partial token and row tiles,
    small grids split along K (the last split partial at K = 4864, 19 blocks)."""
    monkeypatch.setenv("QP_GEMM_TILES", tiles)
    raw = raw_matrix(fmt, N, K, 67)
    W = oracle.dequant(fmt, raw, N * K).reshape(N, K)
    x = (np.random.default_rng(14).standard_normal((T, K)) * 3).astype(np.float32)
    y0 = np.random.default_rng(15).standard_normal((T, N)).astype(np.float32)
    y = dev.buf(y0)
    quipu.dispatch("matmul_%s_t" % capi.FMT_NAME[fmt], [("u", N), ("u", K), ("u", acc), ("u", 0)],
                   [dev.paso(T, 0), dev.matrix(fmt, raw, N, K), dev.buf(x), y], ((N + 63) // 64, 1, (T + 31) // 32))
    got = dev.get(y, (T, N))
    want = (W.astype(np.float64) @ x.astype(np.float64).T).T + (y0 if acc else 0)
    bound = (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)).T).T * 2e-5 + 2e-7 * np.abs(y0) + 1e-30
    assert np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("fmt", KQ_FMTS)
@pytest.mark.parametrize("T,N,K", [(256, 300, 2048), (300, 520, 1024), (513, 130, 4864)])
def test_matmul_swiglu_fused(quipu, dev, oracle, fmt, T, N, K):
    """matmul_<fmt>_t_swiglu: silu(x . gate) * (x . up) in one launch (tiles of 128 gate and 128 up rows), against
    float64: the gate and up sums within the float32 dot bound, propagated through silu and the product."""
    rg, ru = raw_matrix(fmt, N, K, 71), raw_matrix(fmt, N, K, 72)
    Wg = oracle.dequant(fmt, rg, N * K).reshape(N, K).astype(np.float64)
    Wu = oracle.dequant(fmt, ru, N * K).reshape(N, K).astype(np.float64)
    x = (np.random.default_rng(16).standard_normal((T, K)) * 0.5).astype(np.float32)
    y = dev.buf(np.full((T, N), np.nan, np.float32))
    quipu.dispatch("matmul_%s_t_swiglu" % capi.FMT_NAME[fmt], [("u", N), ("u", K)],
                   [dev.paso(T, 0), dev.matrix(fmt, rg, N, K), dev.matrix(fmt, ru, N, K), dev.buf(x), y],
                   ((N + 63) // 64, 1, (T + 31) // 32))
    got = dev.get(y, (T, N)).astype(np.float64)
    x64 = x.astype(np.float64)
    g, u = x64 @ Wg.T, x64 @ Wu.T
    dg, du = 2e-5 * (np.abs(x64) @ np.abs(Wg).T), 2e-5 * (np.abs(x64) @ np.abs(Wu).T)
    sg = g / (1.0 + np.exp(np.minimum(-g, 700.0)))
    want = sg * u
    bound = 1.1 * dg * (np.abs(u) + du) + np.abs(sg) * du + 1e-6 * np.abs(want) + 1e-30
    assert np.all(np.isfinite(got)) and np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("fmt", [capi.Q4_K, capi.Q6_K])
def test_matmul_swiglu_fused_equals_the_three_ops(quipu, dev, monkeypatch, fmt):
    """At 2048 tokens x 4352 rows (136 tiles of 256 x 256: no K split) the fused op gives exactly what
    matmul_<fmt>_t on gate and on up followed by swiglu give: the same sums in the same order."""
    monkeypatch.setenv("QP_GEMM_TILES", "wide")
    monkeypatch.setenv("QP_GLU_SPLIT", "0")  # 272 tiles: on 256 CUs the last 16 would run as K halves
    T, N, K = 2048, 4352, 1024
    rg, ru = raw_matrix(fmt, N, K, 73), raw_matrix(fmt, N, K, 74)
    wg, wu = dev.matrix(fmt, rg, N, K), dev.matrix(fmt, ru, N, K)
    x = dev.buf((np.random.default_rng(17).standard_normal((T, K))).astype(np.float32))
    paso = dev.paso(T, 0)
    grid = ((N + 63) // 64, 1, (T + 31) // 32)
    y = dev.buf(np.zeros((T, N), np.float32))
    quipu.dispatch("matmul_%s_t_swiglu" % capi.FMT_NAME[fmt], [("u", N), ("u", K)], [paso, wg, wu, x, y], grid)
    g, u = dev.buf(np.zeros((T, N), np.float32)), dev.buf(np.zeros((T, N), np.float32))
    name = "matmul_%s_t" % capi.FMT_NAME[fmt]
    quipu.dispatch(name, [("u", N), ("u", K), ("u", 0), ("u", 0)], [paso, wg, x, g], grid)
    quipu.dispatch(name, [("u", N), ("u", K), ("u", 0), ("u", 0)], [paso, wu, x, u], grid)
    quipu.dispatch("swiglu", [("u", N)], [paso, g, u], (-(-T * N // 256), 1, 1))
    assert np.array_equal(dev.get(y, (T, N)), dev.get(g, (T, N)))


def test_matmul_swiglu_split_tail(quipu, dev, oracle, monkeypatch):
    """matmul_q4k_t_swiglu at 256 tokens x 33792 rows (264 tiles): on 256 CUs the last 8 tiles run as K halves,
    the second half to finish adding the first's sums.  Within the float64 bound; the same bits on a second call
    (the arrival words are back at zero, and the sum of the two halves does not depend on their order); close to
    the unsplit launch (QP_GLU_SPLIT=0), whose sums are accumulated in another order."""
    fmt, T, N, K = capi.Q4_K, 256, 33792, 256
    rg, ru = raw_matrix(fmt, N, K, 75), raw_matrix(fmt, N, K, 76)
    Wg = oracle.dequant(fmt, rg, N * K).reshape(N, K).astype(np.float64)
    Wu = oracle.dequant(fmt, ru, N * K).reshape(N, K).astype(np.float64)
    x = (np.random.default_rng(18).standard_normal((T, K)) * 0.5).astype(np.float32)
    wg, wu, xb, paso = dev.matrix(fmt, rg, N, K), dev.matrix(fmt, ru, N, K), dev.buf(x), dev.paso(T, 0)

    def run():
        y = dev.buf(np.full((T, N), np.nan, np.float32))
        quipu.dispatch("matmul_q4k_t_swiglu", [("u", N), ("u", K)], [paso, wg, wu, xb, y],
                       ((N + 63) // 64, 1, (T + 31) // 32))
        return dev.get(y, (T, N))

    a, b = run(), run()
    assert np.array_equal(a, b)
    monkeypatch.setenv("QP_GLU_SPLIT", "0")
    c = run()
    x64 = x.astype(np.float64)
    g, u = x64 @ Wg.T, x64 @ Wu.T
    dg, du = 2e-5 * (np.abs(x64) @ np.abs(Wg).T), 2e-5 * (np.abs(x64) @ np.abs(Wu).T)
    sg = g / (1.0 + np.exp(np.minimum(-g, 700.0)))
    want = sg * u
    bound = 1.1 * dg * (np.abs(u) + du) + np.abs(sg) * du + 1e-6 * np.abs(want) + 1e-30
    for got in (a, c):
        got = got.astype(np.float64)
        assert np.all(np.isfinite(got)) and np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("fg,fd,T,F,D", [(capi.Q4_K, capi.Q6_K, 300, 512, 256), (capi.Q5_K, capi.Q4_K, 2048, 1536, 512),
                                          (capi.Q4_K, capi.Q6_K, 2304, 15360, 256)])
@pytest.mark.parametrize("acc", [0, 1])
def test_matmul_swiglu_planes_feed_down(quipu, dev, fg, fd, T, F, D, acc):
    """matmul_<fmt>_t_swiglu with P[2] = 1 writes the down matmul's input planes itself, and matmul_<fmt>_t with
    P[4] = 2 reads them: the down matmul's output equals, bit for bit, the f32 path (the fused op's f32 outputs
    split by the down matmul).  T = 300: token rows 300 .. 511 of the planes are not written; 2304 tokens x 15360
    rows (1080 tiles): on 256 CUs the fused op's last 56 tiles run as K halves."""
    rg, ru, rd = raw_matrix(fg, F, D, 91), raw_matrix(fg, F, D, 92), raw_matrix(fd, D, F, 93)
    wg, wu, wd = dev.matrix(fg, rg, F, D), dev.matrix(fg, ru, F, D), dev.matrix(fd, rd, D, F)
    x = dev.buf((np.random.default_rng(19).standard_normal((T, D)) * 0.5).astype(np.float32))
    y0 = (np.random.default_rng(20).standard_normal((T, D))).astype(np.float32)
    paso = dev.paso(T, 0)
    rows = -(-T // 256) * 256
    glu = "matmul_%s_t_swiglu" % capi.FMT_NAME[fg]
    down = "matmul_%s_t" % capi.FMT_NAME[fd]
    gz = (T + 31) // 32
    h = dev.buf(np.full((T, F), np.nan, np.float32))
    quipu.dispatch(glu, [("u", F), ("u", D)], [paso, wg, wu, x, h], ((F + 63) // 64, 1, gz))
    ya = dev.buf(y0)
    quipu.dispatch(down, [("u", D), ("u", F), ("u", acc), ("u", 0)], [paso, wd, h, ya], ((D + 63) // 64, 1, gz))
    pl = dev.zeros(4 * rows * F)
    quipu.dispatch(glu, [("u", F), ("u", D), ("u", 1)], [paso, wg, wu, x, pl], ((F + 63) // 64, 1, gz))
    yb = dev.buf(y0)
    quipu.dispatch(down, [("u", D), ("u", F), ("u", acc), ("u", 0), ("u", 2)], [paso, wd, pl, yb],
                   ((D + 63) // 64, 1, gz))
    a, b = dev.get(ya, (T, D)), dev.get(yb, (T, D))
    assert np.all(np.isfinite(a)) and a.view(np.uint32).tolist() == b.view(np.uint32).tolist()


@pytest.mark.parametrize("T,D,N", [(300, 1024, 512), (2048, 4096, 1024), (256, 2048, 768), (300, 5120, 256),
                                   (260, 9216, 256)])
def test_rmsnorm_planes_feed_the_matmuls(quipu, dev, T, D, N):
    """rmsnorm_planes writes the rmsnorm of each row as the matmuls' bf16 input planes: matmul_q4k_t with P[4] = 2
    and matmul_q4k_t_swiglu with P[3] = 1 reading them give, bit for bit, what they give from rmsnorm's f32 rows
    (which they split themselves).  D = 5120 and 9216: 4 and 2 rows per workgroup."""
    x = dev.buf((np.random.default_rng(23).standard_normal((T, D)) * 3.0).astype(np.float32))
    wn = dev.buf((1.0 + 0.1 * np.random.default_rng(24).standard_normal(D)).astype(np.float32))
    paso = dev.paso(T, 0)
    eps = 1e-5
    xn = dev.buf(np.zeros((T, D), np.float32))
    quipu.dispatch("rmsnorm", [("u", D), ("u", 0), ("f", eps), ("u", 0)], [paso, x, wn, xn], (T, 1, 1))
    rows = -(-T // 256) * 256
    xs = dev.zeros(4 * rows * D)
    quipu.dispatch("rmsnorm_planes", [("u", D), ("f", eps)], [paso, x, wn, xs], (-(-T // 8), 1, 1))
    raw = raw_matrix(capi.Q4_K, N, D, 96)
    w = dev.matrix(capi.Q4_K, raw, N, D)
    grid = ((N + 63) // 64, 1, (T + 31) // 32)
    ya, yb = dev.buf(np.zeros((T, N), np.float32)), dev.buf(np.zeros((T, N), np.float32))
    quipu.dispatch("matmul_q4k_t", [("u", N), ("u", D), ("u", 0), ("u", 0)], [paso, w, xn, ya], grid)
    quipu.dispatch("matmul_q4k_t", [("u", N), ("u", D), ("u", 0), ("u", 0), ("u", 2)], [paso, w, xs, yb], grid)
    a, b = dev.get(ya, (T, N)), dev.get(yb, (T, N))
    assert np.all(np.isfinite(a)) and a.view(np.uint32).tolist() == b.view(np.uint32).tolist()
    w2 = dev.matrix(capi.Q4_K, raw_matrix(capi.Q4_K, N, D, 97), N, D)
    ga, gb = dev.buf(np.zeros((T, N), np.float32)), dev.buf(np.zeros((T, N), np.float32))
    quipu.dispatch("matmul_q4k_t_swiglu", [("u", N), ("u", D)], [paso, w, w2, xn, ga], grid)
    quipu.dispatch("matmul_q4k_t_swiglu", [("u", N), ("u", D), ("u", 0), ("u", 1)], [paso, w, w2, xs, gb], grid)
    a, b = dev.get(ga, (T, N)), dev.get(gb, (T, N))
    assert np.all(np.isfinite(a)) and a.view(np.uint32).tolist() == b.view(np.uint32).tolist()


@pytest.mark.parametrize("hd,nh,nkv,T,pos0", [(128, 32, 8, 300, 0), (128, 32, 4, 256, 100), (64, 16, 2, 520, 7)])
def test_atencion_output_planes_feed_wo(quipu, dev, hd, nh, nkv, T, pos0):
    """atencion with P[10] = 1 writes its output as wo's bf16 input planes: matmul_q4k_t with P[4] = 2 reading them
    gives, bit for bit, what it gives from the f32 output rows (which it splits itself)."""
    rows = pos0 + T + 40
    kvd, qd = nkv * hd, nh * hd
    rng = np.random.default_rng(27)
    q = rng.standard_normal((T, qd)).astype(np.float32)
    kc = f16r(rng.standard_normal((rows, kvd)))
    vc = f16r(rng.standard_normal((rows, kvd)))
    paso = dev.paso(T, pos0)
    kb, vb, qb = dev.buf(kc.astype(np.float16)), dev.buf(refs.v_tiled(vc.astype(np.float16), kvd)), dev.buf(q)
    scale = float(np.float32(1 / np.sqrt(hd)))
    P = [("u", hd), ("u", nh), ("u", nkv), ("u", 0), ("f", scale), ("u", 0), ("u", 0), ("u", 0), ("u", 1), ("u", rows)]
    o = dev.zeros(T * qd * 4)
    quipu.dispatch("atencion", P, [paso, qb, kb, vb, o], (nh, T))
    orows = -(-T // 256) * 256
    ob = dev.zeros(4 * orows * qd)
    quipu.dispatch("atencion", P + [("u", 1)], [paso, qb, kb, vb, ob], (nh, T))
    N = 512
    w = dev.matrix(capi.Q4_K, raw_matrix(capi.Q4_K, N, qd, 98), N, qd)
    grid = ((N + 63) // 64, 1, (T + 31) // 32)
    ya, yb = dev.buf(np.zeros((T, N), np.float32)), dev.buf(np.zeros((T, N), np.float32))
    quipu.dispatch("matmul_q4k_t", [("u", N), ("u", qd), ("u", 0), ("u", 0)], [paso, w, o, ya], grid)
    quipu.dispatch("matmul_q4k_t", [("u", N), ("u", qd), ("u", 0), ("u", 0), ("u", 2)], [paso, w, ob, yb], grid)
    a, b = dev.get(ya, (T, N)), dev.get(yb, (T, N))
    assert np.all(np.isfinite(a)) and a.view(np.uint32).tolist() == b.view(np.uint32).tolist()
    with pytest.raises(capi.QuipuError, match="output planes"):
        quipu.dispatch("atencion", P + [("u", 1)], [paso, qb, kb, vb, dev.zeros(4 * orows * qd - 64)], (nh, T))


def test_matmul_planes_rejections(quipu, dev):
    """P[4] = 2 needs the 256-token tiles (under 256 tokens the matmul refuses it), and the planes' buffers must hold
    4 * rows * K bytes (256-token rows)."""
    T, F, D = 300, 256, 256
    raw = raw_matrix(capi.Q4_K, F, D, 94)
    w = dev.matrix(capi.Q4_K, raw, F, D)
    x = dev.buf(np.zeros((T, D), np.float32))
    with pytest.raises(capi.QuipuError, match="output planes"):
        quipu.dispatch("matmul_q4k_t_swiglu", [("u", F), ("u", D), ("u", 1)],
                       [dev.paso(T, 0), w, w, x, dev.zeros(4 * T * F)], (4, 1, 10))
    with pytest.raises(capi.QuipuError, match="input planes"):
        quipu.dispatch("matmul_q4k_t", [("u", D), ("u", F), ("u", 0), ("u", 0), ("u", 2)],
                       [dev.paso(T, 0), w, dev.zeros(4 * T * F), dev.zeros(4 * T * D)], (4, 1, 10))
    with pytest.raises(capi.QuipuError, match="256 tokens or more"):
        quipu.dispatch("matmul_q4k_t", [("u", D), ("u", F), ("u", 0), ("u", 0), ("u", 2)],
                       [dev.paso(100, 0), w, dev.zeros(4 * 256 * F), dev.zeros(4 * 100 * D)], (4, 1, 4))
    with pytest.raises(capi.QuipuError, match="planes' buffer"):
        quipu.dispatch("rmsnorm_planes", [("u", D), ("f", 1e-5)],
                       [dev.paso(T, 0), x, dev.buf(np.ones(D, np.float32)), dev.zeros(4 * T * D)], (-(-T // 8), 1, 1))
    with pytest.raises(capi.QuipuError, match="input planes' buffer"):
        quipu.dispatch("matmul_q4k_t_swiglu", [("u", F), ("u", D), ("u", 0), ("u", 1)],
                       [dev.paso(T, 0), w, w, dev.zeros(4 * T * D), dev.zeros(4 * T * F)], (4, 1, 10))


def test_matmul_reuses_the_split_input(quipu, dev):
    """P[4] = 1 (Q, then K and V of the same input): the bf16 planes the previous matrix-core matmul split are used
    again; results equal those of a fresh split.  With another input (x2), or after the workspace grew (a larger
    call in between), the flag still splits, so the results stay right."""
    T, K = 300, 1024
    fm = capi.Q4_K
    raws = [raw_matrix(fm, N, K, 80 + N) for N in (512, 256, 768)]
    ws = [dev.matrix(fm, r, r.size * 256 // 144 // K, K) for r in raws]
    x1, x2 = (dev.buf(np.random.default_rng(s).standard_normal((T, K)).astype(np.float32)) for s in (30, 31))
    paso = dev.paso(T, 0)
    grid = lambda N: ((N + 63) // 64, 1, (T + 31) // 32)

    def mm(i, x, reuse):
        N = (512, 256, 768)[i]
        y = dev.zeros(T * N * 4)
        u = [("u", N), ("u", K), ("u", 0), ("u", 0)] + ([("u", 1)] if reuse else [])
        quipu.dispatch("matmul_q4k_t", u, [paso, ws[i], x, y], grid(N))
        return dev.get(y, (T, N))

    fresh = [mm(i, x1, False) for i in range(3)]
    mm(0, x1, False)
    assert np.array_equal(mm(1, x1, True), fresh[1]) and np.array_equal(mm(2, x1, True), fresh[2])
    mm(0, x2, False)
    assert np.array_equal(mm(1, x1, True), fresh[1])  # the planes hold x2: x1 is split again
    big = dev.buf(np.zeros((2048, 4096), np.float32))  # a larger call reallocates the workspace
    quipu.dispatch("matmul_q4k_t", [("u", 256), ("u", 4096), ("u", 0), ("u", 0)],
                   [dev.paso(2048, 0), dev.matrix(fm, raw_matrix(fm, 256, 4096, 90), 256, 4096), big,
                    dev.zeros(2048 * 256 * 4)], (4, 1, 64))
    assert np.array_equal(mm(2, x1, True), fresh[2])


def test_matmul_swiglu_fused_rejections(quipu, dev):
    """Prompt chunks under 256 tokens (grid z < 8) and weight buffers smaller than their tensors are refused with a
    message (the op is registered for K-quants only: see the host test of the op table)."""
    N, K = 256, 256
    raw = raw_matrix(capi.Q4_K, N, K, 75)
    w = dev.matrix(capi.Q4_K, raw, N, K)
    bufs = [dev.paso(100, 0), w, w, dev.buf(np.zeros((100, K), np.float32)), dev.buf(np.zeros((100, N), np.float32))]
    with pytest.raises(capi.QuipuError, match="256 tokens"):
        quipu.dispatch("matmul_q4k_t_swiglu", [("u", N), ("u", K)], bufs, (4, 1, 4))
    bufs[2] = dev.zeros(N * K // 256 * 144 - 16)  # an up tensor one chunk short
    with pytest.raises(capi.QuipuError, match="up tensor"):
        quipu.dispatch("matmul_q4k_t_swiglu", [("u", N), ("u", K)], bufs, (4, 1, 8))


@pytest.mark.parametrize("T,N,K", [(256, 300, 4096), (700, 130, 1024)])
def test_matmul_q4k_prefill_row_magnitudes(quipu, dev, oracle, T, N, K):
    """Q4_K prefill from 256 tokens on (the 256-token tiles, inputs as bf16 high + low planes): token rows of
    magnitude 1e-20 .. 1e20, an all-zero row and rows with one outlier 1e6 times the rest stay within the float32
    dot bound; the all-zero row gives exact zeros."""
    raw = raw_matrix(capi.Q4_K, N, K, 62)
    W = oracle.dequant(capi.Q4_K, raw, N * K).reshape(N, K)
    rng = np.random.default_rng(14)
    x = rng.standard_normal((T, K)).astype(np.float32)
    mags = 10.0 ** rng.integers(-20, 21, size=T)
    x *= mags[:, None].astype(np.float32)
    x[3] = 0.0
    x[5, 7] *= 1e6
    x[6, K - 1] = 1e4
    x = x.astype(np.float32)
    y = dev.zeros(4 * T * N)
    quipu.dispatch("matmul_q4k_t", [("u", N), ("u", K), ("u", 0), ("u", 0)],
                   [dev.paso(T, 0), dev.matrix(capi.Q4_K, raw, N, K), dev.buf(x), y],
                   ((N + 63) // 64, 1, (T + 31) // 32))
    got = dev.get(y, (T, N))
    want = (W.astype(np.float64) @ x.astype(np.float64).T).T
    bound = (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)).T).T * 2e-5 + 1e-30
    assert np.all(np.isfinite(got))
    assert np.all(got[3] == 0.0)
    assert np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("fmt,K", [(capi.Q8_0, 288), (capi.Q8_0, 544), (capi.IQ4_NL, 288), (capi.F32, 80),
                                   (capi.F32, 272),
                                   (capi.F32, 528)])
@pytest.mark.parametrize("T,N", [(64, 77), (130, 300)])
def test_matmul_prefill_mfma_ragged_k(quipu, dev, oracle, fmt, T, N, K):
    """Q8_0 (K % 32) and f32 (K % 16) prefill matmuls whose K is not a multiple of the 64-input step, through the
    pre-split bf16 planes, without and with split-K (K = 544, 528: three K chunks, the last one partial).  The
    workspace is first filled by a call whose input is all NaN at more tokens, so a read past the end of a row's
    planes would bring NaN into the result."""
    raw = raw_matrix(fmt, N, K, 77)
    W = (oracle.dequant(fmt, raw, N * K) if fmt != capi.F32 else raw.view(np.float32)).reshape(N, K)
    wb = [dev.matrix(fmt, raw, N, K)]
    if fmt in PLANAR:
        wb.append(capi.scale_plane(fmt, wb[0], N, K))
    name = "matmul_%s_t" % capi.FMT_NAME[fmt]
    uni = [("u", N), ("u", K), ("u", 0), ("u", 0)]
    Tp = T + 200
    nan_x = np.full((Tp, K), np.nan, np.float32)
    quipu.dispatch(name, uni, [dev.paso(Tp, 0)] + wb + [dev.buf(nan_x), dev.zeros(4 * Tp * N)],
                   ((N + 63) // 64, 1, (Tp + 31) // 32))
    x = np.random.default_rng(5).standard_normal((T, K)).astype(np.float32)
    y = dev.zeros(4 * T * N)
    quipu.dispatch(name, uni, [dev.paso(T, 0)] + wb + [dev.buf(x), y], ((N + 63) // 64, 1, (T + 31) // 32))
    got = dev.get(y, (T, N))
    want = (W.astype(np.float64) @ x.astype(np.float64).T).T
    bound = (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)).T).T * 2e-5 + 1e-30
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - want) <= bound)


def group_jobs(sel, E):
    """moe_group's result from its definition: per expert, the job indices holding it, in increasing order."""
    lst = [i for e in range(E) for i in range(len(sel)) if sel[i] == e]
    cnt = np.bincount(np.asarray(sel, np.int64)[np.asarray(sel) < E], minlength=E)
    return np.array(lst, np.uint32), np.concatenate([[0], np.cumsum(cnt)]).astype(np.uint32)


@pytest.mark.parametrize("E,k,T", [(16, 4, 70), (128, 8, 300), (7, 1, 1), (128, 8, 2048), (256, 8, 4000), (5, 3, 21800)])
def test_moe_group(quipu, dev, E, k, T):
    """moe_group (kds.js:491-516): jobs listed per expert in increasing order, off the running counts; one expert
    takes more than half of the tokens, several none; an id >= E (not a valid expert) is not listed."""
    rng = np.random.default_rng(E + T)
    sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32).ravel()
    if T > 2:
        sel[0:T * k // 2:k] = 3 % E  # a popular expert (first slot of half the tokens)
        sel[k * (T - 1)] = E + 5      # not an expert
    lst_want, off_want = group_jobs(sel, E)
    sb, lb, ob = dev.buf(sel), dev.zeros(4 * T * k), dev.zeros(4 * (E + 1))
    quipu.dispatch("moe_group", [("u", E), ("u", k)], [dev.paso(T, 0), sb, lb, ob])
    off = dev.get(ob, (E + 1,), np.uint32)
    assert off.tolist() == off_want.tolist()
    assert dev.get(lb, (T * k,), np.uint32)[:int(off[E])].tolist() == lst_want.tolist()


@pytest.mark.parametrize("fmt", [capi.Q4_K, capi.Q6_K, capi.Q5_K, capi.Q3_K, capi.Q2_K, capi.Q8_0, capi.F32,
                                 capi.IQ4_NL])
@pytest.mark.parametrize("tfijo,acc", [(4, 0), (1, 1)])
def test_matmul_grouped_by_expert(quipu, dev, oracle, fmt, tfijo, acc):
    """matmul_<fmt>_eg (kquants.js:386-460): the expert matmul over the job lists of moe_group, on the matrix cores.
    Expert 2 has 150 jobs (two job tiles), several experts none; rows N = 200 (a partial row tile).  tfijo = 4:
    job j reads input row j / 4 (gate/up); tfijo = 1 with acc: row j, added to y (down).  The same bits with the
    input split into planes first (P[4]), and with that split reused (P[5])."""
    E, N, K, k = 8, 200, 512, 4
    T = 160 if tfijo > 1 else 40
    rng = np.random.default_rng(9)
    njob = T * k
    sel = np.stack([rng.choice([0, 2, 3, 5], k, replace=False) for _ in range(T)]).astype(np.uint32).ravel()
    sel[2::k] = 2                          # expert 2 in every token (150+ jobs)
    sel[1::k] = np.where(sel[1::k] == 2, 7, sel[1::k])
    raw = raw_matrix(fmt, E * N, K, 31)
    W = (oracle.dequant(fmt, raw, E * N * K) if fmt != capi.F32 else raw.view(np.float32)).reshape(E, N, K)
    xr = njob // tfijo
    x = rng.standard_normal((xr, K)).astype(np.float32)
    y0 = rng.standard_normal((njob, N)).astype(np.float32)
    sb, lb, ob = dev.buf(sel), dev.zeros(4 * njob), dev.zeros(4 * (E + 1))
    quipu.dispatch("moe_group", [("u", E), ("u", k)], [dev.paso(T, 0), sb, lb, ob])
    hw = dev.matrix(fmt, raw, E * N, K)
    wb = [hw, capi.scale_plane(fmt, hw, E * N, K)] if fmt in PLANAR else [hw]
    yb, xb, pb = dev.buf(y0), dev.buf(x), dev.paso(T, 0)
    u = [("u", N), ("u", K), ("u", acc), ("u", tfijo)]
    name, grid = "matmul_%s_eg" % capi.FMT_NAME[fmt], ((N + 63) // 64, E, (T + 31) // 32)
    quipu.dispatch(name, u, [pb] + wb + [xb, yb, lb, ob], grid)
    got = dev.get(yb, (njob, N))
    # x split into bf16 planes once (P[4] = its rows per token: 1 for token rows, k for job rows) gives the same
    # bits; then P[5] = 1 reuses that split
    for reuse in (0, 1):
        y2 = dev.buf(y0)
        quipu.dispatch(name, u + [("u", 1 if tfijo > 1 else k), ("u", reuse)], [pb] + wb + [xb, y2, lb, ob], grid)
        assert np.array_equal(dev.get(y2, (njob, N)), got), reuse
    for j in range(njob):
        e = int(sel[j])
        if e >= E:
            continue
        xv = x[j // tfijo].astype(np.float64)
        want = W[e].astype(np.float64) @ xv + (y0[j] if acc else 0)
        bound = 2e-5 * (np.abs(W[e].astype(np.float64)) @ np.abs(xv)) + 2e-7 * np.abs(y0[j]) + 1e-30
        assert np.all(np.abs(got[j] - want) <= bound), (j, e, np.abs(got[j] - want).max())


@pytest.mark.parametrize("fmt", FMTS)
def test_matmul_expert_jobs(quipu, dev, oracle, fmt):
    """matmul_<fmt>_e (one job per selected expert) and the fused gate/up _e_swiglu; tfijo = k routes job z to
    input row z / k."""
    E, N, K, k, T = 6, 96, 512, 2, 2
    rg, ru = raw_matrix(fmt, E * N, K, 70), raw_matrix(fmt, E * N, K, 71)
    Wg = (oracle.dequant(fmt, rg, E * N * K) if fmt != capi.F32 else rg.view(np.float32)).reshape(E, N, K)
    x = np.random.default_rng(11).standard_normal((T, K)).astype(np.float32)
    sel = np.array([4, 1, 0, 5], np.uint32)
    hg, hu = dev.matrix(fmt, rg, E * N, K), dev.matrix(fmt, ru, E * N, K)
    y = dev.zeros(T * k * N * 4)
    u = [("u", N), ("u", K), ("u", 0), ("u", k), ("u", E)]
    wb = [hg, capi.scale_plane(fmt, hg, E * N, K)] if fmt in PLANAR else [hg]
    xb, sb, pb = dev.buf(x), dev.buf(sel), dev.paso(T, 0)
    quipu.dispatch("matmul_%s_e" % capi.FMT_NAME[fmt], u, [pb] + wb + [xb, y, sb], (1, 1, T * k))
    got = dev.get(y, (T * k, N))
    want = oracle.matmul_e(fmt, rg, N, K, x, sel, k)
    for z in range(T * k):
        assert np.all(np.abs(got[z] - want[z]) <= dot_bound(Wg[sel[z]], x[z // k])), z
    y2 = dev.zeros(T * k * N * 4)
    quipu.dispatch("matmul_%s_e_swiglu" % capi.FMT_NAME[fmt], u, [pb] + wb + [hu, xb, y2, sb], (1, 1, T * k))
    got2 = dev.get(y2, (T * k, N))
    want2 = oracle.swiglu(want, oracle.matmul_e(fmt, ru, N, K, x, sel, k))
    np.testing.assert_allclose(got2, want2, rtol=1e-4, atol=1e-4 * np.abs(want2).max())


def expert_rows(oracle, fmt, raw, e, N, K):
    """Dequantized rows of expert e of a stacked [E*N][K] K-quant tensor (GGUF block bytes)."""
    bb = {capi.Q4_K: 144, capi.Q6_K: 210}[fmt] * (K // 256)
    return oracle.dequant(fmt, raw[e * N * bb:(e + 1) * N * bb], N * K).reshape(N, K).astype(np.float64)


@pytest.mark.parametrize("fmt", [capi.Q4_K, capi.Q6_K])
@pytest.mark.parametrize("E,k,D,Fe,norm", [(128, 8, 2048, 768, 1), (16, 4, 512, 256, 0), (20, 6, 8448, 1536, 1)])
def test_moe_fused_decode(quipu, dev, oracle, fmt, E, k, D, Fe, norm):
    """moe_gate_up_<fmt> then moe_down_<fmt> (one token) against the reference sequence in float64: rmsnorm, routing
    (oracle moe_topk, ties to the lower expert), gate/up GEMVs of the chosen experts, SwiGLU, down GEMVs and the
    weighted combine into the residual.  The last shape stages more than 8192 inputs (the two-pass variants)."""
    rng = np.random.default_rng([E, k, D, fmt])
    rg, ru, rd = raw_matrix(fmt, E * Fe, D, 81), raw_matrix(fmt, E * Fe, D, 82), raw_matrix(fmt, E * D, Fe, 83)
    hg, hu, hd = dev.matrix(fmt, rg, E * Fe, D), dev.matrix(fmt, ru, E * Fe, D), dev.matrix(fmt, rd, E * D, Fe)
    nw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    eps, scale = 1e-6, 1.0 if norm else 2.5
    name = capi.FMT_NAME[fmt]
    for call in range(2):
        x = rng.standard_normal(D).astype(np.float32)
        lg = rng.standard_normal(E).astype(np.float32)
        if call == 0:
            lg[3] = lg[E - 2] = lg.max() + 1.0  # an exact tie at the top: the lower expert first
        s_want, w_want = oracle.moe_topk(lg[None, :], E, k, norm, scale)
        xb, h, sel, wts = dev.buf(x), dev.zeros(k * Fe * 4), dev.zeros(k * 4), dev.zeros(k * 4)
        ug = [("u", Fe), ("u", D), ("u", E), ("u", k), ("f", eps), ("f", scale), ("u", norm)]
        ud = [("u", D), ("u", Fe), ("u", E), ("u", k), ("f", eps), ("f", scale), ("u", norm)]
        quipu.dispatch("moe_gate_up_" + name, ug, [dev.paso(1, 0), hg, hu, xb, dev.buf(nw), dev.buf(lg), h, sel, wts])
        np.testing.assert_array_equal(dev.get(sel, (k,), np.uint32), s_want)
        np.testing.assert_allclose(dev.get(wts, (k,)), w_want, rtol=2e-6, atol=1e-7)
        if call == 0:
            assert list(s_want[:2]) == [3, E - 2]
        xn = oracle.rmsnorm(x[None, :], nw, eps)[0].astype(np.float64)
        got_h = dev.get(h, (k, Fe))
        for j, e in enumerate(s_want):
            g = expert_rows(oracle, fmt, rg, e, Fe, D) @ xn
            u = expert_rows(oracle, fmt, ru, e, Fe, D) @ xn
            want = g / (1 + np.exp(-g)) * u
            np.testing.assert_allclose(got_h[j], want, rtol=1e-4, atol=1e-4 * np.abs(want).max(), err_msg=str(j))
        # down + combine on the GPU's h: x + sum_j wts_j Wd_j h_j
        quipu.dispatch("moe_down_" + name, ud, [dev.paso(1, 0), hd, h, xb, sel, wts])
        got = dev.get(xb, (D,))
        want = x.astype(np.float64)
        bound = 2e-7 * np.abs(want) + 1e-30
        for j, e in enumerate(s_want):
            Wd = expert_rows(oracle, fmt, rd, e, D, Fe)
            want = want + float(w_want[j]) * (Wd @ got_h[j].astype(np.float64))
            bound = bound + 2e-5 * abs(float(w_want[j])) * (np.abs(Wd) @ np.abs(got_h[j].astype(np.float64)))
        assert np.all(np.abs(got - want) <= bound), np.abs(got - want).max()


@pytest.mark.parametrize("E,k,D,nw,norm", [(128, 8, 2048, 32, 1), (16, 4, 512, 4, 0), (256, 8, 4096, 64, 1),
                                           (60, 4, 6144, 16, 1)])
def test_moe_router(quipu, dev, oracle, E, k, D, nw, norm):
    """moe_router: the f32 router GEMV of the normalized token (column 0's nw workgroups on one XCD) and the routing
    by the last of them to finish.  Logits within 2e-5 sum |w x| of the oracle's rmsnorm + matmul; sel and wts
    the oracle's moe_topk of those logits (sel exact, an exact tie at the top to the lower expert; wts within
    2e-6), over three
    launches in a row (the last arrival resets the counter; the error word stays clear); then moe_gate_up with the
    routing read from sel (P[7] = 1)
    and moe_down give bit-identical results to moe_gate_up routing from the same logits itself."""
    rng = np.random.default_rng([E, k, D])
    W = (0.02 * rng.standard_normal((E, D))).astype(np.float32)
    W[E - 3] = W[5]  # rows 5 and E - 3 equal: an exact tie of their logits
    nw_ = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    eps, scale = 1e-6, 1.0 if norm else 2.5
    hw, hn, lg, sel, wts, cnt = dev.buf(W), dev.buf(nw_), dev.zeros(E * 4), dev.zeros(k * 4), dev.zeros(k * 4), dev.zeros(8)
    u = [("u", E), ("u", D), ("u", k), ("u", nw), ("f", eps), ("f", scale), ("u", norm)]
    for call in range(3):
        x = rng.standard_normal(D).astype(np.float32)
        x *= np.float32(1 + call)
        xb = dev.buf(x)
        if call == 1:
            # make rows 5 / E - 3 the largest logits: x along their row
            x = (W[5] * 50).astype(np.float32)
            quipu.upload(xb, x)
        quipu.dispatch("moe_router", u, [dev.paso(1, 0), hw, xb, hn, lg, sel, wts, cnt], (8, nw, 1))
        got = dev.get(lg, (E,))
        xn = oracle.rmsnorm(x[None, :], nw_, eps)[0]
        want = W.astype(np.float64) @ xn.astype(np.float64)
        assert np.all(np.abs(got - want) <= dot_bound(W, xn)), np.abs(got - want).max()
        s_want, w_want = oracle.moe_topk(got[None, :], E, k, norm, scale)
        np.testing.assert_array_equal(dev.get(sel, (k,), np.uint32), s_want)
        np.testing.assert_allclose(dev.get(wts, (k,)), w_want, rtol=2e-6, atol=1e-7)
        if call == 1:
            assert list(s_want[:2]) == [5, E - 3]
    assert list(dev.get(cnt, (2,), np.uint32)) == [0, 0]
    if D % 256 or E * 64 * D * 0.5625 > 2 ** 30:
        return
    # the expert FFN from the router's routing: presel against routing in moe_gate_up, bit for bit
    Fe = 256
    rg, ru, rd = raw_matrix(capi.Q4_K, E * Fe, D, 84), raw_matrix(capi.Q4_K, E * Fe, D, 85), raw_matrix(capi.Q4_K, E * D, Fe, 86)
    hg, hu, hd = (dev.matrix(capi.Q4_K, rg, E * Fe, D), dev.matrix(capi.Q4_K, ru, E * Fe, D),
                  dev.matrix(capi.Q4_K, rd, E * D, Fe))
    outs = []
    for presel in (1, 0):
        xb, h, s2, w2 = dev.buf(x), dev.zeros(k * Fe * 4), dev.zeros(k * 4), dev.zeros(k * 4)
        if presel:
            quipu.upload(s2, dev.get(sel, (k,), np.uint32))
            quipu.upload(w2, dev.get(wts, (k,)))
        ug = [("u", Fe), ("u", D), ("u", E), ("u", k), ("f", eps), ("f", scale), ("u", norm), ("u", presel)]
        ud = [("u", D), ("u", Fe), ("u", E), ("u", k), ("f", eps), ("f", scale), ("u", norm)]
        quipu.dispatch("moe_gate_up_q4k", ug, [dev.paso(1, 0), hg, hu, xb, hn, lg, h, s2, w2])
        quipu.dispatch("moe_down_q4k", ud, [dev.paso(1, 0), hd, h, xb, s2, w2])
        outs.append((dev.get(h, (k, Fe)), dev.get(xb, (D,)), dev.get(s2, (k,), np.uint32)))
    for a_, b_ in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(a_, b_)


def test_moe_router_rejections(quipu, dev):
    """Shapes and bindings the kernel cannot take are refused on the host."""
    b = [dev.zeros(16 * 512 * 4), dev.zeros(2048), dev.zeros(2048), dev.zeros(64), dev.zeros(64), dev.zeros(64), dev.zeros(8)]
    for u3, msg in [((16, 512, 4, 3), "nw=3"), ((300, 512, 4, 4), "300 experts"), ((16, 512, 20, 4), "20 experts used"),
                    ((16, 510, 4, 4), "k=510"), ((16, 512, 4, 256), "nw=256")]:
        u = [("u", v) for v in u3] + [("f", 1e-6), ("f", 1.0), ("u", 1)]
        with pytest.raises(capi.QuipuError, match=msg):
            quipu.dispatch("moe_router", u, [0] + b, (8, 4, 1))


# ------------------------------------------------------------------------------------------------ elementwise
def test_rmsnorm(quipu, dev, oracle):
    T, D = 5, 4096
    x = (np.random.default_rng(12).standard_normal((T, D)) * 3).astype(np.float32)
    w = np.random.default_rng(13).standard_normal(D).astype(np.float32)
    for ultima in (0, 1):
        y = dev.zeros(T * D * 4)
        quipu.dispatch("rmsnorm", [("u", D), ("u", ultima), ("f", 1e-5), ("u", 0)],
                       [dev.paso(T, 0), dev.buf(x), dev.buf(w), y], (T,))
        got = dev.get(y, (1 if ultima else T, D))
        np.testing.assert_allclose(got, oracle.rmsnorm(x, w, 1e-5, ultima=bool(ultima)), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("hd,neox,use_norm", [(128, 0, 0), (128, 1, 1), (64, 1, 0), (64, 0, 1)])
def test_norm_rope(quipu, dev, oracle, hd, neox, use_norm):
    nh, T, pos0 = 8, 3, 1000
    v = np.random.default_rng(14).standard_normal((T, nh, hd)).astype(np.float32)
    w = (1 + 0.1 * np.random.default_rng(15).standard_normal(hd)).astype(np.float32)
    vb = dev.buf(v)
    quipu.dispatch("norm_rope", [("u", hd), ("u", nh), ("u", use_norm), ("u", neox), ("f", 1e-6), ("f", 5e5),
                                 ("u", hd), ("u", 0)], [dev.paso(T, pos0), vb, dev.buf(w)], (nh, T))
    got = dev.get(vb, (T * nh * hd,))
    want = oracle.norm_rope(v, w, nh, hd, use_norm, neox, 1e-6, 5e5, hd, pos0).reshape(-1)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    # with the host's frequency table as a fourth binding: the same bits
    vb2 = dev.buf(v)
    quipu.dispatch("norm_rope", [("u", hd), ("u", nh), ("u", use_norm), ("u", neox), ("f", 1e-6), ("f", 5e5),
                                 ("u", hd), ("u", 0)], [dev.paso(T, pos0), vb2, dev.buf(w), dev.buf(rope_table(5e5, hd))],
                   (nh, T))
    assert np.array_equal(dev.get(vb2, (T * nh * hd,)), got)


@pytest.mark.parametrize("f16", [0, 1])
@pytest.mark.parametrize("kvd,rows,T,pos0", [(256, 20, 4, 15), (1024, 200, 100, 37), (132, 300, 130, 101)])
def test_kv_write(quipu, dev, oracle, f16, kvd, rows, T, pos0):
    """kv_write at positions pos0..pos0+T-1; from 64 tokens on the f16 cache takes the 64 x 64 tiles (K four
    channels per thread, V through LDS), here with partial token and channel tiles and slots past a 32-slot tile."""
    k = np.random.default_rng(16).standard_normal((T, kvd)).astype(np.float32)
    v = np.random.default_rng(17).standard_normal((T, kvd)).astype(np.float32)
    es = 2 if f16 else 4
    vrows = (rows + 31) // 32 * 32 if f16 else rows  # the f16 value cache is stored in whole tiles of 32 slots
    kc, vc = dev.zeros(rows * kvd * es), dev.zeros(vrows * kvd * es)
    quipu.dispatch("kv_write", [("u", kvd), ("u", 0), ("u", f16), ("u", rows)],
                   [dev.paso(T, pos0), dev.buf(k), dev.buf(v), kc, vc], ((T * kvd + 255) // 256,))
    dt = np.float16 if f16 else np.float32
    gk, gv = dev.get(kc, (rows, kvd), dt), dev.get(vc, (vrows, kvd), dt)
    if f16:
        gv = refs.v_rows(gv, rows, kvd)
    # rows pos0..pos0+T-1 written (f16: round to nearest even), everything else untouched
    np.testing.assert_array_equal(gk[pos0:pos0 + T], k.astype(dt))
    np.testing.assert_array_equal(gv[pos0:pos0 + T], v.astype(dt))
    assert not gk[:pos0].any() and not gk[pos0 + T:].any()
    assert not gv[:pos0].any() and not gv[pos0 + T:].any()


@pytest.mark.parametrize("f16", [0, 1])
@pytest.mark.parametrize("big", [False, True])
def test_kv_write_ring(quipu, dev, f16, big):
    """kv_write into a ring of cap slots (the reference's sliding-window cache, transformer.js:106-111 and
    gpu.js:461-462): position p goes to slot p % cap; 8 tokens from position 20 of a 24-slot ring wrap to slots
    20..23 and 0..3, and the other slots keep their contents."""
    kvd, cap, T, pos0 = 128, 24, 8, 20
    if big:  # 90 tokens from position 150 of a 96-slot ring: the 64 x 64 tiles of the f16 cache, wrapping once
        cap, T, pos0 = 96, 90, 150
    rng = np.random.default_rng(26)
    k = rng.standard_normal((T, kvd)).astype(np.float32)
    v = rng.standard_normal((T, kvd)).astype(np.float32)
    dt = np.float16 if f16 else np.float32
    old_k = rng.standard_normal((cap, kvd)).astype(dt)
    old_v = rng.standard_normal((cap, kvd)).astype(dt)
    kc = dev.buf(old_k)
    vc = dev.buf(refs.v_tiled(old_v, kvd) if f16 else old_v)
    quipu.dispatch("kv_write", [("u", kvd), ("u", cap), ("u", f16), ("u", cap)],
                   [dev.paso(T, pos0), dev.buf(k), dev.buf(v), kc, vc], ((T * kvd + 255) // 256,))
    gk = dev.get(kc, (cap, kvd), dt)
    gv = dev.get(vc, ((cap + 31) // 32 * 32 if f16 else cap, kvd), dt)
    if f16:
        gv = refs.v_rows(gv, cap, kvd)
    want_k, want_v = old_k.copy(), old_v.copy()
    for t in range(T):
        want_k[(pos0 + t) % cap] = k[t].astype(dt)
        want_v[(pos0 + t) % cap] = v[t].astype(dt)
    np.testing.assert_array_equal(gk, want_k)
    np.testing.assert_array_equal(gv, want_v)


@pytest.mark.parametrize("f16", [0, 1])
@pytest.mark.parametrize("hd,nh,nkv,T,pos0,swa", [(64, 8, 2, 16, 150, 40), (128, 16, 4, 1, 300, 100),
                                                  (64, 4, 4, 32, 10, 40)])
def test_atencion_window_over_a_ring(quipu, dev, oracle, hd, nh, nkv, T, pos0, swa, f16):
    """atencion with a sliding window of swa keys (measured from each query position) over a ring cache of
    cap = swa + 32 slots holding positions p at slot p % cap: the same result as the window over the whole cache
    (the oracle, reference gpu.js:467-539 with swa)."""
    kvd, cap = nkv * hd, swa + 32
    rng = np.random.default_rng(27)
    full = pos0 + T
    kf = rng.standard_normal((full, kvd)).astype(np.float32)
    vf = rng.standard_normal((full, kvd)).astype(np.float32)
    if f16:
        kf, vf = f16r(kf), f16r(vf)
    q = rng.standard_normal((T, nh * hd)).astype(np.float32)
    kr = np.zeros((cap, kvd), np.float32)
    vr = np.zeros((cap, kvd), np.float32)
    for p in range(max(0, full - cap), full):
        kr[p % cap], vr[p % cap] = kf[p], vf[p]
    dt = np.float16 if f16 else np.float32
    o = dev.zeros(T * nh * hd * 4)
    scale = float(np.float32(1 / np.sqrt(hd)))
    quipu.dispatch("atencion", [("u", hd), ("u", nh), ("u", nkv), ("u", swa), ("f", scale), ("u", cap), ("u", 0),
                                ("u", 0), ("u", f16), ("u", cap)],
                   [dev.paso(T, pos0), dev.buf(q), dev.buf(kr.astype(dt)),
                    dev.buf(refs.v_tiled(vr.astype(dt), kvd) if f16 else vr), o], (nh, T))
    got = dev.get(o, (T, nh * hd))
    want = oracle.attention(q, kf, vf, T, pos0, nh, nkv, hd, scale, swa=swa)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


def test_kv_write_past_the_cache_writes_nothing(quipu, dev):
    kvd, rows = 64, 4
    kc, vc = dev.zeros(rows * kvd * 4), dev.zeros(rows * kvd * 4)
    k = np.ones((2, kvd), np.float32)
    quipu.dispatch("kv_write", [("u", kvd), ("u", 0), ("u", 0), ("u", rows)],
                   [dev.paso(2, 3), dev.buf(k), dev.buf(k), kc, vc], (1,))
    gk = dev.get(kc, (rows, kvd))
    assert gk[3].all() and not gk[:3].any()  # slot 4 is past the cache: skipped


def test_geglu_escalar_suma_esc(quipu, dev, oracle):
    """geglu (gpu.js:318-330; tanhf of the device library against the C library's, so within a float32 bound
    scaled like the computation), escalar and suma_esc (gpu.js:635-660; one product and one sum per element:
    bit-exact)."""
    rng = np.random.default_rng(19)
    T, F = 3, 2500
    g = (rng.standard_normal(T * F) * 4).astype(np.float32)
    g[:5] = [-30.0, -9.0, 0.0, 9.0, 30.0]
    uu = rng.standard_normal(T * F).astype(np.float32)
    gb = dev.buf(g)
    quipu.dispatch("geglu", [("u", F)], [dev.paso(T, 0), gb, dev.buf(uu)], ((T * F + 255) // 256,))
    got, want = dev.get(gb, (T * F,)), oracle.geglu(g, uu)
    assert np.all(np.abs(got - want) <= 2e-6 * (np.abs(g) + 1.0) * np.abs(uu) + 1e-30)
    D = 700
    x, t = rng.standard_normal(T * D).astype(np.float32), rng.standard_normal(T * D).astype(np.float32)
    xb = dev.buf(x)
    quipu.dispatch("escalar", [("u", D), ("f", 22.627417)], [dev.paso(T, 0), xb], ((T * D + 255) // 256,))
    x1 = dev.get(xb, (T * D,))
    np.testing.assert_array_equal(x1, oracle.escalar(x, 22.627417))
    quipu.dispatch("suma_esc", [("u", D), ("f", 0.375)], [dev.paso(T, 0), xb, dev.buf(t)], ((T * D + 255) // 256,))
    np.testing.assert_array_equal(dev.get(xb, (T * D,)), oracle.suma_esc(x1, t, 0.375))


def test_swiglu_moe_ops(quipu, dev, oracle):
    rng = np.random.default_rng(18)
    T, F = 2, 3000
    g = (rng.standard_normal(T * F) * 4).astype(np.float32)
    uu = rng.standard_normal(T * F).astype(np.float32)
    gb = dev.buf(g)
    quipu.dispatch("swiglu", [("u", F)], [dev.paso(T, 0), gb, dev.buf(uu)], ((T * F + 255) // 256,))
    np.testing.assert_allclose(dev.get(gb, (T * F,)), oracle.swiglu(g, uu), rtol=2e-6, atol=1e-7)
    # routing: E = 128, k = 8, with normalization and an exact tie at the top of token 1
    E, k = 128, 8
    lg = rng.standard_normal((3, E)).astype(np.float32)
    lg[1, 9] = lg[1, 100] = 5.0
    for norm, scale in ((1, 1.0), (0, 2.5)):
        sel, wts = dev.zeros(3 * k * 4), dev.zeros(3 * k * 4)
        quipu.dispatch("moe_topk", [("u", E), ("u", k), ("u", norm), ("f", scale)],
                       [dev.paso(3, 0), dev.buf(lg), sel, wts], (1,))
        s_want, w_want = oracle.moe_topk(lg, E, k, norm, scale)
        np.testing.assert_array_equal(dev.get(sel, (3 * k,), np.uint32), s_want)
        np.testing.assert_allclose(dev.get(wts, (3 * k,)), w_want, rtol=2e-6, atol=1e-7)
        assert list(s_want[k:k + 2]) == [9, 100]
    # moe_comb: four outputs per thread when D % 4 == 0 and k <= 8, else one
    for D, kc in ((1000, k), (1002, k), (1000, 10)):
        x = rng.standard_normal((T, D)).astype(np.float32)
        de = rng.standard_normal((T * kc, D)).astype(np.float32)
        wts = rng.random(T * kc).astype(np.float32)
        xb = dev.buf(x)
        quipu.dispatch("moe_comb", [("u", D), ("u", kc)], [dev.paso(T, 0), xb, dev.buf(de), dev.buf(wts)],
                       ((T * D + 255) // 256,))
        np.testing.assert_allclose(dev.get(xb, (T, D)), oracle.moe_comb(x, de, wts, D, kc).reshape(T, D),
                                   rtol=1e-6, atol=1e-6)


def test_argmax_ties_nan_negative(quipu, dev, oracle):
    for v in (np.array([1, 3, 3, 2], np.float32), np.array([np.nan, 0.5, np.nan, 0.25], np.float32),
              np.array([-5, -1, -3], np.float32), np.random.default_rng(19).standard_normal(128256).astype(np.float32)):
        out = dev.zeros(16)
        quipu.dispatch("argmax", [("u", v.size)], [0, dev.buf(v), out])
        assert int(dev.get(out, (1,), np.uint32)[0]) == oracle.argmax(v)


# ------------------------------------------------------------------------------------------------ sampling
def topk_cand(quipu, dev, v, k):
    """topk_cand with its buffers sized as the op documents: ceil(V/2048)*(k+1) keys + flags, 2 + 2k words."""
    g = (v.size + 2047) // 2048
    part, out = dev.zeros(g * (k + 1) * 8 + g * 4), dev.zeros(4 * (2 + 2 * k))
    quipu.dispatch("topk_cand", [("u", v.size), ("u", k)], [dev.buf(v), part, out])
    o = dev.get(out, (2 + 2 * k,), np.uint32)
    return int(o[0]), int(o[1]), o[2::2].view(np.float32), o[3::2].astype(np.int64)


def distinct_logits(V, seed):
    # a permutation of V integers over 7: distinct float32 values (V < 2^24), negative and positive
    return ((np.random.default_rng(seed).permutation(V) - V // 2) / 7.0).astype(np.float32)


@pytest.mark.parametrize("V,k", [(3, 2), (100, 1), (100, 40), (2048, 128), (2049, 40), (4096, 7), (32000, 40),
                                 (128256, 40), (128256, 128), (151936, 100)])
def test_topk_candidates(quipu, dev, V, k):
    """The k largest logits, descending, with ids; chunk edges (2048, 2049) and the 8B / MoE vocabularies."""
    v = distinct_logits(V, V + k)
    flags, kk, vals, ids = topk_cand(quipu, dev, v, k)
    order = np.lexsort((np.arange(V), -v))[:k]
    assert (flags, kk) == (0, k)
    assert ids.tolist() == order.tolist()
    assert vals.view(np.uint32).tolist() == v[order].view(np.uint32).tolist()


def test_topk_candidates_flags(quipu, dev):
    """Bit 1 for two equal values among the k+1 largest (inside the set, or the k-th against the (k+1)-th), not
    below it; -0 and +0 count as equal; bit 0 for a NaN anywhere."""
    k = 40
    base = distinct_logits(5000, 3)
    top = np.argsort(-base)
    for i, j, want in ((2, 3, 2), (k - 1, k, 2), (k, k + 1, 0), (0, 1, 2)):
        v = base.copy()
        v[top[j]] = v[top[i]]
        assert topk_cand(quipu, dev, v, k)[0] == want, (i, j)
    v = -np.arange(1, 301, dtype=np.float32)
    v[10], v[20] = 0.0, -0.0
    assert topk_cand(quipu, dev, v, 5)[0] == 2
    v = base.copy()
    v[4321] = np.nan
    assert topk_cand(quipu, dev, v, k)[0] & 1


def test_topk_candidates_rejects(quipu):
    """k outside 1..128, k >= V and partial lists beyond the merge's 16384 keys fail before any launch."""
    for V, k in ((100, 0), (100, 100), (1000, 129), (300000, 128)):
        with pytest.raises(Exception, match="topk_cand"):
            quipu.dispatch("topk_cand", [("u", V), ("u", k)], [0, 0, 0])


@pytest.mark.parametrize("rep,freq,pres", [(1.3, 0.2, 0.1), (1.0, 0.5, 0.0), (0.7, 0.0, 1.25), (1.1, 0.0, 0.0)])
def test_penalizar_matches_oracle(quipu, dev, rep, freq, pres):
    """The reference's penalty arithmetic in double, stored to float: bit-exact with the oracle (ids >= V and
    history beyond the 64-token window are skipped)."""
    from oracle.sampling import Sampler
    rng = np.random.default_rng(int(rep * 100 + freq * 10 + pres))
    V = 5000
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    hist = rng.integers(0, V + 20, 90).tolist()
    want = lg.copy()
    Sampler(temperature=0.0, repeat_penalty=rep, frequency_penalty=freq, presence_penalty=pres).penalize(want, hist)
    cnt = {}
    for t in hist[-64:]:
        cnt[t] = cnt.get(t, 0) + 1
    pairs = np.array([x for kv in cnt.items() for x in kv], np.uint32)
    d = np.array([rep, freq, pres], np.float64).view(np.uint32)
    lb = dev.buf(lg)
    quipu.dispatch("penalizar", [("u", len(cnt)), ("u", V)] + [("u", int(w)) for w in d], [lb, dev.buf(pairs)])
    got = dev.get(lb, (V,))
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


# ------------------------------------------------------------------------------------------------ attention
def rope_table(base, nrot):
    """base^(-2j/nrot) rounded once to float, with the exponent the float quotient (as the JS host builds it)."""
    ex = (np.float32(-2.0) * np.arange(nrot // 2, dtype=np.float32)) / np.float32(nrot)
    return np.power(np.float64(np.float32(base)), ex.astype(np.float64)).astype(np.float32)


def f16r(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("hd,nh,nkv,T,pos0,f16", [(128, 32, 8, 1, 0, 0), (128, 32, 8, 9, 100, 0),
                                                  (64, 8, 2, 33, 40, 1), (128, 16, 16, 5, 300, 1),
                                                  (64, 16, 1, 3, 7, 0), (128, 32, 4, 70, 1000, 1),
                                                  (64, 16, 8, 17, 0, 1), (128, 32, 8, 64, 1031, 1),
                                                  (128, 8, 8, 1, 31, 1)])
def test_atencion_prefill(quipu, dev, oracle, hd, nh, nkv, T, pos0, f16):
    """The reference atencion op for a prefill chunk; with the f16 cache it runs on the matrix cores."""
    rows = max(512, pos0 + T + 5)
    kvd = nkv * hd
    rng = np.random.default_rng(20)
    q = rng.standard_normal((T, nh * hd)).astype(np.float32)
    kc = rng.standard_normal((rows, kvd)).astype(np.float32)
    vc = rng.standard_normal((rows, kvd)).astype(np.float32)
    if f16:
        kc, vc = f16r(kc), f16r(vc)
    dt = np.float16 if f16 else np.float32
    o = dev.zeros(T * nh * hd * 4)
    scale = float(np.float32(1 / np.sqrt(hd)))
    quipu.dispatch("atencion", [("u", hd), ("u", nh), ("u", nkv), ("u", 0), ("f", scale), ("u", 0), ("u", 0), ("u", 0),
                                ("u", f16), ("u", rows)],
                   [dev.paso(T, pos0), dev.buf(q), dev.buf(kc.astype(dt)),
                    dev.buf(refs.v_tiled(vc.astype(dt), kvd) if f16 else vc), o], (nh, T))
    got = dev.get(o, (T, nh * hd))
    want = oracle.attention(q, kc, vc, T, pos0, nh, nkv, hd, scale)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("table", [0, 1])
@pytest.mark.parametrize("hd,nh,nkv,pos0,nsplit,f16,neox,qk_norm",
                         [(128, 32, 8, 0, 4, 0, 0, 0), (128, 32, 8, 4095, 64, 1, 0, 0), (128, 32, 8, 777, 7, 0, 1, 1),
                          (64, 16, 16, 100, 3, 1, 1, 0), (64, 8, 1, 31, 1, 0, 0, 1), (128, 16, 8, 33, 200, 0, 0, 0),
                          (64, 32, 4, 2000, 16, 1, 0, 1), (128, 32, 4, 1500, 33, 1, 1, 1), (128, 8, 8, 5, 256, 0, 0, 0),
                          (128, 16, 8, 31, 2, 1, 0, 0), (128, 8, 1, 64, 5, 1, 1, 1), (64, 8, 4, 95, 1, 1, 0, 0)])
def test_dec_attn_fused(quipu, dev, oracle, hd, nh, nkv, pos0, nsplit, f16, neox, qk_norm, table):
    """One-token attention with the fused q/k norm + RoPE + KV append, split over the keys and merged by
    dec_attn_comb, with the RoPE frequency table bound or computed in the kernel; the expected result is the
    reference op sequence norm_rope(q), norm_rope(k), kv_write, atencion."""
    rows = 4100
    kvd = nkv * hd
    rng = np.random.default_rng(21)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    kc = rng.standard_normal((rows, kvd)).astype(np.float32)
    vc = rng.standard_normal((rows, kvd)).astype(np.float32)
    if f16:
        kc, vc = f16r(kc), f16r(vc)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    eps, base = 1e-6, 1e6
    scale = float(np.float32(1 / np.sqrt(hd)))
    dt = np.float16 if f16 else np.float32
    kcb, vcb = dev.buf(kc.astype(dt)), dev.buf(refs.v_tiled(vc.astype(dt), kvd) if f16 else vc)
    po, pml, o = dev.zeros(nh * nsplit * hd * 4), dev.zeros(nh * nsplit * 8), dev.zeros(nh * hd * 4)
    paso = dev.paso(1, pos0)
    u = [("u", hd), ("u", nh), ("u", nkv), ("u", nsplit), ("f", scale), ("f", eps), ("f", base), ("u", 0),
         ("u", hd), ("u", neox), ("u", f16), ("u", rows)]
    b = [paso, dev.buf(q), dev.buf(k), dev.buf(v), kcb, vcb, dev.buf(qn) if qk_norm else 0,
         dev.buf(kn) if qk_norm else 0, po, pml]
    if table:
        b.append(dev.buf(rope_table(base, hd)))
    quipu.dispatch("dec_attn", u, b)
    quipu.dispatch("dec_attn_comb", [("u", hd), ("u", nh), ("u", nsplit)], [paso, po, pml, o])
    got = dev.get(o, (nh * hd,))
    qr = oracle.norm_rope(q, qn, nh, hd, qk_norm, neox, eps, base, hd, pos0)
    kr = oracle.norm_rope(k, kn, nkv, hd, qk_norm, neox, eps, base, hd, pos0)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[pos0] = f16r(kr) if f16 else kr
    vc2[pos0] = f16r(v) if f16 else v
    want = oracle.attention(qr, kc2, vc2, 1, pos0, nh, nkv, hd, scale)[0]
    np.testing.assert_allclose(got, want, rtol=5e-5, atol=5e-5)
    # the appended cache row: RoPE'd key (to within the rotation's rounding), value copied (rounded if f16)
    gk = dev.get(kcb, (rows, kvd), dt)
    gv = refs.v_rows(dev.get(vcb, ((rows + 31) // 32 * 32, kvd), dt), rows, kvd) if f16 else dev.get(vcb, (rows, kvd))
    np.testing.assert_allclose(gk[pos0].astype(np.float32), kc2[pos0], rtol=1e-5, atol=2e-3 if f16 else 1e-5)
    np.testing.assert_array_equal(gv[pos0].astype(np.float32), vc2[pos0])
    np.testing.assert_array_equal(gv[pos0 + 1:].astype(np.float32), vc[pos0 + 1:])


MERGED_CASES = [(128, 32, 8, 4095, 17, 1, 0, 0), (128, 32, 4, 2047, 18, 1, 1, 1), (128, 32, 8, 777, 7, 0, 1, 1),
                (64, 8, 1, 31, 1, 0, 0, 1), (128, 16, 8, 33, 200, 0, 0, 0), (64, 32, 4, 2000, 16, 1, 0, 1),
                (128, 8, 1, 64, 5, 1, 1, 1), (64, 8, 2, 95, 300, 1, 0, 0), (128, 16, 2, 3000, 1024, 1, 0, 0)]


@pytest.mark.parametrize("hd,nh,nkv,pos0,nsplit,f16,neox,qk_norm,gsplit",
                         [c + (1,) for c in MERGED_CASES] +
                         [c + (g,) for c in MERGED_CASES for g in (2, 4)
                          if c[2] * g <= 8 and (c[1] // c[2]) % g == 0])
def test_dec_attn_merged(quipu, dev, hd, nh, nkv, pos0, nsplit, f16, neox, qk_norm, gsplit):
    """dec_attn with P[12] = 1: the last workgroup of each grid column to finish merges its heads' partials in the
    same launch (grid x = 8, so a column's workgroups share one XCD); with P[13] = gsplit > 1 a KV head's query
    heads are split over gsplit columns (each streams the head's keys, one appends).  The same as dec_attn +
    dec_attn_comb up to the order of the merge's sums (within 1e-5), the same cache row appended, and bit-identical
    over three launches in a row whichever workgroup finishes last (the arrival counters return to zero after
    each), including splits without keys (nsplit 200 .. 1024 over a short cache)."""
    rows = 4100
    kvd = nkv * hd
    rng = np.random.default_rng(22)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    kc = rng.standard_normal((rows, kvd)).astype(np.float32)
    vc = rng.standard_normal((rows, kvd)).astype(np.float32)
    if f16:
        kc, vc = f16r(kc), f16r(vc)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    dt = np.float16 if f16 else np.float32
    u = [("u", hd), ("u", nh), ("u", nkv), ("u", nsplit), ("f", float(np.float32(1 / np.sqrt(hd)))), ("f", 1e-6),
         ("f", 1e6), ("u", 0), ("u", hd), ("u", neox), ("u", f16), ("u", rows)]

    def run(merged):
        kcb, vcb = dev.buf(kc.astype(dt)), dev.buf(refs.v_tiled(vc.astype(dt), kvd) if f16 else vc)
        po, pml, o = dev.zeros(nh * nsplit * hd * 4), dev.zeros(nh * nsplit * 8), dev.zeros(nh * hd * 4)
        paso = dev.paso(1, pos0)
        b = [paso, dev.buf(q), dev.buf(k), dev.buf(v), kcb, vcb, dev.buf(qn) if qk_norm else 0,
             dev.buf(kn) if qk_norm else 0, po, pml, dev.buf(rope_table(1e6, hd))]
        outs = []
        if merged:
            cnt = dev.zeros(8 * 128 + 128)
            for _ in range(3):
                quipu.upload(o, np.full(nh * hd, np.nan, np.float32))
                quipu.dispatch("dec_attn", u + [("u", 1), ("u", gsplit)], b + [o, cnt], (1, 1, 1))
                outs.append(dev.get(o, (nh * hd,)))
            assert np.all(dev.get(cnt, (8 * 32 + 1,), np.uint32) == 0)  # counters back at zero, error word clear
        else:
            quipu.dispatch("dec_attn", u, b)
            quipu.dispatch("dec_attn_comb", [("u", hd), ("u", nh), ("u", nsplit)], [paso, po, pml, o])
            outs.append(dev.get(o, (nh * hd,)))
        return outs, dev.get(kcb, (rows, kvd), dt)

    want, kw = run(False)
    got, kg = run(True)
    np.testing.assert_allclose(got[0], want[0], rtol=1e-5, atol=1e-6)
    for g in got[1:]:
        np.testing.assert_array_equal(g, got[0])
    np.testing.assert_array_equal(kg, kw)


@pytest.mark.parametrize("hd,nh,nkv,D,fv,pos0,ns,neox,qk_norm",
                         [(128, 32, 8, 4096, capi.Q6_K, 4095, 64, 0, 0), (128, 32, 4, 2048, capi.Q4_K, 2047, 64, 1, 1),
                          (128, 32, 8, 4096, capi.Q6_K, 2000, 32, 0, 0),
                          (128, 8, 2, 512, capi.Q6_K, 300, 16, 1, 1), (64, 8, 2, 512, capi.Q6_K, 100, 8, 0, 0),
                          (128, 16, 8, 1024, capi.Q4_K, 31, 4, 0, 1), (64, 32, 8, 1024, capi.Q6_K, 5, 64, 1, 0),
                          (128, 32, 8, 4096, capi.Q6_K, 0, 32, 0, 0), (64, 8, 1, 256, capi.Q4_K, 700, 2, 0, 0)])
def test_dec_attn_block(quipu, dev, hd, nh, nkv, D, fv, pos0, ns, neox, qk_norm):
    """dec_attn_block (Q/K/V GEMV with the fused norm, attention, KV append and the split merge in one launch, the
    8 head groups on the 8 XCDs meeting at barriers in their L2) against the three launches it replaces: gemv (Q,
    K Q4_K and V in one launch) + dec_attn + dec_attn_comb on the same inputs.  q, k, v and the appended cache row
    are bit-identical; the merged output (other split boundaries) within 5e-5.  Three launches in a row (the
    barrier counters only grow) give identical outputs, and no barrier timeout or group spread over two XCDs is
    recorded."""
    rows = 4100
    kvd = nkv * hd
    rng = np.random.default_rng(23)
    x = rng.standard_normal(D).astype(np.float32)
    nw = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    kc = f16r(rng.standard_normal((rows, kvd)).astype(np.float32))
    vc = f16r(rng.standard_normal((rows, kvd)).astype(np.float32))
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    eps, base = 1e-6, 1e6
    scale = float(np.float32(1 / np.sqrt(hd)))
    mats = [(capi.Q4_K, nh * hd, 90), (capi.Q4_K, kvd, 91), (fv, kvd, 92)]
    W = [dev.matrix(f, raw_matrix(f, n, D, sd), n, D) for f, n, sd in mats]
    xb, nwb, paso = dev.buf(x), dev.buf(nw), dev.paso(1, pos0)
    qnb, knb = (dev.buf(qn), dev.buf(kn)) if qk_norm else (0, 0)
    freq = dev.buf(rope_table(base, hd))

    def fresh():
        return (dev.buf(kc.astype(np.float16)), dev.buf(refs.v_tiled(vc.astype(np.float16), kvd)),
                dev.zeros(nh * hd * 4), dev.zeros(kvd * 4), dev.zeros(kvd * 4), dev.zeros(nh * hd * 4))

    # the three launches
    kcb, vcb, q, k, v, o = fresh()
    segs = [(capi.STORE, nh * hd, 0, nh * hd, capi.Q4_K), (capi.STORE, kvd, 0, kvd, capi.Q4_K),
            (capi.STORE, kvd, 0, kvd, fv)]
    quipu.dispatch("gemv", capi.gemv_uniform(3, D, eps=eps, fmt=capi.Q4_K, segs=segs),
                   [paso, xb, nwb, 0, W[0], 0, q, W[1], 0, k, W[2], 0, v])
    nsp = 17
    po, pml = dev.zeros(nh * nsp * hd * 4), dev.zeros(nh * nsp * 8)
    ua = [("u", hd), ("u", nh), ("u", nkv), ("u", nsp), ("f", scale), ("f", eps), ("f", base), ("u", 0),
          ("u", hd), ("u", neox), ("u", 1), ("u", rows)]
    quipu.dispatch("dec_attn", ua, [paso, q, k, v, kcb, vcb, qnb, knb, po, pml, freq])
    quipu.dispatch("dec_attn_comb", [("u", hd), ("u", nh), ("u", nsp)], [paso, po, pml, o])
    want = [dev.get(t, (n,)) for t, n in ((q, nh * hd), (k, kvd), (v, kvd), (o, nh * hd))]
    want_k = dev.get(kcb, (rows, kvd), np.float16)
    want_v = dev.get(vcb, ((rows + 31) // 32 * 32, kvd), np.float16)

    # the one launch
    kcb, vcb, q, k, v, o = fresh()
    po, pml, sync = dev.zeros(nh * ns * hd * 4), dev.zeros(nh * ns * 8), dev.zeros(2304)
    ub = [("u", hd), ("u", nh), ("u", nkv), ("u", ns), ("f", scale), ("f", eps), ("f", base), ("u", 0), ("u", hd),
          ("u", neox), ("u", rows), ("u", D), ("u", capi.Q4_K), ("u", capi.Q4_K), ("u", fv), ("u", 0)]
    outs = []
    for it in range(3):
        if it:  # the same token again: restore the cache row the launch appended
            quipu.upload(kcb, kc.astype(np.float16))
            quipu.upload(vcb, refs.v_tiled(vc.astype(np.float16), kvd))
        quipu.upload(o, np.full(nh * hd, np.nan, np.float32))
        quipu.dispatch("dec_attn_block", ub, [paso, xb, nwb, W[0], W[1], W[2], q, k, v, kcb, vcb, qnb, knb, po, pml,
                                              freq, o, sync], (8, ns, 1))
        outs.append(dev.get(o, (nh * hd,)))
        if it == 0:
            for t, n, w_ in zip((q, k, v), (nh * hd, kvd, kvd), want):
                np.testing.assert_array_equal(dev.get(t, (n,)), w_)
            np.testing.assert_array_equal(dev.get(kcb, (rows, kvd), np.float16), want_k)
            np.testing.assert_array_equal(dev.get(vcb, ((rows + 31) // 32 * 32, kvd), np.float16), want_v)
    sw = dev.get(sync, (576,), np.uint32)
    bad = np.abs(outs[0] - want[3]) > 5e-5 + 5e-5 * np.abs(want[3])
    print("error word %#x, XCD words %s, counters %s, mismatches per head %s, per launch %s" % (
        sw[528], [hex(m) for m in sw[512:520]], sw[0:512:64].tolist(),
        bad.reshape(nh, hd).sum(axis=1).tolist(), [int((np.abs(o_ - want[3]) > 1e-3).sum()) for o_ in outs]))
    np.testing.assert_allclose(outs[0], want[3], rtol=5e-5, atol=5e-5)
    for o_ in outs[1:]:
        np.testing.assert_array_equal(o_, outs[0])
    assert sw[528] == 0, "barrier timeout or a group on two XCDs (error word %#x)" % sw[528]
    xw = sw[512:520]
    assert len(set(xw.tolist())) == 8 and all(1 <= w <= 16 for w in xw)  # each group on an XCD of its own
    # each group's counter: 2 barriers x ns arrivals per launch
    assert np.all(sw[0:512:64] == 3 * 2 * ns)


def test_dec_attn_block_wait_bound(quipu, dev):
    """The barriers' bounded wait, forced from the host: with spin_max = 1 a workgroup that arrives early gives up
    after two polls, sets bit 0 of the error word and goes on, so the launch still ends (its results are not
    meaningful).  Every workgroup still arrives at both barriers, so the counters stay consistent: after the error
    word is cleared, a launch with the default bound gives the three-launch result again with no error."""
    hd, nh, nkv, D, rows, pos0, ns = 128, 32, 8, 4096, 4100, 3000, 32
    kvd = nkv * hd
    rng = np.random.default_rng(24)
    x = rng.standard_normal(D).astype(np.float32)
    nw = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    kc = f16r(rng.standard_normal((rows, kvd)).astype(np.float32))
    vc = f16r(rng.standard_normal((rows, kvd)).astype(np.float32))
    mats = [(capi.Q4_K, nh * hd, 90), (capi.Q4_K, kvd, 91), (capi.Q6_K, kvd, 92)]
    W = [dev.matrix(f, raw_matrix(f, n, D, sd), n, D) for f, n, sd in mats]
    xb, nwb, paso, freq = dev.buf(x), dev.buf(nw), dev.paso(1, pos0), dev.buf(rope_table(1e6, hd))
    scale = float(np.float32(1 / np.sqrt(hd)))
    kcb, vcb = dev.buf(kc.astype(np.float16)), dev.buf(refs.v_tiled(vc.astype(np.float16), kvd))
    q, k, v, o = dev.zeros(nh * hd * 4), dev.zeros(kvd * 4), dev.zeros(kvd * 4), dev.zeros(nh * hd * 4)
    po, pml, sync = dev.zeros(nh * ns * hd * 4), dev.zeros(nh * ns * 8), dev.zeros(2304)
    b = [paso, xb, nwb, W[0], W[1], W[2], q, k, v, kcb, vcb, 0, 0, po, pml, freq, o, sync]

    def launch(spin):
        u = [("u", hd), ("u", nh), ("u", nkv), ("u", ns), ("f", scale), ("f", 1e-6), ("f", 1e6), ("u", 0),
             ("u", hd), ("u", 0), ("u", rows), ("u", D), ("u", capi.Q4_K), ("u", capi.Q4_K), ("u", capi.Q6_K),
             ("u", spin)]
        quipu.upload(kcb, kc.astype(np.float16))
        quipu.upload(vcb, refs.v_tiled(vc.astype(np.float16), kvd))
        quipu.dispatch("dec_attn_block", u, b, (8, ns, 1))
        return dev.get(o, (nh * hd,)), dev.get(sync, (576,), np.uint32)

    want, sw = launch(0)
    assert sw[528] == 0
    _, sw = launch(1)
    assert sw[528] & 1, "no barrier wait ran past a bound of one poll"
    assert np.all(sw[0:512:64] == 2 * 2 * ns)
    quipu.upload(sync, np.concatenate([sw[:528], np.zeros(576 - 528, np.uint32)]))
    got, sw = launch(0)
    assert sw[528] == 0
    np.testing.assert_array_equal(got, want)


def test_dec_attn_block_rejections(quipu, dev):
    """Shapes the kernel cannot take are refused on the host before any launch."""
    base = [("u", 128), ("u", 32), ("u", 8), ("u", 32), ("f", 0.1), ("f", 1e-5), ("f", 1e4), ("u", 0), ("u", 128),
            ("u", 0), ("u", 64), ("u", 4096), ("u", capi.Q4_K), ("u", capi.Q4_K), ("u", capi.Q6_K), ("u", 0)]
    bufs = [dev.zeros(64) for _ in range(18)]
    for i, v, msg in [(3, 24, "ns=24"), (3, 128, "ns=128"), (2, 16, "nkv 1, 2, 4 or 8"), (0, 96, "head_dim 96"),
                      (11, 4000, "model width 4000"), (14, capi.Q8_0, "Q/K/V format"), (1, 64, "query heads per group")]:
        u = list(base)
        u[i] = ("u", v)
        with pytest.raises(capi.QuipuError, match=msg):
            quipu.dispatch("dec_attn_block", u, bufs, (8, 32, 1))
    with pytest.raises(capi.QuipuError, match="sync must be"):
        quipu.dispatch("dec_attn_block", base, bufs, (8, 32, 1))


def test_dec_attn_merged_rejections(quipu, dev):
    """The merged form needs at most 8 columns (KV heads x gsplit), a gsplit of 1, 2, 4 or 8 dividing the query
    group, the output and a counter buffer of this library."""
    hd, nh, nkv, rows = 64, 16, 16, 64
    b = [dev.paso(1, 3)] + [dev.zeros(4 * nh * hd)] * 3 + [dev.zeros(4 * rows * nkv * hd)] * 2 + [0, 0] + \
        [dev.zeros(4 * nh * hd), dev.zeros(8 * nh), 0, dev.zeros(4 * nh * hd), dev.zeros(1028)]
    u = [("u", hd), ("u", nh), ("u", nkv), ("u", 1), ("f", 0.125), ("f", 1e-6), ("f", 1e4), ("u", 0), ("u", hd),
         ("u", 0), ("u", 0), ("u", rows), ("u", 1)]
    with pytest.raises(capi.QuipuError, match="at most 8 columns"):
        quipu.dispatch("dec_attn", u, b)
    u[2] = ("u", 8)  # groups of 2 query heads
    for g, msg in ((2, "at most 8 columns"), (3, "gsplit=3"), (4, "does not divide")):
        with pytest.raises(capi.QuipuError, match=msg):
            quipu.dispatch("dec_attn", u + [("u", g)], b)
    with pytest.raises(capi.QuipuError, match="at least 1028 bytes"):
        quipu.dispatch("dec_attn", u, b[:12] + [dev.zeros(1024)])


def test_xcd_placement_checks_fire_and_recover(quipu, dev):
    """The merged attention and moe_router count arrivals in their XCD's L2 and rely on every workgroup of a grid
    column running on one XCD.  Each arrival adds 1 + (XCD id << 16) to the column's counter and the last one checks
    the sum, so a column spread over XCDs sets the op's error word instead of failing silently.  Forced from the host:
    a counter seeded with an arrival from a foreign XCD (high half 1, count 0) makes the last arrival's check fire
    while the results stay exact (the merge and the routing still run), and the counter is reset, so the next launch
    is exact with the error word clear; a counter seeded with a full launch's arrivals left over (every later count
    past the grid) fires too.  Every kernel ends normally in all cases."""
    # merged attention: the 8B shapes at position 4095, 17 splits, f16 cache
    hd, nh, nkv, pos0, nsplit, rows = 128, 32, 8, 4095, 17, 4100
    kvd = nkv * hd
    rng = np.random.default_rng(31)
    kc = f16r(rng.standard_normal((rows, kvd)).astype(np.float32))
    vc = f16r(rng.standard_normal((rows, kvd)).astype(np.float32))
    u = [("u", hd), ("u", nh), ("u", nkv), ("u", nsplit), ("f", float(np.float32(1 / np.sqrt(hd)))), ("f", 1e-6),
         ("f", 5e5), ("u", 0), ("u", hd), ("u", 0), ("u", 1), ("u", rows), ("u", 1), ("u", 1)]
    q, k, v = (rng.standard_normal(n).astype(np.float32) for n in (nh * hd, kvd, kvd))
    kcb, vcb = dev.buf(kc.astype(np.float16)), dev.buf(refs.v_tiled(vc.astype(np.float16), kvd))
    po, pml, o, cnt = dev.zeros(nh * nsplit * hd * 4), dev.zeros(nh * nsplit * 8), dev.zeros(nh * hd * 4), \
        dev.zeros(8 * 128 + 128)
    b = [dev.paso(1, pos0), dev.buf(q), dev.buf(k), dev.buf(v), kcb, vcb, 0, 0, po, pml, dev.buf(rope_table(5e5, hd)),
         o, cnt]

    def attn(seed=None):
        if seed is not None:
            quipu.upload(cnt, np.array([seed if i % 32 == 0 and i < 256 else 0 for i in range(8 * 32 + 1)], np.uint32))
        quipu.upload(o, np.full(nh * hd, np.nan, np.float32))
        quipu.dispatch("dec_attn", u, b, (1, 1, 1))
        w = dev.get(cnt, (8 * 32 + 1,), np.uint32)
        return dev.get(o, (nh * hd,)), int(w[256]), [int(w[32 * i]) for i in range(8)]

    want, err, c = attn()
    assert err == 0 and c == [0] * 8 and np.isfinite(want).all()
    got, err, c = attn(seed=1 << 16)          # a foreign XCD's arrival in every column
    assert err == 1 and c == [0] * 8
    np.testing.assert_array_equal(got, want)
    got, err, c = attn(seed=0)                # error word cleared by the host: the next launch is exact and clean
    assert err == 0 and c == [0] * 8
    np.testing.assert_array_equal(got, want)
    _, err, _ = attn(seed=nsplit)             # a full launch's arrivals left over: every count passes the grid
    assert err == 1
    got, err, c = attn(seed=0)
    assert err == 0 and c == [0] * 8
    np.testing.assert_array_equal(got, want)

    # moe_router: 128 experts, 32 workgroups
    E, kk, D, nw = 128, 8, 2048, 32
    W = (0.02 * rng.standard_normal((E, D))).astype(np.float32)
    x = rng.standard_normal(D).astype(np.float32)
    lg, sel, wts, rc = dev.zeros(E * 4), dev.zeros(kk * 4), dev.zeros(kk * 4), dev.zeros(8)
    ur = [("u", E), ("u", D), ("u", kk), ("u", nw), ("f", 1e-6), ("f", 1.0), ("u", 1)]
    br = [dev.paso(1, 0), dev.buf(W), dev.buf(x), dev.buf(np.ones(D, np.float32)), lg, sel, wts, rc]

    def route(seed):
        quipu.upload(rc, np.array([seed, 0], np.uint32))
        quipu.upload(sel, np.full(kk, 0xffffffff, np.uint32))
        quipu.dispatch("moe_router", ur, br, (8, nw, 1))
        w = dev.get(rc, (2,), np.uint32)
        return dev.get(sel, (kk,), np.uint32), dev.get(wts, (kk,)), int(w[1]), int(w[0])

    s0, w0, err, c = route(0)
    assert err == 0 and c == 0 and np.all(s0 < E)
    s1, w1, err, c = route(1 << 16)
    assert err == 1 and c == 0
    np.testing.assert_array_equal(s1, s0)
    np.testing.assert_array_equal(w1, w0)
    s1, w1, err, c = route(0)
    assert err == 0 and c == 0
    np.testing.assert_array_equal(s1, s0)
    _, _, err, _ = route(nw)
    assert err == 1
    s1, w1, err, c = route(0)
    assert err == 0 and c == 0
    np.testing.assert_array_equal(s1, s0)
    np.testing.assert_array_equal(w1, w0)


@pytest.mark.parametrize("pos0", [4, 40, 700])
def test_attention_large_scores_stay_finite(quipu, dev, oracle, pos0):
    """Scores of order 1e8 (q and k of order 1e4) through the matrix-core decode and prefill attention: the softmax
    exponent must use the rounded score the running max was taken over, or p (scaled into the f16 range) overflows
    and the result turns NaN."""
    hd, nh, nkv, nsplit, rows = 128, 32, 8, 35, 1024
    kvd = nkv * hd
    rng = np.random.default_rng(pos0)
    q = (rng.standard_normal(nh * hd) * 1e4).astype(np.float32)
    k = (rng.standard_normal(kvd) * 1e4).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    kc = f16r(rng.standard_normal((rows, kvd)) * 1e4)
    vc = f16r(rng.standard_normal((rows, kvd)))
    scale = float(np.float32(1 / np.sqrt(hd)))
    kcb, vcb = dev.buf(kc.astype(np.float16)), dev.buf(refs.v_tiled(vc.astype(np.float16), kvd))
    po, pml, o = dev.zeros(nh * nsplit * hd * 4), dev.zeros(nh * nsplit * 8), dev.zeros(nh * hd * 4)
    paso = dev.paso(1, pos0)
    u = [("u", hd), ("u", nh), ("u", nkv), ("u", nsplit), ("f", scale), ("f", 1e-5), ("f", 1e4), ("u", 0),
         ("u", hd), ("u", 0), ("u", 1), ("u", rows)]
    quipu.dispatch("dec_attn", u, [paso, dev.buf(q), dev.buf(k), dev.buf(v), kcb, vcb, 0, 0, po, pml])
    quipu.dispatch("dec_attn_comb", [("u", hd), ("u", nh), ("u", nsplit)], [paso, po, pml, o])
    got = dev.get(o, (nh * hd,))
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[pos0] = f16r(oracle.norm_rope(k, None, nkv, hd, 0, 0, 1e-5, 1e4, hd, pos0))
    vc2[pos0] = f16r(v)
    want = oracle.attention(oracle.norm_rope(q, None, nh, hd, 0, 0, 1e-5, 1e4, hd, pos0), kc2, vc2, 1, pos0, nh, nkv,
                            hd, scale)[0]
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)
    # the prefill op over the same cache (up to 8 queries ending at pos0)
    T = min(8, pos0 + 1)
    qp = (rng.standard_normal((T, nh * hd)) * 1e4).astype(np.float32)
    op = dev.zeros(T * nh * hd * 4)
    quipu.dispatch("atencion", [("u", hd), ("u", nh), ("u", nkv), ("u", 0), ("f", scale), ("u", 0), ("u", 0), ("u", 0),
                                ("u", 1), ("u", rows)],
                   [dev.paso(T, pos0 - T + 1), dev.buf(qp), kcb, vcb, op], (nh, T))  # the cache after the append
    gotp = dev.get(op, (T, nh * hd))
    assert np.isfinite(gotp).all()
    np.testing.assert_allclose(gotp, oracle.attention(qp, kc2, vc2, T, pos0 - T + 1, nh, nkv, hd, scale), rtol=1e-4,
                               atol=1e-4)


def test_dec_attn_past_the_cache_reads_and_writes_nothing(quipu, dev):
    hd, nh, nkv, rows, nsplit = 64, 4, 2, 16, 2
    kvd = nkv * hd
    kc = dev.zeros(rows * kvd * 4)
    po, pml = dev.zeros(nh * nsplit * hd * 4), dev.zeros(nh * nsplit * 8)
    o = dev.buf(np.ones(nh * hd, np.float32))
    one = dev.buf(np.ones(nh * hd, np.float32))
    paso = dev.paso(1, rows)
    u = [("u", hd), ("u", nh), ("u", nkv), ("u", nsplit), ("f", 0.125), ("f", 1e-6), ("f", 1e4), ("u", 0), ("u", hd),
         ("u", 0), ("u", 0), ("u", rows)]
    quipu.dispatch("dec_attn", u, [paso, one, one, one, kc, kc, 0, 0, po, pml])
    quipu.dispatch("dec_attn_comb", [("u", hd), ("u", nh), ("u", nsplit)], [paso, po, pml, o])
    assert not dev.get(kc, (rows * kvd,)).any()
    assert not dev.get(o, (nh * hd,)).any()


def test_dec_attn_consecutive_tokens(quipu, dev, oracle):
    """Three tokens in a row, each appending its key and attending over everything before it; checked against
    the reference op sequence."""
    hd, nh, nkv, nsplit, rows = 128, 32, 8, 16, 64
    kvd = nkv * hd
    rng = np.random.default_rng(23)
    kc = rng.standard_normal((rows, kvd)).astype(np.float32)
    vc = rng.standard_normal((rows, kvd)).astype(np.float32)
    kcb, vcb = dev.buf(kc), dev.buf(vc)
    o = dev.zeros(nh * hd * 4)
    po, pml = dev.zeros(nh * nsplit * hd * 4), dev.zeros(nh * nsplit * 8)
    scale = float(np.float32(1 / np.sqrt(hd)))
    u = [("u", hd), ("u", nh), ("u", nkv), ("u", nsplit), ("f", scale), ("f", 1e-5), ("f", 1e4), ("u", 0), ("u", hd),
         ("u", 0), ("u", 0), ("u", rows)]
    for pos0 in (40, 41, 42):
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k = rng.standard_normal(kvd).astype(np.float32)
        v = rng.standard_normal(kvd).astype(np.float32)
        paso = dev.paso(1, pos0)
        quipu.dispatch("dec_attn", u, [paso, dev.buf(q), dev.buf(k), dev.buf(v), kcb, vcb, 0, 0, po, pml])
        quipu.dispatch("dec_attn_comb", [("u", hd), ("u", nh), ("u", nsplit)], [paso, po, pml, o])
        kc[pos0] = oracle.norm_rope(k, None, nkv, hd, 0, 0, 1e-5, 1e4, hd, pos0)
        vc[pos0] = v
        want = oracle.attention(oracle.norm_rope(q, None, nh, hd, 0, 0, 1e-5, 1e4, hd, pos0), kc, vc, 1, pos0, nh,
                                nkv, hd, scale)[0]
        np.testing.assert_allclose(dev.get(o, (nh * hd,)), want, rtol=5e-5, atol=5e-5)


# ------------------------------------------------------------------------------------------------ graphs
def test_graph_replay_matches_eager(quipu, dev, oracle):
    """A captured decode-like step (fused-norm GEMV + argmax with position advance) replayed 5 times with host
    reads between the replays; each replay must reproduce the eager result and advance the position."""
    V, K, maxwg = 800, 1024, 64
    raw = raw_matrix(capi.Q4_K, V, K, 80)
    x = np.random.default_rng(22).standard_normal(K).astype(np.float32)
    nw = np.ones(K, np.float32)
    w = dev.matrix(capi.Q4_K, raw, V, K)
    y, amax, ids, step = dev.zeros(V * 4), dev.zeros(8 * maxwg), dev.zeros(16), dev.zeros(16)
    toks = dev.zeros(4 * 16)
    paso = dev.paso(1, 0)
    xb, nb = dev.buf(x), dev.buf(nw)
    u = capi.gemv_uniform(1, K, eps=1e-5, R=4, max_wg=maxwg, fmt=capi.Q4_K, segs=[(capi.ARGMAX, V, 0, V)])

    def step_ops():
        quipu.dispatch("gemv", u, [paso, xb, nb, amax, w, 0, y])
        quipu.dispatch("argmax_fin", [("u", maxwg), ("u", 1), ("u", 16)], [paso, amax, ids, toks, step])

    step_ops()
    eager_y = dev.get(y, (V,)).copy()
    eager_id = int(dev.get(ids, (1,), np.uint32)[0])
    assert eager_id == oracle.argmax(eager_y)
    quipu.sync()
    quipu.graph_begin()
    step_ops()
    g = quipu.graph_end()
    try:
        for r in range(5):
            quipu.upload(y, np.zeros(V, np.float32))
            quipu.graph_launch(g)
            np.testing.assert_array_equal(dev.get(y, (V,)), eager_y)
            assert int(dev.get(ids, (1,), np.uint32)[0]) == eager_id
            assert list(dev.get(paso, (2,), np.uint32)) == [1, 2 + r]
        assert list(dev.get(toks, (6,), np.uint32)) == [eager_id] * 6
    finally:
        quipu.graph_free(g)


# ------------------------------------------------------------------------------------------------ errors
def raw_fmt_word(u, fmt):
    """A gemv uniform with its format word replaced by fmt."""
    u = list(u)
    u[6] = ("u", fmt)
    return u


def test_host_checks_reject_bad_dispatches(quipu, dev):
    """Shapes and bindings the kernels cannot take are refused on the host, before any launch."""
    x = dev.zeros(4096 * 4)
    y = dev.zeros(4096 * 4)
    w = dev.zeros(144 * 16)
    p = dev.paso(1, 0)
    wbig, am1 = dev.zeros(144 * 4096), dev.zeros(8)
    bad = [
        ("gemv", capi.gemv_uniform(0, 256, segs=[]), [p, x, 0, 0]),
        ("gemv", capi.gemv_uniform(1, 256, R=3, segs=[(capi.STORE, 16, 0, 16)]), [p, x, 0, 0, w, 0, y]),
        ("gemv", capi.gemv_uniform(1, 300, segs=[(capi.STORE, 16, 0, 16)]), [p, x, 0, 0, w, 0, y]),
        ("gemv", capi.gemv_uniform(1, 256, segs=[(capi.SWIGLU, 16, 0, 16)]), [p, x, 0, 0, w, 0, y]),
        ("gemv", capi.gemv_uniform(1, 256, segs=[(capi.ARGMAX, 16, 0, 16)]), [p, x, 0, 0, w, 0, y]),
        ("gemv", capi.gemv_uniform(1, 256, segs=[(capi.STORE, 16, 0, 16)]), [p, x, 0, 0, w]),
        ("gemv", capi.gemv_uniform(1, 256 * 61, segs=[(capi.STORE, 1, 0, 1)]), [p, x, 0, 0, w, 0, y]),
        ("kv_write", [("u", 64), ("u", 0), ("u", 0), ("u", 0)], [p, x, x, y, y]),
        ("atencion", [("u", 96), ("u", 4), ("u", 2), ("u", 0), ("f", 1), ("u", 0), ("u", 0), ("u", 0), ("u", 0),
                      ("u", 8)], [p, x, y, y, x]),
        ("dec_attn", [("u", 128), ("u", 12), ("u", 4), ("u", 1), ("f", 1), ("f", 0), ("f", 1), ("u", 0), ("u", 128),
                      ("u", 0), ("u", 0), ("u", 8)], [p, x, x, x, y, y, 0, 0, y, y]),
        ("moe_topk", [("u", 2000), ("u", 8), ("u", 1), ("f", 1)], [p, x, y, y]),
        ("matmul_q8_1", [("u", 16), ("u", 256), ("u", 0), ("u", 0)], [p, w, w + 8, x, y]),
        # a format word that is not a device layout (the GGUF type of F16, converted to f32 at load), and weights
        # smaller than their format and rows need (16 f32 rows of 256 in 2304 bytes; 32 Q4_K rows)
        ("gemv", raw_fmt_word(capi.gemv_uniform(1, 256, segs=[(capi.STORE, 16, 0, 16)]), 1),
         [p, x, 0, 0, w, 0, y]),
        ("gemv", capi.gemv_uniform(1, 256, fmt=capi.F32, R=1, segs=[(capi.STORE, 16, 0, 16)]), [p, x, 0, 0, w, 0, y]),
        ("gemv", capi.gemv_uniform(1, 256, segs=[(capi.STORE, 16, 0, 32)]), [p, x, 0, 0, w, 0, y]),
        ("dequant", [("u", 1), ("u", 512), ("u", 0), ("u", 256)], [0, w, y]),
        ("dequant", [("u", capi.Q4_K), ("u", 32 * 256), ("u", 0), ("u", 256)], [0, w, y]),
        # an argmax segment whose partials buffer holds fewer entries than the launch has workgroups (4096 Q4_K
        # rows of 256: 64 units, 16 workgroups, one 8-byte entry each)
        ("gemv", capi.gemv_uniform(1, 256, segs=[(capi.ARGMAX, 4096, 0, 4096)]), [p, x, 0, am1, wbig, 0, y]),
    ]
    for name, u, b in bad:
        with pytest.raises(capi.QuipuError):
            quipu.dispatch(name, u, b)
    quipu.sync()  # nothing was launched, the stream is healthy
    with pytest.raises(capi.QuipuError):
        quipu.free(12345)


def test_allocation_accounting(quipu):
    before = quipu.bytes_used()
    h = quipu.alloc(1 << 20)
    assert quipu.bytes_used() >= before + (1 << 20)
    quipu.free(h)
    assert quipu.bytes_used() == before
