"""Pins the CPU oracle (oracle/qp_oracle.c) -- the checker every GPU parity test relies on.

The reference path (WGSL on WebGPU) cannot run here and commits no golden vectors for it, so each oracle function is
checked against what fixes it independently: exact library conversions, the ggml-spec dequantizers of refs.py,
float64 textbook formulas, closed forms and invariants.  Each check is chosen so that a plausible mistake (a dropped
min term, a swapped nibble, a wrong RoPE pairing, a GQA off-by-one, an exp sign) fails it.
"""
import numpy as np
import pytest

import refs
from quipullm_amd import synth


def blocks(fmt, n_elem, seed=0, centered=False):
    return np.frombuffer(synth.gen_blocks(np.random.default_rng(seed), fmt, n_elem, "w", centered), np.uint8)


# ------------------------------------------------------------------------------------------------ formats
def test_f16_all_values_exact(oracle):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16(int(x)) for x in h[::7]], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32)[~np.isnan(got)],
                                  ref[::7].view(np.uint32)[~np.isnan(ref[::7])])
    assert np.array_equal(np.isnan(got), np.isnan(ref[::7]))


def test_f16_rounding_matches_numpy(oracle):
    # every finite f16, the midpoints between neighbours (ties to even), random floats over the whole range,
    # the subnormal range and the overflow threshold 65520
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2
    rng = np.random.default_rng(0)
    xs = np.concatenate([h, mids, -mids, rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                         np.array([65504, 65519.99, 65520, 1e6, -1e9, 2.0 ** -25, 2.0 ** -24 * 1.5, 0.0, -0.0])]
                        ).astype(np.float32)
    got = np.array([oracle.f16_from(float(x)) for x in xs], np.uint16)
    with np.errstate(over="ignore"):  # the values past 65520 round to infinity on purpose
        want = xs.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    assert oracle.f16_from(float("nan")) & 0x7c00 == 0x7c00 and oracle.f16_from(float("nan")) & 0x3ff


def test_f16_bf16_matrix_widening(oracle):
    """or_dequant of F16 / BF16 matrices (the reference widens them to f32 at upload, weights.js:127-133): every
    one of the 65536 bit patterns of each.  F16 against numpy's float16; BF16 against the value its fields define,
    computed in float64 (sign, 8-bit exponent with bias 127, 7-bit fraction, subnormals at 2^-126, all-ones
    exponent inf / NaN), plus known answers."""
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.dequant(oracle.F16, h.view(np.uint8), 65536)
    ref = h.view(np.float16).astype(np.float32)
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(got.view(np.uint32)[fin], ref.view(np.uint32)[fin])
    assert np.isnan(got[~fin]).all()
    with np.errstate(invalid="ignore"):  # signalling NaN patterns
        got = oracle.dequant(oracle.BF16, h.view(np.uint8), 65536).astype(np.float64)
    s, e, f = (h >> 15).astype(np.float64), ((h >> 7) & 255).astype(np.int64), (h & 127).astype(np.float64)
    mag = np.where(e == 0, np.ldexp(f / 128.0, -126), np.ldexp(1.0 + f / 128.0, (e - 127).clip(-200, 200)))
    mag = np.where(e == 255, np.where(f == 0, np.inf, np.nan), mag)
    want = np.where(s == 1, -mag, mag)
    fin = ~np.isnan(want)
    np.testing.assert_array_equal(got[fin], want[fin])
    assert np.isnan(got[~fin]).all()
    kat = np.array([0x3F80, 0xC000, 0x4049, 0x0001, 0x7F80, 0x8000], np.uint16)
    np.testing.assert_array_equal(oracle.dequant(oracle.BF16, kat.view(np.uint8), 6),
                                  np.array([1.0, -2.0, 3.140625, 2.0 ** -133, np.inf, -0.0], np.float32))


@pytest.mark.parametrize("fmt,n", [(refs.Q2_K, 256 * 300), (refs.Q3_K, 256 * 300), (refs.Q4_K, 256 * 300),
                                   (refs.Q5_K, 256 * 300), (refs.Q6_K, 256 * 300), (refs.Q8_0, 32 * 500),
                                   (refs.IQ4_NL, 32 * 500)])
@pytest.mark.parametrize("centered", [False, True])
def test_dequant_bit_exact_vs_ggml_spec(oracle, fmt, n, centered):
    raw = blocks(fmt, n, 1, centered)
    got = oracle.dequant(fmt, raw, n)
    ref = refs.dequant(fmt, raw)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_q4k_known_answer(oracle):
    # d = 1, dmin = 0.5, scale/min of sub-block j = (j + 1, j), quant q at element e: q = e % 16
    sc = np.arange(1, 9, dtype=np.uint8)[None]
    mn = np.arange(0, 8, dtype=np.uint8)[None]
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2:4] = np.array([0.5], np.float16).view(np.uint8)
    b[4:16] = synth.pack_q4k_scales(sc, mn)[0]
    q = np.arange(256) % 16
    for g in range(4):  # low nibble -> sub-block 2g, high nibble -> 2g+1
        lo, hi = q[g * 64:g * 64 + 32], q[g * 64 + 32:g * 64 + 64]
        b[16 + g * 32:16 + g * 32 + 32] = (lo | (hi << 4)).astype(np.uint8)
    got = oracle.dequant(refs.Q4_K, b, 256)
    j = np.arange(256) // 32
    np.testing.assert_array_equal(got, (j + 1) * q - 0.5 * j)


def test_q5k_known_answer(oracle):
    # the Q4_K case above with a fifth bit: h = 1 for elements e with (e // 3) odd, so q5 = e % 16 + 16 h and the
    # value is (j + 1) * q5 - 0.5 j; bit j of qh[l] holds h of element 32 j + l
    sc = np.arange(1, 9, dtype=np.uint8)[None]
    mn = np.arange(0, 8, dtype=np.uint8)[None]
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2:4] = np.array([0.5], np.float16).view(np.uint8)
    b[4:16] = synth.pack_q4k_scales(sc, mn)[0]
    e = np.arange(256)
    q, h, j, l = e % 16, (e // 3) % 2, e // 32, e % 32
    for i in range(256):
        b[16 + l[i]] |= h[i] << j[i]
    for g in range(4):
        lo, hi = q[g * 64:g * 64 + 32], q[g * 64 + 32:g * 64 + 64]
        b[48 + g * 32:48 + g * 32 + 32] = (lo | (hi << 4)).astype(np.uint8)
    got = oracle.dequant(refs.Q5_K, b, 256)
    np.testing.assert_array_equal(got, (j + 1) * (q + 16 * h) - 0.5 * j)


def test_q3k_known_answer(oracle):
    # d = 0.5; 6-bit scale of group s: v_s = (7 s + 5) % 64 (value v_s - 32, negative for some groups), packed as
    # ggml does (low nibbles of groups 0..7 / high nibbles of 8..15 in bytes 0..7, the top 2 bits of group 4g + k
    # at bits 2g of byte 8 + k); element e = 128 n + 32 jj + l: q2 = e % 4, hmask bit h = (e // 5) % 2, so the
    # value is 0.5 (v_s - 32) (q2 - 4 (1 - h))
    v = (7 * np.arange(16) + 5) % 64
    b = np.zeros(110, np.uint8)
    for i in range(8):
        b[96 + i] = (v[i] & 15) | ((v[i + 8] & 15) << 4)
    for g in range(4):
        for k in range(4):
            b[104 + k] |= ((v[4 * g + k] >> 4) & 3) << (2 * g)
    b[108:110] = np.array([0.5], np.float16).view(np.uint8)
    e = np.arange(256)
    n, jj, l = e // 128, (e % 128) // 32, e % 32
    q2, h = e % 4, (e // 5) % 2
    for i in range(256):
        b[32 + 32 * n[i] + l[i]] |= q2[i] << (2 * jj[i])
        b[l[i]] |= h[i] << (4 * n[i] + jj[i])
    want = 0.5 * (v[e // 16] - 32) * (q2 - 4 * (1 - h))
    np.testing.assert_array_equal(oracle.dequant(refs.Q3_K, b, 256), want.astype(np.float32))


def test_q2k_known_answer(oracle):
    # d = 1, dmin = 0.5; group j: scale j % 16, min (3 j) % 16; q = e % 4: value = (j % 16) q - 0.5 ((3 j) % 16)
    b = np.zeros(84, np.uint8)
    j = np.arange(16)
    b[0:16] = (j % 16) | (((3 * j) % 16) << 4)
    e = np.arange(256)
    n, jj, l, q = e // 128, (e % 128) // 32, e % 32, e % 4
    for i in range(256):
        b[16 + 32 * n[i] + l[i]] |= q[i] << (2 * jj[i])
    b[80:82] = np.array([1.0], np.float16).view(np.uint8)
    b[82:84] = np.array([0.5], np.float16).view(np.uint8)
    g = e // 16
    want = (g % 16) * q - 0.5 * ((3 * g) % 16)
    np.testing.assert_array_equal(oracle.dequant(refs.Q2_K, b, 256), want.astype(np.float32))


def test_q6k_known_answer(oracle):
    # d = 1, all scales 1: value = q - 32 with q the 6-bit quant (low 4 bits in ql, high 2 in qh)
    q = (np.arange(256) * 7) % 64
    b = np.zeros(210, np.uint8)
    for n in range(2):
        for k in range(4):
            for l in range(32):
                v = int(q[n * 128 + k * 32 + l])
                lo, hi = v & 15, v >> 4
                qli = n * 64 + (k & 1) * 32 + l
                b[qli] |= lo << (4 * (k >> 1))
                b[128 + n * 32 + l] |= hi << (2 * k)
    b[192:208] = 1
    b[208:210] = np.array([1.0], np.float16).view(np.uint8)
    np.testing.assert_array_equal(oracle.dequant(refs.Q6_K, b, 256), q - 32.0)


def test_q8_known_answer(oracle):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([0.25], np.float16).view(np.uint8)
    b[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    np.testing.assert_array_equal(oracle.dequant(refs.Q8_0, b, 32), np.arange(-16, 16) * 0.25)


def test_iq4nl_known_answer(oracle):
    # d = 0.5; byte l holds index l (weight l) and 15 - l (weight 16 + l): the table in order, then reversed
    table = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([0.5], np.float16).view(np.uint8)
    b[2:] = np.arange(16, dtype=np.uint8) | ((15 - np.arange(16, dtype=np.uint8)) << 4)
    want = np.array(table + table[::-1], np.float32) * 0.5
    np.testing.assert_array_equal(oracle.dequant(refs.IQ4_NL, b, 32), want)


# ------------------------------------------------------------------------------------------------ matmul
@pytest.mark.parametrize("fmt,N,K", [(refs.Q2_K, 13, 512), (refs.Q3_K, 15, 768), (refs.Q4_K, 33, 512),
                                     (refs.Q5_K, 21, 512), (refs.Q6_K, 17, 768),
                                     (refs.Q8_0, 19, 320), (refs.IQ4_NL, 19, 1088), (refs.F32, 9, 96)])
@pytest.mark.parametrize("T,mode", [(1, 0), (3, 0), (9, 1)])
def test_matmul_vs_float64(oracle, fmt, N, K, T, mode):
    rng = np.random.default_rng(5)
    raw = blocks(fmt, N * K, 2) if fmt != refs.F32 else rng.standard_normal(N * K).astype(np.float32).view(np.uint8)
    W = refs.dequant(fmt, raw).reshape(N, K).astype(np.float64)
    x = rng.standard_normal((T, K)).astype(np.float32)
    got = oracle.matmul(fmt, raw, N, K, x, T, mode=mode)
    ref = x.astype(np.float64) @ W.T
    bound = 2e-6 * (np.abs(x.astype(np.float64)) @ np.abs(W).T) + 1e-30
    assert np.all(np.abs(got - ref) <= bound)


@pytest.mark.parametrize("fmt,N,K", [(refs.Q2_K, 13, 512), (refs.Q3_K, 6, 256), (refs.Q4_K, 33, 512),
                                     (refs.Q5_K, 7, 256), (refs.Q6_K, 17, 768), (refs.Q8_0, 19, 320),
                                     (refs.F32, 9, 96)])
@pytest.mark.parametrize("T,acc", [(9, 0), (17, 1), (40, 0)])
def test_matmul_serial_order_is_exact(oracle, fmt, N, K, T, acc):
    """The tiled prefill order (mode 1: rows dequantized once, 16 tokens' sums advanced together) gives every
    (token, row) exactly the serial sum c = c + w[k] * x[k] over k = 0..K-1: against numpy float32 arithmetic of
    that definition (each product and sum rounded to float32, weights from the independent numpy dequantizer)
    and against mode 2 (the oracle's one-pair-at-a-time loop), bit for bit, for token counts that are not a
    multiple of 16 and row counts that are not a multiple of 4."""
    rng = np.random.default_rng(7)
    raw = blocks(fmt, N * K, 9) if fmt != refs.F32 else rng.standard_normal(N * K).astype(np.float32).view(np.uint8)
    W = refs.dequant(fmt, raw).reshape(N, K).astype(np.float32)
    x = (rng.standard_normal((T, K)) * 2).astype(np.float32)
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    c = np.zeros((T, N), np.float32)
    for k in range(K):
        c = c + x[:, k:k + 1] * W[None, :, k]
    want = (y0 + c) if acc else c
    got1 = oracle.matmul(fmt, raw, N, K, x, T, y=y0, acc=bool(acc), mode=1)
    got2 = oracle.matmul(fmt, raw, N, K, x, T, y=y0, acc=bool(acc), mode=2)
    np.testing.assert_array_equal(got2, want)
    np.testing.assert_array_equal(got1, want)


def test_matmul_e_serial_order_is_exact(oracle):
    """The grouped expert order (mode 1: each expert's jobs together over its rows dequantized once) equals the
    one-(job, row)-at-a-time serial loop (mode 2) bit for bit, with experts of 0, 1 and 20 jobs."""
    E, N, K, k = 5, 11, 512, 3
    raw = blocks(refs.Q4_K, E * N * K, 6)
    x = np.random.default_rng(3).standard_normal((12, K)).astype(np.float32)
    sel = np.array([(z * 7 + (z // 3)) % 4 for z in range(36)], np.uint32)
    sel[:20] = 2
    sel[35] = 4
    got1 = oracle.matmul_e(refs.Q4_K, raw, N, K, x, sel, tfijo=k, mode=1)
    got2 = oracle.matmul_e(refs.Q4_K, raw, N, K, x, sel, tfijo=k, mode=2)
    np.testing.assert_array_equal(got1, got2)
    W = refs.dequant(refs.Q4_K, raw).reshape(E, N, K).astype(np.float64)
    for z in (0, 25, 35):
        np.testing.assert_allclose(got1[z], W[sel[z]] @ x[z // k], rtol=1e-5, atol=1e-5 * np.abs(W[sel[z]]).sum())


def test_matmul_acc_onehot_zero(oracle):
    N, K = 8, 256
    raw = blocks(refs.Q4_K, N * K, 3)
    W = refs.dequant(refs.Q4_K, raw).reshape(N, K)
    e = np.zeros(K, np.float32)
    e[37] = 1.0
    np.testing.assert_array_equal(oracle.matmul(refs.Q4_K, raw, N, K, e)[0], W[:, 37])
    y0 = np.arange(N, dtype=np.float32)
    got = oracle.matmul(refs.Q4_K, raw, N, K, e, y=y0, acc=True)[0]
    np.testing.assert_array_equal(got, y0 + W[:, 37])
    zero = np.zeros(N * 144, np.uint8)
    assert not np.any(oracle.matmul(refs.Q4_K, zero, N, K, np.ones(K, np.float32)))


def test_matmul_e_selects_expert_rows(oracle):
    E, N, K, k = 6, 8, 256, 2
    raw = blocks(refs.Q4_K, E * N * K, 4)
    W = refs.dequant(refs.Q4_K, raw).reshape(E, N, K).astype(np.float64)
    x = np.random.default_rng(1).standard_normal((1, K)).astype(np.float32)
    sel = np.array([4, 1], np.uint32)
    got = oracle.matmul_e(refs.Q4_K, raw, N, K, x, sel, tfijo=k)
    for z in range(k):
        np.testing.assert_allclose(got[z], W[sel[z]] @ x[0], rtol=2e-6, atol=1e-6 * np.abs(W[sel[z]]).sum())


# ------------------------------------------------------------------------------------------------ elementwise
def test_rmsnorm(oracle):
    x = np.random.default_rng(2).standard_normal((5, 1000)).astype(np.float32) * 3
    w = np.random.default_rng(3).standard_normal(1000).astype(np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-5), refs.rmsnorm64(x, w, 1e-5), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-5, ultima=True)[0], refs.rmsnorm64(x[-1], w, 1e-5),
                               rtol=1e-6, atol=1e-6)


def test_sincos_cody_waite_cephes(oracle):
    for x in np.concatenate([np.linspace(-10, 10, 2001), np.linspace(-4500, 4500, 1001)]):
        s, c = oracle.sincos2(float(np.float32(x)))
        xf = float(np.float32(x))
        assert abs(s - np.sin(xf)) < 2e-6 * max(1.0, abs(xf) / 1000) and abs(c - np.cos(xf)) < 2e-6 * max(1.0, abs(xf) / 1000)


@pytest.mark.parametrize("neox", [0, 1])
@pytest.mark.parametrize("use_norm", [0, 1])
def test_norm_rope(oracle, neox, use_norm):
    nh, hd, T, pos0 = 3, 64, 4, 37
    v = np.random.default_rng(4).standard_normal((T, nh, hd)).astype(np.float32)
    w = (1 + 0.1 * np.random.default_rng(5).standard_normal(hd)).astype(np.float32)
    got = oracle.norm_rope(v, w, nh, hd, use_norm, neox, 1e-6, 10000.0, hd, pos0).reshape(T, nh, hd)
    for t in range(T):
        src = refs.rmsnorm64(v[t], w, 1e-6) if use_norm else v[t]
        np.testing.assert_allclose(got[t], refs.rope64(src, pos0 + t, 10000.0, hd, neox), rtol=2e-5, atol=2e-5)
    # position 0 without the norm is the identity; the rotation preserves each pair's norm
    np.testing.assert_array_equal(oracle.norm_rope(v[:1], w, nh, hd, 0, neox, 1e-6, 1e4, hd, 0).reshape(-1),
                                  v[:1].reshape(-1))
    r = oracle.norm_rope(v, w, nh, hd, 0, neox, 1e-6, 1e4, hd, 123).reshape(T, nh, hd)
    np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(v, axis=-1), rtol=1e-5)


@pytest.mark.parametrize("nh,nkv,T,pos0", [(4, 1, 1, 0), (4, 2, 1, 70), (8, 2, 5, 130), (2, 2, 3, 64)])
def test_attention(oracle, nh, nkv, T, pos0):
    hd, ctx = 64, 256
    rng = np.random.default_rng(6)
    q = rng.standard_normal((T, nh * hd)).astype(np.float32)
    kc = rng.standard_normal((ctx, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((ctx, nkv * hd)).astype(np.float32)
    got = oracle.attention(q, kc, vc, T, pos0, nh, nkv, hd, 0.125)
    np.testing.assert_allclose(got, refs.attention64(q, kc, vc, pos0, nh, nkv, hd, 0.125), rtol=1e-5, atol=1e-5)


def test_attention_closed_forms(oracle):
    hd, nh = 64, 2
    rng = np.random.default_rng(7)
    kc = rng.standard_normal((8, nh * hd)).astype(np.float32)
    vc = rng.standard_normal((8, nh * hd)).astype(np.float32)
    q = rng.standard_normal((1, nh * hd)).astype(np.float32)
    np.testing.assert_allclose(oracle.attention(q, kc, vc, 1, 0, nh, nh, hd, 1.0), vc[:1], rtol=1e-6)  # one key
    z = np.zeros((1, nh * hd), np.float32)
    np.testing.assert_allclose(oracle.attention(z, kc, vc, 1, 7, nh, nh, hd, 1.0)[0], vc.mean(0), rtol=1e-5,
                               atol=1e-6)  # uniform scores


def test_swiglu(oracle):
    g = np.linspace(-30, 30, 301).astype(np.float32)
    u = np.linspace(1, 2, 301).astype(np.float32)
    np.testing.assert_allclose(oracle.swiglu(g, u), refs.silu64(g) * u, rtol=1e-6, atol=1e-30)


def test_geglu_vs_float64(oracle):
    # the tanh-form GELU gate; |a| large enough that the clamp of the tanh argument (at 20) is reached
    rng = np.random.default_rng(31)
    g = np.concatenate([rng.standard_normal(4000) * 3, [-30.0, -9.0, 0.0, 9.0, 30.0]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    got = oracle.geglu(g, u)
    want = refs.gelu_tanh64(g) * u.astype(np.float64)
    # float32 rounding of a (|a| + 1) |u|-sized computation: for large negative a, 1 + tanh(z) cancels, so the
    # bound is absolute in that scale rather than relative to the (tiny) result
    assert np.all(np.abs(got - want) <= 1e-6 * (np.abs(g) + 1.0) * np.abs(u) + 1e-30)
    assert np.all(np.abs(got - want) <= 2e-6 * np.abs(want) + 1e-30 + 1e-6 * np.abs(u) * (g < 0))


def test_escalar_suma_esc(oracle):
    rng = np.random.default_rng(32)
    x, t = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(oracle.escalar(x, 22.627417), x * np.float32(22.627417))
    np.testing.assert_array_equal(oracle.suma_esc(x, t, 0.25), x + np.float32(0.25) * t)


def test_moe_topk(oracle):
    lg = np.array([[0.5, 2.0, 2.0, -1.0, 1.0, 2.0]], np.float32)
    sel, wts = oracle.moe_topk(lg, 6, 3, 1, 2.5)
    assert list(sel) == [1, 2, 5]  # ties go to the lower index
    np.testing.assert_allclose(wts.sum(), 2.5, rtol=1e-6)
    sel, wts = oracle.moe_topk(lg, 6, 2, 0, 1.0)
    r_sel, r_w = refs.topk64(lg[0].astype(np.float64), 2, False, 1.0)
    assert list(sel) == list(r_sel)
    np.testing.assert_allclose(wts, r_w, rtol=1e-6)
    rng = np.random.default_rng(8)
    for _ in range(20):
        lg = rng.standard_normal((1, 128)).astype(np.float32)
        sel, wts = oracle.moe_topk(lg, 128, 8, 1, 1.0)
        r_sel, r_w = refs.topk64(lg[0].astype(np.float64), 8, True, 1.0)
        assert list(sel) == list(r_sel)
        np.testing.assert_allclose(wts, r_w, rtol=1e-5)


def test_moe_comb(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 16)).astype(np.float32)
    de = rng.standard_normal((2 * 3, 16)).astype(np.float32)
    w = rng.random(6).astype(np.float32)
    ref = x.astype(np.float64) + np.einsum("tk,tkd->td", w.reshape(2, 3).astype(np.float64),
                                           de.reshape(2, 3, 16).astype(np.float64))
    np.testing.assert_allclose(oracle.moe_comb(x, de, w, 16, 3), ref, rtol=1e-6, atol=1e-6)


def test_argmax_ties_nan(oracle):
    assert oracle.argmax([1, 3, 3, 2]) == 1
    assert oracle.argmax([np.nan, 1, np.nan, 1]) == 1
    assert oracle.argmax([np.nan, np.nan]) == 0
    assert oracle.argmax([-np.inf, -np.inf]) == 0


# ------------------------------------------------------------------------------------------------ model
@pytest.mark.parametrize("name,neox", [("mini_llama_q4km_c", 0), ("mini_llama_q5km_c", 0), ("mini_llama_q3k_c", 0),
                                       ("mini_llama_q2k_c", 0), ("mini_qwen3_q4km_c", 1),
                                       ("mini_qwen3moe_q5k_c", 1), ("mini_qwen3moe_q4k_c", 1),
                                       ("mini_llama_q8_c", 0), ("mini_llama_iq4nl_c", 0),
                                       ("mini_qwen3moe_iq4nl_c", 1), ("mini_gemma3_q4km_c", 1),
                                       ("mini_llama_f16_c", 0)])
def test_model_forward_vs_float64(oracle, models_dir, name, neox):
    # float32 rounding, amplified by near-ties of the large activations of the centered models, stays below these
    # bounds; a semantic slip (RoPE pairing, norm placement, GQA head map, missing residual) is O(0.1)
    path = synth.ensure_model(name, models_dir)
    m = oracle.Model(path, ctx=64)
    prompt = synth.random_prompt(m.vocab, 12, 3)
    ref = refs.Model64(m.g, neox)
    lg = m.forward(prompt[:9], True)  # T = 9: the tiled (serial) prefill order
    for t in prompt[:9]:
        lr = ref.step(t)
    assert refs.rel_err(lg, lr) < 2e-3
    m2 = oracle.Model(path, ctx=64)
    ref2 = refs.Model64(m2.g, neox)
    for t in prompt:  # T = 1: the lane order
        assert refs.rel_err(m2.forward([t], True), ref2.step(t)) < 2e-4


def test_gemma3_windows_vs_float64(oracle, models_dir):
    """Gemma 3 over 46 positions (windows of 24 keys on the local layers): a 30-token chunk (the tiled order), then
    16 single tokens, each against the float64 model.  The float64 model without windows disagrees (the test would
    catch a window that is ignored or off by one position)."""
    path = synth.ensure_model("mini_gemma3_q4km_c", models_dir)
    m = oracle.Model(path, ctx=128)
    prompt = synth.random_prompt(m.vocab, 46, 8)
    ref, nowin = refs.Model64(m.g, 1), refs.Model64(m.g, 1)
    nowin.window = [0] * nowin.L
    lg = m.forward(prompt[:30], True)
    for t in prompt[:30]:
        lr, ln = ref.step(t), nowin.step(t)
    assert refs.rel_err(lg, lr) < 2e-3
    assert refs.rel_err(lr, ln) > 1e-2
    for t in prompt[30:]:
        assert refs.rel_err(m.forward([t], True), ref.step(t)) < 2e-4


@pytest.mark.parametrize("name,neox", [("mini_llama_q4km_c", 0), ("mini_qwen3moe_q4k_c", 1)])
def test_model_kv_f16_vs_float64(oracle, models_dir, name, neox):
    """The f16 KV-cache option: cache rows rounded to half precision when written."""
    path = synth.ensure_model(name, models_dir)
    m = oracle.Model(path, ctx=64, kv_f16=True)
    ref = refs.Model64(m.g, neox, kv_f16=True)
    ref32 = refs.Model64(m.g, neox)
    prompt = synth.random_prompt(m.vocab, 8, 4)
    differs = False
    for t in prompt:
        lg, lr, l32 = m.forward([t], True), ref.step(t), ref32.step(t)
        assert refs.rel_err(lg, lr) < 2e-4
        differs |= refs.rel_err(lg, l32) > 1e-5  # the rounding is really applied
    assert differs


def test_model_context_overflow(oracle, models_dir):
    m = oracle.Model(synth.ensure_model("mini_llama_q8", models_dir), ctx=8)
    m.forward(list(range(8)), False)
    with pytest.raises(RuntimeError):
        m.forward([1], True)


# ------------------------------------------------------------------------------------------------ GGUF
def test_gguf_roundtrip(oracle, models_dir):
    c = synth.CONFIGS["mini_qwen3moe_q4k"]
    g = oracle.GGUF(synth.ensure_model("mini_qwen3moe_q4k", models_dir))
    plan = synth.tensor_plan(c)
    assert g.order == [p[0] for p in plan]
    for name, dims, gtype, _ in plan:
        t = g.tensors[name]
        assert t["dims"] == dims and t["tipo"] == gtype
        assert t["bytes"] == synth.tensor_nbytes(dims, gtype)
        assert t["abs"] % 32 == 0
    assert g.kv["general.architecture"] == "qwen3moe"
    assert g.kv["qwen3moe.expert_count"] == 16 and g.kv["qwen3moe.expert_weights_norm"] is True
    assert len(g.kv["tokenizer.ggml.tokens"]) == c.vocab


def test_resume_from_reference_cache_is_bit_exact(oracle, models_dir):
    """resume_from_reference (the entry the long-context GPU check uses): a run that prefills P - 1 tokens, then
    takes token P - 1 and 8 greedy steps one token at a time (f16 cache), and a second model given the first run's
    own cache rows and resumed at position P - 1, must produce the same logits bit for bit and the same ids.  The
    resumed model really reads the rows it was given: the value rows of the positions before P - 1 scaled by 1.5
    give other logits."""
    path = synth.ensure_model("mini_llama_q4km_c", models_dir)
    P, n = 40, 8
    a = oracle.Model(path, ctx=64, kv_f16=True)
    prompt = synth.random_prompt(a.vocab, P, 5)
    a.forward(prompt[:-1], False)
    lg = a.forward([prompt[-1]], True)
    want_lg, want_ids = [lg], []
    for i in range(n):
        want_ids.append(oracle.argmax(lg))
        if i + 1 < n:
            lg = a.forward([want_ids[-1]], True)
            want_lg.append(lg)
    k16, v16 = a.kv_cache_f16(P + n - 1)
    a.close()

    def resumed(k, v):
        b = oracle.Model(path, ctx=64, kv_f16=True)
        b.set_kv_reference(k, v)
        b.resume_from_reference(P - 1)
        assert b.pos == P - 1
        lg = b.forward([prompt[-1]], True)
        lgs, ids = [lg], []
        for i in range(n):
            ids.append(oracle.argmax(lg))
            if i + 1 < n:
                lg = b.forward([ids[-1]], True)
                lgs.append(lg)
        b.close()
        return lgs, ids

    got_lg, got_ids = resumed(k16, v16)
    assert got_ids == want_ids
    for g, w in zip(got_lg, want_lg):
        np.testing.assert_array_equal(g.view(np.uint32), w.view(np.uint32))
    v2 = v16.copy()
    v2[:, :P - 1] = (v2[:, :P - 1].view(np.float16) * np.float16(1.5)).view(np.uint16)
    other, _ = resumed(k16, v2)
    assert not np.array_equal(other[0], want_lg[0])
