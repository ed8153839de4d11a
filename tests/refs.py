"""Independent references used to pin the CPU oracle (and through it the GPU kernels).

Nothing here shares code with oracle/qp_oracle.c:
* dequantization is written from the public ggml block layouts (the loop structure of ggml's dequantize_row_q4_K /
  dequantize_row_q6_K / dequantize_row_q8_0: 64-element halves with get_scale_min_k4, 128-element halves with four
  interleaved quarter-lanes), vectorized with numpy;
* everything else is the textbook float64 formula (RMSNorm, RoPE rotation, softmax attention, SiLU, softmax top-k)
  and a float64 forward pass of the decoder.
"""
from __future__ import annotations

import numpy as np

F32, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL = 0, 8, 10, 11, 12, 13, 14, 20


# ------------------------------------------------------------------------------------------------ dequant
def _scale_min_k4(s, j):
    """ggml get_scale_min_k4 for sub-block j (0..7) over an array of 12-byte scale groups s [nb, 12]."""
    if j < 4:
        return s[:, j] & 63, s[:, j + 4] & 63
    sc = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
    mn = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, mn


def dequant_q4k(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 144)
    nb = b.shape[0]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(nb)
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(nb)
    s = b[:, 4:16].astype(np.uint32)
    qs = b[:, 16:144]
    out = np.empty((nb, 256), np.float32)
    for half in range(4):  # 64 elements per step: low nibbles (sub-block 2h) then high nibbles (2h+1)
        q = qs[:, half * 32:(half + 1) * 32]
        sc1, m1 = _scale_min_k4(s, 2 * half)
        sc2, m2 = _scale_min_k4(s, 2 * half + 1)
        d1 = (d * sc1.astype(np.float32)).astype(np.float32)
        mm1 = (dmin * m1.astype(np.float32)).astype(np.float32)
        d2 = (d * sc2.astype(np.float32)).astype(np.float32)
        mm2 = (dmin * m2.astype(np.float32)).astype(np.float32)
        out[:, half * 64:half * 64 + 32] = (d1[:, None] * (q & 0xF).astype(np.float32)) - mm1[:, None]
        out[:, half * 64 + 32:half * 64 + 64] = (d2[:, None] * (q >> 4).astype(np.float32)) - mm2[:, None]
    return out.reshape(-1)


def dequant_q5k(raw: np.ndarray) -> np.ndarray:
    """ggml's dequantize_row_q5_K, vectorized: the Q4_K scheme with a fifth bit per element taken from qh, bit
    2h (low nibbles) / 2h+1 (high nibbles) for the h-th 64-element step."""
    b = raw.reshape(-1, 176)
    nb = b.shape[0]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(nb)
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(nb)
    s = b[:, 4:16].astype(np.uint32)
    qh = b[:, 16:48].astype(np.uint32)
    qs = b[:, 48:176]
    out = np.empty((nb, 256), np.float32)
    for half in range(4):
        q = qs[:, half * 32:(half + 1) * 32].astype(np.uint32)
        sc1, m1 = _scale_min_k4(s, 2 * half)
        sc2, m2 = _scale_min_k4(s, 2 * half + 1)
        d1 = (d * sc1.astype(np.float32)).astype(np.float32)
        mm1 = (dmin * m1.astype(np.float32)).astype(np.float32)
        d2 = (d * sc2.astype(np.float32)).astype(np.float32)
        mm2 = (dmin * m2.astype(np.float32)).astype(np.float32)
        lo = (q & 0xF) + 16 * ((qh >> (2 * half)) & 1)
        hi = (q >> 4) + 16 * ((qh >> (2 * half + 1)) & 1)
        out[:, half * 64:half * 64 + 32] = (d1[:, None] * lo.astype(np.float32)) - mm1[:, None]
        out[:, half * 64 + 32:half * 64 + 64] = (d2[:, None] * hi.astype(np.float32)) - mm2[:, None]
    return out.reshape(-1)


def dequant_q3k(raw: np.ndarray) -> np.ndarray:
    """ggml's dequantize_row_q3_K, vectorized: 16 signed 6-bit scales (low 4 bits from bytes 0..7, high 2 bits
    from bytes 8..11) minus 32; y = d*(scale - 32) * (q2 - (hmask bit set ? 0 : 4)), the hmask bit advancing
    per 32-element step of the 256."""
    b = raw.reshape(-1, 110)
    nb = b.shape[0]
    hm = b[:, 0:32].astype(np.int32)
    qs = b[:, 32:96].astype(np.int32)
    sb = b[:, 96:108].astype(np.int32)
    d = b[:, 108:110].copy().view(np.float16).astype(np.float32).reshape(nb)
    sc = np.empty((nb, 16), np.int32)
    for i in range(16):
        lo = (sb[:, i % 8] >> (4 * (i // 8))) & 0xF          # scales 0..7: low nibbles, 8..15: high nibbles
        hi = (sb[:, 8 + i % 4] >> (2 * (i // 4))) & 3
        sc[:, i] = (lo | (hi << 4)) - 32
    out = np.empty((nb, 256), np.float32)
    for n in range(2):
        for j in range(4):
            for lh in range(2):
                idx = n * 8 + j * 2 + lh
                dl = (d * sc[:, idx].astype(np.float32)).astype(np.float32)
                l = np.arange(16) + 16 * lh
                q = (qs[:, n * 32 + l] >> (2 * j)) & 3
                h = (hm[:, l] >> (4 * n + j)) & 1
                out[:, n * 128 + j * 32 + 16 * lh:n * 128 + j * 32 + 16 * lh + 16] = \
                    dl[:, None] * (q - 4 * (1 - h)).astype(np.float32)
    return out.reshape(-1)


def dequant_q2k(raw: np.ndarray) -> np.ndarray:
    """ggml's dequantize_row_q2_K, vectorized: y = d*(sc & 15) * q - dmin*(sc >> 4), q the 2-bit quant."""
    b = raw.reshape(-1, 84)
    nb = b.shape[0]
    sc = b[:, 0:16].astype(np.int32)
    qs = b[:, 16:80].astype(np.int32)
    d = b[:, 80:82].copy().view(np.float16).astype(np.float32).reshape(nb)
    dmin = b[:, 82:84].copy().view(np.float16).astype(np.float32).reshape(nb)
    out = np.empty((nb, 256), np.float32)
    for n in range(2):
        for j in range(4):
            for lh in range(2):
                idx = n * 8 + j * 2 + lh
                dl = (d * (sc[:, idx] & 0xF).astype(np.float32)).astype(np.float32)
                ml = (dmin * (sc[:, idx] >> 4).astype(np.float32)).astype(np.float32)
                q = (qs[:, n * 32 + 16 * lh:n * 32 + 16 * lh + 16] >> (2 * j)) & 3
                out[:, n * 128 + j * 32 + 16 * lh:n * 128 + j * 32 + 16 * lh + 16] = \
                    dl[:, None] * q.astype(np.float32) - ml[:, None]
    return out.reshape(-1)


def dequant_q6k(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 210)
    nb = b.shape[0]
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32).reshape(nb)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    out = np.empty((nb, 256), np.float32)
    for n in range(2):  # 128-element halves
        ql = b[:, n * 64:(n + 1) * 64].astype(np.int32)
        qh = b[:, 128 + n * 32:128 + (n + 1) * 32].astype(np.int32)
        q1 = ((ql[:, :32] & 0xF) | (((qh >> 0) & 3) << 4)) - 32
        q2 = ((ql[:, 32:] & 0xF) | (((qh >> 2) & 3) << 4)) - 32
        q3 = ((ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4)) - 32
        q4 = ((ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4)) - 32
        for k, q in enumerate((q1, q2, q3, q4)):
            for half in range(2):  # 16 elements share one scale
                is_ = n * 8 + k * 2 + half
                ds = (d * sc[:, is_]).astype(np.float32)
                out[:, n * 128 + k * 32 + half * 16:n * 128 + k * 32 + half * 16 + 16] = \
                    ds[:, None] * q[:, half * 16:half * 16 + 16].astype(np.float32)
    return out.reshape(-1)


def dequant_q8_0(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    return (b[:, 2:].view(np.int8).astype(np.float32) * d).reshape(-1)


# ggml's kvalues_iq4nl (the table of the reference's conversion script tests/conformance/gen_ds.py:104)
_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)


def dequant_iq4_nl(raw: np.ndarray) -> np.ndarray:
    """ggml dequantize_row_iq4_nl: per 18-byte block, y[j] = d * table[qs[j] & 15], y[j + 16] = d * table[qs[j] >> 4]."""
    b = raw.reshape(-1, 18)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:18]
    vals = np.concatenate([_IQ4NL[q & 15], _IQ4NL[q >> 4]], axis=1)
    return (d * vals).astype(np.float32).reshape(-1)


def dequant(fmt, raw):
    raw = np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else np.asarray(raw, np.uint8)
    if fmt == Q4_K:
        return dequant_q4k(raw)
    if fmt == Q5_K:
        return dequant_q5k(raw)
    if fmt == Q3_K:
        return dequant_q3k(raw)
    if fmt == Q2_K:
        return dequant_q2k(raw)
    if fmt == Q6_K:
        return dequant_q6k(raw)
    if fmt == Q8_0:
        return dequant_q8_0(raw)
    if fmt == IQ4_NL:
        return dequant_iq4_nl(raw)
    if fmt == 1:   # F16
        return raw.view(np.float16).astype(np.float32)
    if fmt == 30:  # BF16: the upper half of a float32
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    return raw.view(np.float32).copy()


# ------------------------------------------------------------------------------------------------ float64 ops
def rmsnorm64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def rope64(v, pos, base, nrot, neox):
    """Rotation of a [.., hd] head vector at position pos: pairs (2j, 2j+1) or (j, j + nrot/2)."""
    v = np.asarray(v, np.float64).copy()
    half = nrot // 2
    j = np.arange(half)
    theta = pos * np.power(float(base), -2.0 * j / nrot)
    c, s = np.cos(theta), np.sin(theta)
    if neox:
        a, b = v[..., :half].copy(), v[..., half:nrot].copy()
        v[..., :half] = a * c - b * s
        v[..., half:nrot] = a * s + b * c
    else:
        a, b = v[..., 0:nrot:2].copy(), v[..., 1:nrot:2].copy()
        v[..., 0:nrot:2] = a * c - b * s
        v[..., 1:nrot:2] = a * s + b * c
    return v


def attention64(q, kc, vc, pos0, nh, nkv, hd, scale):
    """Causal GQA softmax attention: query t (at position pos0 + t) over cache rows 0..pos0+t."""
    q = np.asarray(q, np.float64).reshape(-1, nh, hd)
    T = q.shape[0]
    kc = np.asarray(kc, np.float64).reshape(-1, nkv, hd)
    vc = np.asarray(vc, np.float64).reshape(-1, nkv, hd)
    out = np.zeros((T, nh, hd))
    g = nh // nkv
    for t in range(T):
        n = pos0 + t + 1
        for h in range(nh):
            s = kc[:n, h // g] @ q[t, h] * scale
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ vc[:n, h // g]
    return out.reshape(T, nh * hd)


def silu64(g):
    g = np.asarray(g, np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g))


def gelu_tanh64(g):
    """GELU, tanh approximation: 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3)))."""
    g = np.asarray(g, np.float64)
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))


def topk64(logits, k, norm, scale):
    p = np.exp(logits - logits.max())
    p /= p.sum()
    order = sorted(range(len(p)), key=lambda e: (-p[e], e))[:k]  # descending, ties to the lower index
    w = p[order]
    f = scale / max(w.sum(), 2.0 ** -14) if norm else scale
    return np.array(order), w * f


# ------------------------------------------------------------------------------------------------ float64 model
class Model64:
    """Float64 forward of the decoder (pre-norm residual blocks; GQA attention with RoPE; SwiGLU or softmax top-k
    MoE), built from a GGUF through the oracle's header reader and the dequantizers above."""

    def __init__(self, gguf, neox, kv_f16=False):
        self.g = gguf
        self.kv_f16 = kv_f16
        kv = gguf.kv
        a = kv["general.architecture"]
        get = lambda k, d=None: kv.get(f"{a}.{k}", d)
        self.L, self.D = get("block_count"), get("embedding_length")
        self.nh, self.nkv = get("attention.head_count"), get("attention.head_count_kv")
        self.hd = get("attention.key_length", self.D // self.nh)
        self.eps, self.base = get("attention.layer_norm_rms_epsilon", 1e-5), get("rope.freq_base", 10000.0)
        self.nexp, self.k = get("expert_count", 0), get("expert_used_count", 0)
        self.norm_w = bool(get("expert_weights_norm", False))
        self.neox = neox
        self.scale = get("attention.scale", 0) or 1.0 / np.sqrt(self.hd)
        self.emb_scale = get("embedding_scale", 0) or 0
        self.res_scale = get("residual_scale", 0) or 1.0
        self.logit_scale = get("logit_scale", 0) or 0
        self.softcap = get("final_logit_softcapping", 0) or 0
        # Gemma 3: local layers see the last `window` positions (every `pattern`-th layer is global) and rotate with
        # their own base; global layers divide positions by the linear scaling factor; embeddings times sqrt(D);
        # GELU(tanh) gating
        self.gemma = a == "gemma3"
        self.window = [0] * self.L
        self.rbase, self.rpos = [self.base] * self.L, [1.0] * self.L
        if self.gemma:
            w, pat = get("attention.sliding_window", 0) or 0, get("attention.sliding_window_pattern", 6) or 6
            fac = get("rope.scaling.factor", 1.0)
            lin = 1.0 / fac if get("rope.scaling.type", "") == "linear" and fac > 0 else 1.0
            for i in range(self.L):
                local = w > 0 and i % pat != pat - 1
                self.window[i] = w if local else 0
                self.rbase[i] = get("rope.freq_base_swa", 10000.0) if local else self.base
                self.rpos[i] = 1.0 if local else lin
            self.emb_scale = np.sqrt(self.D)
        self.cache = {}
        self.kc = [[] for _ in range(self.L)]
        self.vc = [[] for _ in range(self.L)]

    def W(self, name):
        if name not in self.cache:
            t = self.g.tensors[name]
            m = dequant(t["tipo"], self.g.raw(name)).astype(np.float64)
            self.cache[name] = m.reshape(int(np.prod(t["dims"][1:])), t["dims"][0])
        return self.cache[name]

    def v(self, name):
        return self.g.f32(name).astype(np.float64)

    def step(self, tok):
        """One token through the model at the next position; returns its logits."""
        pos = len(self.kc[0])
        emb = self.W("token_embd.weight")
        x = emb[tok].copy()
        if self.emb_scale:
            x = x * self.emb_scale
        for i in range(self.L):
            p = f"blk.{i}."
            h = rmsnorm64(x, self.v(p + "attn_norm.weight"), self.eps)
            q = (self.W(p + "attn_q.weight") @ h).reshape(self.nh, self.hd)
            k = (self.W(p + "attn_k.weight") @ h).reshape(self.nkv, self.hd)
            v = (self.W(p + "attn_v.weight") @ h).reshape(self.nkv, self.hd)
            if p + "attn_q_norm.weight" in self.g.tensors:
                q = rmsnorm64(q, self.v(p + "attn_q_norm.weight"), self.eps)
                k = rmsnorm64(k, self.v(p + "attn_k_norm.weight"), self.eps)
            q = rope64(q, pos * self.rpos[i], self.rbase[i], self.hd, self.neox)
            k = rope64(k, pos * self.rpos[i], self.rbase[i], self.hd, self.neox)
            if self.kv_f16:  # cache rows stored in half precision (rounded to nearest even from float32)
                k = k.astype(np.float32).astype(np.float16).astype(np.float64)
                v = v.astype(np.float32).astype(np.float16).astype(np.float64)
            self.kc[i].append(k)
            self.vc[i].append(v)
            lo = max(0, pos + 1 - self.window[i]) if self.window[i] else 0
            att = attention64(q.reshape(1, -1), np.array(self.kc[i][lo:]), np.array(self.vc[i][lo:]), pos - lo,
                              self.nh, self.nkv, self.hd, self.scale)[0]
            x = x + self.res_scale * self.post(p + "post_attention_norm.weight", self.W(p + "attn_output.weight") @ att)
            h = rmsnorm64(x, self.v(p + "ffn_norm.weight"), self.eps)
            if self.nexp:
                sel, w = topk64(self.v(p + "ffn_gate_inp.weight").reshape(self.nexp, self.D) @ h, self.k,
                                self.norm_w, 1.0)
                G, U, Dn = self.W(p + "ffn_gate_exps.weight"), self.W(p + "ffn_up_exps.weight"), \
                    self.W(p + "ffn_down_exps.weight")
                ffe = G.shape[0] // self.nexp
                for e, we in zip(sel, w):
                    gg = G[e * ffe:(e + 1) * ffe] @ h
                    uu = U[e * ffe:(e + 1) * ffe] @ h
                    x = x + we * (Dn[e * self.D:(e + 1) * self.D] @ (silu64(gg) * uu))
            else:
                gg = self.W(p + "ffn_gate.weight") @ h
                uu = self.W(p + "ffn_up.weight") @ h
                act = gelu_tanh64(gg) if self.gemma else silu64(gg)
                x = x + self.res_scale * self.post(p + "post_ffw_norm.weight", self.W(p + "ffn_down.weight") @ (act * uu))
        h = rmsnorm64(x, self.v("output_norm.weight"), self.eps)
        out = "output.weight" if "output.weight" in self.g.tensors else "token_embd.weight"
        lg = self.W(out) @ h
        if self.logit_scale:
            lg = lg / self.logit_scale
        if self.softcap:
            lg = self.softcap * np.tanh(lg / self.softcap)
        return lg

    def post(self, name, y):
        """A block's output before the residual add: RMS-normalized when the model has the post-norm weight."""
        return rmsnorm64(y, self.v(name), self.eps) if name in self.g.tensors else y


def rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def vt_pos(k):
    """Position of slot k (of 32) in a row of the device's f16 value-cache tile."""
    return 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3)


def v_tiled(v, kvd):
    """f16 value cache rows [slots][kvd] -> the device tile layout: tiles of 32 slots, each [kvd][32] with slot k
    at vt_pos(k) (slots past the last row are zero)."""
    v = np.asarray(v).reshape(-1, kvd)
    nt = (v.shape[0] + 31) // 32
    pad = np.zeros((nt * 32, kvd), v.dtype)
    pad[:v.shape[0]] = v
    out = np.zeros((nt, kvd, 32), v.dtype)
    out[:, :, [vt_pos(k) for k in range(32)]] = pad.reshape(nt, 32, kvd).transpose(0, 2, 1)
    return out


def v_rows(tiled, rows, kvd):
    """Inverse of v_tiled: rows [rows][kvd]."""
    t = np.asarray(tiled).reshape(-1, kvd, 32)[:, :, [vt_pos(k) for k in range(32)]]
    return t.transpose(0, 2, 1).reshape(-1, kvd)[:rows]


def read_kv_f16(path, n_layers, ctx, kvd, npos):
    """The f16 KV cache that `cli.js generate --kv-out` wrote (per layer: K rows [ctx][kvd], then the V cache in
    32-slot tiles), as uint16 [n_layers][npos][kvd] arrays of K and V rows."""
    raw = np.memmap(path, np.uint16, "r")
    kn, vn = ctx * kvd, -(-ctx // 32) * 32 * kvd
    assert raw.size == n_layers * (kn + vn), (raw.size, n_layers, kn, vn)
    ks = np.empty((n_layers, npos, kvd), np.uint16)
    vs = np.empty((n_layers, npos, kvd), np.uint16)
    nt = -(-npos // 32)
    for i in range(n_layers):
        base = i * (kn + vn)
        ks[i] = raw[base:base + kn].reshape(ctx, kvd)[:npos]
        vs[i] = v_rows(raw[base + kn:base + kn + nt * 32 * kvd], npos, kvd)
    return ks, vs
