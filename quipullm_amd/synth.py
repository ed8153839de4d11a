"""Seeded synthetic GGUF writer for the benchmark and test configurations.

The files are ordinary GGUF v3 (the format that quipullm's loader reads: server.py:404-441 parses the header,
web/js/weights.js:96-139 consumes the tensors).  Weight blocks are filled straight from the distributions
the configurations specify, so no quantizer is needed:

* Q8_0 (34 B blocks): int8 quants uniform in [-127, 127]; f16 scale |N(0, 0.02)| / 127.
* Q4_K (144 B): d and dmin f16 |N(0, 0.01)|; the 12 packed bytes of 6-bit scales/mins uniform (every byte
  pattern decodes to 6-bit values, each uniform on 0..63); 4-bit quants uniform 0..15.
* Q5_K (176 B): the Q4_K header distributions; qh and qs bytes uniform (5-bit quants uniform 0..31).
* Q3_K (110 B): hmask, 2-bit quants and the 12 packed 6-bit scale bytes uniform; d f16 |N(0, 0.01)|.
* Q2_K (84 B): 4-bit scale/min nibbles and 2-bit quants uniform; d and dmin f16 |N(0, 0.01)| (centered: mins
  equal to scales and dmin = 1.5 d, the mean quant).
* Q6_K (210 B): 6-bit quants uniform 0..63 (ql/qh bytes uniform); int8 sub-scales uniform in [-64, 63];
  d f16 |N(0, 0.01)|.
* F32 vectors (norms, f32 embeddings): N(1, 0.02); the f32 MoE router: N(0, 0.02).
* F16 / BF16 matrices: N(0, wstd) (0.02 when unset) rounded to the nearest half / bfloat16 (ties to even);
  F16 embeddings of a centered model N(0, 1).

Test variants marked `centered` make the weights zero-mean, so that greedy decoding does not collapse onto
one token: Q4_K blocks get mins equal to their scales and dmin = f16(7.5 d) (the mean nibble is 7.5; Q5_K: 15.5), and
f32 embeddings are N(0, 1).

Every tensor draws from its own generator seeded by (seed, tensor index), so a tensor's bytes do not depend on
how many tensors precede it in generation order.  Tensors are streamed to disk one at a time.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field

import numpy as np

GGML_F32, GGML_Q8_0, GGML_Q2_K, GGML_Q3_K, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 0, 8, 10, 11, 12, 13, 14
GGML_IQ4_NL = 20
GGML_F16, GGML_BF16 = 1, 30
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_BF16: (1, 2), GGML_Q8_0: (32, 34), GGML_Q2_K: (256, 84), GGML_Q3_K: (256, 110), GGML_Q4_K: (256, 144),
         GGML_Q5_K: (256, 176), GGML_Q6_K: (256, 210), GGML_IQ4_NL: (32, 18)}
ALIGN = 32

# GGUF metadata value types
_U32, _I32, _F32, _BOOL, _STR, _ARR, _U64 = 4, 5, 6, 7, 8, 9, 10


@dataclass
class ModelConfig:
    name: str
    arch: str                 # general.architecture: "llama", "qwen3" or "qwen3moe"
    n_layers: int
    D: int
    nh: int
    nkv: int
    hd: int
    F: int                    # dense FFN width (0 for MoE)
    vocab: int
    eps: float = 1e-5
    base: float = 10000.0
    fmt: dict = field(default_factory=dict)   # tensor kind -> ggml type
    n_exp: int = 0
    n_used: int = 0
    ffe: int = 0
    qk_norm: bool = False
    ctx: int = 4096
    centered: bool = False    # zero-mean weights (test variants; see gen_blocks)
    wstd: float = 0.0         # > 0: K-quant block scales drawn so the weights' standard deviation is about wstd
    flat_d: bool = False      # centered Q4_K: one d for every block (rows of nearly equal norm; see gen_blocks)
    post_norms: bool = False  # post_attention_norm / post_ffw_norm per layer (gemma3)
    extra_kv: tuple = ()      # further (key after "<arch>.", gguf value type, value) entries

    def tensor_type(self, kind: str) -> int:
        return self.fmt.get(kind, self.fmt.get("default", GGML_Q4_K))


def _q5km():
    """Q5_K_M: Q5_K for most tensors, Q6_K for attn_v, ffn_down and output."""
    return {"default": GGML_Q5_K, "attn_v": GGML_Q6_K, "ffn_down": GGML_Q6_K, "output": GGML_Q6_K}


def _q4km(**kw):
    """Q4_K_M: Q4_K for most tensors, Q6_K for attn_v, ffn_down and output."""
    f = {"default": GGML_Q4_K, "attn_v": GGML_Q6_K, "ffn_down": GGML_Q6_K, "output": GGML_Q6_K}
    f.update(kw)
    return f


CONFIGS = {
    # tiny LLaMA, Q8_0 weights, f32 embeddings and norms
    "tiny_q8": ModelConfig("tiny_q8", "llama", 8, 1024, 16, 16, 64, 2816, 32000, 1e-5, 10000.0,
                           {"default": GGML_Q8_0, "token_embd": GGML_F32}),
    # Llama-3-8B shape, Q4_K_M
    "llama8b_q4km": ModelConfig("llama8b_q4km", "llama", 32, 4096, 32, 8, 128, 14336, 128256, 1e-5, 500000.0,
                                _q4km()),
    # the same shape in Q5_K_M (Q5_K, with Q6_K for attn_v, ffn_down and output)
    "llama8b_q5km": ModelConfig("llama8b_q5km", "llama", 32, 4096, 32, 8, 128, 14336, 128256, 1e-5, 500000.0,
                                _q5km()),
    # Qwen3-30B-A3B-like MoE, Q4_K everywhere except the f32 router
    "qwen3moe_q4k": ModelConfig("qwen3moe_q4k", "qwen3moe", 48, 2048, 32, 4, 128, 0, 151936, 1e-6, 1000000.0,
                                {"default": GGML_Q4_K}, n_exp=128, n_used=8, ffe=768, qk_norm=True),
    # the configs' shapes in depth the CPU checker can follow through long prompts, centered (varied greedy ids)
    # and with weights of standard deviation 0.02 (about 1/sqrt(hidden)), so activations and attention scores stay
    # of the order of a real model's: the 8B shape in 2 layers (ctx 4096 parity, the 2048-token prefill) and the MoE
    # shape in 4 layers
    "llama8b_q4km_c2": ModelConfig("llama8b_q4km_c2", "llama", 2, 4096, 32, 8, 128, 14336, 128256, 1e-5, 500000.0,
                                   _q4km(), ctx=4400, centered=True, wstd=0.02),
    # the 8B shape at full depth, centered with weights of standard deviation 0.02: the timed decode path (f16 KV at
    # ctx 4096) checked end to end with varied greedy ids, and the full-depth fixture at ctx 512
    "llama8b_q4km_c": ModelConfig("llama8b_q4km_c", "llama", 32, 4096, 32, 8, 128, 14336, 128256, 1e-5, 500000.0,
                                  _q4km(), ctx=4400, centered=True, wstd=0.02),
    # the MoE shape at full depth, centered with weights of standard deviation 0.1 (full-depth fixture, after a short
    # prompt: at 0.02 or 0.05 the context-averaged attention outweighs the experts and greedy decoding cycles through
    # a few tokens; after hundreds of prompt tokens the 48 layers amplify rounding and routing near-ties past the
    # 1e-3 logit bar)
    "qwen3moe_q4k_c": ModelConfig("qwen3moe_q4k_c", "qwen3moe", 48, 2048, 32, 4, 128, 0, 151936, 1e-6, 1000000.0,
                                  {"default": GGML_Q4_K}, n_exp=128, n_used=8, ffe=768, qk_norm=True, ctx=2400,
                                  centered=True, wstd=0.1),
    "qwen3moe_q4k_c4": ModelConfig("qwen3moe_q4k_c4", "qwen3moe", 4, 2048, 32, 4, 128, 0, 151936, 1e-6, 1000000.0,
                                   {"default": GGML_Q4_K}, n_exp=128, n_used=8, ffe=768, qk_norm=True, ctx=2400,
                                   centered=True, wstd=0.02),
    # small variants with the same formats, for parity tests
    "mini_llama_q4km": ModelConfig("mini_llama_q4km", "llama", 2, 512, 8, 2, 64, 768, 1000, 1e-5, 500000.0,
                                   _q4km(), ctx=512),
    "mini_llama_q8": ModelConfig("mini_llama_q8", "llama", 2, 256, 4, 4, 64, 704, 800, 1e-5, 10000.0,
                                 {"default": GGML_Q8_0, "token_embd": GGML_F32}, ctx=256),
    "mini_qwen3_q4km": ModelConfig("mini_qwen3_q4km", "qwen3", 2, 512, 8, 2, 128, 768, 1000, 1e-6, 1000000.0,
                                   _q4km(), qk_norm=True, ctx=512),
    "mini_qwen3moe_q4k": ModelConfig("mini_qwen3moe_q4k", "qwen3moe", 2, 512, 8, 2, 128, 0, 1000, 1e-6,
                                     1000000.0, {"default": GGML_Q4_K}, n_exp=16, n_used=4, ffe=256,
                                     qk_norm=True, ctx=512),
    # centered variants (non-degenerate greedy sequences)
    "mini_llama_q4km_c": ModelConfig("mini_llama_q4km_c", "llama", 2, 512, 8, 2, 64, 768, 1000, 1e-5, 500000.0,
                                     _q4km(), ctx=512, centered=True),
    "mini_llama_q8_c": ModelConfig("mini_llama_q8_c", "llama", 2, 256, 4, 4, 64, 704, 800, 1e-5, 10000.0,
                                   {"default": GGML_Q8_0, "token_embd": GGML_F32}, ctx=256, centered=True),
    "mini_qwen3_q4km_c": ModelConfig("mini_qwen3_q4km_c", "qwen3", 2, 512, 8, 2, 128, 768, 1000, 1e-6, 1000000.0,
                                     _q4km(), qk_norm=True, ctx=512, centered=True),
    "mini_llama_q5km_c": ModelConfig("mini_llama_q5km_c", "llama", 2, 512, 8, 2, 64, 768, 1000, 1e-5, 500000.0,
                                     _q5km(), ctx=512, centered=True),
    # Gemma 3 text (reference transformer.js:46-54): windows of 24 keys on the even layers (pattern 2), their RoPE
    # base 1e4 against 1e6 on the odd (global) layers with linear scaling 8, q/k norms, post norms, GeGLU, logit
    # soft-capping 30, sqrt(D) embedding scale
    "mini_gemma3_q4km_c": ModelConfig("mini_gemma3_q4km_c", "gemma3", 4, 512, 8, 2, 64, 768, 1000, 1e-6, 1000000.0,
                                      _q4km(), qk_norm=True, ctx=512, centered=True, post_norms=True,
                                      extra_kv=(("attention.sliding_window", _U32, 24),
                                                ("attention.sliding_window_pattern", _U32, 2),
                                                ("rope.freq_base_swa", _F32, 10000.0),
                                                ("rope.scaling.type", _STR, "linear"),
                                                ("rope.scaling.factor", _F32, 8.0),
                                                ("final_logit_softcapping", _F32, 30.0))),
    # IQ4_NL matrices (the reference loads them for its DeepSeek2 class, weights.js:110-116): dense and MoE
    "mini_llama_iq4nl_c": ModelConfig("mini_llama_iq4nl_c", "llama", 2, 512, 8, 2, 64, 768, 1000, 1e-5, 500000.0,
                                      {"default": GGML_IQ4_NL, "token_embd": GGML_F32}, ctx=512, centered=True),
    "mini_qwen3moe_iq4nl_c": ModelConfig("mini_qwen3moe_iq4nl_c", "qwen3moe", 2, 512, 8, 2, 64, 0, 1000, 1e-6,
                                         1000000.0, {"default": GGML_IQ4_NL, "token_embd": GGML_F32},
                                         n_exp=16, n_used=4, ffe=256,
                                         qk_norm=True, ctx=512, centered=True),
    "mini_llama_q3k_c": ModelConfig("mini_llama_q3k_c", "llama", 2, 512, 8, 2, 64, 768, 1000, 1e-5, 500000.0,
                                    {"default": GGML_Q3_K, "attn_v": GGML_Q5_K, "output": GGML_Q6_K}, ctx=512,
                                    centered=True),
    # F16 and BF16 matrices (the reference widens them to f32 at upload, weights.js:127-133): F16 embeddings, q, k
    # and wo; BF16 v, ffn_down and output; Q4_K gate/up
    "mini_llama_f16_c": ModelConfig("mini_llama_f16_c", "llama", 2, 512, 8, 2, 64, 768, 1000, 1e-5, 500000.0,
                                    {"default": GGML_Q4_K, "token_embd": GGML_F16, "attn_q": GGML_F16,
                                     "attn_k": GGML_F16, "attn_output": GGML_F16, "attn_v": GGML_BF16,
                                     "ffn_down": GGML_BF16, "output": GGML_BF16}, ctx=512, centered=True,
                                    wstd=0.02),
    "mini_llama_q2k_c": ModelConfig("mini_llama_q2k_c", "llama", 2, 512, 8, 2, 64, 768, 1000, 1e-5, 500000.0,
                                    {"default": GGML_Q2_K, "ffn_down": GGML_Q3_K, "output": GGML_Q6_K}, ctx=512,
                                    centered=True),
    "mini_qwen3moe_q5k_c": ModelConfig("mini_qwen3moe_q5k_c", "qwen3moe", 2, 512, 8, 2, 128, 0, 1000, 1e-6,
                                       1000000.0, {"default": GGML_Q5_K}, n_exp=16, n_used=4, ffe=256,
                                       qk_norm=True, ctx=512, centered=True),
    "mini_qwen3moe_q4k_c": ModelConfig("mini_qwen3moe_q4k_c", "qwen3moe", 2, 512, 8, 2, 128, 0, 1000, 1e-6,
                                       1000000.0, {"default": GGML_Q4_K}, n_exp=16, n_used=4, ffe=256,
                                       qk_norm=True, ctx=512, centered=True),
}


def tensor_plan(c: ModelConfig):
    """(name, ggml dims [K, N(, E)], ggml type, kind) in file order."""
    qd, kvd = c.nh * c.hd, c.nkv * c.hd
    out = [("token_embd.weight", [c.D, c.vocab], c.tensor_type("token_embd"), "embd"),
           ("output_norm.weight", [c.D], GGML_F32, "norm"),
           ("output.weight", [c.D, c.vocab], c.tensor_type("output"), "w")]
    for i in range(c.n_layers):
        p = f"blk.{i}."
        out += [(p + "attn_norm.weight", [c.D], GGML_F32, "norm"),
                (p + "attn_q.weight", [c.D, qd], c.tensor_type("attn_q"), "w"),
                (p + "attn_k.weight", [c.D, kvd], c.tensor_type("attn_k"), "w"),
                (p + "attn_v.weight", [c.D, kvd], c.tensor_type("attn_v"), "w"),
                (p + "attn_output.weight", [qd, c.D], c.tensor_type("attn_output"), "w")]
        if c.qk_norm:
            out += [(p + "attn_q_norm.weight", [c.hd], GGML_F32, "norm"),
                    (p + "attn_k_norm.weight", [c.hd], GGML_F32, "norm")]
        out.append((p + "ffn_norm.weight", [c.D], GGML_F32, "norm"))
        if c.n_exp:
            out += [(p + "ffn_gate_inp.weight", [c.D, c.n_exp], GGML_F32, "router"),
                    (p + "ffn_gate_exps.weight", [c.D, c.ffe, c.n_exp], c.tensor_type("ffn_gate_exps"), "w"),
                    (p + "ffn_up_exps.weight", [c.D, c.ffe, c.n_exp], c.tensor_type("ffn_up_exps"), "w"),
                    (p + "ffn_down_exps.weight", [c.ffe, c.D, c.n_exp], c.tensor_type("ffn_down_exps"), "w")]
        else:
            out += [(p + "ffn_gate.weight", [c.D, c.F], c.tensor_type("ffn_gate"), "w"),
                    (p + "ffn_up.weight", [c.D, c.F], c.tensor_type("ffn_up"), "w"),
                    (p + "ffn_down.weight", [c.F, c.D], c.tensor_type("ffn_down"), "w")]
        if c.post_norms:
            out += [(p + "post_attention_norm.weight", [c.D], GGML_F32, "norm"),
                    (p + "post_ffw_norm.weight", [c.D], GGML_F32, "norm")]
    return out


def tensor_nbytes(dims, gtype):
    n = int(np.prod(dims))
    epb, bpb = BLOCK[gtype]
    assert n % epb == 0, (dims, gtype)
    return n // epb * bpb


def _abs_normal_f16(rng, n, sigma):
    return np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(sigma)).astype(np.float16)


def pack_q4k_scales(sc, mn):
    """12-byte 6-bit scale/min packing of Q4_K (inverse of ggml's get_scale_min_k4); sc, mn: [nb, 8] in 0..63."""
    nb = sc.shape[0]
    s = np.zeros((nb, 12), np.uint8)
    for j in range(4):
        s[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        s[:, j + 4] = (mn[:, j] & 63) | ((mn[:, j + 4] >> 4) << 6)
        s[:, j + 8] = (sc[:, j + 4] & 15) | ((mn[:, j + 4] & 15) << 4)
    return s


# Standard deviation of a K-quant weight per unit of the d scale's sigma: Q4_K / Q5_K centered (scale uniform 0..63,
# rms 36.4; q - 7.5 or q - 15.5 with rms 4.6 or 9.2) and Q6_K (int8 scale, rms 36.9; q - 32, rms 18.5).
_STD_PER_SIGMA = {GGML_Q4_K: 36.4 * 4.61, GGML_Q5_K: 36.4 * 9.23, GGML_Q6_K: 36.9 * 18.5}


def gen_blocks(rng, gtype, nelem, kind="w", centered=False, wstd=0.0, flat_d=False):
    """Bytes of one tensor of `nelem` elements.  wstd > 0 (Q4_K, Q5_K centered and Q6_K): the d scales' sigma
    is chosen so that the weights' standard deviation is about wstd, instead of the configs' 0.01.  flat_d
    (centered Q4_K): every block's d is that sigma instead of |N(0, sigma)|, so that the rows' norms vary little
    and no row outweighs the others in every argmax (greedy sequences that wander instead of repeating a few
    tokens)."""
    sig = np.float32(wstd / _STD_PER_SIGMA[gtype]) if wstd > 0 and gtype in _STD_PER_SIGMA else 0.01
    if gtype in (GGML_F16, GGML_BF16):
        sd = np.float32(1.0 if (kind == "embd" and centered) else (wstd or 0.02))
        a = rng.standard_normal(nelem, dtype=np.float32) * sd
        if gtype == GGML_F16:
            return a.astype("<f2").tobytes()
        u = a.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype("<u2").tobytes()
    if gtype == GGML_F32:
        if kind == "embd" and centered:
            a = rng.standard_normal(nelem, dtype=np.float32)
        elif kind == "router":
            a = rng.standard_normal(nelem, dtype=np.float32) * np.float32(0.02)
        else:
            a = np.float32(1.0) + rng.standard_normal(nelem, dtype=np.float32) * np.float32(0.02)
        return a.astype("<f4").tobytes()
    epb, bpb = BLOCK[gtype]
    nb = nelem // epb
    if gtype == GGML_IQ4_NL:
        # f16 scale |N(0, 0.02)| / 127 (the table spans -127 .. 113), random 4-bit indices
        blk = np.empty((nb, 18), np.uint8)
        d = (np.abs(rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)) / np.float32(127.0))
        blk[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
        blk[:, 2:18] = np.frombuffer(rng.bytes(nb * 16), np.uint8).reshape(nb, 16)
        return blk.tobytes()
    if gtype == GGML_Q8_0:
        blk = np.empty((nb, 34), np.uint8)
        d = (np.abs(rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)) / np.float32(127.0))
        blk[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
        q = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8)
        blk[:, 2:34] = q.view(np.uint8)
        return blk.tobytes()
    blk = np.frombuffer(rng.bytes(nb * bpb), np.uint8).reshape(nb, bpb).copy()
    if gtype in (GGML_Q4_K, GGML_Q5_K):
        d = _abs_normal_f16(rng, nb, sig)
        if flat_d and centered:
            d = np.full(nb, sig, np.float32).astype(np.float16)
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        if centered:
            mean = np.float32(7.5 if gtype == GGML_Q4_K else 15.5)
            sc = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
            blk[:, 2:4] = (d.astype(np.float32) * mean).astype(np.float16).view(np.uint8).reshape(nb, 2)
            blk[:, 4:16] = pack_q4k_scales(sc, sc)
        else:
            blk[:, 2:4] = _abs_normal_f16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    elif gtype == GGML_Q3_K:
        blk[:, 108:110] = _abs_normal_f16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    elif gtype == GGML_Q2_K:
        d = _abs_normal_f16(rng, nb, 0.01)
        blk[:, 80:82] = d.view(np.uint8).reshape(nb, 2)
        if centered:
            sc = rng.integers(0, 16, size=(nb, 16), dtype=np.uint8)
            blk[:, 0:16] = sc | (sc << 4)
            blk[:, 82:84] = (d.astype(np.float32) * np.float32(1.5)).astype(np.float16).view(np.uint8).reshape(nb, 2)
        else:
            blk[:, 82:84] = _abs_normal_f16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    elif gtype == GGML_Q6_K:
        blk[:, 192:208] = rng.integers(-64, 64, size=(nb, 16), dtype=np.int8).view(np.uint8)
        blk[:, 208:210] = _abs_normal_f16(rng, nb, sig).view(np.uint8).reshape(nb, 2)
    else:
        raise ValueError(gtype)
    return blk.tobytes()


def _s(b: str) -> bytes:
    e = b.encode("utf-8")
    return struct.pack("<Q", len(e)) + e


def _kv(key, vtype, value) -> bytes:
    out = _s(key) + struct.pack("<I", vtype)
    if vtype == _U32:
        out += struct.pack("<I", value)
    elif vtype == _F32:
        out += struct.pack("<f", value)
    elif vtype == _BOOL:
        out += struct.pack("<?", bool(value))
    elif vtype == _STR:
        out += _s(value)
    elif vtype == _ARR:
        etype, items = value
        out += struct.pack("<IQ", etype, len(items))
        if etype == _STR:
            out += b"".join(_s(x) for x in items)
        elif etype == _I32:
            out += np.asarray(items, "<i4").tobytes()
        else:
            raise ValueError(etype)
    else:
        raise ValueError(vtype)
    return out


def metadata(c: ModelConfig):
    a = c.arch
    kv = [("general.architecture", _STR, a), ("general.name", _STR, "synthetic-" + c.name),
          ("general.alignment", _U32, ALIGN),
          (f"{a}.block_count", _U32, c.n_layers), (f"{a}.context_length", _U32, c.ctx),
          (f"{a}.embedding_length", _U32, c.D),
          (f"{a}.attention.head_count", _U32, c.nh), (f"{a}.attention.head_count_kv", _U32, c.nkv),
          (f"{a}.attention.key_length", _U32, c.hd), (f"{a}.attention.value_length", _U32, c.hd),
          (f"{a}.attention.layer_norm_rms_epsilon", _F32, c.eps), (f"{a}.rope.freq_base", _F32, c.base),
          (f"{a}.rope.dimension_count", _U32, c.hd)]
    if c.n_exp:
        kv += [(f"{a}.expert_count", _U32, c.n_exp), (f"{a}.expert_used_count", _U32, c.n_used),
               (f"{a}.expert_feed_forward_length", _U32, c.ffe), (f"{a}.expert_weights_norm", _BOOL, True)]
    else:
        kv.append((f"{a}.feed_forward_length", _U32, c.F))
    kv += [(f"{a}.{k}", t, v) for k, t, v in c.extra_kv]
    kv += [("tokenizer.ggml.model", _STR, "synthetic"),
           ("tokenizer.ggml.tokens", _ARR, (_STR, [f"<t{i}>" for i in range(c.vocab)])),
           ("tokenizer.ggml.eos_token_id", _U32, c.vocab - 1)]
    return kv


def write_gguf(path: str, c: ModelConfig, seed: int = 0) -> str:
    """Writes the synthetic model `c` to `path` (atomically, via a temporary name) and returns the path."""
    plan = tensor_plan(c)
    kv = metadata(c)
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(plan), len(kv)))
    for k, t, v in kv:
        head += _kv(k, t, v)
    off = 0
    offsets = []
    for name, dims, gtype, _ in plan:
        off = (off + ALIGN - 1) // ALIGN * ALIGN
        offsets.append(off)
        head += _s(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", gtype, off)
        off += tensor_nbytes(dims, gtype)
    pad = (-len(head)) % ALIGN
    head += b"\0" * pad
    tmp = path + ".tmp%d" % os.getpid()
    with open(tmp, "wb") as f:
        f.write(head)
        pos = 0
        for i, ((name, dims, gtype, kind), o) in enumerate(zip(plan, offsets)):
            if o > pos:
                f.write(b"\0" * (o - pos))
                pos = o
            rng = np.random.default_rng([seed, i])
            data = gen_blocks(rng, gtype, int(np.prod(dims)), kind, c.centered, c.wstd, c.flat_d)
            f.write(data)
            pos += len(data)
    os.replace(tmp, path)
    return path


def ensure_model(name: str, directory: str, seed: int = 0) -> str:
    """Path of the synthetic model `name`, written on first use (file name carries the seed)."""
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, f"{name}-s{seed}.gguf")
    if not os.path.exists(path):
        write_gguf(path, CONFIGS[name], seed)
    return path


def random_prompt(vocab: int, n: int, seed: int) -> list:
    """Uniform random token ids in [0, vocab)."""
    return np.random.default_rng([seed, 0x5eed]).integers(0, vocab, size=n).tolist()


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(description="write a seeded synthetic GGUF")
    ap.add_argument("config", choices=sorted(CONFIGS))
    ap.add_argument("out")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--prompt", type=int, default=0, help="also write N uniform-random prompt ids to OUT.prompt.json")
    ap.add_argument("--prompt-seed", type=int, default=7)
    a = ap.parse_args()
    if not os.path.exists(a.out):
        write_gguf(a.out, CONFIGS[a.config], a.seed)
    if a.prompt:
        import json
        with open(a.out + ".prompt.json", "w") as f:
            json.dump(random_prompt(CONFIGS[a.config].vocab, a.prompt, a.prompt_seed), f)
    print(a.out)
