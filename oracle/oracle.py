"""Python face of the CPU restatement (qp_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker.  The product (quipullm_amd/) never imports it.

It also carries a GGUF v2/v3 reader written from the public GGUF layout; it restates what quipullm's
`leer_gguf` computes (server.py:404-441: key/values, tensor infos, `bytes` from the block table at
server.py:353-355, `abs = data_start + offset` with `general.alignment`), independently of the product's
JavaScript reader.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL = 0, 8, 10, 11, 12, 13, 14, 20
F16, BF16 = 1, 30  # matrices the reference widens to f32 when it uploads them (weights.js:127-133)
_BLOCKS = {0: (1, 4), 1: (1, 2), 8: (32, 34), 20: (32, 18), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
           14: (256, 210), 30: (1, 2)}
_NAMES = {0: "F32", 1: "F16", 8: "Q8_0", 20: "IQ4_NL", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 30: "BF16"}

_lib = None


def build():
    """Compiles liboracle.so (the checker) with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i, f = C.c_void_p, C.c_int, C.c_float
        L.or_f16.restype = f
        L.or_f16.argtypes = [C.c_uint16]
        L.or_f16_from.restype = C.c_uint16
        L.or_f16_from.argtypes = [f]
        L.or_dequant.argtypes = [i, vp, C.c_int64, vp]
        L.or_matmul.argtypes = [i, vp, i, i, vp, i, vp, i, i]
        L.or_matmul_e.argtypes = [i, vp, i, i, vp, vp, i, i, vp, i]
        L.or_embed.argtypes = [i, vp, i, vp, i, vp]
        L.or_rmsnorm.argtypes = [vp, vp, vp, i, i, f, i]
        L.or_sincos2.argtypes = [f, vp, vp]
        L.or_norm_rope.argtypes = [vp, vp, i, i, i, i, i, f, f, i, f, i]
        L.or_kv_write.argtypes = [vp, vp, vp, vp, i, i, i, i]
        L.or_attention.argtypes = [vp, vp, vp, vp, i, i, i, i, i, f, i, i]
        L.or_swiglu.argtypes = [vp, vp, C.c_int64]
        L.or_geglu.argtypes = [vp, vp, C.c_int64]
        L.or_escalar.argtypes = [vp, C.c_int64, f]
        L.or_suma_esc.argtypes = [vp, vp, C.c_int64, f]
        L.or_moe_topk.argtypes = [vp, i, i, i, i, f, vp, vp]
        L.or_moe_comb.argtypes = [vp, vp, vp, i, i, i]
        L.or_argmax.restype = i
        L.or_argmax.argtypes = [vp, i]
        L.or_model_new.restype = vp
        L.or_model_layers.restype = vp
        L.or_model_layers.argtypes = [vp, i]
        L.or_model_alloc_kv.argtypes = [vp]
        L.or_model_reset.argtypes = [vp]
        L.or_model_pos.argtypes = [vp]
        L.or_model_free.argtypes = [vp]
        L.or_model_forward.argtypes = [vp, vp, i, vp]
        L.or_model_sizeof.restype = C.c_size_t
        L.or_layer_sizeof.restype = C.c_size_t
        L.or_set_threads.argtypes = [i]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------------------------------------ ops
def f16(h: int) -> float:
    return lib().or_f16(h)


def f16_from(x: float) -> int:
    return lib().or_f16_from(x)


def dequant(fmt, raw, nelem):
    raw = np.ascontiguousarray(np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else raw)
    out = np.empty(nelem, np.float32)
    lib().or_dequant(fmt, _p(raw), nelem, _p(out))
    return out


def matmul(fmt, W, N, K, x, T=1, y=None, acc=False, mode=0):
    W = np.ascontiguousarray(W)
    x = _f32(x).reshape(T, K)
    y = np.zeros((T, N), np.float32) if y is None else _f32(y).reshape(T, N).copy()
    lib().or_matmul(fmt, _p(W), N, K, _p(x), T, _p(y), int(acc), mode)
    return y


def matmul_e(fmt, W, N, K, x, sel, tfijo, mode=0):
    W = np.ascontiguousarray(W)
    sel = np.ascontiguousarray(sel, np.uint32)
    x = _f32(x)
    y = np.zeros((len(sel), N), np.float32)
    lib().or_matmul_e(fmt, _p(W), N, K, _p(x), _p(sel), len(sel), tfijo, _p(y), mode)
    return y


def embed(fmt, W, D, ids):
    W = np.ascontiguousarray(W)
    ids = np.ascontiguousarray(ids, np.uint32)
    y = np.empty((len(ids), D), np.float32)
    lib().or_embed(fmt, _p(W), D, _p(ids), len(ids), _p(y))
    return y


def rmsnorm(x, w, eps, ultima=False):
    x = _f32(x)
    T, D = x.shape
    y = np.empty((1 if ultima else T, D), np.float32)
    lib().or_rmsnorm(_p(x), _p(_f32(w)), _p(y), T, D, eps, int(ultima))
    return y


def sincos2(x: float):
    s, c = C.c_float(), C.c_float()
    lib().or_sincos2(x, C.byref(s), C.byref(c))
    return s.value, c.value


def norm_rope(v, w, nh, hd, use_norm, neox, eps, base, nrot, pos0, esc=1.0):
    v = _f32(v).copy()
    T = v.size // (nh * hd)
    w = _f32(w if w is not None else np.ones(hd, np.float32))
    lib().or_norm_rope(_p(v), _p(w), T, nh, hd, int(use_norm), int(neox), eps, base, nrot, esc, pos0)
    return v


def kv_write(k, v, kc, vc, kvd, pos0, cap=0):
    k, v = _f32(k), _f32(v)
    lib().or_kv_write(_p(k), _p(v), _p(kc), _p(vc), k.size // kvd, kvd, pos0, cap)


def attention(q, kc, vc, T, pos0, nh, nkv, hd, scale, swa=0, cap=0):
    q, kc, vc = _f32(q), _f32(kc), _f32(vc)
    o = np.empty((T, nh * hd), np.float32)
    lib().or_attention(_p(q), _p(kc), _p(vc), _p(o), T, pos0, nh, nkv, hd, scale, swa, cap)
    return o


def swiglu(g, u):
    g = _f32(g).copy()
    lib().or_swiglu(_p(g), _p(_f32(u)), g.size)
    return g


def geglu(g, u):
    g = _f32(g).copy()
    lib().or_geglu(_p(g), _p(_f32(u)), g.size)
    return g


def escalar(x, s):
    x = _f32(x).copy()
    lib().or_escalar(_p(x), x.size, s)
    return x


def suma_esc(x, t, s):
    x = _f32(x).copy()
    lib().or_suma_esc(_p(x), _p(_f32(t)), x.size, s)
    return x


def moe_topk(lg, E, k, norm, scale):
    lg = _f32(lg)
    T = lg.size // E
    sel = np.empty(T * k, np.uint32)
    wts = np.empty(T * k, np.float32)
    lib().or_moe_topk(_p(lg), T, E, k, int(norm), scale, _p(sel), _p(wts))
    return sel, wts


def moe_comb(x, de, wts, D, k):
    x = _f32(x).copy()
    T = x.size // D
    lib().or_moe_comb(_p(x), _p(_f32(de)), _p(_f32(wts)), T, D, k)
    return x


def argmax(v) -> int:
    v = _f32(v)
    return lib().or_argmax(_p(v), v.size)


def set_threads(n: int):
    lib().or_set_threads(n)


# ------------------------------------------------------------------------------------------------ GGUF
class GGUF:
    """Header of a GGUF v2+ file plus a read-only memory map of its tensor data."""

    _SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q",
               12: "<d"}

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            if f.read(4) != b"GGUF":
                raise ValueError("not a GGUF file")
            self._f = f
            version = self._u32()
            if version < 2:
                raise ValueError("GGUF version %d not supported" % version)
            nt, nkv = self._u64(), self._u64()
            self.kv = {}
            for _ in range(nkv):
                k = self._str()
                self.kv[k] = self._val(self._u32())
            self.tensors = {}
            order = []
            for _ in range(nt):
                name = self._str()
                nd = self._u32()
                dims = [self._u64() for _ in range(nd)]
                t = self._u32()
                off = self._u64()
                self.tensors[name] = {"dims": dims, "tipo": t, "offset": off}
                order.append(name)
            align = self.kv.get("general.alignment", 32) or 32
            self.data_start = (f.tell() + align - 1) // align * align
        self.order = order
        for t in self.tensors.values():
            n = int(np.prod(t["dims"]))
            epb, bpb = _BLOCKS.get(t["tipo"], (0, 0))
            t["bytes"] = n // epb * bpb if epb else None
            t["tipo_nombre"] = _NAMES.get(t["tipo"], str(t["tipo"]))
            t["abs"] = self.data_start + t["offset"]
        self.mm = np.memmap(path, np.uint8, "r")

    def _u32(self):
        return struct.unpack("<I", self._f.read(4))[0]

    def _u64(self):
        return struct.unpack("<Q", self._f.read(8))[0]

    def _str(self):
        return self._f.read(self._u64()).decode("utf-8", "replace")

    def _val(self, t):
        if t in self._SCALAR:
            fmt = self._SCALAR[t]
            return struct.unpack(fmt, self._f.read(struct.calcsize(fmt)))[0]
        if t == 8:
            return self._str()
        if t == 9:
            sub, n = self._u32(), self._u64()
            return [self._val(sub) for _ in range(n)]
        raise ValueError("unknown GGUF value type %d" % t)

    def raw(self, name):
        t = self.tensors[name]
        return self.mm[t["abs"]:t["abs"] + t["bytes"]]

    def f32(self, name):
        t = self.tensors[name]
        assert t["tipo"] == F32
        return np.frombuffer(self.raw(name), np.float32)


# ------------------------------------------------------------------------------------------------ model
class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("attn_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_norm",
                                          "gate", "up", "down", "router", "gate_e", "up_e", "down_e")] + \
               [(n, C.c_int) for n in ("fq", "fk", "fv", "fo", "fgate", "fup", "fdown", "frouter", "fgate_e",
                                       "fup_e", "fdown_e")] + \
               [("post_att", C.c_void_p), ("post_ffn", C.c_void_p), ("swa", C.c_int), ("rbase", C.c_float),
                ("resc", C.c_float)]


class _Model(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "D", "nh", "nkv", "hd", "F", "vocab", "nrot", "neox", "ctx",
                                       "n_exp", "n_used", "ffe", "moe_norm", "tiled")] + \
               [(n, C.c_float) for n in ("eps", "base", "escala", "moe_scale")] + \
               [("tok_embd", C.c_void_p), ("output", C.c_void_p), ("output_norm", C.c_void_p),
                ("f_embd", C.c_int), ("f_output", C.c_int), ("layers", C.POINTER(_Layer)), ("pos", C.c_int),
                ("kc", C.c_void_p), ("vc", C.c_void_p), ("kv_f16", C.c_int), ("kref", C.c_void_p),
                ("vref", C.c_void_p), ("nref", C.c_int)] + \
               [(n, C.c_float) for n in ("emb_scale", "res_scale", "logit_scale", "softcap")] + [("geglu", C.c_int)]


ROPE_NEOX = {"qwen2", "qwen3", "qwen3moe", "phi3", "gemma", "gemma2", "gemma3", "stablelm", "olmo2"}


class Model:
    """The reference's model forward (transformer.js:252-336; MoE FFN of deepseek2.js:374-386) on the CPU,
    over a GGUF file.  Hyper-parameters are read with the reference's defaults (transformer.js:16-61)."""

    def __init__(self, path, ctx=None, tiled=True, rope=None, kv_f16=False):
        L = lib()
        assert L.or_model_sizeof() == C.sizeof(_Model) and L.or_layer_sizeof() == C.sizeof(_Layer)
        self.g = g = GGUF(path)
        kv = g.kv
        a = kv["general.architecture"]
        get = lambda k, d=None: kv.get(f"{a}.{k}", d)
        self.arch = a
        self.n_layers = get("block_count")
        self.D = get("embedding_length")
        self.nh = get("attention.head_count")
        self.nkv = get("attention.head_count_kv", self.nh)
        self.hd = get("attention.key_length", self.D // self.nh)
        self.eps = get("attention.layer_norm_rms_epsilon", 1e-5)
        self.base = get("rope.freq_base", 10000.0)
        self.nrot = get("rope.dimension_count", self.hd)
        self.neox = (rope == "neox") if rope else (a in ROPE_NEOX)
        self.ctx = ctx or get("context_length", 4096)
        self.n_exp = get("expert_count", 0)
        self.vocab = g.tensors["token_embd.weight"]["dims"][1]
        self._kvref = None
        self.ptr = L.or_model_new()
        m = _Model.from_address(self.ptr)
        m.n_layers, m.D, m.nh, m.nkv, m.hd = self.n_layers, self.D, self.nh, self.nkv, self.hd
        m.vocab, m.nrot, m.neox, m.ctx, m.tiled = self.vocab, self.nrot, int(self.neox), self.ctx, int(tiled)
        m.eps, m.base = self.eps, self.base
        m.kv_f16 = int(kv_f16)
        # scales (transformer.js:35-45): 0 = not set; the attention scale defaults to 1/sqrt(hd)
        m.escala = float(np.float32(get("attention.scale", 0) or 1.0 / np.sqrt(self.hd)))
        m.emb_scale = get("embedding_scale", 0) or 0
        m.res_scale = get("residual_scale", 0) or 0
        m.logit_scale = get("logit_scale", 0) or 0
        m.softcap = get("final_logit_softcapping", 0) or 0
        # gemma3 (transformer.js:46-54): windowed layers (pattern: the last of every `patron` layers is global),
        # their RoPE base, the global layers' linear RoPE scaling, sqrt(D) embedding scale, GeGLU
        self.gemma = a == "gemma3"
        ventana = patron = 0
        base_swa, esc_global = 10000.0, 1.0
        if self.gemma:
            ventana = get("attention.sliding_window", 0) or 0
            patron = get("attention.sliding_window_pattern", 6) or 6
            base_swa = get("rope.freq_base_swa", 10000.0)
            fac = get("rope.scaling.factor", 1.0)
            esc_global = 1.0 / fac if get("rope.scaling.type", "") == "linear" and fac > 0 else 1.0
            m.emb_scale = float(np.float32(np.sqrt(self.D)))
            m.escala = float(np.float32(1.0 / np.sqrt(self.D / self.nh) if self.n_layers == 62 else
                                        1.0 / np.sqrt(self.hd)))
            m.geglu = 1
        self.swa = [ventana if ventana > 0 and (i % patron) < patron - 1 else 0 for i in range(self.n_layers)]
        m.n_exp = self.n_exp
        m.n_used = get("expert_used_count", 0)
        m.ffe = get("expert_feed_forward_length", 0)
        m.moe_norm = int(bool(get("expert_weights_norm", False)))
        m.moe_scale = get("expert_weights_scale", 1.0) or 1.0
        m.F = get("feed_forward_length", 0) or 0
        t = g.tensors
        # F16 / BF16 tensors widened to f32 once, as the reference's loader does at upload (weights.js:127-133)
        self._wide = {}
        for n, ti in t.items():
            if ti["tipo"] in (F16, BF16):
                self._wide[n] = dequant(ti["tipo"], g.raw(n), int(np.prod(ti["dims"])))
        ptr = lambda n: (self._wide[n].ctypes.data if n in self._wide else g.raw(n).ctypes.data) if n in t else None
        tipo = lambda n: F32 if n in self._wide else t[n]["tipo"]
        m.tok_embd, m.f_embd = ptr("token_embd.weight"), tipo("token_embd.weight")
        out = "output.weight" if "output.weight" in t else "token_embd.weight"
        m.output, m.f_output = ptr(out), tipo(out)
        m.output_norm = ptr("output_norm.weight")
        layers = C.cast(L.or_model_layers(self.ptr, self.n_layers), C.POINTER(_Layer))
        for i in range(self.n_layers):
            p = f"blk.{i}."
            ly = layers[i]
            for field, name in (("attn_norm", "attn_norm"), ("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"),
                                ("wo", "attn_output"), ("q_norm", "attn_q_norm"), ("k_norm", "attn_k_norm"),
                                ("ffn_norm", "ffn_norm"), ("gate", "ffn_gate"), ("up", "ffn_up"),
                                ("down", "ffn_down"), ("router", "ffn_gate_inp"), ("gate_e", "ffn_gate_exps"),
                                ("up_e", "ffn_up_exps"), ("down_e", "ffn_down_exps")):
                n = p + name + ".weight"
                setattr(ly, field, ptr(n))
            for field, name in (("fq", "attn_q"), ("fk", "attn_k"), ("fv", "attn_v"), ("fo", "attn_output"),
                                ("fgate", "ffn_gate"), ("fup", "ffn_up"), ("fdown", "ffn_down"),
                                ("frouter", "ffn_gate_inp"), ("fgate_e", "ffn_gate_exps"),
                                ("fup_e", "ffn_up_exps"), ("fdown_e", "ffn_down_exps")):
                n = p + name + ".weight"
                setattr(ly, field, tipo(n) if n in t else 0)
            if self.n_exp == 0 and m.F == 0:
                m.F = t[p + "ffn_gate.weight"]["dims"][1]
            ly.post_att, ly.post_ffn = ptr(p + "post_attention_norm.weight"), ptr(p + "post_ffw_norm.weight")
            ly.swa = self.swa[i]
            ly.rbase = base_swa if self.gemma and self.swa[i] else self.base
            ly.resc = esc_global if self.gemma and not self.swa[i] else 1.0
        if L.or_model_alloc_kv(self.ptr) != 0:
            raise MemoryError("oracle KV cache")
        self.batch = 32

    def set_kv_reference(self, k16, v16):
        """f16 mode: take the cache rows of the first positions from another implementation's f16 cache (k16, v16:
        uint16 [n_layers][npos][nkv * hd]) instead of rounding this model's own k and v."""
        m = _Model.from_address(self.ptr)
        assert m.kv_f16, "set_kv_reference needs kv_f16"
        kvd = self.nkv * self.hd
        k16 = np.ascontiguousarray(k16, np.uint16)
        v16 = np.ascontiguousarray(v16, np.uint16)
        assert k16.shape == v16.shape and k16.ndim == 3 and k16.shape[0] == self.n_layers and k16.shape[2] == kvd
        self._kvref = (k16, v16)
        m.kref, m.vref, m.nref = k16.ctypes.data, v16.ctypes.data, k16.shape[1]

    def resume_from_reference(self, pos):
        """f16 mode: continue from position `pos` of the run whose cache rows set_kv_reference gave, without
        recomputing its first pos tokens: the cache rows of positions 0 .. pos-1 are those rows (f16, widened
        exactly as the cache holds them) and the position moves to pos.  The next forward then computes what that
        run computed at position pos, over the same keys and values (the reference rows also stand in for the
        positions this model writes afterwards, up to their count)."""
        m = _Model.from_address(self.ptr)
        assert m.kv_f16 and self._kvref is not None, "resume_from_reference needs kv_f16 and set_kv_reference"
        k16, v16 = self._kvref
        assert 0 < pos <= k16.shape[1] and pos < self.ctx
        kvd = self.nkv * self.hd
        n = self.n_layers * self.ctx * kvd
        for ptr, r in ((m.kc, k16), (m.vc, v16)):
            a = np.ctypeslib.as_array((C.c_float * n).from_address(ptr)).reshape(self.n_layers, self.ctx, kvd)
            for li in range(self.n_layers):
                a[li, :pos] = dequant(F16, np.ascontiguousarray(r[li, :pos]).view(np.uint8), pos * kvd).reshape(pos, kvd)
        m.pos = pos

    def kv_cache_f16(self, npos):
        """f16 mode: this model's own cache rows of positions 0 .. npos-1 as f16 bits, uint16 [n_layers][npos][kvd]
        each for K and V (the layout set_kv_reference takes)."""
        m = _Model.from_address(self.ptr)
        assert m.kv_f16 and 0 < npos <= self.ctx
        kvd = self.nkv * self.hd
        n = self.n_layers * self.ctx * kvd
        out = []
        for ptr in (m.kc, m.vc):
            a = np.ctypeslib.as_array((C.c_float * n).from_address(ptr)).reshape(self.n_layers, self.ctx, kvd)
            out.append(a[:, :npos].astype(np.float16).view(np.uint16).copy())
        return out[0], out[1]

    def fill_cache_to(self, npos):
        """For timing only: copies the cached rows of positions 0 .. pos-1 over positions pos .. npos-1 and moves the
        position to npos, so the next forward does the arithmetic of a decode step at KV length npos (without a
        prefill of npos tokens, which would take the checker minutes)."""
        m = _Model.from_address(self.ptr)
        kvd, p = self.nkv * self.hd, m.pos
        assert 0 < p <= npos < self.ctx
        n = self.n_layers * self.ctx * kvd
        for ptr in (m.kc, m.vc):
            a = np.ctypeslib.as_array((C.c_float * n).from_address(ptr)).reshape(self.n_layers, self.ctx, kvd)
            for q in range(p, npos, p):
                a[:, q:min(q + p, npos)] = a[:, :min(p, npos - q)]
        m.pos = npos

    def reset(self):
        lib().or_model_reset(self.ptr)

    @property
    def pos(self):
        return lib().or_model_pos(self.ptr)

    def forward(self, ids, want_logits=True):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.vocab, np.float32) if want_logits else None
        rc = lib().or_model_forward(self.ptr, _p(ids), len(ids), _p(out) if want_logits else None)
        if rc != 0:
            raise RuntimeError("oracle forward: invalid batch or context exceeded")
        return out

    def generate(self, prompt, n, batch=None):
        """Greedy continuation as engine.js:generar does it (prefill in chunks of `batch`, then one token per
        forward).  Returns (ids, list of logits per generated step)."""
        batch = batch or self.batch
        self.reset()
        logits = None
        for i in range(0, len(prompt), batch):
            chunk = prompt[i:i + batch]
            logits = self.forward(chunk, i + batch >= len(prompt))
        out, all_logits = [], []
        while len(out) < n:
            t = argmax(logits)
            out.append(t)
            all_logits.append(logits)
            if len(out) >= n:
                break
            logits = self.forward([t], True)
        return out, all_logits

    def close(self):
        if self.ptr:
            lib().or_model_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
