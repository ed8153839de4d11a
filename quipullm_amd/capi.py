"""ctypes binding of include/quipu.h, shaped like quipullm's GPU facade (web/js/gpu.js:1167-1282).

The product host is the JavaScript engine in quipullm_amd/js (through the N-API addon); this module is the
same C ABI seen from Python, for tests, smoke checks and the benchmark.  It loads only the in-tree
libquipu.so and raises if it is missing -- there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import json
import math
import os
import struct

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
# QP_LIB selects another build of the library (the profiling build in lib/timeline/)
LIB_PATH = os.path.abspath(os.environ["QP_LIB"]) if os.environ.get("QP_LIB") else os.path.join(PKG, "lib", "libquipu.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "quipu.h")

F32, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL = 0, 8, 10, 11, 12, 13, 14, 20
BLOCK = {F32: (1, 4), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210), IQ4_NL: (32, 18)}
FMT_NAME = {F32: "f32", Q8_0: "q8", Q2_K: "q2k", Q3_K: "q3k", Q4_K: "q4k", Q5_K: "q5k", Q6_K: "q6k",
            IQ4_NL: "iq4nl"}

# gemv segment modes (qp_args.h)
STORE, ACC, SWIGLU, ARGMAX = 0, 1, 2, 3


class QuipuError(RuntimeError):
    pass


_lib = None


def load_library():
    """The in-tree C ABI; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QuipuError(f"{LIB_PATH} is missing: run __graft_entry__.build() (or python quipullm_amd/build.py)")
        L = C.CDLL(LIB_PATH)
        u64, u32, vp = C.c_uint64, C.c_uint32, C.c_void_p
        L.qp_init.argtypes = [C.c_int]
        L.qp_info.argtypes = [C.c_char_p, C.c_size_t]
        L.qp_last_error.argtypes = [C.c_char_p, C.c_size_t]
        L.qp_bytes_used.restype = u64
        L.qp_alloc.argtypes = [u64, C.POINTER(u64)]
        L.qp_free.argtypes = [u64]
        L.qp_upload.argtypes = [u64, u64, vp, u64]
        L.qp_download.argtypes = [vp, u64, u64, u64]
        L.qp_copy.argtypes = [u64, u64, u64, u64, u64]
        L.qp_op_id.argtypes = [C.c_char_p]
        L.qp_dispatch.argtypes = [C.c_int, vp, u32, vp, u32, u32, u32, u32]
        L.qp_dispatch_noalloc.argtypes = [C.c_int, vp, u32, vp, u32, u32, u32, u32]
        L.qp_module_load.argtypes = [C.c_char_p, C.POINTER(u64)]
        L.qp_kernel.argtypes = [u64, C.c_char_p, C.POINTER(u64)]
        L.qp_launch.argtypes = [u64, vp, vp, u32, vp, u64]
        L.qp_graph_end.argtypes = [C.POINTER(u64)]
        L.qp_graph_launch.argtypes = [u64]
        L.qp_graph_free.argtypes = [u64]
        L.qp_event_create.argtypes = [C.POINTER(u64)]
        L.qp_event_record.argtypes = [u64]
        L.qp_event_elapsed.argtypes = [u64, u64, C.POINTER(C.c_float)]
        L.qp_event_free.argtypes = [u64]
        _lib = L
    return _lib


def declared_symbols():
    """Function names declared in include/quipu.h."""
    import re
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|uint64_t)\s+(qp_\w+)\s*\(", src, re.M)))


def uniform(vals):
    """Packs [(type, value), ...] ('u' = u32, 'f' = f32) into 16-byte-padded bytes, as gpu.uniforme does
    (gpu.js:1248-1256)."""
    n = max(4, (len(vals) + 3) // 4 * 4)
    out = bytearray(4 * n)
    for i, (t, v) in enumerate(vals):
        if t == "f":
            struct.pack_into("<f", out, 4 * i, float(v))
        else:
            struct.pack_into("<I", out, 4 * i, int(v) & 0xFFFFFFFF)
    return bytes(out)


def dim2(n):
    """Splits n workgroups into 2-D under the 65535 limit (gpu.js:1278-1282)."""
    if n <= 65535:
        return (n, 1)
    y = math.ceil(n / 65535)
    return (math.ceil(n / y), y)


def gguf_bytes(fmt, N, K):
    """Packed bytes of an N x K matrix in the GGUF block format (the algorithmic bytes of one pass over it)."""
    epb, bpb = BLOCK[fmt]
    return N * K // epb * bpb


def scale_plane(fmt, h, N, K):
    """Address of the f16 scale plane of the planar device tensor h (Q8_0, IQ4_NL) of N x K weights: after the N*K/32
    blocks' quants (32 bytes each for Q8_0, 16 for IQ4_NL), the second binding of the planar formats' ops."""
    return h + N * K // 32 * (32 if fmt == Q8_0 else 16)


def device_bytes(fmt, N, K):
    """Bytes of the device tensor: the GGUF size, except Q3_K blocks padded to 112 bytes."""
    return N * K // 256 * 112 if fmt == Q3_K else gguf_bytes(fmt, N, K)


class Quipu:
    """One device context (qp_init) with buffer helpers and named-op dispatch."""

    def __init__(self, device=0):
        self.L = load_library()
        self._check(self.L.qp_init(device), "qp_init")
        self._ops = {}

    # -------------------------------------------------------------- errors / info
    def _check(self, rc, what):
        if rc != 0:
            buf = C.create_string_buffer(512)
            self.L.qp_last_error(buf, 512)
            raise QuipuError(f"{what}: {buf.value.decode()} (status {rc})")

    def info(self):
        buf = C.create_string_buffer(1024)
        self._check(self.L.qp_info(buf, 1024), "qp_info")
        return json.loads(buf.value.decode())

    def bytes_used(self):
        return self.L.qp_bytes_used()

    # -------------------------------------------------------------- buffers
    def alloc(self, nbytes):
        h = C.c_uint64()
        self._check(self.L.qp_alloc(int(nbytes), C.byref(h)), "qp_alloc")
        return h.value

    def free(self, h):
        self._check(self.L.qp_free(h), "qp_free")

    def upload(self, h, data, off=0):
        a = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray, memoryview))
                                 else data)
        self._check(self.L.qp_upload(h, off, a.ctypes.data, a.nbytes), "qp_upload")

    def buffer_from(self, arr):
        a = np.ascontiguousarray(arr)
        h = self.alloc(max(a.nbytes, 16))
        self.upload(h, a)
        return h

    def download(self, h, shape, dtype=np.float32, off=0):
        out = np.empty(shape, dtype)
        self._check(self.L.qp_download(out.ctypes.data, h, off, out.nbytes), "qp_download")
        return out

    def copy(self, dst, src, n, dst_off=0, src_off=0):
        self._check(self.L.qp_copy(dst, dst_off, src, src_off, n), "qp_copy")

    def sync(self):
        self._check(self.L.qp_sync(), "qp_sync")

    # -------------------------------------------------------------- ops
    def op(self, name):
        i = self._ops.get(name)
        if i is None:
            i = self.L.qp_op_id(name.encode())
            if i < 0:
                raise QuipuError(f"unknown op {name}")
            self._ops[name] = i
        return i

    def dispatch(self, name, u, bufs, grid=(1, 1, 1), noalloc=False):
        """grupo(name, [u, paso, ...bufs]) + despachar(pass, g, *grid) of the reference facade; noalloc: through
        qp_dispatch_noalloc (workspace from the library's fixed scratch array)."""
        ub = uniform(u) if isinstance(u, (list, tuple)) else bytes(u)
        b = (C.c_uint64 * len(bufs))(*[int(x or 0) for x in bufs])
        g = tuple(grid) + (1,) * (3 - len(grid))
        ubuf = C.create_string_buffer(ub, len(ub))
        fn = self.L.qp_dispatch_noalloc if noalloc else self.L.qp_dispatch
        self._check(fn(self.op(name), ubuf, len(ub), b, len(bufs), *g), name)

    # -------------------------------------------------------------- weights (device layout)
    def upload_matrix(self, fmt, raw, N, K):
        """GGUF blocks of an N x K matrix -> device tensor in this backend's layout (repacked on the device: Q4_K,
        Q5_K and Q6_K to row chunk planes, Q8_0 and IQ4_NL to planar qs | d).  Returns the handle."""
        raw = np.ascontiguousarray(np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else raw)
        assert raw.nbytes == gguf_bytes(fmt, N, K), (raw.nbytes, gguf_bytes(fmt, N, K))
        if fmt == F32:
            return self.buffer_from(raw)
        staging = self.buffer_from(raw)
        dst = self.alloc(device_bytes(fmt, N, K))
        nb = N * K // BLOCK[fmt][0]
        op = {Q2_K: "repack_q2k", Q3_K: "repack_q3k", Q4_K: "repack_q4k", Q5_K: "repack_q5k", Q6_K: "repack_q6k",
              Q8_0: "repack_q8", IQ4_NL: "repack_iq4nl"}[fmt]
        self.dispatch(op, [("u", nb & 0xFFFFFFFF), ("u", nb >> 32), ("u", K)], [0, staging, dst])
        self.sync()
        self.free(staging)
        return dst

    def dequant(self, fmt, h, nelem, K):
        """The device tensor h (rows of K elements) dequantized to f32, in element order."""
        y = self.alloc(nelem * 4)
        self.dispatch("dequant", [("u", fmt), ("u", nelem & 0xFFFFFFFF), ("u", nelem >> 32), ("u", K)], [0, h, y])
        out = self.download(y, (nelem,))
        self.free(y)
        return out

    def paso(self, T, pos0):
        h = self.alloc(16)
        self.upload(h, np.array([T, pos0, 0, 0], np.uint32))
        return h

    # -------------------------------------------------------------- graphs / events
    def graph_begin(self):
        self._check(self.L.qp_graph_begin(), "qp_graph_begin")

    def graph_end(self):
        g = C.c_uint64()
        self._check(self.L.qp_graph_end(C.byref(g)), "qp_graph_end")
        return g.value

    def graph_launch(self, g):
        self._check(self.L.qp_graph_launch(g), "qp_graph_launch")

    def graph_free(self, g):
        self._check(self.L.qp_graph_free(g), "qp_graph_free")

    def event(self):
        e = C.c_uint64()
        self._check(self.L.qp_event_create(C.byref(e)), "qp_event_create")
        return e.value

    def record(self, e):
        self._check(self.L.qp_event_record(e), "qp_event_record")

    def elapsed_ms(self, e0, e1):
        ms = C.c_float()
        self._check(self.L.qp_event_elapsed(e0, e1, C.byref(ms)), "qp_event_elapsed")
        return ms.value

    def event_free(self, e):
        self._check(self.L.qp_event_free(e), "qp_event_free")


def gemv_uniform(nseg, K, eps=0.0, last_row=0, R=0, max_wg=0, fmt=Q4_K, segs=()):
    """P of the fused `gemv` op: segs = [(mode, n, row_base, rows_total[, seg_fmt]), ...]; a segment's own format
    (Q4_K / Q6_K mixed in one launch) rides in bits 8..15 of its mode word.  Formats are GGUF type ids."""
    u = [("u", nseg), ("u", K), ("f", eps), ("u", last_row), ("u", R), ("u", max_wg), ("u", fmt), ("u", 0)]
    for sg in segs:
        mode, n, rb, rt = sg[:4]
        sf = sg[4] if len(sg) > 4 else 0
        u += [("u", mode | (sf << 8)), ("u", n), ("u", rb), ("u", rt)]
    return u
