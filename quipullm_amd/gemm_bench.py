"""Prefill matmul microbenchmark: Y[T][N] = X[T][K] W[N][K]^T through the reference op `matmul_<fmt>_t` (the
matrix-core kernel for T >= 64), with random packed weights and X ~ N(0, 1).

    python -m quipullm_amd.gemm_bench [--shape q4k:14336x4096] [--tokens 512] [--iters 20]

Launches rotate through enough weight copies (>= --rotate-mb) that the last-level cache cannot hold them; HIP
events on the backend's stream time the loop.  Algorithmic FLOPs are 2*T*N*K per launch (the kernel issues 3x as
many matrix-core operations: the bf16 high/low products).  One JSON line per shape on stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np

if __package__ in (None, ""):
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from quipullm_amd import capi, synth  # noqa: E402
from quipullm_amd.gemv_bench import parse_shape  # noqa: E402


def time_gemm(q, fmt, N, K, T, iters=20, rotate_bytes=640 << 20):
    nbytes = capi.gguf_bytes(fmt, N, K)
    ncopy = max(2, rotate_bytes // nbytes + 1)
    raw = np.frombuffer(synth.gen_blocks(np.random.default_rng([5, N, K]), fmt, N * K), np.uint8)
    hs = [q.upload_matrix(fmt, raw, N, K) for _ in range(ncopy)]
    xb = q.buffer_from(np.random.default_rng(6).standard_normal(T * K).astype(np.float32))
    yb = q.alloc(T * N * 4)
    paso = q.paso(T, 0)
    name = "matmul_%s_t" % capi.FMT_NAME[fmt]
    u = [("u", N), ("u", K), ("u", 0), ("u", 0)]
    for i in range(3):
        q.dispatch(name, u, [paso, hs[i % ncopy], xb, yb], (1, 1, (T + 31) // 32))
    q.sync()
    e0, e1 = q.event(), q.event()
    q.record(e0)
    for i in range(iters):
        q.dispatch(name, u, [paso, hs[i % ncopy], xb, yb], (1, 1, (T + 31) // 32))
    q.record(e1)
    us = q.elapsed_ms(e0, e1) * 1000.0 / iters
    for h in hs + [xb, yb, paso]:
        q.free(h)
    q.event_free(e0)
    q.event_free(e1)
    flop = 2.0 * T * N * K
    return {"op": name, "format": capi.FMT_NAME[fmt], "T": T, "N": N, "K": K, "launches": iters,
            "us_per_launch": us, "TFLOPs": flop / (us * 1e-6) / 1e12}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", action="append", help="fmt:NxK with fmt in q4k, q6k, q8, f32")
    ap.add_argument("--tokens", type=int, default=512)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--rotate-mb", type=int, default=640)
    a = ap.parse_args()
    q = capi.Quipu(0)
    for s in a.shape or ["q4k:14336x4096", "q6k:4096x14336"]:
        fmt, N, K = parse_shape(s)
        print(json.dumps(time_gemm(q, fmt, N, K, a.tokens, a.iters, a.rotate_mb << 20)), flush=True)


if __name__ == "__main__":
    main()
