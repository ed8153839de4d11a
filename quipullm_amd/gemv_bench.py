"""Single-op GEMV microbenchmark (batch 1, y = W x with x ~ N(0, 1)) and the streaming-copy calibration kernel.

    python -m quipullm_amd.gemv_bench [--shape q4k:14336x4096 ...] [--iters 200] [--rotate-mb 640]
    python -m quipullm_amd.gemv_bench --copy-bytes 1073741824 [--iters 20]

Each shape is timed over back-to-back launches of the fused `gemv` op that rotate through enough copies of the
weight matrix (>= --rotate-mb) that the last-level cache cannot hold them, with HIP events recorded on the
backend's stream.  The algorithmic bytes of one launch are the weight blocks plus the f32 input and output.
--copy-bytes times the plain copy kernel (reads and writes that many bytes per launch): the reference point
for scaling hardware byte counters.  One JSON line per measurement on stdout.
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

FMT_BY_NAME = {v: k for k, v in capi.FMT_NAME.items()}


def parse_shape(s):
    f, nk = s.split(":")
    n, k = nk.lower().split("x")
    return FMT_BY_NAME[f], int(n), int(k)


def time_gemv(q, fmt, N, K, iters=200, rotate_bytes=640 << 20, R=0, max_wg=0):
    """Average launch duration of the fused GEMV on one shape; returns a dict.  R, max_wg: the op's rows per
    wavefront and grid cap (0: the backend's defaults)."""
    paso = q.paso(1, 0)
    nbytes = capi.gguf_bytes(fmt, N, K)
    ncopy = max(2, rotate_bytes // nbytes + 1)
    raw = np.frombuffer(synth.gen_blocks(np.random.default_rng([3, N, K]), fmt, N * K), np.uint8)
    hs = [q.upload_matrix(fmt, raw, N, K) for _ in range(ncopy)]
    xb = q.buffer_from(np.random.default_rng(4).standard_normal(K).astype(np.float32))
    yb = q.alloc(N * 4)
    u = capi.gemv_uniform(1, K, R=R, max_wg=max_wg, fmt=fmt, segs=[(capi.STORE, N, 0, N)])
    for i in range(10):
        q.dispatch("gemv", u, [paso, xb, 0, 0, hs[i % ncopy], 0, yb])
    q.sync()
    e0, e1 = q.event(), q.event()
    q.record(e0)
    for i in range(iters):
        q.dispatch("gemv", u, [paso, xb, 0, 0, hs[i % ncopy], 0, yb])
    q.record(e1)
    us = q.elapsed_ms(e0, e1) * 1000.0 / iters
    alg = nbytes + 4 * K + 4 * N
    for h in hs:
        q.free(h)
    for h in (xb, yb, paso):
        q.free(h)
    q.event_free(e0)
    q.event_free(e1)
    return {"kernel": "qp_gemv_%s" % capi.FMT_NAME[fmt], "format": capi.FMT_NAME[fmt], "N": N, "K": K, "R": R,
            "max_wg": max_wg, "bytes": alg, "launches": iters, "us_per_launch": us, "GBs": alg / (us * 1e-6) / 1e9}


def time_copy(q, nbytes, iters=20):
    """Average launch duration of the streaming copy kernel over nbytes (read nbytes, write nbytes)."""
    n4 = nbytes // 16
    src, dst = q.alloc(nbytes), q.alloc(nbytes)
    q.dispatch("fill_u32", [("u", 0x3F800000), ("u", (nbytes // 4) & 0xFFFFFFFF), ("u", (nbytes // 4) >> 32)],
               [0, src])
    u = [("u", n4 & 0xFFFFFFFF), ("u", n4 >> 32), ("u", 0)]
    for _ in range(3):
        q.dispatch("copy_f4", u, [0, src, dst])
    q.sync()
    e0, e1 = q.event(), q.event()
    q.record(e0)
    for _ in range(iters):
        q.dispatch("copy_f4", u, [0, src, dst])
    q.record(e1)
    us = q.elapsed_ms(e0, e1) * 1000.0 / iters
    q.free(src)
    q.free(dst)
    q.event_free(e0)
    q.event_free(e1)
    return {"kernel": "qp_copy_f4", "read_bytes": n4 * 16, "write_bytes": n4 * 16, "launches": iters,
            "us_per_launch": us, "GBs": 2 * n4 * 16 / (us * 1e-6) / 1e9}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", action="append", help="fmt:NxK with fmt in q2k, q3k, q4k, q5k, q6k, q8, iq4nl, f32")
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--rotate-mb", type=int, default=640)
    ap.add_argument("--R", type=int, default=0, help="rows per wavefront (0: the backend default)")
    ap.add_argument("--max-wg", type=int, default=0, help="grid cap (0: the backend default)")
    ap.add_argument("--copy-bytes", type=int, default=0)
    a = ap.parse_args()
    q = capi.Quipu(0)
    if a.copy_bytes:
        print(json.dumps(time_copy(q, a.copy_bytes, a.iters)), flush=True)
    shapes = a.shape or ([] if a.copy_bytes else ["q4k:14336x4096"])
    for s in shapes:
        fmt, N, K = parse_shape(s)
        print(json.dumps(time_gemv(q, fmt, N, K, a.iters, a.rotate_mb << 20, a.R, a.max_wg)), flush=True)


if __name__ == "__main__":
    main()
