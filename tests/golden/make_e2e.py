"""Writes the end-to-end parity fixtures of the benchmark configurations (tests/golden/e2e_<case>.npz) by running
the CPU oracle (oracle/, the C restatement of the reference's WGSL semantics) on the seeded synthetic GGUF files
that quipullm_amd.synth writes, the same files the GPU tests generate on the GPU box.

    python tests/golden/make_e2e.py [case ...]      (cases: see CASES; default all)

Per case: the prompt (synth.random_prompt), prefilled in chunks of `batch` tokens, then `n` greedy tokens, all with
the reference's f32 KV cache.  Stored per generated step: the greedy id, max |logit|, the 16 largest logits with
their ids (descending value, ties to the lower id) and the top-1 / top-2 margin; and for the steps in `full` the
whole logit row as int16 of 32767 * logit / max|logit| (absolute error at most max|logit| / 65534).  Also a digest
of sampled bytes of the model file, so a test can tell whether its regenerated file is the same.

Run here (CPU, 8 threads: a few minutes per case); the GPU box only reads the .npz files.
"""
from __future__ import annotations

import argparse
import hashlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from quipullm_amd import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TOPK = 16

# case -> (model, prompt tokens, prompt seed, prefill chunk, greedy tokens, steps stored whole)
CASES = {
    # C3: the 8B Q4_K_M model itself, context 512 (its greedy output is nearly constant: random weights)
    "c3_ctx512": ("llama8b_q4km", 512, 21, 512, 128, (0, 127)),
    # the 8B shapes (2 centered layers): 128 greedy tokens after 4096 prompt ids
    "c3s_ctx4096": ("llama8b_q4km_c2", 4096, 22, 512, 128, (0, 127)),
    # C4: the 2048-token prefill in one chunk, its last token's logits and 8 greedy tokens
    "c4_prefill2048": ("llama8b_q4km_c2", 2048, 23, 2048, 8, (0, 7)),
    # C5: the 48-layer MoE after a 2048-token prompt
    "c5_ctx2048": ("qwen3moe_q4k", 2048, 24, 2048, 128, (0, 127)),
    # the MoE shapes (4 centered layers): varied greedy ids after 2048 prompt ids
    "c5s_ctx2048": ("qwen3moe_q4k_c4", 2048, 25, 2048, 128, (0, 127)),
    # full depth with varied greedy ids: the 8B shape (32 centered layers, weights of standard deviation 0.02) at
    # context 512, and the MoE shape (48 centered layers, 0.1) after a 64-token prompt
    "c3c_ctx512": ("llama8b_q4km_c", 512, 27, 512, 128, (0, 64, 127)),
    "c5c_ctx64": ("qwen3moe_q4k_c", 64, 28, 64, 128, (0, 64, 127)),
}


def model_digest(path: str) -> str:
    """sha256 over one 4 KiB page every 16 MiB of the file, plus its size."""
    h = hashlib.sha256()
    size = os.path.getsize(path)
    h.update(str(size).encode())
    with open(path, "rb") as f:
        for off in range(0, size, 16 << 20):
            f.seek(off)
            h.update(f.read(4096))
    return h.hexdigest()


def top_of(lg: np.ndarray, k: int = TOPK):
    order = np.lexsort((np.arange(len(lg)), -lg.astype(np.float64)))[:k]
    return order.astype(np.int32), lg[order].astype(np.float32)


def run_case(name: str, model_dir: str) -> str:
    model, P, seed, batch, n, full = CASES[name]
    path = synth.ensure_model(model, model_dir)
    c = synth.CONFIGS[model]
    prompt = synth.random_prompt(c.vocab, P, seed)
    t0 = time.time()
    m = O.Model(path, ctx=P + n + 8, kv_f16=False, tiled=True)
    ids, lgs = m.generate(prompt, n, batch=batch)
    m.close()
    dt = time.time() - t0
    lgs = np.stack(lgs).astype(np.float32)
    maxabs = np.max(np.abs(lgs), axis=1).astype(np.float32)
    tops = [top_of(r) for r in lgs]
    full = [s for s in full if s < n]
    scale = maxabs[full] / 32767.0
    rows = np.clip(np.rint(lgs[full] / scale[:, None]), -32767, 32767).astype(np.int16)
    out = os.path.join(HERE, f"e2e_{name}.npz")
    np.savez_compressed(
        out, model=np.array(model), prompt_len=np.int32(P), prompt_seed=np.int32(seed), batch=np.int32(batch),
        ids=np.array(ids, np.int32), maxabs=maxabs, top_ids=np.stack([t[0] for t in tops]),
        top_vals=np.stack([t[1] for t in tops]),
        margin=np.array([t[1][0] - t[1][1] for t in tops], np.float32), full_steps=np.array(full, np.int32),
        full_rows=rows, full_scale=scale.astype(np.float32), model_digest=np.array(model_digest(path)),
        oracle_seconds=np.float32(dt), threads=np.int32(O.lib().or_num_threads()))
    return f"{name}: {len(set(ids))} distinct of {n} ids, min margin {min(t[1][0] - t[1][1] for t in tops):.4g}, " \
           f"{dt:.0f} s -> {out}"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("cases", nargs="*", default=list(CASES))
    ap.add_argument("--model-dir", default=os.environ.get("QP_MODEL_DIR", "/tmp/quipu_models"))
    a = ap.parse_args()
    os.makedirs(a.model_dir, exist_ok=True)
    for name in a.cases:
        print(run_case(name, a.model_dir), flush=True)


if __name__ == "__main__":
    main()
