"""Benchmark of the MI355X token loop: decode tok/s of the 8B-shape Q4_K_M model, plus the Q4_K GEMV roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one greedy decode token of the Llama-3-8B-shaped Q4_K_M model (32 layers, hidden 4096, GQA 32/8,
head_dim 128, FFN 14336, vocab 128256; random weights written to a seeded synthetic GGUF), batch 1, f16 KV.
The KV cache is first filled by prefilling 4096 uniform-random prompt ids (the headline figure) and, in further
measurements, 2048 and 512.  Weights and activations are resident in HBM when the timed region starts; the timed
region is K back-to-back replays of the captured one-token step, bracketed by HIP events on the backend's stream,
with the greedy argmax on the device.

Also measured live: the dominant kernel, the Q4_K GEMV (14336 x 4096, batch 1), over back-to-back launches that
rotate through >= 512 MB of weight copies (so the 256 MB last-level cache cannot hold them), timed with HIP
events on the backend's stream.

Parity (config.parity_vs_oracle): the 8B shape at full depth with centered weights (varied greedy ids) after a
512-token prompt, 128 steps of the fused path teacher-forced on the oracle's ids, with the reference's f32 KV
cache, against the CPU oracle's fixture tests/golden/e2e_c3c_ctx512.npz (every step's device argmax against the
oracle's id; the 16 largest logits of every step and three whole rows within 1e-3 of max|logit|).  The CPU baseline is the C
restatement of the reference semantics (the test oracle) on this host's cores: decode steps of the same model
at KV length 4096 (cpu_baseline), and in config.cpu_baselines the C1 tiny Q8_0 model end to end and the C2 GEMVs,
on all threads and on one.

Process layout: this process runs the CPU checker first, then the GPU decode in child Node.js processes (the
product host), and only then opens the GPU itself (ctypes) for the GEMV measurement, so no program is started
from a process that has initialised the GPU.  One JSON line is printed.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from quipullm_amd import synth  # noqa: E402

PEAK_HBM_GBS = 8000.0
MODEL = "llama8b_q4km"
METRIC = "decode tok/s @8B-shape Q4_K ctx 4096; Q4_K GEMV HBM GB/s vs peak"
# Prefill of 2048 tokens on the 8B shape: 2*M*sum(N*K) over the 7 matrices of 32 layers, causal attention
# 2*2*sum_i(i)*hd*nh*L, and the last token's output row (algorithmic FLOPs, not the MFMA instructions issued)
PREFILL_2048_FLOP = (2 * 2048 * 32 * (4096 * 4096 * 2 + 1024 * 4096 * 2 + 14336 * 4096 * 3)
                     + 2 * 2 * (2048 * 2049 // 2) * 128 * 32 * 32 + 2 * 128256 * 4096)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_dir():
    d = os.environ.get("QP_MODEL_DIR") or os.path.join((os.environ.get("TMPDIR") or "/tmp"), "quipu_models")
    os.makedirs(d, exist_ok=True)
    return d


def ensure_built():
    from quipullm_amd import build
    if not build.built() or not os.path.exists(build.NAPI):
        log("bench: native parts missing, building")
        build.build_all(oracle=True)


def decode_bytes_per_token(model, path, P, n):
    """Algorithmic HBM bytes of one decode token, averaged over the n timed steps after a P-token prefill:
    every weight tensor read once (embedding: one row; stacked expert tensors: the n_used selected experts of
    n_exp), plus the f16 K and V rows of every cached position."""
    from oracle.oracle import GGUF  # header reader only
    g = GGUF(path)
    c = synth.CONFIGS[model]
    w = 0
    for name, t in g.tensors.items():
        if name == "token_embd.weight":
            w += t["bytes"] // c.vocab
        elif "_exps." in name:
            w += t["bytes"] * c.n_used // c.n_exp
        else:
            w += t["bytes"]
    kv_per_pos = c.n_layers * 2 * c.nkv * c.hd * 2
    mean_pos = P + (n + 1) / 2.0
    return w, w + kv_per_pos * mean_pos


CPU_PROMPT = [1, 128000, 9906, 1917]


def cpu_baseline(path, seconds=20.0, kv_len=4096):
    """The oracle on this host: greedy decode steps of the same model (f16 KV, as the GPU run) at KV length kv_len,
    as many as fit in about `seconds` (at least 2).  The cache holds a 4-token prompt's rows copied over positions
    4 .. kv_len-1, so each step does the arithmetic of a decode step at that length (a real 4096-token prefill
    would take the checker minutes)."""
    from oracle import oracle as O
    threads = O.lib().or_num_threads()
    m = O.Model(path, ctx=kv_len + 48, kv_f16=True)
    lg = m.forward(CPU_PROMPT, True)  # also pages the weights in
    m.fill_cache_to(kv_len)
    ids = [O.argmax(lg)]
    t0 = time.time()
    steps = 0
    while steps < 2 or (time.time() - t0 < seconds and steps < 40):
        lg = m.forward([ids[-1]], True)
        ids.append(O.argmax(lg))
        steps += 1
    dt = time.time() - t0
    m.close()
    return {"value": steps / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{steps} greedy decode steps of the same 8B Q4_K_M model at KV length {kv_len}..{kv_len + steps} "
                      f"(f16 KV; the cache filled with copies of a 4-token prompt's rows) in {dt:.1f} s on {threads} "
                      f"OpenMP threads; C restatement of the reference WGSL semantics"}


def cpu_side_baselines(tiny_path, gemv_shapes, rotate=3):
    """The other CPU timings of the hot path on the oracle, on all threads and on one: the C1 tiny Q8_0 LLaMA end to
    end (32-token prompt, then greedy tokens: 128 on all threads, 16 on one) and the C2 GEMVs (lane order of
    matmul_*_1, the best of `rotate` calls on distinct weights)."""
    from oracle import oracle as O
    L = O.lib()
    nthr = L.or_num_threads()
    out = {"threads_all": nthr}
    prompt = synth.random_prompt(32000, 32, 2)
    for thr, n in ((nthr, 128), (1, 16)):
        L.or_set_threads(thr)
        m = O.Model(tiny_path, ctx=200)
        t0 = time.time()
        lg = m.forward(prompt, True)
        t1 = time.time()
        tok = O.argmax(lg)
        for _ in range(n - 1):
            tok = O.argmax(m.forward([tok], True))
        t2 = time.time()
        m.close()
        out[f"c1_tiny_q8_{thr}thr"] = {"prompt_tokens": 32, "decode_tokens": n, "prefill_ms": round(1e3 * (t1 - t0), 1),
                                       "decode_tok_s": round((n - 1) / (t2 - t1), 2)}
    gem = []
    for fmt, N, K in gemv_shapes:
        bpr = {synth.GGML_Q4_K: 144, synth.GGML_Q6_K: 210}[fmt] * (K // 256)
        raws = [np.frombuffer(synth.gen_blocks(np.random.default_rng(40 + i), fmt, N * K), np.uint8)
                for i in range(rotate)]
        x = np.random.default_rng(3).standard_normal(K).astype(np.float32)
        for thr in (nthr, 1):
            L.or_set_threads(thr)
            best = 1e9
            for r in raws:
                t0 = time.time()
                O.matmul(fmt, r, N, K, x)
                best = min(best, time.time() - t0)
            nbytes = N * bpr + 4 * K + 4 * N
            gem.append({"format": {synth.GGML_Q4_K: "q4k", synth.GGML_Q6_K: "q6k"}[fmt], "N": N, "K": K,
                        "threads": thr, "ms": round(1e3 * best, 3), "GBs": round(nbytes / best / 1e9, 2)})
    L.or_set_threads(nthr)
    out["c2_gemv"] = gem
    out["kind"] = "port (C restatement of the reference WGSL semantics)"
    return out


def run_decode(model, path, steps, warmup, prefills, eager=False, seed=7, sample=False):
    """The product host (Node.js CLI) on `model`: for each P in prefills, prefill P uniform-random ids, then time
    `steps` greedy decode tokens (with `sample`, also `steps` tokens with the reference's default sampler from the
    same position)."""
    c = synth.CONFIGS[model]
    ctx = max(prefills) + steps + warmup + 8
    ids = synth.random_prompt(c.vocab, max(prefills), seed)
    pf = os.path.join(model_dir(), f"{model}.bench_prompt.json")
    with open(pf, "w") as f:
        json.dump(ids, f)
    cmd = ["node", os.path.join(ROOT, "quipullm_amd", "js", "cli.js"), "bench", "--model", path, "--prompt-file", pf,
           "--n", str(steps), "--warmup", str(warmup), "--kv", "f16", "--ctx", str(ctx), "--batch", "2048",
           "--max-gen", str(max(steps, warmup) + 8), "--prefill", ",".join(str(p) for p in prefills)]
    if eager:
        cmd.append("--eager")
    if sample:
        cmd.append("--sample")
    log("bench: " + " ".join(cmd))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError("decode benchmark failed:\n" + r.stderr[-3000:])
    return json.loads(r.stdout.strip().splitlines()[-1])


def side_configs(steps, warmup, eager):
    """The other decode workloads of the hot path, measured on the same product path (no parity check here; the
    GPU tests pin their parity on smaller models of the same formats): the MoE model (48 layers, 128 experts,
    top-8, Q4_K) at ctx 2048, the 8B shape in Q5_K_M at ctx 4096 and the tiny Q8_0 LLaMA after a 32-token
    prompt."""
    out = {}
    for model, P, n in (("qwen3moe_q4k", 2048, steps), ("llama8b_q5km", 4096, steps), ("tiny_q8", 32, 128)):
        path = synth.ensure_model(model, model_dir())
        r = run_decode(model, path, n, warmup, [P], eager=eager, seed=11)["runs"][0]
        _, bpt = decode_bytes_per_token(model, path, P, n)
        out[model] = {"prompt_tokens": P, "steps": n, "decode_tok_s": round(r["decode_tok_s"], 3),
                      "ms_per_token": round(r["ms_per_token"], 4), "prefill_tok_s": round(r["prefill_tok_s"], 1),
                      "bytes_per_token": int(bpt), "hbm_GBs": round(bpt * r["decode_tok_s"] / 1e9, 1),
                      "roofline_frac": round(bpt * r["decode_tok_s"] / 1e9 / PEAK_HBM_GBS, 4)}
        log(f"bench: {model} " + json.dumps(out[model]))
    return out


def parity_fixture(case="c3c_ctx512", eager=False):
    """The fused path against the CPU oracle's fixture of `case` (tests/golden/make_e2e.py; by default the 8B shape
    at full depth with centered weights, whose greedy ids vary), the same prompt and greedy length, the reference's
    f32 KV cache.  The run is teacher-forced on the fixture's ids (each step consumes the oracle's previous id), so
    every step is compared: the largest relative logit error over the fixture's per-step top-16 logits and its whole
    rows, and at each step whether the device's own argmax is the oracle's id or a tie within 2e-3 of max|logit|.
    eager: the one-token step dispatched op by op (for profilers) instead of replaying its graph."""
    fp = os.path.join(ROOT, "tests", "golden", f"e2e_{case}.npz")
    if not os.path.exists(fp):
        return {"case": case, "error": "fixture missing"}
    fx = np.load(fp, allow_pickle=False)
    model = str(fx["model"])
    P, n, batch = int(fx["prompt_len"]), len(fx["ids"]), int(fx["batch"])
    c = synth.CONFIGS[model]
    path = synth.ensure_model(model, model_dir())
    pf, ff, lf = (os.path.join(model_dir(), f"{case}.{x}") for x in ("prompt.json", "force.json", "logits.f32"))
    with open(pf, "w") as f:
        json.dump(synth.random_prompt(c.vocab, P, int(fx["prompt_seed"])), f)
    with open(ff, "w") as f:
        json.dump([int(t) for t in fx["ids"]], f)
    cmd = ["node", os.path.join(ROOT, "quipullm_amd", "js", "cli.js"), "generate", "--model", path, "--prompt-file",
           pf, "--n", str(n), "--mode", "fast", "--kv", "f32", "--ctx", str(P + n + 8), "--batch", str(batch),
           "--logits-out", lf, "--force-ids", ff] + (["--eager"] if eager else [])
    log("bench: " + " ".join(cmd))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError("parity run failed:\n" + r.stderr[-3000:])
    ids = json.loads(r.stdout.strip().splitlines()[-1])["ids"]
    lg = np.fromfile(lf, np.float32).reshape(n, c.vocab)
    maxabs, want = fx["maxabs"], fx["ids"].tolist()
    rel = [float(np.max(np.abs(lg[i, fx["top_ids"][i]] - fx["top_vals"][i])) / maxabs[i]) for i in range(n)]
    for s_, q, sc in zip(fx["full_steps"], fx["full_rows"], fx["full_scale"]):
        rel.append(float(np.max(np.abs(lg[s_] - q.astype(np.float64) * float(sc))) / maxabs[s_]))
    equal, ties, wrong = 0, [], []
    for i in range(n):
        if ids[i] == want[i]:
            equal += 1
            continue
        pos = np.nonzero(fx["top_ids"][i] == ids[i])[0]
        gap = float(fx["top_vals"][i][0] - fx["top_vals"][i][pos[0]]) if pos.size else float("inf")
        (ties if gap < 2e-3 * maxabs[i] else wrong).append(i)
    # np.max propagates a NaN (Python's max would skip it depending on the order)
    return {"case": case, "model": model, "prompt_tokens": P, "tokens": n, "kv": "f32", "teacher_forced": True,
            "steps_compared": n, "device_ids_equal": equal, "tie_steps": ties, "wrong_steps": wrong,
            "max_rel_logits": float(np.max(rel)), "min_margin_rel": float(np.min(fx["margin"] / maxabs)),
            "distinct_ids": len(set(want)), "reference": "CPU restatement of the reference semantics (oracle fixture)"}


def gemv_microbench(shapes, iters=200, rotate_bytes=640 << 20):
    """Average launch duration (HIP events over back-to-back launches) of the fused GEMV op, per shape."""
    from quipullm_amd import capi, gemv_bench
    q = capi.Quipu(0)
    return [gemv_bench.time_gemv(q, fmt, N, K, iters, rotate_bytes) for fmt, N, K in shapes]


def committed_traffic():
    """HBM bytes per launch of the Q4_K GEMV from the committed rocprofv3 counter summary, if present."""
    p = os.path.join(ROOT, "profiles", "gemv_q4k_14336x4096_traffic.md")
    if not os.path.exists(p):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.e+]+)", open(p).read(), re.M)
    return float(m.group(1)) if m else None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-side", action="store_true", help="skip the MoE and tiny Q8_0 decode measurements")
    ap.add_argument("--decode-launch", choices=["graph", "eager"], default="graph",
                    help="the one-token step as a captured HIP graph (default) or dispatched op by op (same kernels; "
                         "for profilers that cannot follow graph launches)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {a.gpus}); the multi-GPU sharding of the "
              f"token loop is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    if "RANK" in os.environ and os.environ.get("WORLD_SIZE", "1") != "1":
        print("bench.py: one GPU only", file=sys.stderr)
        sys.exit(2)
    ensure_built()
    t0 = time.time()
    path = synth.ensure_model(MODEL, model_dir())
    log(f"bench: model {path} ready in {time.time() - t0:.1f}s")
    cpu = cpu_baseline(path, a.cpu_seconds)
    log(f"bench: cpu baseline {cpu['value']:.3f} tok/s")
    cpu_side = {} if a.no_side else cpu_side_baselines(
        synth.ensure_model("tiny_q8", model_dir()),
        [(synth.GGML_Q4_K, 4096, 4096), (synth.GGML_Q4_K, 14336, 4096), (synth.GGML_Q4_K, 4096, 14336),
         (synth.GGML_Q6_K, 4096, 4096), (synth.GGML_Q6_K, 14336, 4096), (synth.GGML_Q6_K, 4096, 14336)])
    log("bench: cpu side baselines " + json.dumps(cpu_side))
    prefills = [4096, 2048, 512]
    dec = run_decode(MODEL, path, a.steps, a.warmup, prefills, a.decode_launch == "eager", sample=True)
    check = parity_fixture(eager=a.decode_launch == "eager")
    runs = {r["prompt_tokens"]: r for r in dec["runs"]}
    log("bench: decode " + json.dumps(dec))
    log("bench: parity " + json.dumps(check))
    from quipullm_amd import capi
    gem = gemv_microbench([(capi.Q4_K, 14336, 4096), (capi.Q4_K, 4096, 4096), (capi.Q4_K, 4096, 14336),
                           (capi.Q6_K, 4096, 4096), (capi.Q6_K, 14336, 4096), (capi.Q6_K, 4096, 14336)])
    dom = gem[0]
    main_run = runs[4096]
    wbytes, bpt = decode_bytes_per_token(MODEL, path, 4096, a.steps)
    _, bpt512 = decode_bytes_per_token(MODEL, path, 512, a.steps)
    side = {} if a.no_side else side_configs(a.steps, a.warmup, a.decode_launch == "eager")
    tok_s = main_run["decode_tok_s"]
    result = {
        "metric": METRIC, "value": round(tok_s, 3), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(main_run["ms_per_token"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"Llama-3-8B-shape Q4_K_M (Q6_K attn_v/ffn_down/output) greedy decode, batch 1, "
                               f"KV prefilled with {prefills[0]} random prompt ids, f16 KV, {a.steps} timed tokens "
                               f"after {a.warmup} warm-up tokens (also after prefills of {prefills[1]} and "
                               f"{prefills[2]} ids)",
                   "ctx": 4096, "kv": "f16", "batch": 1, "prefill_tokens": 4096, "decode_launch": a.decode_launch,
                   "decode_tok_s_ctx512": round(runs[512]["decode_tok_s"], 3),
                   "decode_hbm_GBs_ctx4096": round(bpt * tok_s / 1e9, 1),
                   "decode_roofline_frac_ctx4096": round(bpt * tok_s / 1e9 / PEAK_HBM_GBS, 4),
                   "decode_roofline_frac_ctx512": round(bpt512 * runs[512]["decode_tok_s"] / 1e9 / PEAK_HBM_GBS, 4),
                   "bytes_per_token_ctx4096": int(bpt), "weight_bytes_per_token": int(wbytes),
                   "wall_tok_s_ctx4096": round(main_run["wall_tok_s"], 3),
                   "prefill_tok_s_4096": round(main_run["prefill_tok_s"], 1),
                   "prefill_tok_s_2048": round(runs[2048]["prefill_tok_s"], 1),
                   "decode_tok_s_ctx2048": round(runs[2048]["decode_tok_s"], 3),
                   "decode_sampled_tok_s_ctx4096": round(main_run["sampled_tok_s"], 3),
                   "prefill_2048_TFLOPs": round(PREFILL_2048_FLOP / (runs[2048]["prefill_ms"] * 1e-3) / 1e12, 2),
                   "side_configs": side,
                   "gemv": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in g.items()} for g in gem],
                   "parity_vs_oracle": check, "cpu_baselines": cpu_side},
        "roofline": {"bound": "hbm", "kernel": "qp_gemv_q4k_r1 (Q4_K GEMV 14336x4096, batch 1)",
                     "achieved": round(dom["GBs"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(dom["GBs"] / PEAK_HBM_GBS, 4), "traffic": committed_traffic(),
                     "bytes_per_launch": dom["bytes"], "us_per_launch": round(dom["us_per_launch"], 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
