"""End-to-end parity of the benchmark configurations on the GPU against the CPU oracle.

Two kinds of case.

Fixture cases.  The oracle is too slow to follow these models through their long prompts inside a GPU test, so
its results were written once by tests/golden/make_e2e.py (same seeded synthetic GGUF files, which this test
regenerates with quipullm_amd.synth and identifies by a digest of sampled bytes):

* C3 (8B Q4_K_M, 32 layers) at context 512 (its random weights repeat one token);
* the 8B shape in 32 centered layers at context 512 (varied greedy ids);
* the 8B shapes in 2 centered layers at context 4096;
* C4: a 2048-token prompt in one prefill chunk, its last token's logits and 8 greedy tokens;
* C5 (48-layer MoE, 128 experts, top-8) after a 2048-token prompt;
* the MoE shape in 48 centered layers after a 64-token prompt (varied greedy ids), and in 4 centered layers after
  2048.

The GPU runs the product host (Node.js engine, fused one-token graph) with the reference's f32 KV cache, as the
oracle did, teacher-forced on the fixture's ids (`cli.js generate --force-ids`: step i consumes the oracle's id
i - 1, the same graph replays with the step's input written from the host), so every step is compared even after
a near tie: the device's own argmax at each step must be the oracle's id, or a tie within the tolerance (the
oracle's value of the device's choice within twice the logit allowance of its top; the reference's EMPATES policy,
tests/conformance/test_transformer.py:16, 110-113).  Logits within 1e-3 relative (max |a - b| / max |b|), checked
on the oracle's 16 largest logits of every step and in full on the stored whole rows (the fixture's int16
rounding, at most max|b| / 65534, is taken off the allowance).

The timed path itself.  The bench's decode (the 8B shape at full depth, f16 KV cache, 4096 prompt ids prefilled in
2048-token chunks, 128 greedy tokens of the captured one-token graph with the merged 17-split matrix-core
attention, the device choosing and feeding each token) against the oracle resumed from the GPU's own f16 cache rows
at position 4095 (Model.resume_from_reference), which then follows the GPU's ids: logits within 1e-3 at every
step, every device choice the oracle's argmax or a tie as above.

Each case adds a line to the run's summary ("end-to-end parity"): steps compared, distinct ids, ties, errors.
"""
import json
import os

import numpy as np
import pytest

import refs
from conftest import E2E_SUMMARY, ROOT, run
from quipullm_amd import build, synth

pytestmark = pytest.mark.gpu

CLI = os.path.join(ROOT, "quipullm_amd", "js", "cli.js")
GOLDEN = os.path.join(ROOT, "tests", "golden")
TOL = 1e-3
CASES = ["c3_ctx512", "c3c_ctx512", "c3s_ctx4096", "c4_prefill2048", "c5_ctx2048", "c5c_ctx64", "c5s_ctx2048"]


def fixture(case):
    p = os.path.join(GOLDEN, f"e2e_{case}.npz")
    if not os.path.exists(p):
        pytest.fail(f"fixture {p} missing: run tests/golden/make_e2e.py {case}")
    return np.load(p, allow_pickle=False)


def model_digest(path):
    import hashlib
    h = hashlib.sha256()
    size = os.path.getsize(path)
    h.update(str(size).encode())
    with open(path, "rb") as f:
        for off in range(0, size, 16 << 20):
            f.seek(off)
            h.update(f.read(4096))
    return h.hexdigest()


def compare_forced(fx, gpu_ids, lg):
    """Checks a teacher-forced GPU run against the fixture at every step; returns a summary."""
    want = fx["ids"].tolist()
    maxabs, top_ids, top_vals, margin = fx["maxabs"], fx["top_ids"], fx["top_vals"], fx["margin"]
    n = len(want)
    assert len(gpu_ids) == n and lg.shape[0] == n
    errs, ties = [], []
    for i in range(n):
        assert np.isfinite(lg[i]).all(), f"non-finite logits at step {i}"
        got = lg[i, top_ids[i]]
        e = float(np.max(np.abs(got - top_vals[i])) / maxabs[i])
        errs.append(e)
        assert e < TOL, f"step {i}: top-16 logits off by {e:.2e} of max|logit|"
        assert abs(float(np.max(np.abs(lg[i]))) - float(maxabs[i])) <= TOL * maxabs[i], f"step {i}: max|logit|"
        if gpu_ids[i] != want[i]:
            # the device chose another id: it must be among the oracle's largest, within the tie allowance
            pos = np.nonzero(top_ids[i] == gpu_ids[i])[0]
            assert pos.size, f"step {i}: device chose {gpu_ids[i]}, not among the oracle's 16 largest"
            gap = float(top_vals[i][0] - top_vals[i][pos[0]])
            assert gap < 2 * TOL * maxabs[i], \
                f"step {i}: device chose {gpu_ids[i]} over the oracle's {want[i]} with a gap of {gap / maxabs[i]:.2e}"
            ties.append(i)
    for s, q, sc in zip(fx["full_steps"], fx["full_rows"], fx["full_scale"]):
        ref = q.astype(np.float64) * float(sc)
        e = float(np.max(np.abs(lg[s].astype(np.float64) - ref)) / maxabs[s])
        assert e < TOL - 1.0 / 65534, f"step {s}: whole logit row off by {e:.2e} of max|logit|"
    return (f"{n}/{n} steps compared, {len(set(want))} distinct ids, device ids equal at {n - len(ties)} "
            f"(ties within tolerance at {ties}), max top-16 error {max(errs):.2e}, "
            f"min oracle margin {float(np.min(margin / maxabs)):.2e} of max|logit|")


@pytest.mark.timeout(600)
@pytest.mark.parametrize("case", CASES)
def test_config_matches_oracle_fixture(models_dir, tmp_path, case):
    if not build.built() or not os.path.exists(build.NAPI):
        pytest.fail("native parts not built: run __graft_entry__.build() first")
    fx = fixture(case)
    model = str(fx["model"])
    P, seed, batch, n = int(fx["prompt_len"]), int(fx["prompt_seed"]), int(fx["batch"]), len(fx["ids"])
    path = synth.ensure_model(model, models_dir)
    assert model_digest(path) == str(fx["model_digest"]), "regenerated model differs from the fixture's"
    c = synth.CONFIGS[model]
    prompt = synth.random_prompt(c.vocab, P, seed)
    pf, ff, lf = (os.path.join(str(tmp_path), f) for f in ("prompt.json", "force.json", "logits.f32"))
    with open(pf, "w") as f:
        json.dump([int(t) for t in prompt], f)
    with open(ff, "w") as f:
        json.dump([int(t) for t in fx["ids"]], f)
    cmd = ["timeout", "-k", "5", "200", "node", CLI, "generate", "--model", path, "--prompt-file", pf, "--n", str(n),
           "--mode", "fast", "--kv", "f32", "--ctx", str(P + n + 8), "--batch", str(batch), "--logits-out", lf,
           "--force-ids", ff]
    print(case, model, "prompt", P, "batch", batch, "steps", n, flush=True)
    rc, out, err = run(cmd, timeout=240)
    assert rc == 0, err[-3000:]
    r = json.loads(out.strip().splitlines()[-1])
    assert r.get("forced") is True
    lg = np.fromfile(lf, np.float32).reshape(n, c.vocab)
    line = compare_forced(fx, r["ids"], lg)
    print(case, line, flush=True)
    E2E_SUMMARY.append(f"{case} ({model}, f32 KV, teacher-forced): {line}")


@pytest.mark.timeout(900)
def test_timed_path_f16_ctx4096_matches_resumed_oracle(oracle, models_dir, tmp_path):
    """The bench's decode end to end: 32 centered 8B-shape layers, f16 KV, 4096 prompt ids in 2048-token chunks,
    128 greedy ids chained on the device through the captured graph; the oracle resumed from the GPU's own cache
    rows at position 4095 follows the GPU's ids.  Logits within 1e-3 at every step; every device choice the
    oracle's argmax or a tie within 2e-3 of max|logit|."""
    if not build.built() or not os.path.exists(build.NAPI):
        pytest.fail("native parts not built: run __graft_entry__.build() first")
    name = "llama8b_q4km_c"
    c = synth.CONFIGS[name]
    P, n, batch = 4096, 128, 2048
    ctx = P + n
    path = synth.ensure_model(name, models_dir)
    prompt = synth.random_prompt(c.vocab, P, 26)
    pf, lf, kvf = (os.path.join(str(tmp_path), f) for f in ("prompt.json", "logits.f32", "kv.bin"))
    with open(pf, "w") as f:
        json.dump([int(t) for t in prompt], f)
    cmd = ["timeout", "-k", "5", "240", "node", CLI, "generate", "--model", path, "--prompt-file", pf, "--n", str(n),
           "--mode", "fast", "--kv", "f16", "--ctx", str(ctx), "--batch", str(batch), "--logits-out", lf,
           "--kv-out", kvf]
    print("timed path:", name, "prompt", P, "batch", batch, "steps", n, "f16 KV", flush=True)
    rc, out, err = run(cmd, timeout=300)
    assert rc == 0, err[-3000:]
    r = json.loads(out.strip().splitlines()[-1])
    gpu_ids = r["ids"]
    lg = np.fromfile(lf, np.float32).reshape(n, c.vocab)
    assert r["pos"] == P + n - 1
    kvd = c.nkv * c.hd
    k16, v16 = refs.read_kv_f16(kvf, c.n_layers, ctx, kvd, P + n - 1)
    os.remove(kvf)
    oracle.set_threads(min(16, os.cpu_count() or 1))
    m = oracle.Model(path, ctx=ctx, kv_f16=True)
    m.set_kv_reference(k16, v16)
    m.resume_from_reference(P - 1)
    errs, ties, margins = [], [], []
    try:
        for i in range(n):
            want = m.forward([prompt[-1] if i == 0 else gpu_ids[i - 1]], True)
            mx = float(np.max(np.abs(want)))
            e = float(np.max(np.abs(lg[i].astype(np.float64) - want)) / mx)
            errs.append(e)
            best = oracle.argmax(want)
            srt = np.sort(want.astype(np.float64))
            margins.append((srt[-1] - srt[-2]) / mx)
            assert np.isfinite(lg[i]).all(), f"step {i}: non-finite logits"
            assert e < TOL, f"step {i}: logits off by {e:.2e} of max|logit|"
            if gpu_ids[i] != best:
                gap = float(want[best]) - float(want[gpu_ids[i]])
                assert gap < 2 * TOL * mx, \
                    f"step {i}: device chose {gpu_ids[i]} over the oracle's {best} with a gap of {gap / mx:.2e}"
                ties.append(i)
            if i % 32 == 31:
                print(f"  step {i + 1}/{n}: max error so far {max(errs):.2e}", flush=True)
    finally:
        m.close()
    line = (f"{n}/{n} steps compared, {len(set(gpu_ids))} distinct ids, device ids equal to the oracle's argmax at "
            f"{n - len(ties)} (ties within tolerance at {ties}), max logit error {max(errs):.2e}, "
            f"min oracle margin {min(margins):.2e} of max|logit|")
    print("timed path:", line, flush=True)
    E2E_SUMMARY.append(f"c3c_ctx4096_f16 ({name}, f16 KV, captured graph, resumed oracle): {line}")
