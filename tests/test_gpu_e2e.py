"""End-to-end parity of the benchmark configurations on the GPU against committed oracle fixtures.

The CPU oracle is too slow to follow these models through their long prompts inside a GPU test, so its results
were written once by tests/golden/make_e2e.py (same seeded synthetic GGUF files, which this test regenerates
with quipullm_amd.synth and identifies by a digest of sampled bytes).  Cases:

* C3 (8B Q4_K_M, 32 layers) at context 512: 128 greedy tokens;
* the 8B shapes in 2 centered layers at context 4096: 128 greedy tokens (varied ids);
* C4: a 2048-token prompt in one prefill chunk, its last token's logits and 8 greedy tokens;
* C5 (48-layer MoE, 128 experts, top-8) after a 2048-token prompt: 128 greedy tokens;
* the MoE shapes in 4 centered layers after 2048 prompt ids: 128 greedy tokens (varied ids).

The GPU runs the product host (Node.js engine, fused one-token graph) with the reference's f32 KV cache, as the
oracle did.  Bars (north star): greedy ids identical; logits within 1e-3 relative (max |a - b| / max |b|), checked
in full on the stored whole rows (the fixture's int16 rounding, at most max|b| / 65534, is taken off the allowance)
and on the oracle's 16 largest logits of every step.  A divergence of the ids is accepted only at a step whose
oracle top-1 / top-2 margin is below twice the logit allowance (a tie within the tolerance, the reference's
EMPATES policy of tests/conformance/test_transformer.py:16, 110-113, decided from the data); steps after it are
not compared.  The per-step margins are printed.
"""
import json
import os

import numpy as np
import pytest

from conftest import ROOT, run
from quipullm_amd import build, synth

pytestmark = pytest.mark.gpu

CLI = os.path.join(ROOT, "quipullm_amd", "js", "cli.js")
GOLDEN = os.path.join(ROOT, "tests", "golden")
TOL = 1e-3
CASES = ["c3_ctx512", "c3s_ctx4096", "c4_prefill2048", "c5_ctx2048", "c5s_ctx2048"]


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


def compare(fx, gpu_ids, lg):
    """Checks the GPU run against the fixture; returns a summary line."""
    want = fx["ids"].tolist()
    maxabs, top_ids, top_vals, margin = fx["maxabs"], fx["top_ids"], fx["top_vals"], fx["margin"]
    n = len(want)
    assert len(gpu_ids) == n and lg.shape[0] == n
    # first divergence of the greedy ids: only at a tie within the logit tolerance
    upto = n
    for i in range(n):
        if gpu_ids[i] != want[i]:
            assert margin[i] < 2 * TOL * maxabs[i], \
                f"ids diverge at step {i} (gpu {gpu_ids[i]}, oracle {want[i]}) where the oracle's margin " \
                f"{margin[i]:.4g} is {margin[i] / maxabs[i]:.2e} of max|logit|"
            upto = i + 1  # the diverging step's logits are still from the same sequence
            break
    errs = []
    for i in range(upto):
        got = lg[i, top_ids[i]]
        e = float(np.max(np.abs(got - top_vals[i])) / maxabs[i])
        errs.append(e)
        assert np.isfinite(lg[i]).all(), f"non-finite logits at step {i}"
        assert e < TOL, f"step {i}: top-16 logits off by {e:.2e} of max|logit|"
        assert abs(float(np.max(np.abs(lg[i]))) - float(maxabs[i])) <= TOL * maxabs[i], f"step {i}: max|logit|"
    for s, q, sc in zip(fx["full_steps"], fx["full_rows"], fx["full_scale"]):
        if s >= upto:
            continue
        ref = q.astype(np.float64) * float(sc)
        e = float(np.max(np.abs(lg[s].astype(np.float64) - ref)) / maxabs[s])
        assert e < TOL - 1.0 / 65534, f"step {s}: whole logit row off by {e:.2e} of max|logit|"
    return f"{upto}/{n} steps compared, {len(set(want))} distinct ids, max top-16 error {max(errs):.2e}, " \
           f"min margin {float(np.min(margin[:upto] / maxabs[:upto])):.2e} of max|logit|"


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
    pf, lf = os.path.join(str(tmp_path), "prompt.json"), os.path.join(str(tmp_path), "logits.f32")
    with open(pf, "w") as f:
        json.dump([int(t) for t in prompt], f)
    cmd = ["timeout", "-k", "5", "200", "node", CLI, "generate", "--model", path, "--prompt-file", pf, "--n", str(n),
           "--mode", "fast", "--kv", "f32", "--ctx", str(P + n + 8), "--batch", str(batch), "--logits-out", lf]
    print(case, model, "prompt", P, "batch", batch, "steps", n, flush=True)
    rc, out, err = run(cmd, timeout=240)
    assert rc == 0, err[-3000:]
    r = json.loads(out.strip().splitlines()[-1])
    lg = np.fromfile(lf, np.float32).reshape(n, c.vocab)
    print(case, compare(fx, r["ids"], lg), flush=True)
