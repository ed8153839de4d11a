"""Token sampling (reference web/js/sampling.js): the oracle restatement pinned by hand-derived cases, and the
product's JavaScript sampler (quipullm_amd/js/sampling.js) choosing exactly the oracle's tokens.

Hand-derived cases use logits ln(1..4) (as float32), whose softmax is 0.1 .. 0.4, with a stubbed uniform draw u,
so the chosen token follows from the cumulative weights written out in each test.
"""
import json
import math
import os

import numpy as np
import pytest

from conftest import ROOT, run
from oracle.sampling import Sampler, mulberry32

JS = os.path.join(ROOT, "quipullm_amd", "js", "sampling.js")
LN = np.log(np.array([1.0, 2.0, 3.0, 4.0])).astype(np.float32)


def fixed(u):
    return lambda: u


# ------------------------------------------------------------------------------------------------ oracle pins
def test_mulberry32_is_uniform_and_seeded():
    r = mulberry32(12345)
    x = np.array([r() for _ in range(200000)])
    assert x.min() >= 0.0 and x.max() < 1.0
    h, _ = np.histogram(x, bins=64, range=(0.0, 1.0))
    chi2 = float(((h - len(x) / 64) ** 2 / (len(x) / 64)).sum())
    assert chi2 < 120, chi2                      # 63 degrees of freedom: p < 1e-5 beyond ~120
    assert abs(np.corrcoef(x[:-1], x[1:])[0, 1]) < 0.01
    a, b, c = mulberry32(7), mulberry32(7), mulberry32(8)
    sa, sb, sc = [a() for _ in range(5)], [b() for _ in range(5)], [c() for _ in range(5)]
    assert sa == sb and sa != sc
    # outputs are k / 2^32 for an integer k
    assert all(float(v * 4294967296.0).is_integer() for v in sa)


@pytest.mark.parametrize("u,want", [(0.2, 3), (0.6, 2), (0.8, 1), (0.95, 0)])
def test_draw_follows_the_softmax_weights(u, want):
    # temperature 1, no cuts: weights exp(l - max) = k/4 -> [1, .75, .5, .25] over ids [3, 2, 1, 0], total 2.5;
    # r = 2.5 u falls in (0,1] -> 3, (1,1.75] -> 2, (1.75,2.25] -> 1, (2.25,2.5] -> 0
    s = Sampler(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, rand=fixed(u))
    assert s.choose(LN, []) == want


@pytest.mark.parametrize("u,want", [(0.5, 3), (0.6, 2)])
def test_temperature_sharpens(u, want):
    # temperature 0.5: weights (k/4)^2 = [1, .5625, .25, .0625], total 1.875; u=.5 -> r=.9375 -> 3;
    # u=.6 -> r=1.125: 1.125-1 > 0, then -.5625 -> 2
    s = Sampler(temperature=0.5, top_k=0, top_p=1.0, min_p=0.0, rand=fixed(u))
    assert s.choose(LN, []) == want


def test_top_p_cut():
    # probabilities .4 .3 .2 .1: cumulative .4, .7 >= .65 -> 2 candidates {3, 2}; weights 1, .75 (total 1.75);
    # u = .99 -> r = 1.7325 -> 2; ids 1 and 0 are never drawn
    s = Sampler(temperature=1.0, top_k=0, top_p=0.65, min_p=0.0, rand=fixed(0.99))
    assert s.choose(LN, []) == 2
    for u in np.linspace(0.001, 0.999, 50):
        assert Sampler(temperature=1.0, top_k=0, top_p=0.65, min_p=0.0, rand=fixed(u)).choose(LN, []) in (2, 3)


@pytest.mark.parametrize("min_p,allowed", [(0.6, {3, 2}), (0.8, {3}), (0.2, {3, 2, 1, 0})])
def test_min_p_cut(min_p, allowed):
    # limit = .4 * min_p: .24 keeps .4 and .3; .32 keeps only .4; .08 keeps all four
    got = {Sampler(temperature=1.0, top_k=0, top_p=1.0, min_p=min_p, rand=fixed(u)).choose(LN, [])
           for u in np.linspace(0.001, 0.999, 200)}
    assert got == allowed


def test_top_k_one_and_tiny_temperature_are_argmax():
    x = np.random.default_rng(3).standard_normal(500).astype(np.float32)
    for u in (0.0001, 0.5, 0.9999):
        assert Sampler(temperature=1.0, top_k=1, rand=fixed(u)).choose(x, []) == int(np.argmax(x))
        assert Sampler(temperature=1e-4, top_k=0, top_p=1.0, min_p=0.0, rand=fixed(u)).choose(x, []) == int(np.argmax(x))


def test_penalty_arithmetic():
    # rep 2, freq .1, pres .5 over history [0, 1, 1, 3]:
    #   token 0 (once): 2/2 - (.1 + .5) = .4;  token 1 (twice): -2*2 - (.2 + .5) = -4.7;  token 3: .5/2 - .6 = -.35
    s = Sampler(temperature=0.0, repeat_penalty=2.0, frequency_penalty=0.1, presence_penalty=0.5)
    lg = np.array([2.0, -2.0, 1.0, 0.5], np.float32)
    s.penalize(lg, [0, 1, 1, 3])
    assert lg.tolist() == np.array([0.4, -4.7, 1.0, -0.35], np.float32).tolist()
    assert s.choose(np.array([2.0, -2.0, 1.0, 0.5], np.float32), [0, 1, 1, 3]) == 2
    # only the last 64 history tokens count: token 0 seen 70 times -> counted 64 times
    lg = np.array([1.0, 0.0], np.float32)
    Sampler(temperature=0.0, frequency_penalty=1.0).penalize(lg, [0] * 70)
    assert lg[0] == np.float32(1.0 - 64.0)


def test_heap_order_among_ties():
    # [0, 1, 1, 2], k=2: push 0, push 1 (parent 0 <= 1: stays) -> [0, 1]; i=2: 1 > 0 -> root = 2, sift down stops
    # (child 1 is not strictly smaller) -> [2, 1]; i=3: 2 > 1 -> root = 3, child 1 smaller -> [1, 3].
    # So of the tied ids 1 and 2, id 1 is kept; after the stable sort the order is [3, 1].
    lg = np.array([0, 1, 1, 2], np.float32)
    s = Sampler(temperature=1.0, top_k=2, top_p=1.0, min_p=0.0, rand=fixed(0.999))
    assert s.candidates(lg) == [1, 3]
    assert s.choose(lg, []) == 1
    # [1, 1, 1, 0], k=2: the first two fill the heap and equal values never replace the root
    assert Sampler(top_k=2).candidates(np.array([1, 1, 1, 0], np.float32)) == [0, 1]


# ------------------------------------------------------------------------------------------------ JS sampler
NODE_DRIVER = r"""
const fs = require('fs');
const { Muestreador, mulberry32 } = require(%s);
const casos = JSON.parse(fs.readFileSync(%s, 'utf8'));
const out = [];
for (const c of casos) {
  if (c.rng) { const r = mulberry32(c.seed); const v = []; for (let i = 0; i < c.n; i++) v.push(r()); out.push(v); continue; }
  const mu = new Muestreador(c.params);
  const hist = c.hist.slice();
  const ids = [];
  for (const lg of c.logits) {
    const id = mu.elegir(Float32Array.from(lg), hist);
    ids.push(id); hist.push(id);
  }
  out.push(ids);
}
console.log(JSON.stringify(out));
"""


def js_run(tmp_path, cases):
    f = tmp_path / "cases.json"
    f.write_text(json.dumps(cases))
    rc, out, err = run(["node", "-e", NODE_DRIVER % (json.dumps(JS), json.dumps(str(f)))], timeout=120)
    assert rc == 0, err[-3000:]
    return json.loads(out.strip().splitlines()[-1])


def oracle_run(case):
    p = dict(case["params"])
    s = Sampler(**{k: v for k, v in p.items()})
    hist = list(case["hist"])
    ids = []
    for lg in case["logits"]:
        i = s.choose(np.array(lg, np.float32), hist)
        ids.append(i)
        hist.append(i)
    return ids


PARAMS = [
    {"seed": 1},                                                             # reference defaults
    {"seed": 2, "temperature": 1.5, "top_k": 0, "top_p": 1.0, "min_p": 0.0},
    {"seed": 3, "temperature": 0.7, "top_k": 5, "top_p": 0.9, "min_p": 0.1},
    {"seed": 4, "temperature": 1.0, "top_k": 200, "top_p": 0.8, "min_p": 0.0, "repeat_penalty": 1.3,
     "frequency_penalty": 0.2, "presence_penalty": 0.1},
    {"seed": 5, "temperature": 0.0, "repeat_penalty": 1.5},                  # greedy with penalties
    {"seed": -77, "temperature": 2.0, "top_k": 1000, "top_p": 0.99, "min_p": 0.01},
]


@pytest.mark.parametrize("ties", [False, True])
def test_js_sampler_matches_oracle(tmp_path, ties):
    rng = np.random.default_rng(40 + ties)
    cases = []
    for p in PARAMS:
        V = 3000
        lg = (rng.standard_normal((24, V)) * 3).astype(np.float32)
        if ties:
            lg = (np.round(lg * 2) / 2).astype(np.float32)   # many equal logits at every cut point
        hist = rng.integers(0, V, 10).tolist()
        cases.append({"params": p, "hist": hist, "logits": lg.tolist()})
    got = js_run(tmp_path, cases)
    want = [oracle_run(c) for c in cases]
    assert got == want


def test_js_mulberry32_matches_oracle(tmp_path):
    cases = [{"rng": True, "seed": s, "n": 2000} for s in (0, 1, 42, -5, 2 ** 31 - 1, 123456789)]
    got = js_run(tmp_path, cases)
    for c, g in zip(cases, got):
        r = mulberry32(c["seed"])
        assert g == [r() for _ in range(c["n"])]
