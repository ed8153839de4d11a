"""CPU restatement of quipullm's token sampler -- TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, as the checker of the product's sampler (quipullm_amd/js/sampling.js and the
device top-k candidates); the product never imports it.

It follows web/js/sampling.js of the reference step by step, in float64 like the JavaScript it restates:
  - mulberry32 (sampling.js:3-10): the 32-bit state update and output, emulated with explicit int32 / uint32
    wrapping;
  - penalties over the last 64 history tokens (sampling.js:27-37), stored back rounded to float32 as a
    Float32Array store rounds;
  - temperature <= 0: strict '>' argmax scan, ties to the lowest index (sampling.js:38-42);
  - top-k with the reference's min-heap (sampling.js:44-57): its exact sift-up / sift-down comparisons, so that
    the candidate order among equal logits is the reference's;
  - stable sort by descending logit (sampling.js:58), softmax without temperature, top-p and min-p cuts,
    temperature, and the draw (sampling.js:59-81).

Parity pins (tests/test_sampling.py): hand-computed cases (explicit softmax weights and draws, the top-p / min-p
cut points, the penalty arithmetic, the heap's choice among ties derived by hand), mulberry32's uniformity, and the
limits that reduce to argmax (top_k = 1, tiny temperature).
"""
from __future__ import annotations

import math

import numpy as np


def _i32(x):
    x &= 0xFFFFFFFF
    return x - (1 << 32) if x & 0x80000000 else x


def _imul(a, b):
    return _i32((a & 0xFFFFFFFF) * (b & 0xFFFFFFFF))


def _shr(a, n):
    # JavaScript `a >>> n` of an int32
    return (a & 0xFFFFFFFF) >> n


def mulberry32(seed):
    """The generator of sampling.js:3-10: a callable returning floats in [0, 1)."""
    state = [_i32(int(seed))]

    def nxt():
        a = _i32(state[0] + 0x6D2B79F5)
        state[0] = a
        t = _imul(a ^ _shr(a, 15), 1 | a)
        t = _i32(t + _imul(t ^ _shr(t, 7), 61 | t)) ^ t
        return _shr(_i32(t ^ _shr(t, 14)), 0) / 4294967296.0

    return nxt


class Sampler:
    """sampling.js:12-23 (defaults: temperature 0.8, top_k 40, top_p 0.95, min_p 0.05, no penalties, window 64)."""

    def __init__(self, temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.0,
                 frequency_penalty=0.0, presence_penalty=0.0, seed=None, rand=None):
        self.temp, self.top_k, self.top_p, self.min_p = temperature, top_k, top_p, min_p
        self.rep, self.freq, self.pres = repeat_penalty, frequency_penalty, presence_penalty
        self.window = 64
        self.rand = rand if rand is not None else (mulberry32(seed) if seed is not None else None)

    def penalize(self, logits, history):
        """sampling.js:27-37, in place on a float32 array."""
        if not history or (self.rep == 1 and not self.freq and not self.pres):
            return
        count = {}
        for t in history[-self.window:]:
            count[t] = count.get(t, 0) + 1
        V = len(logits)
        for t, n in count.items():
            if t >= V:
                continue
            v = float(logits[t])
            if self.rep != 1:
                v = v / self.rep if v > 0 else v * self.rep
            v -= n * self.freq + self.pres
            logits[t] = np.float32(v)

    def candidates(self, logits):
        """The top-k candidate list before the sort (sampling.js:44-57): heap order, or 0..V-1."""
        V = len(logits)
        k = min(self.top_k, V) if self.top_k > 0 else V
        if k >= V:
            return list(range(V))
        lg = [float(v) for v in logits]
        heap = []

        def up(i):
            while i > 0:
                p = (i - 1) >> 1
                if lg[heap[p]] <= lg[heap[i]]:
                    break
                heap[p], heap[i] = heap[i], heap[p]
                i = p

        def down(i):
            while True:
                l, r, m = 2 * i + 1, 2 * i + 2, i
                if l < len(heap) and lg[heap[l]] < lg[heap[m]]:
                    m = l
                if r < len(heap) and lg[heap[r]] < lg[heap[m]]:
                    m = r
                if m == i:
                    break
                heap[m], heap[i] = heap[i], heap[m]
                i = m

        for i in range(V):
            if len(heap) < k:
                heap.append(i)
                up(len(heap) - 1)
            elif lg[i] > lg[heap[0]]:
                heap[0] = i
                down(0)
        return heap

    def draw(self, cand, value, u):
        """sampling.js:58-81 from a candidate list; value(i) is the logit of token i, u the uniform draw."""
        cand = sorted(cand, key=lambda i: -value(i))   # stable, descending (sampling.js:58)
        mx = value(cand[0])
        probs = [math.exp(value(i) - mx) for i in cand]
        s = 0.0
        for p in probs:
            s += p
        probs = [p / s for p in probs]
        n = len(cand)
        if self.top_p < 1:
            acc = 0.0
            for i in range(n):
                acc += probs[i]
                if acc >= self.top_p:
                    n = i + 1
                    break
        if self.min_p > 0:
            lim = probs[0] * self.min_p
            m = 1
            while m < n and probs[m] >= lim:
                m += 1
            n = m
        cand = cand[:n]
        pt = [math.exp((value(i) - mx) / self.temp) for i in cand]
        tot = 0.0
        for p in pt:
            tot += p
        r = u * tot
        for i, p in enumerate(pt):
            r -= p
            if r <= 0:
                return cand[i]
        return cand[-1]

    def choose(self, logits, history):
        """sampling.js:25-82: penalties, then argmax or the stochastic draw (one call of rand)."""
        logits = np.array(logits, np.float32)
        self.penalize(logits, list(history))
        if not (self.temp > 0):
            best, bv = 0, -math.inf
            for i, v in enumerate(logits):
                if v > bv:
                    bv, best = float(v), i
            return best
        cand = self.candidates(logits)
        return self.draw(cand, lambda i: float(logits[i]), self.rand())
