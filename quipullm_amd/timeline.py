"""Summary of a per-workgroup timeline recorded by the profiling build (lib/timeline/, built by
`python quipullm_amd/build.py --timeline`).

That build's kernels stamp, for every launch captured into a graph, each workgroup's start and end
(s_memrealtime, 100 MHz), hardware id and XCC, and thread 0 of the GEMV and decode-attention workgroups stamps
its phase boundaries; the library writes the records of the last replay when the graph is freed:

    QP_TIMELINE_OUT         uint32 x4 per workgroup slot, 4096 slots per launch (t0, t1, hw id, xcc | 1 << 31)
    QP_TIMELINE_OUT.json    [[kernel, gx, gy, gz, block], ...] in launch order
    QP_TIMELINE_OUT.ph      uint32 phase stamps [kind][workgroup][8] (the last launch of a kind keeps its stamps)

    python -m quipullm_amd.timeline QP_TIMELINE_OUT [--launches N]

prints, per kernel, the median over its launches of: span (first workgroup start to last workgroup end), gap
(this launch's first start minus the previous launch's last end: the dependent-launch boundary), start spread
(90th percentile of the workgroup starts after the first one), median and maximum workgroup lifetime and the
end tail (last end minus the 90th percentile of ends); then the step's totals and the phase times.
"""
import argparse
import collections
import json
import os

import numpy as np

TICK_US = 0.01          # s_memrealtime runs at 100 MHz
SLOTS = 4096
PHASE_KINDS = {
    0: ("gemv, mixed Q/K/V formats", ["input arrived", "input staged", "first unit's weights", "all units"]),
    1: ("gemv, Q4_K one row per slot", ["input arrived", "input staged", "first unit's weights", "all units"]),
    2: ("gemv, Q4_K row pairs", ["input arrived", "input staged", "first unit's weights", "all units"]),
    3: ("gemv, Q6_K long rows (512 threads)", ["input arrived", "input staged", "first unit's weights", "all units"]),
    4: ("gemv, Q6_K", ["input arrived", "input staged", "first unit's weights", "all units"]),
    5: ("gemv, other formats", ["input arrived", "input staged", "first unit's weights", "all units"]),
    6: ("decode attention", ["q,k,v loaded", "norm+RoPE", "q split", "key stream", "wave merge", "end"]),
    7: ("attention block", ["Q/K/V GEMV", "barrier 1", "q split", "partials stored", "barrier 2", "merged"]),
    8: ("MoE router (working column)", ["input staged", "rows done", "arrival counted", "routed (last workgroup)"]),
    10: ("decode attention, merge (from the partials' drain; the last workgroups of the columns)",
         ["arrival counted", "weights", "weights barrier", "sums", "sums barrier"]),
    9: ("MoE router, routing (last workgroups)", ["probabilities", "first barrier", "ranks", "second barrier",
                                                "weights stored"]),
}


def load(path):
    meta = json.load(open(path + ".json"))
    raw = np.fromfile(path, np.uint32)
    raw = raw[: len(raw) // (SLOTS * 4) * SLOTS * 4].reshape(-1, SLOTS, 4)
    ph = None
    if os.path.exists(path + ".ph"):
        ph = np.fromfile(path + ".ph", np.uint32).reshape(-1, SLOTS, 8)
    return meta, raw, ph


def launches(meta, raw):
    """One dict per launch: kernel, workgroups, and (when its kernel records) the timing figures in us."""
    recs = []
    for i, (kn, gx, gy, gz, blk) in enumerate(meta):
        n = gx * gy * gz
        d = {"i": i, "kernel": kn, "wgs": n, "block": blk}
        if i < len(raw):
            v = raw[i][: min(n, SLOTS)]
            ok = (v[:, 3] & 0x80000000) != 0
            if ok.any():
                d["t0"], d["t1"] = v[ok, 0].astype(np.int64), v[ok, 1].astype(np.int64)
                d["xcc"] = (v[ok, 3] & 0xF).astype(np.int64)
        recs.append(d)
    timed = [d for d in recs if "t0" in d]
    if not timed:
        return recs
    base = int(timed[0]["t0"].min())
    prev_end = None
    for d in timed:
        # 32-bit stamps: unwrap against the first workgroup (a step lasts far less than 2^32 ticks = 43 s)
        t0 = ((d["t0"] - base) % (1 << 32)) * TICK_US
        t1 = ((d["t1"] - base) % (1 << 32)) * TICK_US
        dur = t1 - t0
        d.update(start=t0.min(), end=t1.max(), span=t1.max() - t0.min(),
                 gap=(t0.min() - prev_end) if prev_end is not None else 0.0,
                 spread=np.percentile(t0, 90) - t0.min(), wg_med=float(np.median(dur)), wg_max=float(dur.max()),
                 tail=t1.max() - np.percentile(t1, 90), xccs=int(len(np.unique(d["xcc"]))))
        prev_end = t1.max()
    return recs


def report(path, n_first=12):
    meta, raw, ph = load(path)
    recs = launches(meta, raw)
    timed = [d for d in recs if "span" in d]
    lines = [f"timeline {os.path.basename(path)}: {len(recs)} launches captured, {len(timed)} with workgroup records",
             ""]
    agg = collections.OrderedDict()
    for d in timed:
        agg.setdefault(d["kernel"], []).append(d)
    hdr = (f"| {'kernel':30s} | {'n':>4s} | {'WGs':>5s} | {'span':>7s} | {'gap':>5s} | {'start90':>7s} | "
           f"{'WG med':>6s} | {'WG max':>6s} | {'tail10':>6s} | {'XCCs':>4s} |")
    lines += [hdr, "|" + "|".join("-" * (len(c)) for c in hdr.split("|")[1:-1]) + "|"]
    for kn, L in agg.items():
        med = lambda k: float(np.median([x[k] for x in L]))
        lines.append(f"| {kn:30s} | {len(L):4d} | {L[0]['wgs']:5d} | {med('span'):7.2f} | {med('gap'):5.2f} | "
                     f"{med('spread'):7.2f} | {med('wg_med'):6.2f} | {med('wg_max'):6.2f} | {med('tail'):6.2f} | "
                     f"{int(med('xccs')):4d} |")
    if timed:
        total = timed[-1]["end"] - timed[0]["start"]
        spans = sum(d["span"] for d in timed)
        gaps = sum(d["gap"] for d in timed)
        lines += ["", f"step: first start to last end {total:.1f} us; sum of spans {spans:.1f} us; "
                      f"sum of gaps {gaps:.1f} us ({len(timed)} launches, {gaps / max(len(timed) - 1, 1):.2f} us "
                      f"per boundary)"]
        lines += ["", f"first {n_first} launches (us from the step's first workgroup):"]
        for d in timed[:n_first]:
            lines.append(f"  {d['i']:3d} {d['kernel']:30s} start {d['start']:8.2f} end {d['end']:8.2f} "
                         f"gap {d['gap']:5.2f} span {d['span']:6.2f}")
    if ph is not None:
        lines += ["", "phases (median / 90th percentile, us from the workgroup's start; the last launch of a kind):"]
        for kind, (name, labels) in PHASE_KINDS.items():
            P = ph[kind].astype(np.int64)
            ok = P[:, 0] != 0
            if not ok.any():
                continue
            P = P[ok]
            # the last launch of the kind: first stamps within 20 us of the latest (launches of one kind are a
            # layer, 40 us or more, apart); workgroup slots that only earlier launches wrote drop out
            P = P[(P[:, 0].max() - P[:, 0]) < int(20.0 / TICK_US)]
            rel = ((P - P[:, :1]) % (1 << 32)) * TICK_US
            # a stamp only some workgroups write is summarized over those that wrote it in this launch (0, or a
            # stale stamp of an earlier launch, in the others: more than 1 ms from the workgroup's first)
            mine = (P != 0) & (rel < 1000.0)
            cols = "; ".join(f"{lab} {np.median(rel[mine[:, j + 1], j + 1]):.2f}/"
                             f"{np.percentile(rel[mine[:, j + 1], j + 1], 90):.2f}"
                             for j, lab in enumerate(labels) if mine[:, j + 1].any())
            lines.append(f"  {name} ({len(P)} WGs): {cols}")
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("path", help="the QP_TIMELINE_OUT file")
    ap.add_argument("--launches", type=int, default=12, help="launches listed one by one")
    a = ap.parse_args(argv)
    print(report(a.path, a.launches))


if __name__ == "__main__":
    main()
