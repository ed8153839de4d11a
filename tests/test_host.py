"""Host side of the boundary, without a GPU: the C ABI library and its exports, the N-API addon, the JavaScript
host's GGUF reader / uniform packing / sampler / architecture registry, and bench.py's command line.

Programs (node, a fresh python) are started through the spawner of conftest.py.
"""
import ctypes as C
import json
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, run
from quipullm_amd import build, capi, synth

JS = os.path.join(ROOT, "quipullm_amd", "js")


@pytest.fixture(scope="module")
def built():
    if not build.built() or not os.path.exists(build.NAPI):
        build.build_all(oracle=False)
    return True


def node(script, timeout=120):
    rc, out, err = run(["node", "-e", script], timeout=timeout)
    assert rc == 0, err[-3000:]
    return json.loads(out.strip().splitlines()[-1])


# ------------------------------------------------------------------------------------------------ C ABI
def test_library_exports_every_declared_symbol(built):
    names = capi.declared_symbols()
    assert len(names) >= 24
    lib = C.CDLL(capi.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_header_declares_the_facade():
    want = {"qp_init", "qp_info", "qp_last_error", "qp_alloc", "qp_free", "qp_upload", "qp_download", "qp_copy",
            "qp_sync", "qp_op_id", "qp_dispatch", "qp_graph_begin", "qp_graph_end", "qp_graph_launch",
            "qp_graph_free", "qp_event_create", "qp_event_record", "qp_event_elapsed", "qp_event_free",
            "qp_module_load", "qp_kernel", "qp_launch", "qp_bytes_used", "qp_lost"}
    assert want <= set(capi.declared_symbols())


# every op name the JavaScript host dispatches (transformer.js, weights.js) and the tests use
FORMATS = ("q2k", "q3k", "q4k", "q5k", "q6k", "q8", "f32", "iq4nl")
OPS = ["matmul_%s_%s" % (f, s) for f in FORMATS for s in ("1", "4", "t", "e", "e_swiglu")] + \
      ["embed_%s" % f for f in FORMATS] + \
      ["rmsnorm", "rmsnorm_planes", "norm_rope", "kv_write", "atencion", "swiglu", "geglu", "escalar", "suma_esc", "moe_topk", "moe_comb", "gemv", "dec_attn",
       "dec_attn_comb", "argmax", "argmax_fin", "repack_q2k", "repack_q3k", "repack_q4k", "repack_q5k", "repack_q6k", "repack_q8", "repack_iq4nl", "fill_u32", "dequant",
       "copy_f4", "read_f4", "moe_gate_up_q4k", "moe_gate_up_q6k", "moe_down_q4k", "moe_down_q6k", "penalizar",
       "topk_cand", "moe_group"] + ["matmul_%s_eg" % f for f in FORMATS] + \
      ["matmul_%s_t_swiglu" % f for f in ("q2k", "q3k", "q4k", "q5k", "q6k")]


def test_op_table(built):
    lib = capi.load_library()
    ids = [lib.qp_op_id(n.encode()) for n in OPS]
    assert min(ids) >= 0 and len(set(ids)) == len(ids)
    assert lib.qp_op_id(b"matmul_iq2xs_1") == -1 and lib.qp_op_id(b"") == -1 and lib.qp_op_id(None) == -1
    assert lib.qp_op_id(b"matmul_q8_t_swiglu") == -1  # the fused gate/up/SwiGLU matmul is for K-quants only


def test_ops_used_by_the_js_host_exist(built):
    import re
    used = set()
    for f in ("transformer.js", "weights.js"):
        src = open(os.path.join(JS, f)).read()
        used |= set(re.findall(r"['\"]((?:matmul|embed)_[a-z0-9_]+|rmsnorm(?:_planes)?|norm_rope|kv_write|atencion|swiglu|"
                               r"moe_topk|moe_comb|moe_group|moe_(?:gate_up|down)_|gemv|dec_attn(?:_comb)?|argmax(?:_fin)?|"
                               r"repack_q[2-68]k?|fill_u32)['\"]", src))
    # names built by concatenation in the host: matmul_<fmt>_<suffix> and embed_<fmt>
    assert used, "no op names found"
    lib = capi.load_library()
    assert all(lib.qp_op_id(n.encode()) >= 0 for n in used if not n.endswith("_")), used


def test_calls_before_init_fail_with_a_message(built):
    # a fresh process: nothing initialised; every device call must return an error code, not crash
    script = r"""
import ctypes as C, json, sys
sys.path.insert(0, %r)
from quipullm_amd import capi
L = capi.load_library()
h = C.c_uint64()
rc = [L.qp_alloc(16, C.byref(h)), L.qp_sync(), L.qp_free(1), L.qp_graph_begin(),
      L.qp_dispatch(L.qp_op_id(b"rmsnorm"), None, 0, None, 0, 1, 1, 1)]
buf = C.create_string_buffer(256)
L.qp_last_error(buf, 256)
print(json.dumps({"rc": rc, "err": buf.value.decode(), "bad_buf": L.qp_last_error(None, 0)}))
""" % ROOT
    rc, out, err = run([sys.executable, "-c", script], timeout=120, env={"HIP_VISIBLE_DEVICES": "-1"})
    assert rc == 0, err[-2000:]
    r = json.loads(out.strip().splitlines()[-1])
    assert all(x != 0 for x in r["rc"]), r
    assert "init" in r["err"].lower() and r["bad_buf"] != 0


def test_uniform_packing():
    b = capi.uniform([("u", 7), ("f", 1.5), ("u", -1)])
    assert len(b) == 16
    assert np.frombuffer(b, np.uint32)[0] == 7 and np.frombuffer(b, np.float32)[1] == 1.5
    assert np.frombuffer(b, np.uint32)[2] == 0xFFFFFFFF and np.frombuffer(b, np.uint32)[3] == 0
    assert len(capi.uniform([("u", 1)] * 5)) == 32
    assert capi.dim2(65535) == (65535, 1) and capi.dim2(65536) == (32768, 2)
    gx, gy = capi.dim2(10 ** 6)
    assert gx <= 65535 and gx * gy >= 10 ** 6


def test_device_layout_sizes():
    assert capi.device_bytes(capi.Q4_K, 14336, 4096) == 14336 * 16 * 144
    assert capi.device_bytes(capi.Q6_K, 4096, 4096) == 4096 * 16 * 210
    assert capi.device_bytes(capi.Q8_0, 64, 2048) == 64 * 64 * 34
    assert capi.device_bytes(capi.IQ4_NL, 64, 2048) == capi.gguf_bytes(capi.IQ4_NL, 64, 2048) == 64 * 64 * 18
    assert capi.device_bytes(capi.F32, 3, 5) == 60
    assert capi.gguf_bytes(capi.Q3_K, 8, 512) == 8 * 2 * 110 and capi.device_bytes(capi.Q3_K, 8, 512) == 8 * 2 * 112
    assert capi.device_bytes(capi.Q2_K, 8, 512) == capi.gguf_bytes(capi.Q2_K, 8, 512) == 8 * 2 * 84


# ------------------------------------------------------------------------------------------------ N-API addon + JS
def test_napi_addon_loads_and_exports(built):
    r = node("const a = require(%r); console.log(JSON.stringify(Object.keys(a).sort()));" % build.NAPI)
    want = {"init", "info", "alloc", "free", "upload", "download", "copy", "sync", "opId", "dispatch", "graphBegin",
            "graphEnd", "graphLaunch", "graphFree", "eventCreate", "eventRecord", "eventElapsed", "eventFree",
            "bytesUsed", "lost"}
    assert want <= set(r), sorted(want - set(r))


def test_napi_op_ids_match_the_c_abi(built):
    names = json.dumps(OPS)
    r = node("const a = require(%r); console.log(JSON.stringify(%s.map(function (n) { return a.opId(n); })));"
             % (build.NAPI, names))
    lib = capi.load_library()
    assert r == [lib.qp_op_id(n.encode()) for n in OPS]


def test_js_packing_matches_python():
    vals = [["u", 3], ["f", -2.25], ["u", 4294967295], ["f", 1e-5], ["u", 0x12345678]]
    r = node("const g = require(%r); console.log(JSON.stringify(Array.from(g.empaquetar(%s))));"
             % (os.path.join(JS, "gpu.js"), json.dumps(vals)))
    assert bytes(r) == capi.uniform([tuple(v) for v in vals])


def test_js_gguf_reader_matches_python(models_dir):
    from oracle.oracle import GGUF
    path = synth.ensure_model("mini_qwen3moe_q4k", models_dir)
    r = node("""
const g = require(%r);
const m = g.leerGGUF(%r);
const t = {};
for (const x of m.tensors) t[x.nombre] = [x.tipo, x.dims.map(Number), Number(x.offset), x.bytes];
const kv = {};
for (const k of Object.keys(m.kv)) { const v = m.kv[k]; kv[k] = (typeof v === 'bigint') ? Number(v) : (Array.isArray(v) ? v.length : v); }
console.log(JSON.stringify({t: t, kv: kv, data: m.data_start}));
""" % (os.path.join(JS, "gguf.js"), path))
    g = GGUF(path)
    assert r["data"] == g.data_start
    assert set(r["t"]) == set(g.tensors)
    for name, t in g.tensors.items():
        tipo, dims, off, nbytes = r["t"][name]
        assert tipo == t["tipo"] and dims == list(t["dims"]) and nbytes == t["bytes"], name
        assert off == t["offset"], name
    for k, v in g.kv.items():
        want = len(v) if isinstance(v, list) else v
        got = r["kv"][k]
        assert (abs(got - want) <= 1e-6 * abs(want)) if isinstance(want, float) else got == want, k


def test_js_sampler_greedy_and_penalties():
    r = node("""
const s = require(%r);
const out = {};
out.tie = s.argmax(new Float32Array([1, 3, 3, 2]));
out.nan = s.argmax(new Float32Array([NaN, 0.5, NaN, 0.25]));
out.neg = s.argmax(new Float32Array([-5, -1, -3]));
const m = new s.Muestreador({temperature: 0, repeat_penalty: 2.0, frequency_penalty: 0.5, presence_penalty: 0.25});
const lg = new Float32Array([4, -2, 3.5, 1]);
out.pick = m.elegir(lg, [0, 0, 1]);
out.lg = Array.from(lg);
out.greedy = new s.Muestreador({temperature: 0}).esVoraz();
out.notGreedy = new s.Muestreador({temperature: 0, repeat_penalty: 1.1}).esVoraz();
const st = new s.Muestreador({temperature: 0.8});
out.stochastic = !st.esVoraz() && st.usaCandidatosDispositivo(32000) && !st.usaCandidatosDispositivo(40) &&
  !new s.Muestreador({temperature: 0.8, top_k: 0}).usaCandidatosDispositivo(32000) &&
  new s.Muestreador({temperature: 0.8, top_k: 128}).usaCandidatosDispositivo(151936) &&
  !new s.Muestreador({temperature: 0.8, top_k: 128}).usaCandidatosDispositivo(262144);
console.log(JSON.stringify(out));
""" % os.path.join(JS, "sampling.js"))
    assert r["tie"] == 1 and r["nan"] == 1 and r["neg"] == 1
    # token 0 (seen twice): 4 / 2 - (2 * 0.5 + 0.25) = 0.75; token 1 (once): -2 * 2 - (0.5 + 0.25) = -4.75
    assert r["lg"] == [0.75, -4.75, 3.5, 1.0] and r["pick"] == 2
    assert r["greedy"] and not r["notGreedy"] and r["stochastic"]


def test_js_rope_table_matches_double_power():
    r = node("const t = require(%r); const o = {};"
             "for (const b of [10000, 500000, 1000000]) for (const n of [64, 128]) o[b + ':' + n] = Array.from(t.tablaRope(b, n));"
             "console.log(JSON.stringify(o));" % os.path.join(JS, "transformer.js"))
    for key, vals in r.items():
        base, nrot = (int(x) for x in key.split(":"))
        ex = (np.float32(-2.0) * np.arange(nrot // 2, dtype=np.float32)) / np.float32(nrot)
        want = np.power(np.float64(base), ex.astype(np.float64)).astype(np.float32)
        np.testing.assert_array_equal(np.array(vals, np.float32), want)


def test_js_moe_grouping_falls_back_past_the_job_limit():
    """Grouping by expert (moe_group + matmul_*_eg) is chosen only when the batch's jobs fit moe_group's 16-bit
    lists (batch x experts used <= 65535) and there are at most 256 experts; otherwise the per-job expert path."""
    r = node("const t = require(%r); console.log(JSON.stringify(["
             "t.agrupable(true, 2048, 8, 128), t.agrupable(true, 8191, 8, 128), t.agrupable(true, 8192, 8, 128),"
             "t.agrupable(true, 512, 8, 257), t.agrupable(false, 512, 8, 128)]));" % os.path.join(JS, "transformer.js"))
    assert r == [True, True, False, False, False]


def test_js_registry():
    r = node("""
const e = require(%r);
const reg = e.cargarRegistro();
const o = {};
for (const a of Object.keys(reg)) o[a] = [reg[a].manifiesto.id, reg[a].manifiesto.options || {}];
console.log(JSON.stringify(o));
""" % os.path.join(JS, "engine.js"))
    assert set(r) >= {"llama", "qwen3", "qwen3moe"}
    assert r["qwen3moe"][1].get("rope") == "neox" and r["qwen3"][1].get("rope") == "neox"
    assert r["llama"][1].get("rope", "norm") == "norm"


# ------------------------------------------------------------------------------------------------ bench contract
def test_bench_refuses_more_than_one_gpu():
    rc, out, err = run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], timeout=120)
    assert rc == 2 and "one GPU" in err and out.strip() == ""


def test_hip_flags_disable_packed_fp32():
    f = build.HIP_FLAGS
    i = f.index("-packed-fp32-ops")
    assert f[i - 1] == "-Xclang" and f[i - 2] == "-target-feature" and "--offload-arch=gfx950" in f


def test_timeline_summary(tmp_path):
    """The profiling build's record files, made up here: two launches of 3 and 2 workgroups."""
    from quipullm_amd import timeline
    p = str(tmp_path / "tl.bin")
    raw = np.zeros((2, timeline.SLOTS, 4), np.uint32)
    base = (1 << 32) - 50                                   # the 32-bit stamps wrap inside the step
    for wg, (a, b) in enumerate([(0, 300), (10, 320), (20, 310)]):
        raw[0, wg] = [(base + a) % (1 << 32), (base + b) % (1 << 32), 0, 0x80000000 | wg]
    for wg, (a, b) in enumerate([(420, 600), (430, 650)]):
        raw[1, wg] = [(base + a) % (1 << 32), (base + b) % (1 << 32), 0, 0x80000003]
    raw.tofile(p)
    json.dump([["gemv_a", 3, 1, 1, 256], ["dec_attn", 2, 1, 1, 256]], open(p + ".json", "w"))
    recs = timeline.launches(*timeline.load(p)[:2])
    assert [d["wgs"] for d in recs] == [3, 2]
    assert recs[0]["span"] == pytest.approx(3.2) and recs[0]["gap"] == 0.0
    assert recs[1]["gap"] == pytest.approx(1.0) and recs[1]["span"] == pytest.approx(2.3)
    assert recs[1]["wg_max"] == pytest.approx(2.2) and recs[0]["xccs"] == 3
    txt = timeline.report(p)
    assert "sum of gaps 1.0 us" in txt and "first start to last end 6.5 us" in txt
