// quipu_napi.node: Node.js binding of the C ABI in include/quipu.h (N-API 6+, so it loads in Node 12).
//
// Device buffers, graphs and events are BigInt handles.  Every nonzero status of the C ABI becomes a thrown
// JavaScript Error whose message is qp_last_error() (the reference engine raises Error objects the same way,
// web/js/engine.js:136-149).
#define NAPI_VERSION 6
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "quipu.h"

namespace {

#define NAPI_OK(call)                                                  \
    do {                                                               \
        if ((call) != napi_ok) {                                       \
            napi_throw_error(env, nullptr, "quipu: N-API call failed"); \
            return nullptr;                                            \
        }                                                              \
    } while (0)

napi_value throw_qp(napi_env env, int rc, const char* what) {
    char msg[600];
    char err[512];
    qp_last_error(err, sizeof err);
    snprintf(msg, sizeof msg, "%s: %s (status %d)", what, err[0] ? err : "error", rc);
    napi_throw_error(env, nullptr, msg);
    return nullptr;
}

#define QP(call, what)                                   \
    do {                                                 \
        int rc_ = (call);                                \
        if (rc_ != 0) return throw_qp(env, rc_, what);   \
    } while (0)

struct Args {
    napi_value v[8];
    size_t n = 8;
};

bool get_args(napi_env env, napi_callback_info info, Args& a, size_t need) {
    if (napi_get_cb_info(env, info, &a.n, a.v, nullptr, nullptr) != napi_ok) return false;
    if (a.n < need) {
        napi_throw_type_error(env, nullptr, "quipu: missing arguments");
        return false;
    }
    return true;
}

bool to_u64(napi_env env, napi_value v, uint64_t* out) {
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_bigint) {
        bool lossless;
        return napi_get_value_bigint_uint64(env, v, out, &lossless) == napi_ok;
    }
    if (t == napi_number) {
        double d;
        if (napi_get_value_double(env, v, &d) != napi_ok) return false;
        *out = (uint64_t)d;
        return true;
    }
    if (t == napi_null || t == napi_undefined) {
        *out = 0;
        return true;
    }
    return false;
}

bool to_u32(napi_env env, napi_value v, uint32_t* out) {
    uint64_t x;
    if (!to_u64(env, v, &x)) return false;
    *out = (uint32_t)x;
    return true;
}

// Pointer and byte length of a TypedArray, DataView, Buffer or ArrayBuffer.
bool bytes_of(napi_env env, napi_value v, void** data, size_t* len) {
    bool is;
    if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
        napi_typedarray_type tt;
        size_t n, off;
        napi_value ab;
        if (napi_get_typedarray_info(env, v, &tt, &n, data, &ab, &off) != napi_ok) return false;
        size_t es = 1;
        switch (tt) {
        case napi_int16_array: case napi_uint16_array: es = 2; break;
        case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
        case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
        default: es = 1;
        }
        *len = n * es;
        return true;
    }
    if (napi_is_dataview(env, v, &is) == napi_ok && is) {
        napi_value ab;
        size_t off;
        return napi_get_dataview_info(env, v, len, data, &ab, &off) == napi_ok;
    }
    if (napi_is_arraybuffer(env, v, &is) == napi_ok && is) return napi_get_arraybuffer_info(env, v, data, len) == napi_ok;
    return false;
}

napi_value big(napi_env env, uint64_t x) {
    napi_value r;
    NAPI_OK(napi_create_bigint_uint64(env, x, &r));
    return r;
}
napi_value num(napi_env env, double x) {
    napi_value r;
    NAPI_OK(napi_create_double(env, x, &r));
    return r;
}
napi_value undef(napi_env env) {
    napi_value r;
    napi_get_undefined(env, &r);
    return r;
}

napi_value Init(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 0)) return nullptr;
    uint32_t dev = 0;
    if (a.n > 0) to_u32(env, a.v[0], &dev);
    QP(qp_init((int)dev), "qp_init");
    return undef(env);
}

napi_value Info(napi_env env, napi_callback_info info) {
    char buf[1024];
    QP(qp_info(buf, sizeof buf), "qp_info");
    napi_value r;
    NAPI_OK(napi_create_string_utf8(env, buf, NAPI_AUTO_LENGTH, &r));
    return r;
}

napi_value Alloc(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    uint64_t n, h = 0;
    if (!to_u64(env, a.v[0], &n)) return throw_qp(env, QP_E_ARG, "alloc: size");
    QP(qp_alloc(n, &h), "qp_alloc");
    return big(env, h);
}

napi_value Free(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    uint64_t h;
    if (!to_u64(env, a.v[0], &h)) return throw_qp(env, QP_E_ARG, "free: handle");
    QP(qp_free(h), "qp_free");
    return undef(env);
}

// upload(handle, offset, bytes)
napi_value Upload(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    uint64_t h, off;
    void* p;
    size_t n;
    if (!to_u64(env, a.v[0], &h) || !to_u64(env, a.v[1], &off) || !bytes_of(env, a.v[2], &p, &n))
        return throw_qp(env, QP_E_ARG, "upload: arguments");
    QP(qp_upload(h, off, p, n), "qp_upload");
    return undef(env);
}

// download(handle, offset, into)
napi_value Download(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    uint64_t h, off;
    void* p;
    size_t n;
    if (!to_u64(env, a.v[0], &h) || !to_u64(env, a.v[1], &off) || !bytes_of(env, a.v[2], &p, &n))
        return throw_qp(env, QP_E_ARG, "download: arguments");
    QP(qp_download(p, h, off, n), "qp_download");
    return undef(env);
}

// copy(dst, dstOff, src, srcOff, n)
napi_value Copy(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 5)) return nullptr;
    uint64_t d, doff, s, soff, n;
    if (!to_u64(env, a.v[0], &d) || !to_u64(env, a.v[1], &doff) || !to_u64(env, a.v[2], &s) ||
        !to_u64(env, a.v[3], &soff) || !to_u64(env, a.v[4], &n))
        return throw_qp(env, QP_E_ARG, "copy: arguments");
    QP(qp_copy(d, doff, s, soff, n), "qp_copy");
    return undef(env);
}

napi_value Sync(napi_env env, napi_callback_info info) {
    QP(qp_sync(), "qp_sync");
    return undef(env);
}

napi_value OpId(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    char name[128];
    size_t n;
    if (napi_get_value_string_utf8(env, a.v[0], name, sizeof name, &n) != napi_ok)
        return throw_qp(env, QP_E_ARG, "opId: name");
    return num(env, qp_op_id(name));
}

// dispatch(op, uniformBytes, BigUint64Array bufs, gx, gy, gz)
napi_value Dispatch(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 6)) return nullptr;
    uint32_t op, gx, gy, gz;
    void *u = nullptr, *b = nullptr;
    size_t un = 0, bn = 0;
    if (!to_u32(env, a.v[0], &op) || !bytes_of(env, a.v[1], &u, &un) || !bytes_of(env, a.v[2], &b, &bn) ||
        !to_u32(env, a.v[3], &gx) || !to_u32(env, a.v[4], &gy) || !to_u32(env, a.v[5], &gz))
        return throw_qp(env, QP_E_ARG, "dispatch: arguments");
    QP(qp_dispatch((int)op, u, (uint32_t)un, (const uint64_t*)b, (uint32_t)(bn / 8), gx, gy, gz), "qp_dispatch");
    return undef(env);
}

napi_value GraphBegin(napi_env env, napi_callback_info info) {
    QP(qp_graph_begin(), "qp_graph_begin");
    return undef(env);
}
napi_value GraphEnd(napi_env env, napi_callback_info info) {
    uint64_t g;
    QP(qp_graph_end(&g), "qp_graph_end");
    return big(env, g);
}
napi_value GraphLaunch(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    uint64_t g, times = 1;
    if (!to_u64(env, a.v[0], &g)) return throw_qp(env, QP_E_ARG, "graphLaunch: handle");
    if (a.n > 1) to_u64(env, a.v[1], &times);
    for (uint64_t i = 0; i < times; i++) QP(qp_graph_launch(g), "qp_graph_launch");
    return undef(env);
}
napi_value GraphFree(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    uint64_t g;
    if (!to_u64(env, a.v[0], &g)) return throw_qp(env, QP_E_ARG, "graphFree: handle");
    QP(qp_graph_free(g), "qp_graph_free");
    return undef(env);
}
napi_value EventCreate(napi_env env, napi_callback_info info) {
    uint64_t e;
    QP(qp_event_create(&e), "qp_event_create");
    return big(env, e);
}
napi_value EventRecord(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    uint64_t e;
    if (!to_u64(env, a.v[0], &e)) return throw_qp(env, QP_E_ARG, "eventRecord: handle");
    QP(qp_event_record(e), "qp_event_record");
    return undef(env);
}
napi_value EventElapsed(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 2)) return nullptr;
    uint64_t e0, e1;
    if (!to_u64(env, a.v[0], &e0) || !to_u64(env, a.v[1], &e1)) return throw_qp(env, QP_E_ARG, "eventElapsed");
    float ms = 0;
    QP(qp_event_elapsed(e0, e1, &ms), "qp_event_elapsed");
    return num(env, ms);
}
napi_value EventFree(napi_env env, napi_callback_info info) {
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    uint64_t e;
    if (!to_u64(env, a.v[0], &e)) return throw_qp(env, QP_E_ARG, "eventFree: handle");
    QP(qp_event_free(e), "qp_event_free");
    return undef(env);
}
napi_value BytesUsed(napi_env env, napi_callback_info info) { return num(env, (double)qp_bytes_used()); }
napi_value Lost(napi_env env, napi_callback_info info) {
    napi_value r;
    NAPI_OK(napi_get_boolean(env, qp_lost() != 0, &r));
    return r;
}

napi_value Register(napi_env env, napi_value exports) {
    struct F {
        const char* name;
        napi_callback cb;
    } fns[] = {{"init", Init},
               {"info", Info},
               {"alloc", Alloc},
               {"free", Free},
               {"upload", Upload},
               {"download", Download},
               {"copy", Copy},
               {"sync", Sync},
               {"opId", OpId},
               {"dispatch", Dispatch},
               {"graphBegin", GraphBegin},
               {"graphEnd", GraphEnd},
               {"graphLaunch", GraphLaunch},
               {"graphFree", GraphFree},
               {"eventCreate", EventCreate},
               {"eventRecord", EventRecord},
               {"eventElapsed", EventElapsed},
               {"eventFree", EventFree},
               {"bytesUsed", BytesUsed},
               {"lost", Lost}};
    for (const F& f : fns) {
        napi_value fn;
        NAPI_OK(napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn));
        NAPI_OK(napi_set_named_property(env, exports, f.name, fn));
    }
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Register)
