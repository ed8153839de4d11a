// libquipu: HIP runtime, code-object loader and the named-op table behind include/quipu.h.
//
// The op table maps quipullm's per-op dispatch interface (op name + uniform struct P + binding list, as
// web/js/gpu.js's grupo()/despachar() build it) onto this backend's gfx950 kernels.  Each handler validates
// the bindings, builds the kernel's argument block (qp_args.h) and launches it with hipModuleLaunchKernel on
// the library's stream.  Launch shapes are chosen here, not taken from the reference's dispatch sizes.
#include "../../include/quipu.h"

#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "qp_args.h"
#include "qp_scratch.h"

namespace {

thread_local std::string g_err;
bool g_init = false;
std::atomic<int> g_lost{0};
int g_device = 0;
hipStream_t g_stream = nullptr;
hipModule_t g_mod = nullptr;
std::mutex g_mu;
std::unordered_map<uint64_t, uint64_t> g_allocs;  // address -> bytes
uint64_t g_bytes = 0;
bool g_capturing = false;
bool g_noalloc = false;    // inside qp_dispatch_noalloc: the prefill workspace is the fixed scratch array
uint64_t g_scratch = 0;    // its device address on this device (qp_scratch.hip)
long g_fail_alloc = -1, g_fail_launch = -1;  // QP_FAIL_ALLOC / QP_FAIL_LAUNCH: fail the Nth call (1-based)
long g_n_alloc = 0, g_n_launch = 0;
std::string g_summary, g_arch;
int g_cus = 0;
uint64_t g_hbm = 0;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    if (e == hipErrorIllegalAddress || e == hipErrorLaunchFailure || e == hipErrorECCNotCorrectable ||
        e == hipErrorAssert)
        g_lost = 1;
    return fail((int)e, "HIP %s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

#define HIPCHK(expr, what)                               \
    do {                                                 \
        hipError_t e_ = (expr);                          \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

#define NEED_INIT()                                                             \
    do {                                                                        \
        if (!g_init) return fail(QP_E_NOT_INIT, "qp_init has not succeeded"); \
        if (g_lost) return fail(QP_E_NOT_INIT, "device lost");                 \
    } while (0)

// ------------------------------------------------------------------------------------------------ kernels
enum Kid {
#define K(name) K_##name,
#include "qp_kernel_list.inc"
#undef K
    K_COUNT
};
const char* kNames[] = {
#define K(name) "qp_" #name,
#include "qp_kernel_list.inc"
#undef K
};
hipFunction_t g_fn[K_COUNT];

#ifdef QP_TIMELINE
// Timeline builds: each launch captured into a graph gets a slot (tseq) in the kernels' record array; the kinds
// whose kernels record take it in their argument block.
struct TlLaunch {
    int k;
    uint32_t gx, gy, gz, block;
};
std::vector<TlLaunch> g_tl;
template <class A> void tl_tag(A&, uint32_t) {}
void tl_tag(QpGemvArgs& a, uint32_t v) { a.tseq = v; }
void tl_tag(QpDecAttnArgs& a, uint32_t v) { a.tseq = v; }
void tl_tag(QpDecCombArgs& a, uint32_t v) { a.tseq = v; }
void tl_tag(QpDecBlockArgs& a, uint32_t v) { a.tseq = v; }
void tl_tag(QpArgmaxFinArgs& a, uint32_t v) { a.tseq = v; }
void tl_tag(QpEmbedArgs& a, uint32_t v) { a.tseq = v; }
void tl_tag(QpMoeArgs& a, uint32_t v) { a.tseq = v; }
void tl_tag(QpRouterArgs& a, uint32_t v) { a.tseq = v; }
#endif

template <class A>
int launch(Kid k, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block, uint32_t lds, const A& args0) {
    if (g_fail_launch > 0 && ++g_n_launch == g_fail_launch)
        return fail(QP_E_INJECTED, "injected launch failure (QP_FAIL_LAUNCH=%ld)", g_fail_launch);
    if (gx == 0 || gy == 0 || gz == 0) return 0;
#ifdef QP_TIMELINE
    A args = args0;
    if (g_capturing && g_tl.size() < 420) {
        g_tl.push_back({(int)k, gx, gy, gz, block});
        tl_tag(args, (uint32_t)g_tl.size());
    }
#else
    const A& args = args0;
#endif
    void* params[] = {(void*)&args};
    HIPCHK(hipModuleLaunchKernel(g_fn[k], gx, gy, gz, block, 1, 1, lds, g_stream, params, nullptr), kNames[k]);
    return 0;
}

uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }
uint32_t grid_cap(uint64_t n_threads) {
    uint64_t g = (n_threads + 255) / 256;
    if (g > 4096) g = 4096;
    return g ? (uint32_t)g : 1u;
}

// ------------------------------------------------------------------------------------------------ op context
struct Ctx {
    const uint8_t* u;
    uint32_t usize;
    const uint64_t* b;
    uint32_t nb;
    uint32_t gx, gy, gz;
    uint32_t U(int i) const {
        if ((uint32_t)(i * 4 + 4) > usize) return 0;
        uint32_t v;
        memcpy(&v, u + i * 4, 4);
        return v;
    }
    float F(int i) const {
        uint32_t v = U(i);
        float f;
        memcpy(&f, &v, 4);
        return f;
    }
    uint64_t U64(int lo) const { return (uint64_t)U(lo) | ((uint64_t)U(lo + 1) << 32); }
    uint64_t B(uint32_t i) const { return i < nb ? b[i] : 0; }
};

int need_bufs(const Ctx& c, uint32_t n, const char* op) {
    if (c.nb < n) return fail(QP_E_ARG, "%s: %u bindings after the uniform expected, got %u", op, n, c.nb);
    return 0;
}

int fmt_of(const char* s) {
    if (!strcmp(s, "q4k")) return QP_Q4_K;
    if (!strcmp(s, "q5k")) return QP_Q5_K;
    if (!strcmp(s, "q3k")) return QP_Q3_K;
    if (!strcmp(s, "q2k")) return QP_Q2_K;
    if (!strcmp(s, "q6k")) return QP_Q6_K;
    if (!strcmp(s, "q8")) return QP_Q8_0;
    if (!strcmp(s, "iq4nl")) return QP_IQ4_NL;
    if (!strcmp(s, "f32")) return QP_F32;
    return -1;
}

bool is_kq(int fmt) {
    return fmt == QP_Q2_K || fmt == QP_Q3_K || fmt == QP_Q4_K || fmt == QP_Q5_K || fmt == QP_Q6_K;
}
// The planar formats (bound as two buffers: quants, then the f16 scales after them) and their quant bytes per block.
bool planar(int fmt) { return fmt == QP_Q8_0 || fmt == QP_IQ4_NL; }
uint32_t planar_qbytes(int fmt) { return fmt == QP_Q8_0 ? 32 : 16; }
// index of a K-quant format in the kernel tables: Q4_K, Q5_K, Q6_K, Q3_K, Q2_K
int kq_index(int fmt) { return fmt == QP_Q5_K ? 1 : fmt == QP_Q6_K ? 2 : fmt == QP_Q3_K ? 3 : fmt == QP_Q2_K ? 4 : 0; }

int check_k(int fmt, uint32_t K, const char* op) {
    if (is_kq(fmt) && K % 256)
        return fail(QP_E_ARG, "%s: K=%u is not a multiple of 256", op, K);
    if (planar(fmt) && K % 32) return fail(QP_E_ARG, "%s: K=%u is not a multiple of 32", op, K);
    if (fmt == QP_F32 && K % 16) return fail(QP_E_ARG, "%s: K=%u is not a multiple of 16", op, K);
    if (K == 0 || K > 15360) return fail(QP_E_ARG, "%s: K=%u outside 1..15360", op, K);
    return 0;
}

// Planar bindings (qs, ds) must be the two planes of one device tensor: ds == qs + NB * (32 for Q8_0, 16 for IQ4_NL).
int planes(int fmt, uint64_t qs, uint64_t ds, uint64_t nb, const char* op) {
    if (ds != qs + nb * planar_qbytes(fmt)) return fail(QP_E_ARG, "%s: ds binding is not the scale plane of qs", op);
    return 0;
}

bool getenv_flag(const char* name) {
    const char* e = getenv(name);
    return e && *e && strcmp(e, "0") != 0;
}

int default_r(int fmt) {
    static int env = -2;
    if (env == -2) {
        const char* e = getenv("QP_GEMV_R");
        env = e ? atoi(e) : -1;
    }
    if (env == 1 || env == 2 || env == 4 || env == 8) return env;
    return 2;
}

Kid gemv_kid(int fmt, int R) {  // the generic kernels (Q8_0, IQ4_NL, F32)
    int f = fmt == QP_Q8_0 ? 0 : fmt == QP_IQ4_NL ? 1 : 2;
    int r = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : 3;
    static const Kid t[3][4] = {{K_gemv_q8_r1, K_gemv_q8_r2, K_gemv_q8_r4, K_gemv_q8_r8},
                                {K_gemv_iq4nl_r1, K_gemv_iq4nl_r2, K_gemv_iq4nl_r4, K_gemv_iq4nl_r8},
                                {K_gemv_f32_r1, K_gemv_f32_r2, K_gemv_f32_r4, K_gemv_f32_r8}};
    return t[f][r];
}

// LDS of the GEMV kernels: the K input floats plus up to K/64 * 4 group sums.
uint32_t gemv_lds(uint32_t K) { return K * 4 + K / 4; }

// Workgroups of kernel k that fit on the whole device at once (occupancy x CUs), cached per (kernel, LDS).
uint32_t resident_wgs(Kid k, uint32_t block, uint32_t lds) {
    static std::unordered_map<uint64_t, uint32_t> cache;
    const uint64_t key = ((uint64_t)k << 40) | ((uint64_t)block << 24) | lds;
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0;
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, g_fn[k], (int)block, lds) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    const uint32_t n = (uint32_t)per_cu * (uint32_t)(g_cus > 0 ? g_cus : 1);
    cache[key] = n;
    return n;
}

// ---- K-quant GEMV (Q4_K / Q6_K): one lane per super-block; a unit is R rows per lane times S = 64/nbp rows per
// load (nbp = blocks per row rounded up to a power of two).
uint32_t kq_nbp(uint32_t K) {
    uint32_t p = 1;
    while (p < K / 256) p <<= 1;
    return p;
}
uint32_t kq_lds(uint32_t K) { return (K / 256) * 65 * 16 + (K / 16) * 4; }
// device bytes of a K-quant tensor (Q3_K blocks padded to 112 bytes; Q6_K / Q2_K with their d arrays)
uint64_t kq_tensor_bytes(int fmt, uint64_t rows, uint32_t K) {
    static const uint32_t bpb[5] = {144, 176, 210, 112, 84};
    return rows * (K / 256) * bpb[kq_index(fmt)];
}

Kid kq_mix_kid(int R, bool x2) {
    static const Kid t[2][2] = {{K_gemv_mix_r1, K_gemv_mix_r1x2}, {K_gemv_mix_r2, K_gemv_mix_r2x2}};
    return t[R == 2][x2];
}

Kid kq_kid(int fmt, int R, bool x2, bool expert) {
    static const Kid t[2][5][2][2] = {
        {{{K_gemv_q4k_r1, K_gemv_q4k_r1x2}, {K_gemv_q4k_r2, K_gemv_q4k_r2x2}},
         {{K_gemv_q5k_r1, K_gemv_q5k_r1x2}, {K_gemv_q5k_r2, K_gemv_q5k_r2x2}},
         {{K_gemv_q6k_r1, K_gemv_q6k_r1x2}, {K_gemv_q6k_r2, K_gemv_q6k_r2x2}},
         {{K_gemv_q3k_r1, K_gemv_q3k_r1x2}, {K_gemv_q3k_r2, K_gemv_q3k_r2x2}},
         {{K_gemv_q2k_r1, K_gemv_q2k_r1x2}, {K_gemv_q2k_r2, K_gemv_q2k_r2x2}}},
        {{{K_gemv_exp_q4k_r1, K_gemv_exp_q4k_r1x2}, {K_gemv_exp_q4k_r2, K_gemv_exp_q4k_r2x2}},
         {{K_gemv_exp_q5k_r1, K_gemv_exp_q5k_r1x2}, {K_gemv_exp_q5k_r2, K_gemv_exp_q5k_r2x2}},
         {{K_gemv_exp_q6k_r1, K_gemv_exp_q6k_r1x2}, {K_gemv_exp_q6k_r2, K_gemv_exp_q6k_r2x2}},
         {{K_gemv_exp_q3k_r1, K_gemv_exp_q3k_r1x2}, {K_gemv_exp_q3k_r2, K_gemv_exp_q3k_r2x2}},
         {{K_gemv_exp_q2k_r1, K_gemv_exp_q2k_r1x2}, {K_gemv_exp_q2k_r2, K_gemv_exp_q2k_r2x2}}}};
    return t[expert ? 1 : 0][kq_index(fmt)][R == 2 ? 1 : 0][x2 ? 1 : 0];
}

int need_room(uint64_t p, uint64_t bytes, const char* op, const char* what);
// An argmax segment's partial maxima: one 8-byte entry per workgroup of the launch.
int amax_room(const QpGemvArgs& a, uint32_t grid) {
    for (uint32_t i = 0; i < a.nseg; i++)
        if (a.seg[i].mode == QP_GEMV_ARGMAX)
            return need_room(a.amax, 8ull * grid, "gemv", "the argmax partials (one entry per workgroup)");
    return 0;
}

// Units per segment, then the grid: one unit per wavefront, at most two workgroups per CU (the kernel strides
// over further units); max_wg caps it (the ARGMAX partials hold one entry per workgroup).
int run_gemv_kq(int fmt, QpGemvArgs& a, uint32_t max_wg, uint32_t* grid_out) {
    int R = 1;
    bool mixed = false;
    for (uint32_t i = 0; i < a.nseg; i++) {
        if (a.seg[i].mode == QP_GEMV_SWIGLU) R = 2;
        if (a.seg[i].fmt != a.seg[0].fmt) mixed = true;
    }
    const uint32_t S = 64 / kq_nbp(a.k);
    uint32_t total = 0;
    for (uint32_t i = 0; i < a.nseg; i++) {
        QpGemvSeg& s = a.seg[i];
        if (s.n == 0) return fail(QP_E_ARG, "gemv: empty segment %u", i);
        if (s.rows_total == 0) s.rows_total = s.row_base + s.n;
        if ((uint64_t)s.row_base + s.n > s.rows_total)
            return fail(QP_E_ARG, "gemv: segment %u rows %u..%u past the tensor's %u", i, s.row_base, s.row_base + s.n,
                        s.rows_total);
        if (kq_tensor_bytes((int)s.fmt, s.rows_total, a.k) >= (1ull << 31))
            return fail(QP_E_ARG, "gemv: tensor of segment %u is 2 GiB or larger", i);
        s.wg0 = total;  // first unit of the segment
        total += cdiv(s.n, (s.mode == QP_GEMV_SWIGLU ? 1 : R) * S);
    }
    a.total_wg = total;
    a.rows_per_wg = R * S;
    // rows of more than 8192 inputs without the fused norm: 512-thread workgroups sharing one input staging
    const bool wide = a.k > 8192 && R == 1 && !mixed && !a.norm_w;
    const uint32_t waves = wide ? 8 : 4;
    uint32_t grid = cdiv(total, waves);
    // (3, 4, 6 or 8 workgroups per CU measured slower: each workgroup stages the input once more)
    if (grid > 2 * (uint32_t)g_cus) grid = 2 * (uint32_t)g_cus;
    if (max_wg && grid > max_wg) grid = max_wg;
    if (grid) {
        // the fewest workgroups that give no wavefront more units than this grid does (gate/up of the 8B: 3584
        // units on 448 instead of 512 workgroups, two units each instead of one or two: decode +0.6%)
        const uint32_t k = cdiv(total, waves * grid);
        grid = cdiv(total, waves * k);
    }
    if (grid == 0) grid = 1;
    if (int e = amax_room(a, grid)) return e;
    if (grid_out) *grid_out = grid;
    if (wide) {
        static const Kid wide_kid[5] = {K_gemv_q4k_r1k2, K_gemv_q5k_r1k2, K_gemv_q6k_r1k2, K_gemv_q3k_r1k2,
                                        K_gemv_q2k_r1k2};
        return launch(wide_kid[kq_index(fmt)], grid, 1, 1, 512, kq_lds(a.k), a);
    }
    const Kid kid = mixed ? kq_mix_kid(R, a.k > 8192) : kq_kid((int)a.seg[0].fmt, R, a.k > 8192, false);
    return launch(kid, grid, 1, 1, 256, kq_lds(a.k), a);
}

// Lays out the segments' workgroups and launches the GEMV kernel of `fmt`.  max_wg caps the grid (the
// kernel grid-strides over the remaining row groups); 0 = one workgroup per row group.
int run_gemv(int fmt, QpGemvArgs& a, int R, uint32_t max_wg, uint32_t* grid_out) {
    if (int e = check_k(fmt, a.k, "gemv")) return e;
    if (is_kq(fmt)) return run_gemv_kq(fmt, a, max_wg, grid_out);
    uint32_t total = 0;
    for (uint32_t i = 0; i < a.nseg; i++) {
        QpGemvSeg& s = a.seg[i];
        if (s.n == 0) return fail(QP_E_ARG, "gemv: empty segment %u", i);
        if (s.mode == QP_GEMV_SWIGLU && R < 2) return fail(QP_E_ARG, "gemv: SwiGLU pairs need R >= 2");
        if (s.rows_total == 0) s.rows_total = s.row_base + s.n;
        const uint32_t outs = (s.mode == QP_GEMV_SWIGLU ? R / 2 : R) * 4;
        s.wg0 = total;
        total += cdiv(s.n, outs);
    }
    a.rows_per_wg = 4 * R;
    a.total_wg = total;
    const Kid kid = gemv_kid(fmt, R);
    const uint32_t lds = gemv_lds(a.k);
    if (!max_wg) max_wg = resident_wgs(kid, 256, lds);  // persistent: one wave of resident workgroups
    uint32_t grid = max_wg && max_wg < total ? max_wg : total;
    if (int e = amax_room(a, grid)) return e;
    if (grid_out) *grid_out = grid;
    return launch(kid, grid, 1, 1, 256, lds, a);
}

// ------------------------------------------------------------------------------------------------ reference ops
// matmul_<fmt>_1 (kquants.js:188-251, gpu.js:123-198): P{N,K,acc,tfijo}; [paso, w, x, y] (q8: [paso,qs,ds,x,y]).
int op_matmul_1(const Ctx& c, int fmt, const char* name) {
    const bool q8 = planar(fmt);
    if (int e = need_bufs(c, q8 ? 5 : 4, name)) return e;
    const uint32_t N = c.U(0), K = c.U(1), acc = c.U(2);
    if (int e = check_k(fmt, K, name)) return e;
    const uint64_t w = c.B(1);
    if (q8)
        if (int e = planes(fmt, c.B(1), c.B(2), (uint64_t)N * K / 32, name)) return e;
    QpGemvArgs a = {};
    a.nseg = 1;
    a.k = K;
    a.paso = c.B(0);
    a.x = c.B(q8 ? 3 : 2);
    a.seg[0].w = w;
    a.seg[0].y = c.B(q8 ? 4 : 3);
    a.seg[0].fmt = fmt;
    a.seg[0].n = N;
    a.seg[0].mode = acc ? QP_GEMV_ACC : QP_GEMV_STORE;
    a.seg[0].rows_total = N;
    return run_gemv(fmt, a, default_r(fmt), 0, nullptr);
}

// matmul_<fmt>_4 / matmul_<fmt>_t (prefill, kquants.js:188-251 nt=4 and 309-386): T tokens from paso.
// The library's scratch buffer for the prefill matmul (split input planes, split-K partials): grown on demand
// (the stream is drained before the old one is freed) and kept until the process ends.  Not while capturing.
uint64_t g_ws = 0, g_ws_bytes = 0;
uint32_t g_ws_gen = 0;  // counts the workspace's reallocations
int workspace(uint64_t bytes, uint64_t* out) {
    if (g_noalloc) {
        if (bytes > QP_SCRATCH_BYTES)
            return fail(QP_E_ARG, "qp_dispatch_noalloc: this matmul needs %llu bytes of workspace; the scratch holds %u "
                                  "(fewer tokens per call)", (unsigned long long)bytes, QP_SCRATCH_BYTES);
        *out = g_scratch;
        return 0;
    }
    if (bytes > g_ws_bytes) {
        if (g_capturing) return fail(QP_E_CAPTURE, "prefill workspace growth during graph capture");
        if (g_ws) {
            HIPCHK(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
            HIPCHK(hipFree((void*)g_ws), "hipFree");
            g_ws = 0;
            g_ws_bytes = 0;
        }
        void* p = nullptr;
        HIPCHK(hipMalloc(&p, bytes), "hipMalloc (prefill workspace)");
        g_ws = (uint64_t)p;
        g_ws_bytes = bytes;
        g_ws_gen++;
    }
    *out = g_ws;
    return 0;
}

// The input split into bf16 planes for the matrix-core matmuls.  reuse (the caller's word: x and paso hold what the
// previous prefill matmul in stream order read): the planes that matmul split are used again when they are still
// there (the same x, paso, K, planes and workspace allocation), else x is split.
struct SplitMemo {
    uint64_t x, xs, paso;
    uint32_t k, rows, mul, cap, gen;
    bool valid;
} g_split_memo = {};
// While a graph is captured nothing runs, so a split recorded then proves nothing about the planes' contents now,
// and a replay may overwrite them (the noalloc scratch is shared): the memo is neither used nor set during capture,
// and graph launches invalidate it.
// mul, cap: rows T * mul of x, at most cap (QpSplitArgs); 0: T rows.
int split_input(uint64_t x, uint64_t xs, uint64_t paso, uint32_t K, uint32_t rows, uint32_t tmax, bool reuse,
                uint32_t mul = 0, uint32_t cap = 0) {
    const SplitMemo& m = g_split_memo;
    if (reuse && !g_capturing && m.valid && m.x == x && m.xs == xs && m.paso == paso && m.k == K && m.rows == rows &&
        m.mul == mul && m.cap == cap && m.gen == g_ws_gen)
        return 0;
    QpSplitArgs sa = {x, xs, paso, K, rows, mul, cap};
    g_split_memo = {x, xs, paso, K, rows, mul, cap, g_ws_gen, false};
    if (int e = launch(K_split_bf16, grid_cap((uint64_t)tmax * K / 8), 1, 1, 256, 0, sa)) return e;
    g_split_memo.valid = !g_capturing;
    return 0;
}

int op_matmul_mt(const Ctx& c, int fmt, const char* name, uint32_t tokens_per_z) {
    const bool q8 = planar(fmt);
    if (int e = need_bufs(c, q8 ? 5 : 4, name)) return e;
    const uint32_t N = c.U(0), K = c.U(1), acc = c.U(2);
    if (int e = check_k(fmt, K, name)) return e;
    if (q8)
        if (int e = planes(fmt, c.B(1), c.B(2), (uint64_t)N * K / 32, name)) return e;
    QpGemmArgs a = {};
    a.w = c.B(1);
    a.x = c.B(q8 ? 3 : 2);
    a.y = c.B(q8 ? 4 : 3);
    a.paso = c.B(0);
    a.fmt = fmt;
    a.n = N;
    a.k = K;
    a.acc = acc;
    const uint32_t tmax = c.gz * tokens_per_z;
    // P[4] = 2 (x holds input planes) is read by the 256-token tiles only (below: K-quants, 256 tokens or more)
    const bool xplanes = c.U(4) == 2;
    if (xplanes && (!is_kq(fmt) || tmax < 256 || (g_capturing && !g_noalloc) || getenv_flag("QP_NO_MFMA")))
        return fail(QP_E_ARG, "%s: P[4] = 2 (x holds input planes) needs K-quant weights and a chunk of 256 tokens "
                              "or more on the matrix cores", name);
    if (tmax >= 64 && !getenv_flag("QP_NO_MFMA")) {
        // matrix cores: 128 x 128 tiles (the kernel reads T from paso; tiles past it exit)
        const Kid k = fmt == QP_Q4_K ? K_gemm_mfma_q4k : fmt == QP_Q6_K ? K_gemm_mfma_q6k
                    : fmt == QP_Q8_0 ? K_gemm_mfma_q8 : fmt == QP_IQ4_NL ? K_gemm_mfma_iq4nl : K_gemm_mfma_f32;
        uint32_t mt = cdiv(tmax, 128);
        uint32_t nt = cdiv(N, 128);
        if (!g_capturing || g_noalloc) {
            // x split into bf16 planes once (not in every weight tile's workgroup), and the K range split when the
            // tiles alone cannot occupy the CUs (a 128-row router at 2048 tokens is 16 tiles); partials summed in
            // order.  K-quants from 256 tokens on: 256-token tiles (one 512-thread workgroup per CU, K steps of 32
            // double-buffered in LDS) dequantize each weight tile half as often.
            // Q5_K, Q3_K and Q2_K have only the 256-token tiles
            const bool big = is_kq(fmt) && (tmax >= 256 || fmt == QP_Q5_K || fmt == QP_Q3_K || fmt == QP_Q2_K);
            if (big) mt = cdiv(tmax, 256);
            // 256 x 256 tiles when they alone occupy three quarters of the CUs, or half of them at K >= 8192 (where
            // splitting K in two costs little); measured at 2048 tokens: 14336 x 4096 789 vs 886 us, 6144 x 4096 375
            // vs 439, 4096 x 14336 917 vs 941, and 4096 x 2048 130 vs 121 against the 256 x 128 tiles.
            // QP_GEMM_TILES=wide / narrow forces one kind, for tests and comparisons.
            const char* tiles = getenv("QP_GEMM_TILES");
            const uint32_t wt = mt * cdiv(N, 256);
            const bool wide = big && (tiles && !strcmp(tiles, "wide") ? true
                                      : tiles && !strcmp(tiles, "narrow") ? false
                                      : 4 * wt >= 3 * (uint32_t)g_cus || (2 * wt >= (uint32_t)g_cus && K >= 8192));
            if (wide) nt = cdiv(N, 256);
            const uint32_t steps = K / 64, slots = (big ? 1 : 2) * (uint32_t)g_cus;
            uint32_t ns2 = 1;  // K splits, a power of two
            while (mt * nt * ns2 * 2 <= slots && steps / (ns2 * 2) >= 4) ns2 *= 2;
            a.rows = mt * (big ? 256 : 128);
            // the bf16 planes: 2 x 2 bytes per token row and input, K rounded up to whole 32-input chunks
            const uint64_t xs_bytes = 4ull * a.rows * ((K + 31) / 32 * 32);
            uint32_t ns;
            uint64_t ws_bytes;
            for (;;) {
                a.kchunk = ns2 > 1 ? cdiv(steps, ns2) * 64 : 0;  // whole 64-input steps (the 256-token tiles take 32)
                ns = ns2 > 1 ? cdiv(K, a.kchunk) : 1;
                ws_bytes = ns > 1 ? 4ull * ns * a.rows * N : 0;
                // the fixed scratch of qp_dispatch_noalloc: fewer K splits (down to none) until the partials fit
                if (!g_noalloc || ns2 == 1 || xs_bytes + ws_bytes <= QP_SCRATCH_BYTES) break;
                ns2 /= 2;
            }
            uint64_t ws = 0;
            const uint32_t xmode = c.U(4);
            if (xmode == 2) {
                // P[4] = 2: x holds the input planes already (matmul_<fmt>_t_swiglu with planes = 1 wrote them for
                // the same T), sized for 256-token tiles (big holds: checked above)
                if (K % 32) return fail(QP_E_ARG, "%s: input planes need K %% 32 == 0", name);
                if (int e = need_room(a.x, xs_bytes, name, "the input planes' buffer")) return e;
                if (ws_bytes)
                    if (int e = workspace(ws_bytes, &ws)) return e;
                a.xs = a.x;
                a.ws = ns > 1 ? ws : 0;
            } else {
                if (int e = workspace(xs_bytes + ws_bytes, &ws)) return e;
                a.xs = ws;
                a.ws = ns > 1 ? ws + xs_bytes : 0;
                // P[4] = 1: reuse the previous matmul's input planes (see split_input)
                if (int e = split_input(a.x, a.xs, a.paso, K, a.rows, tmax, xmode == 1)) return e;
            }
            if (wide) {
                static const Kid kw_of[5] = {K_gemm_mfma256w_q4k, K_gemm_mfma256w_q5k, K_gemm_mfma256w_q6k,
                                             K_gemm_mfma256w_q3k, K_gemm_mfma256w_q2k};
                if (int e = launch(kw_of[kq_index(fmt)], nt, mt, ns, 512, 2 * (256 + 256 + 256 + 256) * 40 * 2, a))
                    return e;
            } else if (big) {
                static const Kid kb_of[5] = {K_gemm_mfma256_q4k, K_gemm_mfma256_q5k, K_gemm_mfma256_q6k,
                                             K_gemm_mfma256_q3k, K_gemm_mfma256_q2k};
                const Kid kb = kb_of[kq_index(fmt)];
                if (int e = launch(kb, nt, mt, ns, 512, 2 * (256 + 256 + 128 + 128) * 40 * 2, a)) return e;
            } else if (int e = launch(k, nt, mt, ns, 256, 0, a)) {
                return e;
            }
            if (ns == 1) return 0;
            QpReduceArgs ra = {a.ws, a.y, a.paso, N, a.rows, ns, acc};
            return launch(K_gemm_reduce, grid_cap((uint64_t)tmax * N), 1, 1, 256, 0, ra);
        }
        if (fmt == QP_Q5_K || fmt == QP_Q3_K || fmt == QP_Q2_K)
            return launch(K_gemm_mt, cdiv(N, 64), cdiv(tmax, 64), 1, 256, 0, a);  // under capture
        return launch(k, nt, mt, 1, 256, 0, a);
    }
    return launch(K_gemm_mt, cdiv(N, 64), cdiv(tmax ? tmax : 1, 64), 1, 256, 0, a);
}

// matmul_<fmt>_t_swiglu: P{N, K, planes, xplanes}; [paso, w_gate, w_up, x, y]; y[t][n] = silu(x[t] . gate[n]) *
// (x[t] . up[n]) for the T tokens of paso (K-quants).  No counterpart in the reference, whose prompt pass runs
// matmul_<fmt>_t on the gate and up tensors and then swiglu (transformer.js:311-313): the same three results in one
// matrix-core launch (256-token tiles of 128 gate and 128 up rows), for prompt chunks of at least 256 tokens.  Same
// accumulation as matmul_<fmt>_t with 256 x 256 tiles.  Not while capturing a graph (the input planes may need a
// larger workspace).  planes = 1 (the third word; absent: 0): y receives the outputs as the input planes of the
// matmul that reads them next (matmul_<fmt>_t with P[4] = 2), the values qp_split_bf16 would make of the f32 rows,
// for R = 256 * ceil(T / 256) token rows and K = N: 4 R N bytes.  P[3] = 1: x holds its input as such planes
// (rmsnorm_planes), 4 R K bytes.
uint64_t tensor_bytes(int fmt, uint64_t rows, uint32_t K);
int need_room(uint64_t p, uint64_t bytes, const char* op, const char* what);
constexpr uint32_t kGluCntWords = 1024;  // split tiles of one launch at most (one arrival word each)
uint64_t g_glu_cnt = 0;                  // the arrival words, allocated on first use, kept until the process ends
int op_matmul_glu(const Ctx& c, int fmt, const char* name) {
    if (int e = need_bufs(c, 5, name)) return e;
    const uint32_t N = c.U(0), K = c.U(1);
    if (!is_kq(fmt)) return fail(QP_E_ARG, "%s: K-quant weights only", name);
    if (int e = check_k(fmt, K, name)) return e;
    if (N == 0) return fail(QP_E_ARG, "%s: N is 0", name);
    const uint32_t tmax = c.gz * 32;
    if (tmax < 256) return fail(QP_E_ARG, "%s: for prompt chunks of 256 tokens or more (grid z %u)", name, c.gz);
    if (g_capturing && !g_noalloc) return fail(QP_E_CAPTURE, "%s: not while capturing a graph", name);
    const uint64_t tb = tensor_bytes(fmt, N, K);
    if (int e = need_room(c.B(1), tb, name, "the gate tensor's buffer")) return e;
    if (int e = need_room(c.B(2), tb, name, "the up tensor's buffer")) return e;
    QpGemmArgs a = {};
    a.w = c.B(1);
    a.w2 = c.B(2);
    a.x = c.B(3);
    a.y = c.B(4);
    a.paso = c.B(0);
    a.fmt = fmt;
    a.n = N;
    a.k = K;
    const uint32_t mt = cdiv(tmax, 256), nt = cdiv(N, 128);
    a.rows = mt * 256;
    a.yplanes = c.U(2);
    if (a.yplanes > 1) return fail(QP_E_ARG, "%s: P[2] = %u (0: f32 rows, 1: input planes)", name, a.yplanes);
    if (a.yplanes) {
        if (N % 32) return fail(QP_E_ARG, "%s: the input planes need N %% 32 == 0 (N = %u)", name, N);
        if (int e = need_room(a.y, 4ull * a.rows * N, name, "the output planes' buffer")) return e;
    }
    // One workgroup per CU (the kernel takes the whole LDS), so the tiles run in rounds of g_cus.  When the last
    // round would leave at least half the CUs idle, its tiles run as K halves instead (two items each, the second to
    // finish adds the other's sums): 896 tiles of the 8B gate/up at 2048 tokens take 3.5 rounds' time, not 4.
    // Needs every XCD to get the same numbers of whole and split tiles and K halves of whole 64-input steps; not
    // under qp_dispatch_noalloc (the partials need workspace); QP_GLU_SPLIT=0 turns it off.
    const uint32_t tiles = mt * nt, C = g_cus > 0 ? (uint32_t)g_cus : 1u, rem = tiles % C;
    const char* sp = getenv("QP_GLU_SPLIT");
    const bool split = !g_noalloc && !(sp && !strcmp(sp, "0")) && tiles > C && rem > 0 && 2 * rem <= C &&
                       rem % 8 == 0 && (tiles - rem) % 8 == 0 && K % 128 == 0 && rem <= kGluCntWords;
    // P[3] = 1: x holds the input planes already (rmsnorm_planes wrote them for the same T)
    const bool xpl = c.U(3) == 1;
    const uint64_t planes = xpl ? 0 : 4ull * a.rows * K, part = split ? (uint64_t)rem * 2 * 512 * 128 * 4 : 0;
    if (xpl)
        if (int e = need_room(a.x, 4ull * a.rows * K, name, "the input planes' buffer")) return e;
    uint64_t ws = 0;
    if (planes + part)
        if (int e = workspace(planes + part, &ws)) return e;
    a.xs = xpl ? a.x : ws;
    if (!xpl)
        if (int e = split_input(a.x, a.xs, a.paso, K, a.rows, tmax, false)) return e;
    static const Kid kg_of[5] = {K_gemm_glu_q4k, K_gemm_glu_q5k, K_gemm_glu_q6k, K_gemm_glu_q3k, K_gemm_glu_q2k};
    const uint32_t lds = 2 * (256 + 256 + 256 + 256) * 40 * 2;
    if (!split) return launch(kg_of[kq_index(fmt)], nt, mt, 1, 512, lds, a);
    if (!g_glu_cnt) {
        // the arrival words: zero once, and every split tile's second arrival sets its word back to zero
        void* p = nullptr;
        HIPCHK(hipMalloc(&p, 4ull * kGluCntWords), "hipMalloc (split-tile counters)");
        HIPCHK(hipMemsetAsync(p, 0, 4ull * kGluCntWords, g_stream), "hipMemsetAsync");
        g_glu_cnt = (uint64_t)p;
    }
    a.tail = rem;
    a.mtiles = mt;
    a.ntiles = nt;
    a.part = ws + planes;
    a.cnt = g_glu_cnt;
    return launch(kg_of[kq_index(fmt)], tiles + rem, 1, 1, 512, lds, a);
}

// matmul_<fmt>_e (kquants.js:256-304, kds.js:110-186): P{N,K,acc,tfijo,E}; [paso, w, x, y, sel]
// (q8: [paso, qs, ds, x, y, sel]); jobs = gz.  E (the 5th word) sizes the planar formats' sub-arrays.
int op_matmul_e(const Ctx& c, int fmt, const char* name, bool swiglu) {
    const bool q8 = planar(fmt);
    const uint32_t nb = (q8 ? 6 : 5) + (swiglu ? 1 : 0);
    if (int e = need_bufs(c, nb, name)) return e;
    const uint32_t N = c.U(0), K = c.U(1), tfijo = c.U(3), E = c.U(4);
    if (int e = check_k(fmt, K, name)) return e;
    if (q8 && E == 0) return fail(QP_E_ARG, "%s: P.E (expert count) is 0", name);
    if (tfijo == 0) return fail(QP_E_ARG, "%s: tfijo is 0", name);
    if (q8)
        if (int e = planes(fmt, c.B(1), c.B(2), (uint64_t)E * N * K / 32, name)) return e;
    QpGemvExpArgs a = {};
    uint32_t i = 1;
    a.w = c.B(i++);
    if (q8) i++;
    if (swiglu) a.w2 = c.B(i++);
    a.x = c.B(i++);
    a.y = c.B(i++);
    a.sel = c.B(i++);
    a.paso = c.B(0);
    a.fmt = fmt;
    a.n = N;
    a.k = K;
    a.tfijo = tfijo;
    a.njobs_fixed = c.gz;
    a.mode = swiglu ? QP_GEMV_SWIGLU : QP_GEMV_STORE;
    a.n_exp = E;
    if (is_kq(fmt)) {
        if (E == 0) return fail(QP_E_ARG, "%s: P.E (expert count) is 0", name);
        if (kq_tensor_bytes(fmt, (uint64_t)E * N, K) >= (1ull << 31))
            return fail(QP_E_ARG, "%s: expert tensor is 2 GiB or larger", name);
        const int R = swiglu ? 2 : 1;
        const uint32_t units = cdiv(N, (swiglu ? 1 : R) * (64 / kq_nbp(K)));
        return launch(kq_kid(fmt, R, K > 8192, true), cdiv(units, 4), c.gz, 1, 256, kq_lds(K), a);
    }
    const int R = 4;
    const uint32_t outs = (swiglu ? R / 2 : R) * 4;
    const Kid k = fmt == QP_Q8_0 ? K_gemv_exp_q8_r4 : fmt == QP_IQ4_NL ? K_gemv_exp_iq4nl_r4 : K_gemv_exp_f32_r4;
    return launch(k, cdiv(N, outs), c.gz, 1, 256, gemv_lds(K), a);
}

// embed_<fmt> (kquants.js:481-504, gpu.js:585-618): P{D, rows}; [paso, w, ids, y] (q8: [paso,qs,ds,ids,y]).
int op_embed(const Ctx& c, int fmt, const char* name) {
    const bool q8 = planar(fmt);
    if (int e = need_bufs(c, q8 ? 5 : 4, name)) return e;
    QpEmbedArgs a = {};
    a.fmt = fmt;
    a.d = c.U(0);
    a.rows = c.U(1);
    if ((fmt == QP_Q6_K || q8) && a.rows == 0) return fail(QP_E_ARG, "%s: P.rows is 0", name);
    if (q8)
        if (int e = planes(fmt, c.B(1), c.B(2), (uint64_t)a.rows * a.d / 32, name)) return e;
    a.w = c.B(1);
    a.ids = c.B(q8 ? 3 : 2);
    a.y = c.B(q8 ? 4 : 3);
    a.paso = c.B(0);
    return launch(K_embed, c.gx ? (c.gx > 4096 ? 4096 : c.gx) : 1, 1, 1, 256, 0, a);
}

// rmsnorm (gpu.js:332-356): P{D, ultima, eps, z}; [paso, x, w, y]; gx rows.
int op_rmsnorm(const Ctx& c) {
    if (int e = need_bufs(c, 4, "rmsnorm")) return e;
    QpRmsArgs a = {};
    a.d = c.U(0);
    a.ultima = c.U(1);
    a.eps = c.F(2);
    a.paso = c.B(0);
    a.x = c.B(1);
    a.w = c.B(2);
    a.y = c.B(3);
    return launch(K_rmsnorm, a.ultima ? 1 : c.gx, 1, 1, 256, 0, a);
}

// rmsnorm_planes: P{D, eps}; [paso, x, w, xs]; grid ceil(T / 8).  No counterpart in the reference: its rmsnorm
// (gpu.js:332-356) of the T rows written as the bf16 input planes of the matmul that reads them next (matmul_<fmt>_t
// with P[4] = 2, matmul_<fmt>_t_swiglu with P[3] = 1; K-quants, T >= 256), for R = 256 ceil(T / 256) token rows:
// 4 R D bytes, D % 32 == 0, D <= 16384.  The planes are those the matmul's own split makes of rmsnorm's rows.  A
// workgroup takes 8 rows (4 above D = 4096, 2 above 8192), kept in LDS between its two passes.
int op_rmsnorm_planes(const Ctx& c) {
    if (int e = need_bufs(c, 4, "rmsnorm_planes")) return e;
    QpRmsPlanesArgs a = {};
    a.d = c.U(0);
    a.eps = c.F(1);
    a.paso = c.B(0);
    a.x = c.B(1);
    a.w = c.B(2);
    a.xs = c.B(3);
    if (!a.d || a.d % 32 || a.d > 16384)
        return fail(QP_E_ARG, "rmsnorm_planes: D=%u (a multiple of 32, at most 16384)", a.d);
    const uint32_t gx = c.gx ? c.gx : 1;  // ceil(T / 8)
    a.rows = cdiv(gx * 8, 256) * 256;
    if (int e = need_room(a.xs, 4ull * a.rows * a.d, "rmsnorm_planes", "the planes' buffer")) return e;
    // rows per workgroup (the rows stay in LDS, 4 * rw * (D + 4) bytes): up to D = 4096 two workgroups fit a CU
    // (2048 rows at D = 4096: 16.0 us with 4 rows, 19.1 with 8, 23.1 with 2)
    const uint32_t rw = a.d <= 2048 ? 8 : a.d <= 8192 ? 4 : 2;
    const Kid k = rw == 8 ? K_rmsnorm_planes : rw == 4 ? K_rmsnorm_planes4 : K_rmsnorm_planes2;
    return launch(k, gx * (8 / rw), 1, 1, 256, 4 * rw * (a.d + 4), a);
}

// norm_rope (gpu.js:394-444): P{hd, nh, usaNorm, neox, eps, base, nrot, z=esc bits}; [paso, v, w]; (nh, T).
int op_norm_rope(const Ctx& c) {
    if (int e = need_bufs(c, 3, "norm_rope")) return e;
    QpRopeArgs a = {};
    a.hd = c.U(0);
    a.nh = c.U(1);
    a.use_norm = c.U(2);
    a.neox = c.U(3);
    a.eps = c.F(4);
    a.base = c.F(5);
    a.nrot = c.U(6);
    a.esc = c.U(7) ? c.F(7) : 1.0f;
    if (a.hd > 256 || a.nrot > a.hd) return fail(QP_E_ARG, "norm_rope: hd=%u nrot=%u", a.hd, a.nrot);
    a.paso = c.B(0);
    a.v = c.B(1);
    a.w = c.B(2);
    // a fourth binding (not the reference's): the frequency table for this base and nrot, base^(-2j/nrot) rounded
    // once to float for j < nrot/2, so that no workgroup evaluates the powers
    a.freq = c.nb > 3 ? c.B(3) : 0;
    if (a.freq)
        if (int e = need_room(a.freq, 4ull * (a.nrot / 2), "norm_rope", "the frequency table")) return e;
    return launch(K_norm_rope, cdiv(a.nh, 4), cdiv(c.gy, 4), 1, 256, 0, a);  // four tokens per workgroup
}

// kv_write (gpu.js:447-466): P{kvd, cap, f16, rows}; [paso, k, v, kc, vc].  rows = cache slots (required).
int op_kv_write(const Ctx& c) {
    if (int e = need_bufs(c, 5, "kv_write")) return e;
    QpKvArgs a = {};
    a.kvd = c.U(0);
    a.cap = c.U(1);
    a.f16 = c.U(2);
    a.rows = c.U(3);
    if (!a.rows) return fail(QP_E_ARG, "kv_write: P.rows (cache slots) is 0");
    a.paso = c.B(0);
    a.k = c.B(1);
    a.v = c.B(2);
    a.kc = c.B(3);
    a.vc = c.B(4);
    // f16 cache, prompt chunks (the dispatch covers 64 tokens or more): tiles of 64 tokens x 64 channels, the tokens
    // the dispatch covers (x = ceil(T * kvd / 256))
    const uint64_t tcap = c.gx ? ((uint64_t)c.gx * 256 + a.kvd - 1) / a.kvd : 0;
    if (a.f16 && a.kvd % 4 == 0 && tcap >= 64)
        return launch(K_kv_write16, cdiv(a.kvd, 64), (uint32_t)((tcap + 63) / 64), 1, 256, 0, a);
    return launch(K_kv_write, c.gx ? (c.gx > 4096 ? 4096 : c.gx) : 1, 1, 1, 256, 0, a);
}

uint32_t attn_lds(uint32_t hd) {
    const uint32_t rows = 32, tk = 32;
    return 4 * (rows * hd + tk * (hd + 1) + tk * hd + rows * (tk + 1) + 3 * rows);
}

// atencion (gpu.js:467-539): P{hd, nh, nkv, swa, escala, cap, z1, z2, f16, rows}; [paso, q, kc, vc, o]; (nh, T).
// rows = cache slots (required).
int op_atencion(const Ctx& c) {
    if (int e = need_bufs(c, 5, "atencion")) return e;
    QpAttnArgs a = {};
    a.hd = c.U(0);
    a.nh = c.U(1);
    a.nkv = c.U(2);
    a.swa = c.U(3);
    a.scale = c.F(4);
    a.cap = c.U(5);
    if (c.U(6) || c.U(7)) return fail(QP_E_ARG, "atencion: bidirectional / non-causal modes are not supported");
    a.f16 = c.U(8);
    a.rows = c.U(9);
    if (!a.rows) return fail(QP_E_ARG, "atencion: P.rows (cache slots) is 0");
    if (a.hd != 64 && a.hd != 128) return fail(QP_E_ARG, "atencion: head_dim %u (64 or 128 supported)", a.hd);
    if (!a.nkv || a.nh % a.nkv || a.nh / a.nkv > 32)
        return fail(QP_E_ARG, "atencion: nh=%u nkv=%u", a.nh, a.nkv);
    a.paso = c.B(0);
    a.q = c.B(1);
    a.kc = c.B(2);
    a.vc = c.B(3);
    a.o = c.B(4);
    const uint32_t G = a.nh / a.nkv;
    // P[10] = 1 (an addition of this backend's): o receives the output as the bf16 input planes of the matmul that
    // reads it next (matmul_<fmt>_t with P[4] = 2: the same T, 256 ceil(T / 256) token rows, K = nh hd), the values
    // its own split would make of the f32 rows.  The two-group matrix-core path only.
    const bool oplanes = c.U(10) == 1;
    const bool mfma = a.f16 && !a.swa && !a.cap && (G == 1 || G == 2 || G == 4 || G == 8) && !getenv_flag("QP_NO_MFMA");
    if (oplanes) {
        if (!mfma || getenv_flag("QP_ATTN_RG1"))
            return fail(QP_E_ARG, "atencion: P[10] = 1 (output planes) needs the matrix-core path (f16 cache, no "
                                  "window or ring, groups of 1, 2, 4 or 8 query heads)");
        a.orows = cdiv(c.gy ? c.gy : 1, 256) * 256;
        if (int e = need_room(a.o, 4ull * a.orows * a.nh * a.hd, "atencion", "the output planes' buffer")) return e;
    }
    if (mfma) {
        // matrix-core path: a wavefront takes 16 rg / G tokens x G heads, a workgroup four wavefronts
        static const Kid km[2][4] = {{K_attn_mfma_h64_g1, K_attn_mfma_h64_g2, K_attn_mfma_h64_g4, K_attn_mfma_h64_g8},
                                     {K_attn_mfma_h128_g1, K_attn_mfma_h128_g2, K_attn_mfma_h128_g4,
                                      K_attn_mfma_h128_g8}};
        static const Kid km2[2][4] = {{K_attn_mfma2_h64_g1, K_attn_mfma2_h64_g2, K_attn_mfma2_h64_g4,
                                       K_attn_mfma2_h64_g8},
                                      {K_attn_mfma2_h128_g1, K_attn_mfma2_h128_g2, K_attn_mfma2_h128_g4,
                                       K_attn_mfma2_h128_g8}};
        const uint32_t gi = G == 1 ? 0 : G == 2 ? 1 : G == 4 ? 2 : 3;
        // two 16-row groups per wavefront sharing each key tile (measured: 8B prefill of 4096 tokens 201 -> 192 ms,
        // MoE 176 -> 160 ms), one token block per workgroup with its keys split over the four wavefronts;
        // QP_ATTN_RG1 keeps one group, two tiles in flight and four token blocks per workgroup, for comparisons
        const bool two = !getenv_flag("QP_ATTN_RG1");
        const uint32_t tpw = 16 * (two ? 2 : 1) / G;  // tokens per wavefront
        return launch((two ? km2 : km)[a.hd == 128][gi], a.nkv, cdiv(c.gy ? c.gy : 1, (two ? 1 : 4) * tpw), 1, 256, 0,
                      a);
    }
    const uint32_t qb = 32 / G;
    a.qb = qb;
    return launch(a.hd == 64 ? K_attn_hd64 : K_attn_hd128, a.nkv, cdiv(c.gy ? c.gy : 1, qb), 1, 256, attn_lds(a.hd),
                  a);
}

// swiglu (gpu.js:570-582): P{F}; [paso, g, u].
int op_swiglu(const Ctx& c) {
    if (int e = need_bufs(c, 3, "swiglu")) return e;
    QpSwigluArgs a = {};
    a.f = c.U(0);
    a.paso = c.B(0);
    a.g = c.B(1);
    a.u = c.B(2);
    return launch(K_swiglu, c.gx ? (c.gx > 4096 ? 4096 : c.gx) : 1, 1, 1, 256, 0, a);
}

// geglu (gpu.js:318-330): P{F}; [paso, g, u].
int op_geglu(const Ctx& c) {
    if (int e = need_bufs(c, 3, "geglu")) return e;
    QpSwigluArgs a = {};
    a.f = c.U(0);
    a.paso = c.B(0);
    a.g = c.B(1);
    a.u = c.B(2);
    return launch(K_geglu, c.gx ? (c.gx > 4096 ? 4096 : c.gx) : 1, 1, 1, 256, 0, a);
}

// escalar (gpu.js:635-646): P{D, escala}; [paso, x].  suma_esc (gpu.js:648-660): P{D, escala}; [paso, x, t].
int op_scale(const Ctx& c, bool suma) {
    const char* name = suma ? "suma_esc" : "escalar";
    if (int e = need_bufs(c, suma ? 3 : 2, name)) return e;
    QpScaleArgs a = {};
    a.d = c.U(0);
    a.s = c.F(1);
    a.paso = c.B(0);
    a.x = c.B(1);
    a.t = suma ? c.B(2) : 0;
    return launch(suma ? K_suma_esc : K_escalar, c.gx ? (c.gx > 4096 ? 4096 : c.gx) : 1, 1, 1, 256, 0, a);
}

// moe_topk (kds.js:191-221): P{E, k, norm, escala}; [paso, lg, sel, wts]; ceil(T/64) groups.
int op_moe_topk(const Ctx& c) {
    if (int e = need_bufs(c, 4, "moe_topk")) return e;
    QpTopkArgs a = {};
    a.e = c.U(0);
    a.k = c.U(1);
    a.norm = c.U(2);
    a.scale = c.F(3);
    if (a.e == 0 || a.e > 1024 || a.k == 0 || a.k > a.e) return fail(QP_E_ARG, "moe_topk: E=%u k=%u", a.e, a.k);
    a.paso = c.B(0);
    a.lg = c.B(1);
    a.sel = c.B(2);
    a.wts = c.B(3);
    return launch(K_moe_topk, (c.gx ? c.gx : 1) * 64, 1, 1, 256, 0, a);
}

// moe_gate_up_<fmt> / moe_down_<fmt>: the MoE FFN of one decode token in two launches (the reference runs
// moe_topk, matmul_*_e for gate and up, swiglu, matmul_*_e for down and moe_comb; deepseek2.js:375-386).
// P{n, k, e, kused, eps, scale, norm}; binding 0 (paso) is not read: one token
//   gate/up: [paso, gate, up, x, norm_w|0, logits, h, sel, wts]: routes from logits [e], h[j] = silu(gate . xn) *
//            (up . xn) over experts sel[j], xn = rmsnorm(x) * norm_w; writes sel, wts [kused]
//   down:    [paso, down, h, x, sel, wts]: x += sum_j wts[j] * down_{sel[j]} . h[j]
int op_moe(const Ctx& c, int fmt, bool down, const char* name) {
    if (int e = need_bufs(c, down ? 6 : 9, name)) return e;
    QpMoeArgs a = {};
    a.n = c.U(0);
    a.k = c.U(1);
    a.e = c.U(2);
    a.kused = c.U(3);
    a.eps = c.F(4);
    a.scale = c.F(5);
    a.norm = c.U(6);
    if (int e = check_k(fmt, a.k, name)) return e;
    if (a.n == 0) return fail(QP_E_ARG, "%s: n is 0", name);
    if (a.e == 0 || a.e > 256) return fail(QP_E_ARG, "%s: %u experts (this kernel routes 1..256)", name, a.e);
    if (a.kused == 0 || a.kused > a.e || a.kused > 64)
        return fail(QP_E_ARG, "%s: %u experts used of %u", name, a.kused, a.e);
    const uint32_t K = down ? a.kused * a.k : a.k;
    if (K > 16384) return fail(QP_E_ARG, "%s: %u inputs per row (at most 16384)", name, K);
    if (kq_tensor_bytes(fmt, (uint64_t)a.e * a.n, a.k) >= (1ull << 31))
        return fail(QP_E_ARG, "%s: expert tensor is 2 GiB or larger", name);
    const int q6 = fmt == QP_Q6_K, x2 = K > 8192;
    const uint32_t units = cdiv(a.n, 64 / kq_nbp(K));
    a.w = c.B(1);
    if (down) {
        static const Kid kd[2][2] = {{K_moe_down_q4k_x1, K_moe_down_q4k_x2}, {K_moe_down_q6k_x1, K_moe_down_q6k_x2}};
        a.x = c.B(2);
        a.y = c.B(3);
        a.sel = c.B(4);
        a.wts = c.B(5);
        uint32_t grid = cdiv(units, 4);
        if (grid > 2 * (uint32_t)g_cus) grid = 2 * (uint32_t)g_cus;
        return launch(kd[q6][x2], grid, 1, 1, 256, kq_lds(K), a);
    }
    static const Kid kg[2][2] = {{K_moe_gate_up_q4k_x1, K_moe_gate_up_q4k_x2},
                                 {K_moe_gate_up_q6k_x1, K_moe_gate_up_q6k_x2}};
    a.w2 = c.B(2);
    a.x = c.B(3);
    a.norm_w = c.B(4);
    a.logits = c.B(5);
    a.y = c.B(6);
    a.sel = c.B(7);
    a.wts = c.B(8);
    a.presel = c.U(7);  // P[7] = 1: sel holds the routing (moe_router), the logits are not read
    return launch(kg[q6][x2], cdiv(units, 4), a.kused, 1, 256, kq_lds(K), a);
}

// moe_router: P{e, k, kused, nw, eps, scale, norm}; [paso, w (f32 [e][k]), x, norm_w|0, logits, sel, wts, cnt].
// The router GEMV of one token with the fused RMSNorm and the routing in one launch (QpRouterArgs); cnt: a library
// buffer of at least 8 bytes (the arrival counter, then the error word), zero at allocation, used by this op only.
uint64_t buf_room(uint64_t p);
int op_moe_router(const Ctx& c) {
    if (int e = need_bufs(c, 8, "moe_router")) return e;
    QpRouterArgs a = {};
    a.e = c.U(0);
    a.k = c.U(1);
    a.kused = c.U(2);
    a.nw = c.U(3);
    a.eps = c.F(4);
    a.scale = c.F(5);
    a.norm = c.U(6);
    if (a.e == 0 || a.e > 256) return fail(QP_E_ARG, "moe_router: %u experts (1..256)", a.e);
    if (a.kused == 0 || a.kused > a.e || a.kused > 64)
        return fail(QP_E_ARG, "moe_router: %u experts used of %u", a.kused, a.e);
    if (a.k == 0 || a.k % 4 || a.k > 16384) return fail(QP_E_ARG, "moe_router: k=%u (a multiple of 4, at most 16384)", a.k);
    const uint32_t per_xcd = g_cus >= 8 ? (uint32_t)g_cus / 8 : 1;
    if (a.nw == 0 || (a.nw & (a.nw - 1)) || a.nw > 2 * per_xcd)
        return fail(QP_E_ARG, "moe_router: nw=%u (a power of two, at most two per CU of an XCD)", a.nw);
    a.w = c.B(1);
    a.x = c.B(2);
    a.norm_w = c.B(3);
    a.logits = c.B(4);
    a.sel = c.B(5);
    a.wts = c.B(6);
    a.cnt = c.B(7);
    if (!a.w || !a.x || !a.logits || !a.sel || !a.wts || !a.cnt)
        return fail(QP_E_ARG, "moe_router: a required binding is missing");
    if (buf_room(a.cnt) < 8) return fail(QP_E_ARG, "moe_router: cnt must be a library buffer of at least 8 bytes");
    struct Need { uint64_t p, n; const char* what; } need[] = {
        {a.w, 4ull * a.e * a.k, "the router weights"}, {a.x, 4ull * a.k, "x"}, {a.norm_w, 4ull * a.k, "norm_w"},
        {a.logits, 4ull * a.e, "logits"}, {a.sel, 4ull * a.kused, "sel"}, {a.wts, 4ull * a.kused, "wts"}};
    for (const Need& n : need)
        if (n.p)
            if (int e = need_room(n.p, n.n, "moe_router", n.what)) return e;
    // LDS: the staged input (k floats), then the routing's keys, partial ranks and slots (896 floats)
    return launch(K_moe_router, 8, a.nw, 1, 256, 4 * (a.k > 896 ? a.k : 896), a);
}

// moe_comb (kds.js:224-240): P{D, k}; [paso, x, de, wts].
int op_moe_comb(const Ctx& c) {
    if (int e = need_bufs(c, 4, "moe_comb")) return e;
    QpCombArgs a = {};
    a.d = c.U(0);
    a.k = c.U(1);
    a.paso = c.B(0);
    a.x = c.B(1);
    a.de = c.B(2);
    a.wts = c.B(3);
    return launch(K_moe_comb, c.gx ? (c.gx > 4096 ? 4096 : c.gx) : 1, 1, 1, 256, 0, a);
}

// Bytes from p to the end of the library buffer that holds it (0: not inside one).
uint64_t buf_room(uint64_t p) {
    for (const auto& kv : g_allocs)
        if (p >= kv.first && p < kv.first + kv.second) return kv.first + kv.second - p;
    return 0;
}

// moe_group (kds.js:491-516): P{E, n}; [paso, sel, lst, off]; one workgroup.  lst[off[e] .. off[e+1]) = the jobs
// i < T*n with sel[i] == e, in increasing order.
int op_moe_group(const Ctx& c) {
    if (int e = need_bufs(c, 4, "moe_group")) return e;
    QpMoeGroupArgs a = {};
    a.n_exp = c.U(0);
    a.n = c.U(1);
    a.paso = c.B(0);
    a.sel = c.B(1);
    a.lst = c.B(2);
    a.off = c.B(3);
    if (a.n_exp == 0 || a.n_exp > 256 || a.n == 0) return fail(QP_E_ARG, "moe_group: E=%u n=%u", a.n_exp, a.n);
    const uint64_t rs = buf_room(a.sel), rl = buf_room(a.lst), ro = buf_room(a.off);
    if (!rs || !rl || !ro) return fail(QP_E_ARG, "moe_group: sel, lst and off must be library buffers");
    if (ro < 4ull * (a.n_exp + 1)) return fail(QP_E_ARG, "moe_group: off holds %llu bytes, E+1 entries need %u",
                                               (unsigned long long)ro, 4 * (a.n_exp + 1));
    const uint64_t ns = (rs < rl ? rs : rl) / 4;
    if (ns > 65535) return fail(QP_E_ARG, "moe_group: sel and lst hold %llu jobs; at most 65535", (unsigned long long)ns);
    a.nsel = (uint32_t)ns;
    return launch(K_moe_group, 1, 1, 1, 256, 256 * a.n_exp * 2 + 4 + 4 * a.n_exp, a);
}

// matmul_<fmt>_eg (kquants.js:386-460, the expert matmul grouped by expert): P{N, K, acc, tfijo};
// [paso, w, x, y, lst, off] (q8: [paso, qs, ds, x, y, lst, off]), dispatched as (ceil(N/64), E, ceil(T/32)).
// y[j][r] (+)= W[e*N + r] . x[j / tfijo] for every job j of expert e (lst / off from moe_group), on the matrix
// cores: 128 jobs x 128 rows per workgroup, E * ceil(32*gz / 128) job tiles.
int op_matmul_eg(const Ctx& c, int fmt, const char* name) {
    const bool q8 = planar(fmt);
    if (int e = need_bufs(c, q8 ? 7 : 6, name)) return e;
    const uint32_t N = c.U(0), K = c.U(1), acc = c.U(2), tfijo = c.U(3), E = c.gy, tz = c.gz;
    if (int e = check_k(fmt, K, name)) return e;
    if (N == 0 || tfijo == 0 || E == 0 || tz == 0)
        return fail(QP_E_ARG, "%s: N=%u tfijo=%u, dispatch y (experts)=%u z=%u", name, N, tfijo, E, tz);
    if (q8)
        if (int e = planes(fmt, c.B(1), c.B(2), (uint64_t)E * N * K / 32, name)) return e;
    if (is_kq(fmt) && kq_tensor_bytes(fmt, (uint64_t)E * N, K) >= (1ull << 31))
        return fail(QP_E_ARG, "%s: expert tensor is 2 GiB or larger", name);
    QpGemmArgs a = {};
    uint32_t i = 1;
    a.w = c.B(i++);
    if (q8) i++;
    a.x = c.B(i++);
    a.y = c.B(i++);
    a.lst = c.B(i++);
    a.off = c.B(i++);
    a.paso = c.B(0);
    a.fmt = fmt;
    a.n = N;
    a.k = K;
    a.acc = acc;
    a.wrows = E * N;
    a.n_exp = E;
    a.tfijo = tfijo;
    const uint64_t rx = buf_room(a.x), ry = buf_room(a.y), rl = buf_room(a.lst), ro = buf_room(a.off);
    if (!rx || !ry || !rl || !ro) return fail(QP_E_ARG, "%s: x, y, lst and off must be library buffers", name);
    if (ro < 4ull * (E + 1)) return fail(QP_E_ARG, "%s: off holds fewer than E+1 = %u entries", name, E + 1);
    auto cap = [](uint64_t v) { return (uint32_t)(v > 0xffffffffull ? 0xffffffffull : v); };
    a.xrows = cap(rx / (4ull * K));
    a.yrows = cap(ry / (4ull * N));
    a.nlst = cap(rl / 4);
    a.tpe = cdiv(32 * tz, 128);
    if ((uint64_t)E * a.tpe > 65535) return fail(QP_E_ARG, "%s: %u experts x %u job tiles", name, E, a.tpe);
    // P[4] = m (not a reference word; absent: 0): x holds m rows per token (1: gate/up, whose job j reads token
    // row j / tfijo; the top-k count: down, job rows), and its first T * m rows are split into bf16 planes once
    // (row-major: a tile gathers rows), which every tile then copies instead of loading and splitting f32 rows (the
    // same planes: the sums are bit-equal).  P[5] = 1: the previous matmul split the same x (see split_input).  Not while capturing a graph or
    // under qp_dispatch_noalloc (the planes need the workspace): there x is split in the tiles as without P[4].
    const uint32_t m = c.U(4);
    if (m && !g_capturing && !g_noalloc) {
        if (K % 8) return fail(QP_E_ARG, "%s: input planes need K %% 8 == 0", name);
        const uint64_t r64 = (uint64_t)32 * tz * m;
        a.rows = (uint32_t)(r64 < a.xrows ? r64 : a.xrows);
        uint64_t ws = 0;
        if (int e = workspace(4ull * a.rows * ((K + 31) / 32 * 32), &ws)) return e;
        a.xs = ws;
        if (int e = split_input(a.x, a.xs, a.paso, K, a.rows, a.rows, c.U(5) == 1, m, a.xrows)) return e;
        a.xrows = a.rows;  // a job whose row the planes do not hold stores nothing (an m too small for tfijo)
    }
    const Kid k = fmt == QP_Q4_K ? K_gemm_mfma_q4k : fmt == QP_Q6_K ? K_gemm_mfma_q6k
                : fmt == QP_Q5_K ? K_gemm_mfma_q5k : fmt == QP_Q3_K ? K_gemm_mfma_q3k
                : fmt == QP_Q2_K ? K_gemm_mfma_q2k : fmt == QP_Q8_0 ? K_gemm_mfma_q8
                : fmt == QP_IQ4_NL ? K_gemm_mfma_iq4nl : K_gemm_mfma_f32;
    return launch(k, cdiv(N, 128), E * a.tpe, 1, 256, 0, a);
}

// ------------------------------------------------------------------------------------------------ backend ops
// Formats a format word may name: f32, Q8_0 and IQ4_NL (planar) and the K-quants (row chunk planes).
bool known_fmt(int f) { return f == QP_F32 || planar(f) || is_kq(f); }

// Bytes of a device tensor of `rows` rows of K elements in the layout of fmt.
uint64_t tensor_bytes(int fmt, uint64_t rows, uint32_t K) {
    if (is_kq(fmt)) return kq_tensor_bytes(fmt, rows, K);
    if (planar(fmt)) return rows * (K / 32) * (planar_qbytes(fmt) + 2);
    return rows * K * 4ull;
}

// A library buffer bound at p must hold `bytes` from p (pointers the library did not allocate are not checked).
int need_room(uint64_t p, uint64_t bytes, const char* op, const char* what) {
    const uint64_t r = buf_room(p);
    if (r && r < bytes)
        return fail(QP_E_ARG, "%s: %s holds %llu bytes from its binding, %llu needed", op, what,
                    (unsigned long long)r, (unsigned long long)bytes);
    return 0;
}

// gemv: fused one-token GEMV over up to 4 same-format segments.
// P{nseg, K, eps, last_row, R, max_wg, fmt, 0, then per segment {mode | seg_fmt << 8, n, row_base, rows_total}};
// seg_fmt 0 means fmt; Q4_K and Q6_K segments may share a launch.
// [paso, x, norm_w|0, amax|0, then per segment w, w2|0, y].
int op_gemv(const Ctx& c) {
    const uint32_t nseg = c.U(0);
    if (nseg == 0 || nseg > QP_MAX_SEG) return fail(QP_E_ARG, "gemv: nseg=%u", nseg);
    if (int e = need_bufs(c, 4 + 3 * nseg, "gemv")) return e;
    QpGemvArgs a = {};
    a.nseg = nseg;
    a.k = c.U(1);
    a.eps = c.F(2);
    a.last_row = c.U(3);
    int R = (int)c.U(4);
    if (R == 0) R = default_r((int)c.U(6));
    if (R != 1 && R != 2 && R != 4 && R != 8) return fail(QP_E_ARG, "gemv: R=%d", R);
    const uint32_t max_wg = c.U(5);
    const int fmt = (int)c.U(6);
    if (!known_fmt(fmt)) return fail(QP_E_ARG, "gemv: format %d is not a device layout (f32 0, Q8_0 8, K-quants 10..14, IQ4_NL 20)", fmt);
    a.paso = c.B(0);
    a.x = c.B(1);
    a.norm_w = c.B(2);
    a.amax = c.B(3);
    for (uint32_t i = 0; i < nseg; i++) {
        QpGemvSeg& s = a.seg[i];
        const uint32_t mw = c.U(8 + 4 * i);
        s.mode = mw & 0xffu;
        s.n = c.U(9 + 4 * i);
        s.row_base = c.U(10 + 4 * i);
        s.rows_total = c.U(11 + 4 * i);
        s.fmt = (mw >> 8) & 0xffu ? (mw >> 8) & 0xffu : (uint32_t)fmt;  // per-segment format (0: the launch's)
        if (s.fmt != (uint32_t)fmt && !((s.fmt == QP_Q4_K || s.fmt == QP_Q6_K) && (fmt == QP_Q4_K || fmt == QP_Q6_K)))
            return fail(QP_E_ARG, "gemv: segment %u format %u cannot share a launch with format %d", i, s.fmt, fmt);
        s.w = c.B(4 + 3 * i);
        s.w2 = c.B(5 + 3 * i);
        s.y = c.B(6 + 3 * i);
        if (s.mode > QP_GEMV_ARGMAX) return fail(QP_E_ARG, "gemv: mode %u", s.mode);
        if (s.mode == QP_GEMV_SWIGLU && !s.w2) return fail(QP_E_ARG, "gemv: SwiGLU segment without w2");
        if (s.mode == QP_GEMV_ARGMAX && !a.amax) return fail(QP_E_ARG, "gemv: argmax segment without amax");
        if (s.row_base + (uint64_t)s.n > s.rows_total)
            return fail(QP_E_ARG, "gemv: segment %u rows %u..%u past the tensor's %u", i, s.row_base,
                        s.row_base + s.n, s.rows_total);
        const uint64_t tb = tensor_bytes((int)s.fmt, s.rows_total, a.k);
        if (int e = need_room(s.w, tb, "gemv", "a segment's weight buffer")) return e;
        if (s.mode == QP_GEMV_SWIGLU)
            if (int e = need_room(s.w2, tb, "gemv", "a segment's second weight buffer")) return e;
    }
    return run_gemv(fmt, a, R, max_wg, nullptr);
}

// dec_attn: split-K decode attention with fused q/k norm, RoPE and KV append; partials merged by dec_attn_comb.
// P{hd, nh, nkv, nsplit, scale, eps, base, esc, nrot, neox, f16, rows}; [paso, q, k, v, kc, vc, qnorm|0,
// knorm|0, part_o, part_ml (, freq)].  rows = cache slots (required); freq = the RoPE frequency table
// base^(-2j/nrot) rounded to float, [nrot/2] (optional: computed in the kernel when absent).
int op_dec_attn(const Ctx& c) {
    if (int e = need_bufs(c, 10, "dec_attn")) return e;
    QpDecAttnArgs a = {};
    a.hd = c.U(0);
    a.nh = c.U(1);
    a.nkv = c.U(2);
    a.nsplit = c.U(3);
    a.scale = c.F(4);
    a.eps = c.F(5);
    a.base = c.F(6);
    a.esc = c.U(7) ? c.F(7) : 1.0f;
    a.nrot = c.U(8);
    a.neox = c.U(9);
    a.f16 = c.U(10);
    a.rows = c.U(11);
    if (!a.rows) return fail(QP_E_ARG, "dec_attn: P.rows (cache slots) is 0");
    if (a.hd != 64 && a.hd != 128) return fail(QP_E_ARG, "dec_attn: head_dim %u", a.hd);
    if (a.nrot > a.hd || a.nrot % 2) return fail(QP_E_ARG, "dec_attn: nrot=%u", a.nrot);
    const uint32_t G = a.nkv ? a.nh / a.nkv : 0;
    if (!a.nkv || a.nh % a.nkv || (G != 1 && G != 2 && G != 4 && G != 8))
        return fail(QP_E_ARG, "dec_attn: nh=%u nkv=%u (group of 1, 2, 4 or 8 query heads)", a.nh, a.nkv);
    if (!a.nsplit || a.nsplit > 1024) return fail(QP_E_ARG, "dec_attn: nsplit=%u (1..1024)", a.nsplit);
    a.paso = c.B(0);
    a.q = c.B(1);
    a.k = c.B(2);
    a.v = c.B(3);
    a.kc = c.B(4);
    a.vc = c.B(5);
    a.qnorm = c.B(6);
    a.knorm = c.B(7);
    a.part_o = c.B(8);
    a.part_ml = c.B(9);
    a.freq = c.B(10);
    // P[12] = 1: the merge of the splits in the same launch (bindings 11: o [nh][hd], 12: the counters, 8 x 128
    // bytes, then the error word: zero before the first launch; the kernel leaves the counters zero and sets the
    // error word only when a column's workgroups ran on more than one XCD), for nkv * gsplit <= 8
    const bool merged = c.U(12) != 0;
    // P[13]: columns per KV head of the merged form (1, 2, 4 or 8; each takes G / gsplit query heads)
    a.gsplit = merged && c.U(13) ? c.U(13) : 1;
    if (a.gsplit != 1 && a.gsplit != 2 && a.gsplit != 4 && a.gsplit != 8)
        return fail(QP_E_ARG, "dec_attn: gsplit=%u (1, 2, 4 or 8)", a.gsplit);
    if (G % a.gsplit) return fail(QP_E_ARG, "dec_attn: gsplit=%u does not divide the group of %u query heads", a.gsplit, G);
    if (merged) {
        if (a.nkv * a.gsplit > 8)
            return fail(QP_E_ARG, "dec_attn: the merged form takes at most 8 columns (nkv=%u x gsplit=%u)", a.nkv,
                        a.gsplit);
        a.att = c.nb > 11 ? c.B(11) : 0;
        a.cnt = c.nb > 12 ? c.B(12) : 0;
        if (!a.att || !a.cnt) return fail(QP_E_ARG, "dec_attn: the merged form needs bindings 11 (o) and 12 (counters)");
        if (!buf_room(a.cnt) || buf_room(a.cnt) < 8 * 128 + 4)
            return fail(QP_E_ARG, "dec_attn: the counters must be a library buffer of at least 1028 bytes");
        if (int e = need_room(a.att, 4ull * a.nh * a.hd, "dec_attn", "the merged output")) return e;
    }
    const uint32_t Gc = G / a.gsplit;  // query heads per column
    const uint32_t gi = Gc == 1 ? 0 : Gc == 2 ? 1 : Gc == 4 ? 2 : 3;
    static const Kid kt[2][2][4] = {
        {{K_dec_attn_h64_f32_g1, K_dec_attn_h64_f32_g2, K_dec_attn_h64_f32_g4, K_dec_attn_h64_f32_g8},
         {K_dec_attn_h64_f16_g1, K_dec_attn_h64_f16_g2, K_dec_attn_h64_f16_g4, K_dec_attn_h64_f16_g8}},
        {{K_dec_attn_h128_f32_g1, K_dec_attn_h128_f32_g2, K_dec_attn_h128_f32_g4, K_dec_attn_h128_f32_g8},
         {K_dec_attn_h128_f16_g1, K_dec_attn_h128_f16_g2, K_dec_attn_h128_f16_g4, K_dec_attn_h128_f16_g8}}};
    const Kid k = kt[a.hd == 128][a.f16 ? 1 : 0][gi];
    // LDS floats: kn, vn [hd] | RoPE sines, cosines [hd/2] each | q/k norm weights [hd] each | wavefront partials
    // 4*G*hd + 64 (also holds q [G][hd] before, and the merge's weights and share sums after)
    // the merge: weights G*nsplit, denominators, then 256 float4 of share sums (aligned to 16 bytes)
    const uint32_t region = 4 * Gc * a.hd + 64, mreg = ((Gc * a.nsplit + 8 + 3) & ~3u) + 4 * 256;
    const uint32_t lds = 4 * (a.hd * 5 + (merged && region < mreg ? mreg : region));
    return launch(k, merged ? 8 : a.nkv, a.nsplit, 1, 256, lds, a);
}

// dec_attn_block: the attention block of one decode token in one launch (QpDecBlockArgs): Q/K/V GEMV with the
// fused RMSNorm, split-K attention with q/k norm, RoPE and the KV append, and the split merge into att.
// P{hd, nh, nkv, ns, scale, eps, base, esc, nrot, neox, rows, dm, fq, fk, fv, spin_max};
// [paso, x, norm_w, wq, wk, wv, q, k, v, kc, vc (f16 cache), qnorm|0, knorm|0, part_o, part_ml, freq|0, att, sync].
// sync: a library buffer of at least 2116 bytes, zero at allocation, used by this op only (group counters 256
// bytes apart, then the 8 groups' XCD words at 2048, the error word at 2112).  ns: workgroups per head group (a power of two,
// at most 64, at most nh / 8 * hd and two per CU of an XCD); spin_max 0: the default bound on a barrier's polls.
int op_dec_attn_block(const Ctx& c) {
    if (int e = need_bufs(c, 18, "dec_attn_block")) return e;
    QpDecBlockArgs a = {};
    a.hd = c.U(0);
    a.nh = c.U(1);
    a.nkv = c.U(2);
    a.ns = c.U(3);
    a.scale = c.F(4);
    a.eps = c.F(5);
    a.base = c.F(6);
    a.esc = c.U(7) ? c.F(7) : 1.0f;
    a.nrot = c.U(8);
    a.neox = c.U(9);
    a.rows = c.U(10);
    a.dm = c.U(11);
    a.fq = c.U(12);
    a.fk = c.U(13);
    a.fv = c.U(14);
    a.spin_max = c.U(15) ? c.U(15) : (1u << 18);
    const char* op = "dec_attn_block";
    if (!a.rows) return fail(QP_E_ARG, "%s: P.rows (cache slots) is 0", op);
    if (a.hd != 64 && a.hd != 128) return fail(QP_E_ARG, "%s: head_dim %u (64 or 128)", op, a.hd);
    if (a.nrot > a.hd || a.nrot % 2) return fail(QP_E_ARG, "%s: nrot=%u", op, a.nrot);
    if (!(a.nkv == 1 || a.nkv == 2 || a.nkv == 4 || a.nkv == 8) || a.nh % 8 || a.nh % a.nkv)
        return fail(QP_E_ARG, "%s: nh=%u nkv=%u (nkv 1, 2, 4 or 8; nh a multiple of 8)", op, a.nh, a.nkv);
    const uint32_t GP = a.nh / 8;
    if (!(GP == 1 || GP == 4 || (GP == 2 && a.hd == 128)))
        return fail(QP_E_ARG, "%s: %u query heads per group of head_dim %u (1, 2 or 4; 1 or 4 at 64)", op, GP, a.hd);
    const uint32_t per_xcd = g_cus >= 8 ? (uint32_t)g_cus / 8 : 1;
    if (a.ns == 0 || (a.ns & (a.ns - 1)) || a.ns > 64 || a.ns > GP * a.hd || a.ns > 2 * per_xcd)
        return fail(QP_E_ARG, "%s: ns=%u (a power of two, at most 64, %u and two per CU of an XCD)", op, a.ns,
                    GP * a.hd);
    if (a.dm == 0 || a.dm % 256 || a.dm > 8192) return fail(QP_E_ARG, "%s: model width %u (a multiple of 256, at most 8192)", op, a.dm);
    for (uint32_t f : {a.fq, a.fk, a.fv})
        if (f != QP_Q4_K && f != QP_Q6_K) return fail(QP_E_ARG, "%s: Q/K/V format %u (Q4_K 12 or Q6_K 14)", op, f);
    a.paso = c.B(0);
    a.x = c.B(1);
    a.norm_w = c.B(2);
    a.wq = c.B(3);
    a.wk = c.B(4);
    a.wv = c.B(5);
    a.q = c.B(6);
    a.k = c.B(7);
    a.v = c.B(8);
    a.kc = c.B(9);
    a.vc = c.B(10);
    a.qnorm = c.B(11);
    a.knorm = c.B(12);
    a.part_o = c.B(13);
    a.part_ml = c.B(14);
    a.freq = c.B(15);
    a.att = c.B(16);
    const uint64_t sync = c.B(17);
    if (!a.x || !a.norm_w || !a.wq || !a.wk || !a.wv || !a.q || !a.k || !a.v || !a.kc || !a.vc || !a.part_o ||
        !a.part_ml || !a.att || !sync)
        return fail(QP_E_ARG, "%s: a required binding is missing", op);
    if (buf_room(sync) < 2116) return fail(QP_E_ARG, "%s: sync must be a library buffer of at least 2116 bytes", op);
    a.cnt = sync;
    a.xcc = sync + 2048;
    a.err = sync + 2112;
    const uint32_t kvd = a.nkv * a.hd;
    struct Need { uint64_t p, n; const char* what; } need[] = {
        {a.wq, kq_tensor_bytes((int)a.fq, (uint64_t)a.nh * a.hd, a.dm), "wq"},
        {a.wk, kq_tensor_bytes((int)a.fk, kvd, a.dm), "wk"},
        {a.wv, kq_tensor_bytes((int)a.fv, kvd, a.dm), "wv"},
        {a.x, 4ull * a.dm, "x"}, {a.norm_w, 4ull * a.dm, "norm_w"},
        {a.q, 4ull * a.nh * a.hd, "q"}, {a.k, 4ull * kvd, "k"}, {a.v, 4ull * kvd, "v"},
        {a.kc, 2ull * a.rows * kvd, "the K cache"}, {a.vc, 2ull * ((a.rows + 31) / 32) * 32 * kvd, "the V cache"},
        {a.part_o, 4ull * a.nh * a.ns * a.hd, "part_o"}, {a.part_ml, 8ull * a.nh * a.ns, "part_ml"},
        {a.att, 4ull * a.nh * a.hd, "att"}};
    for (const Need& n : need)
        if (int e = need_room(n.p, n.n, op, n.what)) return e;
    const bool mix = a.fq != QP_Q4_K || a.fk != QP_Q4_K || a.fv != QP_Q4_K;
    Kid k;
    if (a.hd == 128) {
        static const Kid t[2][3] = {{K_dec_block_q4k_h128_g1, K_dec_block_q4k_h128_g2, K_dec_block_q4k_h128_g4},
                                    {K_dec_block_mix_h128_g1, K_dec_block_mix_h128_g2, K_dec_block_mix_h128_g4}};
        k = t[mix][GP == 1 ? 0 : GP == 2 ? 1 : 2];
    } else {
        static const Kid t[2][2] = {{K_dec_block_q4k_h64_g1, K_dec_block_q4k_h64_g4},
                                    {K_dec_block_mix_h64_g1, K_dec_block_mix_h64_g4}};
        k = t[mix][GP == 1 ? 0 : 1];
    }
    // LDS: the GEMV's input staging; the attention's floats (5 hd + the wavefront partials 4 GP hd + 64); the
    // merge's weights, denominators and weighted partials (GP ns + 8 + GP hd)
    const uint32_t att_lds = 4 * (a.hd * 5 + 4 * GP * a.hd + 64), mrg_lds = 4 * (a.hd * 5 + GP * a.ns + 8 + GP * a.hd);
    uint32_t lds = kq_lds(a.dm);
    if (att_lds > lds) lds = att_lds;
    if (mrg_lds > lds) lds = mrg_lds;
    return launch(k, 8, a.ns, 1, 256, lds, a);
}

// dec_attn_comb: P{hd, nh, nsplit}; [paso, part_o, part_ml, o].
int op_dec_attn_comb(const Ctx& c) {
    if (int e = need_bufs(c, 4, "dec_attn_comb")) return e;
    QpDecCombArgs a = {};
    a.hd = c.U(0);
    a.nh = c.U(1);
    a.nsplit = c.U(2);
    a.paso = c.B(0);
    a.part_o = c.B(1);
    a.part_ml = c.B(2);
    a.o = c.B(3);
    if (a.hd != 64 && a.hd != 128) return fail(QP_E_ARG, "dec_attn_comb: hd=%u", a.hd);
    if (a.nsplit == 0 || a.nsplit > 1024) return fail(QP_E_ARG, "dec_attn_comb: nsplit=%u", a.nsplit);
    return launch(K_dec_attn_comb, a.nh, 1, 1, 256, 0, a);
}

// argmax: P{n}; [paso, v, out] (greedy, sampling.js:38-42).
int op_argmax(const Ctx& c) {
    if (int e = need_bufs(c, 3, "argmax")) return e;
    QpArgmaxArgs a = {};
    a.n = c.U(0);
    a.v = c.B(1);
    a.out = c.B(2);
    return launch(K_argmax, 1, 1, 1, 1024, 0, a);
}

// argmax_fin: P{count, advance, cap}; [paso, amax, ids, tokens|0, step].  cap = entries of tokens.
int op_argmax_fin(const Ctx& c) {
    if (int e = need_bufs(c, 5, "argmax_fin")) return e;
    QpArgmaxFinArgs a = {};
    a.count = c.U(0);
    a.advance = c.U(1);
    a.cap = c.U(2);
    a.paso = c.B(0);
    a.amax = c.B(1);
    a.ids = c.B(2);
    a.tokens = c.B(3);
    a.step = c.B(4);
    return launch(K_argmax_fin, 1, 1, 1, 256, 0, a);
}

// penalizar: P{count, V, rep lo, rep hi, freq lo, hi, pres lo, hi} (the factors as IEEE double bits); [logits,
// pairs]: pairs = count (token, count) u32 pairs of the penalty window, count <= 64.  No reference counterpart (the
// reference penalizes on the host, sampling.js:27-37).
int op_penalizar(const Ctx& c) {
    if (int e = need_bufs(c, 2, "penalizar")) return e;
    QpPenaltyArgs a = {};
    a.count = c.U(0);
    a.n = c.U(1);
    const uint64_t r = c.U64(2), f = c.U64(4), p = c.U64(6);
    memcpy(&a.rep, &r, 8);
    memcpy(&a.freq, &f, 8);
    memcpy(&a.pres, &p, 8);
    if (a.count > 64) return fail(QP_E_ARG, "penalizar: %u pairs (the window holds at most 64)", a.count);
    a.logits = c.B(0);
    a.hist = c.B(1);
    return launch(K_penalizar, 1, 1, 1, 64, 0, a);
}

// topk_cand: P{V, k}; [logits, part, out].  part: ceil(V/2048)*(k+1) u64 keys + ceil(V/2048) u32 flags; out:
// 2 + 2k u32 ({flags, k, (value bits, id) x k}, descending).  1 <= k <= 128, k < V, ceil(V/2048)*(k+1) <= 16384.
// No reference counterpart (the reference's top-k heap runs on the host, sampling.js:44-57).
int op_topk_cand(const Ctx& c) {
    if (int e = need_bufs(c, 3, "topk_cand")) return e;
    QpCandArgs a = {};
    a.n = c.U(0);
    a.k = c.U(1);
    if (a.k < 1 || a.k > 128 || a.k >= a.n)
        return fail(QP_E_ARG, "topk_cand: k=%u must be in 1..128 and below V=%u", a.k, a.n);
    a.kp = a.k + 1;
    a.g = cdiv(a.n, 2048);
    const uint64_t tot = (uint64_t)a.g * a.kp;
    if (tot > 16384) return fail(QP_E_ARG, "topk_cand: V=%u, k=%u: %llu partial candidates exceed 16384", a.n, a.k,
                                 (unsigned long long)tot);
    uint32_t n2 = 2;
    while (n2 < tot) n2 <<= 1;
    a.n2 = n2;
    a.logits = c.B(0);
    a.part = c.B(1);
    a.out = c.B(2);
    if (int e = launch(K_topk_part, a.g, 1, 1, 256, 0, a)) return e;
    return launch(K_topk_merge, 1, 1, 1, 1024, n2 * 8, a);
}

// repack_q2k .. repack_q6k: P{nblocks lo, hi, K}; repack_q8: P{nblocks lo, hi}; [paso|0, src, dst].  K (the row
// length) places the blocks in the row chunk-plane layout of the K-quants (dst: kq_tensor_bytes).
int op_repack(const Ctx& c, Kid k, const char* name) {
    if (int e = need_bufs(c, 3, name)) return e;
    QpRepackArgs a = {};
    a.nblocks = c.U64(0);
    a.k = c.U(2);
    a.src = c.B(1);
    a.dst = c.B(2);
    uint64_t threads = a.nblocks;
    if (k == K_repack_q8 || k == K_repack_iq4nl) {
        // raw blocks of 34 (Q8_0) or 18 (IQ4_NL) bytes -> as many bytes each in the planar layout
        const uint64_t rs = buf_room(a.src), rd = buf_room(a.dst), in = a.nblocks * (k == K_repack_q8 ? 34 : 18);
        if ((rs && rs < in) || (rd && rd < in))
            return fail(QP_E_ARG, "%s: %llu blocks need %llu source and destination bytes", name,
                        (unsigned long long)a.nblocks, (unsigned long long)in);
    }
    if (k == K_repack_q4k || k == K_repack_q5k || k == K_repack_q6k || k == K_repack_q3k || k == K_repack_q2k) {
        if (a.k == 0 || a.k % 256 || a.k > 15360) return fail(QP_E_ARG, "%s: K=%u must be a multiple of 256 <= 15360", name, a.k);
        if (a.nblocks % (a.k / 256)) return fail(QP_E_ARG, "%s: %llu blocks are not whole rows of K=%u", name,
                                                 (unsigned long long)a.nblocks, a.k);
        threads = a.nblocks * (k == K_repack_q4k ? 9 : k == K_repack_q5k ? 11 : k == K_repack_q3k ? 7 : k == K_repack_q2k ? 6 : 14);
    }
    return launch(k, grid_cap(threads), 1, 1, 256, 0, a);
}

// fill_u32: P{value, count lo, hi}; [paso|0, dst].  A kernel, so it may be captured in a graph.
int op_fill(const Ctx& c) {
    if (int e = need_bufs(c, 2, "fill_u32")) return e;
    QpFillArgs a = {};
    a.value = c.U(0);
    a.count = c.U64(1);
    a.dst = c.B(1);
    return launch(K_fill_u32, grid_cap(a.count), 1, 1, 256, 0, a);
}

// copy_f4 / read_f4: P{n float4s lo, hi, grid}; [paso|0, src, dst] -- plain streaming kernels of known traffic
// (read_f4 writes one float per thread of the grid into dst).
int op_stream(const Ctx& c, Kid k, const char* name) {
    if (int e = need_bufs(c, 3, name)) return e;
    QpRepackArgs a = {};
    a.nblocks = c.U64(0);
    a.src = c.B(1);
    a.dst = c.B(2);
    uint32_t grid = c.U(2) ? c.U(2) : resident_wgs(k, 256, 0);
    return launch(k, grid, 1, 1, 256, 0, a);
}

// dequant: P{fmt, n lo, hi}; [paso|0, w, y]: whole tensor to f32.
int op_dequant(const Ctx& c) {
    if (int e = need_bufs(c, 3, "dequant")) return e;
    QpDequantArgs a = {};
    a.fmt = c.U(0);
    a.nelem = c.U64(1);
    a.k = c.U(3);
    a.w = c.B(1);
    a.y = c.B(2);
    if (!known_fmt((int)a.fmt)) return fail(QP_E_ARG, "dequant: format %u is not a device layout", a.fmt);
    if (a.k == 0) a.k = planar((int)a.fmt) ? 32 : (a.fmt == QP_F32 ? 1 : 256);  // one row per block
    if (int e = check_k((int)a.fmt, a.k, "dequant")) return e;
    if (a.nelem % a.k) return fail(QP_E_ARG, "dequant: %llu elements are not whole rows of K=%u",
                                   (unsigned long long)a.nelem, a.k);
    if (int e = need_room(a.w, tensor_bytes((int)a.fmt, a.nelem / a.k, a.k), "dequant", "the tensor")) return e;
    if (int e = need_room(a.y, a.nelem * 4, "dequant", "the output")) return e;
    return launch(K_dequant, grid_cap(a.nelem), 1, 1, 256, 0, a);
}

// ------------------------------------------------------------------------------------------------ registry
typedef int (*OpFn)(const Ctx&);
struct Op {
    std::string name;
    std::function<int(const Ctx&)> fn;
};
std::vector<Op>& ops() {
    static std::vector<Op> v;
    return v;
}

void register_ops() {
    auto& v = ops();
    if (!v.empty()) return;
    for (const char* f : {"q2k", "q3k", "q4k", "q5k", "q6k", "q8", "f32", "iq4nl"}) {
        const int fmt = fmt_of(f);
        std::string s(f);
        std::string n1 = "matmul_" + s + "_1", n4 = "matmul_" + s + "_4", nt = "matmul_" + s + "_t";
        std::string ne = "matmul_" + s + "_e", nes = "matmul_" + s + "_e_swiglu", nem = "embed_" + s;
        v.push_back({n1, [fmt, n1](const Ctx& c) { return op_matmul_1(c, fmt, n1.c_str()); }});
        v.push_back({n4, [fmt, n4](const Ctx& c) { return op_matmul_mt(c, fmt, n4.c_str(), 4); }});
        v.push_back({nt, [fmt, nt](const Ctx& c) { return op_matmul_mt(c, fmt, nt.c_str(), 32); }});
        if (is_kq(fmt)) {
            const std::string ng = nt + "_swiglu";
            v.push_back({ng, [fmt, ng](const Ctx& c) { return op_matmul_glu(c, fmt, ng.c_str()); }});
        }
        v.push_back({ne, [fmt, ne](const Ctx& c) { return op_matmul_e(c, fmt, ne.c_str(), false); }});
        v.push_back({nes, [fmt, nes](const Ctx& c) { return op_matmul_e(c, fmt, nes.c_str(), true); }});
        v.push_back({nem, [fmt, nem](const Ctx& c) { return op_embed(c, fmt, nem.c_str()); }});
    }
    v.push_back({"rmsnorm", op_rmsnorm});
    v.push_back({"rmsnorm_planes", op_rmsnorm_planes});
    v.push_back({"norm_rope", op_norm_rope});
    v.push_back({"kv_write", op_kv_write});
    v.push_back({"atencion", op_atencion});
    v.push_back({"swiglu", op_swiglu});
    v.push_back({"geglu", op_geglu});
    v.push_back({"escalar", [](const Ctx& c) { return op_scale(c, false); }});
    v.push_back({"suma_esc", [](const Ctx& c) { return op_scale(c, true); }});
    v.push_back({"moe_topk", op_moe_topk});
    v.push_back({"moe_comb", op_moe_comb});
    v.push_back({"moe_group", op_moe_group});
    for (const char* f : {"q2k", "q3k", "q4k", "q5k", "q6k", "q8", "f32", "iq4nl"}) {
        const int fmt = fmt_of(f);
        const std::string n = std::string("matmul_") + f + "_eg";
        v.push_back({n, [fmt, n](const Ctx& c) { return op_matmul_eg(c, fmt, n.c_str()); }});
    }
    v.push_back({"moe_gate_up_q4k", [](const Ctx& c) { return op_moe(c, QP_Q4_K, false, "moe_gate_up_q4k"); }});
    v.push_back({"moe_gate_up_q6k", [](const Ctx& c) { return op_moe(c, QP_Q6_K, false, "moe_gate_up_q6k"); }});
    v.push_back({"moe_down_q4k", [](const Ctx& c) { return op_moe(c, QP_Q4_K, true, "moe_down_q4k"); }});
    v.push_back({"moe_down_q6k", [](const Ctx& c) { return op_moe(c, QP_Q6_K, true, "moe_down_q6k"); }});
    v.push_back({"gemv", op_gemv});
    v.push_back({"dec_attn", op_dec_attn});
    v.push_back({"dec_attn_comb", op_dec_attn_comb});
    v.push_back({"dec_attn_block", op_dec_attn_block});
    v.push_back({"moe_router", op_moe_router});
    v.push_back({"argmax", op_argmax});
    v.push_back({"argmax_fin", op_argmax_fin});
    v.push_back({"penalizar", op_penalizar});
    v.push_back({"topk_cand", op_topk_cand});
    v.push_back({"repack_q4k", [](const Ctx& c) { return op_repack(c, K_repack_q4k, "repack_q4k"); }});
    v.push_back({"repack_q5k", [](const Ctx& c) { return op_repack(c, K_repack_q5k, "repack_q5k"); }});
    v.push_back({"repack_q3k", [](const Ctx& c) { return op_repack(c, K_repack_q3k, "repack_q3k"); }});
    v.push_back({"repack_q2k", [](const Ctx& c) { return op_repack(c, K_repack_q2k, "repack_q2k"); }});
    v.push_back({"repack_q6k", [](const Ctx& c) { return op_repack(c, K_repack_q6k, "repack_q6k"); }});
    v.push_back({"repack_q8", [](const Ctx& c) { return op_repack(c, K_repack_q8, "repack_q8"); }});
    v.push_back({"repack_iq4nl", [](const Ctx& c) { return op_repack(c, K_repack_iq4nl, "repack_iq4nl"); }});
    v.push_back({"fill_u32", op_fill});
    v.push_back({"dequant", op_dequant});
    v.push_back({"copy_f4", [](const Ctx& c) { return op_stream(c, K_copy_f4, "copy_f4"); }});
    v.push_back({"read_f4", [](const Ctx& c) { return op_stream(c, K_read_f4, "read_f4"); }});
}

std::string self_dir() {
    Dl_info info;
    if (dladdr((void*)&self_dir, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t s = p.rfind('/');
        if (s != std::string::npos) return p.substr(0, s);
    }
    return ".";
}

}  // namespace

// ================================================================================================ C ABI
extern "C" {

int qp_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_init) {
        if (device != g_device) return fail(QP_E_ARG, "already initialized on device %d", g_device);
        return 0;
    }
    register_ops();
    if (const char* e = getenv("QP_FAIL_ALLOC")) g_fail_alloc = atol(e);
    if (const char* e = getenv("QP_FAIL_LAUNCH")) g_fail_launch = atol(e);
    int n = 0;
    HIPCHK(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(QP_E_ARG, "device %d of %d", device, n);
    HIPCHK(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t p;
    HIPCHK(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
    g_summary = p.name;
    g_arch = p.gcnArchName;
    g_cus = p.multiProcessorCount;
    g_hbm = p.totalGlobalMem;
    if (g_arch.rfind("gfx950", 0) != 0)
        return fail(QP_E_ARG, "device %d is %s; this backend is built for gfx950 only", device, g_arch.c_str());
    HIPCHK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), "hipStreamCreate");
    if (int e = qp_scratch::lookup(device, &g_scratch)) return hip_fail((hipError_t)e, "hipGetSymbolAddress (scratch)");
    std::string path;
    if (const char* e = getenv("QP_KERNELS")) path = e;
    else path = self_dir() + "/quipu_kernels.hsaco";
    HIPCHK(hipModuleLoad(&g_mod, path.c_str()), ("hipModuleLoad " + path).c_str());
    for (int k = 0; k < K_COUNT; k++)
        HIPCHK(hipModuleGetFunction(&g_fn[k], g_mod, kNames[k]), kNames[k]);
    g_device = device;
    g_init = true;
    return 0;
}

int qp_info(char* json, size_t cap) {
    NEED_INIT();
    char buf[512];
    snprintf(buf, sizeof buf,
             "{\"summary\":\"%s\",\"arch\":\"%s\",\"cus\":%d,\"hbm_bytes\":%llu,\"max_buffer\":%llu,"
             "\"bytes_used\":%llu}",
             g_summary.c_str(), g_arch.c_str(), g_cus, (unsigned long long)g_hbm, (unsigned long long)g_hbm,
             (unsigned long long)g_bytes);
    if (!json || cap <= strlen(buf)) return fail(QP_E_ARG, "qp_info: buffer too small");
    strcpy(json, buf);
    return 0;
}

int qp_last_error(char* buf, size_t cap) {
    if (!buf || !cap) return QP_E_ARG;
    snprintf(buf, cap, "%s", g_err.c_str());
    return 0;
}

uint64_t qp_bytes_used(void) { return g_bytes; }
int qp_lost(void) { return g_lost.load(); }

int qp_alloc(uint64_t bytes, uint64_t* dev) {
    NEED_INIT();
    if (!dev) return fail(QP_E_ARG, "qp_alloc: null out");
    if (g_capturing) return fail(QP_E_CAPTURE, "qp_alloc during graph capture");
    if (g_fail_alloc > 0 && ++g_n_alloc == g_fail_alloc)
        return fail(QP_E_INJECTED, "injected allocation failure (QP_FAIL_ALLOC=%ld)", g_fail_alloc);
    uint64_t tam = bytes < 16 ? 16 : (bytes + 3) / 4 * 4;
    if (tam > g_hbm) return fail(QP_E_ARG, "buffer of %llu bytes exceeds the device", (unsigned long long)tam);
    void* p = nullptr;
    HIPCHK(hipMalloc(&p, tam), "hipMalloc");
    *dev = (uint64_t)p;
    std::lock_guard<std::mutex> lk(g_mu);
    g_allocs[*dev] = tam;
    g_bytes += tam;
    return 0;
}

int qp_free(uint64_t dev) {
    NEED_INIT();
    if (!dev) return 0;
    if (g_capturing) return fail(QP_E_CAPTURE, "qp_free during graph capture");
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_allocs.find(dev);
        if (it == g_allocs.end()) return fail(QP_E_ARG, "qp_free: 0x%llx is not a live buffer", (unsigned long long)dev);
        g_bytes -= it->second;
        g_allocs.erase(it);
    }
    HIPCHK(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
    HIPCHK(hipFree((void*)dev), "hipFree");
    return 0;
}

int qp_upload(uint64_t dst, uint64_t off, const void* src, uint64_t n) {
    NEED_INIT();
    if (g_capturing) return fail(QP_E_CAPTURE, "qp_upload during graph capture");
    if (!n) return 0;
    HIPCHK(hipMemcpyAsync((void*)(dst + off), src, n, hipMemcpyHostToDevice, g_stream), "upload");
    HIPCHK(hipStreamSynchronize(g_stream), "upload sync");  // the host buffer may be reused at once
    return 0;
}

int qp_download(void* dst, uint64_t src, uint64_t off, uint64_t n) {
    NEED_INIT();
    if (g_capturing) return fail(QP_E_CAPTURE, "qp_download during graph capture");
    if (!n) return 0;
    HIPCHK(hipMemcpyAsync(dst, (const void*)(src + off), n, hipMemcpyDeviceToHost, g_stream), "download");
    HIPCHK(hipStreamSynchronize(g_stream), "download sync");
    return 0;
}

int qp_copy(uint64_t dst, uint64_t doff, uint64_t src, uint64_t soff, uint64_t n) {
    NEED_INIT();
    if (!n) return 0;
    HIPCHK(hipMemcpyAsync((void*)(dst + doff), (const void*)(src + soff), n, hipMemcpyDeviceToDevice, g_stream),
           "copy");
    return 0;
}

int qp_sync(void) {
    NEED_INIT();
    HIPCHK(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
    return 0;
}

int qp_op_id(const char* name) {
    register_ops();
    if (!name) return -1;
    auto& v = ops();
    for (size_t i = 0; i < v.size(); i++)
        if (v[i].name == name) return (int)i;
    return -1;
}

int qp_dispatch(int op, const void* uniform, uint32_t usize, const uint64_t* bufs, uint32_t nbuf, uint32_t gx,
                uint32_t gy, uint32_t gz) {
    NEED_INIT();
    auto& v = ops();
    if (op < 0 || (size_t)op >= v.size()) return fail(QP_E_ARG, "qp_dispatch: unknown op %d", op);
    if (usize && !uniform) return fail(QP_E_ARG, "%s: null uniform", v[op].name.c_str());
    Ctx c{(const uint8_t*)uniform, usize, bufs, nbuf, gx, gy, gz};
    return v[op].fn(c);
}

int qp_dispatch_noalloc(int op, const void* uniform, uint32_t usize, const uint64_t* bufs, uint32_t nbuf,
                        uint32_t gx, uint32_t gy, uint32_t gz) {
    NEED_INIT();
    struct Flag {
        Flag() { g_noalloc = true; }
        ~Flag() { g_noalloc = false; }
    } flag;
    return qp_dispatch(op, uniform, usize, bufs, nbuf, gx, gy, gz);
}

int qp_module_load(const char* path, uint64_t* module) {
    NEED_INIT();
    hipModule_t m;
    HIPCHK(hipModuleLoad(&m, path), "hipModuleLoad");
    *module = (uint64_t)m;
    return 0;
}

int qp_kernel(uint64_t module, const char* name, uint64_t* fn) {
    NEED_INIT();
    hipFunction_t f;
    HIPCHK(hipModuleGetFunction(&f, (hipModule_t)module, name), name);
    *fn = (uint64_t)f;
    return 0;
}

int qp_launch(uint64_t fn, const uint32_t grid[3], const uint32_t block[3], uint32_t lds, const void* args,
              uint64_t args_size) {
    NEED_INIT();
    if (g_fail_launch > 0 && ++g_n_launch == g_fail_launch)
        return fail(QP_E_INJECTED, "injected launch failure (QP_FAIL_LAUNCH=%ld)", g_fail_launch);
    size_t sz = (size_t)args_size;
    void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, (void*)args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                     HIP_LAUNCH_PARAM_END};
    HIPCHK(hipModuleLaunchKernel((hipFunction_t)fn, grid[0], grid[1], grid[2], block[0], block[1], block[2], lds,
                                 g_stream, nullptr, extra),
           "qp_launch");
    return 0;
}

int qp_graph_begin(void) {
    NEED_INIT();
    if (g_capturing) return fail(QP_E_CAPTURE, "capture already open");
    HIPCHK(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    g_capturing = true;
    return 0;
}

// The captured graph of each instantiated one, kept until qp_graph_free destroys both: a tool that holds on to the
// graph's nodes from instantiation (a tracer) finds them alive for every launch.
std::map<uint64_t, hipGraph_t> g_graphs;

int qp_graph_end(uint64_t* graph) {
    NEED_INIT();
    if (!g_capturing) return fail(QP_E_CAPTURE, "no capture open");
    g_capturing = false;
    hipGraph_t g;
    HIPCHK(hipStreamEndCapture(g_stream, &g), "hipStreamEndCapture");
    hipGraphExec_t ex;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return hip_fail(e, "hipGraphInstantiate");
    }
    g_graphs[(uint64_t)ex] = g;
    *graph = (uint64_t)ex;
    return 0;
}

int qp_graph_launch(uint64_t graph) {
    NEED_INIT();
    if (!g_graphs.count(graph)) return fail(QP_E_ARG, "qp_graph_launch: not a graph of this library");
    g_split_memo.valid = false;  // a replay may rewrite the input planes
    HIPCHK(hipGraphLaunch((hipGraphExec_t)graph, g_stream), "hipGraphLaunch");
    return 0;
}

#ifdef QP_TIMELINE
// Writes the kernels' records of the launches captured since the last graph was freed to QP_TIMELINE_OUT (uint4 per
// workgroup slot, 4096 slots per launch; the last replay's), the phase stamps to QP_TIMELINE_OUT.ph and the
// launches (kernel, grid, block) to QP_TIMELINE_OUT.json.
void tl_dump() {
    const char* out = getenv("QP_TIMELINE_OUT");
    if (!out || g_tl.empty()) return;
    hipStreamSynchronize(g_stream);
    hipDeviceptr_t d;
    size_t sz = 0;
    if (hipModuleGetGlobal(&d, &sz, g_mod, "qp_tl") != hipSuccess) return;
    std::vector<uint8_t> h(std::min(sz, g_tl.size() * 4096 * 16));
    hipMemcpy(h.data(), (void*)d, h.size(), hipMemcpyDeviceToHost);
    if (FILE* f = fopen(out, "wb")) { fwrite(h.data(), 1, h.size(), f); fclose(f); }
    if (hipModuleGetGlobal(&d, &sz, g_mod, "qp_tl_ph") == hipSuccess) {
        std::vector<uint8_t> p(sz);
        hipMemcpy(p.data(), (void*)d, sz, hipMemcpyDeviceToHost);
        if (FILE* f = fopen((std::string(out) + ".ph").c_str(), "wb")) { fwrite(p.data(), 1, sz, f); fclose(f); }
    }
    if (FILE* f = fopen((std::string(out) + ".json").c_str(), "w")) {
        fprintf(f, "[");
        for (size_t i = 0; i < g_tl.size(); i++)
            fprintf(f, "%s[\"%s\", %u, %u, %u, %u]", i ? ", " : "", kNames[g_tl[i].k], g_tl[i].gx, g_tl[i].gy,
                    g_tl[i].gz, g_tl[i].block);
        fprintf(f, "]\n");
        fclose(f);
    }
    g_tl.clear();  // the next graph captured numbers its launches from 1 again
}
#endif

int qp_graph_free(uint64_t graph) {
    NEED_INIT();
#ifdef QP_TIMELINE
    tl_dump();
#endif
    auto it = g_graphs.find(graph);
    if (it == g_graphs.end()) return fail(QP_E_ARG, "qp_graph_free: not a graph of this library");
    const hipGraph_t g = it->second;
    g_graphs.erase(it);
    HIPCHK(hipGraphExecDestroy((hipGraphExec_t)graph), "hipGraphExecDestroy");
    HIPCHK(hipGraphDestroy(g), "hipGraphDestroy");
    return 0;
}

int qp_event_create(uint64_t* ev) {
    NEED_INIT();
    hipEvent_t e;
    HIPCHK(hipEventCreate(&e), "hipEventCreate");
    *ev = (uint64_t)e;
    return 0;
}

int qp_event_record(uint64_t ev) {
    NEED_INIT();
    HIPCHK(hipEventRecord((hipEvent_t)ev, g_stream), "hipEventRecord");
    return 0;
}

int qp_event_elapsed(uint64_t ev0, uint64_t ev1, float* ms) {
    NEED_INIT();
    HIPCHK(hipEventSynchronize((hipEvent_t)ev1), "hipEventSynchronize");
    HIPCHK(hipEventElapsedTime(ms, (hipEvent_t)ev0, (hipEvent_t)ev1), "hipEventElapsedTime");
    return 0;
}

int qp_event_free(uint64_t ev) {
    NEED_INIT();
    HIPCHK(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
    return 0;
}

}  // extern "C"
