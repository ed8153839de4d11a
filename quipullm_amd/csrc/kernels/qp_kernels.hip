// gfx950 kernels of the quipu token loop.  One translation unit, compiled to a code object that the
// runtime loads with hipModuleLoad and launches with hipModuleLaunchKernel.  Every kernel takes one
// argument block from qp_args.h by value.
//
// Semantics follow the reference's WGSL kernels (citations per kernel); the launch shapes, data layouts
// and reduction orders are this build's own (64-lane wavefronts, 16-byte loads, LDS-staged activations).
#include "qp_common.h"

#define KERNEL extern "C" __global__

// ====================================================================================== load-time ops
// GGUF blocks -> the row chunk-plane layout of Q4_K / Q6_K (qp_args.h).  One thread per 16-byte chunk; a.k is
// the row length (nb = K/256 blocks per row).
// Q4_K (144-byte blocks, 9 chunks) and Q5_K (176 bytes, 11 chunks): every chunk of a GGUF block moves whole.
template <int NCH>
QP_DEV void repack_chunks(const QpRepackArgs& a) {
    const uint64_t NB = a.nblocks, nchunk = NB * NCH;
    const uint32_t nb = a.k >> 8;
    for (uint64_t t = blockIdx.x * 256ull + threadIdx.x; t < nchunk; t += (uint64_t)gridDim.x * 256ull) {
        const uint64_t blk = t / NCH, row = blk / nb;
        const uint32_t c = (uint32_t)(t - blk * NCH), b = (uint32_t)(blk - row * nb);
        const uint4 v = cptr<uint4>(a.src)[t];  // GGUF offset blk*16*NCH + c*16
        mptr<uint4>(a.dst + row * nb * (16 * NCH) + (uint64_t)c * nb * 16 + b * 16)[0] = v;
    }
}
KERNEL __launch_bounds__(256) void qp_repack_q4k(QpRepackArgs a) { repack_chunks<9>(a); }
KERNEL __launch_bounds__(256) void qp_repack_q5k(QpRepackArgs a) { repack_chunks<11>(a); }

// Q3_K: 110-byte GGUF blocks (2-byte aligned) into 112-byte slots of 7 chunks (the last chunk: scales, d, 2 zero
// bytes).  Q2_K: 84-byte blocks, bytes 0..79 as 5 chunks, d and dmin (bytes 80..83) to an array after the rows.
KERNEL __launch_bounds__(256) void qp_repack_q3k(QpRepackArgs a) {
    const uint64_t NB = a.nblocks, nchunk = NB * 7;
    const uint32_t nb = a.k >> 8;
    for (uint64_t t = blockIdx.x * 256ull + threadIdx.x; t < nchunk; t += (uint64_t)gridDim.x * 256ull) {
        const uint64_t blk = t / 7, row = blk / nb;
        const uint32_t c = (uint32_t)(t - blk * 7), b = (uint32_t)(blk - row * nb);
        const uint8_t* src = cptr<uint8_t>(a.src) + blk * 110;
        uint8_t* o = mptr<uint8_t>(a.dst) + row * nb * 112 + (uint64_t)c * nb * 16 + b * 16;
        for (int i = 0; i < 16; i++) o[i] = c * 16 + i < 110 ? src[c * 16 + i] : 0;
    }
}

KERNEL __launch_bounds__(256) void qp_repack_q2k(QpRepackArgs a) {
    const uint64_t NB = a.nblocks, nchunk = NB * 6;
    const uint32_t nb = a.k >> 8;
    for (uint64_t t = blockIdx.x * 256ull + threadIdx.x; t < nchunk; t += (uint64_t)gridDim.x * 256ull) {
        const uint64_t blk = t / 6, row = blk / nb;
        const uint32_t c = (uint32_t)(t - blk * 6), b = (uint32_t)(blk - row * nb);
        const uint32_t* src = cptr<uint32_t>(a.src) + blk * 21;  // 84-byte blocks: 4-byte aligned
        uint32_t* dst = mptr<uint32_t>(a.dst);
        if (c < 5) {
            uint32_t* o = dst + (row * nb * 80 + (uint64_t)c * nb * 16 + b * 16) / 4;
            for (int i = 0; i < 4; i++) o[i] = src[c * 4 + i];
        } else {
            dst[(NB * 80) / 4 + blk] = src[20];
        }
    }
}

KERNEL __launch_bounds__(256) void qp_repack_q6k(QpRepackArgs a) {
    const uint64_t NB = a.nblocks, nchunk = NB * 14;
    const uint32_t nb = a.k >> 8;
    for (uint64_t t = blockIdx.x * 256ull + threadIdx.x; t < nchunk; t += (uint64_t)gridDim.x * 256ull) {
        const uint64_t blk = t / 14, row = blk / nb;
        const uint32_t c = (uint32_t)(t - blk * 14), b = (uint32_t)(blk - row * nb);
        const uint8_t* src = cptr<uint8_t>(a.src) + blk * 210;  // 210-byte blocks: only 2-byte aligned
        uint8_t* dst = mptr<uint8_t>(a.dst);
        if (c < 13) {
            uint8_t* o = dst + row * nb * 208 + (uint64_t)c * nb * 16 + b * 16;
            for (int i = 0; i < 16; i++) o[i] = src[c * 16 + i];
        } else {
            uint8_t* o = dst + NB * 208 + blk * 2;
            o[0] = src[208];
            o[1] = src[209];
        }
    }
}

// Q8_0: GGUF 34-byte blocks -> planar qs | d (reference keeps qs + f32 ds, gpu.js:1150-1162).
KERNEL __launch_bounds__(256) void qp_repack_q8(QpRepackArgs a) {
    const uint64_t NB = a.nblocks;
    for (uint64_t b = blockIdx.x * 256ull + threadIdx.x; b < NB; b += (uint64_t)gridDim.x * 256ull) {
        const uint8_t* s = cptr<uint8_t>(a.src) + b * 34;
        uint8_t* d = mptr<uint8_t>(a.dst);
        for (int i = 0; i < 32; i++) d[b * 32 + i] = s[2 + i];
        d[NB * 32 + b * 2] = s[0];
        d[NB * 32 + b * 2 + 1] = s[1];
    }
}

// IQ4_NL (GGML type 20, reference weights.js:110-116 and kds.js:36-39): GGUF 18-byte blocks (d f16, then 16 nibble
// bytes) -> planar qs [NB][16] | d [NB] f16, the nibble bytes unchanged (18 bytes per 32 weights on the device).
KERNEL __launch_bounds__(256) void qp_repack_iq4nl(QpRepackArgs a) {
    const uint64_t NB = a.nblocks;
    for (uint64_t b = blockIdx.x * 256ull + threadIdx.x; b < NB; b += (uint64_t)gridDim.x * 256ull) {
        const uint8_t* s = cptr<uint8_t>(a.src) + b * 18;
        uint8_t* d = mptr<uint8_t>(a.dst);
        for (int l = 0; l < 16; l++) d[b * 16 + l] = s[2 + l];
        d[NB * 16 + b * 2] = s[0];
        d[NB * 16 + b * 2 + 1] = s[1];
    }
}

KERNEL __launch_bounds__(256) void qp_fill_u32(QpFillArgs a) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < a.count; i += (uint64_t)gridDim.x * 256ull)
        mptr<uint32_t>(a.dst)[i] = a.value;
}

// Whole-tensor dequant to f32 in element order, rows of a.k elements (reference's scalar formula; for checks).
KERNEL __launch_bounds__(256) void qp_dequant(QpDequantArgs a) {
    const uint32_t K = a.k;
    const uint64_t NB = total_blocks(a.fmt, a.nelem / K, K);
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < a.nelem; i += (uint64_t)gridDim.x * 256ull) {
        const uint64_t row = i / K;
        mptr<float>(a.y)[i] = deq_elem(a.fmt, cptr<uint8_t>(a.w), NB, row, K, (uint32_t)(i - row * K));
    }
}

// ====================================================================================== embeddings
// Reference embed_q4k/q6k (kquants.js:481-504), embed_q8 (gpu.js:585-604), embed_f32 (gpu.js:605-618):
// y[t][k] = deq(W[ids[t]][k]).  a.rows (the tensor's row count) sizes the planar sub-arrays.
QP_DEV void qp_embed_impl(QpEmbedArgs a);
KERNEL __launch_bounds__(256) void qp_embed(QpEmbedArgs a) {
    const uint64_t t0 = tl_now();
    qp_embed_impl(a);
    tl_rec(a.tseq, t0);
}
QP_DEV void qp_embed_impl(QpEmbedArgs a) {
    const uint32_t T = paso_T(a.paso), D = a.d;
    const uint64_t nrows = a.rows;
    const uint64_t NB = total_blocks(a.fmt, nrows, D);
    const uint64_t n = (uint64_t)T * D;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull) {
        const uint32_t t = (uint32_t)(i / D), k = (uint32_t)(i % D);
        uint32_t id = cptr<uint32_t>(a.ids)[t];
        if (id >= a.rows) id = a.rows - 1;  // the host validates ids; a stray one never reads outside the table
        mptr<float>(a.y)[i] = deq_elem(a.fmt, cptr<uint8_t>(a.w), NB, id, D, k);
    }
}

// ====================================================================================== GEMV (one token), planar
// Q8_0, IQ4_NL and F32 y = W.x for one token: the fused `gemv` op, the reference's matmul_q8_1 / matmul_iq4nl_1 /
// matmul_f32_1 (gpu.js:123-198, kds.js:41-107) and the gathered-expert matmul_*_e (kds.js:110-186).
//
// A wavefront computes R weight rows at once; its lanes stride over the rows' "pieces" (Q8_0, IQ4_NL: one 32-weight
// block; F32: 16 floats), so one load instruction reads 64 consecutive pieces of a row (2 KB of Q8_0 quants, 1 KB of
// IQ4_NL nibbles) and their 128 contiguous bytes of scales.  The work of a wavefront is one sequence of items (pass
// k, piece slot j < ppl): pass k takes the R rows of row group blockIdx.x + k * gridDim.x (a persistent grid), slot j
// the pieces lane + 64 j.  D register sets rotate, so the loads of the D - 1 items after item n are in flight while
// item n is multiplied.  Every item issues the same loads through buffer resources of its rows: a lane past the
// row's pieces passes an offset past the resource, and a row past its segment (or an item past the wave's last
// pass) gets an empty resource; neither moves data.  As the number of loads never depends on the path taken, the
// compiler's waits count exactly the loads in flight (a load issued on one path only would make it wait for all).
// The input's loads are issued before the first items' weights and awaited alone; the input is staged once per
// workgroup in LDS in piece-major order (float4 j of piece p at xs[j * npc + p]: the lanes of an LDS read touch
// consecutive 16-byte words), optionally RMS-normalized on the way in.  Outputs are held in registers and written
// after the item loop: a store in flight counts in the same counter as the loads, and every later wait would
// include it.
// Semantics: reference matmul_*_1 (kquants.js:188-251, gpu.js:123-198): y = W.x; Q8_0 and IQ4_NL take a += d * s
// per block with s the block's dot product, as the reference does (kds.js:80-88).

QP_DEV void q4k_sm(uint32_t s03, uint32_t s47, uint32_t s811, uint32_t j, uint32_t& sc, uint32_t& mn) {
    // 6-bit scale/min unpack of sub-block j (reference scmin, kquants.js:65-76)
    const uint32_t jj = (j & 3) * 8;
    const uint32_t a = (s03 >> jj) & 0xffu, b = (s47 >> jj) & 0xffu, c = (s811 >> jj) & 0xffu;
    if (j < 4) {
        sc = a & 63u;
        mn = b & 63u;
    } else {
        sc = (c & 15u) | ((a >> 6) << 4);
        mn = (c >> 4) | ((b >> 6) << 4);
    }
}

// A value the compiler takes for a per-lane one (read from memory) that is the same in every lane.
QP_DEV uint64_t uni64(uint64_t v) {
    return ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
}

// A row of one pass: its quant (F32: float) bytes and its f16 scales.
struct PlRow {
    __amdgpu_buffer_rsrc_t q, d;
};

// Per-format piece registers for R rows: load() issues the loads of piece p (on: the lane has the piece),
// compute() consumes them with the piece's x values from LDS.  J: float4s of x per piece; QB: quant bytes per
// piece; LOADS: load instructions per row.
template <int FMT, int R>
struct Piece;

QP_DEV float sdot4(uint32_t w, const float4 x) {  // the 4 signed bytes of w with x
    return (float)(int8_t)(w & 0xffu) * x.x + (float)(int8_t)((w >> 8) & 0xffu) * x.y +
           (float)(int8_t)((w >> 16) & 0xffu) * x.z + (float)(int8_t)(w >> 24) * x.w;
}

template <int R>
struct Piece<QP_Q8_0, R> {
    static constexpr uint32_t J = 8, QB = 32, LOADS = 3;
    u32x4 q0[R], q1[R];
    uint16_t dd[R];  // 16-bit until used: a widening right after the load would wait for it
    QP_DEV void load(const PlRow (&rw)[R], uint32_t p, bool on) {
        const uint32_t o = on ? p * 32 : QP_NOOFF, od = on ? p * 2 : QP_NOOFF;
#pragma unroll
        for (int r = 0; r < R; r++) {
            q0[r] = __builtin_amdgcn_raw_buffer_load_b128(rw[r].q, o, 0, 0);
            q1[r] = __builtin_amdgcn_raw_buffer_load_b128(rw[r].q, o, 16, 0);
            dd[r] = __builtin_amdgcn_raw_buffer_load_b16(rw[r].d, od, 0, 0);
        }
    }
    QP_DEV void compute(uint32_t npc, const float4* __restrict__ xs, uint32_t p, float (&acc)[R]) const {
        float4 xv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = xs[i * npc + p];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) s += sdot4(q0[r][i], xv[i]);
#pragma unroll
            for (int i = 0; i < 4; i++) s += sdot4(q1[r][i], xv[4 + i]);
            acc[r] += h2f(dd[r]) * s;
        }
    }
};

// IQ4_NL: word i of the block's 16 nibble bytes holds weights 4i..4i+3 in its low nibbles and 16+4i..16+4i+3 in
// its high ones; s = sum over i of dot(lo_i, x_i) + dot(hi_i, x_(4+i)) (the reference's order, kds.js:80-88).
template <int R>
struct Piece<QP_IQ4_NL, R> {
    static constexpr uint32_t J = 8, QB = 16, LOADS = 2;
    u32x4 q[R];
    uint16_t dd[R];  // 16-bit until used: a widening right after the load would wait for it
    QP_DEV void load(const PlRow (&rw)[R], uint32_t p, bool on) {
        const uint32_t o = on ? p * 16 : QP_NOOFF, od = on ? p * 2 : QP_NOOFF;
#pragma unroll
        for (int r = 0; r < R; r++) {
            q[r] = __builtin_amdgcn_raw_buffer_load_b128(rw[r].q, o, 0, 0);
            dd[r] = __builtin_amdgcn_raw_buffer_load_b16(rw[r].d, od, 0, 0);
        }
    }
    QP_DEV void compute(uint32_t npc, const float4* __restrict__ xs, uint32_t p, float (&acc)[R]) const {
        float4 xv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = xs[i * npc + p];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t lo = iq4nl_lut4(q[r][i] & 0x0f0f0f0fu), hi = iq4nl_lut4((q[r][i] >> 4) & 0x0f0f0f0fu);
                s += sdot4(lo, xv[i]) + sdot4(hi, xv[4 + i]);
            }
            acc[r] += h2f(dd[r]) * s;
        }
    }
};

template <int R>
struct Piece<QP_F32, R> {
    static constexpr uint32_t J = 4, QB = 64, LOADS = 4;
    u32x4 w[R][4];
    QP_DEV void load(const PlRow (&rw)[R], uint32_t p, bool on) {
        const uint32_t o = on ? p * 64 : QP_NOOFF;
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) w[r][i] = __builtin_amdgcn_raw_buffer_load_b128(rw[r].q, o, 16 * i, 0);
    }
    QP_DEV void compute(uint32_t npc, const float4* __restrict__ xs, uint32_t p, float (&acc)[R]) const {
        float4 xv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = xs[i * npc + p];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++)
                s += __uint_as_float(w[r][i][0]) * xv[i].x + __uint_as_float(w[r][i][1]) * xv[i].y +
                     __uint_as_float(w[r][i][2]) * xv[i].z + __uint_as_float(w[r][i][3]) * xv[i].w;
            acc[r] += s;
        }
    }
};

QP_DEV uint64_t amax_key(float v, uint32_t idx) {
    if (v != v) return 0ull;  // NaN is never chosen (reference compares with '>')
    const uint32_t u = __float_as_uint(v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - idx);
}

// One segment as the item loop sees it (wave-uniform): rows row_base .. row_base + n - 1 of a tensor of rows_total
// rows; its row groups are workgroups wg0 .. of the launch's total.
struct PlSeg {
    uint64_t w, w2, y;
    uint32_t n, row_base, rows_total, mode, wg0;
};

// The pass a wavefront is on: its segment, first output row, and the R rows' resources.
template <int R>
struct PlPass {
    uint32_t si, mode, n, r0;
    bool pair;
};

// seg_at(i): segment i < nseg (in order of wg0).  total_wg row groups of 4 waves x R rows (R / 2 output rows per wave
// for a SwiGLU pair segment) over the grid.  x: the input row; norm_w: 0 or the fused RMSNorm weight.
template <int FMT, int R, int D, class SegAt>
QP_DEV void pl_gemv(SegAt seg_at, uint32_t nseg, uint32_t total_wg, uint64_t x, uint64_t norm_w, float eps,
                    uint32_t K, uint64_t amax) {
    using P = Piece<FMT, R>;
    extern __shared__ float4 xs[];
    __shared__ float red[4];
    __shared__ uint64_t wbest[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    x = uni64(x);  // the row read from the device step record: uniform, so its resource stays scalar
    const uint32_t npc = K / (4 * P::J);   // pieces per row
    const uint32_t ppl = (npc + 63) >> 6;  // piece slots per pass
    const uint32_t G = gridDim.x;
    const uint32_t mine = blockIdx.x < total_wg ? (total_wg - 1 - blockIdx.x) / G + 1 : 0;
    if (mine == 0) return;  // the whole workgroup
    const uint32_t n_total = mine * ppl;
    const uint64_t rowq = (uint64_t)npc * P::QB;

    auto seg_of = [&](uint32_t wg) __attribute__((always_inline)) {
        uint32_t s = 0;
        for (uint32_t i = 1; i < nseg; i++) s = wg >= seg_at(i).wg0 ? i : s;
        return s;
    };
    auto setup = [&](uint32_t k, PlPass<R>& ps) __attribute__((always_inline)) {
        const uint32_t wg = blockIdx.x + (k < mine ? k : 0) * G;
        ps.si = seg_of(wg);
        const PlSeg sg = seg_at(ps.si);
        ps.mode = sg.mode;
        ps.n = sg.n;
        ps.pair = sg.mode == QP_GEMV_SWIGLU;
        const uint32_t outs = ps.pair ? R / 2 : R;
        ps.r0 = (wg - sg.wg0) * 4 * outs + wave * outs;
    };
    // the resources of pass k's rows (empty past the wave's passes or the segment's rows)
    auto rows = [&](uint32_t k, PlRow (&rw)[R]) __attribute__((always_inline)) {
        PlPass<R> ps;
        setup(k, ps);
        const PlSeg sg = seg_at(ps.si);
        const uint64_t NB = (uint64_t)sg.rows_total * npc;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t o = (ps.pair && R > 1) ? (uint32_t)(r % (R / 2 > 0 ? R / 2 : 1)) : (uint32_t)r;
            const uint64_t base = (ps.pair && r >= R / 2) ? sg.w2 : sg.w;
            const bool on = k < mine && ps.r0 + o < ps.n;
            const uint64_t row = sg.row_base + (on ? ps.r0 + o : 0);
            rw[r].q = kq_rsrc(base + row * rowq, on ? rowq : 0);
            rw[r].d = kq_rsrc(base + NB * P::QB + row * npc * 2, (on && FMT != QP_F32) ? npc * 2 : 0);
        }
    };

    // 1. the input: this thread's float4s f = tid + 256 i, i < 8 (K <= 8192), as buffer loads (past K: 0); the norm
    // weight's first, under one uniform branch, then x, then the first items' weights, so that the wait for x counts
    // only the weight loads
    constexpr int NF = 8;
    const uint32_t nf4 = K >> 2;
    u32x4 xr[NF], nr[NF];
    if (norm_w) {
        const __amdgpu_buffer_rsrc_t rn = kq_rsrc(norm_w, 16ull * nf4);
#pragma unroll
        for (int i = 0; i < NF; i++) {
            const uint32_t f = tid + 256 * i;
            nr[i] = __builtin_amdgcn_raw_buffer_load_b128(rn, f < nf4 ? 16 * f : QP_NOOFF, 0, 0);
        }
    }
    {
        const __amdgpu_buffer_rsrc_t rx = kq_rsrc(x, 16ull * nf4);
#pragma unroll
        for (int i = 0; i < NF; i++) {
            const uint32_t f = tid + 256 * i;
            xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, f < nf4 ? 16 * f : QP_NOOFF, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the first D - 1 items' weights
    P buf[D];
    PlRow rwL[R];
    uint32_t kL = 0, jL = 0;  // the next item to load
    auto load_next = [&](P& X) __attribute__((always_inline)) {
        if (jL == 0) rows(kL, rwL);
        X.load(rwL, lane + 64 * jL, lane + 64 * jL < npc);
        if (++jL == ppl) {
            jL = 0;
            kL++;
        }
    };
#pragma unroll
    for (int d = 0; d + 1 < D; d++) load_next(buf[d]);
    __builtin_amdgcn_sched_barrier(0);

    // 3. stage x (times the norm weight) in LDS, piece-major; the sum of squares for the norm
    float ss = 0.0f;
    auto put = [&](uint32_t f, float4 v, float4 w) __attribute__((always_inline)) {
        if (norm_w) {
            ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
            v.x *= w.x;
            v.y *= w.y;
            v.z *= w.z;
            v.w *= w.w;
        }
        const uint32_t p = f / P::J, j = f % P::J;
        xs[j * npc + p] = v;
    };
    auto f4 = [](const u32x4 u) __attribute__((always_inline)) {
        return make_float4(__uint_as_float(u[0]), __uint_as_float(u[1]), __uint_as_float(u[2]),
                           __uint_as_float(u[3]));
    };
#pragma unroll
    for (int i = 0; i < NF; i++) {
        const uint32_t f = tid + 256 * i;
        if (f < nf4) put(f, f4(xr[i]), norm_w ? f4(nr[i]) : float4{});
    }
    for (uint32_t f = tid + 256 * NF; f < nf4; f += 256)  // K > 8192: the rest (this wait includes the weights)
        put(f, gload<float4>(x + 16ull * f), norm_w ? gload<float4>(norm_w + 16ull * f) : float4{});
    if (norm_w) {
        ss = wave_sum_v(ss, lane);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    float inv = 1.0f;
    if (norm_w) inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)K + eps);

    // 4. items
    constexpr int NO = 2;  // deferred outputs: lane L of register k holds output slot L + 64 k
    float outv[NO];
    uint32_t outk[NO];     // segment << 28 | row within the segment; all ones: nothing to write
#pragma unroll
    for (int k = 0; k < NO; k++) {
        outv[k] = 0.0f;
        outk[k] = 0xffffffffu;
    }
    uint32_t nout = 0;
    uint64_t best = 0;
    auto flush = [&](bool wait) __attribute__((always_inline)) {
        for (uint32_t si = 0; si < nseg; si++) {
            const PlSeg sg = seg_at(si);
#pragma unroll
            for (int k = 0; k < NO; k++) {
                if (lane + 64 * k < nout && outk[k] != 0xffffffffu && (outk[k] >> 28) == si) {
                    QP_GLOBAL float* y = reinterpret_cast<QP_GLOBAL float*>(sg.y) + (outk[k] & 0x0fffffffu);
                    *y = sg.mode == QP_GEMV_ACC ? *y + outv[k] : outv[k];
                }
            }
        }
        nout = 0;
        if (wait) __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xf << 8));  // drain the stores (rare)
    };
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    PlPass<R> PC;
    uint32_t kC = 0, jC = 0;  // the item being computed
    auto compute = [&](const P& X) __attribute__((always_inline)) {
        if (jC == 0) setup(kC, PC);
        // every lane: one past the row's pieces loaded zero weights (and scales), and reads a valid x; under a
        // branch, the wait for this item's loads would not cover the path that skips it
        const uint32_t p = lane + 64 * jC;
        X.compute(npc, xs, p < npc ? p : npc - 1, acc);
        if (++jC < ppl) return;
        // end of the pass: reduce across the wavefront and defer the outputs
        jC = 0;
        kC++;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = wave_sum_v(acc[r], lane) * inv;
        const uint32_t outs = PC.pair ? R / 2 : R;
        if (nout + outs > 64 * NO) flush(true);
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (PC.pair && r >= R / 2) break;
            const uint32_t row = PC.r0 + r;
            const float val = PC.pair ? (acc[r] / (1.0f + expf(-acc[r]))) * acc[r + R / 2] : acc[r];
            if (PC.mode == QP_GEMV_ARGMAX && row < PC.n) {
                const uint64_t key = amax_key(val, row);
                best = key > best ? key : best;
            }
#pragma unroll
            for (int k = 0; k < NO; k++)
                if (lane + 64 * k == nout + r) {
                    outv[k] = val;
                    outk[k] = row < PC.n ? (PC.si << 28) | row : 0xffffffffu;
                }
        }
        nout += outs;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
    };
    // whole rounds of D items (the loop body has no exit between its loads and the waits for them; loads past the
    // wave's last item are empty), then the remaining items, whose loads are already in flight
    uint32_t n0 = 0;
    for (; n0 + D <= n_total; n0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            load_next(buf[(d + D - 1) % D]);  // item n0 + d + D - 1
            compute(buf[d]);
        }
    }
#pragma unroll
    for (int d = 0; d + 1 < D; d++)
        if (n0 + d < n_total) compute(buf[d]);
    flush(false);
    if (amax) {
        if (lane == 0) wbest[wave] = best;
        __syncthreads();
        if (tid == 0) {
            uint64_t b = wbest[0];
            for (int i = 1; i < 4; i++) b = wbest[i] > b ? wbest[i] : b;
            mptr<uint64_t>(amax)[blockIdx.x] = b;
        }
    }
}

// Register sets in rotation (items whose loads are in flight + the one being multiplied).  Measured on the 14336 x
// 4096 and 4096 x 14336 GEMVs, 2 is faster than 3 or 4 for Q8_0, IQ4_NL and f32.
#ifndef QP_PL_D
#define QP_PL_D 2
#endif
template <int FMT, int R>
QP_DEV void gemv_seg_body(const QpGemvArgs& a) {
    const uint64_t t0 = tl_now();
    auto seg_at = [&](uint32_t i) __attribute__((always_inline)) {
        const QpGemvSeg& q = a.seg[i];
        return PlSeg{q.w, q.w2, q.y, q.n, q.row_base, q.rows_total, q.mode, q.wg0};
    };
    const uint32_t xrow = a.last_row ? paso_T(a.paso) - 1 : 0;
    constexpr int D = QP_PL_D;
    pl_gemv<FMT, R, D>(seg_at, a.nseg, a.total_wg, a.x + 4ull * xrow * a.k, a.norm_w, a.eps, a.k, a.amax);
    tl_rec(a.tseq, t0);
}

#define GEMV_KERNELS(NAME, FMT)                                                                          \
    KERNEL __launch_bounds__(256) void qp_gemv_##NAME##_r1(QpGemvArgs a) { gemv_seg_body<FMT, 1>(a); } \
    KERNEL __launch_bounds__(256) void qp_gemv_##NAME##_r2(QpGemvArgs a) { gemv_seg_body<FMT, 2>(a); } \
    KERNEL __launch_bounds__(256) void qp_gemv_##NAME##_r4(QpGemvArgs a) { gemv_seg_body<FMT, 4>(a); } \
    KERNEL __launch_bounds__(256) void qp_gemv_##NAME##_r8(QpGemvArgs a) { gemv_seg_body<FMT, 8>(a); }
GEMV_KERNELS(q8, QP_Q8_0)
GEMV_KERNELS(iq4nl, QP_IQ4_NL)
GEMV_KERNELS(f32, QP_F32)

// Gathered expert GEMV (reference matmul_*_e, kquants.js:256-304 and kds.js:110-186): grid.x row groups of 4 * R rows
// (R / 2 output rows per wave in SWIGLU mode), grid.y the job; job z multiplies expert sel[z] by input row z / tfijo.
template <int FMT, int R>
QP_DEV void gemv_exp_body(const QpGemvExpArgs& a) {
    const uint32_t njobs = a.njobs_fixed ? a.njobs_fixed : paso_T(a.paso) * a.kused;
    const uint32_t job = blockIdx.y;
    if (job >= njobs) return;
    uint32_t ex = __builtin_amdgcn_readfirstlane(cptr<uint32_t>(a.sel)[job]);
    if (ex >= a.n_exp) ex = a.n_exp - 1;  // routing only produces valid experts; never read outside the tensor
    const PlSeg one{a.w, a.w2, a.y + 4ull * job * a.n, a.n, ex * a.n, a.n_exp * a.n,
                    a.mode == QP_GEMV_SWIGLU ? (uint32_t)QP_GEMV_SWIGLU : (uint32_t)QP_GEMV_STORE, 0};
    pl_gemv<FMT, R, 2>([&](uint32_t) __attribute__((always_inline)) { return one; }, 1, gridDim.x,
                       a.x + 4ull * (job / a.tfijo) * a.k, 0, 0.0f, a.k, 0);
}

#define GEMV_EXP_KERNELS(NAME, FMT)                                                                              \
    KERNEL __launch_bounds__(256) void qp_gemv_exp_##NAME##_r2(QpGemvExpArgs a) { gemv_exp_body<FMT, 2>(a); } \
    KERNEL __launch_bounds__(256) void qp_gemv_exp_##NAME##_r4(QpGemvExpArgs a) { gemv_exp_body<FMT, 4>(a); }
GEMV_EXP_KERNELS(q8, QP_Q8_0)
GEMV_EXP_KERNELS(iq4nl, QP_IQ4_NL)
GEMV_EXP_KERNELS(f32, QP_F32)

// ====================================================================================== K-quant GEMV (one token)
// Q4_K / Q6_K y = W.x for one token: the fused `gemv` op and the reference's matmul_q4k_1 / matmul_q6k_1
// (kquants.js:188-251) and gathered-expert matmul_q4k_e / matmul_q6k_e (kquants.js:256-304).
//
// One lane owns one super-block (256 weights) of a row.  With the row chunk-plane layout (qp_args.h) the lane's
// 9 (Q4_K) or 13 + 1 (Q6_K) loads are 16-byte loads whose lanes read contiguous runs, and the block header needs
// no exchange between lanes.  A load instruction covers S = 64/nbp rows (nbp = nb rounded up to a power of two;
// lanes past nb idle); a "unit" is the R rows per lane that share one pass over the staged input.  Weights are
// read through a buffer resource so that a lane without a row (past the segment) passes an offset past the end
// and costs no memory traffic.  The input vector is staged once per workgroup in LDS (block b's 64 float4 at
// b*65: the one-float4 pad spreads the lanes' 16-byte reads over the banks) with per-group sums of x; its global
// loads are issued before the first unit's weight loads and awaited on their own.  The dot products use the f16
// form of a nibble: (w & 0x000f000f) holds two f16 subnormals q*2^-24, which v_fma_mix multiplies exactly by
// the f32 x; the power of two is taken out of each sub-block sum.  Results are written after the unit loop: a
// store in flight would make every later load wait for it.
//
// Semantics per row follow the reference's factoring: y = sum over sub-blocks of (d*sc)*sum(q*x) - (dmin*m)*sum(x)
// (Q4_K) and (d*sc)*(sum(q*x) - 32*sum(x)) over 16-element groups (Q6_K); the summation order is this kernel's.

template <int FMT>
struct KQ;
template <>
struct KQ<QP_Q4_K> {
    static constexpr int CPB = 9, RB = 144, LOADS = 9, GROUP = 32;  // GROUP: elements per x sum
};
template <>
struct KQ<QP_Q2_K> {
    static constexpr int CPB = 5, RB = 80, LOADS = 6, GROUP = 16;  // + the (d, dmin) word
};
template <>
struct KQ<QP_Q3_K> {
    static constexpr int CPB = 7, RB = 112, LOADS = 7, GROUP = 16;
};
template <>
struct KQ<QP_Q5_K> {
    static constexpr int CPB = 11, RB = 176, LOADS = 11, GROUP = 32;
};
template <>
struct KQ<QP_Q6_K> {
    static constexpr int CPB = 13, RB = 208, LOADS = 14, GROUP = 16;
};
// Segments of either format in one launch (each unit takes its segment's path; a Q4_K unit issues the Q6_K
// number of loads, the extra ones past the end, so the wait counts do not depend on the format).
#define QP_KQ_MIX 255
template <>
struct KQ<QP_KQ_MIX> {
    static constexpr int CPB = 13, RB = 0, LOADS = 14, GROUP = 16;
};

template <int FMT, int R>
struct KUnit {
    u32x4 c[R][KQ<FMT>::CPB];
    uint32_t d[R];  // Q6_K: the block's f16 d; Q2_K: d | dmin << 16
};

// acc + (f16 half SEL of m) * x, in one v_fma_mix_f32 (the f16 operand may be subnormal).
template <int SEL>
QP_DEV float fmix(uint32_t m, float x, float acc) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 h = __builtin_bit_cast(h2, m);
    return fmaf((float)(SEL ? h.y : h.x), x, acc);
}

// v is produced before this point and no memory access moves across it: keeps the compiler from hoisting every
// LDS read of the input above the arithmetic that consumes the previous ones (the reads are loop-invariant).
QP_DEV void kq_fence(float& v) { asm volatile("" : "+v"(v)::"memory"); }

// A 32-bit load past the CU's L1 (sc0): data another CU of the XCD stored before a barrier, never read here before.
QP_DEV uint32_t ld_sc0(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 1);
}

// Arrival of one of the n workgroups that share a counter word in their XCD's L2 (a launch whose workgroups go to
// the 8 XCDs round robin by linear id x + 8y puts every workgroup of grid column x on one XCD; the kernels that call
// this rely on it).  Each arrival adds 1 + (its XCD id << 16): the low half counts the arrivals, the high half sums
// their XCD ids.  The arrival that brings the count to n is the last (returns true) and resets the word; if the ids
// it sums are not n times its own, or a count ever passes n (arrivals left over from a launch whose workgroups were
// spread over XCDs, so that no add saw the full count), it sets bit 0 of *err (a device word the host checks) instead
// of letting the placement fail silently.  The work after a last arrival runs either way, so every workgroup ends.
// One thread per workgroup calls it; n <= 4096.
QP_DEV bool xcd_arrive(uint64_t cnt, uint32_t n, uint64_t err) {
    const uint32_t xid = __builtin_amdgcn_s_getreg(20 | (15 << 11)) & 15u;  // HW_REG_XCC_ID
    const uint32_t add = 1u + (xid << 16);
    QP_GLOBAL uint32_t* c = reinterpret_cast<QP_GLOBAL uint32_t*>(cnt);
    const uint32_t t = __hip_atomic_fetch_add(c, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) + add;
    const uint32_t got = t & 0xffffu;
    const bool last = got == n;
    if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if ((last && (t >> 16) != n * xid) || got > n)
        __hip_atomic_fetch_or(reinterpret_cast<QP_GLOBAL uint32_t*>(err), 1u, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    return last;
}

// Bytes of LDS the K-quant GEMV uses for a K-wide input (staged x + group sums + reduction slots).
QP_DEV uint32_t kq_lds_offset_sum(uint32_t K) { return (K >> 8) * 65 * 16; }

// One segment as the unit loop sees it (wave-uniform).
struct KSeg {
    uint64_t w, w2, y;
    uint32_t n, row_base, rows_total, mode, u0, fmt;
};

// G16: the x sums are per 16 elements (the mixed launch's layout): a sub-block's sum is the sum of its two halves,
// the same value the 32-element staging computes.
template <class U, int R, bool G16 = false>
QP_DEV void kq_dot_q4k(const U& B, const float4* xb4, const float* xsb, float (&tot)[R]) {
    float sxs[8];
    if constexpr (G16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = *reinterpret_cast<const float4*>(xsb + 4 * i);
            sxs[2 * i] = t.x + t.y;
            sxs[2 * i + 1] = t.z + t.w;
        }
    } else {
        const float4 sa = *reinterpret_cast<const float4*>(xsb);
        const float4 sb = *reinterpret_cast<const float4*>(xsb + 4);
        sxs[0] = sa.x; sxs[1] = sa.y; sxs[2] = sa.z; sxs[3] = sa.w;
        sxs[4] = sb.x; sxs[5] = sb.y; sxs[6] = sb.z; sxs[7] = sb.w;
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {  // sub-block pair: quant bytes p*32..p*32+31, chunks 1+2p, 2+2p
        float alo[R], ahi[R];
#pragma unroll
        for (int r = 0; r < R; r++) alo[r] = ahi[r] = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {  // elements l = 16h..16h+15 of sub-blocks 2p (low nibbles), 2p+1 (high)
            float4 x0[4], x1[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x0[i] = xb4[(2 * p) * 8 + 4 * h + i];
                x1[i] = xb4[(2 * p + 1) * 8 + 4 * h + i];
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const u32x4 qq = B.c[r][1 + 2 * p + h];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t wv = qq[i];  // bytes l, l+1, l+2, l+3
                    const uint32_t m0 = wv & 0x000f000fu, m1 = wv & 0x00f000f0u;
                    const uint32_t tw = wv >> 8;
                    const uint32_t m2 = tw & 0x000f000fu, m3 = tw & 0x00f000f0u;
                    alo[r] = fmix<0>(m0, x0[i].x, alo[r]);
                    alo[r] = fmix<0>(m2, x0[i].y, alo[r]);
                    alo[r] = fmix<1>(m0, x0[i].z, alo[r]);
                    alo[r] = fmix<1>(m2, x0[i].w, alo[r]);
                    ahi[r] = fmix<0>(m1, x1[i].x, ahi[r]);
                    ahi[r] = fmix<0>(m3, x1[i].y, ahi[r]);
                    ahi[r] = fmix<1>(m1, x1[i].z, ahi[r]);
                    ahi[r] = fmix<1>(m3, x1[i].w, ahi[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                kq_fence(alo[r]);
                kq_fence(ahi[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const u32x4 hd = B.c[r][0];
            const float d = h2f(hd[0] & 0xffffu), dm = h2f(hd[0] >> 16);
            uint32_t sc0, mn0, sc1, mn1;
            q4k_sm(hd[1], hd[2], hd[3], 2 * p, sc0, mn0);
            q4k_sm(hd[1], hd[2], hd[3], 2 * p + 1, sc1, mn1);
            // low nibbles were summed as q*2^-24, high nibbles as 16q*2^-24
            tot[r] += (d * (float)sc0) * (alo[r] * 16777216.0f) - (dm * (float)mn0) * sxs[2 * p];
            tot[r] += (d * (float)sc1) * (ahi[r] * 1048576.0f) - (dm * (float)mn1) * sxs[2 * p + 1];
        }
    }
}

// Q5_K: chunk 0 the Q4_K header, chunks 1-2 qh[32], chunks 3-10 qs[128].  Each nibble mask of kq_dot_q4k also
// takes its element's high bit: with g = qh >> 2p, bit 2p of a qh byte lands on the nibble's 16 (low nibbles, q
// summed as q*2^-24) and bit 2p+1 on its 256 (high nibbles, summed as 16q*2^-24).
template <class U, int R>
QP_DEV void kq_dot_q5k(const U& B, const float4* xb4, const float* xsb, float (&tot)[R]) {
    float sxs[8];
    {
        const float4 sa = *reinterpret_cast<const float4*>(xsb);
        const float4 sb = *reinterpret_cast<const float4*>(xsb + 4);
        sxs[0] = sa.x; sxs[1] = sa.y; sxs[2] = sa.z; sxs[3] = sa.w;
        sxs[4] = sb.x; sxs[5] = sb.y; sxs[6] = sb.z; sxs[7] = sb.w;
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
        float alo[R], ahi[R];
#pragma unroll
        for (int r = 0; r < R; r++) alo[r] = ahi[r] = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4 x0[4], x1[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x0[i] = xb4[(2 * p) * 8 + 4 * h + i];
                x1[i] = xb4[(2 * p + 1) * 8 + 4 * h + i];
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const u32x4 qq = B.c[r][3 + 2 * p + h];
                const u32x4 hh = B.c[r][1 + h];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t wv = qq[i], g = hh[i] >> (2 * p);  // bytes l .. l+3
                    const uint32_t tw = wv >> 8;
                    const uint32_t m0 = (wv & 0x000f000fu) | ((g << 4) & 0x00100010u);
                    const uint32_t m1 = (wv & 0x00f000f0u) | ((g << 7) & 0x01000100u);
                    const uint32_t m2 = (tw & 0x000f000fu) | ((g >> 4) & 0x00100010u);
                    const uint32_t m3 = (tw & 0x00f000f0u) | ((g >> 1) & 0x01000100u);
                    alo[r] = fmix<0>(m0, x0[i].x, alo[r]);
                    alo[r] = fmix<0>(m2, x0[i].y, alo[r]);
                    alo[r] = fmix<1>(m0, x0[i].z, alo[r]);
                    alo[r] = fmix<1>(m2, x0[i].w, alo[r]);
                    ahi[r] = fmix<0>(m1, x1[i].x, ahi[r]);
                    ahi[r] = fmix<0>(m3, x1[i].y, ahi[r]);
                    ahi[r] = fmix<1>(m1, x1[i].z, ahi[r]);
                    ahi[r] = fmix<1>(m3, x1[i].w, ahi[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                kq_fence(alo[r]);
                kq_fence(ahi[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const u32x4 hd = B.c[r][0];
            const float d = h2f(hd[0] & 0xffffu), dm = h2f(hd[0] >> 16);
            uint32_t sc0, mn0, sc1, mn1;
            q4k_sm(hd[1], hd[2], hd[3], 2 * p, sc0, mn0);
            q4k_sm(hd[1], hd[2], hd[3], 2 * p + 1, sc1, mn1);
            tot[r] += (d * (float)sc0) * (alo[r] * 16777216.0f) - (dm * (float)mn0) * sxs[2 * p];
            tot[r] += (d * (float)sc1) * (ahi[r] * 1048576.0f) - (dm * (float)mn1) * sxs[2 * p + 1];
        }
    }
}

// acc + the dot of 16 consecutive x (4 float4) with the bytes of q4[0..3] (4 per dword, each < 256), as f16
// subnormals q*2^-24.
template <int R>
QP_DEV float kq_dot16(const u32x4& q4, const float4 (&xv)[4], float acc) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t e = __builtin_amdgcn_perm(0u, q4[c], 0x0c020c00u);  // bytes 0, 2 as f16 halves
        const uint32_t o = __builtin_amdgcn_perm(0u, q4[c], 0x0c030c01u);  // bytes 1, 3
        acc = fmix<0>(e, xv[c].x, acc);
        acc = fmix<0>(o, xv[c].y, acc);
        acc = fmix<1>(e, xv[c].z, acc);
        acc = fmix<1>(o, xv[c].w, acc);
    }
    return acc;
}

// Q3_K (chunks: hmask 0-1, qs 2-5, scales and d 6): element (h, jj, l) has q' = q2 | hbit << 2 in 0..7 and the
// value (d * (s6 - 32)) * (q' - 4) over 16-element groups s = 8h + 2jj + l/16.
template <class U, int R>
QP_DEV void kq_dot_q3k(const U& B, const float4* xb4, const float* xsb, float (&tot)[R]) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int lh = 0; lh < 2; lh++) {
            float aq[R][4];
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int qd = 0; qd < 4; qd++) aq[r][qd] = 0.0f;
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                float4 xv[4];
#pragma unroll
                for (int c = 0; c < 4; c++) xv[c] = xb4[(h * 128 + qd * 32 + lh * 16) / 4 + c];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const u32x4 qs = B.c[r][2 + 2 * h + lh], hm = B.c[r][lh];
                    u32x4 q;
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        q[c] = ((qs[c] >> (2 * qd)) & 0x03030303u) | (((hm[c] >> (4 * h + qd)) & 0x01010101u) << 2);
                    aq[r][qd] = kq_dot16<R>(q, xv, aq[r][qd]);
                }
#pragma unroll
                for (int r = 0; r < R; r++) kq_fence(aq[r][qd]);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const u32x4 sw = B.c[r][6];
                const float dd = h2f(sw[3] & 0xffffu);
#pragma unroll
                for (int qd = 0; qd < 4; qd++) {
                    const uint32_t si = h * 8 + qd * 2 + lh;
                    const float sc = (float)q3k_scale6(sw[0], sw[1], sw[2], si) - 32.0f;
                    const float sx = xsb[(h * 128 + qd * 32 + lh * 16) / 16];
                    tot[r] += (dd * sc) * (aq[r][qd] * 16777216.0f - 4.0f * sx);
                }
            }
        }
    }
}

// Q2_K (chunks: scales 0, qs 1-4; d and dmin in B.d): element (h, jj, l) has q = (qs >> 2jj) & 3 and the value
// (d * (sc & 15)) * q - dmin * (sc >> 4) over 16-element groups j = 8h + 2jj + l/16.
template <class U, int R>
QP_DEV void kq_dot_q2k(const U& B, const float4* xb4, const float* xsb, float (&tot)[R]) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int lh = 0; lh < 2; lh++) {
            float aq[R][4];
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int qd = 0; qd < 4; qd++) aq[r][qd] = 0.0f;
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                float4 xv[4];
#pragma unroll
                for (int c = 0; c < 4; c++) xv[c] = xb4[(h * 128 + qd * 32 + lh * 16) / 4 + c];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const u32x4 qs = B.c[r][1 + 2 * h + lh];
                    u32x4 q;
#pragma unroll
                    for (int c = 0; c < 4; c++) q[c] = (qs[c] >> (2 * qd)) & 0x03030303u;
                    aq[r][qd] = kq_dot16<R>(q, xv, aq[r][qd]);
                }
#pragma unroll
                for (int r = 0; r < R; r++) kq_fence(aq[r][qd]);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const u32x4 scw = B.c[r][0];
                const float d = h2f(B.d[r] & 0xffffu), dm = h2f(B.d[r] >> 16);
#pragma unroll
                for (int qd = 0; qd < 4; qd++) {
                    const uint32_t j = h * 8 + qd * 2 + lh;
                    const uint32_t sc = (scw[j >> 2] >> ((j & 3) * 8)) & 0xffu;
                    const float sx = xsb[(h * 128 + qd * 32 + lh * 16) / 16];
                    tot[r] += (d * (float)(sc & 15u)) * (aq[r][qd] * 16777216.0f) - (dm * (float)(sc >> 4)) * sx;
                }
            }
        }
    }
}

template <class U, int R>
QP_DEV void kq_dot_q6k(const U& B, const float4* xb4, const float* xsb, float (&tot)[R]) {
    // element (h, qd, l): ql chunk h*4 + (qd&1)*2 + l/16, nibble qd>>1; qh chunk 8 + h*2 + l/16, bits 2qd;
    // scale s = h*8 + qd*2 + l/16 (chunk 12)
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int lh = 0; lh < 2; lh++) {
            float aq[R][4];
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int qd = 0; qd < 4; qd++) aq[r][qd] = 0.0f;
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                float4 xv[4];
#pragma unroll
                for (int c = 0; c < 4; c++) xv[c] = xb4[(h * 128 + qd * 32 + lh * 16) / 4 + c];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const u32x4 lo = B.c[r][h * 4 + (qd & 1) * 2 + lh];
                    const u32x4 hi = B.c[r][8 + h * 2 + lh];
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const uint32_t q = ((lo[c] >> ((qd >> 1) * 4)) & 0x0f0f0f0fu) |
                                           (((hi[c] >> (qd * 2)) & 0x03030303u) << 4);
                        const uint32_t e = __builtin_amdgcn_perm(0u, q, 0x0c020c00u);  // bytes 0, 2 as f16 halves
                        const uint32_t o = __builtin_amdgcn_perm(0u, q, 0x0c030c01u);  // bytes 1, 3
                        aq[r][qd] = fmix<0>(e, xv[c].x, aq[r][qd]);
                        aq[r][qd] = fmix<0>(o, xv[c].y, aq[r][qd]);
                        aq[r][qd] = fmix<1>(e, xv[c].z, aq[r][qd]);
                        aq[r][qd] = fmix<1>(o, xv[c].w, aq[r][qd]);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; r++) kq_fence(aq[r][qd]);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const u32x4 scw = B.c[r][12];
                const float dd = h2f(B.d[r]);
#pragma unroll
                for (int qd = 0; qd < 4; qd++) {
                    const int si = h * 8 + qd * 2 + lh;
                    const int sc = (int)(int8_t)((scw[si >> 2] >> ((si & 3) * 8)) & 0xffu);
                    const float sx = xsb[(h * 128 + qd * 32 + lh * 16) / 16];
                    tot[r] += (dd * (float)sc) * (aq[r][qd] * 16777216.0f - 32.0f * sx);
                }
            }
        }
    }
}

// Where the weights of x-block b of row `row` live.  KDense: the row's own blocks (row r of a tensor with nb blocks
// per row, the chunk-plane layout above).  A gathered layout maps the x blocks onto rows of several tensors.
struct KDense {
    static constexpr bool SCALED = false;
    QP_DEV uint32_t nbw(uint32_t nb) const { return nb; }  // blocks per weight row
    // weight row and block within it that multiply x-block b of output row `row`
    QP_DEV void loc(uint32_t row, uint32_t b, uint32_t& wr, uint32_t& wb) const { wr = row; wb = b; }
    QP_DEV float xscale(uint32_t) const { return 1.0f; }
};

// The unit loop.  seg_at(i) returns segment i (i < nseg); the wave's units are w, w + W, ... < total_units,
// segment i owning units [u0_i, u0_{i+1}).  XS: x sub-blocks of 32 per thread for staging (K <= XS * 8192).
// lay: the weight layout (KDense, or a gathered one whose x sub-blocks may also carry a scale).  pro: called once
// the input loads are issued and before the first segment is read (work that decides the segments overlaps them).
struct KNoPro {
    QP_DEV void operator()() const {}
};
// NT: threads per workgroup (256, or 512 for the no-norm variant of long rows: one input staging shared by eight
// wavefronts).  NORM: the fused RMSNorm prologue is compiled in.
// EXTRA: vector-memory loads pro() issues (counted in the wait for the input).  wgi / wgn: this workgroup's index
// among the wgn that share the units (wgn = 0: the grid's x dimension).
template <int FMT, int R, int XS, class SegAt, class Lay = KDense, class Pro = KNoPro, int NT = 256, bool NORM = true,
          int EXTRA = 0>
QP_DEV void kq_gemv(SegAt seg_at, uint32_t nseg, uint32_t total_units, uint64_t x, uint64_t norm_w, float eps,
                    uint32_t K, uint64_t amax, Lay lay = Lay(), Pro pro = Pro(), uint32_t wgi = 0, uint32_t wgn = 0) {
    extern __shared__ float4 xs[];
    float* xsum = reinterpret_cast<float*>(xs + (K >> 8) * 65);
    constexpr uint32_t nwv = NT / 64;
    __shared__ float red[nwv];
    __shared__ uint64_t wbest[nwv];
    if constexpr (!NORM) norm_w = 0;
    // timeline phase kinds: 0 mixed Q/K/V, 1 Q4_K one row per slot, 2 Q4_K pairs, 3 Q6_K long rows, 4 Q6_K, 5 other
    constexpr uint32_t TLK = FMT == QP_KQ_MIX ? 0 : (FMT == QP_Q4_K && R == 1 && NT == 256) ? 1
                           : (FMT == QP_Q4_K && R == 2) ? 2 : (FMT == QP_Q6_K && NT == 512) ? 3 : FMT == QP_Q6_K ? 4 : 5;
    tl_ph(TLK, 0);
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nb = K >> 8;
    uint32_t nbp = 1;
    while (nbp < nb) nbp <<= 1;
    const uint32_t S = 64 / nbp, s = lane / nbp, b = lane % nbp;
    const bool lane_on = b < nb;
    const uint32_t W = (wgn ? wgn : gridDim.x) * nwv, w = (wgn ? wgi : blockIdx.x) * nwv + wave;
    const uint32_t nmine = w < total_units ? (total_units - 1 - w) / W + 1 : 0;
    const uint32_t ngrp = K / KQ<FMT>::GROUP;

    // 1. this thread's share of x (and of the norm weight): float4 f = tid + NT i of the K / 4, so that each load
    // instruction of a wave reads 1 KB contiguous (8 lanes per cache line; one lane per line costs the address
    // unit 8x more work, and the weight loads queue behind it).  K % 256 == 0 keeps the bound wave-uniform.
    // Where an earlier load has to be waited for alone (pro()'s, or the caller's ahead of a gathered layout), the
    // input loads are buffer loads out of branches (a float4 past K reads 0) and come last: the compiler then
    // counts at least NF loads after the earlier one.  The norm weight's loads go first, under one uniform branch.
    // Elsewhere a float4 past K is skipped by a wave-uniform branch (K % 256 == 0), which issues fewer loads.
    constexpr int NF = 8 * XS;
    const uint32_t nf4 = K >> 2;
    float4 xr[NF], nr[NF];
    constexpr bool BF = !__is_same(Pro, KNoPro) || !__is_same(Lay, KDense);
    if constexpr (!BF) {
#pragma unroll
        for (int i = 0; i < NF; i++) {
            const uint32_t f = tid + NT * i;
            xr[i] = f < nf4 ? gload<float4>(x + 16ull * f) : float4{0.0f, 0.0f, 0.0f, 0.0f};
            if (norm_w) nr[i] = f < nf4 ? gload<float4>(norm_w + 16ull * f) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    } else {
        const __amdgpu_buffer_rsrc_t rxs = kq_rsrc(x, 16ull * nf4);
        if (norm_w) {
            const __amdgpu_buffer_rsrc_t rns = kq_rsrc(norm_w, 16ull * nf4);
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const uint32_t f = tid + NT * i;
                const u32x4 n = __builtin_amdgcn_raw_buffer_load_b128(rns, f < nf4 ? 16 * f : 0x80000000u, 0, 0);
                nr[i] = make_float4(__uint_as_float(n[0]), __uint_as_float(n[1]), __uint_as_float(n[2]),
                                    __uint_as_float(n[3]));
            }
        }
#pragma unroll
        for (int i = 0; i < NF; i++) {
            const uint32_t f = tid + NT * i;
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rxs, f < nf4 ? 16 * f : 0x80000000u, 0, 0);
            xr[i] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                __uint_as_float(v[3]));
        }
    }
    float xsc[NF];
#pragma unroll
    for (int i = 0; i < NF; i++) {
        const uint32_t q = (tid + NT * i) >> 3;   // the float4's sub-block of 32
        xsc[i] = lay.xscale(q < (K >> 5) ? q : 0);  // every lane (a gathered layout shuffles across the wave)
    }
    pro();
    __builtin_amdgcn_sched_barrier(0);

    // 2. the first unit's weights
    auto seg_of = [&](uint32_t g) __attribute__((always_inline)) {
        uint32_t si = 0;
        for (uint32_t i = 1; i < nseg; i++) si = g >= seg_at(i).u0 ? i : si;
        return si;
    };
    KUnit<FMT, R> buf;
    auto issue = [&](KUnit<FMT, R>& B, uint32_t n) __attribute__((always_inline)) {
        const uint32_t g = w + n * W;
        const bool uv = n < nmine;
        const KSeg sg = seg_at(seg_of(uv ? g : w));
        const uint32_t u = (uv ? g : w) - sg.u0;
        const bool pair = sg.mode == QP_GEMV_SWIGLU;
        const bool q6 = FMT == QP_KQ_MIX ? sg.fmt == QP_Q6_K : FMT == QP_Q6_K;
        const uint32_t nbw = lay.nbw(nb);
        // bytes per weight row (and per tensor row, with the Q6_K d array after the rows)
        const uint32_t rbw = FMT == QP_KQ_MIX ? (q6 ? 208 : 144) : KQ<FMT>::RB;
        const uint64_t tbytes = (uint64_t)sg.rows_total * nbw * (q6 ? 210 : FMT == QP_Q2_K ? 84 : rbw);
        const __amdgpu_buffer_rsrc_t rs0 = kq_rsrc(sg.w, tbytes);
        const __amdgpu_buffer_rsrc_t rs1 = kq_rsrc(pair ? sg.w2 : sg.w, tbytes);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t lr = pair ? u * S + s : (u * R + r) * S + s;
            const bool on = uv && lane_on && lr < sg.n;
            // weight row wr, block wb: chunk c at wr*nbw*rb + c*nbw*16 + wb*16
            uint32_t wr, wb;
            lay.loc(sg.row_base + lr, b, wr, wb);
            const uint32_t vo = on ? wr * nbw * rbw + wb * 16 : 0x80000000u;
            const __amdgpu_buffer_rsrc_t rs = (pair && r == 1) ? rs1 : rs0;
#pragma unroll
            for (int c = 0; c < KQ<FMT>::CPB; c++)
                B.c[r][c] = __builtin_amdgcn_raw_buffer_load_b128(
                    rs, (FMT != QP_KQ_MIX || c < 9 || q6) ? vo : 0x80000000u, c * nbw * 16, 0);
            if constexpr (FMT == QP_Q6_K || FMT == QP_KQ_MIX)
                B.d[r] = __builtin_amdgcn_raw_buffer_load_b16(
                    rs, (on && q6) ? sg.rows_total * nbw * 208 + (wr * nbw + wb) * 2 : 0x80000000u, 0, 0);
            if constexpr (FMT == QP_Q2_K)
                B.d[r] = __builtin_amdgcn_raw_buffer_load_b32(
                    rs, on ? sg.rows_total * nbw * 80 + (wr * nbw + wb) * 4 : 0x80000000u, 0, 0);
        }
    };
    issue(buf, 0);
    // an accumulating segment: the y value each lane adds its first unit's output to is loaded now, behind the
    // weights, so that the stores at the end do not wait for a load (lane L < R S holds output L of the unit: row
    // u R S + L).  One load per lane always (past the rows: offset out of range, no traffic), so the wait below
    // counts it.
    float ypre;
    {
        const KSeg sg0 = seg_at(seg_of(w));
        const uint32_t lr = (w - sg0.u0) * R * S + lane;
        const bool on = nmine > 0 && sg0.mode == QP_GEMV_ACC && lane < R * S && lr < sg0.n;
        ypre = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(kq_rsrc(sg0.y, 4ull * sg0.n), on ? 4 * lr : 0x80000000u, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);
    {
        // the x loads are the oldest in flight: wait for them alone
        constexpr int n = R * KQ<FMT>::LOADS + EXTRA + 1 > 63 ? 63 : R * KQ<FMT>::LOADS + EXTRA + 1;
        __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8));
    }
    tl_ph(TLK, 1);  // input arrived

    // 3. stage x (times the norm weight) in LDS with the group sums; sum of squares for the norm
    // LDS: float4 f at f + f / 64 (one pad per 256 inputs); the group sums of 32 (or 16) inputs over the 8 (or 4)
    // consecutive lanes that hold them
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NF; i++) {
        const uint32_t f = tid + NT * i;
        if (NT * i >= nf4) break;  // uniform: no float4 of this round exists
        float4 v = xr[i];
        if constexpr (Lay::SCALED) {
            const float c = xsc[i];
            v.x *= c;
            v.y *= c;
            v.z *= c;
            v.w *= c;
        }
        if (norm_w) {
            ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
            const float4 nw4 = nr[i];
            v.x *= nw4.x;
            v.y *= nw4.y;
            v.z *= nw4.z;
            v.w *= nw4.w;
        }
        float gs = (v.x + v.y) + (v.z + v.w);
        gs += bfly_f<0>(gs, lane);
        gs += bfly_f<1>(gs, lane);
        if constexpr (KQ<FMT>::GROUP == 32) gs += bfly_f<2>(gs, lane);
        if (f < nf4) {
            xs[f + (f >> 6)] = v;
            if constexpr (KQ<FMT>::GROUP == 32) {
                if ((lane & 7) == 0) xsum[f >> 3] = gs;
            } else {
                if ((lane & 3) == 0) xsum[f >> 2] = gs;
            }
        }
    }
    if (norm_w) {
        ss = wave_sum_v(ss, lane);  // lane exchanges, no LDS round trips
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    float inv = 1.0f;
    if (norm_w) {
        float t = 0.0f;
        for (uint32_t i = 0; i < nwv; i++) t += red[i];
        inv = 1.0f / sqrtf(t / (float)K + eps);
    }
    (void)ngrp;
    tl_ph(TLK, 2);  // input staged

    // 4. units
    constexpr int NO = 2;  // deferred outputs: lane L of register k holds output L + 64k of this wave
    float outv[NO];
    uint32_t outk[NO];     // segment << 28 | row within the segment
    uint32_t pre = 0;      // bit k: outv[k] already holds y + the output (an accumulating first unit)
#pragma unroll
    for (int k = 0; k < NO; k++) {
        outv[k] = 0.0f;
        outk[k] = 0;
    }
    uint32_t nout = 0;
    uint64_t best = 0;
    auto flush = [&](bool wait) __attribute__((always_inline)) {
        for (uint32_t si = 0; si < nseg; si++) {
            const KSeg sg = seg_at(si);
#pragma unroll
            for (int k = 0; k < NO; k++) {
                if (lane + 64 * k < nout && outk[k] != 0xffffffffu && (outk[k] >> 28) == si) {
                    QP_GLOBAL float* y = reinterpret_cast<QP_GLOBAL float*>(sg.y) + (outk[k] & 0x0fffffffu);
                    *y = (sg.mode == QP_GEMV_ACC && !((pre >> k) & 1u)) ? *y + outv[k] : outv[k];
                }
            }
        }
        nout = 0;
        // a store in flight makes the compiler wait for every later load; drain it here (rare)
        if (wait) __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xf << 8));
    };
    const uint32_t sb = lane_on ? b : 0;
    const float4* xb4 = xs + sb * 65;
    const float* xsb = xsum + sb * (256 / KQ<FMT>::GROUP);
    for (uint32_t n = 0; n < nmine; n++) {
        asm volatile("" ::: "memory");
        float tot[R];
#pragma unroll
        for (int r = 0; r < R; r++) tot[r] = 0.0f;
        const uint32_t g = w + n * W;
        const uint32_t si = seg_of(g);
        const KSeg sg = seg_at(si);
        if constexpr (FMT == QP_Q4_K) {
            kq_dot_q4k<KUnit<FMT, R>, R>(buf, xb4, xsb, tot);
        } else if constexpr (FMT == QP_Q5_K) {
            kq_dot_q5k<KUnit<FMT, R>, R>(buf, xb4, xsb, tot);
        } else if constexpr (FMT == QP_Q3_K) {
            kq_dot_q3k<KUnit<FMT, R>, R>(buf, xb4, xsb, tot);
        } else if constexpr (FMT == QP_Q2_K) {
            kq_dot_q2k<KUnit<FMT, R>, R>(buf, xb4, xsb, tot);
        } else if constexpr (FMT == QP_Q6_K) {
            kq_dot_q6k<KUnit<FMT, R>, R>(buf, xb4, xsb, tot);
        } else {
            if (sg.fmt == QP_Q6_K) kq_dot_q6k<KUnit<FMT, R>, R>(buf, xb4, xsb, tot);
            else kq_dot_q4k<KUnit<FMT, R>, R, true>(buf, xb4, xsb, tot);
        }
        const uint32_t u = g - sg.u0;
        const bool pair = sg.mode == QP_GEMV_SWIGLU;
        if (n == 0) tl_ph(TLK, 3);  // first unit's weights consumed
        issue(buf, n + 1);
        // reduce over the nbp lanes of each slot, then hand each output to its deferred lane
        float v[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            // the butterfly of lane exchanges over the slot's nbp lanes (aligned, a power of two; wave-uniform
            // branches): quad steps, then the mirror within 8 and 16 lanes, the row pair, the halves
            float t = lane_on ? tot[r] : 0.0f;
            if (nbp > 1) t += bfly_f<0>(t, lane);
            if (nbp > 2) t += bfly_f<1>(t, lane);
            if (nbp > 4) t += bfly_f<2>(t, lane);
            if (nbp > 8) t += bfly_f<3>(t, lane);
            if (nbp > 16) t += bfly_f<4>(t, lane);
            if (nbp > 32) t += bfly_f<5>(t, lane);
            v[r] = t * inv;
        }
        const uint32_t nper = pair ? 1 : R;
        if (nout + nper * S > 64 * NO) flush(true);
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (pair && r > 0) break;
            const float val = pair ? (v[0] / (1.0f + expf(-v[0]))) * v[R - 1] : v[r];
            const uint32_t lr0 = pair ? u * S : (u * R + r) * S;
            const int base = (int)(nout + r * S);
#pragma unroll
            for (int k = 0; k < NO; k++) {
                const int rel = (int)lane + 64 * k - base;
                const bool slot = rel >= 0 && rel < (int)S;
                const bool take = slot && lr0 + rel < sg.n;
                const float vv = __shfl(val, (take ? rel : 0) * (int)nbp, 64);
                if (take) {
                    // the first unit of an accumulating segment: y + output now, as the store would add them
                    const bool ya = n == 0 && sg.mode == QP_GEMV_ACC;
                    outv[k] = ya ? ypre + vv : vv;
                    pre = ya ? (pre | (1u << k)) : (pre & ~(1u << k));
                    outk[k] = (si << 28) | (lr0 + rel);
                    if (sg.mode == QP_GEMV_ARGMAX) {
                        const uint64_t key = amax_key(vv, lr0 + rel);
                        best = key > best ? key : best;
                    }
                } else if (slot) {
                    outk[k] = 0xffffffffu;  // a row past the segment: nothing to write
                }
            }
        }
        nout += nper * S;
    }
    tl_ph(TLK, 4);  // all units
    flush(false);
    if (amax) {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(best >> 32), m, 64) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)best, m, 64);
            best = o > best ? o : best;
        }
        if (lane == 0) wbest[wave] = best;
        __syncthreads();
        if (tid == 0) {
            uint64_t bb = wbest[0];
            for (uint32_t i = 1; i < nwv; i++) bb = wbest[i] > bb ? wbest[i] : bb;
            mptr<uint64_t>(amax)[blockIdx.x] = bb;
        }
    }
}

template <int FMT, int R, int XS, int NT = 256, bool NORM = true>
QP_DEV void kq_gemv_seg(const QpGemvArgs& a) {
    auto seg_at = [&](uint32_t i) __attribute__((always_inline)) {
        const QpGemvSeg& q = a.seg[i];
        return KSeg{q.w, q.w2, q.y, q.n, q.row_base, q.rows_total, q.mode, q.wg0, q.fmt};
    };
    const uint64_t t0 = tl_now();
    const uint32_t xrow = a.last_row ? paso_T(a.paso) - 1 : 0;
    kq_gemv<FMT, R, XS, decltype(seg_at), KDense, KNoPro, NT, NORM>(seg_at, a.nseg, a.total_wg,
                                                                  a.x + 4ull * xrow * a.k, a.norm_w, a.eps, a.k,
                                                                  a.amax);
    tl_rec(a.tseq, t0);
}

// Gathered expert GEMV: grid.y = job, job z uses expert sel[z] and input row z / tfijo.
template <int FMT, int R, int XS>
QP_DEV void kq_gemv_exp(const QpGemvExpArgs& a) {
    const uint32_t njobs = a.njobs_fixed ? a.njobs_fixed : paso_T(a.paso) * a.kused;
    const uint32_t job = blockIdx.y;
    if (job >= njobs) return;
    uint32_t ex = cptr<uint32_t>(a.sel)[job];
    if (ex >= a.n_exp) ex = a.n_exp - 1;  // routing only produces valid experts; never read outside the tensor
    const bool pair = a.mode == QP_GEMV_SWIGLU;
    const KSeg one{a.w, a.w2, a.y + 4ull * job * a.n, a.n, ex * a.n, a.n_exp * a.n,
                   pair ? (uint32_t)QP_GEMV_SWIGLU : (uint32_t)QP_GEMV_STORE, 0, (uint32_t)FMT};
    uint32_t nbp = 1;
    while (nbp < (a.k >> 8)) nbp <<= 1;
    const uint32_t rpu = (pair ? 1 : R) * (64 / nbp);
    const uint32_t units = (a.n + rpu - 1) / rpu;
    kq_gemv<FMT, R, XS>([&](uint32_t) __attribute__((always_inline)) { return one; }, 1, units,
                        a.x + 4ull * (job / a.tfijo) * a.k, 0, 0.0f, a.k, 0);
}

// ------------------------------------------------------------------------ fused MoE FFN of one decode token
// Routing of the token as one wavefront computes it (reference moe_topk, kds.js:191-221): softmax over the e <= 256
// router logits, kused rounds of strict maximum over the probabilities (ties to the lower expert index), weights =
// chosen probabilities times scale, divided by their running sum (at least 2^-14) when norm.  Lane i < kused
// returns slot i's expert and weight.
// ld(e) returns logit e.  The probabilities of experts lane + 64 j (p[j]; -3, below every candidate, past E).
template <class Ld>
QP_DEV void moe_probs(uint32_t E, Ld ld, uint32_t lane, float (&p)[4]) {
    float m = -3.0e38f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t e = lane + 64 * j;
        p[j] = e < E ? ld(e) : -3.0e38f;
        m = fmaxf(m, p[j]);
    }
    m = wave_max_v(m, lane);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        p[j] = lane + 64 * j < E ? expf(p[j] - m) : 0.0f;
        s += p[j];
    }
    s = wave_sum_v(s, lane);
#pragma unroll
    for (int j = 0; j < 4; j++) p[j] = lane + 64 * j < E ? p[j] / s : -3.0f;
}

template <class Ld>
QP_DEV void moe_route_(uint32_t E, uint32_t kused, float scale, uint32_t norm, Ld ld, uint32_t lane, uint32_t& sel,
                       float& wt) {
    float p[4];
    moe_probs(E, ld, lane, p);
    float tot = 0.0f;
    sel = 0;
    wt = 0.0f;
    // (value, index) of the best candidate kept by a lane and its butterfly partner: higher value, then lower index
    auto step = [&](auto S, float& bv, uint32_t& bi) __attribute__((always_inline)) {
        const float ov = bfly_f<decltype(S)::value>(bv, lane);
        const uint32_t oi = bfly<decltype(S)::value>(bi, lane);
        const bool take = ov > bv || (ov == bv && oi < bi);
        bv = take ? ov : bv;
        bi = take ? oi : bi;
    };
    for (uint32_t i = 0; i < kused; i++) {
        float bv = -1.0f;
        uint32_t bi = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (p[j] > bv) {
                bv = p[j];
                bi = lane + 64 * j;
            }
        step(std::integral_constant<int, 0>(), bv, bi);
        step(std::integral_constant<int, 1>(), bv, bi);
        step(std::integral_constant<int, 2>(), bv, bi);
        step(std::integral_constant<int, 3>(), bv, bi);
        step(std::integral_constant<int, 4>(), bv, bi);
        step(std::integral_constant<int, 5>(), bv, bi);
        if (bi == 0xffffffffu) bi = 0;  // nothing left above -1 (kused > e): expert 0, weight -1, as the reference
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j == bi) p[j] = -2.0f;
        if (lane == i) {
            sel = bi;
            wt = bv;
        }
        tot = tot + bv;
    }
    float f = scale;
    if (norm) f = f / fmaxf(tot, 6.103515625e-5f);
    wt = wt * f;
}

// The same routing by a whole workgroup (256 threads, E <= 256), with the k rounds replaced by ranks: wavefront 0
// computes the probabilities as above; thread t < E counts the experts that come before its own (a higher
// probability, or an equal one at a lower index; a NaN probability never counts and is never chosen), the kused
// first go to their slots in rank order (unfilled slots keep expert 0 with -1, as the rounds leave them), and the
// weights follow from the running sum in rank order: the same experts and the same weights as moe_route_, with no
// chain of dependent rounds.  lds: 896 floats.
template <class Ld>
QP_DEV void moe_route_wg(uint32_t E, uint32_t kused, float scale, uint32_t norm, Ld ld, float* lds, uint64_t sel_out,
                         uint64_t wts_out) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // one 64-bit key per expert: the probability's bits above, 0xffffffff - index below.  The probabilities are
    // non-negative (never -0), so their bits order as the values do and equal bits are equal values: key_e > key_t
    // exactly when p_e > p_t, or p_e == p_t and e < t.  A NaN probability keys to 0, which outranks nothing; the
    // entries past E are 0 too.
    uint64_t* lk = reinterpret_cast<uint64_t*>(lds);                 // [256] keys
    uint32_t* part = reinterpret_cast<uint32_t*>(lds + 512);         // [256] partial ranks
    uint32_t* slot_e = reinterpret_cast<uint32_t*>(lds + 768);       // [64]
    float* slot_p = lds + 832;                                       // [64]
    tl_ph(9, 0);
    if (wave == 0) {
        float p[4];
        moe_probs(E, ld, lane, p);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t e = lane + 64 * j;
            lk[e] = e < E && p[j] == p[j]
                        ? ((uint64_t)__float_as_uint(p[j]) << 32) | (uint64_t)(0xffffffffu - e)
                        : 0ull;
        }
    }
    tl_ph(9, 1);
    if (tid < kused) {
        slot_e[tid] = 0u;
        slot_p[tid] = -1.0f;
    }
    __syncthreads();
    tl_ph(9, 2);
    // up to 128 experts two threads count each expert's rank, over alternate pairs of keys
    const uint32_t two = E <= 128, t = two ? tid & 127 : tid, h = two ? tid >> 7 : 0u, step = two ? 2u : 1u;
    uint32_t r = 0;
    if (t < E) {
        const uint64_t kt = lk[t];
        const ulonglong2* lk2 = reinterpret_cast<const ulonglong2*>(lk);
        const uint32_t n2 = (E + 1) >> 1;
#pragma unroll 8
        for (uint32_t i = h; i < n2; i += step) {
            const ulonglong2 q = lk2[i];
            r += q.x > kt ? 1u : 0u;
            r += q.y > kt ? 1u : 0u;
        }
    }
    part[tid] = r;
    __syncthreads();
    if (tid < E && (!two || tid < 128)) {
        const uint64_t kt = lk[tid];
        const uint32_t rank = kt == 0ull ? E : part[tid] + (two ? part[tid + 128] : 0u);  // NaN: never chosen
        if (rank < kused) {
            slot_e[rank] = tid;
            slot_p[rank] = __uint_as_float((uint32_t)(kt >> 32));
        }
    }
    tl_ph(9, 3);
    __syncthreads();
    tl_ph(9, 4);
    if (wave == 0) {
        float tot = 0.0f;
        for (uint32_t i = 0; i < kused; i++) tot = tot + slot_p[i];
        float f = scale;
        if (norm) f = f / fmaxf(tot, 6.103515625e-5f);
        if (lane < kused) {
            gstore<uint32_t>(sel_out + 4ull * lane, slot_e[lane]);
            gstore<float>(wts_out + 4ull * lane, slot_p[lane] * f);
        }
        tl_ph(9, 5);
    }
}

QP_DEV void moe_route(const QpMoeArgs& a, uint32_t lane, uint32_t& sel, float& wt) {
    moe_route_(a.e, a.kused, a.scale, a.norm, [&](uint32_t e) { return gload<float>(a.logits + 4ull * e); }, lane, sel,
               wt);
}

template <int FMT, int XS>
QP_DEV void moe_gate_up_body_(const QpMoeArgs& a);
template <int FMT, int XS>
QP_DEV void moe_gate_up_body(const QpMoeArgs& a) {
    const uint64_t t0 = tl_now();
    moe_gate_up_body_<FMT, XS>(a);
    tl_rec(a.tseq, t0);
}
template <int FMT, int XS>
QP_DEV void moe_gate_up_body_(const QpMoeArgs& a) {
    const uint32_t lane = threadIdx.x & 63, job = blockIdx.y;
    uint32_t sel = 0, ex = 0;
    float wt = 0.0f;
    // with presel the chosen experts load before the input (loads return in order, so the weight loads wait for
    // them alone); else the routing runs while the input loads are in flight.  The job's expert decides its
    // weight rows.
    if (a.presel) sel = lane < a.kused ? gload<uint32_t>(a.sel + 4ull * lane) : 0u;
    auto route = [&]() __attribute__((always_inline)) {
        if (!a.presel) moe_route(a, lane, sel, wt);
        ex = (uint32_t)__builtin_amdgcn_readlane((int)sel, (int)job);
        if (ex >= a.e) ex = a.e - 1;
    };
    uint32_t nbp = 1;
    while (nbp < (a.k >> 8)) nbp <<= 1;
    const uint32_t units = (a.n + 64 / nbp - 1) / (64 / nbp);
    kq_gemv<FMT, 2, XS>(
        [&](uint32_t) __attribute__((always_inline)) {
            return KSeg{a.w, a.w2, a.y + 4ull * job * a.n, a.n, ex * a.n, a.e * a.n, (uint32_t)QP_GEMV_SWIGLU, 0,
                        (uint32_t)FMT};
        },
        1, units, a.x, a.norm_w, a.eps, a.k, 0, KDense(), route);
    if (!a.presel && blockIdx.x == 0 && job == 0 && threadIdx.x < a.kused) {
        gstore<uint32_t>(a.sel + 4ull * lane, sel);
        gstore<float>(a.wts + 4ull * lane, wt);
    }
}

// ------------------------------------------------------------------------ router logits + routing (moe_router)
// Column 0 of the grid works: its nw workgroups share one XCD (workgroups go to the 8 XCDs round robin by linear id
// x + 8y), so the arrival counter and the logits live in one L2.  Wavefront i of the column takes rows i, i + 4 nw,
// ...: its first row's weights load before the input is staged.  The last workgroup to arrive reads the logits back
// past its L1 and routes.
QP_DEV void moe_router_body_(const QpRouterArgs& a);
QP_DEV void moe_router_body(const QpRouterArgs& a) {
    const uint64_t t0 = tl_now();
    moe_router_body_(a);
    tl_rec(a.tseq, t0);
}
QP_DEV void moe_router_body_(const QpRouterArgs& a) {
    if (blockIdx.x != 0) return;
    tl_ph(8, 0);
    extern __shared__ float4 xs4[];  // k floats: x * norm_w
    __shared__ float red[4];
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nf4 = a.k >> 2, W = 4 * a.nw, r0 = blockIdx.y * 4 + wave;
    constexpr int NP = 8;  // float4 of a row per lane held in flight (k <= 2048; longer rows loop)
    const __amdgpu_buffer_rsrc_t rw = kq_rsrc(a.w, 4ull * a.e * a.k);
    float4 wv[NP];
    auto issue = [&](uint32_t r, uint32_t q0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const uint32_t q = q0 + lane + 64 * i;
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                rw, r < a.e && q < nf4 ? (r * nf4 + q) * 16 : 0x80000000u, 0, 0);
            wv[i] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                __uint_as_float(v[3]));
        }
    };
    issue(r0, 0);
    float ss = 0.0f;
    for (uint32_t q = tid; q < nf4; q += 256) {
        float4 v = gload<float4>(a.x + 16ull * q);
        if (a.norm_w) {
            ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
            const float4 nw = gload<float4>(a.norm_w + 16ull * q);
            v.x *= nw.x;
            v.y *= nw.y;
            v.z *= nw.z;
            v.w *= nw.w;
        }
        xs4[q] = v;
    }
    ss = wave_sum_v(ss, lane);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float inv = a.norm_w ? 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)a.k + a.eps) : 1.0f;
    tl_ph(8, 1);  // input staged
    for (uint32_t r = r0; r < a.e; r += W) {
        float s = 0.0f;
        for (uint32_t q0 = 0; q0 < nf4; q0 += 64 * NP) {
            if (r != r0 || q0 != 0) issue(r, q0);
#pragma unroll
            for (int i = 0; i < NP; i++) {
                const uint32_t q = q0 + lane + 64 * i;
                if (q < nf4) {
                    const float4 xv = xs4[q];
                    s += (wv[i].x * xv.x + wv[i].y * xv.y) + (wv[i].z * xv.z + wv[i].w * xv.w);
                }
            }
        }
        s = wave_sum_v(s, lane) * inv;  // lane exchanges: no LDS round trips on the way to the arrival
        if (lane == 0) gstore<float>(a.logits + 4ull * r, s);
    }
    tl_ph(8, 2);  // rows done
    vm_drain();
    __syncthreads();
    if (tid == 0) last = xcd_arrive(a.cnt, a.nw, a.cnt + 4);
    __syncthreads();
    tl_ph(8, 3);  // arrival counted
    if (!last) return;
    const __amdgpu_buffer_rsrc_t rl = kq_rsrc(a.logits, 4ull * a.e);
    moe_route_wg(a.e, a.kused, a.scale, a.norm, [&](uint32_t e) { return __uint_as_float(ld_sc0(rl, 4 * e)); },
                 reinterpret_cast<float*>(xs4), a.sel, a.wts);
    tl_ph(8, 4);  // routed (the last workgroup)
}
KERNEL __launch_bounds__(256) void qp_moe_router(QpRouterArgs a) { moe_router_body(a); }

// moe_down's gathered layout: x block b (of kused * nbwv) is block b % nbwv of row r of expert sel[b / nbwv], and
// the input sub-blocks of slot j are scaled by wts[j].  Lane j < kused of every wavefront holds sel[j], wts[j].
struct KMoeDown {
    static constexpr bool SCALED = true;
    uint32_t nbwv, rows, nin, ne, selv;
    float wv;
    QP_DEV uint32_t nbw(uint32_t) const { return nbwv; }
    QP_DEV void loc(uint32_t row, uint32_t b, uint32_t& wr, uint32_t& wb) const {
        const uint32_t slot = b / nbwv;
        uint32_t ex = (uint32_t)__shfl((int)selv, (int)(slot & 63), 64);
        ex = ex < ne ? ex : ne - 1;
        wr = ex * rows + row;
        wb = b - slot * nbwv;
    }
    QP_DEV float xscale(uint32_t q) const { return __shfl(wv, (int)((q * 32 / nin) & 63), 64); }
};

template <int FMT, int XS>
QP_DEV void moe_down_body_(const QpMoeArgs& a);
template <int FMT, int XS>
QP_DEV void moe_down_body(const QpMoeArgs& a) {
    const uint64_t t0 = tl_now();
    moe_down_body_<FMT, XS>(a);
    tl_rec(a.tseq, t0);
}
template <int FMT, int XS>
QP_DEV void moe_down_body_(const QpMoeArgs& a) {
    const uint32_t lane = threadIdx.x & 63;
    KMoeDown lay;
    lay.nbwv = a.k >> 8;
    lay.rows = a.n;
    lay.nin = a.k;
    lay.ne = a.e;
    lay.selv = lane < a.kused ? gload<uint32_t>(a.sel + 4ull * lane) : 0u;
    lay.wv = lane < a.kused ? gload<float>(a.wts + 4ull * lane) : 0.0f;
    const uint32_t K = a.kused * a.k;
    const KSeg one{a.w, a.w, a.y, a.n, 0, a.e * a.n, (uint32_t)QP_GEMV_ACC, 0, (uint32_t)FMT};
    uint32_t nbp = 1;
    while (nbp < (K >> 8)) nbp <<= 1;
    const uint32_t units = (a.n + 64 / nbp - 1) / (64 / nbp);
    kq_gemv<FMT, 1, XS>([&](uint32_t) __attribute__((always_inline)) { return one; }, 1, units, a.x, 0, 0.0f, K, 0,
                        lay);
}

#define MOE_KERNELS(NAME, FMT)                                                                                    \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_moe_gate_up_##NAME##_x1(    \
        QpMoeArgs a) { moe_gate_up_body<FMT, 1>(a); }                                                             \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_moe_gate_up_##NAME##_x2(    \
        QpMoeArgs a) { moe_gate_up_body<FMT, 2>(a); }                                                             \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void qp_moe_down_##NAME##_x1(       \
        QpMoeArgs a) { moe_down_body<FMT, 1>(a); }                                                                \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_moe_down_##NAME##_x2(       \
        QpMoeArgs a) { moe_down_body<FMT, 2>(a); }
MOE_KERNELS(q4k, QP_Q4_K)
MOE_KERNELS(q6k, QP_Q6_K)

#define KQ_KERNELS(NAME, FMT)                                                                                     \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void qp_gemv_##NAME##_r1(           \
        QpGemvArgs a) { kq_gemv_seg<FMT, 1, 1>(a); }                                                              \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_##NAME##_r2(           \
        QpGemvArgs a) { kq_gemv_seg<FMT, 2, 1>(a); }                                                              \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_##NAME##_r1x2(         \
        QpGemvArgs a) { kq_gemv_seg<FMT, 1, 2>(a); }                                                              \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_##NAME##_r2x2(         \
        QpGemvArgs a) { kq_gemv_seg<FMT, 2, 2>(a); }                                                              \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void qp_gemv_exp_##NAME##_r1(       \
        QpGemvExpArgs a) { kq_gemv_exp<FMT, 1, 1>(a); }                                                           \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_exp_##NAME##_r2(       \
        QpGemvExpArgs a) { kq_gemv_exp<FMT, 2, 1>(a); }                                                           \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_exp_##NAME##_r1x2(     \
        QpGemvExpArgs a) { kq_gemv_exp<FMT, 1, 2>(a); }                                                           \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_exp_##NAME##_r2x2(     \
        QpGemvExpArgs a) { kq_gemv_exp<FMT, 2, 2>(a); }
KQ_KERNELS(q4k, QP_Q4_K)
KQ_KERNELS(q5k, QP_Q5_K)
KQ_KERNELS(q3k, QP_Q3_K)
KQ_KERNELS(q2k, QP_Q2_K)
KQ_KERNELS(q6k, QP_Q6_K)
// rows of more than 8192 inputs without the fused norm: 512 threads share one input staging, one sub-block each
KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void qp_gemv_q4k_r1k2(QpGemvArgs a) {
    kq_gemv_seg<QP_Q4_K, 1, 1, 512, false>(a);
}
KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void qp_gemv_q3k_r1k2(QpGemvArgs a) {
    kq_gemv_seg<QP_Q3_K, 1, 1, 512, false>(a);
}
KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void qp_gemv_q2k_r1k2(QpGemvArgs a) {
    kq_gemv_seg<QP_Q2_K, 1, 1, 512, false>(a);
}
KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void qp_gemv_q5k_r1k2(QpGemvArgs a) {
    kq_gemv_seg<QP_Q5_K, 1, 1, 512, false>(a);
}
KERNEL __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void qp_gemv_q6k_r1k2(QpGemvArgs a) {
    kq_gemv_seg<QP_Q6_K, 1, 1, 512, false>(a);
}
KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void qp_gemv_mix_r1(QpGemvArgs a) {
    kq_gemv_seg<QP_KQ_MIX, 1, 1>(a);
}
KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_mix_r2(QpGemvArgs a) {
    kq_gemv_seg<QP_KQ_MIX, 2, 1>(a);
}
KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_mix_r1x2(QpGemvArgs a) {
    kq_gemv_seg<QP_KQ_MIX, 1, 2>(a);
}
KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void qp_gemv_mix_r2x2(QpGemvArgs a) {
    kq_gemv_seg<QP_KQ_MIX, 2, 2>(a);
}

// ====================================================================================== multi-token GEMM
// Prefill y[t][r] (+)= W[r].x[t] for T tokens (reference matmul_*_4 and the tiled matmul_*_t,
// kquants.js:309-386): a 64-row x 64-token tile per workgroup, K in steps of 32; the weight tile is
// dequantized to f32 in LDS with the reference's element formula, then each thread accumulates a 4x4
// register tile.
KERNEL __launch_bounds__(256) void qp_gemm_mt(QpGemmArgs a) {
    __shared__ float wt[32][64 + 4];
    __shared__ float xt[32][64 + 4];
    const uint32_t T = a.tfix ? a.tfix : paso_T(a.paso);
    const uint32_t N = a.n, K = a.k;
    const uint32_t r0 = blockIdx.x * 64, t0 = blockIdx.y * 64;
    if (t0 >= T) return;
    const uint32_t tid = threadIdx.x;
    const uint32_t ty = tid >> 4, tx = tid & 15;  // rows ty*4.., tokens tx*4..
    const uint8_t* W = cptr<uint8_t>(a.w);
    const float* X = cptr<float>(a.x);
    const uint64_t NB = total_blocks(a.fmt, N, K);
    float c[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) c[i][j] = 0.0f;
    // loader roles: weight row lr (0..63), 8 consecutive k at lk*8; x token lt, same k split
    const uint32_t lr = tid >> 2, lk = (tid & 3) * 8;
    const uint32_t wrow = min(r0 + lr, N - 1);
    const uint32_t xtok = min(t0 + lr, T - 1);
    for (uint32_t k0 = 0; k0 < K; k0 += 32) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t k = k0 + lk + i;
            wt[lk + i][lr] = k < K ? deq_elem(a.fmt, W, NB, wrow, K, k) : 0.0f;
            xt[lk + i][lr] = k < K ? X[(uint64_t)xtok * K + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < 32; kk++) {
            const float4 wv = *reinterpret_cast<const float4*>(&wt[kk][ty * 4]);
            const float4 xv = *reinterpret_cast<const float4*>(&xt[kk][tx * 4]);
            const float w4[4] = {wv.x, wv.y, wv.z, wv.w}, x4[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) c[i][j] += w4[i] * x4[j];
        }
        __syncthreads();
    }
    float* Y = mptr<float>(a.y);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t r = r0 + ty * 4 + i;
        if (r >= N) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t t = t0 + tx * 4 + j;
            if (t >= T) continue;
            float* o = Y + (uint64_t)t * N + r;
            *o = a.acc ? *o + c[i][j] : c[i][j];
        }
    }
}

// ====================================================================================== prefill GEMM on MFMA
// Y[t][n] (+)= sum_k X[t][k] * W[n][k] for T >= 64 tokens (the reference's tiled matmul_<fmt>_t and
// matmul_<fmt>_4, kquants.js:309-386 and gpu.js:203-266, when a prefill chunk is large enough for matrix cores).
//
// A workgroup computes a 128-token x 128-row tile with v_mfma_f32_32x32x16_bf16: 4 wavefronts in 2 x 2, each
// 64 x 64 (2 x 2 MFMA blocks).  Per K step of 64 every thread dequantizes 32 weights of one row with the
// reference's element formula (exact f32) and converts 32 inputs of one token; each value v goes to LDS as
// bf16 hi = bf16(v) and lo = bf16(v - hi), and the tile accumulates hi*hi + hi*lo + lo*hi in f32, so the
// products keep about 16 significant bits instead of bf16's 8 (the dropped lo*lo term is 2^-18 relative).  The
// global loads of step k+1 are issued before the matrix instructions of step k.  Tiles are numbered so that
// each XCD (workgroup id mod 8) takes a contiguous range of weight tiles with all their token tiles: a weight
// tile is dequantized from one L2.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace mm {
constexpr int TM = 128, TN = 128, TK = 64, LDK = 72;  // LDS rows padded to 72 bf16 (144 B)
}
#define QP_NOJOB 0xffffffffu  // a grouped tile's row without a job

// Byte offset of input k of token row t in a bf16 plane written by qp_split_bf16 (rows token rows per plane): the
// 8 inputs 8q .. 8q + 7 of 32-input chunk c are 16 bytes at ((4c + q) * rows + t) * 16.
QP_DEV uint64_t xs_off(uint32_t t, uint32_t k, uint32_t rows) {
    return ((uint64_t)((k >> 5) * 4 + ((k >> 3) & 3)) * rows + t) * 16 + (k & 7) * 2;
}

// Eight values -> their bf16 high parts and the bf16 of the remainders, each written to LDS as one 16-byte store.
QP_DEV void split_store8(const float* v, __bf16* hi, __bf16* lo) {
    bf16x8 h, l;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const __bf16 t = (__bf16)v[i];
        h[i] = t;
        l[i] = (__bf16)(v[i] - (float)t);
    }
    *reinterpret_cast<bf16x8*>(hi) = h;
    *reinterpret_cast<bf16x8*>(lo) = l;
}

// Source registers of one thread's 32 weights for one K step (row `row`, k = k0 + koff .. ).
struct MmW {
    uint4 a, b, c, d, e;
    uint32_t f;
};

template <int FMT>
QP_DEV void mm_wload(MmW& r, const QpGemmArgs& g, uint32_t row, bool on, uint32_t k0, uint32_t part) {
    const uint32_t K = g.k;
    if (!on) row = 0;
    if constexpr (FMT == QP_Q4_K) {
        // chunk 1 + 2p + part: bytes 16*part.. of sub-block pair p (16 elements of sub-blocks 2p and 2p+1)
        const uint32_t nb = K >> 8, b = k0 >> 8, p = (k0 & 255) >> 6;
        const uint64_t base = g.w + (uint64_t)row * nb * 144 + b * 16;
        r.a = gload<uint4>(base + (uint64_t)(1 + 2 * p + part) * nb * 16);
        r.b = gload<uint4>(base);  // header chunk
    } else if constexpr (FMT == QP_Q6_K) {
        // qd = 2*kk + part with kk = (k0 & 127) >> 6, h = (k0 & 255) >> 7: 32 elements l = 0..31
        const uint32_t nb = K >> 8, b = k0 >> 8, h = (k0 & 255) >> 7, qd = 2 * ((k0 & 127) >> 6) + part;
        const uint64_t base = g.w + (uint64_t)row * nb * 208 + b * 16;
        const uint32_t cl = h * 4 + (qd & 1) * 2, ch = 8 + h * 2;
        r.a = gload<uint4>(base + (uint64_t)cl * nb * 16);
        r.b = gload<uint4>(base + (uint64_t)(cl + 1) * nb * 16);
        r.c = gload<uint4>(base + (uint64_t)ch * nb * 16);
        r.d = gload<uint4>(base + (uint64_t)(ch + 1) * nb * 16);
        r.e = gload<uint4>(base + (uint64_t)12 * nb * 16);
        const uint64_t NB = (uint64_t)(g.wrows ? g.wrows : g.n) * nb;
        r.f = gload<uint16_t>(g.w + NB * 208 + ((uint64_t)row * nb + b) * 2);
    } else if constexpr (FMT == QP_Q5_K || FMT == QP_Q3_K || FMT == QP_Q2_K) {
        // sub-block J of 32 (elements l = 0..31 in k order): its 32 quant bytes (a, b), the high-bit bytes (c, d:
        // Q5_K qh, Q3_K hmask), the scales chunk (e) and, for Q2_K, the (d, dmin) word (f)
        constexpr uint32_t RB = KQ<FMT>::RB;
        const uint32_t nb = K >> 8, b = k0 >> 8, J = ((k0 & 255) >> 5) + part, n = J >> 2;
        const uint64_t base = g.w + (uint64_t)row * nb * RB + b * 16;
        const uint32_t cq = FMT == QP_Q5_K ? 3 + 2 * (J >> 1) : FMT == QP_Q3_K ? 2 + 2 * n : 1 + 2 * n;
        r.a = gload<uint4>(base + (uint64_t)cq * nb * 16);
        r.b = gload<uint4>(base + (uint64_t)(cq + 1) * nb * 16);
        if constexpr (FMT != QP_Q2_K) {
            const uint32_t ch = FMT == QP_Q5_K ? 1 : 0;
            r.c = gload<uint4>(base + (uint64_t)ch * nb * 16);
            r.d = gload<uint4>(base + (uint64_t)(ch + 1) * nb * 16);
        }
        r.e = gload<uint4>(base + (uint64_t)(FMT == QP_Q3_K ? 6 : 0) * nb * 16);
        if constexpr (FMT == QP_Q2_K) {
            const uint64_t NB = (uint64_t)(g.wrows ? g.wrows : g.n) * nb;
            r.f = gload<uint32_t>(g.w + NB * 80 + ((uint64_t)row * nb + b) * 4);
        }
    } else if constexpr (FMT == QP_Q8_0) {
        const uint64_t NB = (uint64_t)(g.wrows ? g.wrows : g.n) * (K >> 5);
        const uint64_t blk = (uint64_t)row * (K >> 5) + (k0 >> 5) + part;
        const bool in = k0 + 32 * part < K;
        const uint64_t bb = in ? blk : (uint64_t)row * (K >> 5);
        r.a = gload<uint4>(g.w + bb * 32);
        r.b = gload<uint4>(g.w + bb * 32 + 16);
        r.f = gload<uint16_t>(g.w + NB * 32 + bb * 2);
    } else if constexpr (FMT == QP_IQ4_NL) {
        const uint64_t NB = (uint64_t)(g.wrows ? g.wrows : g.n) * (K >> 5);
        const uint64_t blk = (uint64_t)row * (K >> 5) + (k0 >> 5) + part;
        const bool in = k0 + 32 * part < K;
        const uint64_t bb = in ? blk : (uint64_t)row * (K >> 5);
        r.a = gload<uint4>(g.w + bb * 16);
        r.f = gload<uint16_t>(g.w + NB * 16 + bb * 2);
    }
}

// 32 weights in k order from the loaded registers (F32 reads its row directly).
template <int FMT>
QP_DEV void mm_wdeq(const MmW& r, const QpGemmArgs& g, uint32_t row, bool on, uint32_t k0, uint32_t part,
                    float (&w)[32]) {
#pragma clang fp contract(off)
    if constexpr (FMT == QP_Q4_K) {
        // element order: w[0..15] = sub-block 2p, l = 16*part..; w[16..31] = sub-block 2p+1, same l
        const uint32_t p = (k0 & 255) >> 6;
        uint32_t sc0, mn0, sc1, mn1;
        q4k_sm(r.b.y, r.b.z, r.b.w, 2 * p, sc0, mn0);
        q4k_sm(r.b.y, r.b.z, r.b.w, 2 * p + 1, sc1, mn1);
        const float d = h2f(r.b.x & 0xffffu), dm = h2f(r.b.x >> 16);
        const float fd0 = d * (float)sc0, fm0 = dm * (float)mn0, fd1 = d * (float)sc1, fm1 = dm * (float)mn1;
        const uint32_t q4[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t byte = (q4[i >> 2] >> ((i & 3) * 8)) & 0xffu;
            const float a0 = fd0 * (float)(byte & 15u), a1 = fd1 * (float)(byte >> 4);
            w[i] = a0 - fm0;
            w[16 + i] = a1 - fm1;
        }
    } else if constexpr (FMT == QP_Q6_K) {
        const uint32_t h = (k0 & 255) >> 7, qd = 2 * ((k0 & 127) >> 6) + part;
        const uint32_t lo[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t hi[8] = {r.c.x, r.c.y, r.c.z, r.c.w, r.d.x, r.d.y, r.d.z, r.d.w};
        const uint32_t scw[4] = {r.e.x, r.e.y, r.e.z, r.e.w};
        const float d = h2f(r.f);
        const uint32_t s0 = h * 8 + qd * 2;  // scale of l < 16; s0 + 1 for l >= 16
        const float fd0 = d * (float)(int8_t)((scw[s0 >> 2] >> ((s0 & 3) * 8)) & 0xffu);
        const float fd1 = d * (float)(int8_t)((scw[(s0 + 1) >> 2] >> (((s0 + 1) & 3) * 8)) & 0xffu);
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t lb = (lo[l >> 2] >> ((l & 3) * 8 + (qd >> 1) * 4)) & 15u;
            const uint32_t hb = (hi[l >> 2] >> ((l & 3) * 8 + qd * 2)) & 3u;
            const float q = (float)(lb | (hb << 4)) - 32.0f;
            w[l] = (l < 16 ? fd0 : fd1) * q;
        }
    } else if constexpr (FMT == QP_Q5_K || FMT == QP_Q3_K || FMT == QP_Q2_K) {
        // the element formulas of deq_q5k_dev / deq_q3k_dev / deq_q2k_dev, same roundings
        const uint32_t J = ((k0 & 255) >> 5) + part, n = J >> 2, jj = J & 3;
        const uint32_t qv[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        if constexpr (FMT == QP_Q5_K) {
            const uint32_t hv[8] = {r.c.x, r.c.y, r.c.z, r.c.w, r.d.x, r.d.y, r.d.z, r.d.w};
            uint32_t sc, mn;
            q4k_sm(r.e.y, r.e.z, r.e.w, J, sc, mn);
            const float fd = h2f(r.e.x & 0xffffu) * (float)sc, fm = h2f(r.e.x >> 16) * (float)mn;
#pragma unroll
            for (int l = 0; l < 32; l++) {
                const uint32_t lo = (qv[l >> 2] >> ((l & 3) * 8 + (J & 1) * 4)) & 15u;
                const uint32_t hi = (hv[l >> 2] >> ((l & 3) * 8 + J)) & 1u;
                const float a = fd * (float)(lo + 16u * hi);
                w[l] = a - fm;
            }
        } else if constexpr (FMT == QP_Q3_K) {
            const uint32_t hv[8] = {r.c.x, r.c.y, r.c.z, r.c.w, r.d.x, r.d.y, r.d.z, r.d.w};
            const float d = h2f(r.e.w & 0xffffu);
            const uint32_t s0 = 8 * n + 2 * jj;  // scale group of l < 16; s0 + 1 for l >= 16
            const float fd0 = d * ((float)q3k_scale6(r.e.x, r.e.y, r.e.z, s0) - 32.0f);
            const float fd1 = d * ((float)q3k_scale6(r.e.x, r.e.y, r.e.z, s0 + 1) - 32.0f);
#pragma unroll
            for (int l = 0; l < 32; l++) {
                const uint32_t q2 = (qv[l >> 2] >> ((l & 3) * 8 + 2 * jj)) & 3u;
                const uint32_t hm = (hv[l >> 2] >> ((l & 3) * 8 + 4 * n + jj)) & 1u;
                w[l] = (l < 16 ? fd0 : fd1) * ((float)q2 - 4.0f * (float)(1u - hm));
            }
        } else {
            const float d = h2f(r.f & 0xffffu), dmin = h2f(r.f >> 16);
            const uint32_t sv[4] = {r.e.x, r.e.y, r.e.z, r.e.w};
            const uint32_t j0 = 8 * n + 2 * jj;  // scale byte of l < 16; j0 + 1 for l >= 16
            const uint32_t sc0 = (sv[j0 >> 2] >> ((j0 & 3) * 8)) & 0xffu;
            const uint32_t sc1 = (sv[(j0 + 1) >> 2] >> (((j0 + 1) & 3) * 8)) & 0xffu;
            const float fd0 = d * (float)(sc0 & 15u), fm0 = dmin * (float)(sc0 >> 4);
            const float fd1 = d * (float)(sc1 & 15u), fm1 = dmin * (float)(sc1 >> 4);
#pragma unroll
            for (int l = 0; l < 32; l++) {
                const uint32_t q = (qv[l >> 2] >> ((l & 3) * 8 + 2 * jj)) & 3u;
                const float a = (l < 16 ? fd0 : fd1) * (float)q;
                w[l] = a - (l < 16 ? fm0 : fm1);
            }
        }
    } else if constexpr (FMT == QP_Q8_0) {
        const float d = h2f(r.f);
        const uint32_t q8[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        const bool in = k0 + 32 * part < g.k;
#pragma unroll
        for (int i = 0; i < 32; i++)
            w[i] = in ? (float)(int8_t)((q8[i >> 2] >> ((i & 3) * 8)) & 0xffu) * d : 0.0f;
    } else if constexpr (FMT == QP_IQ4_NL) {
        // w[4i..4i+3]: the low nibbles of word i; w[16+4i..]: its high nibbles (d * table[nibble])
        const float d = h2f(r.f);
        const uint32_t qw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const bool in = k0 + 32 * part < g.k;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = iq4nl_lut4(qw[i] & 0x0f0f0f0fu), hi = iq4nl_lut4((qw[i] >> 4) & 0x0f0f0f0fu);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                w[4 * i + b] = in ? d * (float)(int8_t)((lo >> (8 * b)) & 0xffu) : 0.0f;
                w[16 + 4 * i + b] = in ? d * (float)(int8_t)((hi >> (8 * b)) & 0xffu) : 0.0f;
            }
        }
    } else {
        const uint32_t kb = k0 + 32 * part;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t k = kb + i;
            w[i] = (on && k < g.k) ? cptr<float>(g.w)[(uint64_t)row * g.k + k] : 0.0f;
        }
    }
}

template <int FMT>
QP_DEV void gemm_mfma_body(const QpGemmArgs& g) {
    using namespace mm;
    __shared__ __bf16 xh[TM * LDK], xl[TM * LDK], wh[TN * LDK], wl[TN * LDK];
    const uint32_t T = g.tfix ? g.tfix : paso_T(g.paso);
    const uint32_t N = g.n, K = g.k;
    // XCD-aware tile order: workgroup i runs on XCD i % 8, as the j-th workgroup of that XCD; XCD x holds
    // base + (x < rem) of the workgroups, so it takes the contiguous logical tiles starting at x*base + min(x, rem).
    // Logical order: weight tile, then K split, then token tile (the token tiles of one weight tile and split are
    // neighbours: they share its dequantized rows through one L2).
    const uint32_t mt = (uint32_t)gridDim.y, ntl = (uint32_t)gridDim.x, nz = (uint32_t)gridDim.z;
    const uint32_t total = mt * ntl * nz, id = (blockIdx.z * mt + blockIdx.y) * ntl + blockIdx.x;
    const uint32_t base = total >> 3, rem = total & 7, xcd = id & 7, j = id >> 3;
    const uint32_t L = xcd * base + (xcd < rem ? xcd : rem) + j;
    const uint32_t m_tile = L % mt, rest = L / mt, zs = rest % nz, n_tile = rest / nz;
    uint32_t t0 = m_tile * TM;
    const uint32_t n0 = n_tile * TN;
    // grouped by expert: this slot's expert and 128 jobs (staged in LDS; an entry past the list or whose x / y row
    // does not exist is QP_NOJOB and loads row 0, stores nothing)
    const bool grp = g.lst != 0;
    __shared__ uint32_t jobs[TM];
    uint32_t ex = 0;
    if (grp) {
        ex = m_tile / g.tpe;
        t0 = (m_tile % g.tpe) * TM;
        if (ex >= g.n_exp) return;
        const uint32_t c0 = min(gload<uint32_t>(g.off + 4ull * ex), g.nlst);
        const uint32_t c1 = min(gload<uint32_t>(g.off + 4ull * (ex + 1)), g.nlst);
        const uint32_t cn = c1 > c0 ? c1 - c0 : 0;
        if (t0 >= cn) return;
        if (threadIdx.x < TM) {
            uint32_t jb = QP_NOJOB;
            if (t0 + threadIdx.x < cn) {
                const uint32_t j = gload<uint32_t>(g.lst + 4ull * (c0 + t0 + threadIdx.x));
                if (j / g.tfijo < g.xrows && j < g.yrows) jb = j;
            }
            jobs[threadIdx.x] = jb;
        }
        __syncthreads();
    } else if (t0 >= T) {
        return;
    }
    const uint32_t kbeg = g.kchunk ? zs * g.kchunk : 0;
    const uint32_t kend = g.kchunk ? min(K, kbeg + g.kchunk) : K;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    // loader roles: token / row = tid >> 1, 32-element part = tid & 1
    const uint32_t lr = tid >> 1, part = tid & 1;
    const uint32_t wr = n0 + lr, wrow = grp ? ex * N + wr : wr;
    const bool xon = grp ? jobs[lr] != QP_NOJOB : t0 + lr < T, won = wr < N;
    const uint32_t xt = grp ? (xon ? jobs[lr] / g.tfijo : 0) : t0 + lr;
    const uint64_t xrow = g.x + 4ull * (uint64_t)(xon ? xt : 0) * K;

    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;

    // x as f32 (split here) or, with xs, as its bf16 high / low planes (copied to LDS as they are)
    float4 xr[8];
    uint4 xp[8];
    const bool pre = g.xs != 0;
    const uint64_t xplane = 2ull * g.rows * (((K + 31) >> 5) << 5);
    const uint32_t xst = xon ? xt : 0;
    MmW wrg;
    auto load = [&](uint32_t k0) __attribute__((always_inline)) {
        const uint32_t kb = k0 + 32 * part;
        if (pre) {
            // K is a multiple of 16 (f32) or 32 (Q8_0), so a group of 8 is wholly inside or past the row; a group
            // past the last 32-input chunk reads as zeros (the row's end is not a 64-multiple when K % 64 != 0)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const bool in = kb + 8 * i < K;
                // grouped by expert: row-major planes (a tile gathers rows; each lane reads 64 bytes of one)
                const uint64_t o = g.xs + (grp ? 2ull * ((uint64_t)xst * (((K + 31) >> 5) << 5) + kb + 8 * i)
                                               : xs_off(xst, kb + 8 * i, g.rows));
                xp[i] = in ? gload<uint4>(o) : uint4{0, 0, 0, 0};
                xp[4 + i] = in ? gload<uint4>(o + xplane) : uint4{0, 0, 0, 0};
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t k = kb + 4 * i;
                xr[i] = (k < K) ? gload<float4>(xrow + 4ull * k) : float4{0.f, 0.f, 0.f, 0.f};
            }
        }
        mm_wload<FMT>(wrg, g, wrow, won, k0, part);
    };
    const uint32_t nsteps = (kend - kbeg + TK - 1) / TK;
    load(kbeg);
    for (uint32_t s = 0; s < nsteps; s++) {
        const uint32_t k0 = kbeg + s * TK;
        // registers -> LDS (bf16 hi / lo)
        {
            __bf16* xh_r = xh + lr * LDK + 32 * part;
            __bf16* xl_r = xl + lr * LDK + 32 * part;
            if (pre) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    *reinterpret_cast<uint4*>(xh_r + 8 * i) = xon ? xp[i] : uint4{0, 0, 0, 0};
                    *reinterpret_cast<uint4*>(xl_r + 8 * i) = xon ? xp[4 + i] : uint4{0, 0, 0, 0};
                }
            } else {
                float xv[32];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float4 v = xon ? xr[i] : float4{0.f, 0.f, 0.f, 0.f};
                    xv[4 * i] = v.x;
                    xv[4 * i + 1] = v.y;
                    xv[4 * i + 2] = v.z;
                    xv[4 * i + 3] = v.w;
                }
#pragma unroll
                for (int i = 0; i < 4; i++) split_store8(xv + 8 * i, xh_r + 8 * i, xl_r + 8 * i);
            }
            float w[32];
            mm_wdeq<FMT>(wrg, g, wrow, won, k0, part, w);
#pragma unroll
            for (int i = 0; i < 32; i++) w[i] = won ? w[i] : 0.f;
            __bf16* wh_r = wh + lr * LDK;
            __bf16* wl_r = wl + lr * LDK;
            if constexpr (FMT == QP_Q4_K) {
                // w[0..15] -> k = 16*part + i (sub-block 2p), w[16..31] -> k = 32 + 16*part + i (sub-block 2p+1)
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    split_store8(w + 8 * i, wh_r + 16 * part + 8 * i, wl_r + 16 * part + 8 * i);
                    split_store8(w + 16 + 8 * i, wh_r + 32 + 16 * part + 8 * i, wl_r + 32 + 16 * part + 8 * i);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) split_store8(w + 8 * i, wh_r + 32 * part + 8 * i, wl_r + 32 * part + 8 * i);
            }
        }
        __syncthreads();
        if (s + 1 < nsteps) load(k0 + TK);
        // 4 k slices of 16: A = x (tokens x k), B = w^T (k x rows)
#pragma unroll
        for (int ks = 0; ks < TK / 16; ks++) {
            const uint32_t kk = ks * 16 + 8 * (lane >> 5);
            bf16x8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int a = 0; a < 2; a++) {
                const uint32_t tr = wm * 64 + a * 32 + (lane & 31);
                ah[a] = *reinterpret_cast<const bf16x8*>(xh + tr * LDK + kk);
                al[a] = *reinterpret_cast<const bf16x8*>(xl + tr * LDK + kk);
                const uint32_t nr = wn * 64 + a * 32 + (lane & 31);
                bh[a] = *reinterpret_cast<const bf16x8*>(wh + nr * LDK + kk);
                bl[a] = *reinterpret_cast<const bf16x8*>(wl + nr * LDK + kk);
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], bh[b], acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], bl[b], acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[a], bh[b], acc[a][b], 0, 0, 0);
                }
        }
        __syncthreads();
    }
    // D layout (32 x 32 block): lane holds column lane & 31, rows 8*(v/4) + 4*(lane/32) + v%4.  With ws, the
    // split's partial goes to its own plane.
    float* Y = g.ws ? mptr<float>(g.ws) + (uint64_t)zs * g.rows * N : mptr<float>(g.y);
    const bool add = g.acc && !g.ws;
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const uint32_t n = n0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t lt = wm * 64 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3), t = t0 + lt;
                const uint32_t row = grp ? jobs[lt] : t;
                if ((grp ? row != QP_NOJOB : t < T) && n < N) {
                    float* o = Y + (uint64_t)row * N + n;
                    *o = add ? *o + acc[a][b][v] : acc[a][b][v];
                }
            }
        }
}

// x [T][k] -> its bf16 high / low planes for the matrix-core matmul, in the layout of xs_off: one K step's quarter
// q of 256 consecutive tokens is 4 KB contiguous (a wavefront's load covers 1 KB), and a chunk's inputs past K
// are zeros.  Token rows T .. rows - 1 are not written: their products reach only outputs that are not
// stored.  One 16-byte group per thread and step, consecutive threads on consecutive tokens.  With mul (the grouped
// expert matmul's rows): row-major planes, consecutive threads on consecutive groups of one row.
KERNEL __launch_bounds__(256) void qp_split_bf16(QpSplitArgs a) {
    const uint32_t T = a.mul ? min(paso_T(a.paso) * a.mul, a.cap) : paso_T(a.paso), nq = ((a.k + 31) >> 5) * 4;
    const uint64_t n = (uint64_t)nq * T, plane = 2ull * a.rows * (((a.k + 31) >> 5) << 5);
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull) {
        uint32_t cq, t;
        if (a.mul) {
            t = (uint32_t)(i / nq);
            cq = (uint32_t)(i - (uint64_t)t * nq);
        } else {
            cq = (uint32_t)(i / T);
            t = (uint32_t)(i - (uint64_t)cq * T);
        }
        const uint32_t k8 = cq * 8;
        float v[8];
        if (k8 < a.k) {  // K is a multiple of 8 (16 for f32, 32 for Q8_0): a group is wholly inside or past the row
            const float4 v0 = gload<float4>(a.x + 4ull * ((uint64_t)t * a.k + k8));
            const float4 v1 = gload<float4>(a.x + 4ull * ((uint64_t)t * a.k + k8) + 16);
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        }
        const uint64_t o = a.mul ? 2ull * ((uint64_t)t * (nq * 8) + k8) : xs_off(t, k8, a.rows);
        split_store8(v, reinterpret_cast<__bf16*>(a.xs + o), reinterpret_cast<__bf16*>(a.xs + plane + o));
    }
}

// y[t][n] = (acc ? y : 0) + (ws[0] + ws[1] + ...)[t][n], the splits summed in order.
KERNEL __launch_bounds__(256) void qp_gemm_reduce(QpReduceArgs a) {
    const uint64_t tn = (uint64_t)paso_T(a.paso) * a.n, plane = (uint64_t)a.rows * a.n;
    const float* ws = cptr<float>(a.ws);
    float* y = mptr<float>(a.y);
    if ((a.n & 3) == 0 && a.splits <= 8 && ((a.ws | a.y) & 15) == 0) {
        // four outputs per thread, the splits' loads issued together; per output the same sum as below
        const float4* w4 = reinterpret_cast<const float4*>(ws);
        float4* y4 = reinterpret_cast<float4*>(y);
        const uint64_t p4 = plane >> 2;
        for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < (tn >> 2); i += (uint64_t)gridDim.x * 256ull) {
            float4 p[8];
#pragma unroll
            for (uint32_t z = 0; z < 8; z++)
                if (z < a.splits) p[z] = w4[z * p4 + i];
            float4 s = p[0];
#pragma unroll
            for (uint32_t z = 1; z < 8; z++)
                if (z < a.splits) {
                    s.x += p[z].x;
                    s.y += p[z].y;
                    s.z += p[z].z;
                    s.w += p[z].w;
                }
            if (a.acc) {
                const float4 o = y4[i];
                s = float4{o.x + s.x, o.y + s.y, o.z + s.z, o.w + s.w};
            }
            y4[i] = s;
        }
        return;
    }
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < tn; i += (uint64_t)gridDim.x * 256ull) {
        float s = ws[i];
        for (uint32_t z = 1; z < a.splits; z++) s += ws[z * plane + i];
        y[i] = a.acc ? y[i] + s : s;
    }
}

// ---- 256-token tiles (T >= 256, K-quant weights, the input split beforehand): 8 wavefronts in 4 x 2, each 64 x 64,
// so each dequantized weight tile feeds 256 tokens.  K steps of 32 with two LDS buffers and three register
// buffers: while the matrix instructions of step s read one LDS buffer, the waves dequantize step s + 1 into the
// other (the arithmetic overlaps the matrix cores) and the global loads of step s + 2 are in flight; one barrier
// per step.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// bf16 high/low parts of 8 floats, both rounded to nearest: 3 vector operations per value (the packed conversion
// of a pair, unpacking the high parts, the exact difference).
QP_DEV void split_store8_pk(const float (&v)[8], __bf16* hi, __bf16* lo) {
    u32x4 h, l;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){v[2 * p], v[2 * p + 1]}, bf16x2));
        const float l0 = v[2 * p] - __uint_as_float(hb << 16), l1 = v[2 * p + 1] - __uint_as_float(hb & 0xffff0000u);
        h[p] = hb;
        l[p] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){l0, l1}, bf16x2));
    }
    *reinterpret_cast<u32x4*>(hi) = h;
    *reinterpret_cast<u32x4*>(lo) = l;
}

// One thread's share of one 32-input K step: 16 inputs of one token row (both bf16 planes) and 8 weights of one
// output row.
struct MmW8 {
    u32x4 x[4];   // bf16 high (x[0..1]) and low (x[2..3]) of the 16 inputs
    u32x2 q;      // Q4_K: the 8 nibble bytes; Q6_K: the 8 low-bit bytes
    u32x4 h;      // Q4_K: the super-block header (d, dmin, 12 scale bytes)
    u32x2 qh;     // Q6_K: the 8 high-bit bytes; Q5_K: the 8 qh bytes
    uint32_t sc;  // Q6_K: the dword holding this sub-block's scale byte
    uint32_t d;   // Q6_K: the f16 super-block scale
};

// Per-thread byte offsets, fixed over the K loop; the step's own offsets are uniform (scalar soffset).  Weights of
// row r, inputs 8*sub .. 8*sub + 7 of the step at k0.  Q4_K: sub-block j = (k0 % 256) / 32 is the low (j even) or
// high (j odd) nibble of bytes l = 8*sub .. of the 32 qs bytes 32*(j/2) .., chunk 1 + 2*(j/2) + l/16.  Q6_K:
// block half h, quarter qd: ql chunk h*4 + (qd%2)*2 + l/16, qh chunk 8 + h*2 + l/16, scale byte h*8 + qd*2 + l/16.
struct MmOff {
    uint32_t x, q, h, d;
};

// quarters q and q + 2 of the step's 32-input chunk (xs_off), high plane then low plane
QP_DEV void mm8_xload(MmW8& r, const MmOff& o, __amdgpu_buffer_rsrc_t rx, uint32_t xplane, uint32_t xrows,
                      uint32_t k0) {
    const uint32_t xk = (k0 >> 5) * 64 * xrows, xq2 = 32 * xrows;
    r.x[0] = __builtin_amdgcn_raw_buffer_load_b128(rx, o.x, xk, 0);
    r.x[1] = __builtin_amdgcn_raw_buffer_load_b128(rx, o.x + xq2, xk, 0);
    r.x[2] = __builtin_amdgcn_raw_buffer_load_b128(rx, o.x, xplane + xk, 0);
    r.x[3] = __builtin_amdgcn_raw_buffer_load_b128(rx, o.x + xq2, xplane + xk, 0);
}

template <int FMT>
QP_DEV void mm8_wload(MmW8& r, const MmOff& o, __amdgpu_buffer_rsrc_t rw, uint32_t nb, uint32_t k0) {
    const uint32_t b = k0 >> 8, e0 = k0 & 255;
    if constexpr (FMT == QP_Q4_K) {
        const uint32_t j = e0 >> 5;
        r.q = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16 + (1 + 2 * (j >> 1)) * nb * 16, 0);
        r.h = __builtin_amdgcn_raw_buffer_load_b128(rw, o.h, b * 16, 0);
    } else if constexpr (FMT == QP_Q3_K || FMT == QP_Q2_K) {
        // element 128 n + 32 jj + l: Q3_K qs chunk 2 + 2n + l/16, hmask chunk l/16, scales and d chunk 6; Q2_K qs
        // chunk 1 + 2n + l/16, the scale byte 8n + 2jj + l/16 in chunk 0, (d, dmin) in the array after the rows
        const uint32_t n = e0 >> 7;
        if constexpr (FMT == QP_Q3_K) {
            r.q = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16 + (2 + 2 * n) * nb * 16, 0);
            r.qh = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16, 0);
            r.h = __builtin_amdgcn_raw_buffer_load_b128(rw, o.h, b * 16 + 6 * nb * 16, 0);
        } else {
            r.q = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16 + (1 + 2 * n) * nb * 16, 0);
            r.sc = __builtin_amdgcn_raw_buffer_load_b32(rw, o.h, b * 16 + 4 * ((8 * n + 2 * ((e0 & 127) >> 5)) >> 2), 0);
            r.d = __builtin_amdgcn_raw_buffer_load_b32(rw, o.d, b * 4, 0);
        }
    } else if constexpr (FMT == QP_Q5_K) {
        // qs chunk 3 + 2*(j/2) + l/16, qh chunk 1 + l/16 (the same 8 bytes l of both)
        const uint32_t j = e0 >> 5;
        r.q = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16 + (3 + 2 * (j >> 1)) * nb * 16, 0);
        r.qh = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16 + nb * 16, 0);
        r.h = __builtin_amdgcn_raw_buffer_load_b128(rw, o.h, b * 16, 0);
    } else {
        const uint32_t h = e0 >> 7, qd = (e0 & 127) >> 5;
        r.q = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16 + (h * 4 + (qd & 1) * 2) * nb * 16, 0);
        r.qh = __builtin_amdgcn_raw_buffer_load_b64(rw, o.q, b * 16 + (8 + h * 2) * nb * 16, 0);
        r.sc = __builtin_amdgcn_raw_buffer_load_b32(rw, o.h, b * 16 + 12 * nb * 16 + 4 * (h * 2 + (qd >> 1)), 0);
        r.d = __builtin_amdgcn_raw_buffer_load_b16(rw, o.d, b * 2, 0);
    }
}

template <int FMT>
QP_DEV void mm8_load(MmW8& r, const MmOff& o, __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rw, uint32_t xplane,
                     uint32_t xrows, uint32_t nb, uint32_t k0) {
    mm8_xload(r, o, rx, xplane, xrows, k0);
    mm8_wload<FMT>(r, o, rw, nb, k0);
}

template <int FMT>
QP_DEV void mm8_deq(const MmW8& r, uint32_t k0, uint32_t sub, float (&w)[8]) {
    const uint32_t e0 = k0 & 255;
    uint32_t v[2];
    float f, c;
    if constexpr (FMT == QP_Q3_K) {
        // fma(fd, q', -4 fd) = fd * (q' - 4) exactly (one rounding of the same value), q' = q2 | hbit << 2
        const uint32_t n = e0 >> 7, jj = (e0 & 127) >> 5, s = 8 * n + 2 * jj + (sub >> 1);
        f = h2f(r.h.w & 0xffffu) * ((float)q3k_scale6(r.h.x, r.h.y, r.h.z, s) - 32.0f);
        c = -4.0f * f;
        v[0] = ((r.q.x >> (2 * jj)) & 0x03030303u) | (((r.qh.x >> (4 * n + jj)) & 0x01010101u) << 2);
        v[1] = ((r.q.y >> (2 * jj)) & 0x03030303u) | (((r.qh.y >> (4 * n + jj)) & 0x01010101u) << 2);
    } else if constexpr (FMT == QP_Q2_K) {
        const uint32_t n = e0 >> 7, jj = (e0 & 127) >> 5, j = 8 * n + 2 * jj + (sub >> 1);
        const uint32_t sc = (r.sc >> ((j & 3) * 8)) & 0xffu;
        f = h2f(r.d & 0xffffu) * (float)(sc & 15u);
        c = -(h2f(r.d >> 16) * (float)(sc >> 4));
        v[0] = (r.q.x >> (2 * jj)) & 0x03030303u;
        v[1] = (r.q.y >> (2 * jj)) & 0x03030303u;
    } else if constexpr (FMT == QP_Q4_K || FMT == QP_Q5_K) {
        // fd*q - fm; a Q4_K high nibble is masked in place (16*q) with the scale divided by 16 (exact); Q5_K
        // shifts the nibble down and adds 16 * bit j of qh
        const uint32_t j = e0 >> 5, jj = (j & 3) * 8;  // the scale/min unpack of q4k_sm, without a branch
        const uint32_t sa = (r.h.y >> jj) & 0xffu, sb = (r.h.z >> jj) & 0xffu, s8 = (r.h.w >> jj) & 0xffu;
        const uint32_t lo4 = 0u - (uint32_t)(j < 4);  // all ones for j < 4: a blend, not a branch
        const uint32_t sc = ((sa & 63u) & lo4) | (((s8 & 15u) | ((sa >> 6) << 4)) & ~lo4);
        const uint32_t mn = ((sb & 63u) & lo4) | (((s8 >> 4) | ((sb >> 6) << 4)) & ~lo4);
        c = -(h2f(r.h.x >> 16) * (float)mn);
        if constexpr (FMT == QP_Q4_K) {
            const uint32_t mask = (j & 1) ? 0xf0f0f0f0u : 0x0f0f0f0fu;
            f = h2f(r.h.x & 0xffffu) * (float)sc * ((j & 1) ? 0.0625f : 1.0f);
            v[0] = r.q.x & mask;
            v[1] = r.q.y & mask;
        } else {
            const uint32_t ns = (j & 1) * 4;
            f = h2f(r.h.x & 0xffffu) * (float)sc;
            v[0] = ((r.q.x >> ns) & 0x0f0f0f0fu) | (((r.qh.x >> j) & 0x01010101u) << 4);
            v[1] = ((r.q.y >> ns) & 0x0f0f0f0fu) | (((r.qh.y >> j) & 0x01010101u) << 4);
        }
    } else {
        // fd*(q - 32) = fma(fd, q, -32*fd) exactly (both are one rounding of the same product)
        const uint32_t qd = (e0 & 127) >> 5, sb = ((qd & 1) * 2 + (sub >> 1)) * 8;
        f = h2f(r.d & 0xffffu) * (float)(int8_t)((r.sc >> sb) & 0xffu);
        c = -32.0f * f;
        const uint32_t ls = (qd >> 1) * 4, hs = qd * 2;
        v[0] = ((r.q.x >> ls) & 0x0f0f0f0fu) | (((r.qh.x >> hs) & 0x03030303u) << 4);
        v[1] = ((r.q.y >> ls) & 0x0f0f0f0fu) | (((r.qh.y >> hs) & 0x03030303u) << 4);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = __builtin_fmaf(f, (float)((v[i >> 2] >> (8 * (i & 3))) & 0xffu), c);
}

template <int FMT>
QP_DEV void gemm_mfma256_body(const QpGemmArgs& g) {
    constexpr int TM = 256, TN = 128, TK = 32, LDK = 40, BUF = (TM + TM + TN + TN) * LDK;  // bf16 per buffer
    extern __shared__ float4 smem4[];
    __bf16* lds = reinterpret_cast<__bf16*>(smem4);
    const uint32_t T = g.tfix ? g.tfix : paso_T(g.paso);
    const uint32_t N = g.n, K = g.k;
    const uint32_t mt = (uint32_t)gridDim.y, ntl = (uint32_t)gridDim.x, nz = (uint32_t)gridDim.z;
    const uint32_t total = mt * ntl * nz, id = (blockIdx.z * mt + blockIdx.y) * ntl + blockIdx.x;
    const uint32_t base = total >> 3, rem = total & 7, xcd = id & 7, j = id >> 3;
    const uint32_t L = xcd * base + (xcd < rem ? xcd : rem) + j;
    const uint32_t m_tile = L % mt, rest = L / mt, zs = rest % nz, n_tile = rest / nz;
    const uint32_t t0 = m_tile * TM, n0 = n_tile * TN;
    if (t0 >= T) return;
    const uint32_t kbeg = g.kchunk ? zs * g.kchunk : 0;
    const uint32_t kend = g.kchunk ? min(K, kbeg + g.kchunk) : K;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    // loaders, so that each 16-lane phase of an LDS store covers 16 rows: input row lr, quarters xq and xq + 2 of
    // the step's 32 inputs (a wavefront loads 64 consecutive rows of one quarter: 1 KB contiguous); weight row wq (8
    // inputs at 8*sub).  Weight rows past N load row 0; input rows past T read rows of the planes that the split
    // did not write (rows < g.rows, inside the buffer), whose outputs are not stored.
    const uint32_t lr = tid & 255, xq = tid >> 8, wq = wave * 16 + (lane & 15), sub = lane >> 4;
    const uint32_t wr = n0 + wq < N ? n0 + wq : 0;
    const uint32_t nb = K >> 8, xplane = 2 * g.rows * K;
    const __amdgpu_buffer_rsrc_t rx = kq_rsrc(g.xs, 2ull * xplane);
    constexpr uint32_t RBW = KQ<FMT>::RB;  // bytes per weight row and 256 inputs (Q6_K: its d array follows)
    const __amdgpu_buffer_rsrc_t rw = kq_rsrc(g.w, (uint64_t)N * nb * (FMT == QP_Q6_K ? 210 : FMT == QP_Q2_K ? 84 : RBW));
    MmOff off;
    off.x = (xq * g.rows + t0 + lr) * 16;
    off.q = wr * nb * RBW + (sub >> 1) * nb * 16 + (sub & 1) * 8;
    off.h = wr * nb * RBW;
    off.d = FMT == QP_Q2_K ? N * nb * 80 + wr * nb * 4 : N * nb * 208 + wr * nb * 2;
    const uint32_t nsteps = (kend - kbeg + TK - 1) / TK;
    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;
    MmW8 r0, r1;
    auto load = [&](MmW8& r, uint32_t st) __attribute__((always_inline)) {
        // past the last step: reload it (unused)
        mm8_load<FMT>(r, off, rx, rw, xplane, g.rows, nb, kbeg + min(st, nsteps - 1) * TK);
    };
    auto stage = [&](const MmW8& r, uint32_t st, __bf16* buf) __attribute__((always_inline)) {
        __bf16* xh = buf;
        __bf16* xl = xh + TM * LDK;
        __bf16* wh = xl + TM * LDK;
        __bf16* wl = wh + TN * LDK;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            *reinterpret_cast<u32x4*>(xh + lr * LDK + 8 * (xq + 2 * i)) = r.x[i];
            *reinterpret_cast<u32x4*>(xl + lr * LDK + 8 * (xq + 2 * i)) = r.x[2 + i];
        }
        float w[8];
        mm8_deq<FMT>(r, kbeg + min(st, nsteps - 1) * TK, sub, w);
        split_store8_pk(w, wh + wq * LDK + 8 * sub, wl + wq * LDK + 8 * sub);
    };
    // step s: the loads of step s + 2 go into the registers step s came in (staged during step s - 1), the
    // matrix instructions read LDS buffer s % 2, and step s + 1 is dequantized into the other buffer
    auto step = [&](uint32_t s, MmW8& mine, MmW8& next) __attribute__((always_inline)) {
        load(mine, s + 2);
        const __bf16* xh = lds + (s & 1) * BUF;
        const __bf16* xl = xh + TM * LDK;
        const __bf16* wh = xl + TM * LDK;
        const __bf16* wl = wh + TN * LDK;
#pragma unroll
        for (int ks = 0; ks < TK / 16; ks++) {
            const uint32_t kk = ks * 16 + 8 * (lane >> 5);
            bf16x8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int a = 0; a < 2; a++) {
                const uint32_t tr = wm * 64 + a * 32 + (lane & 31);
                ah[a] = *reinterpret_cast<const bf16x8*>(xh + tr * LDK + kk);
                al[a] = *reinterpret_cast<const bf16x8*>(xl + tr * LDK + kk);
                const uint32_t nr = wn * 64 + a * 32 + (lane & 31);
                bh[a] = *reinterpret_cast<const bf16x8*>(wh + nr * LDK + kk);
                bl[a] = *reinterpret_cast<const bf16x8*>(wl + nr * LDK + kk);
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], bh[b], acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], bl[b], acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[a], bh[b], acc[a][b], 0, 0, 0);
                }
        }
        stage(next, s + 1, lds + ((s + 1) & 1) * BUF);  // after the last step: a copy of it, never read
        // issue order: the step's global loads, the first operand reads, then each matrix instruction followed by
        // two vector operations of the next step's dequantization (so both pipes stay busy), the remaining operand
        // reads spread between them, the LDS stores last
        __builtin_amdgcn_sched_group_barrier(0x020, 16, 0);  // VMEM reads
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);   // DS reads (ks 0)
#pragma unroll
        for (int i = 0; i < 12; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read (ks 1)
            __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // VALU
        }
#pragma unroll
        for (int i = 0; i < 12; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
        __builtin_amdgcn_sched_group_barrier(0x200, 16, 0);  // DS writes
        __syncthreads();
    };
    load(r0, 0);
    load(r1, 1);
    stage(r0, 0, lds);
    __syncthreads();
    for (uint32_t s = 0; s < nsteps; s += 2) {  // nsteps is even: every K range is whole 64-input steps
        step(s, r0, r1);
        step(s + 1, r1, r0);
    }
    float* Y = g.ws ? mptr<float>(g.ws) + (uint64_t)zs * g.rows * N : mptr<float>(g.y);
    const bool add = g.acc && !g.ws;
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const uint32_t n = n0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t t = t0 + wm * 64 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (t < T && n < N) {
                    float* o = Y + (uint64_t)t * N + n;
                    *o = add ? *o + acc[a][b][v] : acc[a][b][v];
                }
            }
        }
}

// ---- 256-token x 256-row tiles (large K-quant matmuls): 8 wavefronts in 2 x 4, each 128 tokens x 64 rows (4 x 2
// matrix blocks), so that every operand fragment read from LDS feeds more matrix instructions and each input step
// loaded feeds twice the rows of the 256 x 128 tile.  Same K steps of 32, two LDS buffers of 80 KB (the whole
// 160 KB), the loads of step s + 2 in flight during step s, one barrier per step.  Thread tid stages input row
// tid % 256 (quarters tid / 256 and + 2) and the 8 weights at 8*sub of rows wq and wq + 128.
// GLU (matmul_<fmt>_t_swiglu): the tile's rows 0..127 are rows n0.. of the gate tensor and rows 128..255 the same
// rows of the up tensor (w2), so a tile covers 128 outputs; the up wavefronts hand their sums to the gate
// wavefronts through LDS and y = silu(gate) * up is stored (the swiglu kernel's formula; no K split).
template <int FMT, bool GLU = false>
QP_DEV void gemm_mfma256w_body(const QpGemmArgs& g) {
    constexpr int TM = 256, TN = 256, TK = 32, LDK = 40, BUF = (TM + TM + TN + TN) * LDK;  // bf16 per buffer
    extern __shared__ float4 smem4[];
    __bf16* lds = reinterpret_cast<__bf16*>(smem4);
    const uint32_t T = g.tfix ? g.tfix : paso_T(g.paso);
    const uint32_t N = g.n, K = g.k;
    const bool split_tail = GLU && g.tail != 0;
    const uint32_t mt = split_tail ? g.mtiles : (uint32_t)gridDim.y, ntl = split_tail ? g.ntiles : (uint32_t)gridDim.x;
    const uint32_t nz = split_tail ? 1u : (uint32_t)gridDim.z;
    uint32_t L, half = 0, stile = 0;  // stile: the split tile's index among the tail tiles
    bool split = false;
    if (split_tail) {
        // per XCD x (item % 8): whole tiles x * F .. x * F + F - 1, then K halves of tail tiles full + x * H ..
        const uint32_t full = mt * ntl - g.tail, F = full >> 3, H = g.tail >> 3;
        const uint32_t xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
        if (j < F) {
            L = xcd * F + j;
        } else {
            const uint32_t jj = j - F;
            stile = xcd * H + (jj >> 1);
            L = full + stile;
            half = jj & 1;
            split = true;
        }
    } else {
        const uint32_t total = mt * ntl * nz, id = (blockIdx.z * mt + blockIdx.y) * ntl + blockIdx.x;
        const uint32_t base = total >> 3, rem = total & 7, xcd = id & 7, j = id >> 3;
        L = xcd * base + (xcd < rem ? xcd : rem) + j;
    }
    const uint32_t m_tile = L % mt, rest = L / mt, zs = rest % nz, n_tile = rest / nz;
    const uint32_t t0 = m_tile * TM, n0 = n_tile * (GLU ? TN / 2 : TN);
    if (t0 >= T) return;  // (both halves of a split tile: neither counts, nothing is stored)
    const uint32_t kbeg = split ? half * (K >> 1) : g.kchunk ? zs * g.kchunk : 0;
    const uint32_t kend = split ? kbeg + (K >> 1) : g.kchunk ? min(K, kbeg + g.kchunk) : K;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave >> 2, wn = wave & 3;
    const uint32_t lr = tid & 255, xq = tid >> 8, wq = wave * 16 + (lane & 15), sub = lane >> 4;
    // weight rows past N load row 0 (finite values whose outputs are not stored)
    const uint32_t wr0 = n0 + wq < N ? n0 + wq : 0;
    const uint32_t wr1 = GLU ? wr0 : n0 + wq + 128 < N ? n0 + wq + 128 : 0;
    const uint32_t nb = K >> 8, xplane = 2 * g.rows * K;
    const __amdgpu_buffer_rsrc_t rx = kq_rsrc(g.xs, 2ull * xplane);
    constexpr uint32_t RBW = KQ<FMT>::RB;
    const uint64_t wbytes = (uint64_t)N * nb * (FMT == QP_Q6_K ? 210 : FMT == QP_Q2_K ? 84 : RBW);
    const __amdgpu_buffer_rsrc_t rw = kq_rsrc(g.w, wbytes);
    const __amdgpu_buffer_rsrc_t rw1 = GLU ? kq_rsrc(g.w2, wbytes) : rw;  // the tensor of row wq + 128
    MmOff o0;
    o0.x = (xq * g.rows + t0 + lr) * 16;
    o0.q = wr0 * nb * RBW + (sub >> 1) * nb * 16 + (sub & 1) * 8;
    o0.h = wr0 * nb * RBW;
    o0.d = FMT == QP_Q2_K ? N * nb * 80 + wr0 * nb * 4 : N * nb * 208 + wr0 * nb * 2;
    MmOff o1 = o0;  // row wq + 128 (GLU: row wq of the up tensor)
    o1.q = wr1 * nb * RBW + (sub >> 1) * nb * 16 + (sub & 1) * 8;
    o1.h = wr1 * nb * RBW;
    o1.d = FMT == QP_Q2_K ? N * nb * 80 + wr1 * nb * 4 : N * nb * 208 + wr1 * nb * 2;
    const uint32_t nsteps = (kend - kbeg + TK - 1) / TK;
    f32x16 acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;
    struct R2 {
        MmW8 a, b;  // a: the inputs and the weights of row wq; b: the weights of row wq + 128
    };
    R2 r0, r1;
    auto load = [&](R2& r, uint32_t st) __attribute__((always_inline)) {
        const uint32_t k0 = kbeg + min(st, nsteps - 1) * TK;  // past the last step: reload it (unused)
        mm8_xload(r.a, o0, rx, xplane, g.rows, k0);
        mm8_wload<FMT>(r.a, o0, rw, nb, k0);
        mm8_wload<FMT>(r.b, o1, rw1, nb, k0);
    };
    auto stage = [&](const R2& r, uint32_t st, __bf16* buf) __attribute__((always_inline)) {
        __bf16* xh = buf;
        __bf16* xl = xh + TM * LDK;
        __bf16* wh = xl + TM * LDK;
        __bf16* wl = wh + TN * LDK;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            *reinterpret_cast<u32x4*>(xh + lr * LDK + 8 * (xq + 2 * i)) = r.a.x[i];
            *reinterpret_cast<u32x4*>(xl + lr * LDK + 8 * (xq + 2 * i)) = r.a.x[2 + i];
        }
        const uint32_t k0 = kbeg + min(st, nsteps - 1) * TK;
        float w[8];
        mm8_deq<FMT>(r.a, k0, sub, w);
        split_store8_pk(w, wh + wq * LDK + 8 * sub, wl + wq * LDK + 8 * sub);
        mm8_deq<FMT>(r.b, k0, sub, w);
        split_store8_pk(w, wh + (wq + 128) * LDK + 8 * sub, wl + (wq + 128) * LDK + 8 * sub);
    };
    auto step = [&](uint32_t s, R2& mine, R2& next) __attribute__((always_inline)) {
        load(mine, s + 2);
        const __bf16* xh = lds + (s & 1) * BUF;
        const __bf16* xl = xh + TM * LDK;
        const __bf16* wh = xl + TM * LDK;
        const __bf16* wl = wh + TN * LDK;
#pragma unroll
        for (int ks = 0; ks < TK / 16; ks++) {
            const uint32_t kk = ks * 16 + 8 * (lane >> 5);
            // the weight fragments for all four token blocks; the token fragments one block at a time (registers)
            bf16x8 bh[2], bl[2];
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const uint32_t nr = wn * 64 + b * 32 + (lane & 31);
                bh[b] = *reinterpret_cast<const bf16x8*>(wh + nr * LDK + kk);
                bl[b] = *reinterpret_cast<const bf16x8*>(wl + nr * LDK + kk);
            }
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const uint32_t tr = wm * 128 + a * 32 + (lane & 31);
                const bf16x8 ah = *reinterpret_cast<const bf16x8*>(xh + tr * LDK + kk);
                const bf16x8 al = *reinterpret_cast<const bf16x8*>(xl + tr * LDK + kk);
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    f32x16& c = acc[a][b];
                    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[b], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[b], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[b], c, 0, 0, 0);
                }
            }
        }
        stage(next, s + 1, lds + ((s + 1) & 1) * BUF);  // after the last step: a copy of it, never read
        __builtin_amdgcn_sched_group_barrier(0x020, 24, 0);  // VMEM reads
        __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // DS reads (ks 0)
#pragma unroll
        for (int i = 0; i < 24; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
#pragma unroll
        for (int i = 0; i < 12; i++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read (ks 1)
            __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // VALU
        }
#pragma unroll
        for (int i = 0; i < 24; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
        __builtin_amdgcn_sched_group_barrier(0x200, 16, 0);  // DS writes
        __syncthreads();
    };
    load(r0, 0);
    load(r1, 1);
    stage(r0, 0, lds);
    __syncthreads();
    for (uint32_t s = 0; s < nsteps; s += 2) {  // nsteps is even: every K range is whole 64-input steps
        step(s, r0, r1);
        step(s + 1, r1, r0);
    }
    if constexpr (GLU) {
        if (split) {
            // this half's sums to its slot, [wave][a][b][v][lane]; drained, then one agent-scope arrival (its
            // release writes the L2 back); the second arrival adds the other slot (the sum of the two halves does
            // not depend on which arrives last) and goes on with the whole tile
            float* mine = mptr<float>(g.part) + ((uint64_t)stile * 2 + half) * (512u * 128u);
            const float* other = cptr<float>(g.part) + ((uint64_t)stile * 2 + (half ^ 1u)) * (512u * 128u);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int v = 0; v < 16; v++) mine[(((wave * 4 + a) * 2 + b) * 16 + v) * 64 + lane] = acc[a][b][v];
            vm_drain();
            uint32_t* second = reinterpret_cast<uint32_t*>(smem4);  // the K loop's LDS is free after this barrier
            __syncthreads();
            if (tid == 0) {
                QP_GLOBAL uint32_t* c = reinterpret_cast<QP_GLOBAL uint32_t*>(g.cnt) + stile;
                const uint32_t old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
                *second = old == 1u;
                if (old == 1u) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (!*second) return;
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        acc[a][b][v] = acc[a][b][v] + other[(((wave * 4 + a) * 2 + b) * 16 + v) * 64 + lane];
        }
        // the up sums (wavefronts wn = 2, 3) to LDS, read by the gate wavefronts wn - 2 at the same index
        __syncthreads();  // every wavefront has read the last step's LDS buffer
        float* ex = reinterpret_cast<float*>(smem4);  // [wm][2][4][2][16][64] floats: 128 KB
        if (wn >= 2) {
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        ex[((((wm * 2 + (wn - 2)) * 4 + a) * 2 + b) * 16 + v) * 64 + lane] = acc[a][b][v];
        }
        __syncthreads();
        if (g.yplanes) {
            // y as the next matmul's input planes (xs_off's layout, g.rows token rows, K = N): the gate wavefronts'
            // outputs go to an LDS tile [256 tokens][128 outputs] (rows padded to 132 floats) once the up sums are
            // read, then every thread splits eight consecutive outputs of one token with qp_split_bf16's formula
            // (the same planes that kernel makes of the f32 outputs) and stores their 16-byte high and low parts;
            // token rows past T are not written
            if (wn < 2) {
#pragma unroll
                for (int a = 0; a < 4; a++)
#pragma unroll
                    for (int b = 0; b < 2; b++)
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const float gv = acc[a][b][v];
                            const float uv = ex[((((wm * 2 + wn) * 4 + a) * 2 + b) * 16 + v) * 64 + lane];
                            acc[a][b][v] = (gv / (1.0f + expf(-gv))) * uv;
                        }
            }
            __syncthreads();
            float* tile = reinterpret_cast<float*>(smem4);
            if (wn < 2) {
#pragma unroll
                for (int a = 0; a < 4; a++)
#pragma unroll
                    for (int b = 0; b < 2; b++)
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const uint32_t t = wm * 128 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                            tile[t * 132 + wn * 64 + b * 32 + (lane & 31)] = acc[a][b][v];
                        }
            }
            __syncthreads();
            const uint64_t plane = 2ull * g.rows * N;  // bytes of the high plane (N % 32 == 0)
            for (uint32_t i = tid; i < 256 * 16; i += 512) {
                const uint32_t t = i & 255, c8 = i >> 8, n = n0 + 8 * c8;
                if (t0 + t >= T || n >= N) continue;
                const float4 v0 = *reinterpret_cast<const float4*>(tile + t * 132 + 8 * c8);
                const float4 v1 = *reinterpret_cast<const float4*>(tile + t * 132 + 8 * c8 + 4);
                const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                const uint64_t o = xs_off(t0 + t, n, g.rows);
                split_store8(v, reinterpret_cast<__bf16*>(g.y + o), reinterpret_cast<__bf16*>(g.y + plane + o));
            }
            return;
        }
        if (wn >= 2) return;
        float* Y = mptr<float>(g.y);
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const uint32_t n = n0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const uint32_t t = t0 + wm * 128 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    const float gv = acc[a][b][v];
                    const float uv = ex[((((wm * 2 + wn) * 4 + a) * 2 + b) * 16 + v) * 64 + lane];
                    if (t < T && n < N) Y[(uint64_t)t * N + n] = (gv / (1.0f + expf(-gv))) * uv;
                }
            }
        return;
    }
    float* Y = g.ws ? mptr<float>(g.ws) + (uint64_t)zs * g.rows * N : mptr<float>(g.y);
    const bool add = g.acc && !g.ws;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const uint32_t n = n0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t t = t0 + wm * 128 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (t < T && n < N) {
                    float* o = Y + (uint64_t)t * N + n;
                    *o = add ? *o + acc[a][b][v] : acc[a][b][v];
                }
            }
        }
}

KERNEL __launch_bounds__(512) void qp_gemm_mfma256w_q4k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q4_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256w_q5k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q5_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256w_q6k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q6_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256w_q3k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q3_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256w_q2k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q2_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_glu_q4k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q4_K, true>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_glu_q5k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q5_K, true>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_glu_q6k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q6_K, true>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_glu_q3k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q3_K, true>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_glu_q2k(QpGemmArgs a) { gemm_mfma256w_body<QP_Q2_K, true>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256_q4k(QpGemmArgs a) { gemm_mfma256_body<QP_Q4_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256_q5k(QpGemmArgs a) { gemm_mfma256_body<QP_Q5_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256_q3k(QpGemmArgs a) { gemm_mfma256_body<QP_Q3_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256_q2k(QpGemmArgs a) { gemm_mfma256_body<QP_Q2_K>(a); }
KERNEL __launch_bounds__(512) void qp_gemm_mfma256_q6k(QpGemmArgs a) { gemm_mfma256_body<QP_Q6_K>(a); }

KERNEL __launch_bounds__(256) void qp_gemm_mfma_q4k(QpGemmArgs a) { gemm_mfma_body<QP_Q4_K>(a); }
KERNEL __launch_bounds__(256) void qp_gemm_mfma_q6k(QpGemmArgs a) { gemm_mfma_body<QP_Q6_K>(a); }
KERNEL __launch_bounds__(256) void qp_gemm_mfma_q8(QpGemmArgs a) { gemm_mfma_body<QP_Q8_0>(a); }
KERNEL __launch_bounds__(256) void qp_gemm_mfma_iq4nl(QpGemmArgs a) { gemm_mfma_body<QP_IQ4_NL>(a); }
KERNEL __launch_bounds__(256) void qp_gemm_mfma_q5k(QpGemmArgs a) { gemm_mfma_body<QP_Q5_K>(a); }
KERNEL __launch_bounds__(256) void qp_gemm_mfma_q3k(QpGemmArgs a) { gemm_mfma_body<QP_Q3_K>(a); }
KERNEL __launch_bounds__(256) void qp_gemm_mfma_q2k(QpGemmArgs a) { gemm_mfma_body<QP_Q2_K>(a); }
KERNEL __launch_bounds__(256) void qp_gemm_mfma_f32(QpGemmArgs a) { gemm_mfma_body<QP_F32>(a); }

// ====================================================================================== RMSNorm
// Reference rmsnorm (gpu.js:332-356), same reduction order: 256 threads stride the row, LDS tree 128..1,
// y = (x * inv) * w.  ultima = 1: only row T-1, written to row 0.
KERNEL __launch_bounds__(256) void qp_rmsnorm(QpRmsArgs a) {
    __shared__ float red[256];
    const uint32_t T = a.rows_fixed ? a.rows_fixed : paso_T(a.paso);
    const uint32_t li = threadIdx.x, D = a.d;
    uint32_t fila = blockIdx.x, out = blockIdx.x;
    if (a.ultima) { fila = T - 1; out = 0; }
    else if (fila >= T) return;
    const float* x = cptr<float>(a.x) + (uint64_t)fila * D;
    float s = 0.0f;
    for (uint32_t i = li; i < D; i += 256) { const float v = x[i]; s = s + v * v; }
    red[li] = s;
    __syncthreads();
    for (uint32_t k = 128; k > 0; k >>= 1) {
        if (li < k) red[li] = red[li] + red[li + k];
        __syncthreads();
    }
    const float inv = 1.0f / sqrtf(red[0] / (float)D + a.eps);
    const float* w = cptr<float>(a.w);
    float* y = mptr<float>(a.y) + (uint64_t)out * D;
    for (uint32_t i = li; i < D; i += 256) y[i] = (x[i] * inv) * w[i];
}

// The rmsnorm of R token rows per workgroup written as the next matmul's input planes (xs_off's layout, a.rows
// rows; rows past T are not written): qp_rmsnorm's sums in its order (256 threads stride each row, the LDS tree
// 128 .. 1, the R trees side by side) and its y = (x * inv) * w, split with qp_split_bf16's formula, so the planes
// are those qp_split_bf16 makes of qp_rmsnorm's rows.  The rows are kept in LDS from the first pass (row stride
// D + 4 floats: the R rows' reads of one chunk fall in different banks); the second takes eight consecutive inputs
// per thread, consecutive threads on consecutive rows (R threads store 16 R contiguous bytes of a plane).  R = 8 up
// to D = 4096, 4 up to 8192, 2 up to 16384 (the rows fill up to 128 KB of dynamic LDS).
template <uint32_t R>
QP_DEV void rmsnorm_planes_body(const QpRmsPlanesArgs& a) {
    extern __shared__ float4 smem4[];
    float* xr = reinterpret_cast<float*>(smem4);  // [R][D + 4]
    __shared__ float red[R][256];
    __shared__ float inv_s[R];
    const uint32_t T = paso_T(a.paso), li = threadIdx.x, D = a.d, t0 = blockIdx.x * R, ld = D + 4;
    if (t0 >= T) return;
    const uint32_t nr = min(R, T - t0);
    // the R rows' loads of U stride steps issued together (each row's sum still in qp_rmsnorm's order)
    float s[R];
#pragma unroll
    for (uint32_t r = 0; r < R; r++) s[r] = 0.0f;
    // four stride steps' loads in flight at once (a step past D loads 0, which adds nothing to a sum)
    const float* xb = cptr<float>(a.x) + (uint64_t)t0 * D;
    constexpr uint32_t U = 32 / R;
    for (uint32_t i0 = li; i0 < D; i0 += 256 * U) {
        float v[U][R];
#pragma unroll
        for (uint32_t u = 0; u < U; u++)
#pragma unroll
            for (uint32_t r = 0; r < R; r++) {
                const uint32_t i = i0 + 256 * u;
                v[u][r] = r < nr && i < D ? xb[(uint64_t)r * D + i] : 0.0f;
            }
#pragma unroll
        for (uint32_t u = 0; u < U; u++)
#pragma unroll
            for (uint32_t r = 0; r < R; r++) {
                const uint32_t i = i0 + 256 * u;
                s[r] = s[r] + v[u][r] * v[u][r];
                if (i < D) xr[r * ld + i] = v[u][r];
            }
    }
#pragma unroll
    for (uint32_t r = 0; r < R; r++) red[r][li] = s[r];
    __syncthreads();
    for (uint32_t k = 128; k > 0; k >>= 1) {
        if (li < k)
            for (uint32_t r = 0; r < R; r++) red[r][li] = red[r][li] + red[r][li + k];
        __syncthreads();
    }
    if (li < R) inv_s[li] = 1.0f / sqrtf(red[li][0] / (float)D + a.eps);
    __syncthreads();
    const uint64_t plane = 2ull * a.rows * D;  // bytes of the high plane (D % 32 == 0)
    // four chunks per round, their norm weight loads issued first (r and the chunk's first input: the thread's
    // row stays r = li % R since 256 is a multiple of R)
    const uint32_t r = li % R, t = t0 + r;
    const float inv = inv_s[r];
    const bool on = r < nr;
    for (uint32_t i0 = li; i0 < R * (D / 8); i0 += 4 * 256) {
        float4 wv[4][2];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t k8 = ((i0 + 256 * u) / R) * 8;
            const bool in = i0 + 256 * u < R * (D / 8);
            wv[u][0] = in ? gload<float4>(a.w + 4ull * k8) : float4{0.0f, 0.0f, 0.0f, 0.0f};
            wv[u][1] = in ? gload<float4>(a.w + 4ull * k8 + 16) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            // no contraction: the product must be rounded to y before the split subtracts its high part (an FMA of
            // (x * inv) * w - hi would give another low part than qp_split_bf16 gives of the rounded y)
#pragma clang fp contract(off)
            const uint32_t i = i0 + 256 * u, k8 = (i / R) * 8;
            if (!on || i >= R * (D / 8)) continue;
            const float4 x0 = *reinterpret_cast<const float4*>(xr + r * ld + k8);
            const float4 x1 = *reinterpret_cast<const float4*>(xr + r * ld + k8 + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const float ww[8] = {wv[u][0].x, wv[u][0].y, wv[u][0].z, wv[u][0].w,
                                 wv[u][1].x, wv[u][1].y, wv[u][1].z, wv[u][1].w};
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = (xv[j] * inv) * ww[j];
            const uint64_t o = xs_off(t, k8, a.rows);
            split_store8(v, reinterpret_cast<__bf16*>(a.xs + o), reinterpret_cast<__bf16*>(a.xs + plane + o));
        }
    }
}
KERNEL __launch_bounds__(256) void qp_rmsnorm_planes(QpRmsPlanesArgs a) { rmsnorm_planes_body<8>(a); }
KERNEL __launch_bounds__(256) void qp_rmsnorm_planes4(QpRmsPlanesArgs a) { rmsnorm_planes_body<4>(a); }
KERNEL __launch_bounds__(256) void qp_rmsnorm_planes2(QpRmsPlanesArgs a) { rmsnorm_planes_body<2>(a); }

// ====================================================================================== norm + RoPE
// Reference norm_rope (gpu.js:394-444), one wavefront per head vector.
QP_DEV void wave_norm_rope_f(float* v, const float* w, uint32_t hd, bool use_norm, float eps, float pos_esc,
                             const float* freq, uint32_t nrot, bool neox, int lane);

// grid (ceil(nh / 4), ceil(T / 4)): wavefront i of a workgroup takes head 4*blockIdx.x + i of the four tokens
// from 4*blockIdx.y.  The frequency table base^(-2j/nrot) (each value rounded once to float from double, as
// rope_elem computes it per element) is read from a.freq (the host's table of the same values), or built once per
// workgroup.
KERNEL __launch_bounds__(256) void qp_norm_rope(QpRopeArgs a) {
    __shared__ float v[4][256];
    __shared__ float freq[128];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = blockIdx.x * 4 + wave;
    const uint32_t T = paso_T(a.paso), t0 = blockIdx.y * 4;
    if (t0 >= T) return;
    if (threadIdx.x < a.nrot / 2)
        freq[threadIdx.x] = a.freq ? cptr<float>(a.freq)[threadIdx.x]
                                   : (float)pow((double)a.base, (double)((-2.0f * (float)threadIdx.x) / (float)a.nrot));
    __syncthreads();
    if (h >= a.nh) return;
    // the four rows' loads issued together (hd <= 256: at most 4 values per lane and row)
    const uint32_t nt = min(T, t0 + 4) - t0;
    float pre[4][4];
#pragma unroll
    for (uint32_t r = 0; r < 4; r++)
#pragma unroll
        for (uint32_t c = 0; c < 4; c++) {
            const uint32_t i = lane + 64 * c;
            pre[r][c] = r < nt && i < a.hd ? cptr<float>(a.v)[((uint64_t)(t0 + r) * a.nh + h) * a.hd + i] : 0.0f;
        }
#pragma unroll
    for (uint32_t r = 0; r < 4; r++) {
        if (r >= nt) break;
        const uint32_t t = t0 + r;
        float* row = mptr<float>(a.v) + ((uint64_t)t * a.nh + h) * a.hd;
#pragma unroll
        for (uint32_t c = 0; c < 4; c++)
            if (lane + 64 * c < a.hd) v[wave][lane + 64 * c] = pre[r][c];
        __builtin_amdgcn_wave_barrier();
        const float pos = (float)(paso_pos(a.paso) + t);
        wave_norm_rope_f(v[wave], a.w ? cptr<float>(a.w) : nullptr, a.hd, a.use_norm != 0, a.eps, pos * a.esc, freq,
                         a.nrot, a.neox != 0, (int)lane);
        for (uint32_t i = lane; i < a.hd; i += 64) row[i] = v[wave][i];
        __builtin_amdgcn_wave_barrier();  // the row's reads of v are done before the next row is loaded into it
    }
}

// ====================================================================================== KV write
// Reference kv_write (gpu.js:447-466): slot = pos0 + t (mod cap); f32 cache, or f16 (round to nearest even).
KERNEL __launch_bounds__(256) void qp_kv_write(QpKvArgs a) {
    const uint32_t T = paso_T(a.paso), pos0 = paso_pos(a.paso);
    const uint64_t n = (uint64_t)T * a.kvd;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull) {
        const uint32_t t = (uint32_t)(i / a.kvd), c = (uint32_t)(i % a.kvd);
        uint32_t slot = pos0 + t;
        if (a.cap) slot %= a.cap;
        if (slot >= a.rows) continue;
        const uint64_t o = (uint64_t)slot * a.kvd + c;
        if (a.f16) {
            mptr<uint16_t>(a.kc)[o] = f2h(cptr<float>(a.k)[i]);
            mptr<uint16_t>(a.vc)[vt_index(slot, a.kvd, c)] = f2h(cptr<float>(a.v)[i]);
        } else {
            mptr<float>(a.kc)[o] = cptr<float>(a.k)[i];
            mptr<float>(a.vc)[o] = cptr<float>(a.v)[i];
        }
    }
}

// The f16 cache for prompt chunks (kvd % 4 == 0): a workgroup takes 64 tokens x 64 channels.  K and V rows are read
// four channels per thread; K goes out as four f16 per thread ([slot][kvd], rows contiguous); V goes through LDS so
// that each thread writes 16 consecutive slots of one channel, which sit in that channel's 64-byte tile rows
// (vt_index).  The same values and slots as qp_kv_write.  Grid (ceil(kvd / 64), ceil(T / 64)).
KERNEL __launch_bounds__(256) void qp_kv_write16(QpKvArgs a) {
    __shared__ float vt[64][65];  // [channel][token]
    const uint32_t T = paso_T(a.paso), pos0 = paso_pos(a.paso);
    const uint32_t c0 = blockIdx.x * 64, t0 = blockIdx.y * 64, tid = threadIdx.x;
    if (t0 >= T) return;
    const uint32_t cq = tid & 15, r0 = tid >> 4;
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        const uint32_t lt = r0 + 16 * i, t = t0 + lt, c = c0 + 4 * cq;
        if (t < T && c < a.kvd) {
            const uint64_t src = 4ull * ((uint64_t)t * a.kvd + c);
            const float4 kv = gload<float4>(a.k + src), vv = gload<float4>(a.v + src);
            uint32_t slot = pos0 + t;
            if (a.cap) slot %= a.cap;
            if (slot < a.rows) {
                const uint32_t lo = (uint32_t)f2h(kv.x) | ((uint32_t)f2h(kv.y) << 16);
                const uint32_t hi = (uint32_t)f2h(kv.z) | ((uint32_t)f2h(kv.w) << 16);
                *reinterpret_cast<uint2*>(mptr<uint16_t>(a.kc) + (uint64_t)slot * a.kvd + c) = uint2{lo, hi};
            }
            vt[4 * cq][lt] = vv.x;
            vt[4 * cq + 1][lt] = vv.y;
            vt[4 * cq + 2][lt] = vv.z;
            vt[4 * cq + 3][lt] = vv.w;
        }
    }
    __syncthreads();
    const uint32_t lc = tid >> 2, lt0 = (tid & 3) * 16, c = c0 + lc;
    if (c >= a.kvd) return;
    for (uint32_t j = 0; j < 16; j++) {
        const uint32_t t = t0 + lt0 + j;
        if (t >= T) break;
        uint32_t slot = pos0 + t;
        if (a.cap) slot %= a.cap;
        if (slot >= a.rows) continue;
        mptr<uint16_t>(a.vc)[vt_index(slot, a.kvd, c)] = f2h(vt[lc][lt0 + j]);
    }
}

// ====================================================================================== SwiGLU
// Reference swiglu (gpu.js:570-582): g = g / (1 + exp(-g)) * u over T*F.
// GeGLU, the tanh form (reference geglu, gpu.js:318-330): g = 0.5 a (1 + tanh(z)) u with
// z = clamp(0.79788456 (a + 0.044715 a^3), -20, 20), evaluated in the reference's order, one rounding per operation.
KERNEL __launch_bounds__(256) void qp_geglu(QpSwigluArgs a) {
#pragma clang fp contract(off)
    const uint64_t n = (uint64_t)paso_T(a.paso) * a.f;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull) {
        const float g = cptr<float>(a.g)[i];
        const float c = ((0.044715f * g) * g) * g;
        const float z = fminf(fmaxf(0.79788456f * (g + c), -20.0f), 20.0f);
        mptr<float>(a.g)[i] = ((0.5f * g) * (1.0f + tanhf(z))) * cptr<float>(a.u)[i];
    }
}

// escalar (gpu.js:635-646): x = x * s over T rows of d; suma_esc (gpu.js:648-660): x = x + s * t.
KERNEL __launch_bounds__(256) void qp_escalar(QpScaleArgs a) {
    const uint64_t n = (uint64_t)paso_T(a.paso) * a.d;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull)
        mptr<float>(a.x)[i] = cptr<float>(a.x)[i] * a.s;
}
KERNEL __launch_bounds__(256) void qp_suma_esc(QpScaleArgs a) {
#pragma clang fp contract(off)
    const uint64_t n = (uint64_t)paso_T(a.paso) * a.d;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull)
        mptr<float>(a.x)[i] = cptr<float>(a.x)[i] + a.s * cptr<float>(a.t)[i];
}

KERNEL __launch_bounds__(256) void qp_swiglu(QpSwigluArgs a) {
    const uint64_t n = (uint64_t)paso_T(a.paso) * a.f;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull) {
        const float g = cptr<float>(a.g)[i];
        mptr<float>(a.g)[i] = (g / (1.0f + expf(-g))) * cptr<float>(a.u)[i];
    }
}

// ====================================================================================== MoE routing
// Reference moe_topk (kds.js:191-221): softmax over E router logits, k rounds of strict argmax (ties to the
// lower index), weights = probs * scale (/ max(sum, 2^-14) when norm).  One workgroup per token.
KERNEL __launch_bounds__(256) void qp_moe_topk(QpTopkArgs a) {
    __shared__ float pr[1024];
    __shared__ float rv[4];
    __shared__ uint32_t ri[4];
    __shared__ float tot_s;
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (t >= paso_T(a.paso)) return;
    const uint32_t E = a.e;
    const float* lg = cptr<float>(a.lg) + (uint64_t)t * E;
    float m = -3.0e38f;
    for (uint32_t e = tid; e < E; e += 256) { pr[e] = lg[e]; m = fmaxf(m, pr[e]); }
    m = wave_max(m);
    if (lane == 0) rv[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(rv[0], rv[1]), fmaxf(rv[2], rv[3]));
    __syncthreads();
    float s = 0.0f;
    for (uint32_t e = tid; e < E; e += 256) { const float v = expf(pr[e] - m); pr[e] = v; s += v; }
    s = wave_sum(s);
    if (lane == 0) rv[wave] = s;
    __syncthreads();
    s = (rv[0] + rv[1]) + (rv[2] + rv[3]);
    for (uint32_t e = tid; e < E; e += 256) pr[e] = pr[e] / s;
    if (tid == 0) tot_s = 0.0f;
    __syncthreads();
    for (uint32_t i = 0; i < a.k; i++) {
        float bv = -1.0f;
        uint32_t bi = 0xffffffffu;
        for (uint32_t e = tid; e < E; e += 256)
            if (pr[e] > bv) { bv = pr[e]; bi = e; }
#pragma unroll
        for (int msk = 32; msk >= 1; msk >>= 1) {
            const float ov = __shfl_xor(bv, msk, 64);
            const uint32_t oi = __shfl_xor(bi, msk, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { rv[wave] = bv; ri[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            float b = rv[0];
            uint32_t bix = ri[0];
            for (int w = 1; w < 4; w++)
                if (rv[w] > b || (rv[w] == b && ri[w] < bix)) { b = rv[w]; bix = ri[w]; }
            if (bix == 0xffffffffu) bix = 0;
            mptr<uint32_t>(a.sel)[t * a.k + i] = bix;
            mptr<float>(a.wts)[t * a.k + i] = b;
            tot_s = tot_s + b;
            pr[bix] = -2.0f;
        }
        __syncthreads();
    }
    if (tid == 0) {
        float f = a.scale;
        if (a.norm) f = f / fmaxf(tot_s, 6.103515625e-5f);
        for (uint32_t i = 0; i < a.k; i++) mptr<float>(a.wts)[t * a.k + i] = mptr<float>(a.wts)[t * a.k + i] * f;
    }
}

// Reference moe_comb (kds.js:224-240): x[t][i] += sum_s wts[t*k+s] * de[(t*k+s)*D + i].
KERNEL __launch_bounds__(256) void qp_moe_comb(QpCombArgs a) {
    const uint64_t n = (uint64_t)paso_T(a.paso) * a.d;
    if ((a.d & 3) == 0 && a.k <= 8) {
        // four consecutive outputs per thread, the k expert rows' loads issued together; per output the same sum
        // as below (acc = acc + w * de over s in order, then x + acc)
        const uint32_t d4 = a.d >> 2;
        const uint64_t n4 = n >> 2;
        for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n4; i += (uint64_t)gridDim.x * 256ull) {
            const uint32_t t = (uint32_t)(i / d4), c = (uint32_t)(i - (uint64_t)t * d4) * 4;
            float4 r[8];
            float w[8];
#pragma unroll
            for (uint32_t s = 0; s < 8; s++) {
                if (s < a.k) {
                    r[s] = gload<float4>(a.de + 4ull * (((uint64_t)t * a.k + s) * a.d + c));
                    w[s] = cptr<float>(a.wts)[t * a.k + s];
                }
            }
            float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t s = 0; s < 8; s++) {
                if (s < a.k) {
                    acc.x = acc.x + w[s] * r[s].x;
                    acc.y = acc.y + w[s] * r[s].y;
                    acc.z = acc.z + w[s] * r[s].z;
                    acc.w = acc.w + w[s] * r[s].w;
                }
            }
            float4* xo = reinterpret_cast<float4*>(mptr<float>(a.x)) + i;
            const float4 xv = *xo;
            *xo = float4{xv.x + acc.x, xv.y + acc.y, xv.z + acc.z, xv.w + acc.w};
        }
        return;
    }
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256ull) {
        const uint32_t t = (uint32_t)(i / a.d), c = (uint32_t)(i % a.d);
        float acc = 0.0f;
        for (uint32_t s = 0; s < a.k; s++)
            acc = acc + cptr<float>(a.wts)[t * a.k + s] * cptr<float>(a.de)[((uint64_t)t * a.k + s) * a.d + c];
        mptr<float>(a.x)[i] = mptr<float>(a.x)[i] + acc;
    }
}

// Reference moe_group (kds.js:491-516): the jobs i < T*n of each expert e < n_exp, in increasing i, listed at
// lst[off[e] .. off[e + 1]).  One workgroup: thread t takes the contiguous jobs [t*c, t*c + c) and counts them per
// expert in its own LDS row (16-bit counts, c <= 65535); each expert's counts become running offsets over t; the
// experts' totals are scanned into off; a second pass over the same jobs writes each at off[e] + its running
// offset.  The order within an expert is the jobs' order, the reference's.  LDS: 256 * n_exp * 2 + 2 KB.
KERNEL __launch_bounds__(256) void qp_moe_group(QpMoeGroupArgs a) {
    extern __shared__ float4 smg[];
    uint16_t* cnt = reinterpret_cast<uint16_t*>(smg);  // [256][n_exp]
    uint32_t* base = reinterpret_cast<uint32_t*>(cnt + 256 * a.n_exp + (a.n_exp & 1));  // [n_exp]
    const uint32_t tid = threadIdx.x, E = a.n_exp;
    uint64_t nj64 = (uint64_t)paso_T(a.paso) * a.n;
    const uint32_t nj = (uint32_t)(nj64 < a.nsel ? nj64 : a.nsel);
    const uint32_t c = (nj + 255) / 256, i0 = min(nj, tid * c), i1 = min(nj, i0 + c);
    uint16_t* mine = cnt + tid * E;
    for (uint32_t e = 0; e < E; e++) mine[e] = 0;
    for (uint32_t i = i0; i < i1; i++) {
        const uint32_t e = gload<uint32_t>(a.sel + 4ull * i);
        if (e < E) mine[e] = (uint16_t)(mine[e] + 1);
    }
    __syncthreads();
    if (tid < E) {
        uint32_t run = 0;
        for (uint32_t t = 0; t < 256; t++) {
            const uint32_t v = cnt[t * E + tid];
            cnt[t * E + tid] = (uint16_t)run;  // (fits: nsel < 65536)
            run += v;
        }
        base[tid] = run;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0;
        for (uint32_t e = 0; e < E; e++) {
            const uint32_t v = base[e];
            base[e] = acc;
            gstore<uint32_t>(a.off + 4ull * e, acc);
            acc += v;
        }
        gstore<uint32_t>(a.off + 4ull * E, acc);
    }
    __syncthreads();
    for (uint32_t i = i0; i < i1; i++) {
        const uint32_t e = gload<uint32_t>(a.sel + 4ull * i);
        if (e < E) {
            const uint32_t r = mine[e];
            mine[e] = (uint16_t)(r + 1);
            gstore<uint32_t>(a.lst + 4ull * (base[e] + r), i);
        }
    }
}

// ====================================================================================== attention
// Causal GQA attention over the cache for any T (reference atencion, gpu.js:467-539): a workgroup takes one
// KV head and a block of queries for all the query heads that share it; keys and values are staged in LDS
// in tiles of 32 and an online softmax runs per (head, query) row.  32 rows per workgroup.
template <int HD>
QP_DEV float kv_load(uint64_t base, uint32_t f16, uint64_t idx) {
    return f16 ? h2f(cptr<uint16_t>(base)[idx]) : cptr<float>(base)[idx];
}

template <int HD>
QP_DEV void attn_gen_body(const QpAttnArgs& a) {
    constexpr int ROWS = 32, TK = 32;
    constexpr int RPT = ROWS * HD / 256;  // P.V rows per thread
    extern __shared__ float4 smem4[];
    float* qs = reinterpret_cast<float*>(smem4);  // [ROWS][HD]
    float* ks = qs + ROWS * HD;                   // [TK][HD+1]
    float* vs = ks + TK * (HD + 1);               // [TK][HD]
    float* ps = vs + TK * HD;                     // [ROWS][TK+1]
    float* mr = ps + ROWS * (TK + 1);             // [ROWS]
    float* lr = mr + ROWS;
    float* cr = lr + ROWS;
    const uint32_t tid = threadIdx.x;
    const uint32_t T = paso_T(a.paso), pos0 = paso_pos(a.paso);
    const uint32_t G = a.nh / a.nkv, kvh = blockIdx.x;
    const uint32_t QB = ROWS / G;
    const uint32_t t0 = blockIdx.y * QB;
    if (t0 >= T) return;
    const uint32_t kvd = a.nkv * HD;
    const uint32_t nrows = G * QB;
    // rows: r = g*QB + qi
    for (uint32_t i = tid; i < ROWS * HD; i += 256) {
        const uint32_t r = i / HD, d = i % HD;
        const uint32_t g = r / QB, qi = r % QB;
        const uint32_t t = min(t0 + qi, T - 1);
        qs[i] = (r < nrows) ? cptr<float>(a.q)[((uint64_t)t * a.nh + kvh * G + g) * HD + d] : 0.0f;
    }
    if (tid < ROWS) { mr[tid] = -3.0e38f; lr[tid] = 0.0f; }
    const uint32_t tlast = min(t0 + QB, T) - 1;
    const uint32_t kend = a.cap ? pos0 + tlast + 1 : min(pos0 + tlast + 1, a.rows);
    uint32_t kbeg = 0;
    if (a.swa) {
        const uint32_t nk0 = pos0 + t0 + 1;
        kbeg = nk0 > a.swa ? nk0 - a.swa : 0;
    }
    // score roles: key j, rows rg*4..+4
    const uint32_t j = tid & 31, rg = tid >> 5;
    // P.V roles: column d, rows pv*RPT..
    const uint32_t d = tid % HD, pv = tid / HD;
    float acc[RPT];
#pragma unroll
    for (int i = 0; i < RPT; i++) acc[i] = 0.0f;
    __syncthreads();
    for (uint32_t kt = kbeg - (kbeg % TK); kt < kend; kt += TK) {
        for (uint32_t i = tid; i < TK * HD; i += 256) {
            const uint32_t jj = i / HD, dd = i % HD;
            const uint32_t key = kt + jj;
            float kv = 0.0f, vv = 0.0f;
            if (key < kend) {
                const uint32_t sl = a.cap ? key % a.cap : key;
                const uint64_t idx = (uint64_t)sl * kvd + kvh * HD + dd;
                kv = kv_load<HD>(a.kc, a.f16, idx);
                vv = kv_load<HD>(a.vc, a.f16, a.f16 ? vt_index(sl, kvd, kvh * HD + dd) : idx);
            }
            ks[jj * (HD + 1) + dd] = kv;
            vs[jj * HD + dd] = vv;
        }
        __syncthreads();
        const uint32_t key = kt + j;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t r = rg * 4 + i;
            const uint32_t qi = r % QB;
            const uint32_t t = t0 + qi;
            const uint32_t nk = pos0 + t + 1;
            uint32_t ini = 0;
            if (a.swa && nk > a.swa) ini = nk - a.swa;
            const bool valid = r < nrows && t < T && key < nk && key >= ini;
            float s = -3.0e38f;
            if (valid) {
                float dot = 0.0f;
                const float* qr = qs + r * HD;
                const float* kr = ks + j * (HD + 1);
#pragma unroll 8
                for (int q = 0; q < HD; q++) dot += qr[q] * kr[q];
                s = dot * a.scale;
            }
            const float mold = mr[r];
            const float mt = fmaxf(mold, half_max(s));
            const float p = valid ? expf(s - mt) : 0.0f;
            const float sum = half_sum(p);
            ps[r * (TK + 1) + j] = p;
            if (j == 0) {
                const float corr = expf(mold - mt);
                cr[r] = corr;
                lr[r] = lr[r] * corr + sum;
                mr[r] = mt;
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const uint32_t r = pv * RPT + i;
            float v = acc[i] * cr[r];
            const float* pr = ps + r * (TK + 1);
#pragma unroll 8
            for (int jj = 0; jj < TK; jj++) v += pr[jj] * vs[jj * HD + d];
            acc[i] = v;
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const uint32_t r = pv * RPT + i;
        const uint32_t g = r / QB, qi = r % QB, t = t0 + qi;
        if (r < nrows && t < T)
            mptr<float>(a.o)[((uint64_t)t * a.nh + kvh * G + g) * HD + d] = acc[i] / lr[r];
    }
}

KERNEL __launch_bounds__(256) void qp_attn_hd64(QpAttnArgs a) { attn_gen_body<64>(a); }
KERNEL __launch_bounds__(256) void qp_attn_hd128(QpAttnArgs a) { attn_gen_body<128>(a); }

// Split-K decode attention for one token, with the per-head q/k RMSNorm, RoPE and the KV append fused in.
// grid (nkv, nsplit); a workgroup covers a contiguous key range of one KV head for the G query heads of its
// group, split again over its 4 wavefronts.  Each wavefront streams its keys straight from HBM into registers:
// a key row is spread over LPK lanes (16 bytes each), KPI keys per load instruction, U instructions per step,
// with the next step's loads in flight while the current one is consumed.  Scores are per-lane partial dot
// products reduced over the key's lanes with DPP; every lane group keeps its own online-softmax state
// (m, l, acc over its dims), merged across groups by shuffles and across wavefronts in LDS into one partial
// per (head, workgroup), which qp_dec_attn_comb merges.  The q/k/v loads are issued first, then the first
// step's K/V loads, so the q/k preparation runs while those are in flight (vector-memory waits are in order).
template <int CTRL>
QP_DEV float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
// Sum over aligned groups of L lanes (L = 8, 16, 32 or 64); every lane of a group ends with the same bits.
template <int L>
QP_DEV float group_sum(float v) {
    if (L >= 16) v += dpp_mov<0x140>(v);  // row_mirror: lane i + lane 15-i
    v += dpp_mov<0x141>(v);               // row_half_mirror: lane i + lane 7-i
    v += dpp_mov<0x4E>(v);                // quad_perm [2,3,0,1]
    v += dpp_mov<0xB1>(v);                // quad_perm [1,0,3,2]
    if (L >= 32) v += __shfl_xor(v, 16, 64);
    if (L >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// A wavefront's head in LDS: optional RMSNorm (weight w), then RoPE at angle pos_esc * freq[j] (the frequency
// table base^(-2j/nrot) in LDS), pairs (j, j + nrot/2) when neox, else (2j, 2j + 1).
QP_DEV void wave_norm_rope_f(float* v, const float* w, uint32_t hd, bool use_norm, float eps, float pos_esc,
                             const float* freq, uint32_t nrot, bool neox, int lane) {
    if (use_norm) {
        float vals[4], ss = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = lane + 64 * c;
            vals[c] = i < hd ? v[i] : 0.0f;
            ss += vals[c] * vals[c];
        }
        ss = wave_sum_v(ss, (uint32_t)lane);  // the cross-lane steps on DPP / permlane, not through LDS
        const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = lane + 64 * c;
            if (i < hd) v[i] = (vals[c] * inv) * w[i];
        }
        __builtin_amdgcn_wave_barrier();
    }
    // one lane per rotated pair (elements p and p + nrot/2, or 2p and 2p + 1): the angle's sine and cosine once
    // per pair; each lane reads and writes only its own pair, so no barrier separates the reads from the writes
    const uint32_t mitad = nrot / 2;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const uint32_t pr = lane + 64 * c;
        if (pr < mitad) {
            const uint32_t i0 = neox ? pr : 2 * pr, i1 = neox ? pr + mitad : 2 * pr + 1;
            const float a = v[i0], b = v[i1];
            const float theta = pos_esc * freq[pr];
            float sn, cs;
            sincos2(theta, sn, cs);
            v[i0] = a * cs - b * sn;
            v[i1] = a * sn + b * cs;
        }
    }
    __builtin_amdgcn_wave_barrier();
}

// The same with the angles' sines and cosines from tables in LDS (sn[p], cs[p] for pair p: the values
// wave_norm_rope_f computes per pair, computed once for every head of a workgroup).
QP_DEV void wave_norm_rope_t(float* v, const float* w, uint32_t hd, bool use_norm, float eps, const float* snt,
                             const float* cst, uint32_t nrot, bool neox, int lane) {
    if (use_norm) {
        float vals[4], ss = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = lane + 64 * c;
            vals[c] = i < hd ? v[i] : 0.0f;
            ss += vals[c] * vals[c];
        }
        ss = wave_sum_v(ss, (uint32_t)lane);
        const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = lane + 64 * c;
            if (i < hd) v[i] = (vals[c] * inv) * w[i];
        }
        __builtin_amdgcn_wave_barrier();
    }
    const uint32_t mitad = nrot / 2;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const uint32_t pr = lane + 64 * c;
        if (pr < mitad) {
            const uint32_t i0 = neox ? pr : 2 * pr, i1 = neox ? pr + mitad : 2 * pr + 1;
            const float a = v[i0], b = v[i1], sn = snt[pr], cs = cst[pr];
            v[i0] = a * cs - b * sn;
            v[i1] = a * sn + b * cs;
        }
    }
    __builtin_amdgcn_wave_barrier();
}

template <int HD, bool F16>
struct DecCfg {
    static constexpr int E = F16 ? 8 : 4;   // cache elements per 16-byte chunk
    static constexpr int LPK = HD / E;      // lanes per key row
    static constexpr int KPI = 64 / LPK;    // keys per load instruction
    static constexpr int U = 4;             // load instructions per step
    static constexpr int KS = U * KPI;      // keys per step
};

struct DecBuf {
    uint4 k[4], v[4];
};

// Loads of KS keys from kb for this lane's key slot: through buffer resources over the cache, so a key at or past
// kend (past the wavefront's range) passes an offset past the end and costs no memory traffic.
template <int HD, bool F16>
QP_DEV void dec_load(DecBuf& b, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, uint32_t nkv, uint32_t kvh,
                     uint32_t kb, uint32_t kend, uint32_t kq, uint32_t dsub) {
    using C = DecCfg<HD, F16>;
    const uint32_t kvd = nkv * HD, eb = F16 ? 2 : 4;
#pragma unroll
    for (int u = 0; u < C::U; u++) {
        const uint32_t key = kb + u * C::KPI + kq;
        const uint32_t off = key < kend ? (key * kvd + kvh * HD) * eb + dsub * 16 : 0x80000000u;
        const u32x4 kk = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
        const u32x4 vv = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
        b.k[u] = uint4{kk[0], kk[1], kk[2], kk[3]};
        b.v[u] = uint4{vv[0], vv[1], vv[2], vv[3]};
    }
}

template <bool F16>
QP_DEV void dec_unpack(const uint4 w, float (&f)[F16 ? 8 : 4]) {
    if constexpr (F16) {
        const uint32_t x[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            f[2 * i] = h2f(x[i] & 0xffffu);
            f[2 * i + 1] = h2f(x[i] >> 16);
        }
    } else {
        f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y);
        f[2] = __uint_as_float(w.z); f[3] = __uint_as_float(w.w);
    }
}

constexpr float QP_LOG2E = 1.4426950408889634f;

// One step of KS keys starting at kb: scores for the G heads, then the online-softmax update of this lane
// group's state.  Keys at or past kend are masked; the key pos0 (this token's) comes from kn / vn.
template <int HD, bool F16, int G>
QP_DEV void dec_consume(const DecBuf& b, uint32_t kb, uint32_t kend, uint32_t pos0, const float* kn,
                        const float* vn, uint32_t kq, uint32_t dsub, const float (&qr)[G][DecCfg<HD, F16>::E],
                        float scale, float (&m)[G], float (&l)[G], float (&acc)[G][DecCfg<HD, F16>::E]) {
    using C = DecCfg<HD, F16>;
    constexpr int E = C::E;
    const bool has_new = kb <= pos0 && pos0 < kb + C::KS;  // wave-uniform
    float s[C::U][G];
#pragma unroll
    for (int u = 0; u < C::U; u++) {
        float kf[E];
        dec_unpack<F16>(b.k[u], kf);
        if (has_new && kb + u * C::KPI + kq == pos0) {
#pragma unroll
            for (int e = 0; e < E; e++) kf[e] = kn[dsub * E + e];
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < E; e++) d = fmaf(qr[g][e], kf[e], d);
            s[u][g] = group_sum<C::LPK>(d) * scale;
        }
    }
    float mn[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float mx = m[g];
#pragma unroll
        for (int u = 0; u < C::U; u++)
            if (kb + u * C::KPI + kq < kend) mx = fmaxf(mx, s[u][g]);
        const float c = __builtin_amdgcn_exp2f((m[g] - mx) * QP_LOG2E);
        l[g] *= c;
#pragma unroll
        for (int e = 0; e < E; e++) acc[g][e] *= c;
        mn[g] = mx;
        m[g] = mx;
    }
#pragma unroll
    for (int u = 0; u < C::U; u++) {
        const uint32_t key = kb + u * C::KPI + kq;
        if (key < kend) {
            float vf[E];
            dec_unpack<F16>(b.v[u], vf);
            if (has_new && key == pos0) {
#pragma unroll
                for (int e = 0; e < E; e++) vf[e] = vn[dsub * E + e];
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = __builtin_amdgcn_exp2f((s[u][g] - mn[g]) * QP_LOG2E);
                l[g] += p;
#pragma unroll
                for (int e = 0; e < E; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
            }
        }
    }
}

// The value of lane `lane ^ OFF`.  Exchanges across 16-lane rows use the gfx950 permlane swaps (plain VALU
// operations); within a row, a shuffle.  permlane16_swap(x, x) returns {x with odd rows replaced by the row below,
// x with even rows replaced by the row above}; permlane32_swap(x, x) likewise for the two halves.
template <int OFF>
QP_DEV float lane_xor(float x, uint32_t lane) {
    if constexpr (OFF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float(lane < 32 ? r[1] : r[0]);
    } else if constexpr (OFF == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float(((lane >> 4) & 1) == 0 ? r[1] : r[0]);
    } else {
        return __shfl_xor(x, OFF, 64);
    }
}

// Online-softmax states of lane groups OFF apart merged: (m, l, acc) <- the combination of both.
template <int OFF, int G, int E>
QP_DEV void dec_merge_groups(float (&m)[G], float (&l)[G], float (&acc)[G][E], uint32_t lane) {
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float mo = lane_xor<OFF>(m[g], lane), lo = lane_xor<OFF>(l[g], lane);
        const float M = fmaxf(m[g], mo);
        const float fa = __builtin_amdgcn_exp2f((m[g] - M) * QP_LOG2E);
        const float fb = __builtin_amdgcn_exp2f((mo - M) * QP_LOG2E);
        l[g] = l[g] * fa + lo * fb;
#pragma unroll
        for (int e = 0; e < E; e++) {
            const float ao = lane_xor<OFF>(acc[g][e], lane);
            acc[g][e] = acc[g][e] * fa + ao * fb;
        }
        m[g] = M;
    }
}

// ---- matrix-core key stream (f16 cache).  A wavefront takes its keys in tiles of 32 with v_mfma_f32_16x16x32_f16
// (lane l: r = l % 16, q = l / 16; an A/B operand lane holds 8 consecutive k of row/column r, k = 8q..8q+7; the
// 16x16 result lane holds rows 4q..4q+3 of column r):
//   S^T (16 keys x 16 heads) = K (16 keys x 32 dims) . Q^T, per half of the tile and 32-dim chunk, with q split in
//     f16 high and low parts (two products: near-f32 scores; the cache values are exact f16);
//   O^T (16 channels x 16 heads) += V^T (16 channels x 32 slots) . P^T, with P split likewise.  The S^T result lane
//     holds keys 4q+i and 16+4q+i of head r, exactly the slots 8q..8q+7 of the P^T operand in the V tile order.
// Heads past G are zero columns.
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

// The f16 high/low split of a lane's row of q (8 dims per 32-dim chunk, the row spread over the 4 lane groups).
// The row is first scaled by an exact power of two f that puts its largest magnitude in [2^13, 2^14), so the low
// parts stay normal f16 numbers (a subnormal low part would lose the precision the split is for); returns 1/f,
// the factor that takes the products back to the row's scale.
template <int HD>
QP_DEV float mt_split_q(const float (&v)[HD / 32][8], h8v (&qh)[HD / 32], h8v (&ql)[HD / 32], uint32_t lane) {
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < HD / 32; c++)
#pragma unroll
        for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(v[c][j]));
    mx = fmaxf(mx, bfly_f<4>(mx, lane));
    mx = fmaxf(mx, bfly_f<5>(mx, lane));
    int e = 0;
    (void)frexpf(mx, &e);  // mx = m * 2^e, m in [0.5, 1)
    const int sh = mx > 0.0f ? min(max(14 - e, -100), 100) : 0;
    const float f = ldexpf(1.0f, sh);
#pragma unroll
    for (int c = 0; c < HD / 32; c++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float x = v[c][j] * f;
            const _Float16 hi = (_Float16)x;
            qh[c][j] = hi;
            ql[c][j] = (_Float16)(x - (float)hi);
        }
    return ldexpf(1.0f, -sh);
}

// Probabilities enter P.V scaled by 2^14 (exact): their low f16 parts stay normal down to p ~ 1e-5.  The running
// sums l carry the same factor, so o = acc / l is unchanged.
constexpr float QP_PSCALE = 16384.0f;

// k[hh][c]: key t + 16 hh + r, dims 32 c + 8 q .. + 7; v[mm]: V tile row of channel 16 mm + r, slots 8q..8q+7
template <int HD>
struct MTile {
    u32x4 k[2][HD / 32];
    u32x4 v[HD / 16];
};

// Loads of the tile of keys t..t+31 (keys at or past kend load nothing and read as 0; a V tile is loaded whole
// when it holds any key below kend: its other slots are finite values of the cache, weighted by 0).
template <int HD>
QP_DEV void mt_load(MTile<HD>& b, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, uint32_t kvd, uint32_t kvh,
                    uint32_t t, uint32_t kend, uint32_t lane) {
    const uint32_t r = lane & 15, q = lane >> 4;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const uint32_t key = t + 16 * hh + r;
        const uint32_t off = key < kend ? (key * kvd + kvh * HD + 8 * q) * 2 : 0x80000000u;
#pragma unroll
        for (int c = 0; c < HD / 32; c++) b.k[hh][c] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 64 * c, 0);
    }
    const uint32_t offv = t < kend ? ((t >> 5) * kvd + kvh * HD + r) * 64 + 16 * q : 0x80000000u;
#pragma unroll
    for (int mm = 0; mm < HD / 16; mm++) b.v[mm] = __builtin_amdgcn_raw_buffer_load_b128(rv, offv, mm * 1024, 0);
}

// The online-softmax step of one tile: keys at or past kend and the new key pos0 (not in the cache yet) are
// masked.  scale: this lane's score factor (the attention scale times the 1/f of its q split).  m: running max of
// this lane's row (the same in its 4 lane groups); l: this lane's share of the sum (its 8 keys per tile), times
// QP_PSCALE; acc: O^T, channels 16 mm + 4q + i of row r, times QP_PSCALE.
template <int HD>
QP_DEV void mt_consume(const MTile<HD>& b, uint32_t t, uint32_t kend, uint32_t pos0, const h8v (&qh)[HD / 32],
                       const h8v (&ql)[HD / 32], float scale, float& m, float& l, f4v (&acc)[HD / 16],
                       uint32_t lane) {
    // no contraction: the exponent must use the same rounded score the max was taken over (an FMA of s * scale - m
    // would not, and with large scores p could exceed 1 and the scaled p the f16 range)
#pragma clang fp contract(off)
    const uint32_t q = lane >> 4;
    f4v s[2];
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        s[hh] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < HD / 32; c++) {
            const h8v kk = __builtin_bit_cast(h8v, b.k[hh][c]);
            s[hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, qh[c], s[hh], 0, 0, 0);
            s[hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, ql[c], s[hh], 0, 0, 0);
        }
    }
    float sv[8];
    bool ok[8];
    float mx = -3.0e38f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t key = t + 16 * (j >> 2) + 4 * q + (j & 3);
        ok[j] = key < kend && key != pos0;
        sv[j] = s[j >> 2][j & 3] * scale;
        if (ok[j]) mx = fmaxf(mx, sv[j]);
    }
    mx = fmaxf(mx, bfly_f<4>(mx, lane));
    mx = fmaxf(mx, bfly_f<5>(mx, lane));
    const float mn = fmaxf(m, mx);
    const float cf = __builtin_amdgcn_exp2f((m - mn) * QP_LOG2E);
    m = mn;
    float ps = 0.0f;
    h8v ph, pl;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float p = ok[j] ? __builtin_amdgcn_exp2f(fminf(sv[j] - mn, 0.0f) * QP_LOG2E) * QP_PSCALE : 0.0f;
        ps += p;
        const _Float16 hi = (_Float16)p;
        ph[j] = hi;
        pl[j] = (_Float16)(p - (float)hi);
    }
    l = l * cf + ps;
#pragma unroll
    for (int mm = 0; mm < HD / 16; mm++) {
        acc[mm] = acc[mm] * cf;
        const h8v vv = __builtin_bit_cast(h8v, b.v[mm]);
        acc[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, ph, acc[mm], 0, 0, 0);
        acc[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, pl, acc[mm], 0, 0, 0);
    }
}

// LDS (floats): kn [HD] | vn [HD] | freq [HD/2] | q-norm, k-norm weights [HD] each | region R: q [G][HD]
// during the preparation, then the wavefront partials wacc [4][G][HD], wm [4][8], wl [4][8].
template <bool COH>
QP_DEV void comb_head(uint64_t part_o, uint64_t part_ml, uint64_t out, uint32_t hd, uint32_t ns, uint32_t h, float* ws,
                      float* red, float* part);
template <int HD, bool F16, int G>
QP_DEV void attn_dec_body_(const QpDecAttnArgs& a);
template <int HD, bool F16, int G>
QP_DEV void attn_dec_body(const QpDecAttnArgs& a) {
    const uint64_t t0 = tl_now();
    tl_ph(6, 0);
    attn_dec_body_<HD, F16, G>(a);
    tl_ph(6, 6);
    tl_rec(a.tseq, t0);
}
template <int HD, bool F16, int G>
QP_DEV void attn_dec_body_(const QpDecAttnArgs& a) {
    using C = DecCfg<HD, F16>;
    constexpr int E = C::E, LPK = C::LPK, KS = C::KS;
    constexpr int QN = (G * HD + 255) / 256;  // q floats per thread
    extern __shared__ float4 smem4[];
    float* kn = reinterpret_cast<float*>(smem4);
    float* vn = kn + HD;
    float* snt = vn + HD;   // sine and cosine of this position's RoPE angles, one per rotated pair
    float* cst = snt + HD / 2;
    float* qw = cst + HD / 2;
    float* kw = qw + HD;
    float* R = kw + HD;
    float* qs = R;
    float* wacc = R;
    float* wm = R + 4 * G * HD;
    float* wl = wm + 32;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // column c: KV head c / gsplit, query heads c * G ..; the padding of a merged launch's grid (x = 8) exits
    const uint32_t gs = a.gsplit ? a.gsplit : 1u;
    const uint32_t col = blockIdx.x, kvh = col / gs, wg = blockIdx.y, h0 = col * G;
    const bool app = col % gs == 0;  // this column appends its KV head's new key and value
    if (kvh >= a.nkv) return;
    const uint32_t kq = lane / LPK, dsub = lane % LPK;
    // 1. the position first, then q, the frequency table and the q norm weight (none of them depends on it) as
    // buffer loads out of branches (past the end: 0), so the wait for the position leaves them in flight
    const uint32_t pos_w = __builtin_amdgcn_raw_buffer_load_b32(kq_rsrc(a.paso, 8), 4, 0, 0);
    float qt[QN], knt = 0.0f, vnt = 0.0f, ft, qwt, kwt = 0.0f;
    {
        const __amdgpu_buffer_rsrc_t rq = kq_rsrc(a.q + 4ull * h0 * HD, 4ull * G * HD);
#pragma unroll
        for (int c = 0; c < QN; c++) {
            const uint32_t i = tid + 256 * c;
            qt[c] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rq, i < G * HD ? 4 * i : 0x80000000u, 0, 0));
        }
        const __amdgpu_buffer_rsrc_t rf = kq_rsrc(a.freq ? a.freq : a.q, a.freq ? 4ull * (a.nrot / 2) : 0ull);
        ft = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rf, 4 * tid, 0, 0));
        const __amdgpu_buffer_rsrc_t rqn = kq_rsrc(a.qnorm ? a.qnorm : a.q, a.qnorm ? 4ull * HD : 0ull);
        qwt = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rqn, 4 * tid, 0, 0));
    }
    const uint32_t pos0 = pos_w;
    const uint32_t nk = pos0 < a.rows ? pos0 + 1 : 0;  // a position past the cache reads and writes nothing
    const uint32_t W = 4 * a.nsplit;
    // keys per wavefront (whole tiles of 32 for the matrix-core stream)
    const uint32_t per = F16 ? ((nk + W - 1) / W + 31) & ~31u : (nk + W - 1) / W;
    const uint32_t kw0 = min(nk, (wg * 4 + wave) * per), kw1 = min(nk, kw0 + per);
    const uint32_t g0 = min(nk, wg * 4 * per), g1 = min(nk, g0 + 4 * per);
    const bool wg_new = g0 <= pos0 && pos0 < g1;  // this workgroup holds the new key: it appends it
    // the new k and v (and the k norm weight) where this workgroup appends them, then the first K/V step: buffer
    // loads out of branches (elsewhere past the end: 0), so that the compiler counts them and the wait for q, k, v
    // leaves the key/value tiles in flight
    {
        const bool on = wg_new && tid < HD;
        const uint32_t o = on ? 4 * ((uint32_t)kvh * HD + tid) : 0x80000000u;
        knt = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(kq_rsrc(a.k, 4ull * a.nkv * HD), o, 0, 0));
        vnt = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(kq_rsrc(a.v, 4ull * a.nkv * HD), o, 0, 0));
        const __amdgpu_buffer_rsrc_t rkn = kq_rsrc(a.knorm ? a.knorm : a.k, a.knorm ? 4ull * HD : 0ull);
        kwt = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rkn, on ? 4 * tid : 0x80000000u, 0, 0));
    }
    // issued by every wavefront (one without keys loads nothing: its offsets are past the end), so the waits below
    // can count these loads as still in flight
    const uint32_t kvd = a.nkv * HD;
    const uint64_t cbytes = (uint64_t)a.rows * kvd * (F16 ? 2 : 4);
    const uint64_t vbytes = F16 ? (uint64_t)((a.rows + 31) / 32) * 32 * kvd * 2 : cbytes;  // whole tiles
    const __amdgpu_buffer_rsrc_t rk = kq_rsrc(a.kc, cbytes), rv = kq_rsrc(a.vc, vbytes);
    DecBuf A, B;
    MTile<HD> MA;  // one tile in flight per wavefront
    if constexpr (F16) {
        mt_load<HD>(MA, rk, rv, kvd, kvh, kw0, kw1, lane);
    } else {
        dec_load<HD, F16>(A, rk, rv, a.nkv, kvh, kw0, kw1, kq, dsub);
        dec_load<HD, F16>(B, rk, rv, a.nkv, kvh, kw0 + KS, kw1, kq, dsub);
    }
    // 2. the preparation (waits for the loads of 1 only); the angles' sines and cosines once for all the heads
    const float pos_esc = (float)pos0 * a.esc;
    if (tid < a.nrot / 2) {
        const float fr = a.freq ? ft : (float)pow((double)a.base, (double)((-2.0f * (float)tid) / (float)a.nrot));
        float sn, cs;
        sincos2(pos_esc * fr, sn, cs);
        snt[tid] = sn;
        cst[tid] = cs;
    }
#pragma unroll
    for (int c = 0; c < QN; c++) {
        const uint32_t i = tid + 256 * c;
        if (i < G * HD) qs[i] = qt[c];
    }
    if (wg_new && tid < HD) {
        kn[tid] = knt;
        vn[tid] = vnt;
    }
    if (tid < HD) {
        qw[tid] = qwt;
        kw[tid] = kwt;
    }
    __syncthreads();
    tl_ph(6, 1);  // q, k, v loaded
    for (uint32_t g = wave; g < G + (wg_new ? 1u : 0u); g += 4) {
        if (g < G)
            wave_norm_rope_t(qs + g * HD, qw, HD, a.qnorm != 0, a.eps, snt, cst, a.nrot, a.neox != 0, (int)lane);
        else
            wave_norm_rope_t(kn, kw, HD, a.knorm != 0, a.eps, snt, cst, a.nrot, a.neox != 0, (int)lane);
    }
    __syncthreads();
    if (F16 && wg_new && tid < HD) {
        // in f16 mode the new key and value are used as the cache will hold them (appended at the end: a store in
        // flight here would make the key loop wait for it)
        kn[tid] = h2f(f2h(kn[tid]));
        vn[tid] = h2f(f2h(vn[tid]));
    }
    __syncthreads();
    if constexpr (F16) {
        // q of head r = lane % 16 as the B operand (dims 32c + 8q + j), split in f16 high and low parts
        const uint32_t hr = lane & 15, qg = lane >> 4;
        h8v qh[HD / 32], ql[HD / 32];
        float qv[HD / 32][8];
#pragma unroll
        for (int c = 0; c < HD / 32; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) qv[c][j] = hr < G ? qs[hr * HD + 32 * c + 8 * qg + j] : 0.0f;
        tl_ph(6, 2);  // norm + RoPE done
        const float qsc = a.scale * mt_split_q<HD>(qv, qh, ql, lane);
        __syncthreads();  // every wavefront holds its q before region R is reused
        tl_ph(6, 3);
        float m = -3.0e38f, l = 0.0f;
        f4v acc[HD / 16];
#pragma unroll
        for (int mm = 0; mm < HD / 16; mm++) acc[mm] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t t = kw0; t < kw1; t += 32) {
            mt_consume<HD>(MA, t, kw1, pos0, qh, ql, qsc, m, l, acc, lane);
            if (t + 32 < kw1) mt_load<HD>(MA, rk, rv, kvd, kvh, t + 32, kw1, lane);
        }
        if (kw0 <= pos0 && pos0 < kw1) {
            // the new key, from kn / vn (the cache slot is written at the end)
#pragma clang fp contract(off)
            float d = 0.0f;
#pragma unroll
            for (int c = 0; c < HD / 32; c++)
#pragma unroll
                for (int j = 0; j < 8; j++) d = fmaf((float)qh[c][j] + (float)ql[c][j], kn[32 * c + 8 * qg + j], d);
            d += bfly_f<4>(d, lane);
            d += bfly_f<5>(d, lane);
            const float sn = d * qsc;
            const float mn = fmaxf(m, sn);
            const float cf = __builtin_amdgcn_exp2f((m - mn) * QP_LOG2E);
            const float p = __builtin_amdgcn_exp2f(fminf(sn - mn, 0.0f) * QP_LOG2E) * QP_PSCALE;
            m = mn;
            l = l * cf + (qg == 0 ? p : 0.0f);
#pragma unroll
            for (int mm = 0; mm < HD / 16; mm++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[mm][i] = fmaf(p, vn[16 * mm + 4 * qg + i], acc[mm][i] * cf);
        }
        tl_ph(6, 4);  // key stream done
        float lt = l + bfly_f<4>(l, lane);
        lt += bfly_f<5>(lt, lane);
        if (hr < G) {
#pragma unroll
            for (int mm = 0; mm < HD / 16; mm++)
#pragma unroll
                for (int i = 0; i < 4; i++) wacc[(wave * G + hr) * HD + 16 * mm + 4 * qg + i] = acc[mm][i];
            if (qg == 0) {
                wm[wave * 8 + hr] = m;
                wl[wave * 8 + hr] = lt;
            }
        }
    } else {
    float qr[G][E];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < E; e++) qr[g][e] = qs[g * HD + dsub * E + e];
    __syncthreads();  // every wavefront holds its q before region R is reused
    float m[G], l[G], acc[G][E];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -3.0e38f;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < E; e++) acc[g][e] = 0.0f;
    }
    // 3. the key stream: two steps in flight from the start, loads issued unconditionally (steps past the range
    // load nothing) and keys past kw1 masked
    if (kw0 < kw1) {
        const uint32_t nsteps = (kw1 - kw0 + KS - 1) / KS;
        for (uint32_t s = 0; s < nsteps; s += 2) {
            dec_consume<HD, F16, G>(A, kw0 + s * KS, kw1, pos0, kn, vn, kq, dsub, qr, a.scale, m, l, acc);
            dec_load<HD, F16>(A, rk, rv, a.nkv, kvh, kw0 + (s + 2) * KS, kw1, kq, dsub);
            dec_consume<HD, F16, G>(B, kw0 + (s + 1) * KS, kw1, pos0, kn, vn, kq, dsub, qr, a.scale, m, l, acc);
            dec_load<HD, F16>(B, rk, rv, a.nkv, kvh, kw0 + (s + 3) * KS, kw1, kq, dsub);
        }
    }
    // 4. merge the lane groups of this wavefront (groups hold different keys, the same dims)
    if constexpr (LPK <= 4) dec_merge_groups<4, G, E>(m, l, acc, lane);
    if constexpr (LPK <= 8) dec_merge_groups<8, G, E>(m, l, acc, lane);
    if constexpr (LPK <= 16) dec_merge_groups<16, G, E>(m, l, acc, lane);
    if constexpr (LPK <= 32) dec_merge_groups<32, G, E>(m, l, acc, lane);
    if (lane < LPK) {
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int e = 0; e < E; e++) wacc[(wave * G + g) * HD + lane * E + e] = acc[g][e];
            if (lane == 0) {
                wm[wave * 8 + g] = m[g];
                wl[wave * 8 + g] = l[g];
            }
        }
    }
    }
    __syncthreads();
    tl_ph(6, 5);
    // 5. this workgroup's partial per head: merge of its 4 wavefronts (those with no key have l = 0), four
    // consecutive dimensions of one head per thread
    for (uint32_t t = tid; t < G * (HD / 4); t += 256) {
        const uint32_t g = t / (HD / 4), d = (t % (HD / 4)) * 4;
        float M = -3.0e38f;
        for (int w = 0; w < 4; w++)
            if (wl[w * 8 + g] > 0.0f) M = fmaxf(M, wm[w * 8 + g]);
        float4 o = {0.0f, 0.0f, 0.0f, 0.0f};
        float L = 0.0f;
        for (int w = 0; w < 4; w++)
            if (wl[w * 8 + g] > 0.0f) {
                const float f = __builtin_amdgcn_exp2f((wm[w * 8 + g] - M) * QP_LOG2E);
                const float4 c = *reinterpret_cast<const float4*>(wacc + (w * G + g) * HD + d);
                o.x = fmaf(f, c.x, o.x);
                o.y = fmaf(f, c.y, o.y);
                o.z = fmaf(f, c.z, o.z);
                o.w = fmaf(f, c.w, o.w);
                L = fmaf(f, wl[w * 8 + g], L);
            }
        const uint64_t i = (uint64_t)(h0 + g) * a.nsplit + wg;
        gstore<float4>(a.part_o + 4 * (i * HD + d), o);
        if (d == 0) gstore<float2>(a.part_ml + 8 * i, make_float2(M, L));
    }
    if (app && wg_new && tid < HD) {
        // append the new key and value to the cache at slot pos0 (kn / vn hold them, f16-rounded in f16 mode)
        const uint64_t o = (uint64_t)pos0 * kvd + (uint64_t)kvh * HD + tid;
        if (F16) {
            gstore<uint16_t>(a.kc + 2 * o, f2h(kn[tid]));
            gstore<uint16_t>(a.vc + 2 * vt_index(pos0, kvd, kvh * HD + tid), f2h(vn[tid]));
        } else {
            gstore<float>(a.kc + 4 * o, kn[tid]);
            gstore<float>(a.vc + 4 * o, vn[tid]);
        }
    }
    if (a.att) {
        // 6. the last of the head's workgroups to finish merges its G heads (the dec_attn_comb computation).  With
        // the grid's x = 8, workgroup (x, y) has linear id x + 8y, and workgroups are handed to the 8 XCDs round
        // robin by that id: all workgroups of KV head x run on one XCD and share its L2, where the counter's atomic
        // add executes and the partial stores land once acknowledged: every wavefront waits for that (a
        // workgroup-scope release fence does not) before the barrier that precedes the add.  The merge reads them
        // past this CU's L1.  The placement is checked by the same add (xcd_arrive).
        vm_drain();
        __syncthreads();
        tl_ph(10, 0);
        __shared__ uint32_t last;
        if (tid == 0) last = xcd_arrive(a.cnt + 128ull * col, gridDim.y, a.cnt + 1024);
        __syncthreads();
        tl_ph(10, 1);
        if (last) {
            // the column's G heads at once.  Thread t takes the float4 q = t % NQ of the outputs (four dimensions
            // of one head; NQ = G HD / 4 divides 256) and share r = t / NQ of the splits (RS = 256 / NQ shares of
            // consecutive splits).  Its partials' loads are issued PB at a time (one batch up to RS PB splits),
            // the first batch before the weights are known, so the merge waits for about one round of loads; they
            // are read past this CU's L1 (sc0).  Wavefront w finds the weights e[g][s] = exp(m_s - M) (0 for a split without keys) and the
            // denominator L = sum l_s e_s of heads g = w, w + 4.  Each share sums its splits in order, and the
            // shares are added in order.
            const uint32_t ns = a.nsplit;
            constexpr uint32_t NQ = G * HD / 4, RS = 256 / NQ;
            constexpr int PB = 16;
            float* eb = R;                                             // [G][ns]
            float* lb = R + G * ns;                                    // [G]
            float4* pb = reinterpret_cast<float4*>(R + ((G * ns + 8 + 3) & ~3u));  // [RS][NQ]
            const __amdgpu_buffer_rsrc_t rml = kq_rsrc(a.part_ml, 8ull * a.nh * ns);
            const __amdgpu_buffer_rsrc_t rpo = kq_rsrc(a.part_o, 4ull * a.nh * ns * HD);
            const uint32_t q = tid % NQ, r = tid / NQ, g = q / (HD / 4), d = (q % (HD / 4)) * 4, h = h0 + g;
            const uint32_t per = (ns + RS - 1) / RS, s0 = min(ns, r * per), s1 = min(ns, s0 + per);
            u32x4 pv[PB];
            auto issue = [&](uint32_t base) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < PB; i++) {
                    const uint32_t sp = base + i;
                    pv[i] = __builtin_amdgcn_raw_buffer_load_b128(
                        rpo, sp < s1 ? 4 * ((h * ns + sp) * HD + d) : 0x80000000u, 0, 1);
                }
            };
            // the first 128 splits' (m, l) stay in registers from the maximum to the weights (one round of
            // loads); splits past 128 are read twice.  A load past ns reads l = 0 (the buffer's bound).  The first
            // head's (m, l) loads go out before the partials', which return after them.
            u32x2 v2[2];
            auto load_ml = [&](uint32_t hh) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t sp = lane + 64 * j;
                    v2[j] = __builtin_amdgcn_raw_buffer_load_b64(rml, sp < ns ? 8 * (hh * ns + sp) : 0x80000000u, 0,
                                                                 1);
                }
            };
            if (wave < (uint32_t)G) load_ml(h0 + wave);
            issue(s0);
            for (uint32_t gg = wave; gg < (uint32_t)G; gg += 4) {
                const uint32_t hh = h0 + gg;
                if (gg != wave) load_ml(hh);
                float mx = -3.0e38f;
#pragma unroll
                for (int j = 0; j < 2; j++)
                    if (__uint_as_float(v2[j].y) > 0.0f) mx = fmaxf(mx, __uint_as_float(v2[j].x));
                for (uint32_t sp = lane + 128; sp < ns; sp += 64) {
                    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rml, 8 * (hh * ns + sp), 0, 1);
                    if (__uint_as_float(v.y) > 0.0f) mx = fmaxf(mx, __uint_as_float(v.x));
                }
                mx = wave_max_v(mx, lane);  // lane exchanges, no LDS round trips
                float ls = 0.0f;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t sp = lane + 64 * j;
                    const float l = __uint_as_float(v2[j].y);
                    const float e = l > 0.0f ? expf(__uint_as_float(v2[j].x) - mx) : 0.0f;
                    if (sp < ns) eb[gg * ns + sp] = e;
                    ls += l * e;
                }
                for (uint32_t sp = lane + 128; sp < ns; sp += 64) {
                    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rml, 8 * (hh * ns + sp), 0, 1);
                    const float l = __uint_as_float(v.y);
                    const float e = l > 0.0f ? expf(__uint_as_float(v.x) - mx) : 0.0f;
                    eb[gg * ns + sp] = e;
                    ls += l * e;
                }
                ls = wave_sum_v(ls, lane);
                if (lane == 0) lb[gg] = ls;
            }
            tl_ph(10, 2);
            __syncthreads();
            tl_ph(10, 3);
            float4 o = {0.0f, 0.0f, 0.0f, 0.0f};
            for (uint32_t base = s0; base < s1; base += PB) {
                if (base != s0) issue(base);
#pragma unroll
                for (int i = 0; i < PB; i++) {
                    const uint32_t sp = base + i;
                    if (sp < s1) {
                        const float e = eb[g * ns + sp];
                        o.x = fmaf(e, __uint_as_float(pv[i][0]), o.x);
                        o.y = fmaf(e, __uint_as_float(pv[i][1]), o.y);
                        o.z = fmaf(e, __uint_as_float(pv[i][2]), o.z);
                        o.w = fmaf(e, __uint_as_float(pv[i][3]), o.w);
                    }
                }
            }
            pb[r * NQ + q] = o;
            tl_ph(10, 4);
            __syncthreads();
            tl_ph(10, 5);
            for (uint32_t t = tid; t < NQ; t += 256) {
                float4 sum = pb[t];
                for (uint32_t rr = 1; rr < RS; rr++) {
                    const float4 v = pb[rr * NQ + t];
                    sum.x += v.x;
                    sum.y += v.y;
                    sum.z += v.z;
                    sum.w += v.w;
                }
                const uint32_t tg = t / (HD / 4), td = (t % (HD / 4)) * 4, th = h0 + tg;
                const float L = lb[tg];
                const float4 res =
                    L > 0.0f ? make_float4(sum.x / L, sum.y / L, sum.z / L, sum.w / L) : make_float4(0, 0, 0, 0);
                gstore<float4>(a.att + 4ull * (th * HD + td), res);  // no key: zeros
            }
        }
    }
}

// (two workgroups per CU: at most 256 registers per lane)
#define DEC_ATTN_KERNEL(HD, KV, F16, G)                                                                          \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void qp_dec_attn_h##HD##_##KV##_g##G( \
        QpDecAttnArgs a) { attn_dec_body<HD, F16, G>(a); }
#define DEC_ATTN_KERNELS(HD, KV, F16) \
    DEC_ATTN_KERNEL(HD, KV, F16, 1) DEC_ATTN_KERNEL(HD, KV, F16, 2) DEC_ATTN_KERNEL(HD, KV, F16, 4) DEC_ATTN_KERNEL(HD, KV, F16, 8)
DEC_ATTN_KERNELS(64, f16, true)
DEC_ATTN_KERNELS(64, f32, false)
DEC_ATTN_KERNELS(128, f16, true)
DEC_ATTN_KERNELS(128, f32, false)

// ------------------------------------------------------------------------ attention block of one decode token
// dec_attn_block (QpDecBlockArgs documents the three phases).  Head group c = blockIdx.x runs on one XCD: the
// workgroups of a launch are handed to the 8 XCDs round robin by linear id x + 8y, so the ns workgroups of column c
// share one L2.  The group's barrier counter lives there (its adds and polls are atomics, executed in the L2), and
// the stores a workgroup makes before a barrier are there once acknowledged; after the barrier they are read past
// the CU's L1 (sc0 loads).  A group found on more than one XCD sets err (checked by the host), so the assumption
// cannot fail silently.

// Barrier of the ns workgroups of a group (ns a power of two).  Every barrier adds ns to the counter, so arrival
// number n belongs to the barrier that completes when the counter reaches (n rounded down to ns) + ns, compared
// modulo 2^32.  The polls are atomic adds of a zero the compiler cannot see (it would turn an add of a known 0
// into a plain load, which may be served by a cache level the increments do not update): they execute where the
// increments do.  Past spin_max polls the wait sets err bit 0 and stops, so every workgroup always ends.
QP_DEV void group_barrier(uint64_t cnt, uint32_t ns, uint32_t spin_max, uint64_t err) {
    vm_drain();
    __syncthreads();
    if (threadIdx.x == 0) {
        QP_GLOBAL uint32_t* c = reinterpret_cast<QP_GLOBAL uint32_t*>(cnt);
        const uint32_t n = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const uint32_t target = (n & ~(ns - 1)) + ns;
        uint32_t zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
        for (uint32_t it = 0;; it++) {
            const uint32_t v = __hip_atomic_fetch_add(c, zero, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if ((int32_t)(v - target) >= 0) break;
            if (it >= spin_max) {
                __hip_atomic_fetch_or(reinterpret_cast<QP_GLOBAL uint32_t*>(err), 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
}

template <int FQ, int HD, int GP>
QP_DEV void dec_block_body_(const QpDecBlockArgs& a);
template <int FQ, int HD, int GP>
QP_DEV void dec_block_body(const QpDecBlockArgs& a) {
    const uint64_t t0 = tl_now();
    dec_block_body_<FQ, HD, GP>(a);
    tl_rec(a.tseq, t0);
}
template <int FQ, int HD, int GP>
QP_DEV void dec_block_body_(const QpDecBlockArgs& a) {
    extern __shared__ float4 smem4[];
    tl_ph(7, 0);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t c = blockIdx.x, y = blockIdx.y, ns = a.ns;
    const uint32_t r8 = 8 / a.nkv, kvh = c / r8, h0 = c * GP;
    const bool app = c % r8 == 0;  // this group appends its KV head's new key and value
    const uint64_t cnt = a.cnt + 256ull * c;
    // the XCD of this workgroup; workgroup (c, 0) stores its XCD + 1 before the first barrier, and the others compare
    // after it (the XCD a group lands on can change from launch to launch, the sharing within a launch cannot)
    const uint32_t xid = (__builtin_amdgcn_s_getreg(20 | (15 << 11)) & 15u) + 1u;  // HW_REG_XCC_ID
    if (tid == 0 && y == 0) gstore<uint32_t>(a.xcc + 4ull * c, xid);
    const uint32_t pos0 = paso_pos(a.paso);
    const uint32_t nk = pos0 < a.rows ? pos0 + 1 : 0;  // a position past the cache reads and writes nothing
    // keys in whole tiles of 32: wavefront i of the group's W = 4 ns takes tiles [i nt / W, (i + 1) nt / W)
    const uint32_t W = 4 * ns, nt = (nk + 31) / 32, wi = 4 * y + wave;
    const uint32_t kw0 = min(nk, 32 * (wi * nt / W)), kw1 = min(nk, 32 * ((wi + 1) * nt / W));
    const uint32_t g0 = min(nk, 32 * (4 * y * nt / W)), g1 = min(nk, 32 * ((4 * y + 4) * nt / W));
    const bool wg_new = g0 <= pos0 && pos0 < g1;  // this workgroup's keys hold the new one
    const uint32_t kvd = a.nkv * HD;
    const uint64_t cbytes = (uint64_t)a.rows * kvd * 2;
    const uint64_t vbytes = (uint64_t)((a.rows + 31) / 32) * 32 * kvd * 2;  // whole tiles
    const __amdgpu_buffer_rsrc_t rk = kq_rsrc(a.kc, cbytes), rv = kq_rsrc(a.vc, vbytes);

    // 1. the group's q rows and its KV head's k and v rows; each wavefront's first key/value tile loads meanwhile
    MTile<HD> MA;
    {
        uint32_t nbp = 1;
        while (nbp < (a.dm >> 8)) nbp <<= 1;
        const uint32_t S = 64 / nbp, nq = GP * HD, uq = (nq + S - 1) / S, uk = (HD + S - 1) / S;
        // segments q, k, v (field by field: selects, not a table in private memory)
        auto seg_at = [&](uint32_t i) __attribute__((always_inline)) {
            const bool s1 = i >= 1, s2 = i >= 2;
            KSeg sg;
            sg.w = s2 ? a.wv : s1 ? a.wk : a.wq;
            sg.w2 = sg.w;
            sg.y = s2 ? a.v + 4ull * kvh * HD : s1 ? a.k + 4ull * kvh * HD : a.q + 4ull * h0 * HD;
            sg.n = s1 ? HD : nq;
            sg.row_base = s1 ? kvh * HD : h0 * HD;
            sg.rows_total = s1 ? kvd : a.nh * HD;
            sg.mode = QP_GEMV_STORE;
            sg.u0 = (s1 ? uq : 0u) + (s2 ? uk : 0u);
            sg.fmt = s2 ? a.fv : s1 ? a.fk : a.fq;
            return sg;
        };
        auto pro = [&]() __attribute__((always_inline)) { mt_load<HD>(MA, rk, rv, kvd, kvh, kw0, kw1, lane); };
        kq_gemv<FQ, 1, 1, decltype(seg_at), KDense, decltype(pro), 256, true, HD / 8>(
            seg_at, 3, uq + 2 * uk, a.x, a.norm_w, a.eps, a.dm, 0, KDense(), pro, y, ns);
    }
    tl_ph(7, 1);
    group_barrier(cnt, ns, a.spin_max, a.err);
    tl_ph(7, 2);
    // (read past the L1, which has never held the line in this launch: the L1 is invalidated at each launch)
    const uint32_t xseen = tid == 0 ? ld_sc0(kq_rsrc(a.xcc, 32), 4 * c) : xid;

    // 2. attention of the group's GP query heads over keys [kw0, kw1) of this wavefront.  LDS (floats): kn [HD] |
    // vn [HD] | RoPE sines, cosines [HD/2] each | q/k norm weights [HD] each | region R: q [GP][HD], then the
    // wavefront partials wacc [4][GP][HD], wm [4][8], wl [4][8]
    constexpr int QN = (GP * HD + 255) / 256;
    float* kn = reinterpret_cast<float*>(smem4);
    float* vn = kn + HD;
    float* snt = vn + HD;
    float* cst = snt + HD / 2;
    float* qw = cst + HD / 2;
    float* kw = qw + HD;
    float* R = kw + HD;
    float* qs = R;
    float* wacc = R;
    float* wm = R + 4 * GP * HD;
    float* wl = wm + 32;
    const __amdgpu_buffer_rsrc_t rq = kq_rsrc(a.q, 4ull * a.nh * HD);
    const __amdgpu_buffer_rsrc_t rkn = kq_rsrc(a.k, 4ull * kvd), rvn = kq_rsrc(a.v, 4ull * kvd);
    float qt[QN], knt = 0.0f, vnt = 0.0f, ft = 0.0f, qwt = 0.0f, kwt = 0.0f;
#pragma unroll
    for (int j = 0; j < QN; j++) {
        const uint32_t i = tid + 256 * j;
        qt[j] = i < GP * HD ? __uint_as_float(ld_sc0(rq, 4 * (h0 * HD + i))) : 0.0f;
    }
    if (wg_new && tid < HD) {
        knt = __uint_as_float(ld_sc0(rkn, 4 * (kvh * HD + tid)));
        vnt = __uint_as_float(ld_sc0(rvn, 4 * (kvh * HD + tid)));
    }
    if (a.freq && tid < a.nrot / 2) ft = gload<float>(a.freq + 4ull * tid);
    if (a.qnorm && tid < HD) qwt = gload<float>(a.qnorm + 4ull * tid);
    if (a.knorm && wg_new && tid < HD) kwt = gload<float>(a.knorm + 4ull * tid);
    const float pos_esc = (float)pos0 * a.esc;
    if (tid < a.nrot / 2) {
        const float fr = a.freq ? ft : (float)pow((double)a.base, (double)((-2.0f * (float)tid) / (float)a.nrot));
        float sn, cs;
        sincos2(pos_esc * fr, sn, cs);
        snt[tid] = sn;
        cst[tid] = cs;
    }
#pragma unroll
    for (int j = 0; j < QN; j++) {
        const uint32_t i = tid + 256 * j;
        if (i < GP * HD) qs[i] = qt[j];
    }
    if (wg_new && tid < HD) {
        kn[tid] = knt;
        vn[tid] = vnt;
    }
    if (tid < HD) {
        qw[tid] = qwt;
        kw[tid] = kwt;
    }
    __syncthreads();
    for (uint32_t g = wave; g < GP + (wg_new ? 1u : 0u); g += 4) {
        if (g < GP)
            wave_norm_rope_t(qs + g * HD, qw, HD, a.qnorm != 0, a.eps, snt, cst, a.nrot, a.neox != 0, (int)lane);
        else
            wave_norm_rope_t(kn, kw, HD, a.knorm != 0, a.eps, snt, cst, a.nrot, a.neox != 0, (int)lane);
    }
    __syncthreads();
    if (wg_new && tid < HD) {
        // the new key and value as the f16 cache will hold them
        kn[tid] = h2f(f2h(kn[tid]));
        vn[tid] = h2f(f2h(vn[tid]));
    }
    __syncthreads();
    {
        const uint32_t hr = lane & 15, qg = lane >> 4;
        h8v qh[HD / 32], ql[HD / 32];
        float qv[HD / 32][8];
#pragma unroll
        for (int j = 0; j < HD / 32; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) qv[j][e] = hr < GP ? qs[hr * HD + 32 * j + 8 * qg + e] : 0.0f;
        const float qsc = a.scale * mt_split_q<HD>(qv, qh, ql, lane);
        __syncthreads();  // every wavefront holds its q before region R is reused
        tl_ph(7, 3);
        float m = -3.0e38f, l = 0.0f;
        f4v acc[HD / 16];
#pragma unroll
        for (int mm = 0; mm < HD / 16; mm++) acc[mm] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t t = kw0; t < kw1; t += 32) {
            mt_consume<HD>(MA, t, kw1, pos0, qh, ql, qsc, m, l, acc, lane);
            if (t + 32 < kw1) mt_load<HD>(MA, rk, rv, kvd, kvh, t + 32, kw1, lane);
        }
        if (kw0 <= pos0 && pos0 < kw1) {
            // the new key, from kn / vn (the cache slot is written at the end)
#pragma clang fp contract(off)
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < HD / 32; j++)
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf((float)qh[j][e] + (float)ql[j][e], kn[32 * j + 8 * qg + e], d);
            d += bfly_f<4>(d, lane);
            d += bfly_f<5>(d, lane);
            const float sn = d * qsc;
            const float mn = fmaxf(m, sn);
            const float cf = __builtin_amdgcn_exp2f((m - mn) * QP_LOG2E);
            const float p = __builtin_amdgcn_exp2f(fminf(sn - mn, 0.0f) * QP_LOG2E) * QP_PSCALE;
            m = mn;
            l = l * cf + (qg == 0 ? p : 0.0f);
#pragma unroll
            for (int mm = 0; mm < HD / 16; mm++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[mm][i] = fmaf(p, vn[16 * mm + 4 * qg + i], acc[mm][i] * cf);
        }
        float lt = l + bfly_f<4>(l, lane);
        lt += bfly_f<5>(lt, lane);
        if (hr < GP) {
#pragma unroll
            for (int mm = 0; mm < HD / 16; mm++)
#pragma unroll
                for (int i = 0; i < 4; i++) wacc[(wave * GP + hr) * HD + 16 * mm + 4 * qg + i] = acc[mm][i];
            if (qg == 0) {
                wm[wave * 8 + hr] = m;
                wl[wave * 8 + hr] = lt;
            }
        }
    }
    __syncthreads();
    // this workgroup's partial per head: merge of its 4 wavefronts, four dimensions per thread
    for (uint32_t t = tid; t < GP * (HD / 4); t += 256) {
        const uint32_t g = t / (HD / 4), d = (t % (HD / 4)) * 4;
        float M = -3.0e38f;
        for (int w = 0; w < 4; w++)
            if (wl[w * 8 + g] > 0.0f) M = fmaxf(M, wm[w * 8 + g]);
        float4 o = {0.0f, 0.0f, 0.0f, 0.0f};
        float L = 0.0f;
        for (int w = 0; w < 4; w++)
            if (wl[w * 8 + g] > 0.0f) {
                const float f = __builtin_amdgcn_exp2f((wm[w * 8 + g] - M) * QP_LOG2E);
                const float4 cc = *reinterpret_cast<const float4*>(wacc + (w * GP + g) * HD + d);
                o.x = fmaf(f, cc.x, o.x);
                o.y = fmaf(f, cc.y, o.y);
                o.z = fmaf(f, cc.z, o.z);
                o.w = fmaf(f, cc.w, o.w);
                L = fmaf(f, wl[w * 8 + g], L);
            }
        const uint64_t i = (uint64_t)(h0 + g) * ns + y;
        gstore<float4>(a.part_o + 4 * (i * HD + d), o);
        if (d == 0) gstore<float2>(a.part_ml + 8 * i, make_float2(M, L));
    }
    if (app && wg_new && tid < HD) {
        // append the new key and value at slot pos0 (f16-rounded in kn / vn)
        const uint64_t o = (uint64_t)pos0 * kvd + (uint64_t)kvh * HD + tid;
        gstore<uint16_t>(a.kc + 2 * o, f2h(kn[tid]));
        gstore<uint16_t>(a.vc + 2 * vt_index(pos0, kvd, kvh * HD + tid), f2h(vn[tid]));
    }
    tl_ph(7, 4);
    group_barrier(cnt, ns, a.spin_max, a.err);
    tl_ph(7, 5);

    // 3. the split merge (log-sum-exp weights; a split without keys has l = 0 and weight 0; no key at all gives 0):
    // workgroup y writes outputs [y cs, (y + 1) cs) of the group's GP * HD (the host keeps ns <= GP * HD).  The
    // partials of those outputs are loaded with the (m, l) pairs, one (split, output) pair per thread, so the merge
    // waits for one round of loads; the products go through LDS and are summed in split order.
    {
        const uint32_t cs = GP * HD / ns;
        float* eb = R;                       // [GP][ns] weights
        float* lb = R + GP * ns;             // [GP] denominators
        float* pb = R + GP * ns + 8;         // [ns][cs] weighted partials
        const __amdgpu_buffer_rsrc_t rml = kq_rsrc(a.part_ml, 8ull * a.nh * ns);
        const __amdgpu_buffer_rsrc_t rpo = kq_rsrc(a.part_o, 4ull * a.nh * ns * HD);
        constexpr uint32_t NPV = (GP * HD + 255) / 256;  // (split, output) pairs per thread
        float pv[NPV];
#pragma unroll
        for (uint32_t j = 0; j < NPV; j++) {
            const uint32_t t = tid + 256 * j, sp = t / cs, i = y * cs + t % cs;
            pv[j] = t < GP * HD ? __uint_as_float(ld_sc0(rpo, 4 * (((h0 + i / HD) * ns + sp) * HD + i % HD))) : 0.0f;
        }
        for (uint32_t g = wave; g < (uint32_t)GP; g += 4) {
            const uint32_t h = h0 + g;
            float mv = -3.0e38f, lv = 0.0f;
            if (lane < ns) {
                const u32x2 r = __builtin_amdgcn_raw_buffer_load_b64(rml, 8 * (h * ns + lane), 0, 1);
                mv = __uint_as_float(r.x);
                lv = __uint_as_float(r.y);
            }
            const float mx = wave_max(lv > 0.0f ? mv : -3.0e38f);
            const float e = lv > 0.0f ? expf(mv - mx) : 0.0f;
            if (lane < ns) eb[g * ns + lane] = e;
            const float ls = wave_sum(lv * e);
            if (lane == 0) lb[g] = ls;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t j = 0; j < NPV; j++) {
            const uint32_t t = tid + 256 * j, sp = t / cs, i = y * cs + t % cs;
            if (t < GP * HD) pb[t] = eb[(i / HD) * ns + sp] * pv[j];
        }
        __syncthreads();
        for (uint32_t t = tid; t < cs; t += 256) {
            const uint32_t i = y * cs + t, g = i / HD, h = h0 + g;
            float o = 0.0f;
            for (uint32_t sp = 0; sp < ns; sp++) o += pb[sp * cs + t];
            const float L = lb[g];
            gstore<float>(a.att + 4ull * (h * HD + i % HD), L > 0.0f ? o / L : 0.0f);
        }
    }
    tl_ph(7, 6);
    if (tid == 0 && xseen != xid)
        __hip_atomic_fetch_or(reinterpret_cast<QP_GLOBAL uint32_t*>(a.err), 2u, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
}

#define DEC_BLOCK_KERNEL(NAME, FQ, HD, GP)                                                                        \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void qp_dec_block_##NAME##_h##HD##_g##GP( \
        QpDecBlockArgs a) { dec_block_body<FQ, HD, GP>(a); }
DEC_BLOCK_KERNEL(q4k, QP_Q4_K, 128, 1)
DEC_BLOCK_KERNEL(q4k, QP_Q4_K, 128, 2)
DEC_BLOCK_KERNEL(q4k, QP_Q4_K, 128, 4)
DEC_BLOCK_KERNEL(mix, QP_KQ_MIX, 128, 1)
DEC_BLOCK_KERNEL(mix, QP_KQ_MIX, 128, 2)
DEC_BLOCK_KERNEL(mix, QP_KQ_MIX, 128, 4)
DEC_BLOCK_KERNEL(q4k, QP_Q4_K, 64, 1)
DEC_BLOCK_KERNEL(q4k, QP_Q4_K, 64, 4)
DEC_BLOCK_KERNEL(mix, QP_KQ_MIX, 64, 1)
DEC_BLOCK_KERNEL(mix, QP_KQ_MIX, 64, 4)

// Causal attention of a prefill chunk on the matrix cores (f16 cache; no sliding window, no ring cap), the
// reference atencion (gpu.js:467-539).  A wavefront takes RG groups of 16 rows: TPW = 16 RG / G tokens x the G heads
// of KV head kvh (row r of group g: token t0 + (16 g + r) / G, head r % G), and streams keys in tiles of 32 with the
// decode tile step, each row masked at its own causal limit pos0 + its token.
// RG = 1: wavefront w of workgroup (kvh, y) takes token block 4y + w and all its keys, two tiles in flight.
// RG = 2: every tile loaded feeds both row groups (half the key and value loads per row; one tile in flight, for
// the registers of the second group's query and accumulators).  Workgroup (kvh, y) takes one token block (the
// longest first: y counts from the last block), its key tiles dealt to the four wavefronts in four ranges, and the
// wavefronts' partial softmax states merged in LDS (weights e^(m_w - M), in wavefront order).  A token block's
// serial chain of tiles is then a quarter of its keys: the longest rows of a prompt chunk no longer set the launch's
// time alone (2048 tokens: 64 tiles in one wavefront before).
template <int HD, int G, int RG>
QP_DEV void attn_mfma_body(const QpAttnArgs& a) {
    constexpr uint32_t TPW = 16 * RG / G;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t T = paso_T(a.paso), pos0 = paso_pos(a.paso);
    const uint32_t kvh = blockIdx.x;
    const uint32_t blk = RG == 2 ? gridDim.y - 1 - blockIdx.y : blockIdx.y * 4 + wave;
    const uint32_t t0 = blk * TPW;
    if (t0 >= T) return;  // RG = 1: the wavefront; RG = 2: the whole workgroup (t0 is the same in its wavefronts)
    const uint32_t kvd = a.nkv * HD, r = lane & 15, qg = lane >> 4;
    const uint32_t tlast = min(t0 + TPW, T) - 1;
    const uint32_t kend = min(pos0 + tlast + 1, a.rows);  // keys the token block reads
    // this wavefront's keys [kb, ke): RG = 2, a quarter of the block's tiles (whole tiles, so the ranges do not meet
    // inside a tile); RG = 1, all of them
    uint32_t kb = 0, ke = kend;
    if constexpr (RG == 2) {
        const uint32_t q = ((kend + 31) / 32 + 3) / 4 * 32;
        kb = min(kend, wave * q);
        ke = min(kend, kb + q);
    }
    const __amdgpu_buffer_rsrc_t rk = kq_rsrc(a.kc, (uint64_t)a.rows * kvd * 2);
    const __amdgpu_buffer_rsrc_t rv = kq_rsrc(a.vc, (uint64_t)((a.rows + 31) / 32) * 32 * kvd * 2);
    MTile<HD> A, B;
    mt_load<HD>(A, rk, rv, kvd, kvh, kb, ke, lane);
    if constexpr (RG == 1) mt_load<HD>(B, rk, rv, kvd, kvh, 32, kend, lane);
    h8v qh[RG][HD / 32], ql[RG][HD / 32];
    float qsc[RG], m[RG], l[RG];
    uint32_t tr[RG], hr[RG], kend_row[RG], kend_grp[RG];
    bool row_ok[RG];
    f4v acc[RG][HD / 16];
#pragma unroll
    for (int g = 0; g < RG; g++) {
        tr[g] = t0 + (16 * g + r) / G;  // this lane's row in group g
        hr[g] = kvh * G + r % G;
        row_ok[g] = tr[g] < T;
        kend_row[g] = row_ok[g] ? min(pos0 + tr[g] + 1, a.rows) : 0u;  // keys this row attends to
        // keys the group's last row attends to (uniform: a group past T reads none)
        const uint32_t tg = t0 + (16 * g + 15) / G;
        kend_grp[g] = t0 + (16 * g) / G < T ? min(pos0 + min(tg, T - 1) + 1, a.rows) : 0u;
        float qv[HD / 32][8];
        const uint64_t qrow = a.q + 4ull * (((uint64_t)(row_ok[g] ? tr[g] : 0) * a.nh + hr[g]) * HD);
#pragma unroll
        for (int c = 0; c < HD / 32; c++) {
            const float4 x0 = gload<float4>(qrow + 4 * (32 * c + 8 * qg));
            const float4 x1 = gload<float4>(qrow + 4 * (32 * c + 8 * qg + 4));
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int jj = 0; jj < 8; jj++) qv[c][jj] = row_ok[g] ? xv[jj] : 0.0f;
        }
        qsc[g] = a.scale * mt_split_q<HD>(qv, qh[g], ql[g], lane);
        m[g] = -3.0e38f;
        l[g] = 0.0f;
#pragma unroll
        for (int mm = 0; mm < HD / 16; mm++) acc[g][mm] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if constexpr (RG == 1) {
        for (uint32_t t = 0; t < kend; t += 64) {
            mt_consume<HD>(A, t, kend_row[0], 0xffffffffu, qh[0], ql[0], qsc[0], m[0], l[0], acc[0], lane);
            mt_load<HD>(A, rk, rv, kvd, kvh, t + 64, kend, lane);
            if (t + 32 < kend)
                mt_consume<HD>(B, t + 32, kend_row[0], 0xffffffffu, qh[0], ql[0], qsc[0], m[0], l[0], acc[0], lane);
            mt_load<HD>(B, rk, rv, kvd, kvh, t + 96, kend, lane);
        }
    } else {
        for (uint32_t t = kb; t < ke; t += 32) {
#pragma unroll
            for (int g = 0; g < RG; g++)
                if (t < kend_grp[g])  // a group whose rows all stop before this tile skips it
                    mt_consume<HD>(A, t, kend_row[g], 0xffffffffu, qh[g], ql[g], qsc[g], m[g], l[g], acc[g], lane);
            mt_load<HD>(A, rk, rv, kvd, kvh, t + 32, ke, lane);
        }
        // the merge: each wavefront's row maxima, row sums (the lane groups' shares added) and O^T values to LDS;
        // wavefront w then finishes dimensions 16 mm + 4 qg + i of both groups for mm = 2 w, 2 w + 1
        __shared__ float pm[4][RG][64], pl[4][RG][64];
        __shared__ f4v pa[4][RG][HD / 16][64];
#pragma unroll
        for (int g = 0; g < RG; g++) {
            float lt = l[g] + bfly_f<4>(l[g], lane);
            lt += bfly_f<5>(lt, lane);
            pm[wave][g][lane] = m[g];
            pl[wave][g][lane] = lt;
#pragma unroll
            for (int mm = 0; mm < HD / 16; mm++) pa[wave][g][mm][lane] = acc[g][mm];
        }
        __syncthreads();
        constexpr int MW = HD / 64;  // dimensions blocks of 16 per wavefront
#pragma unroll
        for (int g = 0; g < RG; g++) {
            float M = -3.0e38f;
#pragma unroll
            for (int w = 0; w < 4; w++) M = fmaxf(M, pm[w][g][lane]);
            float f[4], L = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                f[w] = __builtin_amdgcn_exp2f((pm[w][g][lane] - M) * QP_LOG2E);
                L = fmaf(f[w], pl[w][g][lane], L);
            }
            const uint64_t orow = a.o + 4ull * (((uint64_t)tr[g] * a.nh + hr[g]) * HD);
#pragma unroll
            for (int j = 0; j < MW; j++) {
                const int mm = (int)wave * MW + j;
                f4v o = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int w = 0; w < 4; w++) o = o + pa[w][g][mm][lane] * f[w];
                float4 v;
                v.x = L > 0.0f ? o[0] / L : 0.0f;
                v.y = L > 0.0f ? o[1] / L : 0.0f;
                v.z = L > 0.0f ? o[2] / L : 0.0f;
                v.w = L > 0.0f ? o[3] / L : 0.0f;
                if (!a.orows) {
                    if (row_ok[g]) gstore<float4>(orow + 4 * (16 * mm + 4 * qg), v);
                    continue;
                }
                // as the next matmul's input planes: lanes qg and qg + 1 (lane ^ 16, the same row) hold the two
                // halves of eight consecutive outputs; the even one splits them with qp_split_bf16's formula
                const float p0 = bfly_f<4>(v.x, lane), p1 = bfly_f<4>(v.y, lane), p2 = bfly_f<4>(v.z, lane),
                            p3 = bfly_f<4>(v.w, lane);
                if (row_ok[g] && !(qg & 1)) {
                    const float e[8] = {v.x, v.y, v.z, v.w, p0, p1, p2, p3};
                    const uint32_t K = a.nh * HD, k = hr[g] * HD + 16 * mm + 4 * qg;
                    const uint64_t off = xs_off(tr[g], k, a.orows), plane = 2ull * a.orows * K;
                    split_store8(e, reinterpret_cast<__bf16*>(a.o + off), reinterpret_cast<__bf16*>(a.o + plane + off));
                }
            }
        }
        return;
    }
#pragma unroll
    for (int g = 0; g < RG; g++) {
        float lt = l[g] + bfly_f<4>(l[g], lane);
        lt += bfly_f<5>(lt, lane);
        if (row_ok[g]) {
            const uint64_t orow = a.o + 4ull * (((uint64_t)tr[g] * a.nh + hr[g]) * HD);
#pragma unroll
            for (int mm = 0; mm < HD / 16; mm++) {
                float4 v;
                v.x = lt > 0.0f ? acc[g][mm][0] / lt : 0.0f;
                v.y = lt > 0.0f ? acc[g][mm][1] / lt : 0.0f;
                v.z = lt > 0.0f ? acc[g][mm][2] / lt : 0.0f;
                v.w = lt > 0.0f ? acc[g][mm][3] / lt : 0.0f;
                gstore<float4>(orow + 4 * (16 * mm + 4 * qg), v);
            }
        }
    }
}

#define ATTN_MFMA_KERNEL(HD, G)                                                                                   \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void qp_attn_mfma_h##HD##_g##G(        \
        QpAttnArgs a) { attn_mfma_body<HD, G, 1>(a); }                                                            \
    KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void qp_attn_mfma2_h##HD##_g##G(       \
        QpAttnArgs a) { attn_mfma_body<HD, G, 2>(a); }
ATTN_MFMA_KERNEL(64, 1) ATTN_MFMA_KERNEL(64, 2) ATTN_MFMA_KERNEL(64, 4) ATTN_MFMA_KERNEL(64, 8)
ATTN_MFMA_KERNEL(128, 1) ATTN_MFMA_KERNEL(128, 2) ATTN_MFMA_KERNEL(128, 4) ATTN_MFMA_KERNEL(128, 8)

// Merge of the split partials: o = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), splits with l = 0 skipped
// (all of them empty, for a position past the cache: o = 0).
// grid nh; every load of the first batch of splits (up to 16 per thread) and of the (m, l) pairs is issued
// before any of them is used, so the kernel waits for one memory round trip.
// Merge of one head's split partials (log-sum-exp weights; empty splits skipped; no keys gives zeros), by a whole
// workgroup of 256 threads: ws [1024], red [4] and part [256] in LDS.  COH: read the partials past the CU's L1 (they
// were written by other workgroups of the same launch).
template <bool COH>
QP_DEV void comb_head(uint64_t part_o, uint64_t part_ml, uint64_t out, uint32_t hd, uint32_t ns, uint32_t h, float* ws,
                      float* red, float* part) {
    constexpr int CB = 16;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t P = 256 / hd, d = tid % hd, pt = tid / hd;
    const uint64_t ml = part_ml + 8ull * h * ns;
    const uint64_t po = part_o + 4ull * h * ns * hd;
    const __amdgpu_buffer_rsrc_t rml = kq_rsrc(ml, 8ull * ns), rpo = kq_rsrc(po, 4ull * ns * hd);
    auto ldo = [&](uint32_t sp) __attribute__((always_inline)) {
        const uint32_t off = 4 * (sp * hd + d);
        return COH ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rpo, off, 0, 1)) : gload<float>(po + off);
    };
    float pv[CB];
#pragma unroll
    for (int i = 0; i < CB; i++) {
        const uint32_t sp = pt + P * i;
        pv[i] = pt < P && sp < ns ? ldo(sp) : 0.0f;
    }
    float2 mv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t sp = tid + 256 * i;
        if (sp < ns) {
            if (COH) {
                const u32x2 r = __builtin_amdgcn_raw_buffer_load_b64(rml, 8 * sp, 0, 1);
                mv[i] = make_float2(__uint_as_float(r.x), __uint_as_float(r.y));
            } else {
                mv[i] = gload<float2>(ml + 8ull * sp);
            }
        } else {
            mv[i] = make_float2(-3.0e38f, 0.0f);
        }
    }
    float mx = -3.0e38f;
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (mv[i].y > 0.0f) mx = fmaxf(mx, mv[i].x);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float ls = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t sp = tid + 256 * i;
        const float e = mv[i].y > 0.0f ? expf(mv[i].x - M) : 0.0f;
        if (sp < ns) ws[sp] = e;
        ls += mv[i].y * e;
    }
    ls = wave_sum(ls);
    if (lane == 0) red[wave] = ls;
    __syncthreads();
    const float L = (red[0] + red[1]) + (red[2] + red[3]);
    float o = 0.0f;
    if (pt < P) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const uint32_t sp = pt + P * i;
            if (sp < ns) o = fmaf(ws[sp], pv[i], o);
        }
        for (uint32_t sp = pt + P * CB; sp < ns; sp += P)  // more than CB splits per thread: the rest in turn
            o = fmaf(ws[sp], ldo(sp), o);
    }
    part[tid] = o;
    __syncthreads();
    if (tid < hd) {
        float t = 0.0f;
        for (uint32_t i = 0; i < P; i++) t += part[i * hd + tid];
        gstore<float>(out + 4ull * ((uint64_t)h * hd + tid), L > 0.0f ? t / L : 0.0f);  // no key: zeros
    }
    __syncthreads();  // ws, red and part may be reused by the caller
}

QP_DEV void qp_dec_attn_comb_impl(QpDecCombArgs a);
KERNEL __launch_bounds__(256) void qp_dec_attn_comb(QpDecCombArgs a) {
    const uint64_t t0 = tl_now();
    qp_dec_attn_comb_impl(a);
    tl_rec(a.tseq, t0);
}
QP_DEV void qp_dec_attn_comb_impl(QpDecCombArgs a) {
    __shared__ float ws[1024];
    __shared__ float red[4];
    __shared__ float part[256];
    comb_head<false>(a.part_o, a.part_ml, a.o, a.hd, a.nsplit, blockIdx.x, ws, red, part);
}

// ====================================================================================== argmax
// Greedy (reference sampling.js:38-42): strict '>' from -Infinity, so ties go to the lowest index and NaN is
// never chosen.  Single workgroup.
KERNEL __launch_bounds__(1024) void qp_argmax(QpArgmaxArgs a) {
    __shared__ uint64_t wb[16];
    const uint32_t tid = threadIdx.x;
    uint64_t best = 0;
    for (uint32_t i = tid; i < a.n; i += 1024) {
        const uint64_t k = amax_key(cptr<float>(a.v)[i], i);
        best = k > best ? k : best;
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = __shfl_xor(best, m, 64);
        best = o > best ? o : best;
    }
    if ((tid & 63) == 0) wb[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t b = 0;
        for (int i = 0; i < 16; i++) b = wb[i] > b ? wb[i] : b;
        mptr<uint32_t>(a.out)[0] = b ? 0xffffffffu - (uint32_t)(b & 0xffffffffu) : 0u;
    }
}

// Finish of the fused output GEMV's partial maxima: ids[0] = token, tokens[step] = token, step++, pos0 += T.
QP_DEV void qp_argmax_fin_impl(QpArgmaxFinArgs a);
KERNEL __launch_bounds__(256) void qp_argmax_fin(QpArgmaxFinArgs a) {
    const uint64_t t0 = tl_now();
    qp_argmax_fin_impl(a);
    tl_rec(a.tseq, t0);
}
QP_DEV void qp_argmax_fin_impl(QpArgmaxFinArgs a) {
    __shared__ uint64_t wb[4];
    const uint32_t tid = threadIdx.x;
    uint64_t best = 0;
    for (uint32_t i = tid; i < a.count; i += 256) {
        const uint64_t k = cptr<uint64_t>(a.amax)[i];
        best = k > best ? k : best;
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = __shfl_xor(best, m, 64);
        best = o > best ? o : best;
    }
    if ((tid & 63) == 0) wb[tid >> 6] = best;
    __syncthreads();
    // the partials are cleared once read, so a later launch with fewer producing workgroups sees no stale entry
    for (uint32_t i = tid; i < a.count; i += 256) mptr<uint64_t>(a.amax)[i] = 0ull;
    if (tid == 0) {
        uint64_t b = wb[0];
        for (int i = 1; i < 4; i++) b = wb[i] > b ? wb[i] : b;
        const uint32_t tok = b ? 0xffffffffu - (uint32_t)(b & 0xffffffffu) : 0u;
        mptr<uint32_t>(a.ids)[0] = tok;
        uint32_t* st = mptr<uint32_t>(a.step);
        if (a.tokens && st[0] < a.cap) mptr<uint32_t>(a.tokens)[st[0]] = tok;
        st[0] = st[0] + 1;
        if (a.advance) {
            uint32_t* p = mptr<uint32_t>(a.paso);
            p[1] = p[1] + p[0];
        }
    }
}

// ====================================================================================== sampling
// The reference samples on the host (web/js/sampling.js:25-82) from the whole logits array.  These kernels apply
// the penalties and select the top-k candidates on the device, so the host reads back k (value, id) pairs and
// draws from them with the reference's float64 steps.

// sampling.js:30-36 for the window's (token, count) pairs: in double like the JavaScript (no contraction), stored
// rounded to float as a Float32Array store rounds.
KERNEL __launch_bounds__(64) void qp_penalizar(QpPenaltyArgs a) {
#pragma clang fp contract(off)
    const uint32_t i = threadIdx.x;
    if (i >= a.count) return;
    const uint32_t t = cptr<uint32_t>(a.hist)[2 * i], n = cptr<uint32_t>(a.hist)[2 * i + 1];
    if (t >= a.n) return;
    float* lg = mptr<float>(a.logits);
    double l = (double)lg[t];
    if (a.rep != 1.0) l = l > 0 ? l / a.rep : l * a.rep;
    l -= (double)n * a.freq + a.pres;
    lg[t] = (float)l;
}

// Order-preserving key of (logit, id): a larger key is a larger value, then a lower id.
QP_DEV uint64_t topk_key(float v, uint32_t i) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (0xffffffffu - i);
}
QP_DEV float topk_val(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
QP_DEV uint32_t topk_id(uint64_t k) { return 0xffffffffu - (uint32_t)k; }

// Descending bitonic sort of n (a power of two) keys in LDS by nt threads.
QP_DEV void bitonic_desc(uint64_t* s, uint32_t n, uint32_t tid, uint32_t nt) {
    for (uint32_t size = 2; size <= n; size <<= 1)
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = tid; t < n / 2; t += nt) {
                const uint32_t i = 2 * t - (t & (stride - 1)), j = i + stride;
                const uint64_t x = s[i], y = s[j];
                if ((i & size) == 0 ? x < y : x > y) {
                    s[i] = y;
                    s[j] = x;
                }
            }
            __syncthreads();
        }
}

// Stage 1: workgroup g sorts logits [2048 g, 2048 g + 2048) and keeps its kp = k + 1 largest keys, plus a NaN
// flag.  part: kp keys per workgroup, then one u32 flag per workgroup.
KERNEL __launch_bounds__(256) void qp_topk_part(QpCandArgs a) {
    __shared__ uint64_t s[2048];
    const uint32_t tid = threadIdx.x, base = blockIdx.x * 2048;
    const float* lg = cptr<float>(a.logits);
    int nan = 0;
    for (uint32_t i = tid; i < 2048; i += 256) {
        const uint32_t g = base + i;
        uint64_t key = 0;  // padding sorts below every non-NaN value
        if (g < a.n) {
            const float v = lg[g];
            nan |= v != v;
            key = topk_key(v, g);
        }
        s[i] = key;
    }
    nan = __syncthreads_or(nan);
    bitonic_desc(s, 2048, tid, 256);
    uint64_t* part = mptr<uint64_t>(a.part);
    for (uint32_t i = tid; i < a.kp; i += 256) part[(uint64_t)blockIdx.x * a.kp + i] = s[i];
    if (tid == 0) reinterpret_cast<uint32_t*>(part + (uint64_t)a.g * a.kp)[blockIdx.x] = nan ? 1u : 0u;
}

// Stage 2 (one workgroup): merges the g*kp partial keys (n2 = next power of two, in dynamic LDS) and writes
// out = {flags, k, (value bits, id) x k} in descending order.  flags bit 0: a NaN logit; bit 1: two equal values
// among the k + 1 largest (float equality, so -0 == +0), i.e. the candidate set or its order would depend on the
// reference's heap; the host then takes the whole logits array.
KERNEL __launch_bounds__(1024) void qp_topk_merge(QpCandArgs a) {
    extern __shared__ float4 smk[];
    uint64_t* s = reinterpret_cast<uint64_t*>(smk);
    const uint32_t tid = threadIdx.x, tot = a.g * a.kp;
    const uint64_t* part = cptr<uint64_t>(a.part);
    const uint32_t* pf = reinterpret_cast<const uint32_t*>(part + tot);
    for (uint32_t i = tid; i < a.n2; i += 1024) s[i] = i < tot ? part[i] : 0ull;
    int nan = 0;
    for (uint32_t i = tid; i < a.g; i += 1024) nan |= pf[i] != 0;
    nan = __syncthreads_or(nan);
    bitonic_desc(s, a.n2, tid, 1024);
    const int tie = __syncthreads_or(tid < a.k && topk_val(s[tid]) == topk_val(s[tid + 1]));
    uint32_t* out = mptr<uint32_t>(a.out);
    if (tid == 0) {
        out[0] = (nan ? 1u : 0u) | (tie ? 2u : 0u);
        out[1] = a.k;
    }
    if (tid < a.k) {
        out[2 + 2 * tid] = __float_as_uint(topk_val(s[tid]));
        out[3 + 2 * tid] = topk_id(s[tid]);
    }
}

// ====================================================================================== calibration
// Plain streaming kernels of known traffic: copy n float4s (reads and writes 16n bytes each) and a read-only
// sum of n float4s (one float written per thread).  Used to calibrate HBM traffic counters and bandwidth.
KERNEL __launch_bounds__(256) void qp_copy_f4(QpRepackArgs a) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < a.nblocks; i += (uint64_t)gridDim.x * 256ull)
        gstore<float4>(a.dst + 16 * i, gload<float4>(a.src + 16 * i));
}

KERNEL __launch_bounds__(256) void qp_read_f4(QpRepackArgs a) {
    float s = 0.0f;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < a.nblocks; i += (uint64_t)gridDim.x * 256ull) {
        const float4 v = gload<float4>(a.src + 16 * i);
        s += (v.x + v.y) + (v.z + v.w);
    }
    gstore<float>(a.dst + 4 * (blockIdx.x * 256ull + threadIdx.x), s);
}
