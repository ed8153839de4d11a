// Device helpers shared by the gfx950 kernels (64-lane wavefronts).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../qp_args.h"

#define QP_DEV __device__ __forceinline__

QP_DEV float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
QP_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

template <class T>
QP_DEV const T* cptr(uint64_t a) { return reinterpret_cast<const T*>(a); }
template <class T>
QP_DEV T* mptr(uint64_t a) { return reinterpret_cast<T*>(a); }

// Loads through a global-address-space pointer.  Addresses that reach a kernel inside an argument block are
// generic to the compiler, which would otherwise emit flat loads; a flat load counts against both the vector-
// memory and the LDS wait counters, so every LDS read would also wait for all in-flight weight loads.
#define QP_GLOBAL __attribute__((address_space(1)))
// (The integer address is converted straight to a global pointer: a cast from a generic pointer stays flat.)
template <class T>
QP_DEV T gload(uint64_t addr) {
    return *(const QP_GLOBAL T*)addr;
}
template <class T>
QP_DEV void gstore(uint64_t addr, T v) {
    *(QP_GLOBAL T*)addr = v;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A buffer resource over `bytes` bytes from base (raw, no stride).  A load whose offset lies past them returns 0 and
// moves no data: kernels pass QP_NOOFF for a lane or row without work, so that every path issues the same loads.
QP_DEV __amdgpu_buffer_rsrc_t kq_rsrc(uint64_t base, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}
constexpr uint32_t QP_NOOFF = 0x80000000u;

QP_DEV float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
QP_DEV float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
// reductions over aligned groups of 32 lanes (half a wavefront)
QP_DEV float half_sum(float v) {
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
QP_DEV float half_max(float v) {
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Value of the partner lane in step S of a wavefront butterfly made of VALU lane exchanges (no LDS traffic):
// S = 0: lane ^ 1, 1: lane ^ 2 (quad permutes), 2: mirror within 8 lanes, 3: mirror within 16 lanes (DPP),
// 4: the other row of a row pair, 5: the other half (gfx950 permlane swaps).  A commutative, associative
// reduction through the six steps leaves every lane with the reduction of all 64, bit-identical in every lane.
template <int S>
QP_DEV uint32_t bfly(uint32_t v, uint32_t lane) {
    if constexpr (S == 0) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false);
    else if constexpr (S == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false);
    else if constexpr (S == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false);
    else if constexpr (S == 3) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false);
    else if constexpr (S == 4) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return ((lane >> 4) & 1) == 0 ? r[1] : r[0];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return lane < 32 ? r[1] : r[0];
    }
}
template <int S>
QP_DEV float bfly_f(float v, uint32_t lane) { return __uint_as_float(bfly<S>(__float_as_uint(v), lane)); }

QP_DEV float wave_max_v(float v, uint32_t lane) {
    v = fmaxf(v, bfly_f<0>(v, lane));
    v = fmaxf(v, bfly_f<1>(v, lane));
    v = fmaxf(v, bfly_f<2>(v, lane));
    v = fmaxf(v, bfly_f<3>(v, lane));
    v = fmaxf(v, bfly_f<4>(v, lane));
    return fmaxf(v, bfly_f<5>(v, lane));
}
QP_DEV float wave_sum_v(float v, uint32_t lane) {
    v += bfly_f<0>(v, lane);
    v += bfly_f<1>(v, lane);
    v += bfly_f<2>(v, lane);
    v += bfly_f<3>(v, lane);
    v += bfly_f<4>(v, lane);
    return v + bfly_f<5>(v, lane);
}

// This wavefront's vector-memory operations complete: loads returned, stores acknowledged by the L2 (what another
// CU of the XCD reads after a barrier needs; a workgroup-scope release fence does not wait for it).
QP_DEV void vm_drain() { __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xf << 8)); }

// Paso in device memory: {T, pos0, a, b}
QP_DEV uint32_t paso_T(uint64_t p) { return cptr<uint32_t>(p)[0]; }
QP_DEV uint32_t paso_pos(uint64_t p) { return cptr<uint32_t>(p)[1]; }

// ------------------------------------------------------------------ timeline (profiling builds only)
// Built with -DQP_TIMELINE, each workgroup of a launch captured in a graph (tseq > 0, set by the host) records its
// start and end (s_memrealtime, 100 MHz), hardware id and XCC into slot (tseq - 1) * QP_TL_SLOTS + workgroup, and
// thread 0 of the GEMV and decode-attention workgroups stamps its phase boundaries (per kernel kind; the last
// launch of a kind keeps its stamps).  The host reads both arrays back when it frees the graph.  Without
// QP_TIMELINE these compile to nothing.
#ifdef QP_TIMELINE
#define QP_TL_SLOTS 4096
#define QP_TL_MAXSEQ 420
__device__ uint4 qp_tl[QP_TL_MAXSEQ * QP_TL_SLOTS];
__device__ uint32_t qp_tl_ph[16 * QP_TL_SLOTS * 8];
QP_DEV uint64_t tl_now() { return __builtin_amdgcn_s_memrealtime(); }
QP_DEV void tl_rec(uint32_t tseq, uint64_t t0) {
    if (tseq == 0 || tseq > QP_TL_MAXSEQ || threadIdx.x != 0) return;
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    const uint32_t wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    if (wg >= QP_TL_SLOTS) return;
    const uint32_t hw = __builtin_amdgcn_s_getreg(4 | (31 << 11));     // HW_REG_HW_ID, 32 bits
    const uint32_t xcc = __builtin_amdgcn_s_getreg(20 | (15 << 11));   // HW_REG_XCC_ID
    qp_tl[(uint64_t)(tseq - 1) * QP_TL_SLOTS + wg] = make_uint4((uint32_t)t0, (uint32_t)t1, hw, xcc | 0x80000000u);
}
QP_DEV void tl_ph(uint32_t kind, uint32_t i) {
    if (threadIdx.x != 0) return;
    const uint32_t wg = blockIdx.x + gridDim.x * blockIdx.y;
    if (wg < QP_TL_SLOTS) qp_tl_ph[(kind * QP_TL_SLOTS + wg) * 8 + i] = (uint32_t)__builtin_amdgcn_s_memrealtime();
}
#else
QP_DEV uint64_t tl_now() { return 0; }
QP_DEV void tl_rec(uint32_t, uint64_t) {}
QP_DEV void tl_ph(uint32_t, uint32_t) {}
#endif

// ------------------------------------------------------------------ scalar dequant (bit-exact formulas)
// These follow the reference's element formulas (kquants.js:166-175, gpu.js:601-603) with every product and
// difference rounded separately; fp-contract is switched off inside them.
QP_DEV void q4k_scmin_bytes(const uint8_t* s, uint32_t j, uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = s[j] & 63u;
        mn = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

// Q4_K and Q6_K device layout (written by the repack ops at load time).  Row r of a tensor with nb = K/256
// blocks per row occupies nb*RB bytes starting at r*nb*RB (RB = 144 for Q4_K, 208 for Q6_K).  Inside a row the
// blocks are stored as 16-byte chunk planes: chunk c (bytes 16c..16c+15 of the GGUF block) of block b sits at
// c*nb*16 + b*16.  A wavefront lane that owns block b of a row therefore loads its chunk c with one 16-byte
// load, and the lanes owning consecutive blocks read one contiguous run per plane.  Q6_K keeps its 13 chunks
// (ql 0..7, qh 8..11, scales 12) in the row; the f16 d of every block goes to a plane [rows][nb] after all rows.
template <int RB>
QP_DEV uint8_t kq_byte(const uint8_t* base, uint32_t nb, uint64_t row, uint32_t b, uint32_t i) {
    return base[row * nb * RB + (i >> 4) * nb * 16 + b * 16 + (i & 15)];
}

QP_DEV float deq_q4k_dev(const uint8_t* base, uint32_t nb, uint64_t row, uint32_t b, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t j = e >> 5, l = e & 31;
    uint8_t s[12];
    for (int i = 0; i < 12; i++) s[i] = kq_byte<144>(base, nb, row, b, 4 + i);
    uint32_t sc, mn;
    q4k_scmin_bytes(s, j, sc, mn);
    const float d = h2f(kq_byte<144>(base, nb, row, b, 0) | (kq_byte<144>(base, nb, row, b, 1) << 8));
    const float dmin = h2f(kq_byte<144>(base, nb, row, b, 2) | (kq_byte<144>(base, nb, row, b, 3) << 8));
    const float fd = d * (float)sc;
    const float fm = dmin * (float)mn;
    const uint32_t q = (kq_byte<144>(base, nb, row, b, 16 + (j >> 1) * 32 + l) >> ((j & 1) * 4)) & 15u;
    const float a = fd * (float)q;
    return a - fm;
}

// NB = blocks of the whole tensor (rows * nb): the d plane starts at NB*208.
QP_DEV float deq_q6k_dev(const uint8_t* base, uint32_t nb, uint64_t NB, uint64_t row, uint32_t b, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t s = e >> 4, h = e >> 7, r = e & 127, qd = r >> 5, l = r & 31;
    const uint32_t lo = (kq_byte<208>(base, nb, row, b, h * 64 + (qd & 1) * 32 + l) >> ((qd >> 1) * 4)) & 15u;
    const uint32_t hi = (kq_byte<208>(base, nb, row, b, 128 + h * 32 + l) >> (qd * 2)) & 3u;
    const int8_t sc = (int8_t)kq_byte<208>(base, nb, row, b, 192 + s);
    const uint8_t* dp = base + NB * 208 + (row * nb + b) * 2;
    const float d = h2f(dp[0] | (dp[1] << 8));
    const float fd = d * (float)sc;
    const float q = (float)(lo | (hi << 4)) - 32.0f;
    return fd * q;
}

QP_DEV float deq_q8_planar(const uint8_t* base, uint64_t NB, uint64_t gb, uint32_t e) {
#pragma clang fp contract(off)
    const int8_t q = reinterpret_cast<const int8_t*>(base)[gb * 32 + e];
    const uint8_t* dp = base + NB * 32 + gb * 2;
    return (float)q * h2f(dp[0] | (dp[1] << 8));
}

// IQ4_NL (ggml type 20, reference kds.js:36-39): weight = d * table[nibble] with the non-linear 16-entry int8 table
// {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113}, held here in four dwords (entry 4j + i
// in byte i of dword j).  iq4nl_lut4 looks up the four nibbles held one per byte of idx (each 0..15) and returns the
// four table bytes with three byte permutes: entries 0..7 for every byte (a nibble of 8 or more selects a constant,
// unused), entries 8..15 for every byte (by nibble ^ 8), then per byte the first or the second by bit 3.
QP_DEV uint32_t iq4nl_lut4(uint32_t idx) {
    constexpr uint32_t T0 = 0xbfad9881u, T1 = 0xf6eaddcfu, T2 = 0x26190d01u, T3 = 0x71594535u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, idx);
    const uint32_t hi = __builtin_amdgcn_perm(T3, T2, idx ^ 0x08080808u);
    return __builtin_amdgcn_perm(hi, lo, 0x03020100u | ((idx >> 1) & 0x04040404u));
}
QP_DEV float deq_iq4nl_planar(const uint8_t* base, uint64_t NB, uint64_t gb, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t byte = base[gb * 16 + (e & 15)];
    const int8_t q = (int8_t)(iq4nl_lut4(e < 16 ? byte & 15u : byte >> 4) & 0xffu);
    const uint8_t* dp = base + NB * 16 + gb * 2;
    return h2f(dp[0] | (dp[1] << 8)) * (float)q;
}

// Q5_K (reference kquants.js:8, deq at 151-153): the Q4_K header and sub-block scales, qh[32] at bytes 16..47 and
// qs[128] at 48..175; q = nibble (low for even sub-blocks, high for odd) + 16 * bit j of qh[l].
QP_DEV float deq_q5k_dev(const uint8_t* base, uint32_t nb, uint64_t row, uint32_t b, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t j = e >> 5, l = e & 31;
    uint8_t s[12];
    for (int i = 0; i < 12; i++) s[i] = kq_byte<176>(base, nb, row, b, 4 + i);
    uint32_t sc, mn;
    q4k_scmin_bytes(s, j, sc, mn);
    const float d = h2f(kq_byte<176>(base, nb, row, b, 0) | (kq_byte<176>(base, nb, row, b, 1) << 8));
    const float dmin = h2f(kq_byte<176>(base, nb, row, b, 2) | (kq_byte<176>(base, nb, row, b, 3) << 8));
    const float fd = d * (float)sc;
    const float fm = dmin * (float)mn;
    const uint32_t lo = (kq_byte<176>(base, nb, row, b, 48 + (j >> 1) * 32 + l) >> ((j & 1) * 4)) & 15u;
    const uint32_t hi = (kq_byte<176>(base, nb, row, b, 16 + l) >> j) & 1u;
    const float a = fd * (float)(lo + 16 * hi);
    return a - fm;
}

// Q3_K (reference kquants.js:10, scq3 at 78-90, deq at 159-162), padded to 112 bytes (7 chunks): hmask[32] at
// 0..31, qs[64] at 32..95, 12 scale bytes at 96..107, d f16 at 108.  Element e = 128 n + 32 jj + l of scale group
// s = e / 16: (d * (s6 - 32)) * (q2 - 4 * (1 - bit (4n + jj) of hmask[l])), q2 = (qs[32 n + l] >> 2 jj) & 3.
QP_DEV uint32_t q3k_scale6(uint32_t a0, uint32_t a1, uint32_t tmp, uint32_t s) {
    const uint32_t k1 = 0x03030303u, k2 = 0x0f0f0f0fu, g = s >> 2;
    const uint32_t wd = g == 0 ? (a0 & k2) | ((tmp & k1) << 4)
                      : g == 1 ? (a1 & k2) | (((tmp >> 2) & k1) << 4)
                      : g == 2 ? ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4)
                               : ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4);
    return (wd >> ((s & 3) * 8)) & 0xffu;
}
QP_DEV float deq_q3k_dev(const uint8_t* base, uint32_t nb, uint64_t row, uint32_t b, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t s = e >> 4, n = e >> 7, r = e & 127, jj = r >> 5, l = r & 31;
    uint32_t w[3];
    for (int i = 0; i < 3; i++)
        w[i] = kq_byte<112>(base, nb, row, b, 96 + 4 * i) | (kq_byte<112>(base, nb, row, b, 97 + 4 * i) << 8) |
               (kq_byte<112>(base, nb, row, b, 98 + 4 * i) << 16) | (kq_byte<112>(base, nb, row, b, 99 + 4 * i) << 24);
    const float d = h2f(kq_byte<112>(base, nb, row, b, 108) | (kq_byte<112>(base, nb, row, b, 109) << 8));
    const float fd = d * ((float)q3k_scale6(w[0], w[1], w[2], s) - 32.0f);
    const uint32_t q2 = (kq_byte<112>(base, nb, row, b, 32 + n * 32 + l) >> (jj * 2)) & 3u;
    const uint32_t hm = (kq_byte<112>(base, nb, row, b, l) >> (n * 4 + jj)) & 1u;
    return fd * ((float)q2 - 4.0f * (float)(1u - hm));
}

// Q2_K (reference kquants.js:11, setup at 108-116): 16 scale bytes (low nibble scale, high nibble min) at 0..15,
// qs[64] at 16..79 in 5 chunks per block; d and dmin (f16 each) in an array of 4 bytes per block after the rows.
// Element e = 128 n + 32 jj + l of group j = e / 16: (d * (sc_j & 15)) * q - dmin * (sc_j >> 4),
// q = (qs[32 n + l] >> 2 jj) & 3.
QP_DEV float deq_q2k_dev(const uint8_t* base, uint32_t nb, uint64_t NB, uint64_t row, uint32_t b, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t j = e >> 4, n = e >> 7, jj = (e & 127) >> 5, l = e & 31;
    const uint32_t sc = kq_byte<80>(base, nb, row, b, j);
    const uint8_t* dp = base + NB * 80 + (row * nb + b) * 4;
    const float d = h2f(dp[0] | (dp[1] << 8)), dmin = h2f(dp[2] | (dp[3] << 8));
    const float fd = d * (float)(sc & 15u), fm = dmin * (float)(sc >> 4);
    const uint32_t q = (kq_byte<80>(base, nb, row, b, 16 + n * 32 + l) >> (jj * 2)) & 3u;
    const float a = fd * (float)q;
    return a - fm;
}

// Element k of row `row` of a K-wide matrix in device layout fmt (NB = total blocks of the tensor).
QP_DEV float deq_elem(uint32_t fmt, const uint8_t* base, uint64_t NB, uint64_t row, uint32_t K, uint32_t k) {
    if (fmt == QP_Q4_K) return deq_q4k_dev(base, K >> 8, row, k >> 8, k & 255);
    if (fmt == QP_Q5_K) return deq_q5k_dev(base, K >> 8, row, k >> 8, k & 255);
    if (fmt == QP_Q3_K) return deq_q3k_dev(base, K >> 8, row, k >> 8, k & 255);
    if (fmt == QP_Q2_K) return deq_q2k_dev(base, K >> 8, NB, row, k >> 8, k & 255);
    if (fmt == QP_Q6_K) return deq_q6k_dev(base, K >> 8, NB, row, k >> 8, k & 255);
    if (fmt == QP_Q8_0) return deq_q8_planar(base, NB, row * (K >> 5) + (k >> 5), k & 31);
    if (fmt == QP_IQ4_NL) return deq_iq4nl_planar(base, NB, row * (K >> 5) + (k >> 5), k & 31);
    return reinterpret_cast<const float*>(base)[row * K + k];
}

QP_DEV uint64_t total_blocks(uint32_t fmt, uint64_t nrows, uint32_t K) {
    if (fmt == QP_Q2_K || fmt == QP_Q3_K || fmt == QP_Q4_K || fmt == QP_Q5_K || fmt == QP_Q6_K) return nrows * (K >> 8);
    if (fmt == QP_Q8_0 || fmt == QP_IQ4_NL) return nrows * (K >> 5);
    return nrows * K;
}

// ------------------------------------------------------------------ f16 V cache layout
// The f16 value cache is stored in tiles of 32 slots: for each of the kvd channels c of a tile, the 32 slots' values
// sit in one 64-byte row, in the order the matrix-core P.V step of the decode attention consumes them.  Slot k of
// a tile goes to position 8 * ((k % 16) / 4) + 4 * (k / 16) + k % 4 of the row, so the row's 16-byte quarter q holds
// slots 4q..4q+3 and 16+4q..16+4q+3.  Channel c of slot s: element ((s / 32) * kvd + c) * 32 + vt_pos(s % 32).
// (The f32 cache keeps the reference's row layout [slot][kvd].)
QP_DEV uint32_t vt_pos(uint32_t k) { return 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3); }
QP_DEV uint64_t vt_index(uint64_t slot, uint32_t kvd, uint32_t c) {
    return ((slot >> 5) * kvd + c) * 32 + vt_pos((uint32_t)(slot & 31));
}

// ------------------------------------------------------------------ sin/cos (reference gpu.js:13-25)
// Cody-Waite reduction by pi/2 in three parts and the Cephes single-precision minimax polynomials.
QP_DEV void sincos2(float x, float& sn_out, float& cs_out) {
#pragma clang fp contract(off)
    const float kx = x * 0.6366197723675814f;
    const int k = (int)__builtin_rintf(kx);
    const float kf = (float)k;
    const float r = ((x - kf * 1.5703125f) - kf * 4.837512969970703125e-4f) - kf * 7.549789948768648e-8f;
    const float r2 = r * r;
    const float sn = r + (r * r2) * (-1.6666654611e-1f + r2 * (8.3321608736e-3f + r2 * -1.9515295891e-4f));
    const float cs = (1.0f - 0.5f * r2) +
                     (r2 * r2) * (4.166664568298827e-2f + r2 * (-1.388731625493765e-3f + r2 * 2.443315711809948e-5f));
    const uint32_t q = (uint32_t)k & 3u;
    if (q == 0) { sn_out = sn; cs_out = cs; }
    else if (q == 1) { sn_out = cs; cs_out = -sn; }
    else if (q == 2) { sn_out = -sn; cs_out = -cs; }
    else { sn_out = -cs; cs_out = sn; }
}

