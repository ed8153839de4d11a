/*
 * qp_oracle.c -- CPU restatement of quipullm's token-loop arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (quipullm_amd/) may call, link or load this
 * code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker.
 *
 * Every function restates one WGSL kernel (or JS routine) of the reference engine, in the same f32
 * operation order where the WGSL fixes it (lane-strided partial sums, fixed reduction trees, serial
 * loops).  Citations are path:line into the reference tree (dagoalguez/quipullm).  Compile with
 * -ffp-contract=off so that no multiply-add is fused: the reference's dequant formula is defined as the
 * non-fused f32 sequence.
 *
 * Raw weight blocks are the GGUF/ggml layouts (Q2_K 84 B, Q3_K 110 B, Q4_K 144 B, Q5_K 176 B, Q6_K 210 B,
 * Q8_0 34 B), unpadded.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_F32 0
#define OR_Q8_0 8
#define OR_Q2_K 10
#define OR_Q3_K 11
#define OR_Q4_K 12
#define OR_Q5_K 13
#define OR_Q6_K 14
#define OR_IQ4_NL 20
#define OR_F16 1   /* matrices widened to f32 at upload */
#define OR_BF16 30

/* ------------------------------------------------------------------ f16 -> f32 (exact)
 * web/js/gpu.js:939-948 (F16 table); unpack2x16float in kquants.js:67 is the same map. */
float or_f16(uint16_t h) {
    int s = (h >> 15) & 1, e = (h >> 10) & 31, f = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)f, -24);
    else if (e == 31) v = f ? NAN : INFINITY;
    else v = ldexpf((float)(f | 1024), e - 25);
    return s ? -v : v;
}

/* f32 -> f16, IEEE 754 round to nearest, ties to even (overflow to infinity, NaN kept quiet).  Used for the
 * f16 KV-cache option of this backend (the reference keeps its cache in f32). */
uint16_t or_f16_from(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds past 65504 */
    uint32_t q, rem, half;
    if (ax < 0x38800000u) {                                   /* below 2^-14: a multiple of 2^-24 */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* below 2^-25 */
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126 - e;
        q = m >> sh;
        rem = m & ((1u << sh) - 1);
        half = 1u << (sh - 1);
    } else {
        const uint32_t r = ax - 0x38000000u;                  /* exponent rebiased from 127 to 15 */
        q = r >> 13;
        rem = r & 0x1fffu;
        half = 0x1000u;
    }
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static inline float f16_round(float f) { return or_f16(or_f16_from(f)); }

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* WGSL dot(vec4, vec4) taken left to right without fusion. */
static inline float dot4(const float* a, const float* b) {
    float r = a[0] * b[0];
    r = r + a[1] * b[1];
    r = r + a[2] * b[2];
    r = r + a[3] * b[3];
    return r;
}
static inline float sum4(const float* a) { return ((a[0] + a[1]) + a[2]) + a[3]; }

/* ------------------------------------------------------------------ Q4_K
 * Block: d f16, dmin f16, scales[12], qs[128] (web/js/kquants.js:7).
 * scmin: kquants.js:65-76.  Element dequant: kquants.js:166-168 (sm.x * q - sm.y). */
static void q4k_scmin(const uint8_t* blk, int j, float* fd, float* fm) {
    float d = or_f16(rd16(blk)), dmin = or_f16(rd16(blk + 2));
    const uint8_t* s = blk + 4;
    unsigned sc, mn;
    if (j < 4) {
        sc = s[j] & 63u;
        mn = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 15u) | ((unsigned)(s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((unsigned)(s[j] >> 6) << 4);
    }
    *fd = d * (float)sc;
    *fm = dmin * (float)mn;
}

static inline float q4k_deq(const uint8_t* blk, int e) {
    int j = e >> 5, l = e & 31;
    float fd, fm;
    q4k_scmin(blk, j, &fd, &fm);
    unsigned by = blk[16 + (j >> 1) * 32 + l];
    unsigned q = (by >> ((j & 1) * 4)) & 15u;
    float a = fd * (float)q;
    return a - fm;
}

/* ------------------------------------------------------------------ Q5_K
 * Block: d f16, dmin f16, scales[12], qh[32], qs[128] (kquants.js:8); the Q4_K scale/min unpack.  Element
 * dequant: kquants.js:151-153 (sm.x * (nibble + 16 * bit j of qh[l]) - sm.y). */
static inline float q5k_deq(const uint8_t* blk, int e) {
    int j = e >> 5, l = e & 31;
    float fd, fm;
    q4k_scmin(blk, j, &fd, &fm);
    unsigned lo = (blk[48 + (j >> 1) * 32 + l] >> ((j & 1) * 4)) & 15u;
    unsigned hi = (blk[16 + l] >> j) & 1u;
    float a = fd * (float)(lo + (hi << 4));
    return a - fm;
}

/* ------------------------------------------------------------------ Q3_K
 * Block: hmask[32], qs[64], scales[12], d f16 (kquants.js:10).  scq3: kquants.js:78-90 (6-bit scale of group s,
 * minus 32, times d).  Element dequant: kquants.js:159-162 (scq3(s) * (q2 - 4 * (1 - hmask bit))). */
static inline float q3k_scale(const uint8_t* blk, int s) {
    uint32_t a0 = rd32(blk + 96), a1 = rd32(blk + 100), tmp = rd32(blk + 104);
    uint32_t k1 = 0x03030303u, k2 = 0x0f0f0f0fu, wd;
    int g = s >> 2;
    if (g == 0) wd = (a0 & k2) | (((tmp >> 0) & k1) << 4);
    else if (g == 1) wd = (a1 & k2) | (((tmp >> 2) & k1) << 4);
    else if (g == 2) wd = ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4);
    else wd = ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4);
    float sc = (float)((wd >> ((s & 3) * 8)) & 0xffu) - 32.0f;
    return or_f16(rd16(blk + 108)) * sc;
}

static inline float q3k_deq(const uint8_t* blk, int e) {
    int s = e >> 4, n = e >> 7, r = e & 127, jj = r >> 5, l = r & 31;
    unsigned q2 = (blk[32 + n * 32 + l] >> (jj * 2)) & 3u;
    unsigned hm = (blk[l] >> (n * 4 + jj)) & 1u;
    return q3k_scale(blk, s) * ((float)q2 - 4.0f * (float)(1u - hm));
}

/* ------------------------------------------------------------------ Q2_K
 * Block: scales[16] (low nibble scale, high nibble min), qs[64], d f16, dmin f16 (kquants.js:11).  Setup:
 * kquants.js:108-116 (fd = d * (sc & 15), fm = dmin * (sc >> 4)); element = fd * q - fm (ggml's
 * dequantize_row_q2_K; the reference has no single-element form for Q2_K). */
static inline float q2k_deq(const uint8_t* blk, int e) {
    int j = e >> 4, n = e >> 7, jj = (e & 127) >> 5, l = e & 31;
    unsigned sc = blk[j];
    float fd = or_f16(rd16(blk + 80)) * (float)(sc & 15u), fm = or_f16(rd16(blk + 82)) * (float)(sc >> 4);
    unsigned q = (blk[16 + n * 32 + l] >> (jj * 2)) & 3u;
    float a = fd * (float)q;
    return a - fm;
}

/* ------------------------------------------------------------------ Q6_K
 * Block: ql[128], qh[64], scales[16] int8, d f16 (kquants.js:9).  scq6: kquants.js:92-96.
 * Element dequant: kquants.js:172-175 (scq6(s) * (q - 32)). */
static inline float q6k_scale(const uint8_t* blk, int s) {
    float d = or_f16(rd16(blk + 208));
    return d * (float)(int8_t)blk[192 + s];
}

static inline float q6k_deq(const uint8_t* blk, int e) {
    int s = e >> 4, h = e >> 7, r = e & 127, qd = r >> 5, l = r & 31;
    unsigned lo = (blk[h * 64 + (qd & 1) * 32 + l] >> ((qd >> 1) * 4)) & 15u;
    unsigned hi = (blk[128 + h * 32 + l] >> (qd * 2)) & 3u;
    float q = (float)(lo | (hi << 4)) - 32.0f;
    return q6k_scale(blk, s) * q;
}

/* ------------------------------------------------------------------ Q8_0
 * Block: d f16 + 32 int8 (gpu.js:1150-1162 repacks to qs + f32 ds); element = q * d (gpu.js:601-603). */
static inline float q8_deq(const uint8_t* blk, int e) {
    float d = or_f16(rd16(blk));
    return (float)(int8_t)blk[2 + e] * d;
}

/* ------------------------------------------------------------------ IQ4_NL
 * Block: d f16 + 16 bytes; the low nibble of byte l indexes weight l, the high nibble weight 16 + l, in the
 * 16-entry table (kds.js:36-39, the reference's conversion tests/conformance/gen_ds.py:104-129); element =
 * d * table[nibble] (kds.js:80-84 scale the block's sum by d; one product per element here). */
static const float IQ4NL_KV[16] = {-127.0f, -104.0f, -83.0f, -65.0f, -49.0f, -35.0f, -22.0f, -10.0f,
                                   1.0f,    13.0f,   25.0f,  38.0f,  53.0f,  69.0f,  89.0f,  113.0f};
static inline float iq4nl_deq(const uint8_t* blk, int e) {
    float d = or_f16(rd16(blk));
    unsigned q = e < 16 ? (blk[2 + e] & 15u) : (blk[2 + e - 16] >> 4);
    return d * IQ4NL_KV[q];
}

void or_dequant(int fmt, const uint8_t* raw, int64_t nelem, float* out) {
    int64_t i;
    if (fmt == OR_Q4_K) {
        for (i = 0; i < nelem; i++) out[i] = q4k_deq(raw + (i >> 8) * 144, (int)(i & 255));
    } else if (fmt == OR_Q5_K) {
        for (i = 0; i < nelem; i++) out[i] = q5k_deq(raw + (i >> 8) * 176, (int)(i & 255));
    } else if (fmt == OR_Q3_K) {
        for (i = 0; i < nelem; i++) out[i] = q3k_deq(raw + (i >> 8) * 110, (int)(i & 255));
    } else if (fmt == OR_Q2_K) {
        for (i = 0; i < nelem; i++) out[i] = q2k_deq(raw + (i >> 8) * 84, (int)(i & 255));
    } else if (fmt == OR_Q6_K) {
        for (i = 0; i < nelem; i++) out[i] = q6k_deq(raw + (i >> 8) * 210, (int)(i & 255));
    } else if (fmt == OR_Q8_0) {
        for (i = 0; i < nelem; i++) out[i] = q8_deq(raw + (i >> 5) * 34, (int)(i & 31));
    } else if (fmt == OR_IQ4_NL) {
        for (i = 0; i < nelem; i++) out[i] = iq4nl_deq(raw + (i >> 5) * 18, (int)(i & 31));
    } else if (fmt == OR_F16) {
        /* F16 matrices are widened to f32 when uploaded (weights.js:128, f16af32 of gpu.js:939-948) */
        for (i = 0; i < nelem; i++) out[i] = or_f16(rd16(raw + 2 * i));
    } else if (fmt == OR_BF16) {
        /* BF16: the 16 bits are the high half of the f32 (weights.js:129-133, v[i] = s[i] << 16) */
        for (i = 0; i < nelem; i++) {
            const uint32_t u = (uint32_t)rd16(raw + 2 * i) << 16;
            memcpy(out + i, &u, 4);
        }
    } else {
        memcpy(out, raw, (size_t)nelem * 4);
    }
}

/* ------------------------------------------------------------------ one-row GEMV, reference lane order
 * 32 lanes stride over items; each lane accumulates in order; then the LDS tree s = 16..1.
 * Q4_K / Q6_K: kquants.js:188-251 (matmul(n,1)), items/setup/q at kquants.js:104-148.
 * Q8_0: gpu.js:123-166 (matmul_q8_1).  F32: gpu.js:169-198 (matmul_f32_1). */
static float tree32(float* a) {
    for (int s = 16; s > 0; s >>= 1)
        for (int i = 0; i < s; i++) a[i] = a[i] + a[i + s];
    return a[0];
}

static float row_q4k(const uint8_t* row, int K, const float* x) {
    int nb = K / 256, ni = nb * 8;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float a = 0.0f;
        for (int it = lane; it < ni; it += 32) {
            int b = it / 8, j = it % 8;
            const uint8_t* blk = row + (size_t)b * 144;
            float fd, fm;
            q4k_scmin(blk, j, &fd, &fm);
            const uint8_t* qb = blk + 16 + (j >> 1) * 32;
            int sh = (j & 1) * 4;
            const float* xb = x + b * 256 + j * 32;
            float s = 0.0f, m = 0.0f;
            for (int wi = 0; wi < 8; wi++) {
                uint32_t w = rd32(qb + wi * 4);
                float q[4] = {(float)((w >> sh) & 15u), (float)((w >> (sh + 8)) & 15u),
                              (float)((w >> (sh + 16)) & 15u), (float)((w >> (sh + 24)) & 15u)};
                s = s + dot4(q, xb + wi * 4);
                m = m + sum4(xb + wi * 4);
            }
            a = a + (fd * s - fm * m);
        }
        lanes[lane] = a;
    }
    return tree32(lanes);
}

/* Q5_K: the Q4_K item loop of kquants.js:188-251 with the q5k setup/q of kquants.js:134-138 (quants at word 12,
 * q = nibble + 16 * bit j of the qh bytes at word 4). */
static float row_q5k(const uint8_t* row, int K, const float* x) {
    int nb = K / 256, ni = nb * 8;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float a = 0.0f;
        for (int it = lane; it < ni; it += 32) {
            int b = it / 8, j = it % 8;
            const uint8_t* blk = row + (size_t)b * 176;
            float fd, fm;
            q4k_scmin(blk, j, &fd, &fm);
            const uint8_t* qb = blk + 48 + (j >> 1) * 32;
            int sh = (j & 1) * 4;
            const float* xb = x + b * 256 + j * 32;
            float s = 0.0f, m = 0.0f;
            for (int wi = 0; wi < 8; wi++) {
                uint32_t w = rd32(qb + wi * 4), h = rd32(blk + 16 + wi * 4);
                float q[4];
                for (int t = 0; t < 4; t++)
                    q[t] = (float)((w >> (sh + 8 * t)) & 15u) + 16.0f * (float)((h >> (8 * t + j)) & 1u);
                s = s + dot4(q, xb + wi * 4);
                m = m + sum4(xb + wi * 4);
            }
            a = a + (fd * s - fm * m);
        }
        lanes[lane] = a;
    }
    return tree32(lanes);
}

/* Q3_K / Q2_K: the 16-element items of kquants.js:188-251 with the q3k / q2k setup and q (kquants.js:106-116,
 * 140-148): item j of block b covers elements 128 n + 32 jj + l0 .. + 15 (n = j >> 3, jj = (j & 7) >> 1,
 * l0 = 16 (j & 1)). */
static float row_q3k(const uint8_t* row, int K, const float* x) {
    int nb = K / 256, ni = nb * 16;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float a = 0.0f;
        for (int it = lane; it < ni; it += 32) {
            int b = it / 16, j = it % 16, n = j >> 3, jj = (j & 7) >> 1, l0 = (j & 1) * 16;
            const uint8_t* blk = row + (size_t)b * 110;
            float fd = q3k_scale(blk, j);
            const float* xb = x + b * 256 + n * 128 + jj * 32 + l0;
            float s = 0.0f;
            for (int wi = 0; wi < 4; wi++) {
                uint32_t w = rd32(blk + 32 + n * 32 + l0 + wi * 4), h = rd32(blk + l0 + wi * 4);
                float q[4];
                for (int t = 0; t < 4; t++)
                    q[t] = (float)(((w >> (8 * t + 2 * jj)) & 3u) + 4u * ((h >> (8 * t + n * 4 + jj)) & 1u)) - 4.0f;
                s = s + dot4(q, xb + wi * 4);
            }
            a = a + fd * s;
        }
        lanes[lane] = a;
    }
    return tree32(lanes);
}

static float row_q2k(const uint8_t* row, int K, const float* x) {
    int nb = K / 256, ni = nb * 16;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float a = 0.0f;
        for (int it = lane; it < ni; it += 32) {
            int b = it / 16, j = it % 16, n = j >> 3, jj = (j & 7) >> 1, l0 = (j & 1) * 16;
            const uint8_t* blk = row + (size_t)b * 84;
            unsigned sc = blk[j];
            float fd = or_f16(rd16(blk + 80)) * (float)(sc & 15u), fm = or_f16(rd16(blk + 82)) * (float)(sc >> 4);
            const float* xb = x + b * 256 + n * 128 + jj * 32 + l0;
            float s = 0.0f, m = 0.0f;
            for (int wi = 0; wi < 4; wi++) {
                uint32_t w = rd32(blk + 16 + n * 32 + l0 + wi * 4);
                float q[4];
                for (int t = 0; t < 4; t++) q[t] = (float)((w >> (8 * t + 2 * jj)) & 3u);
                s = s + dot4(q, xb + wi * 4);
                m = m + sum4(xb + wi * 4);
            }
            a = a + (fd * s - fm * m);
        }
        lanes[lane] = a;
    }
    return tree32(lanes);
}

static float row_q6k(const uint8_t* row, int K, const float* x) {
    int nb = K / 256, ni = nb * 16;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float a = 0.0f;
        for (int it = lane; it < ni; it += 32) {
            int b = it / 16, j = it % 16;
            const uint8_t* blk = row + (size_t)b * 210;
            int h = j >> 3, qd = (j & 7) >> 1, l0 = (j & 1) * 16;
            float fd = q6k_scale(blk, j);
            const float* xb = x + b * 256 + h * 128 + qd * 32 + l0;
            const uint8_t* qlo = blk + h * 64 + (qd & 1) * 32 + l0;
            const uint8_t* qhi = blk + 128 + h * 32 + l0;
            int nsh = (qd >> 1) * 4, hsh = qd * 2;
            float s = 0.0f;
            for (int wi = 0; wi < 4; wi++) {
                uint32_t lo = rd32(qlo + wi * 4), hi = rd32(qhi + wi * 4);
                float q[4];
                for (int c = 0; c < 4; c++) {
                    unsigned v = ((lo >> (8 * c + nsh)) & 15u) | (((hi >> (8 * c + hsh)) & 3u) << 4);
                    q[c] = (float)v - 32.0f;
                }
                s = s + dot4(q, xb + wi * 4);
            }
            a = a + fd * s;
        }
        lanes[lane] = a;
    }
    return tree32(lanes);
}

static float row_q8(const uint8_t* row, int K, const float* x) {
    int nb = K / 32;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float acc = 0.0f;
        for (int b = lane; b < nb; b += 32) {
            const uint8_t* blk = row + (size_t)b * 34;
            float d = or_f16(rd16(blk));
            float t[8];
            for (int w = 0; w < 8; w++) {
                float q[4];
                for (int c = 0; c < 4; c++) q[c] = (float)(int8_t)blk[2 + w * 4 + c];
                t[w] = dot4(q, x + b * 32 + w * 4);
            }
            float s = ((t[0] + t[1]) + t[2]) + t[3];
            s = s + (((t[4] + t[5]) + t[6]) + t[7]);
            acc = acc + d * s;
        }
        lanes[lane] = acc;
    }
    return tree32(lanes);
}

/* matmul_iq4nl_1 (kds.js:41-101, nt = 1): 32 lanes stride over the blocks; a block's sum s over its four words
 * (dot of the 4 low-nibble weights with x[8b + w], then of the 4 high ones with x[8b + 4 + w]), then
 * acc += d * s; the LDS tree over the lanes. */
static float row_iq4nl(const uint8_t* row, int K, const float* x) {
    int nb = K / 32;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float acc = 0.0f;
        for (int b = lane; b < nb; b += 32) {
            const uint8_t* blk = row + (size_t)b * 18;
            float d = or_f16(rd16(blk));
            float s = 0.0f;
            for (int w = 0; w < 4; w++) {
                float lo[4], hi[4];
                for (int c = 0; c < 4; c++) {
                    lo[c] = IQ4NL_KV[blk[2 + w * 4 + c] & 15u];
                    hi[c] = IQ4NL_KV[blk[2 + w * 4 + c] >> 4];
                }
                s = s + (dot4(lo, x + b * 32 + w * 4) + dot4(hi, x + b * 32 + 16 + w * 4));
            }
            acc = acc + d * s;
        }
        lanes[lane] = acc;
    }
    return tree32(lanes);
}

static float row_f32(const float* row, int K, const float* x) {
    int k4 = K / 4;
    float lanes[32];
    for (int lane = 0; lane < 32; lane++) {
        float acc = 0.0f;
        for (int k = lane; k < k4; k += 32) acc = acc + dot4(row + k * 4, x + k * 4);
        lanes[lane] = acc;
    }
    return tree32(lanes);
}

static size_t row_bytes(int fmt, int K) {
    switch (fmt) {
    case OR_Q4_K: return (size_t)(K / 256) * 144;
    case OR_Q5_K: return (size_t)(K / 256) * 176;
    case OR_Q3_K: return (size_t)(K / 256) * 110;
    case OR_Q2_K: return (size_t)(K / 256) * 84;
    case OR_Q6_K: return (size_t)(K / 256) * 210;
    case OR_Q8_0: return (size_t)(K / 32) * 34;
    case OR_IQ4_NL: return (size_t)(K / 32) * 18;
    default: return (size_t)K * 4;
    }
}

static float row_dot(int fmt, const uint8_t* row, int K, const float* x) {
    switch (fmt) {
    case OR_Q4_K: return row_q4k(row, K, x);
    case OR_Q5_K: return row_q5k(row, K, x);
    case OR_Q3_K: return row_q3k(row, K, x);
    case OR_Q2_K: return row_q2k(row, K, x);
    case OR_Q6_K: return row_q6k(row, K, x);
    case OR_Q8_0: return row_q8(row, K, x);
    case OR_IQ4_NL: return row_iq4nl(row, K, x);
    default: return row_f32((const float*)row, K, x);
    }
}

/* Tiled prefill order (kquants.js:309-386): the dequantized weight (fd*q - fm, kquants.js:344) times x,
 * accumulated serially over the whole of K. */
static float row_serial(int fmt, const uint8_t* row, int K, const float* x) {
    float c = 0.0f;
    for (int k = 0; k < K; k++) {
        float w;
        if (fmt == OR_Q4_K) w = q4k_deq(row + (size_t)(k >> 8) * 144, k & 255);
        else if (fmt == OR_Q5_K) w = q5k_deq(row + (size_t)(k >> 8) * 176, k & 255);
        else if (fmt == OR_Q3_K) w = q3k_deq(row + (size_t)(k >> 8) * 110, k & 255);
        else if (fmt == OR_Q2_K) w = q2k_deq(row + (size_t)(k >> 8) * 84, k & 255);
        else if (fmt == OR_Q6_K) w = q6k_deq(row + (size_t)(k >> 8) * 210, k & 255);
        else if (fmt == OR_Q8_0) w = q8_deq(row + (size_t)(k >> 5) * 34, k & 31);
        else if (fmt == OR_IQ4_NL) w = iq4nl_deq(row + (size_t)(k >> 5) * 18, k & 31);
        else w = ((const float*)row)[k];
        c = c + w * x[k];
    }
    return c;
}

/* One row dequantized with the values the element functions give (row_serial's w): Q4_K and Q6_K hoist the
 * per-sub-block factors, which the element functions recompute with the same operations. */
static void row_deq(int fmt, const uint8_t* row, int K, float* w) {
    if (fmt == OR_Q4_K) {
        for (int b = 0; b < K / 256; b++) {
            const uint8_t* blk = row + (size_t)b * 144;
            for (int j = 0; j < 8; j++) {
                float fd, fm;
                q4k_scmin(blk, j, &fd, &fm);
                const uint8_t* qb = blk + 16 + (j >> 1) * 32;
                const int sh = (j & 1) * 4;
                for (int l = 0; l < 32; l++) {
                    float a = fd * (float)((qb[l] >> sh) & 15u);
                    w[b * 256 + j * 32 + l] = a - fm;
                }
            }
        }
    } else if (fmt == OR_Q6_K) {
        for (int b = 0; b < K / 256; b++) {
            const uint8_t* blk = row + (size_t)b * 210;
            for (int s = 0; s < 16; s++) {
                const float sc = q6k_scale(blk, s);
                for (int e = s * 16; e < s * 16 + 16; e++) {
                    int h = e >> 7, r = e & 127, qd = r >> 5, l = r & 31;
                    unsigned lo = (blk[h * 64 + (qd & 1) * 32 + l] >> ((qd >> 1) * 4)) & 15u;
                    unsigned hi = (blk[128 + h * 32 + l] >> (qd * 2)) & 3u;
                    float q = (float)(lo | (hi << 4)) - 32.0f;
                    w[b * 256 + e] = sc * q;
                }
            }
        }
    } else {
        for (int k = 0; k < K; k++) {
            float v;
            if (fmt == OR_Q5_K) v = q5k_deq(row + (size_t)(k >> 8) * 176, k & 255);
            else if (fmt == OR_Q3_K) v = q3k_deq(row + (size_t)(k >> 8) * 110, k & 255);
            else if (fmt == OR_Q2_K) v = q2k_deq(row + (size_t)(k >> 8) * 84, k & 255);
            else if (fmt == OR_Q8_0) v = q8_deq(row + (size_t)(k >> 5) * 34, k & 31);
            else if (fmt == OR_IQ4_NL) v = iq4nl_deq(row + (size_t)(k >> 5) * 18, k & 31);
            else v = ((const float*)row)[k];
            w[k] = v;
        }
    }
}

/* The serial order of row_serial for many (row, token) pairs at once: out(t, r) = sum over k = 0..K-1, in that
 * order, of w_r[k] * x_t[k], every product and sum rounded separately.  Rows row0 .. row0+N-1 of W are
 * dequantized once per call (4 at a time); xT holds the inputs transposed, [K][ntp] (ntp = nt rounded up to 16,
 * zero padded), so the sums of 16 tokens advance together in vector lanes (each token's own operation sequence
 * is unchanged: lanes do not mix).  Token t's value for row r goes to y[yoff[t] + r] (added to it after the sum
 * when acc, as row_serial's callers do). */
#define OR_TB 16
typedef float or_v8 __attribute__((vector_size(32)));
__attribute__((target_clones("avx2", "default")))
static void serial_rows(int fmt, const uint8_t* W, size_t rb, size_t row0, int N, int K, const float* xT, int nt,
                        float* y, const size_t* yoff, int acc) {
    const int ntp = (nt + OR_TB - 1) / OR_TB * OR_TB;
#pragma omp parallel
    {
        float* w = (float*)calloc((size_t)4 * K, 4);
#pragma omp for schedule(dynamic, 1)
        for (int r0 = 0; r0 < N; r0 += 4) {
            const int nr = N - r0 < 4 ? N - r0 : 4;
            for (int i = 0; i < nr; i++) row_deq(fmt, W + rb * (row0 + (size_t)r0 + i), K, w + (size_t)i * K);
            for (int tb = 0; tb < ntp; tb += OR_TB) {
                /* c[i][h]: lanes = tokens tb + 8h .. tb + 8h + 7 of row r0 + i; elementwise mul then add */
                or_v8 c[4][2];
                memset(c, 0, sizeof(c));
                for (int k = 0; k < K; k++) {
                    or_v8 x0, x1;
                    memcpy(&x0, xT + (size_t)k * ntp + tb, 32);
                    memcpy(&x1, xT + (size_t)k * ntp + tb + 8, 32);
                    for (int i = 0; i < 4; i++) {
                        const float wv = w[(size_t)i * K + k];
                        const or_v8 wb = {wv, wv, wv, wv, wv, wv, wv, wv};
                        c[i][0] = c[i][0] + wb * x0;
                        c[i][1] = c[i][1] + wb * x1;
                    }
                }
                for (int i = 0; i < nr; i++)
                    for (int j = 0; j < OR_TB && tb + j < nt; j++) {
                        float* o = y + yoff[tb + j] + r0 + i;
                        const float v = c[i][j >> 3][j & 7];
                        *o = acc ? *o + v : v;
                    }
            }
        }
        free(w);
    }
}

/* [K][ntp] transpose of nt input rows (row j at xrows[j]), zero padded to a multiple of 16 tokens. */
static float* transpose_in(const float* const* xrows, int nt, int K) {
    const int ntp = (nt + OR_TB - 1) / OR_TB * OR_TB;
    float* xT = (float*)calloc((size_t)K * ntp, 4);
    for (int j = 0; j < nt; j++)
        for (int k = 0; k < K; k++) xT[(size_t)k * ntp + j] = xrows[j][k];
    return xT;
}

/* y[t][r] (+)= W[r] . x[t].  mode 0 = per-token lane order (matmul_*_1 and matmul_*_4, whose per-token
 * sums are identical), mode 1 = tiled serial order (matmul_*_t, used by transformer.js:276-279 when T>=8),
 * computed by serial_rows; mode 2 = the same serial order one (token, row) at a time with the element
 * functions (row_serial: the definition mode 1 is checked against). */
void or_matmul(int fmt, const uint8_t* W, int N, int K, const float* x, int T, float* y, int acc, int mode) {
    size_t rb = row_bytes(fmt, K);
    if (mode == 1) {
        const float** xr = (const float**)malloc(sizeof(float*) * (size_t)T);
        size_t* yo = (size_t*)malloc(sizeof(size_t) * (size_t)T);
        for (int t = 0; t < T; t++) {
            xr[t] = x + (size_t)t * K;
            yo[t] = (size_t)t * N;
        }
        float* xT = transpose_in(xr, T, K);
        serial_rows(fmt, W, rb, 0, N, K, xT, T, y, yo, acc);
        free(xT); free(xr); free(yo);
        return;
    }
    for (int t = 0; t < T; t++) {
        const float* xt = x + (size_t)t * K;
        float* yt = y + (size_t)t * N;
#pragma omp parallel for schedule(static)
        for (int r = 0; r < N; r++) {
            const uint8_t* row = W + rb * (size_t)r;
            float v = mode == 2 ? row_serial(fmt, row, K, xt) : row_dot(fmt, row, K, xt);
            yt[r] = acc ? yt[r] + v : v;
        }
    }
}

/* Gathered expert GEMV (kquants.js:256-304, kds.js:110-186): job z uses expert sel[z], row ex*N + r of the
 * stacked tensor, input row z / tfijo; output y[z*N + r].  mode 1 = grouped-tile serial order
 * (kquants.js:392-479, used for T >= 8 by deepseek2.js:377-381): the jobs of each expert together through
 * serial_rows (its rows dequantized once); mode 2 = the same order one (job, row) at a time. */
void or_matmul_e(int fmt, const uint8_t* W, int N, int K, const float* x, const uint32_t* sel, int njobs,
                 int tfijo, float* y, int mode) {
    size_t rb = row_bytes(fmt, K);
    if (mode == 1) {
        uint32_t emax = 0;
        for (int z = 0; z < njobs; z++) emax = sel[z] > emax ? sel[z] : emax;
        const float** xr = (const float**)malloc(sizeof(float*) * (size_t)njobs);
        size_t* yo = (size_t*)malloc(sizeof(size_t) * (size_t)njobs);
        for (uint32_t e = 0; e <= emax; e++) {
            int nj = 0;
            for (int z = 0; z < njobs; z++)
                if (sel[z] == e) {
                    xr[nj] = x + (size_t)(z / tfijo) * K;
                    yo[nj] = (size_t)z * N;
                    nj++;
                }
            if (!nj) continue;
            float* xT = transpose_in(xr, nj, K);
            serial_rows(fmt, W, rb, (size_t)e * N, N, K, xT, nj, y, yo, 0);
            free(xT);
        }
        free(xr); free(yo);
        return;
    }
    for (int z = 0; z < njobs; z++) {
        const float* xz = x + (size_t)(z / tfijo) * K;
        size_t ex = sel[z];
#pragma omp parallel for schedule(static)
        for (int r = 0; r < N; r++) {
            const uint8_t* row = W + rb * (ex * (size_t)N + (size_t)r);
            y[(size_t)z * N + r] = mode == 2 ? row_serial(fmt, row, K, xz) : row_dot(fmt, row, K, xz);
        }
    }
}

/* ------------------------------------------------------------------ embeddings
 * embed_q4k/q6k: kquants.js:481-504; embed_q8: gpu.js:585-604; embed_f32: gpu.js:605-618. */
void or_embed(int fmt, const uint8_t* W, int D, const uint32_t* ids, int T, float* y) {
    size_t rb = row_bytes(fmt, D);
    for (int t = 0; t < T; t++) {
        const uint8_t* row = W + rb * (size_t)ids[t];
        for (int k = 0; k < D; k++) {
            float v;
            if (fmt == OR_Q4_K) v = q4k_deq(row + (size_t)(k >> 8) * 144, k & 255);
            else if (fmt == OR_Q5_K) v = q5k_deq(row + (size_t)(k >> 8) * 176, k & 255);
            else if (fmt == OR_Q3_K) v = q3k_deq(row + (size_t)(k >> 8) * 110, k & 255);
            else if (fmt == OR_Q2_K) v = q2k_deq(row + (size_t)(k >> 8) * 84, k & 255);
            else if (fmt == OR_Q6_K) v = q6k_deq(row + (size_t)(k >> 8) * 210, k & 255);
            else if (fmt == OR_Q8_0) v = q8_deq(row + (size_t)(k >> 5) * 34, k & 31);
            else if (fmt == OR_IQ4_NL) v = iq4nl_deq(row + (size_t)(k >> 5) * 18, k & 31);
            else v = ((const float*)row)[k];
            y[(size_t)t * D + k] = v;
        }
    }
}

/* ------------------------------------------------------------------ RMSNorm
 * gpu.js:332-356: 256 threads stride the row, LDS tree k = 128..1, y = x * inv * w.
 * ultima = 1 normalizes only row T-1 into row 0 (gpu.js:344). */
static float or_rsqrt(float v) { return 1.0f / sqrtf(v); }

void or_rmsnorm(const float* x, const float* w, float* y, int T, int D, float eps, int ultima) {
    int rows = ultima ? 1 : T;
    for (int rr = 0; rr < rows; rr++) {
        int fila = ultima ? T - 1 : rr, out = ultima ? 0 : rr;
        const float* xr = x + (size_t)fila * D;
        float red[256];
        for (int li = 0; li < 256; li++) {
            float s = 0.0f;
            for (int i = li; i < D; i += 256) s = s + xr[i] * xr[i];
            red[li] = s;
        }
        for (int k = 128; k > 0; k >>= 1)
            for (int li = 0; li < k; li++) red[li] = red[li] + red[li + k];
        float inv = or_rsqrt(red[0] / (float)D + eps);
        for (int i = 0; i < D; i++) y[(size_t)out * D + i] = (xr[i] * inv) * w[i];
    }
}

/* ------------------------------------------------------------------ sin/cos
 * gpu.js:13-25: Cody-Waite reduction by pi/2 in three parts, then the Cephes single-precision sinf/cosf
 * minimax polynomials on [-pi/4, pi/4], quadrant from k & 3. */
void or_sincos2(float x, float* sn_out, float* cs_out) {
    float kx = x * 0.6366197723675814f;
    int k = (int)rintf(kx); /* WGSL round(): half to even; rintf in the default mode */
    float kf = (float)k;
    float r = ((x - kf * 1.5703125f) - kf * 4.837512969970703125e-4f) - kf * 7.549789948768648e-8f;
    float r2 = r * r;
    float sn = r + (r * r2) * (-1.6666654611e-1f + r2 * (8.3321608736e-3f + r2 * -1.9515295891e-4f));
    float cs = (1.0f - 0.5f * r2) +
               (r2 * r2) * (4.166664568298827e-2f + r2 * (-1.388731625493765e-3f + r2 * 2.443315711809948e-5f));
    unsigned q = (unsigned)k & 3u;
    if (q == 0) { *sn_out = sn; *cs_out = cs; }
    else if (q == 1) { *sn_out = cs; *cs_out = -sn; }
    else if (q == 2) { *sn_out = -sn; *cs_out = -cs; }
    else { *sn_out = -cs; *cs_out = sn; }
}

/* ------------------------------------------------------------------ per-head norm + RoPE (in place)
 * gpu.js:394-444.  v is [T][nh][hd]; w the per-head norm weight (used when usaNorm); neox selects pairs
 * (i, i + nrot/2) instead of (2i, 2i+1); theta = pos * esc * base^(-2j/nrot). */
void or_norm_rope(float* v, const float* w, int T, int nh, int hd, int usaNorm, int neox, float eps, float base,
                  int nrot, float esc, int pos0) {
    float val[512];
    for (int t = 0; t < T; t++) {
        for (int h = 0; h < nh; h++) {
            float* row = v + ((size_t)t * nh + h) * hd;
            float red[256];
            for (int li = 0; li < 256; li++) {
                float s = 0.0f;
                for (int i = li; i < hd; i += 256) { val[i] = row[i]; s = s + row[i] * row[i]; }
                red[li] = s;
            }
            for (int k = 128; k > 0; k >>= 1)
                for (int li = 0; li < k; li++) red[li] = red[li] + red[li + k];
            if (usaNorm) {
                float inv = or_rsqrt(red[0] / (float)hd + eps);
                for (int i = 0; i < hd; i++) val[i] = (val[i] * inv) * w[i];
            }
            float pos = (float)(pos0 + t);
            int mitad = nrot / 2;
            for (int i = 0; i < hd; i++) {
                float r = val[i];
                if (i < nrot) {
                    int j, primero;
                    float a, b;
                    if (neox) {
                        j = i % mitad;
                        if (i < mitad) { a = val[i]; b = val[i + mitad]; } else { a = val[i - mitad]; b = val[i]; }
                        primero = i < mitad;
                    } else {
                        j = i / 2;
                        int i0 = i - (i % 2);
                        a = val[i0]; b = val[i0 + 1];
                        primero = (i % 2) == 0;
                    }
                    float ex = (-2.0f * (float)j) / (float)nrot;
                    /* base^ex rounded once to float (evaluated in double), so the frequency does not depend
                     * on the accuracy of a library powf */
                    float theta = (pos * esc) * (float)pow((double)base, (double)ex);
                    float sn, c;
                    or_sincos2(theta, &sn, &c);
                    r = primero ? (a * c - b * sn) : (a * sn + b * c);
                }
                row[i] = r;
            }
        }
    }
}

/* ------------------------------------------------------------------ KV write (gpu.js:447-466)
 * slot = pos0 + t (mod cap when cap > 0); f32 cache [slot][kvd]. */
void or_kv_write(const float* k, const float* v, float* kc, float* vc, int T, int kvd, int pos0, int cap) {
    for (int t = 0; t < T; t++) {
        int slot = pos0 + t;
        if (cap > 0) slot %= cap;
        memcpy(kc + (size_t)slot * kvd, k + (size_t)t * kvd, (size_t)kvd * 4);
        memcpy(vc + (size_t)slot * kvd, v + (size_t)t * kvd, (size_t)kvd * 4);
    }
}

/* ------------------------------------------------------------------ causal GQA attention (gpu.js:467-539)
 * One (head, query) at a time; 64-key tiles; per tile: serial max over the 64 scores, exp, serial sum,
 * l = l*corr + sum, acc = acc*corr + sum_j p_j v_j (serial over the tile); output acc / l. */
void or_attention(const float* q, const float* kc, const float* vc, float* o, int T, int pos0, int nh, int nkv,
                  int hd, float escala, int swa, int cap) {
    int kvd = nkv * hd, grp = nh / nkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int t = 0; t < T; t++) {
        for (int h = 0; h < nh; h++) {
            int kvh = h / grp;
            int nkc = pos0 + t + 1, nk = nkc;
            int ini = 0;
            if (swa > 0 && nkc > swa) ini = nkc - swa;
            const float* qs = q + ((size_t)t * nh + h) * hd;
            float m = -3.0e38f, l = 0.0f;
            float acc[256];
            float sc[64];
            for (int d = 0; d < hd; d++) acc[d] = 0.0f;
            for (int tile = ini; tile < nk; tile += 64) {
                for (int li = 0; li < 64; li++) {
                    int pk = tile + li;
                    float s = -3.0e38f;
                    if (pk < nk) {
                        int sl = cap > 0 ? pk % cap : pk;
                        const float* kb = kc + (size_t)sl * kvd + (size_t)kvh * hd;
                        float dot = 0.0f;
                        for (int i = 0; i < hd; i++) dot = dot + qs[i] * kb[i];
                        s = dot * escala;
                    }
                    sc[li] = s;
                }
                float mt = m;
                for (int j = 0; j < 64; j++) mt = fmaxf(mt, sc[j]);
                for (int li = 0; li < 64; li++) sc[li] = (tile + li < nk) ? expf(sc[li] - mt) : 0.0f;
                float corr = expf(m - mt);
                float suma = 0.0f;
                for (int j = 0; j < 64; j++) suma = suma + sc[j];
                l = l * corr + suma;
                int nt = nk - tile < 64 ? nk - tile : 64;
                for (int d = 0; d < hd; d++) {
                    float a = acc[d] * corr;
                    for (int j = 0; j < nt; j++) {
                        int sv = cap > 0 ? (tile + j) % cap : tile + j;
                        a = a + sc[j] * vc[(size_t)sv * kvd + (size_t)kvh * hd + d];
                    }
                    acc[d] = a;
                }
                m = mt;
            }
            for (int d = 0; d < hd; d++) o[((size_t)t * nh + h) * hd + d] = acc[d] / l;
        }
    }
}

/* ------------------------------------------------------------------ SwiGLU (gpu.js:570-582) */
void or_swiglu(float* g, const float* u, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float a = g[i];
        g[i] = (a / (1.0f + expf(-a))) * u[i];
    }
}

/* GeGLU, tanh form (gpu.js:318-330), in the WGSL expression's order with one rounding per operation. */
void or_geglu(float* g, const float* u, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float a = g[i];
        float c = ((0.044715f * a) * a) * a;
        float z = 0.79788456f * (a + c);
        z = fminf(fmaxf(z, -20.0f), 20.0f);
        g[i] = ((0.5f * a) * (1.0f + tanhf(z))) * u[i];
    }
}

/* escalar (gpu.js:635-646): x = x * s; suma_esc (gpu.js:648-660): x = x + s * t. */
void or_escalar(float* x, int64_t n, float s) {
    for (int64_t i = 0; i < n; i++) x[i] = x[i] * s;
}
void or_suma_esc(float* x, const float* t, int64_t n, float s) {
    for (int64_t i = 0; i < n; i++) x[i] = x[i] + s * t[i];
}

/* ------------------------------------------------------------------ MoE routing (kds.js:191-221)
 * softmax over E logits; k rounds of strict max (ties -> lower index); weights = probs * f with
 * f = scale / max(sum, 2^-14) when norm, else scale. */
void or_moe_topk(const float* lg, int T, int E, int k, int norm, float escala, uint32_t* sel, float* wts) {
    float pr[1024];
    for (int t = 0; t < T; t++) {
        float m = -3.0e38f;
        for (int e = 0; e < E; e++) { pr[e] = lg[(size_t)t * E + e]; m = fmaxf(m, pr[e]); }
        float s = 0.0f;
        for (int e = 0; e < E; e++) { pr[e] = expf(pr[e] - m); s = s + pr[e]; }
        for (int e = 0; e < E; e++) pr[e] = pr[e] / s;
        float tot = 0.0f;
        for (int i = 0; i < k; i++) {
            int bi = 0;
            float bv = -1.0f;
            for (int e = 0; e < E; e++) if (pr[e] > bv) { bv = pr[e]; bi = e; }
            sel[t * k + i] = (uint32_t)bi;
            wts[t * k + i] = bv;
            tot = tot + bv;
            pr[bi] = -2.0f;
        }
        float f = escala;
        if (norm) f = f / fmaxf(tot, 6.103515625e-5f);
        for (int i = 0; i < k; i++) wts[t * k + i] = wts[t * k + i] * f;
    }
}

/* ------------------------------------------------------------------ MoE combine (kds.js:224-240)
 * x[t][i] += sum_s wts[t*k+s] * de[(t*k+s)*D + i], summed serially over s. */
void or_moe_comb(float* x, const float* de, const float* wts, int T, int D, int k) {
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++) {
            float a = 0.0f;
            for (int s = 0; s < k; s++) a = a + wts[t * k + s] * de[((size_t)t * k + s) * D + c];
            x[(size_t)t * D + c] = x[(size_t)t * D + c] + a;
        }
}

/* ------------------------------------------------------------------ greedy (sampling.js:38-42)
 * strict '>' from -Infinity: ties go to the lowest index, NaN is never chosen. */
int or_argmax(const float* v, int n) {
    int best = 0;
    float mv = -INFINITY;
    for (int i = 0; i < n; i++) if (v[i] > mv) { mv = v[i]; best = i; }
    return best;
}

/* ================================================================== model forward
 * The dense decoder's dispatch order (web/js/transformer.js:252-336, plan at 180-241) and the MoE FFN
 * order of deepseek2.js:374-386 without shared experts (Qwen3-MoE has none).  All activations and the KV
 * cache are f32, as in the reference (transformer.js:110-111). */
typedef struct {
    const uint8_t *attn_norm, *wq, *wk, *wv, *wo, *q_norm, *k_norm, *ffn_norm;
    const uint8_t *gate, *up, *down;             /* dense FFN */
    const uint8_t *router, *gate_e, *up_e, *down_e; /* MoE FFN */
    int fq, fk, fv, fo, fgate, fup, fdown, frouter, fgate_e, fup_e, fdown_e;
    /* gemma3 (transformer.js:46-54, 106-111, 206-207, 218-231): normalized outputs before the residual add,
     * a sliding window of swa keys (0: none), the layer's RoPE base and angle scale (0: the model's, 1) */
    const uint8_t *post_att, *post_ffn;
    int swa;
    float rbase, resc;
} OrLayer;

typedef struct {
    int n_layers, D, nh, nkv, hd, F, vocab, nrot, neox, ctx;
    int n_exp, n_used, ffe, moe_norm; /* n_exp = 0: dense */
    int tiled;                         /* options.tiled_prefill (transformer.js:60) */
    float eps, base, escala, moe_scale;
    const uint8_t *tok_embd, *output, *output_norm;
    int f_embd, f_output;
    OrLayer* layers;
    /* state */
    int pos;
    float *kc, *vc; /* [L][ctx][kvd] */
    int kv_f16;     /* option of this backend: cache rows rounded to f16 when written (reference: f32 only) */
    /* f16 mode, for checking a GPU run: the cache rows of positions < nref are taken from kref / vref
     * ([L][nref][kvd] f16, the GPU's own cache) instead of this restatement's rounding of its own k and v */
    const uint16_t *kref, *vref;
    int nref;
    /* scales (transformer.js:35-45; 0: none) and the GeGLU FFN of gemma3 */
    float emb_scale, res_scale, logit_scale, softcap;
    int geglu;
} OrModel;

OrModel* or_model_new(void) { return (OrModel*)calloc(1, sizeof(OrModel)); }
OrLayer* or_model_layers(OrModel* m, int n) {
    m->n_layers = n;
    m->layers = (OrLayer*)calloc((size_t)n, sizeof(OrLayer));
    return m->layers;
}
int or_model_alloc_kv(OrModel* m) {
    size_t n = (size_t)m->n_layers * m->ctx * m->nkv * m->hd;
    m->kc = (float*)calloc(n, 4);
    m->vc = (float*)calloc(n, 4);
    return (m->kc && m->vc) ? 0 : -1;
}
void or_model_reset(OrModel* m) { m->pos = 0; }
int or_model_pos(OrModel* m) { return m->pos; }
void or_model_free(OrModel* m) {
    if (!m) return;
    free(m->kc); free(m->vc); free(m->layers); free(m);
}
size_t or_model_sizeof(void) { return sizeof(OrModel); }
size_t or_layer_sizeof(void) { return sizeof(OrLayer); }

/* mm() of transformer.js:268-284: one token -> lane order; T >= 8 with a K-quant and tiling on -> tiled. */
static void mm(const OrModel* m, int fmt, const uint8_t* W, int N, int K, const float* x, int T, float* y, int acc) {
    int kq = fmt == OR_Q2_K || fmt == OR_Q3_K || fmt == OR_Q4_K || fmt == OR_Q5_K || fmt == OR_Q6_K;
    int mode = (T >= 8 && kq && m->tiled) ? 1 : 0;
    or_matmul(fmt, W, N, K, x, T, y, acc, mode);
}

/* forward(ids, T, logits): T tokens from the current position; logits (vocab floats) of the last token
 * when logits != NULL.  Returns 0, or -1 on a context overflow / bad batch (transformer.js:256-257). */
int or_model_forward(OrModel* m, const uint32_t* ids, int T, float* logits) {
    int D = m->D, nh = m->nh, nkv = m->nkv, hd = m->hd, kvd = nkv * hd, qd = nh * hd;
    if (T < 1 || m->pos + T > m->ctx) return -1;
    int F = m->n_exp ? m->n_used * m->ffe : m->F;
    float* x = (float*)calloc((size_t)T * D, 4);
    float* xn = (float*)calloc((size_t)T * D, 4);
    float* q = (float*)calloc((size_t)T * qd, 4);
    float* k = (float*)calloc((size_t)T * kvd, 4);
    float* v = (float*)calloc((size_t)T * kvd, 4);
    float* att = (float*)calloc((size_t)T * qd, 4);
    float* g = (float*)calloc((size_t)T * F, 4);
    float* u = (float*)calloc((size_t)T * F, 4);
    float* tmp = (float*)calloc((size_t)T * D, 4);
    const float resid = m->res_scale ? m->res_scale : 1.0f;
    float* rl = NULL; float* de = NULL; float* wts = NULL; uint32_t* sel = NULL;
    if (m->n_exp) {
        rl = (float*)calloc((size_t)T * m->n_exp, 4);
        de = (float*)calloc((size_t)T * m->n_used * D, 4);
        wts = (float*)calloc((size_t)T * m->n_used, 4);
        sel = (uint32_t*)calloc((size_t)T * m->n_used, 4);
    }
    or_embed(m->f_embd, m->tok_embd, D, ids, T, x);
    if (m->emb_scale) or_escalar(x, (int64_t)T * D, m->emb_scale);
    for (int li = 0; li < m->n_layers; li++) {
        const OrLayer* L = &m->layers[li];
        const float rbase = L->rbase ? L->rbase : m->base, resc = L->resc ? L->resc : 1.0f;
        float* kc = m->kc + (size_t)li * m->ctx * kvd;
        float* vc = m->vc + (size_t)li * m->ctx * kvd;
        or_rmsnorm(x, (const float*)L->attn_norm, xn, T, D, m->eps, 0);
        mm(m, L->fq, L->wq, qd, D, xn, T, q, 0);
        mm(m, L->fk, L->wk, kvd, D, xn, T, k, 0);
        mm(m, L->fv, L->wv, kvd, D, xn, T, v, 0);
        or_norm_rope(q, (const float*)L->q_norm, T, nh, hd, L->q_norm != NULL, m->neox, m->eps, rbase, m->nrot,
                     resc, m->pos);
        or_norm_rope(k, (const float*)L->k_norm, T, nkv, hd, L->k_norm != NULL, m->neox, m->eps, rbase, m->nrot,
                     resc, m->pos);
        or_kv_write(k, v, kc, vc, T, kvd, m->pos, 0);
        if (m->kv_f16)
            for (size_t i = (size_t)m->pos * kvd; i < (size_t)(m->pos + T) * kvd; i++) {
                const size_t p = i / kvd;
                if ((int)p < m->nref) {
                    const size_t r = ((size_t)li * m->nref + p) * kvd + i % kvd;
                    kc[i] = or_f16(m->kref[r]);
                    vc[i] = or_f16(m->vref[r]);
                } else {
                    kc[i] = f16_round(kc[i]);
                    vc[i] = f16_round(vc[i]);
                }
            }
        /* a window over the whole cache: the same keys as the reference's ring of swa + batch slots */
        or_attention(q, kc, vc, att, T, m->pos, nh, nkv, hd, m->escala, L->swa, 0);
        if (L->post_att || m->res_scale) { /* transformer.js:218-231: into tmp, normalized, x += resid * it */
            mm(m, L->fo, L->wo, D, qd, att, T, tmp, 0);
            if (L->post_att) or_rmsnorm(tmp, (const float*)L->post_att, xn, T, D, m->eps, 0);
            or_suma_esc(x, L->post_att ? xn : tmp, (int64_t)T * D, resid);
        } else {
            mm(m, L->fo, L->wo, D, qd, att, T, x, 1);
        }
        or_rmsnorm(x, (const float*)L->ffn_norm, xn, T, D, m->eps, 0);
        if (!m->n_exp) {
            mm(m, L->fgate, L->gate, m->F, D, xn, T, g, 0);
            mm(m, L->fup, L->up, m->F, D, xn, T, u, 0);
            if (m->geglu) or_geglu(g, u, (int64_t)T * m->F);
            else or_swiglu(g, u, (int64_t)T * m->F);
            if (L->post_ffn || m->res_scale) {
                mm(m, L->fdown, L->down, D, m->F, g, T, tmp, 0);
                if (L->post_ffn) or_rmsnorm(tmp, (const float*)L->post_ffn, xn, T, D, m->eps, 0);
                or_suma_esc(x, L->post_ffn ? xn : tmp, (int64_t)T * D, resid);
            } else {
                mm(m, L->fdown, L->down, D, m->F, g, T, x, 1);
            }
        } else {
            int E = m->n_exp, K = m->n_used, ffe = m->ffe;
            int grp = T >= 8 && m->tiled; /* deepseek2.js:373, 377 */
            or_matmul(L->frouter, L->router, E, D, xn, T, rl, 0, 0);
            or_moe_topk(rl, T, E, K, m->moe_norm, m->moe_scale, sel, wts);
            or_matmul_e(L->fgate_e, L->gate_e, ffe, D, xn, sel, T * K, K, g, grp);
            or_matmul_e(L->fup_e, L->up_e, ffe, D, xn, sel, T * K, K, u, grp);
            or_swiglu(g, u, (int64_t)T * K * ffe);
            or_matmul_e(L->fdown_e, L->down_e, D, ffe, g, sel, T * K, 1, de, grp);
            or_moe_comb(x, de, wts, T, D, K);
        }
    }
    if (logits) {
        float* xl = (float*)calloc((size_t)D, 4);
        or_rmsnorm(x, (const float*)m->output_norm, xl, T, D, m->eps, 1);
        or_matmul(m->f_output, m->output, m->vocab, D, xl, 1, logits, 0, 0);
        free(xl);
        /* on the host in double, stored to float (transformer.js:333-334) */
        if (m->logit_scale) {
            const double kk = 1.0 / (double)m->logit_scale;
            for (int i = 0; i < m->vocab; i++) logits[i] = (float)((double)logits[i] * kk);
        }
        if (m->softcap) {
            const double c = (double)m->softcap;
            for (int i = 0; i < m->vocab; i++) logits[i] = (float)(c * tanh((double)logits[i] / c));
        }
    }
    m->pos += T;
    free(x); free(xn); free(q); free(k); free(v); free(att); free(g); free(u); free(tmp);
    free(rl); free(de); free(wts); free(sel);
    return 0;
}

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void or_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
