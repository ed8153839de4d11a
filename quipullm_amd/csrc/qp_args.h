// Kernel argument blocks, shared by the host op table (quipu.cpp) and the gfx950 kernels.
// Every kernel takes exactly one of these structs by value.  Device addresses travel as uint64_t so the
// header stays plain C on both sides.
#pragma once
#include <stdint.h>

// ---------------------------------------------------------------- weight formats (ggml type ids)
#define QP_F32 0
#define QP_Q8_0 8
#define QP_Q2_K 10
#define QP_Q3_K 11
#define QP_Q4_K 12
#define QP_Q5_K 13
#define QP_Q6_K 14
#define QP_IQ4_NL 20

// Device layouts (private to the ops that read them; produced at load time by the repack ops):
//  F32  : [N][K] floats.
//  Q4_K : per row of nb = K/256 blocks, 9 planes of 16-byte chunks: chunk c of block b at row*nb*144 + c*nb*16 +
//         b*16 (chunk 0 = d, dmin, 12 scale bytes; chunks 1..8 = the 128 quant bytes).
//  Q6_K : per row, 13 chunk planes (ql 0..7, qh 8..11, scales 12) at row*nb*208 + c*nb*16 + b*16, then after all
//         rows a plane of the f16 d values [rows][nb].
//  Q8_0 : planar over NB = N*K/32 blocks: qs [NB][32] int8 | d [NB] f16.
//  IQ4_NL: planar over NB = N*K/32 blocks: qs [NB][16] bytes as in the GGUF block (byte l: weight l in the low
//         nibble, weight 16 + l in the high one) | d [NB] f16 (the reference's qs / dh pair, kds.js:36-39).
// Planar sub-arrays start at multiples of 16 bytes, so every lane load is a 16-byte vector load.

// Paso (per-forward step record, reference gpu.js:9): {T, pos0, a, b}, in device memory.
// The decode graph advances pos0 on the device.

// ---------------------------------------------------------------- GEMV (one token)
#define QP_GEMV_STORE 0   // y[r] = v
#define QP_GEMV_ACC 1     // y[r] += v   (residual add, reference acc=1)
#define QP_GEMV_SWIGLU 2  // segment pairs gate rows with the same rows of w2 (up): y[r] = silu(g)*u
#define QP_GEMV_ARGMAX 3  // y[r] = v, and a packed (value, index) max per row group into amax
#define QP_MAX_SEG 4

typedef struct {
    uint64_t w;     // weights (device layout of fmt)
    uint64_t w2;    // second matrix (QP_GEMV_SWIGLU: the up projection; same fmt and shape)
    uint64_t y;     // output floats
    uint32_t fmt;   // QP_F32 / QP_Q8_0 / QP_IQ4_NL / the K-quants
    uint32_t n;     // output rows of this segment
    uint32_t wg0;   // first workgroup of this segment
    uint32_t mode;  // QP_GEMV_*
    uint32_t row_base;    // rows of this segment start at weight row row_base of the tensor
    uint32_t rows_total;  // rows of the whole tensor (sizes the planar sub-arrays)
    uint32_t pad[2];
} QpGemvSeg;

typedef struct {
    QpGemvSeg seg[QP_MAX_SEG];
    uint64_t x;       // input floats [K] (row xrow of a [T][K] activation)
    uint64_t norm_w;  // 0, or RMSNorm weight [K]: the input is rmsnorm(x) * norm_w (fused prologue)
    uint64_t paso;    // device Paso (for xrow = T-1 when last_row)
    uint64_t amax;    // QP_GEMV_ARGMAX target: one uint64 (packed value/index), max-reduced
    uint32_t nseg;
    uint32_t k;
    float eps;
    uint32_t last_row;  // 1: read x row T-1 (the reference's rmsnorm "ultima" mode)
    uint32_t rows_per_wg;  // weight rows per workgroup pass (4 waves x R)
    uint32_t total_wg;     // workgroups covering all segments (grid-stride over them)
    uint32_t tseq, pad;    // tseq: timeline slot of a captured launch (timeline builds; 0: none)
} QpGemvArgs;

// Gathered expert GEMV (reference matmul_*_e, kquants.js:256-304): job z uses expert sel[z].
typedef struct {
    uint64_t w, x, y, sel, paso;
    uint32_t fmt, n, k, tfijo;   // n rows per expert; input row = job / tfijo
    uint32_t njobs_fixed;        // 0: njobs = T * kused from paso; else fixed
    uint32_t kused;
    uint32_t mode;               // 0 store; QP_GEMV_SWIGLU: w2 = up, y = silu(gate.x) * up.x
    uint32_t n_exp;              // experts in the stacked tensor (rows = n_exp * n)
    uint64_t w2;
} QpGemvExpArgs;

// Fused MoE FFN of one decode token: the arithmetic of the reference's moe_topk, matmul_*_e (gate, up), swiglu,
// matmul_*_e (down) and moe_comb sequence (deepseek2.js:375-386) in two launches.
// moe_gate_up: every workgroup routes the token from the router logits [e] (softmax, kused strict maxima, ties to
//   the lower expert, weights times scale, divided by their sum when norm); job blockIdx.y then computes
//   y[job][0..n) = silu(gate_x . xn) * (up_x . xn) for its expert x, with xn = rmsnorm(x, eps) * norm_w over k
//   inputs.  Workgroup (0, 0) also writes sel[kused] and wts[kused].
// moe_down: y[r] += sum_j wts[j] * (down_{sel[j]} row r) . x[j][0..k), r < n, as one GEMV over kused * k inputs.
typedef struct {
    uint64_t w, w2;      // gate, up (stacked [e * n][k]) | down (stacked [e * n][k]), 0
    uint64_t x, y;       // gate/up: residual in, h out [kused][n] | down: h in [kused][k], residual accumulated
    uint64_t logits, sel, wts, norm_w;
    uint32_t n, k, e, kused;
    float eps, scale;
    uint32_t norm, tseq;
    uint32_t presel, pad[3];  // gate/up: 1 = the routing is read from sel (written by moe_router), not computed
} QpMoeArgs;

// moe_router (no reference counterpart; the reference runs rmsnorm, matmul_f32 and moe_topk): the router logits
// logits[e] = W[e] . (rmsnorm(x) * norm_w) of one token (W f32 [e][k]) and, in the last of its workgroups to
// finish, the routing of moe_topk (kds.js:191-221) into sel[kused], wts[kused].  Grid (8, nw): only column 0
// works (its nw workgroups share one XCD, whose L2 holds the arrival counter cnt and the logits they store); the
// other columns exit at once.  cnt: two words only this op touches, zero at allocation: the arrival counter (the
// last arrival resets it) and, at cnt + 4, an error word whose bit 0 is set when the workgroups were found on more
// than one XCD (the host checks it).
typedef struct {
    uint64_t w, x, norm_w, logits, sel, wts, cnt;
    uint32_t e, k, kused, nw;
    float eps, scale;
    uint32_t norm, tseq;
} QpRouterArgs;

// Multi-token GEMV for prefill (reference matmul_*_4 / matmul_*_t semantics): y[t][r] (+)= W[r].x[t].
typedef struct {
    uint64_t w, x, y, paso;
    uint64_t xs;      // matrix-core path: 0, or x split into bf16 high and low planes ([rows][k] each, lo at xs + 2*rows*k)
    uint64_t ws;      // matrix-core path: 0, or the split-K partials [splits][rows][n] (summed by qp_gemm_reduce)
    uint32_t fmt, n, k, acc;
    uint32_t tfix;    // 0: T from paso
    uint32_t kchunk;  // matrix-core path: inputs per K split (grid z = splits; a multiple of 64), or 0: all of k
    uint32_t rows;    // matrix-core path: token rows the xs planes and the ws partials are sized for (>= T)
    uint32_t wrows;   // rows of the weight tensor (the Q6_K / Q8_0 / IQ4_NL scale arrays follow them), or 0: n
    // grouped by expert (matmul_*_eg): lst != 0.  Grid y = n_exp * tpe slots; slot s takes tile s % tpe (128 jobs)
    // of expert s / tpe, jobs lst[off[e] ..off[e + 1]); job j reads x row j / tfijo and writes y row j, weights
    // rows e * n .. of the stacked tensor.  xrows, yrows, nlst: rows of x, y and entries of lst that exist.
    uint64_t lst, off;
    uint32_t n_exp, tpe, tfijo, xrows, yrows, nlst;
    uint64_t w2;  // matmul_<fmt>_t_swiglu: the up tensor (w is the gate tensor); y = silu(x w) * (x w2)
    // matmul_<fmt>_t_swiglu with a split tail (tail != 0): a 1-D grid of items over mtiles x ntiles tiles; per XCD
    // (item % 8), whole tiles first, then its share of the last `tail` tiles as K halves.  Each half stores its
    // sums to part (two 256 KB slots per split tile) and counts its arrival in cnt[tile]; the second adds the
    // other's sums and finishes the tile (and resets the word).
    uint32_t tail, mtiles, ntiles;
    // matmul_<fmt>_t_swiglu: 1 = y receives the outputs as the next matmul's input planes (the bf16 high and low
    // planes of qp_split_bf16's layout for rows token rows and K = n), not as f32 rows
    uint32_t yplanes;
    uint64_t part, cnt;
} QpGemmArgs;

// moe_group: lst[off[e] .. off[e + 1]) = the jobs i < T * n (in increasing order) with sel[i] == e, e < n_exp;
// off[n_exp] = the number listed.  nsel: entries of sel and lst that exist.
typedef struct {
    uint64_t sel, lst, off, paso;
    uint32_t n_exp, n, nsel, pad;
} QpMoeGroupArgs;
// x [T][k] -> bf16 high / low planes (hi = bf16(v), lo = bf16(v - hi)) at xs and xs + 2*rows*k.  mul != 0: the
// first min(T * mul, cap) rows of x instead of T, in row-major planes ([rows][k rounded up to 32]: the grouped
// expert matmul, whose tiles gather rows), not the chunk-quarter layout of the 256-token tiles.
typedef struct { uint64_t x, xs, paso; uint32_t k, rows, mul, cap; } QpSplitArgs;
// y[t][n] = (acc ? y : 0) + sum over s (in order) of ws[s][t][n].
typedef struct { uint64_t ws, y, paso; uint32_t n, rows, splits, acc; } QpReduceArgs;

// ---------------------------------------------------------------- elementwise / small ops
typedef struct { uint64_t w, ids, y, paso; uint32_t fmt, d, rows, tseq; } QpEmbedArgs;  // rows: tensor rows
typedef struct { uint64_t x, w, y, paso; uint32_t d, ultima; float eps; uint32_t rows_fixed; } QpRmsArgs;
// rmsnorm_planes: the rmsnorm of each token row written as the next matmul's bf16 input planes (xs, rows token rows)
typedef struct { uint64_t x, w, xs, paso; uint32_t d, rows; float eps; uint32_t pad; } QpRmsPlanesArgs;
typedef struct {
    uint64_t v, w, paso;
    uint32_t hd, nh, use_norm, neox;
    float eps, base;
    uint32_t nrot;
    float esc;
    uint64_t freq;  // RoPE frequencies base^(-2j/nrot) as floats [nrot/2], or 0: computed in every workgroup
} QpRopeArgs;
// rows: slots of the cache (writes at or past it are dropped, never out of bounds)
typedef struct { uint64_t k, v, kc, vc, paso; uint32_t kvd, cap, f16, rows; } QpKvArgs;
typedef struct { uint64_t g, u, paso; uint32_t f, pad; } QpSwigluArgs;
typedef struct { uint64_t x, t, paso; uint32_t d; float s; } QpScaleArgs;  // escalar (t unused), suma_esc
typedef struct { uint64_t lg, sel, wts, paso; uint32_t e, k, norm; float scale; } QpTopkArgs;
typedef struct { uint64_t x, de, wts, paso; uint32_t d, k, pad0, pad1; } QpCombArgs;

// Causal GQA attention over the cache (reference atencion, gpu.js:467-539), any T.
typedef struct {
    uint64_t q, kc, vc, o, paso;
    uint32_t hd, nh, nkv, swa;
    float scale;
    uint32_t cap, f16, qb;   // qb: queries per workgroup
    uint32_t rows;           // slots of the cache; keys at or past it are not read
    uint32_t orows;          // 0: o holds f32 rows; else o receives them as the next matmul's bf16 input planes
                             // (qp_split_bf16's layout, orows token rows, K = nh hd)
    uint32_t pad[2];
} QpAttnArgs;

// Split-K decode attention with fused q/k norm + RoPE + KV append (one token).
typedef struct {
    uint64_t q, k, v, kc, vc, paso;
    uint64_t qnorm, knorm;      // 0 when absent
    uint64_t part_o, part_ml;   // [nh][nsplit][hd], [nh][nsplit][2]
    uint64_t freq;              // RoPE frequencies base^(-2j/nrot) as floats [nrot/2], or 0: computed in the kernel
    uint32_t hd, nh, nkv, nsplit;
    float scale, eps, base, esc;
    uint32_t nrot, neox, f16, rows;  // rows: slots of the cache; a position at or past it writes an empty result
    uint32_t tseq;
    // columns per KV head of a merged launch (1, or 2, 4, 8): column c of the grid takes KV head c / gsplit and its
    // G query heads from c * G (G = the kernel's group, nh / nkv / gsplit); only column c % gsplit == 0 appends
    uint32_t gsplit, pad[2];
    // merged output: 0, or o [nh][hd] written by the last workgroup of each column to finish (the grid's x is then
    // 8: columns past nkv * gsplit exit); cnt: arrival counters, one per column 128 bytes apart, zero between
    // launches, and at cnt + 1024 an error word whose bit 0 is set when a column's workgroups were found on more
    // than one XCD (the host checks it)
    uint64_t att, cnt;
} QpDecAttnArgs;

typedef struct {
    uint64_t part_o, part_ml, o, paso;
    uint32_t hd, nh, nsplit, tseq;
} QpDecCombArgs;

// The attention block of one decode token in one launch (dec_attn_block; no reference counterpart: the reference
// dispatches rmsnorm, matmul q/k/v, norm_rope, kv_write, atencion and matmul wo): grid (8, ns).  The 8 columns
// are head groups, one per XCD: group c takes KV head c / (8 / nkv) and its gq = nh / 8 query heads starting at
// c * gq.  Its ns workgroups
//   1. compute the group's q rows and its KV head's k and v rows of W . (rmsnorm(x) * norm_w) (K = dm; the K/V
//      rows are computed by every group of the KV head), while the first key/value tile of each wavefront loads;
//   2. meet at a barrier of the group (a counter in the XCD's L2), then run the split-K attention of the group's
//      query heads over the cache with the fused q/k norm, RoPE and KV append (groups with c % (8 / nkv) == 0
//      append), storing the split partials;
//   3. meet again, then either (wo == 0) merge the partials into att [nh][hd], a slice per workgroup, or (wo != 0)
//      each merges the group's gq * hd outputs in LDS and computes rows [y * dm / ns, ...) of the group's column
//      slice of wo: xpart[c][r] = sum over the group's columns of wo[r][col] * att[col] (Q4_K wo; the consumer
//      adds x + xpart[0] + ... + xpart[7], in that order).
// cnt: 8 counters 256 bytes apart that only this op touches, zero at allocation (each barrier adds ns to its
// group's counter; ns is a power of two).  err: a word set non-zero when a barrier's wait runs past spin_max
// polls (bit 0) or a workgroup found itself on another XCD than its group's first (bit 1; xcc: 8 words, the XCD
// + 1 of workgroup (c, 0) in the last launch).
typedef struct {
    uint64_t x, norm_w, wq, wk, wv, q, k, v;
    uint64_t kc, vc, paso, qnorm, knorm, part_o, part_ml, freq, att;
    uint64_t wo, xpart, cnt, xcc, err;
    uint32_t fq, fk, fv, dm;     // formats of wq, wk, wv (QP_Q4_K / QP_Q6_K); model width
    uint32_t hd, nh, nkv, ns;    // ns: workgroups per group (power of two, <= 64)
    float scale, eps, base, esc;
    uint32_t nrot, neox, rows, tseq;
    uint32_t spin_max, fo, pad[2];
} QpDecBlockArgs;

// Greedy argmax finish: reads the packed max, writes ids[0] and tokens[step], clears the max, advances
// paso.pos0 by T and the step counter.
// cap: entries of `tokens`; steps at or past it are not recorded
typedef struct { uint64_t amax, ids, tokens, step, paso; uint32_t count, advance, cap, tseq; } QpArgmaxFinArgs;
// Plain argmax over n floats (lowest index wins ties; NaN never chosen) -> out[0].
typedef struct { uint64_t v, out; uint32_t n, pad; } QpArgmaxArgs;

// Sampling helpers (no counterpart in the reference, which samples on the host): penalties over (token, count)
// pairs with double factors; top-k candidates in two stages (kp = k + 1 keys per 2048-logit chunk, g chunks,
// n2 = the merge's power-of-two size).
typedef struct { uint64_t logits, hist; double rep, freq, pres; uint32_t count, n; } QpPenaltyArgs;
typedef struct { uint64_t logits, part, out; uint32_t n, k, kp, g, n2, pad; } QpCandArgs;

// Load-time repacks from the GGUF block layout to the device layout (k: row length, for Q4_K / Q6_K).
typedef struct { uint64_t src, dst; uint64_t nblocks; uint32_t k, pad; } QpRepackArgs;
typedef struct { uint64_t dst; uint64_t count; uint32_t value, pad; } QpFillArgs;
typedef struct { uint64_t w, y; uint32_t fmt, k; uint64_t nelem; } QpDequantArgs;  // k: row length
