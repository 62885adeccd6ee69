/* moe_oracle.h - CPU restatement of the reference's quantized MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY. The HIP path is compared with this oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it. The product library
 * (rosevine_amd/librvmoe.so) never links, loads or calls it. oracle/Makefile also builds the
 * reference's own HIP kernels into oracle/_ref/ (a second reference for the GPU tests).
 *
 * Every function restates the reference's Rust (paths relative to the reference root) in
 * the same operation order, compiled with -ffp-contract=off so that no multiply-add is fused,
 * as runtime/build.rs:33-36 compiles the reference's HIP code. Rust semantics that C does not
 * share are written out: f32::round is roundf (half away from zero), `as i8` saturates and
 * maps NaN to 0, f32::max ignores NaN (fmaxf), total_cmp is the IEEE total order, float sums
 * are sequential folds, f32::exp/tanh are the platform expf/tanhf.
 *
 * Parity pinning: tests/test_oracle.py and tests/test_oracle_attention.py check every function against the reference's literal
 * known answers, independent implementations (numpy's IEEE half conversion, float32 sequential
 * accumulate, stable sort), closed forms, f64 brute force or exhaustive sweeps;
 * tests/test_oracle_mutations.py plants plausible mistakes in a copy of this file and shows that
 * those checks catch each one; tests/golden/ freezes small input/output vectors. Parity
 * unpinned: orc_dot_q8_avx2_order is held only to the exact-integer error bound (its lane order is the
 * CPU baseline's, not a value the GPU path is compared with), and the f32 operation order of
 * orc_gelu and of the combine follows the cited lines by reading, with the reference's own
 * bitwise combine test (runtime/tests/hip_ops.rs:421-439) as the check of the latter.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* runtime/src/ops.rs:7-24 */
float orc_f16_to_f32(uint16_t h);
/* runtime/src/ops.rs:27-59 (round to nearest even) */
uint16_t orc_f32_to_f16(float f);
/* runtime/src/ops.rs:83-92 */
void orc_dequant_q4_0(const uint8_t *row, float *out, size_t k);
/* runtime/src/ops.rs:67-80 */
float orc_dot_q4_0(const uint8_t *row, const float *x, size_t k);
/* runtime/src/ops.rs:249-266 (the reference's check for rvh_q4_mm, runtime/tests/hip_ops.rs:66) */
void orc_matmul_q4_0(const uint8_t *w, size_t k, const float *x, size_t n_in, float *y, size_t n_out);
/* runtime/src/ops.rs:95-105 */
void orc_quantize_q8_0(const float *x, uint8_t *out, size_t k);
/* runtime/src/expert_kernel.rs:147-161 */
float orc_dot_q8_scalar(const uint8_t *row, const uint8_t *xq, size_t k);
/* The per-block integer core of expert_kernel.rs:152-157: sums[b] for each 32-block. */
void orc_q4q8_block_sums(const uint8_t *row, const uint8_t *xq, size_t k, int32_t *sums);
/* runtime/src/expert_kernel.rs:163-191: the avx2_q8 accumulation order (8 lane partials, each
 * block's 8 pair-sums FMA-accumulated per lane, then a sequential sum of the 8 lanes),
 * restated with scalar fmaf so that it runs on any host. */
float orc_dot_q8_avx2_order(const uint8_t *row, const uint8_t *xq, size_t k);
/* runtime/src/ops.rs:321-326 (f32 products, sequential fold) */
void orc_matvec_f32(const float *w, size_t k, const float *x, float *y, size_t n_out);
/* runtime/src/ops.rs:131-139, with the `post` factor of rvhip.h:42 (post = 1 is ops::rms_norm). */
void orc_rms_norm(float *x, const float *weight, size_t n, float eps, float post);
/* runtime/src/ops.rs:145-149 */
float orc_gelu(float x);
/* runtime/src/exec.rs:606-611: out[r][j] = gelu(gu[r][j]) * gu[r][ff + j] for rows of 2*ff. */
void orc_geglu_split(const float *gu, float *out, size_t rows, size_t ff);
/* runtime/src/ops.rs:170-179 */
void orc_softmax(float *x, size_t n);
/* runtime/src/ops.rs:107-118 */
float orc_dot_q8_0(const uint8_t *row, const float *x, size_t k);
/* runtime/src/ops.rs:120-128 */
void orc_axpy_q8_0(const uint8_t *row, float w, float *out, size_t k);
/* runtime/tests/hip_ops.rs:245-271: causal attention over a Q8_0 key/value ring, scale 1.0,
 * window 0 = global. q, out: [n][nh][hd]; kc, vc: [cap][nkv][hd/32 blocks]. */
void orc_attention(const float *q, const uint8_t *kc, const uint8_t *vc, size_t nh, size_t nkv, size_t hd,
                   size_t cap, size_t win, size_t p0, size_t n, float *out);
/* runtime/tests/hip_ops.rs:9-22: the reference tests' generator, so that tests here can feed the
 * kernels the reference tests' own inputs. Advances *state by n draws. */
void orc_test_rng_vec(uint64_t *state, size_t n, float scale, float *out);
/* runtime/src/ops.rs:182-187 */
void orc_top_k(const float *x, size_t n, size_t k, uint32_t *out);
/* Router logits with the plain projection W_r . x (ops.rs:321-326) plus an optional per-expert
 * bias added after the dot. */
void orc_router_logits(const float *w_r, const float *bias, const float *x, size_t n_tok, size_t n_exp, size_t d,
                       float *logits);
/* runtime/src/exec.rs:507-517: softmax, top `used`, renormalised weights (clamp 2^-14, exec.rs:124-125).
 * logits are overwritten by the probabilities, as the reference does. */
void orc_select_experts(float *logits, size_t n_tok, size_t n_exp, size_t used, uint32_t *ids, float *weights);
/* runtime/src/exec.rs:540-558: order sorted by (expert, pair), pos_of, and group_start[n_exp+1]. */
void orc_moe_plan(const uint32_t *ids, size_t pairs, size_t n_exp, uint32_t *order, uint32_t *pos_of,
                  uint32_t *group_start);

/* runtime/src/exec.rs:572-640 in the Q8_0 activation domain (runtime/src/expert_pool.rs:311-320
 * quantises each activation row once per segment; each row is dot_q8_scalar).
 * gate_up[e] / down[e] point at expert e's Q4_0 rows ([2ff][d] and [d][ff]) or are NULL for
 * experts never selected. ids/weights: [n_tok][used]. down_scale may be NULL (1.0).
 * gu (pairs*2ff), h (pairs*ff) and y (pairs*d) receive the intermediates in plan order when
 * non-NULL. Returns 0, or -1 when a selected expert has no weights. */
int orc_experts_q8(const uint8_t *const *gate_up, const uint8_t *const *down, const float *down_scale,
                   const float *moe_in, size_t n_tok, size_t d, size_t ff, size_t used, const uint32_t *ids,
                   const float *weights, float *out, float *gu, float *h, float *y);

/* Whole layer: optional pre-norm (ops.rs:131-139, no weight), router, selection, experts. */
int orc_moe_layer(const float *w_r, const float *bias, const uint8_t *const *gate_up, const uint8_t *const *down,
                  const float *down_scale, const float *x, size_t n_tok, size_t n_exp, size_t d, size_t ff,
                  size_t used, int pre_norm, float eps, uint32_t *ids, float *weights, float *out);

/* ---- CPU baseline (cpu_baseline.c): the reference's CPU expert path with a persistent
 * worker pool claiming 16-row chunks (runtime/src/expert_pool.rs:86-136, 357-447) and the
 * avx2_q8 kernel (expert_kernel.rs:163-191) when the host has AVX2+FMA. ---- */
typedef struct cpb_pool cpb_pool;
cpb_pool *cpb_create(int threads);
void cpb_destroy(cpb_pool *pool);
int cpb_threads(const cpb_pool *pool);
/* 1 when the AVX2+FMA kernel runs, 0 for the scalar kernel. */
int cpb_uses_avx2(void);
/* Nanoseconds spent in the expert part (plan, quantisation, the pooled GEMV segments, GeGLU and
 * combine) of every cpb_moe_layer call on this pool so far; the router and selection before it are
 * not included. */
uint64_t cpb_expert_ns(const cpb_pool *pool);
/* One MoE layer for n_tok tokens on the pool (router and selection on the caller thread, as
 * runtime/src/exec.rs:456-475). Same arguments as orc_moe_layer. */
int cpb_moe_layer(cpb_pool *pool, const float *w_r, const float *bias, const uint8_t *const *gate_up,
                  const uint8_t *const *down, const float *down_scale, const float *x, size_t n_tok,
                  size_t n_exp, size_t d, size_t ff, size_t used, uint32_t *ids, float *weights, float *out);

#ifdef __cplusplus
}
#endif
