/* rvmoe.h - MI355X (gfx950) quantized mixture-of-experts FFN path behind a C ABI.
 *
 * Conventions (same contract as the reference's runtime/hip/rvhip.h:1-14):
 *   - every function returns 0 or a hipError_t code; no exception crosses the ABI;
 *   - scalar arguments and null pointers are validated here (hipErrorInvalidValue);
 *     buffer extents are the caller's contract;
 *   - work is issued in order on the library's current stream (the null stream unless
 *     rvm_set_stream selected another); rvh_download and rvh_sync synchronise;
 *   - device pointers come from rvh_alloc and are released by rvh_free.
 *
 * Layouts:
 *   Q4_0 row (reference/GGUF layout): k/32 blocks of {f16 d; u8 qs[16]}; value j =
 *     ((qs[j] & 15) - 8) * d, value j + 16 = ((qs[j] >> 4) - 8) * d (rvhip.h:10-11).
 *   Q8_0 row: k/32 blocks of {f16 d; i8 q[32]} (runtime/src/ops.rs:61-63, 94-105).
 *   Packed Q4_0 (this library's HBM layout, produced by rvm_pack_q4 from Q4_0 rows): a
 *     nibble plane followed by a scale plane, the same total size as the Q4_0 rows.
 *     Rows are cut into tiles of 64 "lanes"; for tile t, step s and lane l the plane entry
 *     index is (t * S + s) * 64 + l, holding 16 nibble bytes (qs XOR 0x88, so that every
 *     nibble is the signed 4-bit weight) and one f16 scale.
 *       RVM_PACK_GATE_UP: 64-row tiles; lane l < 32 is gate row 32t + l, lane l >= 32 is up
 *         row n_out/2 + 32t + (l - 32); step s is block s (S = k/32).
 *       RVM_PACK_ROWS32: 32-row tiles; lane l is row 32t + (l & 31) at block
 *         (l >> 5) * S + s, with S = k/64.
 *     Matrix m of a stack of n_mat matrices owns tiles m*T .. m*T + T-1.
 *   Activations are row-major f32 [token][width].
 */
#pragma once
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- Runtime, memory and events: same symbols and meaning as rvhip.h:22-38 ---- */
int rvh_init(int device);
int rvh_mem_info(size_t *free_bytes, size_t *total_bytes);
int rvh_alloc(size_t bytes, void **out);
int rvh_free(void *ptr);
int rvh_upload(void *dst, const void *src, size_t bytes);
int rvh_download(void *dst, const void *src, size_t bytes);
int rvh_copy(void *dst, const void *src, size_t bytes); /* device to device, ordered */
int rvh_sync(void);
const char *rvh_error_string(int code);
int rvh_event_create(void **out);
int rvh_event_destroy(void *ev);
int rvh_event_record(void *ev);
int rvh_event_sync(void *ev);
int rvh_event_elapsed(void *start, void *end, float *ms);

/* ---- Reference expert-path kernels: same signatures and results as rvhip.h ---- */
/* out[r] = ((x[r] * rms_scale) * post) * weight (weight may be NULL); rvhip.h:42-43. */
int rvh_rms_norm(const float *x, float *out, const float *weight, int rows, int width, float eps, float post);
/* y[t][r] = W[r] . x[t], f32 router GEMV; rvhip.h:49-50. */
int rvh_f32_mm(const float *w, const float *x, float *y, int n_out, int k, int n_in);
/* y[t][r] = W_q4[r] . x[t], Q4_0 rows (reference layout), f32 activations; rvhip.h:44-45. */
int rvh_q4_mm(const void *w, const float *x, float *y, int n_out, int k, int n_in);
/* rvh_q4_mm's result up to summation order; x 16-byte aligned, w 2-byte aligned; rvhip.h:46-48. */
int rvh_q4_mv(const void *w, const float *x, float *y, int n_out, int k, int n_in);
/* n_mat (1 to 4) rvh_q4_mm products on one input in one launch (matrices of 16384 rows or more,
 * k <= 8192, take a launch each): y[m] = w[m] x for matrices of n_out[m] rows (each 2-byte
 * aligned), the bits of rvh_q4_mm per matrix. w, n_out and y are host
 * arrays. No counterpart in rvhip.h: the reference runs one rvh_q4_mm per projection on the same
 * input (q, k, v: runtime/src/hip_exec.rs:728-731; gate, up: :773-774). */
int rvm_q4_mm_n(int n_mat, const void *const *w, const int *n_out, float *const *y, const float *x, int k, int n_in);
/* Rows of 2*ff (gate then up) to rows of ff: gelu(gate) * up; rvhip.h:70-71. */
int rvh_geglu_split(const float *gu, float *out, int rows, int ff);
/* dst[i] = src[idx[i]], rows of width; rvhip.h:76-77. */
int rvh_gather_rows(const float *src, const int32_t *idx, float *dst, int n, int width);
/* out[t] = sum_j (y[pos[p]] * scale[p]) * weight[p], p = t*used + j, slot order; rvhip.h:78-80. */
int rvh_moe_combine(const float *y, const int32_t *pos, const float *scale, const float *weight, float *out,
                    int n_tok, int used, int width);
/* Q8_0 of the keys and values of n_tok tokens ([n_tok][n_kv][hd] f32) into ring slots
 * (p0 + t) % cap of kc and vc ([cap][n_kv][hd/32 blocks of 34 bytes]); bit for bit the CPU
 * quantiser runtime/src/ops.rs:95-105. rvhip.h:55-56. */
int rvh_kv_store(const float *k, const float *v, void *kc, void *vc, int n_tok, int n_kv, int hd, int p0, int cap);
/* Causal attention, scale 1.0, of n_tok queries at positions p0.. ([n_tok][n_head][hd]); window 0
 * is global, else keys p > pos - window; kv head of query head h is h / (n_head / n_kv).
 * hd % 32 == 0, hd <= 512; the longest key range must be <= max_keys and <= cap. scores is the
 * reference's n_tok * n_head * max_keys scratch: it must be non-NULL and is left untouched (the
 * kernel is rvh_attn_split's with one chunk). rvhip.h:57-60. */
int rvh_attention(const float *q, const void *kc, const void *vc, float *out, float *scores, int n_tok, int n_head,
                  int n_kv, int hd, int p0, int cap, int window, int max_keys);
/* Split-K attention, rvh_attention's result up to summation order. Each query's keys are cut into
 * n_chunks contiguous chunks of ceil(keys / n_chunks); n_chunks == 1 writes out (part may be
 * NULL), else part receives [n_tok * n_head][n_chunks][hd + 2] = {max, sum, acc[hd]} for
 * rvh_attn_combine. n_chunks <= 65535. rvhip.h:61-65. */
int rvh_attn_split(const float *q, const void *kc, const void *vc, float *out, float *part, int n_tok, int n_head,
                   int n_kv, int hd, int p0, int cap, int window, int n_chunks);
/* Merge rows * n_chunks partials of rvh_attn_split into rows outputs of hd. n_chunks > 1.
 * rvhip.h:66-67. */
int rvh_attn_combine(const float *part, float *out, int rows, int hd, int n_chunks);
/* One decode token's attention core: rvh_kv_store of its key and value rows ([n_kv][hd] f32) into
 * slot pos % cap, then rvh_attn_split over keys lo .. pos with n_chunks chunks and, for n_chunks > 1,
 * rvh_attn_combine (part as there) -- the ring bytes and out bit for bit that sequence, which the
 * reference runs as three calls (runtime/src/hip_exec.rs:743-760). No counterpart symbol in rvhip.h:
 * for hd 256 and 512 the store happens inside the split kernel, one launch fewer per layer. */
int rvm_attn_decode(const float *q, const float *k, const float *v, void *kc, void *vc, float *out, float *part,
                    int n_head, int n_kv, int hd, int pos, int cap, int window, int n_chunks);

/* ---- Additive MoE entry points (no counterpart symbol in rvhip.h) ---- */

/* Select the stream for subsequent launches (NULL = null stream). The stream is a hipStream_t. */
int rvm_set_stream(void *stream);
int rvm_stream_create(void **out);
int rvm_stream_destroy(void *stream);
/* Capture the launches issued on the current (non-null) stream into a graph and instantiate it. */
int rvm_graph_begin(void);
int rvm_graph_end(void **graph_exec);
int rvm_graph_launch(void *graph_exec);
int rvm_graph_destroy(void *graph_exec);

/* Packed Q4_0 formats (see the layout notes above). */
#define RVM_PACK_GATE_UP 1
#define RVM_PACK_ROWS32 2

/* Bytes of n_mat packed matrices of n_out x k (equal to the Q4_0 row bytes). */
int rvm_q4_packed_bytes(int n_mat, int n_out, int k, int format, size_t *bytes);
/* Repack n_mat consecutive Q4_0 matrices (reference layout, n_out rows of k) on the device.
 * Replaces the GGUF expert binding of runtime/src/model.rs:33-40 at load time. */
int rvm_pack_q4(const void *src, void *dst, int n_mat, int n_out, int k, int format);

/* Seeded synthetic Q4_0 matrices in the reference layout: scale f16(U(0.005, 0.02)), nibble
 * bytes uniform; matrix m uses stream stream0 + m. The device and host variants write the
 * same bytes. */
int rvm_synth_q4(void *dst, int n_mat, int n_out, int k, uint64_t seed, uint64_t stream0);
int rvm_synth_q4_host(void *dst, int n_mat, int n_out, int k, uint64_t seed, uint64_t stream0);

/* Q8_0 activation quantisation of rows x k floats (k % 32 == 0): runtime/src/ops.rs:94-105. */
int rvm_quantize_q8_0(const float *x, void *xq, int rows, int k);

/* y[t][r] = W[r] . xq[t]: packed Q4_0 rows times Q8_0 activation rows, each block an exact int32
 * sum scaled by d_w * d_x (runtime/src/expert_kernel.rs:85-95, 147-161). */
int rvm_q4q8_mm(const void *w_packed, int format, const void *xq, float *y, int n_out, int k, int n_in);
/* Per-block int32 sums of one activation row: sums[r][b] = sum_j w[r][32b+j] * q[32b+j]. */
int rvm_q4q8_block_sums(const void *w_packed, int format, const void *xq, int32_t *sums, int n_out, int k);

/* GeGLU then Q8_0: hq[r] = quantize_q8_0(gelu(gu[r][:ff]) * gu[r][ff:]) (runtime/src/exec.rs:606-611
 * followed by runtime/src/expert_pool.rs:311-320). */
int rvm_geglu_q8_0(const float *gu, void *hq, int rows, int ff);

/* One MoE layer's device weights. */
typedef struct rvm_layer {
    int n_exp;                /* experts, <= 256 */
    int top_k;                /* experts per token, <= 8 */
    int d;                    /* model width, multiple of 256 */
    int ff;                   /* expert width, multiple of 64 */
    const float *router;      /* [n_exp][d] f32 row-major */
    const float *router_bias; /* [n_exp] f32 added to the logits, or NULL */
    const void *gate_up;      /* n_exp packed RVM_PACK_GATE_UP matrices of [2*ff][d] */
    const void *down;         /* n_exp packed RVM_PACK_ROWS32 matrices of [d][ff] */
    const float *down_scale;  /* [n_exp] f32 (down_exps_scale) or NULL for 1.0 */
} rvm_layer;

/* Flags for the layer entry points. */
#define RVM_PRE_NORM 1     /* the layer input is rms_norm(x, eps) (runtime/src/ops.rs:131-139) */
#define RVM_EXACT_SELECT 2 /* always recompute the router logits in the reference's order */

/* From this many tokens a call folds every router logit in the reference's order (exact logits,
 * ids and weights; no certificate and no fallbacks); decode and smaller batches rank by the
 * certified f64 estimates, with the exact fallback. */
#define RVM_FOLD_MIN_TOKENS 256

/* Workspace bytes for n_tok tokens through rvm_moe_decode (n_tok = 1) or rvm_moe_forward.
 * A workspace is zeroed once with rvm_workspace_init and may be reused by later calls on the
 * same stream; concurrent calls need separate workspaces. */
int rvm_moe_workspace_bytes(const rvm_layer *layer, int n_tok, size_t *bytes);
int rvm_workspace_init(void *ws, size_t bytes);
/* Router-selection exactness fallbacks taken in this workspace so far (synchronises). */
int rvm_workspace_fallbacks(const void *ws, uint32_t *count);
/* The expert ids and weights ([n_tok][top_k], top order) chosen by the last rvm_moe_decode /
 * rvm_moe_forward call of n_tok tokens on this workspace, copied to host memory (synchronises);
 * the reference's selection observer, runtime/src/exec.rs:519-526. */
int rvm_workspace_selection(const rvm_layer *layer, int n_tok, const void *ws, int32_t *ids, float *weights);

/* Router logits, softmax, top-k and renormalised weights for n_tok tokens (runtime/src/exec.rs:
 * 493-517 with the plain projection W_r . x plus bias). ids[t][j] and weights[t][j] are in the
 * reference's top order; the ids are always the reference's. logits (n_tok x n_exp, may be NULL)
 * receives the f32 logits: the reference's bits with RVM_EXACT_SELECT, from RVM_FOLD_MIN_TOKENS
 * tokens, and for every token whose estimate-based ranking could not be certified; a certified
 * token receives its f64 estimates rounded to f32 (within the certificate's bound of the
 * reference's). The weights follow the same split: the reference's arithmetic on the exact paths,
 * the estimates' (within the f32 tolerance) on certified tokens. */
int rvm_router_select(const rvm_layer *layer, const float *x, int n_tok, int flags, float eps, int32_t *ids,
                      float *weights, float *logits, void *ws, size_t ws_bytes);

/* Stable grouping of n_pairs (token, slot) pairs by expert (runtime/src/exec.rs:540-558):
 * order[k] = pair index sorted by (expert, pair); pos_of[pair] = k; group_start[e] .. group_start[e+1]
 * is expert e's range of order (n_exp + 1 entries). */
int rvm_moe_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of,
                 int32_t *group_start);

/* One decode token through one MoE layer: out[d] = sum_j down_j(geglu(gate_up_j(x))) * scale * weight,
 * in slot order (runtime/src/exec.rs:456-475, 572-640; runtime/src/hip_exec.rs:780-843). */
int rvm_moe_decode(const rvm_layer *layer, const float *x, float *out, int flags, float eps, void *ws,
                   size_t ws_bytes);

/* The MoE block's two inputs from one hidden row o, as the reference's executor forms them
 * (runtime/src/hip_exec.rs:784-796; on the CPU runtime/src/exec.rs:465-468 and 493-503). With
 * s = 1 / sqrt(mean(o^2) + eps) (runtime/src/ops.rs:131-139):
 *   router input  ((o[i] * s) * router_post) * router_scale[i]   (ffn_gate_inp.scale; post = 1/sqrt(d))
 *   expert input  (o[i] * s) * expert_scale[i]                  (pre_ffw_norm_2.weight)
 * each product rounded in that order; a NULL scale is no factor. */
typedef struct rvm_block_norms {
    float eps;
    float router_post;
    const float *router_scale; /* [d] or NULL */
    const float *expert_scale; /* [d] or NULL */
} rvm_block_norms;

/* The reference's MoE block in one call per layer: the router norm and GEMV, the selection, the
 * expert-input norm, the expert dispatch and the combine of runtime/src/hip_exec.rs:784-842
 * (rvh_rms_norm(o, router_x, gate_inp_scale, eps, 1/sqrt(d)), rvh_f32_mm, the host's
 * select_experts, rvh_rms_norm(o, moe_in, pre_ffw_norm_2, eps, 1), the experts and rvh_moe_combine),
 * with no host round trip. out receives the combined expert output, before the post_ffw_norm_2
 * norm the reference applies next (hip_exec.rs:845, an rvh_rms_norm call). flags: 0 or
 * RVM_EXACT_SELECT. Decode is one token; forward takes n_tok tokens with device grouping. */
int rvm_moe_block_decode(const rvm_layer *layer, const rvm_block_norms *norms, const float *o, float *out, int flags,
                         void *ws, size_t ws_bytes);
int rvm_moe_block_forward(const rvm_layer *layer, const rvm_block_norms *norms, const float *o, float *out, int n_tok,
                          int flags, void *ws, size_t ws_bytes);

/* rvm_moe_decode without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Its scratch is a static device array of RVM_STATIC_SCRATCH_BYTES
 * in the library, one per GPU, held until the process ends; its address is taken by rvh_init (or
 * by the first call on a device) and the call allocates nothing. Every supported layer shape fits
 * (the largest, 256 experts, top-8, d = 4096, ff = 1024, needs about 8.1 MiB); a layer that needed
 * more would be refused with hipErrorInvalidValue. Calls on one GPU share the array: calls that
 * overlap on one GPU (two streams, or two host threads) race. */
#define RVM_STATIC_SCRATCH_BYTES (9u << 20)
int rvm_moe_decode_static(const rvm_layer *layer, const float *x, float *out, int flags, float eps);

/* n_tok tokens through one MoE layer with device grouping (ragged decode batches and prefill). */
int rvm_moe_forward(const rvm_layer *layer, const float *x, float *out, int n_tok, int flags, float eps, void *ws,
                    size_t ws_bytes);

/* ---- Device-call counters and the stack executor ---- */

/* Device calls issued by the calling thread through this library since the last reset (the
 * reference's per-thread Counters of runtime/src/hip.rs:167-187): kernel launches, host-to-device,
 * device-to-host and device-to-device copies, explicit host synchronisations (rvh_sync and
 * rvh_event_sync; as in the reference, rvh_upload and rvh_download count as copies only, though they
 * wait for their copy), and graph launches. Inside a graph capture the launches counted are the
 * captured ones. */
typedef struct rvm_counters {
    uint64_t launches, h2d, d2h, d2d, syncs, graphs;
} rvm_counters;
int rvm_counters_get(rvm_counters *counters);
int rvm_counters_reset(void);

/* Diagnostic builds only (compiled with RVM_PHASE_TRACE; other builds return hipErrorNotSupported):
 * copies the realtime-counter stamps (100 MHz, u64) of the last decode call to host memory of at
 * least 3 x 4096 x 8 x 8 bytes: [kernel][workgroup][point] for k_router (0: entry, 1: done, 2: row
 * and x loaded), k_gateup_decode (0: entry, 1: expert known, 2: first block terms formed, 3: h block
 * ready, 4: down terms stored) and k_down_fold (0: entry, 1: rows folded, 2: output stored, 3: down
 * terms loaded); the points "loaded" wait for the loads, in this build only. No counterpart
 * in the reference: it measures where a decode token's time goes across workgroups and XCDs. */
int rvm_phase_trace(void *host, size_t bytes);

/* A stack of n_layers MoE layers of one shape evaluated on the device: one workspace for up to
 * max_tokens tokens and two activation buffers, allocated here (the executor of
 * runtime/src/hip_exec.rs:780-843 without its per-layer logits download, host selection and
 * metadata uploads). Between layers either the synthetic stack's RMSNorm with eps (norms NULL:
 * layer 0 takes its input as is, every later layer rms_norm of the previous output), or each
 * layer's block norms norms[l] (the rvm_moe_block_* transform, layer 0 included). */
typedef struct rvm_session rvm_session;
int rvm_session_create(const rvm_layer *layers, int n_layers, const rvm_block_norms *norms, int max_tokens,
                       float eps, rvm_session **out);
int rvm_session_destroy(rvm_session *session);
/* n_tok tokens (rows of x) through every layer into out: per layer only the kernels of one
 * rvm_moe_* call (3 for one token), no transfer and no host synchronisation, so the call can be
 * captured in one graph. flags: 0 or RVM_EXACT_SELECT. */
int rvm_session_eval(rvm_session *session, const float *x, float *out, int n_tok, int flags);
/* Layers [l0, l1) of the same evaluation, so that a caller can stop between ranges: the reference's
 * HipSession::eval polls its cancel closure before every layer (runtime/src/hip_exec.rs:645-655); a
 * caller polls it between ranges instead. A range from l0 = 0 starts an evaluation and reads x; any
 * other range must start where the previous range of this session ended, with the same n_tok (else
 * hipErrorInvalidValue); the range that ends at the last layer writes out (x and out may be NULL
 * where they are not read or written). The ranges of one evaluation issue exactly the kernels of
 * rvm_session_eval, so the result is the same bit for bit. A caller that stops early starts the
 * next evaluation from l0 = 0. */
int rvm_session_eval_range(rvm_session *session, const float *x, float *out, int n_tok, int flags, int l0, int l1);
/* Span events (instrumentation, the device-event mode of runtime/src/instr.rs): events[2l] is recorded
 * on the current stream before layer l's router work, events[2l + 1] once that router work is issued,
 * before its expert work, and events[2 n_layers] after the last layer; n_events = 2 n_layers + 1,
 * each from rvh_event_create. NULL turns the probe off. The spans "router" (2l to 2l + 1) and
 * "gpu_experts" (2l + 1 to 2l + 2) are then read with rvh_event_elapsed; there is no "exp_meta". */
int rvm_session_probe(rvm_session *session, void *const *events, int n_events);
/* The session's workspace (for rvm_workspace_selection / rvm_workspace_fallbacks of its last layer). */
int rvm_session_workspace(const rvm_session *session, const void **ws);

/* ---- GGUF v3 expert binding (host code; the device work is rvh_upload and rvm_pack_q4) ---- */

/* A parsed GGUF v3 image (runtime/src/gguf.rs:217-340): bounded, zero-copy (tensor views point
 * into the caller's bytes, which must outlive the handle), F32 and Q4_0 tensors only. A malformed
 * image returns hipErrorInvalidValue and rvm_gguf_last_error gives the reference's message for the
 * fault ("bad magic", "expected GGUF version 3", "truncated header", ...). */
typedef struct rvm_gguf rvm_gguf;
int rvm_gguf_open(const void *data, size_t size, rvm_gguf **out);
int rvm_gguf_close(rvm_gguf *gguf);
/* The message of this thread's last failed rvm_gguf_* call. */
const char *rvm_gguf_last_error(void);
int rvm_gguf_info(const rvm_gguf *gguf, uint32_t *version, uint32_t *alignment, uint64_t *data_offset,
                  uint64_t *n_tensors);
/* A string metadata value (e.g. general.architecture); valid while the handle lives. */
int rvm_gguf_meta_str(const rvm_gguf *gguf, const char *key, const char **value);
/* A tensor by name: type (0 F32, 2 Q4_0), rank, shape in ggml order (dimension 0 contiguous;
 * unused dimensions 1), its bytes in the image. */
int rvm_gguf_tensor(const rvm_gguf *gguf, const char *name, uint32_t *type, uint32_t *n_dims, uint64_t shape[4],
                    const void **data, size_t *bytes);
/* Binds layer `layer`'s MoE tensors to the device buffers of *layer_dst (the binding of
 * runtime/src/model.rs:33-40 at load, with the expert shapes of runtime/src/contract.rs:66-70):
 * blk.L.ffn_gate_up_exps.weight [d, 2ff, n_exp] and blk.L.ffn_down_exps.weight [ff, d, n_exp] (Q4_0)
 * are uploaded through staging (at least the larger tensor's bytes) and repacked into gate_up and
 * down; blk.L.ffn_gate_inp.weight [d, n_exp] (F32) is copied into router, and
 * blk.L.ffn_down_exps.scale [n_exp] into down_scale when that pointer is set. Shapes and types
 * must match the layer's n_exp, d and ff. Synchronises. */
int rvm_gguf_bind_moe(const rvm_gguf *gguf, int layer, const rvm_layer *layer_dst, void *staging,
                      size_t staging_bytes);

#ifdef __cplusplus
}
#endif
