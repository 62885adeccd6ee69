/* moe_oracle.c - CPU restatement of the reference's quantized MoE expert path.
 * TEST INFRASTRUCTURE ONLY; see moe_oracle.h for the rules it follows.
 * Compile with -ffp-contract=off: every multiply and add below rounds on its own. */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define Q4_BLOCK 18
#define Q8_BLOCK 34

/* Smallest normal f16 (2^-14), the clamp on the routing-weight sum: runtime/src/exec.rs:124-125. */
static const float ROUTER_SUM_MIN = 1.0f / 16384.0f;

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* runtime/src/ops.rs:7-24 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0 && man == 0) {
        bits = sign;
    } else if (exp == 0) {
        /* subnormal: normalise. leading_zeros of a 32-bit man minus 21 */
        uint32_t shift = (uint32_t)__builtin_clz(man) - 21;
        uint32_t m = (man << shift) & 0x3ff;
        bits = sign | ((113 - shift) << 23) | (m << 13);
    } else if (exp == 0x1f && man == 0) {
        bits = sign | 0x7f800000u;
    } else if (exp == 0x1f) {
        bits = sign | 0x7fc00000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    return bits_f32(bits);
}

/* runtime/src/ops.rs:27-59 */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t man = x & 0x7fffff;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (man != 0 ? 0x200 : 0));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t r = m >> shift;
        if (rem > half || (rem == half && (r & 1) == 1)) r += 1;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1) == 1)) r += 1; /* may carry into the exponent */
    return (uint16_t)(sign | r);
}

/* runtime/src/ops.rs:83-92 */
void orc_dequant_q4_0(const uint8_t *row, float *out, size_t k) {
    for (size_t b = 0; b < k / QK; ++b) {
        const uint8_t *blk = row + b * Q4_BLOCK;
        float d = orc_f16_to_f32(le16(blk));
        for (int j = 0; j < 16; ++j) {
            uint8_t q = blk[2 + j];
            out[b * QK + j] = (float)((int)(q & 15) - 8) * d;
            out[b * QK + j + 16] = (float)((int)(q >> 4) - 8) * d;
        }
    }
}

/* runtime/src/ops.rs:67-80 */
float orc_dot_q4_0(const uint8_t *row, const float *x, size_t k) {
    float acc = 0.0f;
    for (size_t b = 0; b < k / QK; ++b) {
        const uint8_t *blk = row + b * Q4_BLOCK;
        const float *xs = x + b * QK;
        float d = orc_f16_to_f32(le16(blk));
        float s = 0.0f;
        for (int j = 0; j < 16; ++j) {
            uint8_t q = blk[2 + j];
            float lo = (float)((int)(q & 15) - 8) * xs[j];
            float hi = (float)((int)(q >> 4) - 8) * xs[j + 16];
            s += lo + hi;
        }
        acc += d * s;
    }
    return acc;
}

/* runtime/src/ops.rs:249-266: dequantise each row, then a sequential f32 fold of products. */
void orc_matmul_q4_0(const uint8_t *w, size_t k, const float *x, size_t n_in, float *y, size_t n_out) {
    size_t row_bytes = k / QK * Q4_BLOCK;
    float *row = (float *)malloc(k * sizeof(float));
    for (size_t r = 0; r < n_out; ++r) {
        orc_dequant_q4_0(w + r * row_bytes, row, k);
        for (size_t t = 0; t < n_in; ++t) {
            const float *xs = x + t * k;
            float v = -0.0f;
            for (size_t i = 0; i < k; ++i) v += row[i] * xs[i];
            y[t * n_out + r] = v;
        }
    }
    free(row);
}

/* Rust `f32 as i8`: saturating, NaN to 0. */
static int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* runtime/src/ops.rs:95-105 */
void orc_quantize_q8_0(const float *x, uint8_t *out, size_t k) {
    for (size_t b = 0; b < k / QK; ++b) {
        const float *xs = x + b * QK;
        uint8_t *blk = out + b * Q8_BLOCK;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) amax = fmaxf(amax, fabsf(xs[j])); /* f32::max ignores NaN */
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = orc_f32_to_f16(d);
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < QK; ++j) blk[2 + j] = (uint8_t)sat_i8(roundf(xs[j] * id));
    }
}

/* runtime/src/expert_kernel.rs:152-157: the exact integer sum of one block. */
static int32_t block_sumi(const uint8_t *w, const uint8_t *x) {
    int32_t sumi = 0;
    for (int j = 0; j < 16; ++j) {
        uint8_t b = w[2 + j];
        sumi += ((int32_t)(b & 15) - 8) * (int32_t)(int8_t)x[2 + j];
        sumi += ((int32_t)(b >> 4) - 8) * (int32_t)(int8_t)x[18 + j];
    }
    return sumi;
}

/* runtime/src/expert_kernel.rs:147-161 */
float orc_dot_q8_scalar(const uint8_t *row, const uint8_t *xq, size_t k) {
    float acc = 0.0f;
    for (size_t b = 0; b < k / QK; ++b) {
        const uint8_t *w = row + b * Q4_BLOCK;
        const uint8_t *x = xq + b * Q8_BLOCK;
        float dw = orc_f16_to_f32(le16(w));
        float dx = orc_f16_to_f32(le16(x));
        int32_t sumi = block_sumi(w, x);
        acc += (float)sumi * (dw * dx);
    }
    return acc;
}

void orc_q4q8_block_sums(const uint8_t *row, const uint8_t *xq, size_t k, int32_t *sums) {
    for (size_t b = 0; b < k / QK; ++b) sums[b] = block_sumi(row + b * Q4_BLOCK, xq + b * Q8_BLOCK);
}

/* runtime/src/expert_kernel.rs:163-191. The 256-bit register holds the 16 low-nibble weights
 * (elements 0..15) then the 16 high-nibble weights (16..31) against activations 0..31;
 * maddubs + madd leave int32 lane m = sum of elements 4m..4m+3; each lane accumulates
 * fma(d, lane, acc); the 8 lanes are then summed in order from -0.0. */
float orc_dot_q8_avx2_order(const uint8_t *row, const uint8_t *xq, size_t k) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < k / QK; ++b) {
        const uint8_t *w = row + b * Q4_BLOCK;
        const uint8_t *x = xq + b * Q8_BLOCK;
        float d = orc_f16_to_f32(le16(w)) * orc_f16_to_f32(le16(x));
        for (int m = 0; m < 8; ++m) {
            int32_t s = 0;
            for (int i = 4 * m; i < 4 * m + 4; ++i) {
                int32_t wv = i < 16 ? (int32_t)(w[2 + i] & 15) - 8 : (int32_t)(w[2 + i - 16] >> 4) - 8;
                s += wv * (int32_t)(int8_t)x[2 + i];
            }
            acc[m] = fmaf(d, (float)s, acc[m]);
        }
    }
    float sum = -0.0f;
    for (int m = 0; m < 8; ++m) sum += acc[m];
    return sum;
}

/* runtime/src/ops.rs:321-326 */
void orc_matvec_f32(const float *w, size_t k, const float *x, float *y, size_t n_out) {
    for (size_t r = 0; r < n_out; ++r) {
        const float *row = w + r * k;
        float s = -0.0f;
        for (size_t i = 0; i < k; ++i) s += row[i] * x[i];
        y[r] = s;
    }
}

/* runtime/src/ops.rs:131-139 (f64 sum of squares) with rvhip.h:42's post factor. */
void orc_rms_norm(float *x, const float *weight, size_t n, float eps, float post) {
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) sum += (double)x[i] * (double)x[i];
    float mean = (float)(sum / (double)n);
    float scale = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; ++i) {
        float v = x[i] * scale;
        if (post != 1.0f) v = v * post;
        if (weight) v = v * weight[i];
        x[i] = v;
    }
}

/* runtime/src/ops.rs:145-149: 0.5 * x * (1 + tanh(S * x * (1 + A * x * x))), left to right. */
float orc_gelu(float x) {
    const float A = 0.044715f;
    const float S = 0.7978846f;
    float inner = S * x * (1.0f + A * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

/* runtime/src/exec.rs:606-611 */
void orc_geglu_split(const float *gu, float *out, size_t rows, size_t ff) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t j = 0; j < ff; ++j) out[r * ff + j] = orc_gelu(gu[r * 2 * ff + j]) * gu[r * 2 * ff + ff + j];
}

/* runtime/src/ops.rs:170-179 */
void orc_softmax(float *x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = fmaxf(max, x[i]);
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - max);
        sum += (double)x[i];
    }
    float inv = (float)(1.0 / sum);
    for (size_t i = 0; i < n; ++i) x[i] *= inv;
}

/* runtime/src/ops.rs:107-118: per block d * (sequential f32 fold of q * x), folded in block order. */
float orc_dot_q8_0(const uint8_t *row, const float *x, size_t k) {
    float acc = 0.0f;
    for (size_t b = 0; b < k / QK; ++b) {
        const uint8_t *blk = row + b * Q8_BLOCK;
        const float *xs = x + b * QK;
        float d = orc_f16_to_f32(le16(blk));
        float s = -0.0f;
        for (int j = 0; j < QK; ++j) s += (float)(int8_t)blk[2 + j] * xs[j];
        acc += d * s;
    }
    return acc;
}

/* runtime/src/ops.rs:120-128: out += q * (d * w), element by element. */
void orc_axpy_q8_0(const uint8_t *row, float w, float *out, size_t k) {
    for (size_t b = 0; b < k / QK; ++b) {
        const uint8_t *blk = row + b * Q8_BLOCK;
        float d = orc_f16_to_f32(le16(blk)) * w;
        for (int j = 0; j < QK; ++j) out[b * QK + j] += (float)(int8_t)blk[2 + j] * d;
    }
}

/* runtime/tests/hip_ops.rs:245-271 (the CPU attention the reference's kernels are checked
 * against): query t at position p0 + t, keys lo..pos with lo = pos + 1 - win saturated at 0
 * (win > 0) or 0, key p in ring row ((p % cap) * nkv + g) for g = h / (nh / nkv); scores
 * dot_q8_0, softmax, then out = sum of axpy_q8_0 in key order from zero. */
void orc_attention(const float *q, const uint8_t *kc, const uint8_t *vc, size_t nh, size_t nkv, size_t hd,
                   size_t cap, size_t win, size_t p0, size_t n, float *out) {
    size_t row = hd / QK * Q8_BLOCK;
    float *sc = (float *)malloc((p0 + n) * sizeof(float));
    memset(out, 0, n * nh * hd * sizeof(float));
    for (size_t t = 0; t < n; ++t) {
        size_t pos = p0 + t;
        size_t lo = win > 0 ? (pos + 1 > win ? pos + 1 - win : 0) : 0;
        for (size_t h = 0; h < nh; ++h) {
            size_t g = h / (nh / nkv);
            const float *qh = q + (t * nh + h) * hd;
            for (size_t p = lo; p <= pos; ++p) sc[p - lo] = orc_dot_q8_0(kc + ((p % cap) * nkv + g) * row, qh, hd);
            orc_softmax(sc, pos - lo + 1);
            float *o = out + (t * nh + h) * hd;
            for (size_t p = lo; p <= pos; ++p) orc_axpy_q8_0(vc + ((p % cap) * nkv + g) * row, sc[p - lo], o, hd);
        }
    }
    free(sc);
}

/* runtime/tests/hip_ops.rs:9-22: the reference tests' xorshift64 generator. unit() maps the top
 * 24 bits of each state to [-1, 1); vec(n, scale) is n of unit() * scale. */
void orc_test_rng_vec(uint64_t *state, size_t n, float scale, float *out) {
    uint64_t s = *state;
    for (size_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        float u = (float)(s >> 40) / 16777216.0f * 2.0f - 1.0f;
        out[i] = u * scale;
    }
    *state = s;
}

/* Rust f32::total_cmp key (IEEE 754 totalOrder as a signed integer). */
static int32_t total_key(float f) {
    int32_t i = (int32_t)f32_bits(f);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return i;
}

/* runtime/src/ops.rs:182-187: descending by total_cmp, ties to the lower index. The order is
 * total, so k rounds of "pick the first maximum" equal the reference's sort-then-truncate. */
void orc_top_k(const float *x, size_t n, size_t k, uint32_t *out) {
    unsigned char *taken = (unsigned char *)calloc(n, 1);
    for (size_t j = 0; j < k && j < n; ++j) {
        size_t best = n;
        for (size_t i = 0; i < n; ++i) {
            if (taken[i]) continue;
            if (best == n || total_key(x[i]) > total_key(x[best])) best = i;
        }
        taken[best] = 1;
        out[j] = (uint32_t)best;
    }
    free(taken);
}

void orc_router_logits(const float *w_r, const float *bias, const float *x, size_t n_tok, size_t n_exp, size_t d,
                       float *logits) {
    for (size_t t = 0; t < n_tok; ++t) {
        orc_matvec_f32(w_r, d, x + t * d, logits + t * n_exp, n_exp);
        if (bias)
            for (size_t e = 0; e < n_exp; ++e) logits[t * n_exp + e] += bias[e];
    }
}

/* runtime/src/exec.rs:507-517 */
void orc_select_experts(float *logits, size_t n_tok, size_t n_exp, size_t used, uint32_t *ids, float *weights) {
    for (size_t t = 0; t < n_tok; ++t) {
        float *lg = logits + t * n_exp;
        uint32_t *top = ids + t * used;
        orc_softmax(lg, n_exp);
        orc_top_k(lg, n_exp, used, top);
        float sum = -0.0f;
        for (size_t j = 0; j < used; ++j) sum += lg[top[j]];
        sum = fmaxf(sum, ROUTER_SUM_MIN);
        for (size_t j = 0; j < used; ++j) weights[t * used + j] = lg[top[j]] / sum;
    }
}

/* runtime/src/exec.rs:540-558: a stable counting sort by expert is the sort by (expert, pair). */
void orc_moe_plan(const uint32_t *ids, size_t pairs, size_t n_exp, uint32_t *order, uint32_t *pos_of,
                  uint32_t *group_start) {
    for (size_t e = 0; e <= n_exp; ++e) group_start[e] = 0;
    for (size_t i = 0; i < pairs; ++i) group_start[ids[i] + 1]++;
    for (size_t e = 0; e < n_exp; ++e) group_start[e + 1] += group_start[e];
    uint32_t *fill = (uint32_t *)malloc((n_exp + 1) * sizeof(uint32_t));
    memcpy(fill, group_start, (n_exp + 1) * sizeof(uint32_t));
    for (size_t i = 0; i < pairs; ++i) {
        uint32_t k = fill[ids[i]]++;
        order[k] = (uint32_t)i;
        pos_of[i] = k;
    }
    free(fill);
}

/* runtime/src/exec.rs:572-640 in the Q8_0 domain. */
int orc_experts_q8(const uint8_t *const *gate_up, const uint8_t *const *down, const float *down_scale,
                   const float *moe_in, size_t n_tok, size_t d, size_t ff, size_t used, const uint32_t *ids,
                   const float *weights, float *out, float *gu_out, float *h_out, float *y_out) {
    size_t pairs = n_tok * used;
    size_t gu_rows = 2 * ff;
    size_t gu_row_bytes = d / QK * Q4_BLOCK;
    size_t dn_row_bytes = ff / QK * Q4_BLOCK;
    size_t n_exp = 0;
    for (size_t i = 0; i < pairs; ++i)
        if (ids[i] + 1 > n_exp) n_exp = ids[i] + 1;
    uint32_t *order = (uint32_t *)malloc(pairs * sizeof(uint32_t));
    uint32_t *pos_of = (uint32_t *)malloc(pairs * sizeof(uint32_t));
    uint32_t *gs = (uint32_t *)malloc((n_exp + 1) * sizeof(uint32_t));
    float *gu = (float *)malloc(pairs * gu_rows * sizeof(float));
    float *h = (float *)malloc(pairs * ff * sizeof(float));
    float *y = (float *)malloc(pairs * d * sizeof(float));
    uint8_t *xq = (uint8_t *)malloc(d / QK * Q8_BLOCK);
    uint8_t *hq = (uint8_t *)malloc(ff / QK * Q8_BLOCK);
    int rc = 0;
    orc_moe_plan(ids, pairs, n_exp, order, pos_of, gs);
    for (size_t i = 0; i < pairs && rc == 0; ++i)
        if (!gate_up[ids[i]] || !down[ids[i]]) rc = -1;
    if (rc == 0) {
        /* gather (exec.rs:585-588) + gate_up segments: each activation row is quantised once
         * (expert_pool.rs:311-320), then every weight row is dot_q8 against it. */
        for (size_t k = 0; k < pairs; ++k) {
            size_t t = order[k] / used;
            uint32_t ex = ids[order[k]];
            orc_quantize_q8_0(moe_in + t * d, xq, d);
            for (size_t r = 0; r < gu_rows; ++r)
                gu[k * gu_rows + r] = orc_dot_q8_scalar(gate_up[ex] + r * gu_row_bytes, xq, d);
        }
        /* GeGLU (exec.rs:606-611) */
        for (size_t k = 0; k < pairs; ++k)
            for (size_t j = 0; j < ff; ++j) h[k * ff + j] = orc_gelu(gu[k * gu_rows + j]) * gu[k * gu_rows + ff + j];
        /* down segments (exec.rs:612-625) */
        for (size_t k = 0; k < pairs; ++k) {
            uint32_t ex = ids[order[k]];
            orc_quantize_q8_0(h + k * ff, hq, ff);
            for (size_t r = 0; r < d; ++r) y[k * d + r] = orc_dot_q8_scalar(down[ex] + r * dn_row_bytes, hq, ff);
        }
        /* slot-order combine (exec.rs:626-638): first term assigned, then added. */
        for (size_t t = 0; t < n_tok; ++t) {
            float *o = out + t * d;
            for (size_t j = 0; j < used; ++j) {
                uint32_t ex = ids[t * used + j];
                float wt = weights[t * used + j];
                const float *yy = y + (size_t)pos_of[t * used + j] * d;
                float ds = down_scale ? down_scale[ex] : 1.0f;
                if (j == 0)
                    for (size_t i = 0; i < d; ++i) o[i] = yy[i] * ds * wt;
                else
                    for (size_t i = 0; i < d; ++i) o[i] += yy[i] * ds * wt;
            }
        }
        if (gu_out) memcpy(gu_out, gu, pairs * gu_rows * sizeof(float));
        if (h_out) memcpy(h_out, h, pairs * ff * sizeof(float));
        if (y_out) memcpy(y_out, y, pairs * d * sizeof(float));
    }
    free(order);
    free(pos_of);
    free(gs);
    free(gu);
    free(h);
    free(y);
    free(xq);
    free(hq);
    return rc;
}

int orc_moe_layer(const float *w_r, const float *bias, const uint8_t *const *gate_up, const uint8_t *const *down,
                  const float *down_scale, const float *x, size_t n_tok, size_t n_exp, size_t d, size_t ff,
                  size_t used, int pre_norm, float eps, uint32_t *ids, float *weights, float *out) {
    float *xin = (float *)malloc(n_tok * d * sizeof(float));
    float *logits = (float *)malloc(n_tok * n_exp * sizeof(float));
    memcpy(xin, x, n_tok * d * sizeof(float));
    if (pre_norm)
        for (size_t t = 0; t < n_tok; ++t) orc_rms_norm(xin + t * d, NULL, d, eps, 1.0f);
    orc_router_logits(w_r, bias, xin, n_tok, n_exp, d, logits);
    orc_select_experts(logits, n_tok, n_exp, used, ids, weights);
    int rc = orc_experts_q8(gate_up, down, down_scale, xin, n_tok, d, ff, used, ids, weights, out, NULL, NULL, NULL);
    free(xin);
    free(logits);
    return rc;
}
