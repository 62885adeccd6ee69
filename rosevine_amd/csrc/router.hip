// router.hip - router logits, softmax/top-k selection with an exactness guard, and the stable
// device grouping of (token, slot) pairs by expert.
//
// The reference logit is a sequential f32 fold of d f32 products, W_r[e][i] * x[i]
// (runtime/src/ops.rs:321-326, called from runtime/src/exec.rs:493-503). The router kernel
// computes, per expert, S = the sum of the same f32 products in f64 (one wave per expert, lanes
// own contiguous chunks, a wave scan joins them) and a bound on the fold's rounding error:
//     |fold - S| <= u/(1-u) * sum_i |s_i| / (1 - d*u/(1-u)),  u = 2^-24,
// where s_i are the exact prefix sums. Selection (runtime/src/exec.rs:507-517: softmax, top_k by
// total_cmp with ties to the lower index, weights renormalised with the 2^-14 clamp) is done by
// the last workgroup to finish a token. If the intervals [S - eps, S + eps] of the top k + 1
// experts are separated by a margin that keeps expf and the 1/sum product order-preserving, the
// reference's ids are certified and taken from S; otherwise (and under RVM_EXACT_SELECT) the
// selecting workgroup recomputes every logit in the reference's order and selects exactly.
#include <math.h>

#include "internal.hpp"

namespace rvm {

constexpr int RWAVES = 4;  // waves (experts) per router workgroup

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ double wave_max_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Block reductions over 256 threads in a fixed order (deterministic).
__device__ double block_sum_d(double v, double *sh) {
    v = wave_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((sh[0] + sh[1]) + sh[2]) + sh[3];
}

__device__ double block_max_d(double v, double *sh) {
    v = wave_max_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmax(fmax(sh[0], sh[1]), fmax(sh[2], sh[3]));
}

__device__ float block_max_f(float v, float *sh) {
    v = wave_max_f(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
}

// Rust f32::total_cmp key.
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t i = __builtin_bit_cast(int32_t, f);
    return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// Margin that keeps p_a > p_b whenever R_a - R_b exceeds it: covers the rounding of R - max,
// expf's error (< 1 ulp) and the rounding of the product with 1/sum.
__device__ __forceinline__ double order_margin(double a, double b, double m) {
    return 1e-6 + 0x1p-22 * (fabs(a) + fabs(b) + 2.0 * fabs(m));
}

// The layer input element i of this token: rms_norm'ed when pre-normalisation is on.
__device__ __forceinline__ float xin(const float *xt, int i, float scale, int pre_norm) {
    return pre_norm ? xt[i] * scale : xt[i];
}

// Selection for one token by the 256 threads of the last router workgroup (thread e = expert e).
__device__ void select_token(const double2 *st, const float *__restrict__ bias, const float *__restrict__ W,
                             const float *xt, float scale, int pre_norm, int n_exp, int d, int top_k, int exact,
                             uint32_t *ctl, int32_t *ids, float *wts, float *logits) {
    __shared__ double sS[256], sE[256];
    __shared__ double red_d[4];
    __shared__ float red_f[4];
    __shared__ float sp[256];
    __shared__ int sel[8];
    __shared__ int pass;
    __shared__ float inv_s;
    const int t = threadIdx.x;
    const bool present = t < n_exp;
    double Sv = -INFINITY, Ev = 0.0;
    bool bad = false;
    if (present) {
        const double2 v = st[t];
        Sv = v.x;
        Ev = v.y;
        if (bias) {
            const double s2 = Sv + (double)bias[t];
            Ev = Ev + (fabs(s2) + Ev) * 0x1p-23;  // the f32 rounding of logit + bias
            Sv = s2;
        }
        bad = !isfinite(Sv) || !isfinite(Ev);
    }
    sS[t] = Sv;
    sE[t] = Ev;
    if (t == 0) pass = exact ? 0 : 1;
    __syncthreads();
    if (bad) pass = 0;
    // rank by (S desc, index asc)
    int rank = 256;
    if (present) {
        rank = 0;
        for (int j = 0; j < n_exp; ++j) {
            const double o = sS[j];
            rank += (o > Sv) || (o == Sv && j < t);
        }
        if (rank < top_k) sel[rank] = t;
    }
    const double M = block_max_d(present ? Sv : -INFINITY, red_d);
    const double U = block_max_d(present && rank >= top_k ? Sv + Ev : -INFINITY, red_d);
    // Guard: every selected lower bound clears the next selected upper bound, and the last one
    // clears every unselected upper bound, by the order-preserving margin.
    if (t == 0 && pass) {
        int ok = 1;
        for (int i = 0; i < top_k && ok; ++i) {
            const int a = sel[i];
            const double lo = sS[a] - sE[a];
            double hi, sb;
            if (i + 1 < top_k) {
                const int b = sel[i + 1];
                hi = sS[b] + sE[b];
                sb = sS[b];
            } else {
                hi = U;
                sb = isfinite(U) ? U : 0.0;
            }
            if (!(lo - order_margin(sS[a], sb, M) > hi)) ok = 0;
        }
        if (ok && !(sS[sel[top_k - 1]] - M > -80.0)) ok = 0;  // clear of expf underflow
        pass = ok;
    }
    __syncthreads();

    if (pass) {
        // Certified ids. Weights from the f32-rounded estimates (tolerance class).
        const float R = present ? (float)Sv : -INFINITY;
        const float Mf = block_max_f(R, red_f);
        const float ex = present ? expf(R - Mf) : 0.0f;
        const double sum = block_sum_d((double)ex, red_d);
        const float inv = (float)(1.0 / sum);
        sp[t] = ex * inv;
        if (logits && present) logits[t] = R;
    } else {
        if (t == 0) atomicAdd(&ctl[0], 1u);
        // Reference order: sequential f32 fold of f32 products from -0.0, then + bias.
        float R = -INFINITY;
        if (present) {
            const float *wr = W + (size_t)t * d;
            float acc = -0.0f;
            for (int i = 0; i < d; ++i) acc = acc + wr[i] * xin(xt, i, scale, pre_norm);
            if (bias) acc = acc + bias[t];
            R = acc;
        }
        // softmax (runtime/src/ops.rs:170-179): max ignoring NaN, f32 z, exp, f64 sum in index order
        const float Mf = block_max_f(R, red_f);
        const float z = R - Mf;
        const float ex = present ? (float)exp((double)z) : 0.0f;
        sp[t] = ex;
        if (logits && present) logits[t] = R;
        __syncthreads();
        if (t == 0) {
            double sum = 0.0;
            for (int j = 0; j < n_exp; ++j) sum += (double)sp[j];
            inv_s = (float)(1.0 / sum);
        }
        __syncthreads();
        const float p = present ? ex * inv_s : 0.0f;
        sp[t] = p;
        __syncthreads();
        // top_k by total_cmp desc, index asc (runtime/src/ops.rs:182-187)
        if (present) {
            const int32_t kp = total_key(p);
            int r = 0;
            for (int j = 0; j < n_exp; ++j) {
                const int32_t kj = total_key(sp[j]);
                r += (kj > kp) || (kj == kp && j < t);
            }
            if (r < top_k) sel[r] = t;
        }
    }
    __syncthreads();
    if (t == 0) {
        float s = -0.0f;
        for (int j = 0; j < top_k; ++j) s = s + sp[sel[j]];
        s = fmaxf(s, 1.0f / 16384.0f);
        for (int j = 0; j < top_k; ++j) {
            ids[j] = sel[j];
            wts[j] = sp[sel[j]] / s;
        }
    }
}

__global__ __launch_bounds__(256) void k_router(const float *__restrict__ W, const float *__restrict__ bias,
                                                const float *__restrict__ x, int n_exp, int d, int top_k,
                                                int pre_norm, float eps, int exact, double2 *__restrict__ stats,
                                                uint32_t *__restrict__ xact, uint32_t *__restrict__ tokctr,
                                                uint32_t *__restrict__ ctl, int32_t *__restrict__ ids,
                                                float *__restrict__ wts, float *__restrict__ logits) {
    __shared__ double red[4];
    __shared__ unsigned last;
    const int tok = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float *xt = x + (size_t)tok * d;

    float scale = 1.0f;
    if (pre_norm) {  // runtime/src/ops.rs:131-139: f64 sum of squares, mean as f32, 1/sqrt(mean+eps)
        double s = 0.0;
        for (int i = threadIdx.x; i < d; i += 256) s += (double)xt[i] * (double)xt[i];
        s = block_sum_d(s, red);
        const float mean = (float)(s / (double)d);
        scale = 1.0f / sqrtf(mean + eps);
    }

    // Logit statistics: one wave per expert; lane owns elements [lane*C, lane*C + C).
    const int C = d / 64;
    const int e = blockIdx.x * RWAVES + w;
    if (e < n_exp) {
        const float *wr = W + (size_t)e * d + (size_t)lane * C;
        const float *xr = xt + (size_t)lane * C;
        double c = 0.0;
        for (int i = 0; i < C; i += 4) {
            const float4 wv = *(const float4 *)(wr + i);
            float4 xv = *(const float4 *)(xr + i);
            if (pre_norm) xv = make_float4(xv.x * scale, xv.y * scale, xv.z * scale, xv.w * scale);
            c += (double)(wv.x * xv.x);
            c += (double)(wv.y * xv.y);
            c += (double)(wv.z * xv.z);
            c += (double)(wv.w * xv.w);
        }
        double incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const double n = __shfl_up(incl, o);
            if (lane >= o) incl += n;
        }
        double run = __shfl_up(incl, 1);
        if (lane == 0) run = 0.0;
        const double total = __shfl(incl, 63);
        double babs = 0.0;
        for (int i = 0; i < C; i += 4) {
            const float4 wv = *(const float4 *)(wr + i);
            float4 xv = *(const float4 *)(xr + i);
            if (pre_norm) xv = make_float4(xv.x * scale, xv.y * scale, xv.z * scale, xv.w * scale);
            run += (double)(wv.x * xv.x);
            babs += fabs(run);
            run += (double)(wv.y * xv.y);
            babs += fabs(run);
            run += (double)(wv.z * xv.z);
            babs += fabs(run);
            run += (double)(wv.w * xv.w);
            babs += fabs(run);
        }
        babs = wave_sum_d(babs);
        if (lane == 0) {
            const double u = 0x1p-24, g = u / (1.0 - u);
            const double bound = babs * g / (1.0 - (double)d * g) * (1.0 + 0x1p-20) + 1e-300;
            stats[(size_t)tok * n_exp + e] = make_double2(total, bound);
        }
    }

    // Q8_0 quantisation of the layer input, one 32-block per half-wave (runtime/src/ops.rs:95-105).
    const int nb = d / QK;
    const int hw_total = gridDim.x * RWAVES * 2;
    for (int base = (blockIdx.x * RWAVES + w) * 2; base < nb; base += hw_total) {
        const int hb = base + (lane >> 5);
        const int j = lane & 31;
        const bool ok = hb < nb;
        const float v = ok ? xin(xt, hb * QK + j, scale, pre_norm) : 0.0f;
        uint16_t dbits;
        const int q = quant_q8_half(v, &dbits);
        store_prep_half(q, dbits, j, xact + ((size_t)tok * nb + (ok ? hb : 0)) * ACT_DW, ok);
    }

    // The last workgroup of this token selects (the counter is left at zero for the next call).
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(&tokctr[tok], 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    select_token(stats + (size_t)tok * n_exp, bias, W, xt, scale, pre_norm, n_exp, d, top_k, exact, ctl,
                 ids + (size_t)tok * top_k, wts + (size_t)tok * top_k, logits ? logits + (size_t)tok * n_exp : nullptr);
    if (threadIdx.x == 0) tokctr[tok] = 0;
}

// Stable counting sort of pair ids by expert in one workgroup of 16 waves: wave w owns a
// contiguous chunk of pairs; per-(wave, expert) counts are scanned in (expert, wave) order, then
// each wave places its pairs 64 at a time, ranking equal experts among lower lanes with ballots.
// Ids outside [0, n_exp) are neither counted nor placed (pos_of = -1).
__global__ __launch_bounds__(1024) void k_plan(const int32_t *__restrict__ ids, int n, int n_exp,
                                               int32_t *__restrict__ order, int32_t *__restrict__ pos_of,
                                               int32_t *__restrict__ gstart) {
    __shared__ int cnt[16][256];
    __shared__ int tot[257];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int i = threadIdx.x; i < 16 * 256; i += 1024) (&cnt[0][0])[i] = 0;
    __syncthreads();
    const int chunk = ((n + 15) / 16 + 63) / 64 * 64;
    const int lo = w * chunk, hi = min(n, lo + chunk);
    for (int i = lo + lane; i < hi; i += 64) {
        const int e = ids[i];
        if (e >= 0 && e < n_exp) atomicAdd(&cnt[w][e], 1);
    }
    __syncthreads();
    if ((int)threadIdx.x < n_exp) {
        int s = 0;
        for (int ww = 0; ww < 16; ++ww) s += cnt[ww][threadIdx.x];
        tot[threadIdx.x] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int e = 0; e < n_exp; ++e) {
            const int c = tot[e];
            tot[e] = run;
            run += c;
        }
        tot[n_exp] = run;
    }
    __syncthreads();
    if ((int)threadIdx.x <= n_exp) gstart[threadIdx.x] = tot[threadIdx.x];
    if ((int)threadIdx.x < n_exp) {
        int run = tot[threadIdx.x];
        for (int ww = 0; ww < 16; ++ww) {
            const int c = cnt[ww][threadIdx.x];
            cnt[ww][threadIdx.x] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int base = lo; base < hi; base += 64) {
        const int i = base + lane;
        const int raw = i < hi ? ids[i] : -1;
        const bool valid = raw >= 0 && raw < n_exp;
        const int e = valid ? raw : 0;
        if (i < hi && !valid) pos_of[i] = -1;  // an id outside [0, n_exp) is left out of the plan
        uint64_t m = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool set = (e >> bit) & 1;
            const uint64_t b = __ballot(valid && set);
            m &= set ? b : ~b;
        }
        if (valid) {
            const uint64_t below = (1ull << lane) - 1ull;
            const int pos = cnt[w][e] + __popcll(m & below);
            order[pos] = i;
            pos_of[i] = pos;
            if ((m >> lane) == 1ull) cnt[w][e] = pos + 1;  // highest lane of its group
        }
    }
}

int launch_router(const rvm_layer *L, const float *x, int n_tok, int flags, float eps, uint8_t *ws,
                  const WsLayout &lay, int32_t *ids, float *wts, float *logits) {
    const int groups = grid_blocks(L->n_exp, RWAVES);
    hipLaunchKernelGGL(k_router, dim3(groups, n_tok), dim3(256), 0, cur_stream(), L->router, L->router_bias, x,
                       L->n_exp, L->d, L->top_k, (flags & RVM_PRE_NORM) ? 1 : 0, eps,
                       (flags & RVM_EXACT_SELECT) ? 1 : 0, (double2 *)(ws + lay.stats), (uint32_t *)(ws + lay.xact),
                       (uint32_t *)(ws + lay.tokctr), (uint32_t *)(ws + lay.ctl), ids, wts, logits);
    return launched();
}

int launch_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of, int32_t *gstart) {
    hipLaunchKernelGGL(k_plan, dim3(1), dim3(1024), 0, cur_stream(), ids, n_pairs, n_exp, order, pos_of, gstart);
    return launched();
}

}  // namespace rvm

using namespace rvm;

extern "C" {

int rvm_router_select(const rvm_layer *layer, const float *x, int n_tok, int flags, float eps, int32_t *ids,
                      float *weights, float *logits, void *ws, size_t ws_bytes) {
    RVM_CHECK(layer_ok(layer) && x && n_tok > 0 && n_tok <= 65535 && ids && weights && ws);
    const WsLayout lay = ws_layout(layer, n_tok);
    RVM_CHECK(ws_bytes >= lay.total);
    return launch_router(layer, x, n_tok, flags, eps, (uint8_t *)ws, lay, ids, weights, logits);
}

int rvm_moe_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of, int32_t *group_start) {
    RVM_CHECK(ids && order && pos_of && group_start && n_pairs > 0 && n_exp > 0 && n_exp <= 256);
    return launch_plan(ids, n_pairs, n_exp, order, pos_of, group_start);
}

}  // extern "C"
