// router.hip - router logits, softmax/top-k selection with an exactness certificate, and the
// stable device grouping of (token, slot) pairs by expert.
//
// The reference logit is a sequential f32 fold of d f32 products, W_r[e][i] * x[i]
// (runtime/src/ops.rs:321-326, called from runtime/src/exec.rs:493-503). k_router computes, per
// expert, S = the sum of the same f32 products in f64 (one wave per expert, lanes own contiguous
// chunks, a wave scan joins them) and a bound on the fold's rounding error:
//     |fold - S| <= u/(1-u) * sum_i |s_i| / (1 - d*u/(1-u)),  u = 2^-24,
// where s_i are the exact prefix sums; it also quantises the token to Q8_0 activation blocks.
//
// k_select (one workgroup per token) implements runtime/src/exec.rs:507-517 (softmax; top_k by
// total_cmp with ties to the lower index; weights renormalised with the 2^-14 clamp). One wave
// ranks the experts by S and checks that the intervals [S - eps, S + eps] of the selected experts
// and the best unselected one are separated by a margin that keeps expf and the 1/sum product
// order-preserving: then the reference's ids are certified. Otherwise the workgroup recomputes,
// in the reference's order, the logits of every expert that could still be selected (one wave per
// expert: one coalesced row load, then a single lane folds the products); if even the exact values
// are closer than the margin, every logit and the softmax are recomputed exactly.
#include <math.h>

#include "internal.hpp"

namespace rvm {

constexpr int RWAVES = 4;    // waves (experts) per router workgroup
constexpr int SEL_WAVES = 8; // waves of the selecting workgroup

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

// Orders LDS traffic between lanes of one wave (a wave's LDS operations complete in issue order).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Rust f32::total_cmp key, and an unsigned key with the same order (for packed ranking).
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t i = __builtin_bit_cast(int32_t, f);
    return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}
__device__ __forceinline__ uint32_t order_key(float f) { return (uint32_t)total_key(f) ^ 0x80000000u; }

// Margin that keeps p_a > p_b whenever R_a - R_b exceeds it: covers the rounding of R - max,
// expf's error (< 1 ulp) and the rounding of the product with 1/sum.
__device__ __forceinline__ double order_margin(double a, double b, double m) {
    return 1e-6 + 0x1p-22 * (fabs(a) + fabs(b) + 2.0 * fabs(m));
}

// Max of a u32 over the 64 lanes of a wave (all lanes active): DPP within each row of 16 lanes
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror), then the four row
// results through readlane. The result is wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xb1, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4e, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xf, 0xf, false));
    const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return max(max(a, b), max(c, d));
}

// Inverse of order_key.
__device__ __forceinline__ float key_float(uint32_t k) {
    const int32_t t = (int32_t)(k ^ 0x80000000u);
    return __builtin_bit_cast(float, t ^ (int32_t)(((uint32_t)(t >> 31)) >> 1));
}

// The smallest f32 >= v (v finite or infinite, not NaN).
__device__ __forceinline__ float round_up_f32(double v) {
    float f = (float)v;
    if ((double)f < v) {
        const uint32_t b = __builtin_bit_cast(uint32_t, f);
        f = __builtin_bit_cast(float, f >= 0.0f ? b + 1u : b - 1u);
    }
    return f;
}

// Top n of a wave's keys (lane l holds experts l + 64 i in k[i]; alive[i] false for experts out
// of range), descending by key, equal keys by ascending index: n rounds of a wave max and a ballot
// for the lowest index holding it. The chosen experts leave alive[] and get their rank in rk[]
// (255 for the others); lane 0 writes them to sel[0..n).
__device__ __forceinline__ void wave_top_k(const uint32_t (&k)[4], bool (&alive)[4], int n, int (&rk)[4], int *sel) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; ++i) rk[i] = 255;
    for (int r = 0; r < n; ++r) {
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (alive[i]) m = max(m, k[i]);
        m = wave_max_u32(m);
        int e = -1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t b = __ballot(alive[i] && k[i] == m);
            if (e < 0 && b) e = 64 * i + (int)__builtin_ctzll(b);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (64 * i + lane == e) {
                alive[i] = false;
                rk[i] = r;
            }
        if (lane == 0) sel[r] = e;
    }
}

// This lane's chunk of the layer input, x or rms_norm(x) (runtime/src/ops.rs:131-139: f64 sum of
// squares, mean as f32, 1/sqrt(mean + eps)); every wave that calls this computes the same scale.
template <int F4>
__device__ __forceinline__ float load_x_chunk(const float *xt, int lane, int pre_norm, float eps, float4 (&xv)[F4]) {
    const float4 *x4 = (const float4 *)xt + lane * F4;
#pragma unroll
    for (int i = 0; i < F4; ++i) xv[i] = x4[i];
    float scale = 1.0f;
    if (pre_norm) {
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < F4; ++i)
            s += (double)xv[i].x * (double)xv[i].x + (double)xv[i].y * (double)xv[i].y +
                 (double)xv[i].z * (double)xv[i].z + (double)xv[i].w * (double)xv[i].w;
        s = wave_sum_d(s);  // the same value in every lane
        // The reference sums sequentially. Both sums are within d * 2^-53 * s of the exact one, so
        // the f32 mean is the reference's unless it sits at an f32 rounding boundary; then the
        // sum is redone in the reference's order.
        const double n = 256.0 * F4, bnd = s * (2.0 * n * 0x1p-53) * 1.01;
        if ((float)((s - bnd) / n) != (float)((s + bnd) / n)) {
            s = 0.0;
            for (int i = 0; i < 256 * F4; ++i) {
                const double v = (double)xt[i];
                s += v * v;
            }
        }
        const float mean = (float)(s / (double)(256 * F4));
        scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int i = 0; i < F4; ++i) xv[i] = make_float4(xv[i].x * scale, xv[i].y * scale, xv[i].z * scale, xv[i].w * scale);
    }
    return scale;
}

// F4 = d / 256: lane l owns elements [4*F4*l, 4*F4*(l+1)) of a router row.
template <int F4>
__global__ __launch_bounds__(256) void k_router(const float *__restrict__ W, const float *__restrict__ x, int n_exp,
                                                int pre_norm, float eps, double2 *__restrict__ stats,
                                                uint32_t *__restrict__ xact) {
    constexpr int d = 256 * F4, C = 4 * F4, nb = d / QK;
    const int tok = blockIdx.y;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const float *xt = x + (size_t)tok * d;
    const int e = blockIdx.x * RWAVES + w;
    const bool have = e < n_exp;

    // All loads first: the row chunk, the x chunk, and this lane's quantisation element.
    float4 wv[F4];
    const float4 *w4 = (const float4 *)(W + (size_t)(have ? e : 0) * d) + lane * F4;
#pragma unroll
    for (int i = 0; i < F4; ++i) wv[i] = w4[i];
    const int hw_total = gridDim.x * RWAVES * 2;
    const int base0 = (blockIdx.x * RWAVES + w) * 2;
    const int j = lane & 31;
    const int hb0 = base0 + (lane >> 5);
    const float qv0 = hb0 < nb ? xt[hb0 * QK + j] : 0.0f;
    float4 xv[F4];
    const float scale = load_x_chunk<F4>(xt, lane, pre_norm, eps, xv);

    if (have) {
        float p[C];
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            p[4 * i] = wv[i].x * xv[i].x;
            p[4 * i + 1] = wv[i].y * xv[i].y;
            p[4 * i + 2] = wv[i].z * xv[i].z;
            p[4 * i + 3] = wv[i].w * xv[i].w;
        }
        double c = 0.0;
#pragma unroll
        for (int i = 0; i < C; ++i) c += (double)p[i];
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
#pragma unroll
        for (int i = 0; i < C; ++i) {
            run += (double)p[i];
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
    for (int base = base0; base < nb; base += hw_total) {
        const int hb = base + (lane >> 5);
        const bool ok = hb < nb;
        float v = base == base0 ? qv0 : (ok ? xt[hb * QK + j] : 0.0f);
        if (pre_norm) v = v * scale;
        uint16_t dbits;
        const int q = quant_q8_half(v, &dbits);
        store_prep_half(q, dbits, j, xact + ((size_t)tok * nb + (ok ? hb : 0)) * ACT_DW, ok);
    }
}

// Exact reference-order logits of cand[0..nc) into R[cand[c]]: wave w folds candidate c0 + w of
// each round. The wave loads the row (coalesced) and forms the f32 products as k_router does; the
// products then pass through LDS a quarter row at a time and lane 0 folds them in element order
// from -0.0 (runtime/src/ops.rs:324), then adds the bias.
template <int F4>
__device__ void exact_fold(const float *__restrict__ W, const float *__restrict__ bias, const float4 (&xv)[F4],
                           const int *cand, int nc, float *R, float *fold) {
    constexpr int C = 4 * F4, Q = 16 * C;  // products per quarter row
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    float *buf = fold + w * Q;
    for (int c0 = 0; c0 < nc; c0 += SEL_WAVES) {
        const int c = c0 + w;
        const int e = c < nc ? cand[c] : cand[0];
        float4 wv[F4];
        const float4 *w4 = (const float4 *)(W + (size_t)e * (256 * F4)) + lane * F4;
#pragma unroll
        for (int i = 0; i < F4; ++i) wv[i] = w4[i];
        float p[C];
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            p[4 * i] = wv[i].x * xv[i].x;
            p[4 * i + 1] = wv[i].y * xv[i].y;
            p[4 * i + 2] = wv[i].z * xv[i].z;
            p[4 * i + 3] = wv[i].w * xv[i].w;
        }
        float acc = -0.0f;
        for (int quarter = 0; quarter < 4; ++quarter) {
            if ((lane >> 4) == quarter) {
#pragma unroll
                for (int i = 0; i < C; ++i) buf[(lane & 15) * C + i] = p[i];
            }
            wave_lds_sync();
            if (lane == 0) {
#pragma unroll 16
                for (int i = 0; i < Q; ++i) acc = acc + buf[i];
            }
            wave_lds_sync();
        }
        if (lane == 0 && c < nc) R[e] = bias ? acc + bias[e] : acc;
    }
}

template <int F4>
__global__ __launch_bounds__(SEL_WAVES * 64) void k_select(const double2 *__restrict__ stats,
                                                           const float *__restrict__ bias,
                                                           const float *__restrict__ W, const float *__restrict__ x,
                                                           int n_exp, int top_k, int pre_norm, float eps, int exact,
                                                           uint32_t *__restrict__ ctl, int32_t *__restrict__ ids,
                                                           float *__restrict__ wts, float *__restrict__ logits) {
    constexpr int d = 256 * F4, Q = 64 * F4;
    __shared__ uint32_t key[256];
    __shared__ float sR[256], sp[256];
    __shared__ double selS[8], selE[8];
    __shared__ int cand[256];
    __shared__ int sel[8];
    __shared__ int s_pass, s_nc, s_level;
    __shared__ float fold[SEL_WAVES * Q];
    const int tok = blockIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const double2 *st = stats + (size_t)tok * n_exp;
    const float *xt = x + (size_t)tok * d;
    int32_t *ids_t = ids + (size_t)tok * top_k;
    float *wts_t = wts + (size_t)tok * top_k;
    float *lg_t = logits ? logits + (size_t)tok * n_exp : nullptr;

    // ---- fast path: one wave, lane l owns experts l, l + 64, l + 128, l + 192 ----
    if (w == 0) {
        double S[4], E[4];
        uint32_t k[4];
        bool alive[4];
        int rk[4];
        bool bad = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            S[i] = -INFINITY;
            E[i] = 0.0;
            if (e < n_exp) {
                const double2 v = st[e];
                S[i] = v.x;
                E[i] = v.y;
                if (bias) {
                    const double s2 = S[i] + (double)bias[e];
                    E[i] = E[i] + (fabs(s2) + E[i]) * 0x1p-23;  // the f32 rounding of logit + bias
                    S[i] = s2;
                }
                bad |= !isfinite(S[i]) || !isfinite(E[i]);
            }
            k[i] = e < n_exp ? order_key((float)S[i]) : 0u;
            alive[i] = e < n_exp;
        }
        // S-top-k by (f32 key desc, index asc): experts whose keys tie fail the certificate below
        wave_top_k(k, alive, top_k, rk, sel);
        uint32_t uk = 0;  // the highest upper bound among unselected experts, rounded up to f32
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (rk[i] < top_k) {
                selS[rk[i]] = S[i];
                selE[rk[i]] = E[i];
            }
            if (alive[i]) uk = max(uk, order_key(round_up_f32(S[i] + E[i])));
        }
        uk = wave_max_u32(uk);
        const double U = uk ? (double)key_float(uk) : -INFINITY;
        const bool any_bad = __ballot(bad) != 0;
        wave_lds_sync();
        const double M = selS[0];
        // certificate: lane i < top_k checks rank i against rank i + 1 (or every unselected one)
        bool ok = true;
        if (lane < top_k) {
            const double lo = selS[lane] - selE[lane];
            double hi, sb;
            if (lane + 1 < top_k) {
                hi = selS[lane + 1] + selE[lane + 1];
                sb = selS[lane + 1];
            } else {
                hi = U;
                sb = isfinite(U) ? U : 0.0;
            }
            ok = lo - order_margin(selS[lane], sb, M) > hi;
            if (lane == top_k - 1) ok = ok && selS[lane] - M > -80.0;  // clear of expf underflow
        }
        const bool pass = !exact && !any_bad && __ballot(!ok) == 0;
        if (pass) {
            // certified ids; weights from the f32-rounded estimates (tolerance class)
            const float Mf = (float)M;
            float ex[4];
            double sum = 0.0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ex[i] = lane + 64 * i < n_exp ? expf((float)S[i] - Mf) : 0.0f;
                sum += (double)ex[i];
            }
            sum = wave_sum_d(sum);
            const float inv = (float)(1.0 / sum);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (rk[i] < top_k) sp[rk[i]] = ex[i] * inv;
                if (lg_t && lane + 64 * i < n_exp) lg_t[lane + 64 * i] = (float)S[i];
            }
            wave_lds_sync();
            if (lane == 0) {
                float s = -0.0f;
                for (int j = 0; j < top_k; ++j) s = s + sp[j];
                s = fmaxf(s, 1.0f / 16384.0f);
                for (int j = 0; j < top_k; ++j) {
                    ids_t[j] = sel[j];
                    wts_t[j] = sp[j] / s;
                }
            }
        } else {
            // level 1 candidates: the S-top-k and every expert whose upper bound reaches the
            // lowest selected lower bound; non-finite statistics or RVM_EXACT_SELECT: all experts
            double Lstar = INFINITY;
            for (int j = 0; j < top_k; ++j) Lstar = fmin(Lstar, selS[j] - selE[j]);
            const bool all = exact || any_bad || !isfinite(M) || !isfinite(Lstar);
            int base = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = lane + 64 * i;
                const bool c =
                    e < n_exp && (all || rk[i] < top_k || S[i] + E[i] + order_margin(S[i], Lstar, M) > Lstar);
                const uint64_t m = __ballot(c);
                if (c) cand[base + __popcll(m & ((1ull << lane) - 1ull))] = e;
                base += __popcll(m);
                sR[e] = e < n_exp ? (float)S[i] : -INFINITY;
            }
            if (lane == 0) {
                s_nc = base;
                s_level = all ? 2 : 1;
                atomicAdd(&ctl[0], 1u);
            }
        }
        if (lane == 0) s_pass = pass;
    }
    __syncthreads();
    if (s_pass) return;

    // ---- exact path: every wave folds candidates ----
    float4 xv[F4];
    load_x_chunk<F4>(xt, lane, pre_norm, eps, xv);
    exact_fold<F4>(W, bias, xv, cand, s_nc, sR, fold);
    __syncthreads();
    if (s_level == 1) {
        if (w == 0) {
            // rank the candidates by their exact logits; level 1 holds if the exact top-k and
            // the best candidate left out are separated by the margin
            const int nc = s_nc;
            for (int c = lane; c < nc; c += 64) {
                const int e = cand[c];
                const float Rt = sR[e];
                int r = 0;
                for (int j = 0; j < nc; ++j) {
                    const int o = cand[j];
                    const float v = sR[o];
                    r += (v > Rt) || (v == Rt && o < e);
                }
                if (r < top_k) sel[r] = e;
            }
            wave_lds_sync();
            bool ok = true;
            const double Mx = sR[sel[0]];
            if (lane + 1 < top_k) {
                const double a = sR[sel[lane]], b = sR[sel[lane + 1]];
                ok = a - b > order_margin(a, b, Mx);
            }
            double nb = -INFINITY;
            for (int c = lane; c < nc; c += 64) {
                const int e = cand[c];
                bool chosen = false;
                for (int i = 0; i < top_k; ++i) chosen |= sel[i] == e;
                if (!chosen) nb = fmax(nb, (double)sR[e]);
            }
            nb = wave_max_d(nb);
            const double a = sR[sel[top_k - 1]];
            if (lane == 0 && isfinite(nb)) ok = ok && a - nb > order_margin(a, nb, Mx);
            if (lane == 0) ok = ok && a - Mx > -80.0;
            const bool good = __ballot(!ok) == 0;
            if (lane == 0) {
                s_level = good ? 1 : 2;
                // level 2 folds the experts that are not candidates yet
                if (!good) s_nc = 0;
            }
            if (!good) {
                wave_lds_sync();
                // mark the existing candidates in the key array, then list the rest
                for (int c = lane; c < nc; c += 64) key[cand[c]] = 0xffffffffu;
                wave_lds_sync();
                int base = 0;
                for (int i = 0; i < 4; ++i) {
                    const int e = lane + 64 * i;
                    const bool c = e < n_exp && key[e] != 0xffffffffu;
                    const uint64_t m = __ballot(c);
                    wave_lds_sync();
                    if (c) cand[base + __popcll(m & ((1ull << lane) - 1ull))] = e;
                    base += __popcll(m);
                }
                if (lane == 0) s_nc = base;
            }
        }
        __syncthreads();
        if (s_level == 2) {
            exact_fold<F4>(W, bias, xv, cand, s_nc, sR, fold);
            __syncthreads();
        }
    }
    if (w != 0) return;
    // ---- selection from the (partly) exact logits ----
    float R[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) R[i] = lane + 64 * i < n_exp ? sR[lane + 64 * i] : -INFINITY;
    float Mf = -INFINITY;  // max ignoring NaN (runtime/src/ops.rs:171)
#pragma unroll
    for (int i = 0; i < 4; ++i) Mf = fmaxf(Mf, R[i]);
    Mf = wave_max_f(Mf);
    if (lg_t)
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < n_exp) lg_t[lane + 64 * i] = R[i];
    if (s_level == 1) {
        // ids certified from the exact candidates (sel); weights tolerance class
        float ex[4];
        double sum = 0.0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ex[i] = lane + 64 * i < n_exp ? expf(R[i] - Mf) : 0.0f;
            sum += (double)ex[i];
        }
        sum = wave_sum_d(sum);
        const float inv = (float)(1.0 / sum);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < n_exp) sp[lane + 64 * i] = ex[i] * inv;
    } else {
        // every logit exact: softmax (runtime/src/ops.rs:170-179) with an f64 sum in index order
        // and expf correctly rounded, then top_k by total_cmp (ops.rs:182-187)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < n_exp) sp[lane + 64 * i] = (float)exp((double)(R[i] - Mf));
        wave_lds_sync();
        float inv = 0.0f;
        if (lane == 0) {
            double sum = 0.0;
            for (int j = 0; j < n_exp; ++j) sum += (double)sp[j];
            inv = (float)(1.0 / sum);
        }
        inv = __shfl(inv, 0);
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = lane + 64 * i < n_exp ? sp[lane + 64 * i] * inv : 0.0f;
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < n_exp) sp[lane + 64 * i] = p[i];
        uint32_t k[4];
        bool alive[4];
        int rk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            alive[i] = lane + 64 * i < n_exp;
            k[i] = alive[i] ? order_key(p[i]) : 0u;
        }
        wave_top_k(k, alive, top_k, rk, sel);
    }
    wave_lds_sync();
    if (lane == 0) {
        float s = -0.0f;
        for (int j = 0; j < top_k; ++j) s = s + sp[sel[j]];
        s = fmaxf(s, 1.0f / 16384.0f);
        for (int j = 0; j < top_k; ++j) {
            ids_t[j] = sel[j];
            wts_t[j] = sp[sel[j]] / s;
        }
    }
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
    const int pre = (flags & RVM_PRE_NORM) ? 1 : 0;
    return with_steps(L->d / 256, [&](auto f4) {
        constexpr int F4 = decltype(f4)::value;
        hipLaunchKernelGGL(k_router<F4>, dim3(groups, n_tok), dim3(256), 0, cur_stream(), L->router, x, L->n_exp,
                           pre, eps, (double2 *)(ws + lay.stats), (uint32_t *)(ws + lay.xact));
        int rc = launched();
        if (rc) return rc;
        hipLaunchKernelGGL(k_select<F4>, dim3(n_tok), dim3(SEL_WAVES * 64), 0, cur_stream(),
                           (const double2 *)(ws + lay.stats), L->router_bias, L->router, x, L->n_exp, L->top_k, pre,
                           eps, (flags & RVM_EXACT_SELECT) ? 1 : 0, (uint32_t *)(ws + lay.ctl), ids, wts, logits);
        return launched();
    });
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
    RVM_CHECK(layer_ok(layer) && x && n_tok > 0 && n_tok <= MAX_TOKENS && ids && weights && ws);
    const WsLayout lay = ws_layout(layer, n_tok);
    RVM_CHECK(ws_bytes >= lay.total);
    return launch_router(layer, x, n_tok, flags, eps, (uint8_t *)ws, lay, ids, weights, logits);
}

int rvm_moe_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of, int32_t *group_start) {
    RVM_CHECK(ids && order && pos_of && group_start && n_pairs > 0 && n_exp > 0 && n_exp <= 256);
    return launch_plan(ids, n_pairs, n_exp, order, pos_of, group_start);
}

}  // extern "C"
