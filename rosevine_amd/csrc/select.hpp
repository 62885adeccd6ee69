// select.hpp - expert selection for one token from the router's logit statistics, with an
// exactness certificate (runtime/src/exec.rs:507-517: softmax, top_k by total_cmp with ties to
// the lower index, weights renormalised with the 2^-14 clamp of exec.rs:124-125).
//
// The router kernel (router.hip) leaves, per expert, S = the f64 sum of the reference's f32
// products W_r[e][i] * x[i] and a bound E on how far the reference's sequential f32 fold can be
// from S. The workgroup ranks the experts by S (f32 keys) and checks that the intervals
// [S - E, S + E] of the selected experts and the best unselected one are separated by a margin
// that keeps expf and the 1/sum product order-preserving: then the reference's ids are certified.
// Otherwise (about 2% of tokens with iid logits, or tied keys, or non-finite statistics, or when
// exact selection is asked for) every logit is recomputed in the reference's order, one lane per
// expert, and the reference's softmax and top-k run on the exact values.
//
// select_token is called by every thread of a workgroup of NW waves; it is used by the selection
// kernel (one workgroup per token) and by the decode gate/up kernel, whose workgroups each
// select for themselves so that no launch separates the router from the experts.
#pragma once
#include <math.h>

#include "expf.hpp"
#include "internal.hpp"

namespace rvm {

template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = dpp<CTRL>((uint32_t)u), hi = dpp<CTRL>((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, (hi << 32) | lo);
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(double, (hi << 32) | lo);
}
// v moved by DPP control CTRL in the rows of ROW_MASK; lanes of other rows, and lanes whose
// source lies outside their row, read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_zero_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xf, true);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xf, true);
    return __builtin_bit_cast(double, (hi << 32) | lo);
}
// Inclusive prefix sum over the 64 lanes (all active), by DPP only: row_shr 1, 2, 4, 8 within
// each row of 16, then row_bcast:15 (row r's last lane into row r + 1, for rows 1 and 3) and
// row_bcast:31 (lane 31 into rows 2 and 3).
__device__ __forceinline__ double wave_scan_d(double v) {
    v += dpp_zero_d<0x111>(v);
    v += dpp_zero_d<0x112>(v);
    v += dpp_zero_d<0x114>(v);
    v += dpp_zero_d<0x118>(v);
    v += dpp_zero_d<0x142, 0xa>(v);
    v += dpp_zero_d<0x143, 0xc>(v);
    return v;
}
// Sum over the wave (all lanes active): quads, octets and rows of 16 by DPP (each step adds the
// same two values in every lane, so all lanes agree), then the four rows. Wave-uniform result.
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xb1>(v);
    v += dpp_d<0x4e>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
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


// Rust f32::total_cmp key, and an unsigned key with the same order (for packed ranking).
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t i = __builtin_bit_cast(int32_t, f);
    return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}
__device__ __forceinline__ uint32_t order_key(float f) { return (uint32_t)total_key(f) ^ 0x80000000u; }

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

// The reference's selection from its exact logits, one wave (runtime/src/exec.rs:507-517):
// softmax (runtime/src/ops.rs:170-179: max ignoring NaN, numerators expf(R - max) as glibc's expf,
// their f64 sum in index order, inv = (1/sum) as f32, p * inv), top_k by total_cmp with
// ties to the lower index (ops.rs:182-187), and the weights p_j / max(sum of the selected p in top
// order, 2^-14). R[i] is expert lane + 64 i (-inf past n_exp); sp (256 floats), sel and wsel are
// LDS of this wave; lg_t, when set, receives the logits. Every lane of the wave calls this.
__device__ __forceinline__ void exact_softmax_top_k(const float (&R)[4], int n_exp, int top_k, float *sp, int *sel,
                                                    float *wsel, float *lg_t, int lane) {
    float Mf = -INFINITY;  // max ignoring NaN (runtime/src/ops.rs:171)
#pragma unroll
    for (int i = 0; i < 4; ++i) Mf = fmaxf(Mf, R[i]);
    Mf = wave_max_f(Mf);
    if (lg_t)
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < n_exp) lg_t[lane + 64 * i] = R[i];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (lane + 64 * i < n_exp) sp[lane + 64 * i] = glibc_expf(R[i] - Mf);
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
    wave_lds_sync();
    float s = -0.0f;
    for (int j = 0; j < top_k; ++j) s = s + sp[sel[j]];
    s = fmaxf(s, 1.0f / 16384.0f);
    if (lane < top_k) wsel[lane] = sp[sel[lane]] / s;
}

// rms_norm of this lane's chunk xv of the layer input xt, in place (runtime/src/ops.rs:131-139:
// f64 sum of squares, mean as f32, 1/sqrt(mean + eps)); every wave computes the same scale.
template <int F4>
__device__ __forceinline__ float norm_x_chunk(const float *xt, float4 (&xv)[F4], float eps) {
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < F4; ++i)
        s += (double)xv[i].x * (double)xv[i].x + (double)xv[i].y * (double)xv[i].y +
             (double)xv[i].z * (double)xv[i].z + (double)xv[i].w * (double)xv[i].w;
    s = wave_sum_d(s);  // the same value in every lane
    // The reference sums sequentially. Both sums are within d * 2^-53 * s of the exact one, so
    // the f32 mean is the reference's unless it sits at an f32 rounding boundary; then the sum is
    // redone in the reference's order.
    const double n = 256.0 * F4, bnd = s * (2.0 * n * 0x1p-53) * 1.01;
    if ((float)((s - bnd) / n) != (float)((s + bnd) / n)) {
        s = 0.0;
        for (int i = 0; i < 256 * F4; ++i) {
            const double v = (double)xt[i];
            s += v * v;
        }
    }
    const float mean = (float)(s / (double)(256 * F4));
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int i = 0; i < F4; ++i)
        xv[i] = make_float4(xv[i].x * scale, xv[i].y * scale, xv[i].z * scale, xv[i].w * scale);
    return scale;
}

// The rms_norm scale s of the row xt (every lane computes the same value).
template <int F4>
__device__ __forceinline__ float rms_scale(const float *xt, int lane, float eps) {
    float4 xv[F4];
    const float4 *x4 = (const float4 *)xt + lane * F4;
#pragma unroll
    for (int i = 0; i < F4; ++i) xv[i] = x4[i];
    return norm_x_chunk<F4>(xt, xv, eps);
}

// The router's factors on this lane's chunk of the normed input: ((x * s) * rpost) * rg[i].
template <int F4>
__device__ __forceinline__ void router_gain(const XForm &xf, int lane, float4 (&xv)[F4]) {
    if (xf.rpost != 1.0f) {
        const float p = xf.rpost;
#pragma unroll
        for (int i = 0; i < F4; ++i) xv[i] = make_float4(xv[i].x * p, xv[i].y * p, xv[i].z * p, xv[i].w * p);
    }
    if (xf.rg) {
        const float4 *g4 = (const float4 *)xf.rg + lane * F4;
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const float4 g = g4[i];
            xv[i] = make_float4(xv[i].x * g.x, xv[i].y * g.y, xv[i].z * g.z, xv[i].w * g.w);
        }
    }
}

// This lane's chunk of the router input (elements [4 F4 lane, 4 F4 (lane + 1))): x, or the normed
// x with the router's factors (XForm). Returns the rms_norm scale s (1 without pre_norm).
template <int F4>
__device__ __forceinline__ float load_x_chunk(const float *xt, int lane, const XForm &xf, float4 (&xv)[F4]) {
    const float4 *x4 = (const float4 *)xt + lane * F4;
#pragma unroll
    for (int i = 0; i < F4; ++i) xv[i] = x4[i];
    if (!xf.pre_norm) return 1.0f;
    const float s = norm_x_chunk<F4>(xt, xv, xf.eps);
    router_gain<F4>(xf, lane, xv);
    return s;
}

constexpr int SEL_P_FLOATS = 2 * 16 * 260;  // >= 128 * 36
// LDS of select_token for a workgroup of NW waves and d = 256 * F4.
template <int F4, int NW>
struct SelShared {
    double Sx[256], Ex[256];  // per expert: the f64 estimate (bias included) and its bound
    alignas(16) uint32_t key32[256];  // f32 order keys of the estimates (0 past n_exp)
    int hits[8];  // experts counted at each top rank: 1 unless f32 keys tie
    int rank[256];
    float sR[256], sp[256];
    double selS[8], selE[8];
    int sel[8];
    int spec[8];  // the ids the S ranking gives (the certified ids when pass), the same in every workgroup
    float wsel[8];
    uint32_t ukw[NW];
    int badw[NW];
    int pass;
    alignas(16) float xs[256 * F4];  // the exact path's layer input (x, or rms_norm(x))
    alignas(16) float P[SEL_P_FLOATS];  // the exact paths' products: 128 rows x 32 columns at pitch
                                        // 36 (exact_all), or two buffers of 16 rows x 256 at 260
    int cand[32];                    // the candidate path's experts, ascending
    float csp[32], csel[9];          // their softmax numerators; ranks 0 .. 8 in order
    int ncand, cok;
};

// Exact reference-order logits of every expert into sh.sR: the f32 products W_r[e][i] * x'[i]
// added in element order from -0.0 (runtime/src/ops.rs:321-326), then the bias. The workgroup
// streams the rows 32 columns at a time (coalesced, kept PF chunks ahead), forms the products
// into LDS, and lane l of waves 0 and 1 folds the chunk of expert 64 w + l (128 experts per pass).
// Called by every thread.
template <int F4, int NW>
__device__ void exact_all(SelShared<F4, NW> &sh, const float *__restrict__ W, const float *__restrict__ bias,
                          const float *__restrict__ xt, int n_exp, const XForm &xf) {
    static_assert(NW == 8, "512 threads: 128 rows x 8 column quads per pass");
    constexpr int d = 256 * F4, CH = 32, NCH = d / CH, PIT = 36, PF = 8;
    static_assert(NCH % PF == 0, "whole rounds of prefetched chunks");
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    if (w == 0) {
        float4 xv[F4];
        load_x_chunk<F4>(xt, lane, xf, xv);
#pragma unroll
        for (int i = 0; i < F4; ++i) ((float4 *)sh.xs)[lane * F4 + i] = xv[i];
    }
    __syncthreads();
    const int rr = tid >> 3, c4 = tid & 7;  // rows rr and rr + 64 of the pass, column quad c4
    float4 *P4 = (float4 *)sh.P;
    for (int r0 = 0; r0 < n_exp; r0 += 128) {
        const float4 *rp[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) rp[i] = (const float4 *)(W + (size_t)min(r0 + rr + 64 * i, n_exp - 1) * d) + c4;
        float4 pf[PF][2];
#pragma unroll
        for (int u = 0; u < PF; ++u)
#pragma unroll
            for (int i = 0; i < 2; ++i) pf[u][i] = rp[i][u * (CH / 4)];
        float acc = -0.0f;
        for (int c0 = 0; c0 < NCH; c0 += PF) {
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                const int c = c0 + u;
                const float4 xv = ((const float4 *)sh.xs)[c * (CH / 4) + c4];
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    P4[(rr + 64 * i) * (PIT / 4) + c4] = make_float4(pf[u][i].x * xv.x, pf[u][i].y * xv.y,
                                                                     pf[u][i].z * xv.z, pf[u][i].w * xv.w);
                const int cn = min(c + PF, NCH - 1);
#pragma unroll
                for (int i = 0; i < 2; ++i) pf[u][i] = rp[i][cn * (CH / 4)];
                __syncthreads();
                if (w < 2) {
                    float4 v[CH / 4];
#pragma unroll
                    for (int j = 0; j < CH / 4; ++j) v[j] = P4[(w * 64 + lane) * (PIT / 4) + j];
#pragma unroll
                    for (int j = 0; j < CH / 4; ++j) {
                        acc = acc + v[j].x;
                        acc = acc + v[j].y;
                        acc = acc + v[j].z;
                        acc = acc + v[j].w;
                    }
                }
                __syncthreads();
            }
        }
        const int fe = r0 + w * 64 + lane;
        if (w < 2 && fe < n_exp) sh.sR[fe] = bias ? acc + bias[fe] : acc;
    }
    __syncthreads();
}

// Exact ids from the experts that can still reach the top k, when the certificate fails
// (runtime/src/exec.rs:507-517, ops.rs:170-187). L = the lowest lower bound S - E among the top
// k of the S ranking; every expert whose upper bound is within order_margin of L is a candidate
// (at most 16; ties among the top keys or non-finite statistics leave this to exact_all). Lane c
// of wave 0 folds candidate c's logit in the reference's order, so the candidates' softmax
// numerators expf(R - max) are the reference's. The reference ranks p = numerator * (1/sum as
// f32); sum depends on every expert and is not known exactly here, but the ranking does not
// depend on it when the numerators at ranks 0 .. top_k are equal or clearly apart, and every
// other expert's largest numerator is clearly below the k-th; that is checked. The weights are
// then formed as on the certified path (tolerance class). Returns false (nothing selected) when
// a check fails; then sh.sel and sh.wsel are the exact_all path's to fill. Called by every thread.
template <int F4, int NW>
__device__ bool exact_candidates(SelShared<F4, NW> &sh, const float *__restrict__ W, const float *__restrict__ bias,
                                 const float *__restrict__ xt, int n_exp, int top_k, const XForm &xf) {
    constexpr int d = 256 * F4, CM = 16, CK = 256, NCH = d / CK, PP = CK + 4, D = 3;
    static_assert(2 * CM * PP <= SEL_P_FLOATS, "two product buffers fit the exact path's LDS");
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    uint64_t cmask[4] = {0, 0, 0, 0};  // wave 0: the candidates among experts l + 64 i
    if (w == 0) {
        bool ok = true;
        for (int j = 0; j < top_k; ++j) ok = ok && sh.hits[j] == 1;
        for (int i = 0; i < NW; ++i) ok = ok && sh.badw[i] == 0;
        double L = INFINITY;
        for (int j = 0; j < top_k; ++j) L = fmin(L, sh.selS[j] - sh.selE[j]);
        const double M = sh.selS[0];
        int nc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            bool c = false;
            if (e < n_exp) {
                const double S = sh.Sx[e], E = sh.Ex[e];
                c = S + E + order_margin(S, L, M) >= L;
            }
            cmask[i] = __ballot(c);
            const int pos = nc + __popcll(cmask[i] & ((1ull << lane) - 1ull));
            if (c && pos < CM) sh.cand[pos] = e;
            nc += __popcll(cmask[i]);
        }
        if (lane == 0) sh.ncand = ok && nc <= CM ? nc : -1;
    } else if (w == 1) {
        float4 xv[F4];
        load_x_chunk<F4>(xt, lane, xf, xv);
#pragma unroll
        for (int i = 0; i < F4; ++i) ((float4 *)sh.xs)[lane * F4 + i] = xv[i];
    }
    __syncthreads();
    const int nc = sh.ncand;
    if (nc < 0) return false;
    // The candidates' logits: f32 products added in element order from -0.0, then the bias. Waves
    // 1.. form the products of CK-column chunks into LDS (double-buffered; each thread keeps its
    // loads D chunks ahead in a register ring), and lane c of wave 0 adds candidate c's.
    constexpr int NPT = 64 * (NW - 1), IT = (CM * CK / 4 + NPT - 1) / NPT;
    const int pt = tid - 64;
    const float *src[IT];
    int dst[IT], col[IT];
    bool vok[IT];
#pragma unroll
    for (int k = 0; k < IT; ++k) {
        const int i = pt + k * NPT;
        vok[k] = pt >= 0 && i < nc * (CK / 4);
        const int ii = vok[k] ? i : 0, c = ii / (CK / 4), q = ii - c * (CK / 4);
        src[k] = W + (size_t)sh.cand[c] * d + 4 * q;
        dst[k] = c * PP + 4 * q;
        col[k] = 4 * q;
    }
    auto load = [&](int ch, float4 (&r)[IT]) {  // unconditional: the chunk index is clamped
        const int cc = min(ch, NCH - 1);
#pragma unroll
        for (int k = 0; k < IT; ++k) r[k] = *(const float4 *)(src[k] + cc * CK);
    };
    auto store = [&](int ch, int buf, const float4 (&r)[IT]) {
#pragma unroll
        for (int k = 0; k < IT; ++k)
            if (vok[k]) {
                const float4 xv = *(const float4 *)(sh.xs + ch * CK + col[k]);
                *(float4 *)(sh.P + buf * CM * PP + dst[k]) =
                    make_float4(r[k].x * xv.x, r[k].y * xv.y, r[k].z * xv.z, r[k].w * xv.w);
            }
    };
    float acc = -0.0f;
    auto fold = [&](int buf) {  // the next 32 products are read from LDS while these are added
        if (w != 0) return;
        const float4 *pr = (const float4 *)(sh.P + buf * CM * PP + min(lane, nc - 1) * PP);
        constexpr int G = CK / 32;
        float4 v[2][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[0][j] = pr[j];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (g + 1 < G)
#pragma unroll
                for (int j = 0; j < 8; ++j) v[(g + 1) & 1][j] = pr[(g + 1) * 8 + j];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc = acc + v[g & 1][j].x;
                acc = acc + v[g & 1][j].y;
                acc = acc + v[g & 1][j].z;
                acc = acc + v[g & 1][j].w;
            }
        }
    };
    float4 ring[D][IT];
#pragma unroll
    for (int u = 0; u < D; ++u) load(u, ring[u]);
    store(0, 0, ring[0]);
    __syncthreads();
    for (int c0 = 0; c0 < NCH; c0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int c = c0 + u;
            if (c < NCH) {
                load(c + D, ring[u]);  // ring[u] held chunk c, stored one step ago
                fold(c & 1);
                if (c + 1 < NCH) store(c + 1, (c + 1) & 1, ring[(u + 1) % D]);
                __syncthreads();
            }
        }
    }
    if (w == 0) {
        const int ce = sh.cand[min(lane, nc - 1)];
        const float R = bias ? acc + bias[ce] : acc;
        const float Mf = wave_max_f(lane < nc ? R : -INFINITY);  // the largest logit is a candidate's
        const float spc = glibc_expf(R - Mf);                   // exactly the reference's numerator
        // rank of each candidate by (numerator desc, index asc); the candidates are in index order
        if (lane < nc) sh.csp[lane] = spc;
        wave_lds_sync();
        int rk = 64;
        if (lane < nc) {
            const uint32_t k = order_key(spc);
            rk = 0;
            for (int c2 = 0; c2 < nc; ++c2) {
                const uint32_t k2 = order_key(sh.csp[c2]);
                rk += (k2 > k || (k2 == k && c2 < lane)) ? 1 : 0;
            }
            if (rk <= top_k) sh.csel[rk] = spc;
        }
        wave_lds_sync();
        // The reference orders p = numerator * inv. Multiplying by one positive inv keeps equal
        // numerators equal (their order is by index, as here) and keeps numerators more than a
        // factor 1 + 2^-21 apart strictly ordered, whatever inv is; closer pairs at ranks
        // 0 .. top_k, or an expert outside the candidates closer than that to the k-th, are left
        // to exact_all.
        const float sep = 1.0f + 0x1p-21f;
        bool ok = true;
        if (lane < nc && rk < top_k) {
            const float next = rk + 1 < nc ? sh.csel[rk + 1] : 0.0f;
            ok = spc == next || spc > next * sep;
        }
        const float pk = sh.csel[top_k - 1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            if (e < n_exp && !((cmask[i] >> lane) & 1ull)) {
                const float hi = round_up_f32(sh.Sx[e] + sh.Ex[e]);
                ok = ok && glibc_expf(hi - Mf) * sep < pk;
            }
        }
        ok = __ballot(!ok) == 0;
        if (lane < nc && rk < top_k) sh.sel[rk] = ce;
        // weights (tolerance class, as on the certified path): the candidates' exact numerators,
        // the others' from the estimates, their f64 sum, renormalised over the top k
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            if (e < n_exp) sh.sp[e] = expf((float)sh.Sx[e] - Mf);
        }
        wave_lds_sync();
        if (lane < nc) sh.sp[ce] = spc;
        wave_lds_sync();
        double sum = 0.0;  // a tree over the wave, as on the certified path (the weights' class)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            if (e < n_exp) sum += (double)sh.sp[e];
        }
        sum = wave_sum_d(sum);
        const float inv = (float)(1.0 / sum);
        if (ok && lane < top_k) {
            float s = -0.0f;
            for (int j = 0; j < top_k; ++j) s = s + sh.csel[j] * inv;
            s = fmaxf(s, 1.0f / 16384.0f);
            sh.wsel[lane] = sh.csel[lane] * inv / s;
        }
        if (lane == 0) sh.cok = ok;
    }
    __syncthreads();
    return sh.cok != 0;
}

// Selects top_k experts for one token. st: the token's [n_exp] statistics; xt: its layer input,
// which xf turns into the router input.
// Called by every thread of the workgroup. sh.pass tells whether the S ranking is certified; then
// sh.sel[0..top_k) = sh.spec[0..top_k) are the reference's ids in top order and select_weights
// computes the weights. Otherwise, with exact_here set, the exact path leaves the reference's
// ids in sh.sel and its weights in sh.wsel (sh.spec keeps the S-ranking ids); without it only
// sh.spec is meaningful. With publish set, the logits go to lg_t (when not null) and a fallback
// is counted in ctl[0].
// With CERTIFY false only the S ranking runs (no certificate, no exact path): sh.sel and sh.hits
// are set, and spec_id gives the ids every workgroup agrees on.
template <int F4, int NW, bool CERTIFY = true>
__device__ void select_token(SelShared<F4, NW> &sh, const double2 *__restrict__ st, const float *__restrict__ bias,
                             const float *__restrict__ W, const float *__restrict__ xt, int n_exp, int top_k,
                             const XForm &xf, int exact, bool publish, bool exact_here,
                             uint32_t *__restrict__ ctl, float *__restrict__ lg_t) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    static_assert(NW == 8, "the ranking splits up to 256 experts over 512 threads");
    const int tid = threadIdx.x;
    // ---- fast path. A: each expert's estimate, bound and f32 key into LDS ----
    if (tid < n_exp) {
        const double2 v = st[tid];
        double S = v.x, E = v.y;
        if (bias) {
            const double s2 = S + (double)bias[tid];
            E = E + (fabs(s2) + E) * 0x1p-23;  // the f32 rounding of logit + bias
            S = s2;
        }
        sh.Sx[tid] = S;
        sh.Ex[tid] = E;
        sh.key32[tid] = order_key((float)S);
    } else if (tid < 256) {
        sh.key32[tid] = 0u;  // below every expert's key: padding for the ranking slices
    }
    if (tid < 8) {
        sh.hits[tid] = 0;
        sh.sel[tid] = 0;
    }
    __syncthreads();
    // B: the rank of expert e = the number of experts with a larger f32 key, counted by tpe
    // threads over a slice of the experts each and summed across the group's lanes. Experts whose
    // keys tie share a rank; the tie is detected below and sends the token to the exact path,
    // which orders ties by index.
    {
        const int tpe = n_exp <= 128 ? 4 : 2;
        const int e = tid / tpe, part = tid % tpe;
        int r = 0;
        if (e < n_exp) {
            // slices of 32 keys at a time (keys past n_exp are 0 and never count; tpe * span <= 256),
            // with every LDS read of a round issued before its comparisons
            const uint32_t k = sh.key32[e];
            const int span = ((n_exp + tpe - 1) / tpe + 31) & ~31;
            const uint4 *k4 = (const uint4 *)(sh.key32 + part * span);
            for (int g0 = 0; g0 < span / 4; g0 += 8) {
                uint4 q[8];
#pragma unroll
                for (int g = 0; g < 8; ++g) q[g] = k4[g0 + g];
#pragma unroll
                for (int g = 0; g < 8; ++g)
                    r += (int)(q[g].x > k) + (int)(q[g].y > k) + (int)(q[g].z > k) + (int)(q[g].w > k);
            }
        }
        r += (int)dpp<0xb1>((uint32_t)r);
        if (tpe == 4) r += (int)dpp<0x4e>((uint32_t)r);
        const bool own = part == 0 && e < n_exp;
        if (!CERTIFY) {
            if (own && r < top_k) {
                atomicAdd(&sh.hits[r], 1);
                sh.sel[r] = e;
            }
            __syncthreads();
            return;
        }
        uint32_t uk = 0;  // the highest upper bound among unselected experts, rounded up to f32
        bool bad = false;
        if (own) {
            sh.rank[e] = r;
            const double S = sh.Sx[e], E = sh.Ex[e];
            bad = !isfinite(S) || !isfinite(E);
            if (r < top_k) {
                atomicAdd(&sh.hits[r], 1);
                sh.sel[r] = e;
                sh.selS[r] = S;
                sh.selE[r] = E;
            } else if (!bad) {
                uk = order_key(round_up_f32(S + E));
            }
        }
        uk = wave_max_u32(uk);
        const bool badw = __ballot(bad) != 0;
        if (lane == 0) {
            sh.ukw[w] = uk;
            sh.badw[w] = badw;
        }
    }
    __syncthreads();
    // C: the certificate, one wave
    if (w == 0) {
        uint32_t uk = 0;
        bool any_bad = false;  // non-finite statistics, or tied f32 keys among the top ranks
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            uk = max(uk, sh.ukw[i]);
            any_bad |= sh.badw[i] != 0;
        }
        for (int j = 0; j < top_k; ++j) any_bad |= sh.hits[j] != 1;
        const double U = uk ? (double)key_float(uk) : -INFINITY;
        const double M = sh.selS[0];
        // lane i < top_k checks rank i against rank i + 1 (or every unselected one)
        bool ok = true;
        if (lane < top_k) {
            const double lo = sh.selS[lane] - sh.selE[lane];
            double hi, sb;
            if (lane + 1 < top_k) {
                hi = sh.selS[lane + 1] + sh.selE[lane + 1];
                sb = sh.selS[lane + 1];
            } else {
                hi = U;
                sb = isfinite(U) ? U : 0.0;
            }
            ok = lo - order_margin(sh.selS[lane], sb, M) > hi;
            if (lane == top_k - 1) ok = ok && sh.selS[lane] - M > -80.0;  // clear of expf underflow
        }
        const bool pass = !exact && !any_bad && __ballot(!ok) == 0;
        if (pass) {
            if (publish && lg_t)
                for (int i = 0; i < 4; ++i)
                    if (lane + 64 * i < n_exp) lg_t[lane + 64 * i] = (float)sh.Sx[lane + 64 * i];
        } else if (publish && lane == 0) {
            atomicAdd(&ctl[0], 1u);
        }
        if (lane == 0) sh.pass = pass;
        // The S-ranking ids, for workgroups that proceed with them while the exact selection runs
        // elsewhere. Under tied keys the ranks are not unique and which tied expert wrote a rank
        // can differ between workgroups, so every workgroup then uses experts 0.. instead.
        bool ties = false;
        for (int j = 0; j < top_k; ++j) ties |= sh.hits[j] != 1;
        if (lane < top_k) sh.spec[lane] = ties ? lane : sh.sel[lane];  // = spec_id
    }
    __syncthreads();
    if (!sh.pass && exact_here) {
        // ---- exact path: the candidates first (exact_candidates); else every logit in the
        // reference's order, then the reference's softmax
        // (runtime/src/ops.rs:170-179: f64 sum in index order, expf correctly rounded) and top_k
        // by total_cmp (ops.rs:182-187) ----
        const bool done = !(publish && lg_t) &&
                          exact_candidates<F4, NW>(sh, W, bias, xt, n_exp, top_k, xf);
        if (!done) exact_all<F4, NW>(sh, W, bias, xt, n_exp, xf);
        if (!done && w == 0) {
            float R[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) R[i] = lane + 64 * i < n_exp ? sh.sR[lane + 64 * i] : -INFINITY;
            exact_softmax_top_k(R, n_exp, top_k, sh.sp, sh.sel, sh.wsel, publish ? lg_t : nullptr, lane);
        }
    }
    __syncthreads();
}

// The S-ranking id of slot j as every workgroup computes it (experts 0.. under tied keys); valid
// after select_token in either mode.
template <int F4, int NW>
__device__ __forceinline__ int spec_id(const SelShared<F4, NW> &sh, int j, int top_k) {
    bool ties = false;
    for (int i = 0; i < top_k; ++i) ties |= sh.hits[i] != 1;
    return ties ? j : sh.sel[j];
}

// The renormalised weights of a certified selection (sh.pass), from the estimates rounded to
// f32: softmax over every expert, the selected probabilities in top order summed sequentially,
// clamped at 2^-14, and divided (runtime/src/exec.rs:507-517; tolerance class, since the f32
// logits are not the reference's bits). Called by every thread; wave 0 works.
template <int F4, int NW>
__device__ void select_weights(SelShared<F4, NW> &sh, int n_exp, int top_k) {
    if ((threadIdx.x >> 6) != 0) return;
    const int lane = threadIdx.x & 63;
    const float Mf = (float)sh.selS[0];
    float ex[4];
    double sum = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        ex[i] = e < n_exp ? expf((float)sh.Sx[e] - Mf) : 0.0f;
        sum += (double)ex[i];
    }
    sum = wave_sum_d(sum);
    const float inv = (float)(1.0 / sum);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        if (e < n_exp && sh.rank[e] < top_k) sh.sp[sh.rank[e]] = ex[i] * inv;
    }
    wave_lds_sync();
    float s = -0.0f;
    for (int j = 0; j < top_k; ++j) s = s + sh.sp[j];
    s = fmaxf(s, 1.0f / 16384.0f);
    if (lane < top_k) sh.wsel[lane] = sh.sp[lane] / s;
}

// Writes the selection (ids and weights in top order) to global memory; every thread calls this
// after the weights are in sh.wsel and a barrier.
template <int F4, int NW>
__device__ __forceinline__ void select_publish(const SelShared<F4, NW> &sh, int top_k, int32_t *__restrict__ ids_t,
                                               float *__restrict__ wts_t) {
    if (threadIdx.x < (unsigned)top_k) {
        ids_t[threadIdx.x] = sh.sel[threadIdx.x];
        wts_t[threadIdx.x] = sh.wsel[threadIdx.x];
    }
}

}  // namespace rvm
