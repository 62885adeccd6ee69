// grouped.hip - n_tok tokens through one MoE layer with device-side grouping
// (runtime/src/exec.rs:456-475 and 540-640; the reference's host dispatch is
// runtime/src/hip_exec.rs:822-843).
//
//   router (router.hip)       -> ids, weights, Q8_0 activation blocks per token
//   k_plan (router.hip)       -> pairs stably grouped by expert: order, pos_of, group starts
//   k_gateup_grouped          -> per (expert, 64-row tile): the tile's weights are loaded into
//                                registers once and applied to every token of the group, TB at a
//                                time; sequential block fold, GeGLU + Q8_0 epilogue per token
//   k_down_grouped            -> per (expert, four 32-row tiles): y rows of every pair of the group
//   k_combine_pairs           -> out[t] = sum_j (y[pos_of[t*k+j]] * scale) * weight, slot order
// Each token's arithmetic is the decode kernels' (same split of K, same order), so a token's
// result does not depend on the batch it arrives in.
#include "internal.hpp"

namespace rvm {

constexpr int G_WAVES = 8;  // K split of a gate_up tile (as k_gateup_decode)
constexpr int TB = 4;       // tokens per pass

// Staging of n uint4 from global to LDS in two steps, so that a kernel can issue these loads
// before its weight loads (the memory counter drains in order) and store them after: the source
// index is clamped so that the loads need no branch.
template <int MAXN, int NT>
struct StageG {
    static constexpr int IT = (MAXN + NT - 1) / NT;
    static constexpr int SLOTS = IT * NT;  // LDS uint4 the destination must provide
    uint4 v[IT];
    __device__ __forceinline__ void load(const uint4 *__restrict__ src, int n) {
#pragma unroll
        for (int i = 0; i < IT; ++i) v[i] = src[min((int)threadIdx.x + i * NT, n - 1)];
    }
    // Unconditional: entries past n repeat the last one, so the loads never sink into a branch.
    __device__ __forceinline__ void store(uint4 *dst) const {
#pragma unroll
        for (int i = 0; i < IT; ++i) dst[threadIdx.x + i * NT] = v[i];
    }
};

template <int PER>
__device__ __forceinline__ void lane_terms_g(const uint4 (&wv)[PER], const uint32_t (&sv)[PER], const uint4 *act,
                                             float (&t)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint4 a0 = act[i * 3], a1 = act[i * 3 + 1];
        const float dx = __builtin_bit_cast(float, act[i * 3 + 2].x);
        const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        t[i] = block_term(block_dot(wv[i], a), h2f((uint16_t)sv[i]), dx);
    }
}

template <int PER>
__global__ __launch_bounds__(G_WAVES * 64) void k_gateup_grouped(
    const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl, const int32_t *__restrict__ gstart,
    const int32_t *__restrict__ order, const uint4 *__restrict__ xact, uint32_t *__restrict__ hact, int T,
    int top_k) {
    constexpr int S = PER * G_WAVES;
    using St = StageG<S * 3, G_WAVES * 64>;
    __shared__ uint4 act[TB][St::SLOTS];
    __shared__ float terms[64][S + 1];
    const int t = blockIdx.x, e = blockIdx.y;
    const int g0 = gstart[e], g1 = gstart[e + 1];
    if (g0 >= g1) return;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const size_t base = (((size_t)e * T + t) * S + (size_t)w * PER) * 64 + lane;
    uint4 wv[PER];
    uint32_t sv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        wv[i] = nib[base + (size_t)i * 64];
        sv[i] = scl[base + (size_t)i * 64];
    }
    for (int k0 = g0; k0 < g1; k0 += TB) {
        const int nt = min(TB, g1 - k0);
        St st[TB];
#pragma unroll
        for (int q = 0; q < TB; ++q) {
            const int tok = order[k0 + (q < nt ? q : 0)] / top_k;
            st[q].load(xact + (size_t)tok * S * 3, S * 3);
        }
#pragma unroll
        for (int q = 0; q < TB; ++q) st[q].store(act[q]);
        __syncthreads();
        for (int q = 0; q < nt; ++q) {
            float tv[PER];
            lane_terms_g<PER>(wv, sv, act[q] + w * PER * 3, tv);
#pragma unroll
            for (int i = 0; i < PER; ++i) terms[lane][w * PER + i] = tv[i];
            __syncthreads();
            if (w == 0) {
                float y = 0.0f;  // sequential fold of the row's block terms
#pragma unroll 8
                for (int b = 0; b < S; ++b) y = y + terms[lane][b];
                const float up = __shfl_xor(y, 32);
                const float h = gelu(y) * up;
                uint16_t dbits;
                const int qv = quant_q8_half(h, &dbits);
                store_prep_half(qv, dbits, lane & 31, hact + ((size_t)(k0 + q) * T + t) * ACT_DW, lane < 32);
            }
            __syncthreads();
        }
    }
}

template <int S>  // steps per lane = ff / 64
__global__ __launch_bounds__(256) void k_down_grouped(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl,
                                                      const int32_t *__restrict__ gstart,
                                                      const uint4 *__restrict__ hact, float *__restrict__ y, int T,
                                                      int d) {
    constexpr int NB = 2 * S;
    using St = StageG<NB * 3, 256>;
    __shared__ uint4 act[TB][St::SLOTS];
    const int e = blockIdx.y;
    const int g0 = gstart[e], g1 = gstart[e + 1];
    if (g0 >= g1) return;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + w;  // this wave's 32-row tile
    const int kp = lane >> 5;
    const size_t base = ((size_t)e * T + t) * S * 64 + lane;
    uint4 wv[S];
    uint32_t sv[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
        wv[i] = nib[base + (size_t)i * 64];
        sv[i] = scl[base + (size_t)i * 64];
    }
    for (int k0 = g0; k0 < g1; k0 += TB) {
        const int nt = min(TB, g1 - k0);
        St st[TB];
#pragma unroll
        for (int q = 0; q < TB; ++q) st[q].load(hact + (size_t)(k0 + (q < nt ? q : 0)) * NB * 3, NB * 3);
#pragma unroll
        for (int q = 0; q < TB; ++q) st[q].store(act[q]);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < TB; ++q) {
            float tv[S];
            lane_terms_g<S>(wv, sv, act[q] + kp * S * 3, tv);
            float acc = 0.0f;  // block order: this half, then the other half's terms
#pragma unroll
            for (int i = 0; i < S; ++i) acc = acc + tv[i];
#pragma unroll
            for (int i = 0; i < S; ++i) acc = acc + __shfl_xor(tv[i], 32);
            if (q < nt && lane < 32) y[(size_t)(k0 + q) * d + (size_t)t * 32 + lane] = acc;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void k_combine_pairs(const float *__restrict__ y, const int32_t *__restrict__ pos_of,
                                                       const int32_t *__restrict__ ids, const float *__restrict__ wts,
                                                       const float *__restrict__ dscale, float *__restrict__ out,
                                                       int top_k, int d) {
    const int t = blockIdx.x;
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float o = 0.0f;
        for (int j = 0; j < top_k; ++j) {
            const int p = t * top_k + j;
            const float ds = dscale ? dscale[ids[p]] : 1.0f;
            const float v = y[(size_t)pos_of[p] * d + i] * ds * wts[p];
            o = j == 0 ? v : o + v;
        }
        out[(size_t)t * d + i] = o;
    }
}

}  // namespace rvm

using namespace rvm;

extern "C" int rvm_moe_forward(const rvm_layer *L, const float *x, float *out, int n_tok, int flags, float eps,
                               void *ws, size_t ws_bytes) {
    RVM_CHECK(layer_ok(L) && x && out && ws && n_tok > 0 && n_tok <= MAX_TOKENS);
    if (n_tok == 1) return rvm_moe_decode(L, x, out, flags, eps, ws, ws_bytes);
    const WsLayout lay = ws_layout(L, n_tok);
    RVM_CHECK(ws_bytes >= lay.total);
    uint8_t *w = (uint8_t *)ws;
    int32_t *ids = (int32_t *)(w + lay.ids);
    float *wts = (float *)(w + lay.wts);
    int32_t *order = (int32_t *)(w + lay.order);
    int32_t *pos_of = (int32_t *)(w + lay.pos_of);
    int32_t *gstart = (int32_t *)(w + lay.gstart);
    float *y = (float *)(w + lay.y);
    const uint4 *xact = (const uint4 *)(w + lay.xact);
    uint32_t *hact = (uint32_t *)(w + lay.hact);
    int rc = launch_router(L, x, n_tok, flags, eps, w, lay, ids, wts, nullptr, true);
    if (rc) return rc;
    const int pairs = n_tok * L->top_k;
    if ((rc = launch_plan(ids, pairs, L->n_exp, order, pos_of, gstart))) return rc;

    const int Tg = 2 * L->ff / 64;
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint4 *gnib = (const uint4 *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)((const uint8_t *)L->gate_up + gu_entries * 16);
    rc = with_steps(L->d / 256, [&](auto per) {
        hipLaunchKernelGGL(k_gateup_grouped<decltype(per)::value>, dim3(Tg, L->n_exp), dim3(G_WAVES * 64), 0,
                           cur_stream(), gnib, gscl, gstart, order, xact, hact, Tg, L->top_k);
        return launched();
    });
    if (rc) return rc;

    const int Td = L->d / 32;  // a multiple of 8, so the four-tile groups cover it exactly
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint4 *dnib = (const uint4 *)L->down;
    const uint16_t *dscl = (const uint16_t *)((const uint8_t *)L->down + dn_entries * 16);
    rc = with_steps(L->ff / 64, [&](auto s) {
        hipLaunchKernelGGL(k_down_grouped<decltype(s)::value>, dim3(Td / 4, L->n_exp), dim3(256), 0, cur_stream(),
                           dnib, dscl, gstart, (const uint4 *)hact, y, Td, L->d);
        return launched();
    });
    if (rc) return rc;

    hipLaunchKernelGGL(k_combine_pairs, dim3(n_tok), dim3(256), 0, cur_stream(), y, pos_of, ids, wts, L->down_scale,
                       out, L->top_k, L->d);
    return launched();
}
