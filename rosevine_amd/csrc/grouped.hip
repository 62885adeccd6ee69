// grouped.hip - n_tok tokens through one MoE layer with device-side grouping
// (runtime/src/exec.rs:456-475 and 540-640; the reference's host dispatch is
// runtime/src/hip_exec.rs:822-843).
//
//   router (router.hip)       -> ids, weights, Q8_0 activation blocks per token
//   k_plan (router.hip)       -> pairs stably grouped by expert: order, pos_of, group starts
//   k_gateup_grouped          -> per (expert, 64-row tile): each weight step is loaded once and
//                                applied to up to TB tokens of the group; GeGLU + Q8_0 epilogue
//   k_down_grouped            -> per (expert, 32-row tile): y rows of every pair of the group
//   k_combine_pairs           -> out[t] = sum_j (y[pos_of[t*k+j]] * scale) * weight, slot order
#include "internal.hpp"

namespace rvm {

constexpr int G_WAVES = 4;
constexpr int G_CHUNK = 11;
constexpr int TB = 4;  // tokens per pass over a weight tile

__global__ __launch_bounds__(G_WAVES * 64) void k_gateup_grouped(
    const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl, const int32_t *__restrict__ gstart,
    const int32_t *__restrict__ order, const uint32_t *__restrict__ xact, uint32_t *__restrict__ hact, int T, int S,
    int top_k) {
    __shared__ float part[G_WAVES][TB][64];
    const int t = blockIdx.x, e = blockIdx.y;
    const int g0 = gstart[e], g1 = gstart[e + 1];
    if (g0 >= g1) return;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int per = S / G_WAVES;
    const int s0 = w * per;
    const size_t base = ((size_t)e * T + t) * S + s0;
    const uint4 *np = nib + base * 64 + lane;
    const uint16_t *sp = scl + base * 64 + lane;
    for (int k0 = g0; k0 < g1; k0 += TB) {
        const int nt = min(TB, g1 - k0);
        const uint32_t *ap[TB];
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const int tok = order[k0 + (i < nt ? i : 0)] / top_k;
            ap[i] = xact + ((size_t)tok * S + s0) * ACT_DW;  // xact is [token][S blocks]
        }
        float acc[TB] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int c = 0; c < per; c += G_CHUNK) {
            uint4 wv[G_CHUNK];
            uint16_t sv[G_CHUNK];
#pragma unroll
            for (int i = 0; i < G_CHUNK; ++i)
                if (c + i < per) {
                    wv[i] = np[(size_t)(c + i) * 64];
                    sv[i] = sp[(size_t)(c + i) * 64];
                }
#pragma unroll
            for (int i = 0; i < G_CHUNK; ++i)
                if (c + i < per) {
                    const float dw = h2f(sv[i]);
#pragma unroll
                    for (int q = 0; q < TB; ++q)
                        if (q < nt) {
                            const uint32_t *a = ap[q] + (c + i) * ACT_DW;
                            const int sumi = block_dot(wv[i], a);
                            acc[q] = fmaf((float)sumi, dw * __builtin_bit_cast(float, a[8]), acc[q]);
                        }
                }
        }
#pragma unroll
        for (int q = 0; q < TB; ++q) part[w][q][lane] = acc[q];
        __syncthreads();
        if (w == 0) {
            for (int q = 0; q < nt; ++q) {
                float y = part[0][q][lane];
#pragma unroll
                for (int i = 1; i < G_WAVES; ++i) y += part[i][q][lane];
                const float up = __shfl_xor(y, 32);
                const float h = gelu(y) * up;
                uint16_t dbits;
                const int qv = quant_q8_half(h, &dbits);
                store_prep_half(qv, dbits, lane & 31, hact + ((size_t)(k0 + q) * T + t) * ACT_DW, lane < 32);
            }
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(64) void k_down_grouped(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl,
                                                     const int32_t *__restrict__ gstart,
                                                     const uint32_t *__restrict__ hact, float *__restrict__ y, int T,
                                                     int S, int d) {
    const int t = blockIdx.x, e = blockIdx.y;
    const int g0 = gstart[e], g1 = gstart[e + 1];
    if (g0 >= g1) return;
    const int lane = threadIdx.x;
    const int kp = lane >> 5;
    const size_t base = ((size_t)e * T + t) * S;
    const uint4 *np = nib + base * 64 + lane;
    const uint16_t *sp = scl + base * 64 + lane;
    const int nb = 2 * S;
    for (int k0 = g0; k0 < g1; k0 += TB) {
        const int nt = min(TB, g1 - k0);
        float acc[TB] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int c = 0; c < S; c += G_CHUNK) {
            uint4 wv[G_CHUNK];
            uint16_t sv[G_CHUNK];
#pragma unroll
            for (int i = 0; i < G_CHUNK; ++i)
                if (c + i < S) {
                    wv[i] = np[(size_t)(c + i) * 64];
                    sv[i] = sp[(size_t)(c + i) * 64];
                }
#pragma unroll
            for (int i = 0; i < G_CHUNK; ++i)
                if (c + i < S) {
                    const float dw = h2f(sv[i]);
#pragma unroll
                    for (int q = 0; q < TB; ++q)
                        if (q < nt) {
                            const uint32_t *a = hact + ((size_t)(k0 + q) * nb + kp * S + c + i) * ACT_DW;
                            uint32_t av[9];
#pragma unroll
                            for (int r = 0; r < 9; ++r) av[r] = a[r];
                            const int sumi = block_dot(wv[i], av);
                            acc[q] = fmaf((float)sumi, dw * __builtin_bit_cast(float, av[8]), acc[q]);
                        }
                }
        }
#pragma unroll
        for (int q = 0; q < TB; ++q) {
            const float other = __shfl_xor(acc[q], 32);
            if (q < nt && lane < 32) y[(size_t)(k0 + q) * d + (size_t)t * 32 + lane] = acc[q] + other;
        }
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
    RVM_CHECK(layer_ok(L) && x && out && ws && n_tok > 0 && n_tok <= 65535);
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
    uint32_t *xact = (uint32_t *)(w + lay.xact);
    uint32_t *hact = (uint32_t *)(w + lay.hact);
    int rc = launch_router(L, x, n_tok, flags, eps, w, lay, ids, wts, nullptr);
    if (rc) return rc;
    const int pairs = n_tok * L->top_k;
    if ((rc = launch_plan(ids, pairs, L->n_exp, order, pos_of, gstart))) return rc;

    const int Tg = 2 * L->ff / 64, Sg = L->d / QK;
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * Sg;
    const uint4 *gnib = (const uint4 *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)((const uint8_t *)L->gate_up + gu_entries * 16);
    hipLaunchKernelGGL(k_gateup_grouped, dim3(Tg, L->n_exp), dim3(G_WAVES * 64), 0, cur_stream(), gnib, gscl, gstart,
                       order, xact, hact, Tg, Sg, L->top_k);
    if ((rc = launched())) return rc;

    const int Td = L->d / 32, Sd = L->ff / 64;
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint4 *dnib = (const uint4 *)L->down;
    const uint16_t *dscl = (const uint16_t *)((const uint8_t *)L->down + dn_entries * 16);
    hipLaunchKernelGGL(k_down_grouped, dim3(Td, L->n_exp), dim3(64), 0, cur_stream(), dnib, dscl, gstart, hact, y, Td,
                       Sd, L->d);
    if ((rc = launched())) return rc;

    hipLaunchKernelGGL(k_combine_pairs, dim3(n_tok), dim3(256), 0, cur_stream(), y, pos_of, ids, wts, L->down_scale,
                       out, L->top_k, L->d);
    return launched();
}
