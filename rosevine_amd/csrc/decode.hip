// decode.hip - one decode token through one MoE layer (runtime/src/exec.rs:456-475, 572-640;
// the device dispatch it replaces is runtime/src/hip_exec.rs:780-843).
//
// Three launches, each a full pass over its bytes with no host round trip:
//   1. k_router (router.hip): logits + certified top-k + weights, and the token's Q8_0
//      activation blocks, with the selection done by the last workgroup;
//   2. k_gateup_decode: top_k x (2ff/64) workgroups; each streams one 64-row tile (32 gate rows
//      and the matching 32 up rows) of its expert with the K range split over 4 waves, then
//      applies GeGLU and quantises the 32 resulting h values to one Q8_0 block in-register;
//   3. k_down_decode: d/32 workgroups of 8 waves; wave j streams slot j's 32-row down tile (two
//      half-waves split K) and wave 0 combines the 8 results in slot order.
// The weights are read once per token with 16-byte coalesced loads from the packed planes.
#include "internal.hpp"

namespace rvm {

constexpr int GU_WAVES = 4;  // K split of the gate_up tile
constexpr int CHUNK = 11;    // weight loads issued ahead per lane
constexpr int MAX_TOPK = 8;

__global__ __launch_bounds__(GU_WAVES * 64) void k_gateup_decode(const uint4 *__restrict__ nib,
                                                                 const uint16_t *__restrict__ scl,
                                                                 const int32_t *__restrict__ ids,
                                                                 const uint32_t *__restrict__ xact,
                                                                 uint32_t *__restrict__ hact, int T, int S) {
    __shared__ float part[GU_WAVES][64];
    const int slot = blockIdx.x / T, t = blockIdx.x - slot * T;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int e = ids[slot];
    const int per = S / GU_WAVES;
    const int s0 = w * per;
    const size_t base = ((size_t)e * T + t) * S + s0;
    const uint4 *np = nib + base * 64 + lane;
    const uint16_t *sp = scl + base * 64 + lane;
    const uint32_t *ap = xact + (size_t)s0 * ACT_DW;
    float acc = 0.0f;
    for (int c = 0; c < per; c += CHUNK) {
        uint4 wv[CHUNK];
        uint16_t sv[CHUNK];
#pragma unroll
        for (int i = 0; i < CHUNK; ++i)
            if (c + i < per) {
                wv[i] = np[(size_t)(c + i) * 64];
                sv[i] = sp[(size_t)(c + i) * 64];
            }
#pragma unroll
        for (int i = 0; i < CHUNK; ++i)
            if (c + i < per) {
                const uint32_t *a = ap + (c + i) * ACT_DW;
                const int sumi = block_dot(wv[i], a);
                acc = fmaf((float)sumi, h2f(sv[i]) * __builtin_bit_cast(float, a[8]), acc);
            }
    }
    part[w][lane] = acc;
    __syncthreads();
    if (w == 0) {
        float y = part[0][lane];
#pragma unroll
        for (int i = 1; i < GU_WAVES; ++i) y += part[i][lane];
        const float up = __shfl_xor(y, 32);  // lane l < 32 holds gate row l, lane l + 32 its up row
        const float h = gelu(y) * up;
        uint16_t dbits;
        const int q = quant_q8_half(h, &dbits);
        store_prep_half(q, dbits, lane & 31, hact + ((size_t)slot * T + t) * ACT_DW, lane < 32);
    }
}

__global__ __launch_bounds__(MAX_TOPK * 64) void k_down_decode(const uint4 *__restrict__ nib,
                                                               const uint16_t *__restrict__ scl,
                                                               const int32_t *__restrict__ ids,
                                                               const float *__restrict__ wts,
                                                               const float *__restrict__ dscale,
                                                               const uint32_t *__restrict__ hact,
                                                               float *__restrict__ out, int T, int S, int top_k) {
    extern __shared__ uint32_t act[];  // [top_k][2S][ACT_DW]
    __shared__ float ys[MAX_TOPK][32];
    const int t = blockIdx.x;
    const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int per_slot = 2 * S * ACT_DW;
    for (int i = threadIdx.x; i < top_k * per_slot; i += blockDim.x) act[i] = hact[i];
    __syncthreads();
    if (j < top_k) {
        const int e = ids[j];
        const int kp = lane >> 5;
        const size_t base = ((size_t)e * T + t) * S;
        const uint4 *np = nib + base * 64 + lane;
        const uint16_t *sp = scl + base * 64 + lane;
        const uint32_t *ab = act + j * per_slot + kp * S * ACT_DW;
        float acc = 0.0f;
        for (int c = 0; c < S; c += CHUNK) {
            uint4 wv[CHUNK];
            uint16_t sv[CHUNK];
#pragma unroll
            for (int i = 0; i < CHUNK; ++i)
                if (c + i < S) {
                    wv[i] = np[(size_t)(c + i) * 64];
                    sv[i] = sp[(size_t)(c + i) * 64];
                }
#pragma unroll
            for (int i = 0; i < CHUNK; ++i)
                if (c + i < S) {
                    const uint32_t *a = ab + (c + i) * ACT_DW;
                    uint32_t av[9];
#pragma unroll
                    for (int q = 0; q < 9; ++q) av[q] = a[q];
                    const int sumi = block_dot(wv[i], av);
                    acc = fmaf((float)sumi, h2f(sv[i]) * __builtin_bit_cast(float, av[8]), acc);
                }
        }
        const float other = __shfl_xor(acc, 32);  // half 0 + half 1
        if (lane < 32) ys[j][lane] = acc + other;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        float o = 0.0f;
        for (int jj = 0; jj < top_k; ++jj) {
            const float ds = dscale ? dscale[ids[jj]] : 1.0f;
            const float v = ys[jj][threadIdx.x] * ds * wts[jj];
            o = jj == 0 ? v : o + v;
        }
        out[(size_t)t * 32 + threadIdx.x] = o;
    }
}

}  // namespace rvm

using namespace rvm;

extern "C" int rvm_moe_decode(const rvm_layer *L, const float *x, float *out, int flags, float eps, void *ws,
                              size_t ws_bytes) {
    RVM_CHECK(layer_ok(L) && x && out && ws);
    const WsLayout lay = ws_layout(L, 1);
    RVM_CHECK(ws_bytes >= lay.total);
    uint8_t *w = (uint8_t *)ws;
    int32_t *ids = (int32_t *)(w + lay.ids);
    float *wts = (float *)(w + lay.wts);
    int rc = launch_router(L, x, 1, flags, eps, w, lay, ids, wts, nullptr);
    if (rc) return rc;

    const int Tg = 2 * L->ff / 64, Sg = L->d / QK;  // d % 256 == 0, so Sg % GU_WAVES == 0
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * Sg;
    const uint4 *gnib = (const uint4 *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)((const uint8_t *)L->gate_up + gu_entries * 16);
    hipLaunchKernelGGL(k_gateup_decode, dim3(L->top_k * Tg), dim3(GU_WAVES * 64), 0, cur_stream(), gnib, gscl, ids,
                       (const uint32_t *)(w + lay.xact), (uint32_t *)(w + lay.hact), Tg, Sg);
    if ((rc = launched())) return rc;

    const int Td = L->d / 32, Sd = L->ff / 64;
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint4 *dnib = (const uint4 *)L->down;
    const uint16_t *dscl = (const uint16_t *)((const uint8_t *)L->down + dn_entries * 16);
    const size_t smem = (size_t)L->top_k * 2 * Sd * ACT_DW * 4;
    hipLaunchKernelGGL(k_down_decode, dim3(Td), dim3(MAX_TOPK * 64), smem, cur_stream(), dnib, dscl, ids, wts,
                       L->down_scale, (const uint32_t *)(w + lay.hact), out, Td, Sd, L->top_k);
    return launched();
}
