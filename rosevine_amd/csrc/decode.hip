// decode.hip - one decode token through one MoE layer (runtime/src/exec.rs:456-475, 572-640;
// the device dispatch it replaces is runtime/src/hip_exec.rs:780-843).
//
// Three launches, each a full pass over its bytes with no host round trip:
//   1. k_router (router.hip): logits + certified top-k + weights, and the token's Q8_0
//      activation blocks, with the selection done by the last workgroup;
//   2. k_gateup_decode: top_k x (2ff/64) workgroups; each streams one 64-row tile (32 gate rows
//      and the matching 32 up rows) of its expert with the K range split over 8 waves, then
//      applies GeGLU and quantises the 32 resulting h values to one Q8_0 block in-register;
//   3. k_down_decode: d/32 workgroups of 8 waves; wave j streams slot j's 32-row down tile (two
//      half-waves split K) and wave 0 combines the 8 results in slot order.
// Every lane issues all of its 16-byte weight loads before the first use, and the activation
// blocks are staged once per workgroup in LDS and read as broadcasts.
#include "internal.hpp"

namespace rvm {

constexpr int GU_WAVES = 8;  // K split of the gate_up tile
constexpr int MAX_TOPK = 8;

// Staging of n uint4 from global to LDS in two steps, so that a kernel can issue these loads
// before its weight loads (the memory counter drains in order) and store them after: the source
// index is clamped so that the loads need no branch.
template <int MAXN, int NT>
struct Stage {
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

// This lane's PER block terms (sumi as f32) * (d_w * d_x): weights in registers, activation
// blocks in LDS (read as broadcasts).
template <int PER>
__device__ __forceinline__ void lane_terms(const uint4 (&wv)[PER], const uint32_t (&sv)[PER], const uint4 *act,
                                           float (&t)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint4 a0 = act[i * 3], a1 = act[i * 3 + 1];
        const float dx = __builtin_bit_cast(float, act[i * 3 + 2].x);
        const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        t[i] = block_term(block_dot(wv[i], a), h2f((uint16_t)sv[i]), dx);
    }
}

template <int PER>  // steps per wave = (d / 32) / GU_WAVES = d / 256
__global__ __launch_bounds__(GU_WAVES * 64) void k_gateup_decode(const uint4 *__restrict__ nib,
                                                                 const uint16_t *__restrict__ scl,
                                                                 const int32_t *__restrict__ ids,
                                                                 const uint4 *__restrict__ xact,
                                                                 uint32_t *__restrict__ hact, int T) {
    constexpr int S = PER * GU_WAVES;
    using St = Stage<S * 3, GU_WAVES * 64>;
    __shared__ uint4 act[St::SLOTS];
    __shared__ float terms[64][S + 1];  // odd pitch: the folding lanes read different banks
    const int slot = blockIdx.x / T, t = blockIdx.x - slot * T;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int e = ids[slot];
    const size_t base = (((size_t)e * T + t) * S + (size_t)w * PER) * 64 + lane;
    St st;
    st.load(xact, S * 3);
    __builtin_amdgcn_sched_barrier(0);  // activation loads first: the memory counter drains in order
    uint4 wv[PER];
    uint32_t sv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        wv[i] = nib[base + (size_t)i * 64];
        sv[i] = scl[base + (size_t)i * 64];
    }
    __builtin_amdgcn_sched_barrier(0);
    st.store(act);
    __syncthreads();
    float tv[PER];
    lane_terms<PER>(wv, sv, act + w * PER * 3, tv);
#pragma unroll
    for (int i = 0; i < PER; ++i) terms[lane][w * PER + i] = tv[i];
    __syncthreads();
    if (w == 0) {
        // the reference's sequential fold of the row's S block terms (expert_kernel.rs:148-159)
        float y = 0.0f;
#pragma unroll 8
        for (int b = 0; b < S; ++b) y = y + terms[lane][b];
        const float up = __shfl_xor(y, 32);  // lane l < 32 holds gate row l, lane l + 32 its up row
        const float h = gelu(y) * up;
        uint16_t dbits;
        const int q = quant_q8_half(h, &dbits);
        store_prep_half(q, dbits, lane & 31, hact + ((size_t)slot * T + t) * ACT_DW, lane < 32);
    }
}

template <int S>  // steps per lane = ff / 64
__global__ __launch_bounds__(MAX_TOPK * 64) void k_down_decode(const uint4 *__restrict__ nib,
                                                               const uint16_t *__restrict__ scl,
                                                               const int32_t *__restrict__ ids,
                                                               const float *__restrict__ wts,
                                                               const float *__restrict__ dscale,
                                                               const uint4 *__restrict__ hact,
                                                               float *__restrict__ out, int T, int top_k) {
    constexpr int NB = 2 * S;  // h blocks per slot
    using St = Stage<MAX_TOPK * NB * 3, MAX_TOPK * 64>;
    __shared__ uint4 act[St::SLOTS];
    __shared__ float ys[MAX_TOPK][32];
    const int t = blockIdx.x;
    const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    St st;
    st.load(hact, top_k * NB * 3);
    __builtin_amdgcn_sched_barrier(0);  // activation loads first: the memory counter drains in order
    // Waves past top_k load slot 0's tile too (unused) so that the loads need no branch.
    const int e = ids[j < top_k ? j : 0];
    const size_t base = ((size_t)e * T + t) * S * 64 + lane;
    uint4 wv[S];
    uint32_t sv[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
        wv[i] = nib[base + (size_t)i * 64];
        sv[i] = scl[base + (size_t)i * 64];
    }
    __builtin_amdgcn_sched_barrier(0);
    st.store(act);
    __syncthreads();
    {
        // computed by every wave (those past top_k on slot 0's data) so that the weight loads stay
        // ahead of the barrier instead of sinking into a branch
        const int kp = lane >> 5;
        float tv[S];
        lane_terms<S>(wv, sv, act + ((j < top_k ? j : 0) * NB + kp * S) * 3, tv);
        // sequential fold in block order: this half's blocks, then the other half's (lanes < 32
        // hold blocks 0..S-1 and receive S..2S-1 from lane + 32)
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < S; ++i) acc = acc + tv[i];
#pragma unroll
        for (int i = 0; i < S; ++i) acc = acc + __shfl_xor(tv[i], 32);
        if (j < top_k && lane < 32) ys[j][lane] = acc;
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

    const int Tg = 2 * L->ff / 64;
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint4 *gnib = (const uint4 *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)((const uint8_t *)L->gate_up + gu_entries * 16);
    rc = with_steps(L->d / 256, [&](auto per) {
        hipLaunchKernelGGL(k_gateup_decode<decltype(per)::value>, dim3(L->top_k * Tg), dim3(GU_WAVES * 64), 0,
                           cur_stream(), gnib, gscl, ids, (const uint4 *)(w + lay.xact), (uint32_t *)(w + lay.hact),
                           Tg);
        return launched();
    });
    if (rc) return rc;

    const int Td = L->d / 32;
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint4 *dnib = (const uint4 *)L->down;
    const uint16_t *dscl = (const uint16_t *)((const uint8_t *)L->down + dn_entries * 16);
    return with_steps(L->ff / 64, [&](auto s) {
        hipLaunchKernelGGL(k_down_decode<decltype(s)::value>, dim3(Td), dim3(MAX_TOPK * 64), 0, cur_stream(), dnib,
                           dscl, ids, wts, L->down_scale, (const uint4 *)(w + lay.hact), out, Td, L->top_k);
        return launched();
    });
}
