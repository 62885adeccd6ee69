// decode.hip - one decode token through one MoE layer (runtime/src/exec.rs:456-475, 572-640;
// the device dispatch it replaces is runtime/src/hip_exec.rs:780-843).
//
// Three launches, each a full pass over its bytes with no host round trip:
//   1. k_router (router.hip): the logit statistics and the token's Q8_0 activation blocks;
//   2. k_gateup_decode: 1 + top_k x (2ff/64) workgroups. Each tile workgroup ranks the experts
//      by the statistics itself (select.hpp) and streams one 64-row tile (32 gate rows and the
//      matching 32 up rows) of its slot's expert with the K range split over 8 waves, folds each
//      row's block terms in block order, applies GeGLU and quantises the 32 h values to one Q8_0
//      block. Workgroup 0 certifies that ranking, or computes the exact selection when it cannot
//      be certified, publishes ids and weights, and computes any expert the ranking missed;
//   3. k_down_decode: d/32 workgroups of 8 waves; wave j streams slot j's 32-row down tile (two
//      half-waves split K) and wave 0 combines the 8 results in slot order.
// Every lane issues all of its 16-byte weight loads before the first use, the activation blocks
// are staged once per workgroup in LDS, and each wave reads its blocks from LDS in one burst.
#include "select.hpp"

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

// This lane's N block terms (sumi as f32) * (d_w * d_x): weights in registers, the N prepared
// activation blocks read from LDS in one burst first (they are the same for every lane).
template <int N>
__device__ __forceinline__ void lane_terms(const uint4 (&wv)[N], const uint32_t (&sv)[N], const uint4 *act,
                                           float (&t)[N]) {
    uint4 a0[N], a1[N];
    float dx[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        a0[i] = act[i * 3];
        a1[i] = act[i * 3 + 1];
        dx[i] = __builtin_bit_cast(float, act[i * 3 + 2].x);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint32_t a[8] = {a0[i].x, a0[i].y, a0[i].z, a0[i].w, a1[i].x, a1[i].y, a1[i].z, a1[i].w};
        t[i] = block_term(block_dot(wv[i], a), h2f((uint16_t)sv[i]), dx[i]);
    }
}

// LDS of the gate_up kernel: the selection's scratch is dead once the expert is known, and the
// block terms [block][lane] take its place.
template <int PER>
union GateUpShared {
    SelShared<PER, GU_WAVES> sel;
    float terms[PER * GU_WAVES][64];
};

// One 64-row tile t of expert e: every wave loads its PER steps (16-byte nibble entries and the
// scales), the activation blocks are stored to LDS from st (when STAGE) behind the loads, each
// lane forms its block terms, and wave 0 folds each row's terms in block order (the reference's
// sequential fold, expert_kernel.rs:148-159), pairs gate row l with up row l + 32, applies GeGLU
// and writes the Q8_0 block of the tile's 32 h values to hdst. Called by every thread.
template <int PER, bool STAGE, class St>
__device__ __forceinline__ void gateup_tile(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl, int e,
                                            int t, int T, const St &st, uint4 *act, float (*terms)[64],
                                            uint32_t *__restrict__ hdst) {
    constexpr int S = PER * GU_WAVES;
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
    __builtin_amdgcn_sched_barrier(0);
    if (STAGE) st.store(act);
    __syncthreads();  // act is staged; and the previous user of terms is done
    float tv[PER];
    lane_terms<PER>(wv, sv, act + w * PER * 3, tv);
#pragma unroll
    for (int i = 0; i < PER; ++i) terms[w * PER + i][lane] = tv[i];
    __syncthreads();
    if (w == 0) {
        float tt[S];  // every term read from LDS before the first add
#pragma unroll
        for (int b = 0; b < S; ++b) tt[b] = terms[b][lane];
        float y = 0.0f;
#pragma unroll
        for (int b = 0; b < S; ++b) y = y + tt[b];
        const float up = __shfl_xor(y, 32);  // lane l < 32 holds gate row l, lane l + 32 its up row
        const float h = gelu(y) * up;
        uint16_t dbits;
        const int q = quant_q8_half(h, &dbits);
        store_prep_half(q, dbits, lane & 31, hdst, lane < 32);
    }
}

__device__ __forceinline__ int clamp_expert(int e, int n_exp) { return (unsigned)e < (unsigned)n_exp ? e : 0; }

// Workgroup 0 selects: it certifies the S ranking or runs the exact selection, publishes the
// reference's ids and weights, and maps each selected slot to the h rows that hold its expert
// (hslot): the slot of the S ranking that computed the same expert, or a correction row that it
// computes itself for an expert the S ranking missed. Workgroups 1.. each take slot (b / T),
// tile (b % T) of the S ranking's experts.
template <int PER>  // steps per wave = (d / 32) / GU_WAVES = d / 256
__global__ __launch_bounds__(GU_WAVES * 64) void k_gateup_decode(
    const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl, const double2 *__restrict__ stats,
    const float *__restrict__ bias, const float *__restrict__ W, const float *__restrict__ x, int n_exp, int top_k,
    int pre_norm, float eps, int exact, uint32_t *__restrict__ ctl, int32_t *__restrict__ ids,
    float *__restrict__ wts, const uint4 *__restrict__ xact, uint32_t *__restrict__ hact, int T) {
    constexpr int S = PER * GU_WAVES;
    using St = Stage<S * 3, GU_WAVES * 64>;
    __shared__ uint4 act[St::SLOTS];
    __shared__ GateUpShared<PER> u;
    __shared__ int fix_e[MAX_TOPK];
    __shared__ int n_fix;
    const int lane = threadIdx.x & 63;
    St st;
    st.load(xact, S * 3);  // in flight during the selection
    if (blockIdx.x > 0) {
        const int b = blockIdx.x - 1, slot = b / T, t = b - slot * T;
        select_token<PER, GU_WAVES, false>(u.sel, stats, bias, W, x, n_exp, top_k, pre_norm, eps, exact, false, false,
                                           ctl, nullptr);
        const int e = __builtin_amdgcn_readfirstlane(clamp_expert(spec_id(u.sel, slot, top_k), n_exp));
        gateup_tile<PER, true>(nib, scl, e, t, T, st, act, u.terms, hact + ((size_t)slot * T + t) * ACT_DW);
        return;
    }
    select_token<PER, GU_WAVES>(u.sel, stats, bias, W, x, n_exp, top_k, pre_norm, eps, exact, true, true, ctl,
                                nullptr);
    if (u.sel.pass) select_weights<PER, GU_WAVES>(u.sel, n_exp, top_k);
    __syncthreads();
    if (threadIdx.x < 64) {
        const int ex = lane < top_k ? u.sel.sel[lane] : -1;
        int found = -1;
        for (int j = 0; j < top_k; ++j)
            if (found < 0 && clamp_expert(u.sel.spec[j], n_exp) == ex) found = j;
        const bool need = lane < top_k && found < 0;
        const uint64_t nm = __ballot(need);
        const int m = __popcll(nm & ((1ull << lane) - 1ull));
        if (lane < top_k) {
            ids[lane] = ex;
            wts[lane] = u.sel.wsel[lane];
            ((int32_t *)ctl)[16 + lane] = need ? top_k + m : found;  // hslot
        }
        if (need) fix_e[m] = ex;
        if (lane == 0) n_fix = __popcll(nm);
    }
    __syncthreads();
    // experts the S ranking missed: all their tiles, into the correction rows (rare: the exact
    // selection changed the set of experts)
    for (int m = 0; m < n_fix; ++m)
        for (int t = 0; t < T; ++t) {
            if (m == 0 && t == 0)
                gateup_tile<PER, true>(nib, scl, fix_e[m], t, T, st, act, u.terms,
                                       hact + ((size_t)(top_k + m) * T + t) * ACT_DW);
            else
                gateup_tile<PER, false>(nib, scl, fix_e[m], t, T, st, act, u.terms,
                                        hact + ((size_t)(top_k + m) * T + t) * ACT_DW);
        }
}

template <int S>  // steps per lane = ff / 64
__global__ __launch_bounds__(MAX_TOPK * 64) void k_down_decode(const uint4 *__restrict__ nib,
                                                               const uint16_t *__restrict__ scl,
                                                               const int32_t *__restrict__ ids,
                                                               const float *__restrict__ wts,
                                                               const int32_t *__restrict__ hslot,
                                                               const float *__restrict__ dscale,
                                                               const uint4 *__restrict__ hact,
                                                               float *__restrict__ out, int T, int top_k) {
    constexpr int NB = 2 * S;  // h blocks per slot
    constexpr int IT = (MAX_TOPK * NB * 3 + MAX_TOPK * 64 - 1) / (MAX_TOPK * 64);
    __shared__ uint4 act[IT * MAX_TOPK * 64];
    __shared__ float half2[MAX_TOPK][S][32];  // the second half's block terms of each row
    __shared__ float ys[MAX_TOPK][32];
    __shared__ float coef[2][MAX_TOPK];
    const int t = blockIdx.x;
    const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    // Waves past top_k load slot 0's tile too (unused) so that the loads need no branch.
    const int e = ids[j < top_k ? j : 0];
    if (threadIdx.x < (unsigned)top_k) {
        coef[0][threadIdx.x] = dscale ? dscale[ids[threadIdx.x]] : 1.0f;
        coef[1][threadIdx.x] = wts[threadIdx.x];
    }
    // slot k's h blocks are the hslot[k]-th row of blocks of hact (gathered; indices clamped so
    // that the loads need no branch)
    uint4 av[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
        const int idx = min((int)threadIdx.x + i * MAX_TOPK * 64, top_k * NB * 3 - 1);
        const int k = idx / (NB * 3);
        const int row = min((unsigned)hslot[k], (unsigned)(2 * top_k - 1));
        av[i] = hact[(size_t)row * NB * 3 + (idx - k * NB * 3)];
    }
    __builtin_amdgcn_sched_barrier(0);  // activation loads first: the memory counter drains in order
    const size_t base = ((size_t)e * T + t) * S * 64 + lane;
    uint4 wv[S];
    uint32_t sv[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
        wv[i] = nib[base + (size_t)i * 64];
        sv[i] = scl[base + (size_t)i * 64];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < IT; ++i) act[threadIdx.x + i * MAX_TOPK * 64] = av[i];
    __syncthreads();
    {
        // computed by every wave (those past top_k on slot 0's data) so that the weight loads stay
        // ahead of the barrier instead of sinking into a branch
        const int kp = lane >> 5;
        float tv[S];
        lane_terms<S>(wv, sv, act + ((j < top_k ? j : 0) * NB + kp * S) * 3, tv);
        // sequential fold in block order: lanes < 32 hold blocks 0..S-1 of row `lane`, lanes
        // + 32 blocks S..2S-1 of the same row, passed through LDS
        if (lane >= 32) {
#pragma unroll
            for (int i = 0; i < S; ++i) half2[j][i][lane - 32] = tv[i];
        }
        wave_lds_sync();
        if (lane < 32) {
            float hv[S];
#pragma unroll
            for (int i = 0; i < S; ++i) hv[i] = half2[j][i][lane];
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < S; ++i) acc = acc + tv[i];
#pragma unroll
            for (int i = 0; i < S; ++i) acc = acc + hv[i];
            if (j < top_k) ys[j][lane] = acc;
        }
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        // (y * ds) * w in slot order, the first term assigned (runtime/src/exec.rs:626-638)
        float o = 0.0f;
        for (int jj = 0; jj < top_k; ++jj) {
            const float v = ys[jj][threadIdx.x] * coef[0][jj] * coef[1][jj];
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
    int rc = launch_router(L, x, 1, flags, eps, w, lay, ids, wts, nullptr, false);
    if (rc) return rc;

    const int Tg = 2 * L->ff / 64;
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint4 *gnib = (const uint4 *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)((const uint8_t *)L->gate_up + gu_entries * 16);
    const int pre = (flags & RVM_PRE_NORM) ? 1 : 0, exact = (flags & RVM_EXACT_SELECT) ? 1 : 0;
    rc = with_steps(L->d / 256, [&](auto per) {
        hipLaunchKernelGGL(k_gateup_decode<decltype(per)::value>, dim3(1 + L->top_k * Tg), dim3(GU_WAVES * 64), 0,
                           cur_stream(), gnib, gscl, (const double2 *)(w + lay.stats), L->router_bias, L->router, x,
                           L->n_exp, L->top_k, pre, eps, exact, (uint32_t *)(w + lay.ctl), ids, wts,
                           (const uint4 *)(w + lay.xact), (uint32_t *)(w + lay.hact), Tg);
        return launched();
    });
    if (rc) return rc;

    const int Td = L->d / 32;
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint4 *dnib = (const uint4 *)L->down;
    const uint16_t *dscl = (const uint16_t *)((const uint8_t *)L->down + dn_entries * 16);
    return with_steps(L->ff / 64, [&](auto s) {
        hipLaunchKernelGGL(k_down_decode<decltype(s)::value>, dim3(Td), dim3(MAX_TOPK * 64), 0, cur_stream(), dnib,
                           dscl, ids, wts, (const int32_t *)(w + lay.ctl) + 16, L->down_scale,
                           (const uint4 *)(w + lay.hact), out, Td, L->top_k);
        return launched();
    });
}
