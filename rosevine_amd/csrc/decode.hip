// decode.hip - one decode token through one MoE layer (runtime/src/exec.rs:456-475, 572-640;
// the device dispatch it replaces is runtime/src/hip_exec.rs:780-843).
//
// Three launches, each a full pass over its bytes with no host round trip:
//   1. k_router (router.hip): the logit statistics and the token's Q8_0 activation blocks;
//   2. k_gateup_decode: 1 + top_k x (2ff/64) workgroups. Each tile workgroup ranks the experts
//      by the statistics itself (select.hpp) and streams one 64-row tile (32 gate rows and the
//      matching 32 up rows) of its slot's expert with the K range split over 8 waves, folds each
//      row's block terms in block order, applies GeGLU and quantises the 32 h values to one Q8_0
//      block t of h; with the down entries of block t of every down row of the same expert (loaded
//      with the gate/up entries), it then writes the down terms of that h block for all d rows.
//      Workgroup 0 certifies that ranking, or computes the exact selection when it cannot be
//      certified, publishes ids and weights, and computes any expert the ranking missed;
//   3. k_down_fold: d/32 workgroups; each folds the ff/32 down terms of its 32 rows for every slot
//      in block order and combines the slots in slot order.
// Every lane issues all of its 16-byte weight loads before the first use, the activation blocks
// are staged once per workgroup in LDS, and each wave reads its blocks from LDS in one burst.
#include <mutex>

#include "select.hpp"

namespace rvm {

constexpr int GU_WAVES = 8;  // K split of the gate_up tile

#ifdef RVM_PHASE_TRACE
// k_gateup_decode (0): 0 entry, 1 expert known (workgroup 0: ranking done), 2 wave 0's block terms
// formed (workgroup 0: ids and weights published), 3 h block ready, 4 down terms stored;
// k_down_fold (1): 0 entry, 1 slot rows folded, 2 output stored, 3 down terms loaded
namespace {
__device__ unsigned long long g_stamp[2 * TRACE_WG * TRACE_PT];
}  // namespace
#endif
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

// One 64-row tile t of expert e, and the down terms of the h block it produces.
//   gate/up: every wave loads its PER steps (16-byte nibble entries and the scales), the activation
//   blocks are stored to LDS from st (when STAGE) behind the loads, each lane forms its block
//   terms, and wave 0 folds each row's terms in block order (the reference's sequential fold,
//   expert_kernel.rs:148-159), pairs gate row l with up row l + 32, applies GeGLU and writes the
//   Q8_0 block t of h (32 values) to hdst and to LDS.
//   down: h block t meets block t of every down row r of the same expert: thread i forms the terms
//   (sumi as f32) * (d_w * d_h) of rows i, i + 512, ... (their entries are loaded with the gate/up
//   ones) and writes them to dterm[r]; the down kernel folds each row's T terms in block order.
// Called by every thread.
template <int PER, bool STAGE, bool NT, class St>
__device__ __forceinline__ void gateup_tile(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl,
                                            const uint4 *__restrict__ dnib, const uint16_t *__restrict__ dscl,
                                            int e, int t, int T, const St &st, uint4 *act, float (*terms)[64],
                                            uint32_t *hprep, uint32_t *__restrict__ hdst, float *__restrict__ dterm) {
    constexpr int S = PER * GU_WAVES, d = 256 * PER, RD = (d + GU_WAVES * 64 - 1) / (GU_WAVES * 64);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    // The activation blocks go to LDS before the weight loads are issued: a barrier behind a
    // wave's full set of weight loads would wait until the memory pipeline had taken them all,
    // and the block terms below are formed as their weights arrive.
    if (STAGE) st.store(act);
    __syncthreads();  // act is staged; and the previous user of terms and hprep is done
    const size_t base = (((size_t)e * T + t) * S + (size_t)w * PER) * 64 + lane;
    uint4 wv[PER];
    uint32_t sv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        wv[i] = ld_weights<NT>(nib + base + (size_t)i * 64);
        sv[i] = ld_weights<NT>(scl + base + (size_t)i * 64);
    }
    // down entries of block t: RVM_PACK_ROWS32 with Sd = T / 2 steps; row r is lane
    // (r & 31) + 32 * (t / Sd) of tile r / 32 at step t % Sd
    const int Sd = T >> 1, half = t >= Sd ? 1 : 0, sd = t - half * Sd, Td = d / 32;
    uint4 dv[RD];
    uint32_t ds[RD];
#pragma unroll
    for (int i = 0; i < RD; ++i) {
        const int r = min((int)threadIdx.x + i * GU_WAVES * 64, d - 1);
        const size_t ent = (((size_t)e * Td + (r >> 5)) * Sd + sd) * 64 + 32 * half + (r & 31);
        dv[i] = ld_weights<NT>(dnib + ent);
        ds[i] = ld_weights<NT>(dscl + ent);
    }
    __builtin_amdgcn_sched_barrier(0);
    float tv[PER];
    lane_terms<PER>(wv, sv, act + w * PER * 3, tv);
    RVM_STAMP(g_stamp, 0, 2);
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
        store_prep_half(q, dbits, lane & 31, hprep, lane < 32);
    }
    __syncthreads();
    RVM_STAMP(g_stamp, 0, 3);
    {
        const uint4 *hp = (const uint4 *)hprep;
        const uint4 a0 = hp[0], a1 = hp[1];
        const float dx = __builtin_bit_cast(float, hp[2].x);
        const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int i = 0; i < RD; ++i) {
            const int r = (int)threadIdx.x + i * GU_WAVES * 64;
            const float term = block_term(block_dot(dv[i], a), h2f((uint16_t)ds[i]), dx);
            if (r < d) dterm[r] = term;
        }
    }
    RVM_STAMP(g_stamp, 0, 4);
}

__device__ __forceinline__ int clamp_expert(int e, int n_exp) { return (unsigned)e < (unsigned)n_exp ? e : 0; }

// Workgroup 0 selects: it certifies the S ranking or runs the exact selection, publishes the
// reference's ids and weights, and maps each selected slot to the h rows that hold its expert
// (hslot): the slot of the S ranking that computed the same expert, or a correction row that it
// computes itself for an expert the S ranking missed. Workgroups 1.. each take slot (b / T),
// tile (b % T) of the S ranking's experts.
template <int PER, bool NT>  // steps per wave = (d / 32) / GU_WAVES = d / 256; NT: streaming weight loads
__global__ __launch_bounds__(GU_WAVES * 64) void k_gateup_decode(
    const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl, const uint4 *__restrict__ dnib,
    const uint16_t *__restrict__ dscl, const double2 *__restrict__ stats, const float *__restrict__ bias,
    const float *__restrict__ W, const float *__restrict__ x, int n_exp, int top_k, XForm xf, int exact,
    uint32_t *__restrict__ ctl, int32_t *__restrict__ ids, float *__restrict__ wts, const uint4 *__restrict__ xact,
    uint32_t *__restrict__ hact, float *__restrict__ dterm, int T) {
    constexpr int S = PER * GU_WAVES, d = 256 * PER;
    using St = Stage<S * 3, GU_WAVES * 64>;
    __shared__ uint4 act[St::SLOTS];
    __shared__ GateUpShared<PER> u;
    __shared__ uint4 hprep[3];
    __shared__ int fix_e[MAX_TOPK];
    __shared__ int n_fix;
    // Every argument into scalar registers before the first load is issued: the compiler would
    // otherwise fetch part of them after it, a second round trip on the selection's path.
    asm volatile("" ::"s"(nib), "s"(scl), "s"(dnib), "s"(dscl), "s"(stats), "s"(bias), "s"(W), "s"(x), "s"(n_exp),
                 "s"(top_k), "s"(xf.pre_norm), "s"(xf.eps), "s"(xf.rpost), "s"(xf.rg), "s"(xf.eg), "s"(exact), "s"(ctl), "s"(ids), "s"(wts), "s"(xact), "s"(hact),
                 "s"(dterm), "s"(T));
    const int lane = threadIdx.x & 63;
    RVM_STAMP(g_stamp, 0, 0);
    St st;
    st.load(xact, S * 3);  // in flight during the selection
    if (blockIdx.x > 0) {
        const int b = blockIdx.x - 1, slot = b / T, t = b - slot * T;
        select_token<PER, GU_WAVES, false>(u.sel, stats, bias, W, x, n_exp, top_k, xf, exact, false, false,
                                           ctl, nullptr);
        const int e = __builtin_amdgcn_readfirstlane(clamp_expert(spec_id(u.sel, slot, top_k), n_exp));
        RVM_STAMP(g_stamp, 0, 1);
        gateup_tile<PER, true, NT>(nib, scl, dnib, dscl, e, t, T, st, act, u.terms, (uint32_t *)hprep,
                               hact + ((size_t)slot * T + t) * ACT_DW, dterm + ((size_t)slot * T + t) * d);
        return;
    }
    select_token<PER, GU_WAVES>(u.sel, stats, bias, W, x, n_exp, top_k, xf, exact, true, true, ctl,
                                nullptr);
    RVM_STAMP(g_stamp, 0, 1);
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
    RVM_STAMP(g_stamp, 0, 2);
    // experts the S ranking missed: all their tiles, into the correction rows (rare: the exact
    // selection changed the set of experts)
    for (int m = 0; m < n_fix; ++m)
        for (int t = 0; t < T; ++t) {
            const size_t row = (size_t)(top_k + m) * T + t;
            if (m == 0 && t == 0)
                gateup_tile<PER, true, NT>(nib, scl, dnib, dscl, fix_e[m], t, T, st, act, u.terms, (uint32_t *)hprep,
                                       hact + row * ACT_DW, dterm + row * d);
            else
                gateup_tile<PER, false, NT>(nib, scl, dnib, dscl, fix_e[m], t, T, st, act, u.terms, (uint32_t *)hprep,
                                        hact + row * ACT_DW, dterm + row * d);
        }
}

// Down and combine: thread (slot k, row) folds the T = 2S down terms of its row in block order
// (dot_q8_scalar's sequential fold from 0.0), then the first 32 threads combine (y * ds) * w in
// slot order, the first term assigned (runtime/src/exec.rs:626-638). The terms of selected slot k
// sit in the h row hslot[k]; that is k unless the exact selection changed the experts, so the
// terms are read for k first and again only when the map differs. Every global load is issued
// before the first use.
template <int S>  // ff / 64
__global__ __launch_bounds__(256) void k_down_fold(const float *__restrict__ dterm, const int32_t *__restrict__ ids,
                                                   const float *__restrict__ wts, const int32_t *__restrict__ hslot,
                                                   const float *__restrict__ dscale, float *__restrict__ out, int d,
                                                   int top_k) {
    constexpr int T = 2 * S;
    __shared__ float ys[MAX_TOPK][32];
    __shared__ float coef[2][MAX_TOPK];  // ds and w of each slot
    const int row = blockIdx.x * 32 + (threadIdx.x & 31);
    const int k = threadIdx.x >> 5;  // slot
    const int kc = min(k, top_k - 1);
    RVM_STAMP(g_stamp, 1, 0);
    float v[T];
#pragma unroll
    for (int t = 0; t < T; ++t) v[t] = dterm[((size_t)kc * T + t) * d + row];
    if (threadIdx.x < (unsigned)top_k) {
        coef[0][threadIdx.x] = dscale ? dscale[ids[threadIdx.x]] : 1.0f;
        coef[1][threadIdx.x] = wts[threadIdx.x];
    }
    bool moved = false;
    for (int j = 0; j < top_k; ++j) moved |= hslot[j] != j;
    if (moved) {
        const int hr = min((unsigned)hslot[kc], (unsigned)(2 * top_k - 1));
#pragma unroll
        for (int t = 0; t < T; ++t) v[t] = dterm[((size_t)hr * T + t) * d + row];
    }
    RVM_STAMP_LOADED(g_stamp, 1, 3);
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) acc = acc + v[t];
    if (k < top_k) ys[k][threadIdx.x & 31] = acc;
    RVM_STAMP(g_stamp, 1, 1);
    __syncthreads();
    if (threadIdx.x < 32) {
        float o = 0.0f;
        for (int j = 0; j < top_k; ++j) {
            const float cj = ys[j][threadIdx.x] * coef[0][j] * coef[1][j];
            o = j == 0 ? cj : o + cj;
        }
        out[row] = o;
    }
    RVM_STAMP(g_stamp, 1, 2);
}

}  // namespace rvm

using namespace rvm;

namespace rvm {

// One decode token through the layer, scratch in ws (ws_layout(L, 1) bytes).
int moe_decode(const rvm_layer *L, const float *x, float *out, int flags, const XForm &xf, void *ws,
               size_t ws_bytes, bool stream) {
    RVM_CHECK(layer_ok(L) && x && out && ws);
    const WsLayout lay = ws_layout(L, 1);
    RVM_CHECK(ws_bytes >= lay.total);
    uint8_t *w = (uint8_t *)ws;
    int32_t *ids = (int32_t *)(w + lay.ids);
    float *wts = (float *)(w + lay.wts);
    int rc = launch_router(L, x, 1, flags, xf, w, lay, ids, wts, nullptr, false);
    if (rc || (rc = span_router_done())) return rc;

    const int Tg = 2 * L->ff / 64;
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint4 *gnib = (const uint4 *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)((const uint8_t *)L->gate_up + gu_entries * 16);
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint4 *dnib = (const uint4 *)L->down;
    const uint16_t *dscl = (const uint16_t *)((const uint8_t *)L->down + dn_entries * 16);
    const int exact = (flags & RVM_EXACT_SELECT) ? 1 : 0;
    rc = with_steps(L->d / 256, [&](auto per) {
        constexpr int PER = decltype(per)::value;
        auto *kern = stream ? k_gateup_decode<PER, true> : k_gateup_decode<PER, false>;
        hipLaunchKernelGGL(kern, dim3(1 + L->top_k * Tg), dim3(GU_WAVES * 64), 0, cur_stream(), gnib, gscl, dnib, dscl,
                           (const double2 *)(w + lay.stats), L->router_bias, L->router, x, L->n_exp, L->top_k, xf,
                           exact, (uint32_t *)(w + lay.ctl), ids, wts, (const uint4 *)(w + lay.xact),
                           (uint32_t *)(w + lay.hact), (float *)(w + lay.dterm), Tg);
        return launched();
    });
    if (rc) return rc;
    return with_steps(L->ff / 64, [&](auto s) {
        hipLaunchKernelGGL(k_down_fold<decltype(s)::value>, dim3(L->d / 32), dim3(256), 0, cur_stream(),
                           (const float *)(w + lay.dterm), ids, wts, (const int32_t *)(w + lay.ctl) + 16,
                           L->down_scale, out, L->d, L->top_k);
        return launched();
    });
}

}  // namespace rvm

namespace {

// ---- The workspace-free decode (rvm_moe_decode_static) ----
// Its scratch is this array: one copy per GPU, loaded with the library's code object and held until
// the process ends. Host code uses the array's per-device address (hipGetSymbolAddress, taken once
// per device with that device current), never the array's name, which on the host is only a stand-in.
// No word of it must start at zero: every word a decode call reads was written earlier in that call
// (the fallback counter at offset 0 counts across calls and no kernel reads it).
static __device__ __align__(256) uint8_t scratch[RVM_STATIC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch[MAX_DEVICES];

}  // namespace

namespace rvm {

int phase_trace_decode(void *host) {
#ifdef RVM_PHASE_TRACE
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_stamp), sizeof(g_stamp));
#else
    (void)host;
    return (int)hipErrorNotSupported;
#endif
}

// Takes the scratch array's address on `device`, which must be current; idempotent.
int static_scratch_setup(int device) {
    if (device < 0 || device >= MAX_DEVICES) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[device]) return 0;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    g_scratch[device] = p;
    return 0;
}

}  // namespace rvm

extern "C" int rvm_moe_decode(const rvm_layer *L, const float *x, float *out, int flags, float eps, void *ws,
                              size_t ws_bytes) {
    return moe_decode(L, x, out, flags, xform_of_flags(flags, eps), ws, ws_bytes);
}

extern "C" int rvm_moe_decode_static(const rvm_layer *L, const float *x, float *out, int flags, float eps) {
    RVM_CHECK(layer_ok(L) && x && out);
    const size_t need = ws_layout(L, 1).total;
    if (need > RVM_STATIC_SCRATCH_BYTES) return (int)hipErrorInvalidValue;
    int dev = 0;
    RVM_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return (int)hipErrorInvalidDevice;
    void *ws = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ws = g_scratch[dev];
    }
    if (!ws) {
        if (int rc = static_scratch_setup(dev)) return rc;
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ws = g_scratch[dev];
    }
    return moe_decode(L, x, out, flags, xform_of_flags(flags, eps), ws, need);
}
