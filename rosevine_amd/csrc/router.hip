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
// k_select (one workgroup per token) runs the certified selection of select.hpp
// (runtime/src/exec.rs:507-517); k_plan groups (token, slot) pairs by expert (exec.rs:529-558).
#include <math.h>

#include <utility>

#include "select.hpp"

namespace rvm {

#ifdef RVM_PHASE_TRACE
namespace {
// k_router: 0 entry, 1 done, 2 row and x loaded (statistics workgroups)
__device__ unsigned long long g_stamp[TRACE_WG * TRACE_PT];
}  // namespace
#endif

constexpr int RWAVES = 1;  // waves (experts) per router workgroup: one expert per CU spreads the row loads
constexpr int SEL_WAVES = 8;  // waves of the selecting workgroup

// The logit statistics of one router row and one token: S = the f64 sum of the f32 products
// (lane chunks summed in order, then a DPP wave scan), and the bound on the sequential f32 fold's
// error, g sum_i |s_i| / (1 - d g) with g = u / (1 - u), from a bound on the sum of the exact
// prefix sums' magnitudes. A lane with the C elements a .. a + C - 1 bounds its share from f32
// prefixes: q_0 = fl(r), r the f64 sum of the lanes below, and q_k = fl(q_(k-1) + p_(a+k-1)).
// Each rounding moves a prefix by at most g |q_k| (u |r| for q_0), so |s_(a+k-1)| <= |q_k| + u |r|
// + g (|q_1| + ... + |q_k|), and the lane's share is at most Q (1 + C g)^2 + C u |r|, with Q the
// f32 sum of the |q_k| in order (at most (1 + C g) times smaller than their exact sum); C g is
// about 2^-18 at most (C <= 64), so Q (1 + 2^-16) covers the factor. The f32 chains cost half
// what f64 ones do.
// Every lane returns the same pair.
template <int F4>
__device__ __forceinline__ double2 row_stats(const float4 (&wv)[F4], const float4 (&xv)[F4], int lane) {
    constexpr int d = 256 * F4, C = 4 * F4;
    static_assert(C <= 64, "the lane share's factor (1 + C g)^2 is covered by 1 + 2^-16");
    float pf[C];  // the f32 products
#pragma unroll
    for (int i = 0; i < F4; ++i) {
        pf[4 * i] = wv[i].x * xv[i].x;
        pf[4 * i + 1] = wv[i].y * xv[i].y;
        pf[4 * i + 2] = wv[i].z * xv[i].z;
        pf[4 * i + 3] = wv[i].w * xv[i].w;
    }
    // the lane's f64 sum as a pairwise tree (six dependent additions instead of C - 1 before the
    // scan that the f32 prefixes below wait for)
    double cd[C];
#pragma unroll
    for (int i = 0; i < C; ++i) cd[i] = (double)pf[i];
#pragma unroll
    for (int st = 1; st < C; st *= 2)
#pragma unroll
        for (int i = 0; i + st < C; i += 2 * st) cd[i] += cd[i + st];
    const double c = cd[0];
    const double incl = wave_scan_d(c);
    const double run = dpp_zero_d<0x138>(incl);  // wave_shr:1: the sum of the lanes below
    const double total = readlane_d(incl, 63);
    float q = (float)run, qs = 0.0f;
#pragma unroll
    for (int i = 0; i < C; ++i) {
        q = q + pf[i];
        qs = qs + fabsf(q);
    }
    double babs = (double)qs * (1.0 + 0x1p-16) + (double)C * 0x1p-24 * fabs(run);
    babs = wave_sum_d(babs);
    const double u = 0x1p-24, g = u / (1.0 - u);
    return make_double2(total, babs * g / (1.0 - (double)d * g) * (1.0 + 0x1p-20) + 1e-300);
}

// Q8_0 quantisation of the experts' input (x, or (x * s) * eg[i] with the rms_norm scale s already
// known), one 32-block per half-wave (runtime/src/ops.rs:95-105): blocks base0 + lane / 32,
// base0 + step + lane / 32, ... to the prepared decode blocks (xact) and, when xq8 is set, the plain
// values in MFMA K order and their scales.
template <int F4>
__device__ __forceinline__ void quant_x_blocks(const float *__restrict__ xt, const XForm &xf, float scale, int base0,
                                               int step, float first, uint32_t *__restrict__ xact,
                                               int8_t *__restrict__ xq8, float *__restrict__ xsc, int lane) {
    constexpr int nb = 256 * F4 / QK;
    const int j = lane & 31;
    for (int base = base0; base < nb; base += step) {
        const int hb = base + (lane >> 5);
        const bool ok = hb < nb;
        float v = base == base0 ? first : (ok ? xt[hb * QK + j] : 0.0f);
        if (xf.pre_norm) v = v * scale;
        if (xf.eg) v = v * xf.eg[(ok ? hb : 0) * QK + j];
        uint16_t dbits;
        const int q = quant_q8_half(v, &dbits);
        if (xact) store_prep_half(q, dbits, j, xact + (size_t)(ok ? hb : 0) * ACT_DW, ok);
        if (xq8 && ok) {
            xq8[hb * QK + kperm(j)] = (int8_t)q;
            if (j == 0) xsc[hb] = h2f(dbits);
        }
    }
}

// Decode router: one token. Workgroups 0 .. n_exp/RWAVES - 1 hold one expert per wave and form
// its statistics; the next nb/2 workgroups quantise the token, two Q8_0 blocks each (one per
// half-wave), so that every statistics workgroup does the same work. F4 = d / 256: lane l owns
// elements [4 F4 l, 4 F4 (l + 1)) of a router row.
template <int F4>
__global__ __launch_bounds__(RWAVES * 64) void k_router(const float *__restrict__ W, const float *__restrict__ x, int n_exp,
                                                XForm xf, double2 *__restrict__ stats, uint32_t *__restrict__ xact) {
    constexpr int d = 256 * F4, nb = d / QK;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int groups = (n_exp + RWAVES - 1) / RWAVES;
    RVM_STAMP(g_stamp, 0, 0);
    if ((int)blockIdx.x >= groups) {
        const int base0 = ((int)blockIdx.x - groups) * RWAVES * 2 + w * 2;
        const int hb0 = base0 + (lane >> 5);
        const float first = hb0 < nb ? x[hb0 * QK + (lane & 31)] : 0.0f;
        const float scale = xf.pre_norm ? rms_scale<F4>(x, lane, xf.eps) : 1.0f;
        quant_x_blocks<F4>(x, xf, scale, base0, nb, first, xact, nullptr, nullptr, lane);
        RVM_STAMP(g_stamp, 0, 1);
        return;
    }
    const int e = blockIdx.x * RWAVES + w;
    const bool have = e < n_exp;
    float4 wv[F4];
    const float4 *w4 = (const float4 *)(W + (size_t)(have ? e : 0) * d) + lane * F4;
#pragma unroll
    for (int i = 0; i < F4; ++i) wv[i] = w4[i];
    float4 xv[F4];
    load_x_chunk<F4>(x, lane, xf, xv);
    RVM_STAMP_LOADED(g_stamp, 0, 2);
    if (have) {
        const double2 st = row_stats<F4>(wv, xv, lane);
        if (lane == 0) stats[e] = st;
    }
    RVM_STAMP(g_stamp, 0, 1);
}

// Batched statistics: workgroup (g, r) keeps the rows of experts BW g .. BW g + BW-1 in registers
// (one per wave) and takes tokens r RT .. r RT + RT-1, the next token's x loads in flight while
// the current one is processed; the numbers are row_stats', as in k_router. The Q8_0 blocks of
// each token are shared out over the expert groups.
constexpr int BW = 4;
template <int F4>
__global__ __launch_bounds__(BW * 64) void k_router_batch(const float *__restrict__ W, const float *__restrict__ x,
                                                          int n_tok, int n_exp, int RT, XForm xf,
                                                          double2 *__restrict__ stats, int8_t *__restrict__ xq8,
                                                          float *__restrict__ xsc) {
    constexpr int d = 256 * F4, nb = d / QK;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * BW + w;
    const bool have = e < n_exp;
    float4 wv[F4];
    const float4 *w4 = (const float4 *)(W + (size_t)(have ? e : 0) * d) + lane * F4;
#pragma unroll
    for (int i = 0; i < F4; ++i) wv[i] = w4[i];
    const int t0 = blockIdx.y * RT, t1 = min(t0 + RT, n_tok);
    const int base0 = (blockIdx.x * BW + w) * 2, step = gridDim.x * BW * 2;
    // this lane's element of the first Q8_0 block it quantises (block hb0), loaded a token ahead
    // with the token's chunk
    const int hb0 = base0 + (lane >> 5), qoff = min(hb0, nb - 1) * QK + (lane & 31);
    float4 xr[F4];
    float qr;
    {
        const float4 *x4 = (const float4 *)(x + (size_t)t0 * d) + lane * F4;
#pragma unroll
        for (int i = 0; i < F4; ++i) xr[i] = x4[i];
        qr = x[(size_t)t0 * d + qoff];
    }
    for (int t = t0; t < t1; ++t) {
        const float *xt = x + (size_t)t * d;
        float4 xv[F4];
#pragma unroll
        for (int i = 0; i < F4; ++i) xv[i] = xr[i];
        const float qv = qr;
        {  // the next token's chunk (the last one again at the end; unused)
            const size_t tn = (size_t)min(t + 1, t1 - 1) * d;
            const float4 *x4 = (const float4 *)(x + tn) + lane * F4;
#pragma unroll
            for (int i = 0; i < F4; ++i) xr[i] = x4[i];
            qr = x[tn + qoff];
        }
        float scale = 1.0f;
        if (xf.pre_norm) {
            scale = norm_x_chunk<F4>(xt, xv, xf.eps);
            router_gain<F4>(xf, lane, xv);
        }
        quant_x_blocks<F4>(xt, xf, scale, base0, step, hb0 < nb ? qv : 0.0f, nullptr, xq8 + (size_t)t * d,
                           xsc + (size_t)t * nb, lane);
        if (have) {
            const double2 st = row_stats<F4>(wv, xv, lane);
            if (lane == 0) stats[(size_t)t * n_exp + e] = st;
        }
    }
}

// One workgroup per token: the selection of select.hpp, published to ids / wts / logits.
template <int F4>
__global__ __launch_bounds__(SEL_WAVES * 64) void k_select(const double2 *__restrict__ stats,
                                                           const float *__restrict__ bias,
                                                           const float *__restrict__ W, const float *__restrict__ x,
                                                           int n_exp, int top_k, XForm xf, int exact,
                                                           uint32_t *__restrict__ ctl, int32_t *__restrict__ ids,
                                                           float *__restrict__ wts, float *__restrict__ logits) {
    __shared__ SelShared<F4, SEL_WAVES> sh;
    const int tok = blockIdx.x;
    select_token<F4, SEL_WAVES>(sh, stats + (size_t)tok * n_exp, bias, W, x + (size_t)tok * 256 * F4, n_exp, top_k,
                                xf, exact, true, true, ctl,
                                logits ? logits + (size_t)tok * n_exp : nullptr);
    if (sh.pass) select_weights<F4, SEL_WAVES>(sh, n_exp, top_k);
    __syncthreads();
    select_publish<F4, SEL_WAVES>(sh, top_k, ids + (size_t)tok * top_k, wts + (size_t)tok * top_k);
}

// ---- Large batches: the reference's logits, folded exactly ----
// From FOLD_MIN_TOKENS tokens a batch holds enough (token, expert) pairs to fill the GPU with one
// sequential fold per lane, which is cheaper than the f64 statistics and the certificate: lane l
// of a wave is token t0 + l, the wave's expert is uniform, and each lane adds the f32 products
// W_r[e][i] * r[i] of the router input r in element order from -0.0 (runtime/src/ops.rs:321-326),
// then the bias, so the logits are the reference's bit for bit. 512 tokens x 128 experts are 1024
// waves, one per SIMD: each fold is a chain of d dependent adds (about 4 ns each on one wave), and
// the kernel is bound by that chain and by the LDS reads of the tokens. The tile's 64 tokens are
// staged in LDS FKC columns at a time (double-buffered, the loads of two chunks ahead in flight).
// Column quad q of token t sits at [q][t ^ (q & 7)], so the coalesced stores (eight quads of one
// token) and the per-token reads (one quad of 64 tokens) are free of bank conflicts. The workgroup's
// FW router rows are staged in LDS once; each product is a v_mul_f32_dpp whose row_newbcast operand
// hands one row element to its 16-lane row (fold_quad2). Without the norm, the workgroups also write
// the tokens' Q8_0 blocks of the experts' input (runtime/src/ops.rs:95-105), which k_router_prep
// writes otherwise.
constexpr int FOLD_MIN_TOKENS = RVM_FOLD_MIN_TOKENS;
constexpr int FW = 4;     // waves (experts) per workgroup
constexpr int FKC = 128;  // columns per staged chunk

// The inputs of the fold, one workgroup per token: the rms_norm scale s (runtime/src/ops.rs:131-139),
// the router input ((x * s) * rpost) * rg[i] written to rin when the layer input is normed (the fold
// reads x itself otherwise), and the Q8_0 blocks of the experts' input (x * s) * eg[i]
// (runtime/src/ops.rs:95-105), one block per half-wave. Wave w holds blocks 2w + 8i (+1 in the upper
// half-wave) of the row, all loaded first; the f64 sum of squares is the four waves' partial sums
// (each a fixed tree) added in a fixed order. The reference sums sequentially; both sums lie within
// (d - 1) 2^-53 of the exact one relative to it, so the f32 mean is the reference's unless the sum
// sits that close to an f32 rounding boundary, when it is redone in the reference's order.
template <int F4>
__global__ __launch_bounds__(256) void k_router_prep(const float *__restrict__ x, int n_tok, XForm xf,
                                                     float *__restrict__ rin, int8_t *__restrict__ xq8,
                                                     float *__restrict__ xsc) {
    constexpr int d = 256 * F4, nb = d / QK, NI = nb / 8;
    static_assert(nb % 8 == 0, "eight blocks per round of four waves");
    __shared__ double part[4];
    const int t = blockIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, j = lane & 31;
    const float *xt = x + (size_t)t * d;
    float v[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) v[i] = xt[(2 * w + 8 * i + (lane >> 5)) * QK + j];
    float s = 1.0f;
    if (xf.pre_norm) {
        double p = 0.0;
#pragma unroll
        for (int i = 0; i < NI; ++i) p += (double)v[i] * (double)v[i];
        p = wave_sum_d(p);
        if (lane == 0) part[w] = p;
        __syncthreads();
        double ss = (part[0] + part[1]) + (part[2] + part[3]);
        const double bnd = ss * (2.0 * d * 0x1p-53) * 1.01;
        if ((float)((ss - bnd) / d) != (float)((ss + bnd) / d)) {
            ss = 0.0;
            for (int i = 0; i < d; ++i) {
                const double u = (double)xt[i];
                ss += u * u;
            }
        }
        const float mean = (float)(ss / (double)d);
        s = 1.0f / sqrtf(mean + xf.eps);
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int hb = 2 * w + 8 * i + (lane >> 5), col = hb * QK + j;
        float e = v[i];
        if (xf.pre_norm) {
            float r = v[i] * s;
            e = r;
            if (xf.rpost != 1.0f) r = r * xf.rpost;
            if (xf.rg) r = r * xf.rg[col];
            rin[(size_t)t * d + col] = r;
            if (xf.eg) e = e * xf.eg[col];
        }
        uint16_t dbits;
        const int q = quant_q8_half(e, &dbits);
        xq8[(size_t)t * d + hb * QK + kperm(j)] = (int8_t)q;
        if (j == 0) xsc[(size_t)t * nb + hb] = h2f(dbits);
    }
}

// Quads MA and MB of a 64-column row block: columns 4M .. 4M+3 sit in lane M of each row of 16
// lanes (w.x .. w.w). Each is handed to every lane by a DPP row broadcast inside the multiply
// (v_mul_f32_dpp row_newbcast: the plain f32 product, rounded) and added to this lane's fold in
// column order. The products are formed ahead of the adds that take them (quad MA's four first,
// quad MB's between quad MA's adds), so each add waits only for the add before it: the fold is the
// chain of dependent adds, and a product made just before its add put a multiply's latency on that
// chain for every column. Written out because the compiler keeps the broadcast as a separate move
// (its unused old operand comes from another block) and puts a wait state in front of every
// statement that holds a DPP instruction. The hardware needs two wait states between a VALU write
// of a DPP source and its read: every w here comes from an LDS read.
template <int MA, int MB>
__device__ __forceinline__ void fold_quad2(float &acc, const float4 &w, const float4 &a, const float4 &b) {
    float t0, t1, t2, t3, t4, t5, t6, t7;
    asm("v_mul_f32_dpp %1, %9, %13 row_newbcast:%21 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_mul_f32_dpp %2, %10, %14 row_newbcast:%21 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_mul_f32_dpp %3, %11, %15 row_newbcast:%21 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_mul_f32_dpp %4, %12, %16 row_newbcast:%21 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32 %0, %0, %1\n\t"
        "v_mul_f32_dpp %5, %9, %17 row_newbcast:%22 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32 %0, %0, %2\n\t"
        "v_mul_f32_dpp %6, %10, %18 row_newbcast:%22 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32 %0, %0, %3\n\t"
        "v_mul_f32_dpp %7, %11, %19 row_newbcast:%22 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32 %0, %0, %4\n\t"
        "v_mul_f32_dpp %8, %12, %20 row_newbcast:%22 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32 %0, %0, %5\n\t"
        "v_add_f32 %0, %0, %6\n\t"
        "v_add_f32 %0, %0, %7\n\t"
        "v_add_f32 %0, %0, %8"
        : "+v"(acc), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7)
        : "v"(w.x), "v"(w.y), "v"(w.z), "v"(w.w), "v"(a.x), "v"(a.y), "v"(a.z), "v"(a.w), "v"(b.x), "v"(b.y),
          "v"(b.z), "v"(b.w), "i"(MA), "i"(MB));
}
template <int BASE, int... Q>
__device__ __forceinline__ void fold_quads(float &acc, const float4 &w, const float4 *xv,
                                           std::integer_sequence<int, Q...>) {
    // left to right: the quad pairs in column order
    (fold_quad2<BASE + 2 * Q, BASE + 2 * Q + 1>(acc, w, xv[2 * Q], xv[2 * Q + 1]), ...);
}

// The Q8_0 blocks of 32 router-input values of one token, all in this thread (v[4 i + k] = quad i's
// element k), stored as k_router_prep stores them: the same numbers as quant_q8_half's, whose block
// maximum (of non-negative values, NaN ignored) is the same in any order; quant j at byte kperm(j),
// so quad i (elements 4i .. 4i+3) is dword 2 (i mod 4) + i / 4.
__device__ __forceinline__ void quant_q8_block(const float4 (&v)[8], int8_t *__restrict__ dst, float *__restrict__ dsc) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        m = fmaxf(m, fmaxf(fmaxf(fmaxf(0.0f, fabsf(v[i].x)), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    const float dq = m / 127.0f;
    const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
    uint32_t dw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t b0 = (uint8_t)sat_i8(roundf(v[i].x * id)), b1 = (uint8_t)sat_i8(roundf(v[i].y * id));
        const uint32_t b2 = (uint8_t)sat_i8(roundf(v[i].z * id)), b3 = (uint8_t)sat_i8(roundf(v[i].w * id));
        dw[2 * (i & 3) + (i >> 2)] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
    ((uint4 *)dst)[0] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    ((uint4 *)dst)[1] = make_uint4(dw[4], dw[5], dw[6], dw[7]);
    *dsc = h2f(f2h_rne(dq));
}

// With xq8 set (batches whose router input is x itself), the workgroups also write the tokens'
// Q8_0 blocks for the expert kernels, which k_router_prep writes otherwise: expert group g of a
// token tile quantises the chunks c = g, g + groups, ... of the tile's staged input, one block of
// one token per thread.
template <int F4>
__global__ __launch_bounds__(FW * 64) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_router_fold(
    const float *__restrict__ W, const float *__restrict__ xin, const float *__restrict__ bias, int n_tok, int n_exp,
    float *__restrict__ R, int8_t *__restrict__ xq8, float *__restrict__ xsc) {
    constexpr int d = 256 * F4, NCH = d / FKC, KQ = FKC / 4, LD = 64 * KQ / (FW * 64), SQ = 8, RS = KQ / SQ;
    constexpr int WQ = d / 4, WL = (FW * WQ + FW * 64 - 1) / (FW * 64);  // row quads, and per thread
    static_assert(FKC == 128 && NCH % 2 == 0 && RS == 4, "two 64-column row blocks and four sub-steps per chunk");
    __shared__ float4 xs[2][KQ][64];  // the tile's router input, column quad q of token t at [q][t ^ (q & 7)]
    __shared__ float4 wl[FW][WQ];     // the workgroup's router rows
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    // Workgroup g takes token tile g % tiles and expert group g / tiles: consecutive workgroups go to
    // different XCDs (g % 8), so the expert groups of one tile share an XCD whenever the tile count
    // divides 8 or is a multiple of it, and the tile's tokens are read into that XCD's L2 once.
    const int tiles = (n_tok + 63) / 64;
    const int t0 = (int)(blockIdx.x % tiles) * 64;
    const int e0 = (int)(blockIdx.x / tiles) * FW;
    const int ew = e0 + w;
    // the rows of experts e0 .. e0 + FW - 1 (clamped), all loads issued first
    float4 wv[WL];
#pragma unroll
    for (int i = 0; i < WL; ++i) {
        const int k = min(tid + i * FW * 64, FW * WQ - 1), r = k / WQ;
        wv[i] = ((const float4 *)(W + (size_t)min(e0 + r, n_exp - 1) * d))[k - r * WQ];
    }
    // staging: thread tid moves quad (tid % KQ) of tokens tid / KQ + j (256 / KQ), j < LD. Two
    // register sets alternate: chunk c stages chunk c + 1 from its set and refills the set with
    // chunk c + 3, so every load has two chunks' fold time to arrive.
    const int sq = tid % KQ, st = tid / KQ;
    const __amdgpu_buffer_rsrc_t xres = buffer_rsrc(xin, (uint32_t)((size_t)n_tok * d * 4));
    uint32_t xoff[LD];
#pragma unroll
    for (int j = 0; j < LD; ++j) xoff[j] = (uint32_t)((min(t0 + st + j * (256 / KQ), n_tok - 1) * d + 4 * sq) * 4);
    float4 p0[LD], pa[LD], pb[LD];
#pragma unroll
    for (int j = 0; j < LD; ++j) p0[j] = buffer_load4(xres, xoff[j], 0);
#pragma unroll
    for (int j = 0; j < LD; ++j) pa[j] = buffer_load4(xres, xoff[j], 1 * FKC * 4);
#pragma unroll
    for (int j = 0; j < LD; ++j) pb[j] = buffer_load4(xres, xoff[j], min(2, NCH - 1) * FKC * 4);
#pragma unroll
    for (int i = 0; i < WL; ++i) {
        const int k = tid + i * FW * 64;
        if (k < FW * WQ) wl[k / WQ][k % WQ] = wv[i];
    }
    auto stage = [&](int buf, const float4 (&p)[LD]) {
#pragma unroll
        for (int j = 0; j < LD; ++j) {
            const int tt = st + j * (256 / KQ);
            xs[buf][sq][tt ^ (sq & 7)] = p[j];
        }
    };
    stage(0, p0);
    __syncthreads();
    // The wave's row, 64 columns per LDS read: lane l reads columns 4 (l & 15) .. + 3 of the block,
    // so every row of 16 lanes holds the block once and DPP row broadcasts hand each column to all
    // lanes.
    const float4 *wrow = wl[w] + (lane & 15);
    float acc = -0.0f;
    // chunk c: set p holds chunk c + 1, staged into the other buffer halfway through the fold (that
    // buffer was last read in chunk c - 1), then p loads chunk c + 3. Sub-step r folds quads
    // 8r .. 8r+7 while the tokens' quads of sub-step r + 1 come from LDS; the scheduling barriers
    // keep each sub-step's reads in their place.
    const int groups = (n_exp + FW - 1) / FW, g = (int)(blockIdx.x / tiles);
    auto chunk = [&](int c, float4 (&p)[LD]) {
        const int buf = c & 1;
        if (xq8 && c % groups == g) {  // block tid / 64 of chunk c for token tid % 64
            const int tt = tid & 63, kb = tid >> 6;
            static_assert(FW * 64 == 64 * (FKC / QK), "one block of one token per thread");
            if (t0 + tt < n_tok) {
                float4 v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = xs[buf][8 * kb + i][tt ^ i];
                const int hb = c * (FKC / QK) + kb;
                quant_q8_block(v, xq8 + (size_t)(t0 + tt) * d + hb * QK, xsc + (size_t)(t0 + tt) * (d / QK) + hb);
            }
        }
        float4 wb[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) wb[k] = wrow[(2 * c + k) * 16];
        float4 xv[2][SQ];
#pragma unroll
        for (int q = 0; q < SQ; ++q) xv[0][q] = xs[buf][q][lane ^ (q & 7)];
        auto sub = [&](auto rc) {
            constexpr int r = decltype(rc)::value;
            if (r + 1 < RS)
#pragma unroll
                for (int q = 0; q < SQ; ++q) {
                    const int qq = (r + 1) * SQ + q;
                    xv[(r + 1) & 1][q] = xs[buf][qq][lane ^ (qq & 7)];
                }
            fold_quads<(r & 1) * SQ>(acc, wb[r >> 1], xv[r & 1], std::make_integer_sequence<int, SQ / 2>{});
            __builtin_amdgcn_sched_barrier(0);
        };
        sub(std::integral_constant<int, 0>{});
        sub(std::integral_constant<int, 1>{});
        if (c + 1 < NCH) stage(buf ^ 1, p);
        // unconditional loads (past the end the last chunk loads again, unused): exact wait counts
        const int c3 = min(c + 3, NCH - 1);
#pragma unroll
        for (int j = 0; j < LD; ++j) p[j] = buffer_load4(xres, xoff[j], c3 * FKC * 4);
        sub(std::integral_constant<int, 2>{});
        sub(std::integral_constant<int, 3>{});
        __syncthreads();
    };
    for (int c = 0; c < NCH; c += 2) {
        chunk(c, pa);
        chunk(c + 1, pb);
    }
    const int t = t0 + lane;
    if (ew < n_exp && t < n_tok) R[(size_t)t * n_exp + ew] = bias ? acc + bias[ew] : acc;
}

// The reference's softmax and top-k from the exact logits, one wave per token.
__global__ __launch_bounds__(256) void k_select_exact(const float *__restrict__ R, int n_tok, int n_exp, int top_k,
                                                      int32_t *__restrict__ ids, float *__restrict__ wts,
                                                      float *__restrict__ logits) {
    __shared__ float sp[4][256];
    __shared__ int sel[4][8];
    __shared__ float wsel[4][8];
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + w;
    if (t >= n_tok) return;  // the whole wave
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = lane + 64 * i < n_exp ? R[(size_t)t * n_exp + lane + 64 * i] : -INFINITY;
    exact_softmax_top_k(r, n_exp, top_k, sp[w], sel[w], wsel[w], logits ? logits + (size_t)t * n_exp : nullptr,
                        lane);
    wave_lds_sync();
    if (lane < top_k) {
        ids[(size_t)t * top_k + lane] = sel[w][lane];
        wts[(size_t)t * top_k + lane] = wsel[w][lane];
    }
}

// Stable counting sort of pair ids by expert in one workgroup of 16 waves: wave w owns a
// contiguous chunk of pairs; per-(wave, expert) counts are scanned in (expert, wave) order, then
// each wave places its pairs 64 at a time, ranking equal experts among lower lanes with ballots.
// Ids outside [0, n_exp) are neither counted nor placed (pos_of = -1). With tiles (and tiles2)
// set, every group is also cut into tiles of up to cap (cap2) pairs. A wave reads its ids PLAN_R
// rows of 64 at a time, the loads of a batch issued together; a chunk of at most PLAN_R rows (up to
// 8192 pairs) stays in registers from the count to the placement.
constexpr int PLAN_R = 8;
__device__ __forceinline__ void plan_load(const int32_t *__restrict__ ids, int base, int hi, int lane,
                                          int (&ev)[PLAN_R]) {
#pragma unroll
    for (int r = 0; r < PLAN_R; ++r) {
        const int i = base + 64 * r + lane;
        ev[r] = i < hi ? ids[i] : -1;
    }
}
// Inclusive prefix sum of an int over the 64 lanes (all active), by DPP only: row_shr 1, 2, 4, 8
// within each row of 16 (lanes whose source lies outside the row add 0), then row_bcast:15 (row
// r's last lane into row r + 1, for rows 1 and 3) and row_bcast:31 (lane 31 into rows 2 and 3).
__device__ __forceinline__ int wave_scan_i(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, true);
    return v;
}

// Tile classes: a tile of n pairs has class min(PLAN_NC, ceil(n / 16)) - 1 (its m-tiles of 16 pairs).
// The tiles are listed class by class, the most m-tiles first, and by expert within a class: the
// batched kernels' workgroups start in grid order, so the longest tiles start first and the
// remainder tiles, which run fewer m-tiles, fill the end of the grid.
constexpr int PLAN_NC = 3;
__device__ __forceinline__ int tile_class(int n) { return min(PLAN_NC, (n + 15) / 16) - 1; }
// n / cap for 0 <= n < 2^20 and 1 <= cap <= 128 (inv = 1 / cap as f32): the f32 estimate is within
// one of the quotient and is corrected once each way (checked for every such n and cap).
__device__ __forceinline__ int div_small(int n, int cap, float inv) {
    int q = (int)((float)n * inv);
    q += (q + 1) * cap <= n ? 1 : 0;
    q -= q * cap > n ? 1 : 0;
    return q;
}
// A group of n pairs in tiles of up to cap: full tiles of cap pairs (class kf, wave-uniform), then
// the remainder's tile (class kr, -1 when there is none).
struct GroupTiles {
    int full, kr;
};
__device__ __forceinline__ GroupTiles group_tiles(int n, int cap, float inv) {
    const int full = div_small(n, cap, inv), rem = n - full * cap;
    return GroupTiles{full, rem ? tile_class(rem) : -1};
}
// Adds a group's tiles to the per-class counts.
__device__ __forceinline__ void tile_counts(const GroupTiles &t, int kf, int (&cnt)[PLAN_NC]) {
#pragma unroll
    for (int k = 0; k < PLAN_NC; ++k) cnt[k] += (k == kf ? t.full : 0) + (k == t.kr ? 1 : 0);
}
// The places of a group's tiles in the list: its full tiles from *f on, its remainder's at *r (-1
// when there is none); pos holds the next place of each class.
__device__ __forceinline__ void place_tiles(const GroupTiles &t, int kf, int (&pos)[PLAN_NC], int *f, int *r) {
    int fp = 0, rp = -1;
#pragma unroll
    for (int k = 0; k < PLAN_NC; ++k) {
        if (k == kf) {
            fp = pos[k];
            pos[k] += t.full;
        }
        if (k == t.kr) rp = pos[k]++;
    }
    *f = fp;
    *r = rp;
}
// Writes expert e's tiles (expert, first position in order) for its n pairs at run, at the places
// place_tiles gave.
__device__ __forceinline__ void put_tiles(int32_t *__restrict__ tl, int cap, float inv, int e, int n, int run,
                                          int f, int r) {
    const int full = div_small(n, cap, inv);
    for (int q = 0; q < full; ++q) {
        tl[1 + 2 * (f + q)] = e;
        tl[2 + 2 * (f + q)] = run + q * cap;
    }
    if (r >= 0) {
        tl[1 + 2 * r] = e;
        tl[2 + 2 * r] = run + full * cap;
    }
}

__global__ __launch_bounds__(1024) void k_plan(const int32_t *__restrict__ ids, int n, int n_exp,
                                               int32_t *__restrict__ order, int32_t *__restrict__ pos_of,
                                               int32_t *__restrict__ gstart, int32_t *__restrict__ tiles, int cap,
                                               int32_t *__restrict__ tiles2, int cap2) {
    __shared__ int cnt[16][256];
    __shared__ int tot[257];
    __shared__ int tplace[2][2][256];  // per tile list and expert: first full tile's place, remainder's
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int chunk = ((n + 15) / 16 + 63) / 64 * 64;
    const int lo = w * chunk, hi = min(n, lo + chunk);
    const bool one_batch = chunk <= 64 * PLAN_R;
    int ev[PLAN_R];
    if (one_batch) plan_load(ids, lo, hi, lane, ev);  // in flight while the counts are cleared
    for (int i = threadIdx.x; i < 16 * 256; i += 1024) (&cnt[0][0])[i] = 0;
    __syncthreads();
    for (int base = lo; base < hi; base += 64 * PLAN_R) {
        if (!one_batch) plan_load(ids, base, hi, lane, ev);
#pragma unroll
        for (int r = 0; r < PLAN_R; ++r)
            if (ev[r] >= 0 && ev[r] < n_exp) atomicAdd(&cnt[w][ev[r]], 1);
    }
    __syncthreads();
    if ((int)threadIdx.x < n_exp) {
        int s = 0;
        for (int ww = 0; ww < 16; ++ww) s += cnt[ww][threadIdx.x];
        tot[threadIdx.x] = s;
    }
    __syncthreads();
    if (w == 0) {  // exclusive scans of the group sizes and of their tile counts by class, 4 experts a lane
        const int cp2 = tiles2 ? cap2 : 1;
        const float inv1 = 1.0f / (float)cap, inv2 = 1.0f / (float)cp2;
        const int kf1 = tile_class(cap), kf2 = tile_class(cp2);
        int c[4], cs = 0, s1[PLAN_NC], s2[PLAN_NC];
        GroupTiles g1[4], g2[4];
#pragma unroll
        for (int k = 0; k < PLAN_NC; ++k) s1[k] = s2[k] = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = 4 * lane + k;
            c[k] = e < n_exp ? tot[e] : 0;
            cs += c[k];
            g1[k] = group_tiles(c[k], cap, inv1);
            g2[k] = group_tiles(c[k], cp2, inv2);
            tile_counts(g1[k], kf1, s1);
            tile_counts(g2[k], kf2, s2);
        }
        const int ic = wave_scan_i(cs);
        int i1[PLAN_NC], i2[PLAN_NC];
#pragma unroll
        for (int k = 0; k < PLAN_NC; ++k) {
            i1[k] = wave_scan_i(s1[k]);
            i2[k] = wave_scan_i(s2[k]);
        }
        // this lane's first tile of each class: the classes with more m-tiles come first
        int p1[PLAN_NC], p2[PLAN_NC], t1 = 0, t2 = 0;
#pragma unroll
        for (int k = PLAN_NC - 1; k >= 0; --k) {
            p1[k] = t1 + i1[k] - s1[k];
            p2[k] = t2 + i2[k] - s2[k];
            t1 += __builtin_amdgcn_readlane(i1[k], 63);
            t2 += __builtin_amdgcn_readlane(i2[k], 63);
        }
        int run = ic - cs;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = 4 * lane + k;
            if (e < n_exp) {
                tot[e] = run;
                place_tiles(g1[k], kf1, p1, &tplace[0][0][e], &tplace[0][1][e]);
                place_tiles(g2[k], kf2, p2, &tplace[1][0][e], &tplace[1][1][e]);
            }
            run += c[k];
        }
        if (lane == 63) {
            tot[n_exp] = ic;
            if (tiles) tiles[0] = t1;
            if (tiles2) tiles2[0] = t2;
        }
    }
    __syncthreads();
    if ((int)threadIdx.x <= n_exp) gstart[threadIdx.x] = tot[threadIdx.x];
    if ((int)threadIdx.x < n_exp) {  // one expert a thread: its tiles, then its waves' first positions
        const int e = threadIdx.x, ne = tot[e + 1] - tot[e];
        if (tiles) put_tiles(tiles, cap, 1.0f / (float)cap, e, ne, tot[e], tplace[0][0][e], tplace[0][1][e]);
        if (tiles2)
            put_tiles(tiles2, cap2, 1.0f / (float)cap2, e, ne, tot[e], tplace[1][0][e], tplace[1][1][e]);
        int run = tot[threadIdx.x];
        for (int ww = 0; ww < 16; ++ww) {
            const int c = cnt[ww][threadIdx.x];
            cnt[ww][threadIdx.x] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int base0 = lo; base0 < hi; base0 += 64 * PLAN_R) {
        if (!one_batch) plan_load(ids, base0, hi, lane, ev);
#pragma unroll
        for (int r = 0; r < PLAN_R; ++r) {
            const int base = base0 + 64 * r;
            if (base >= hi) break;  // wave-uniform
            const int i = base + lane, raw = ev[r];
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
}

int launch_router(const rvm_layer *L, const float *x, int n_tok, int flags, const XForm &xf, uint8_t *ws,
                  const WsLayout &lay, int32_t *ids, float *wts, float *logits, bool select) {
    const int pre = xf.pre_norm;
    RVM_CHECK(pre || !xform_split(xf));  // the router's and experts' factors apply to the normed input
    return with_steps(L->d / 256, [&](auto f4) {
        constexpr int F4 = decltype(f4)::value;
        if (n_tok == 1) {  // decode: one wave per expert, and the prepared activation blocks
            const int groups = grid_blocks(L->n_exp, RWAVES), qgroups = grid_blocks(L->d / QK, 2 * RWAVES);
            hipLaunchKernelGGL(k_router<F4>, dim3(groups + qgroups), dim3(RWAVES * 64), 0, cur_stream(), L->router, x,
                               L->n_exp, xf, (double2 *)(ws + lay.stats), (uint32_t *)(ws + lay.xact));
        } else if (select && n_tok >= FOLD_MIN_TOKENS) {  // large batches: exact logits, no certificate
            // R (the logits) in the statistics region; the normed router input in the region of the
            // down rows y (pairs x d floats, at least n_tok x d), which the expert kernels write later
            float *R = (float *)(ws + lay.stats), *rin = (float *)(ws + lay.y);
            // with the norm, k_router_prep forms the router and expert inputs and the Q8_0 blocks;
            // without it the router input is x, and the fold's workgroups write the Q8_0 blocks
            int8_t *xq8 = (int8_t *)(ws + lay.xq8);
            float *xsc = (float *)(ws + lay.xsc);
            if (pre) {
                hipLaunchKernelGGL(k_router_prep<F4>, dim3(n_tok), dim3(256), 0, cur_stream(), x, n_tok, xf, rin, xq8,
                                   xsc);
                if (int rc = launched()) return rc;
            }
            hipLaunchKernelGGL(k_router_fold<F4>, dim3(grid_blocks(L->n_exp, FW) * grid_blocks(n_tok, 64)),
                               dim3(FW * 64), 0, cur_stream(), L->router, pre ? rin : x, L->router_bias, n_tok,
                               L->n_exp, R, pre ? nullptr : xq8, pre ? nullptr : xsc);
            if (int rc = launched()) return rc;
            hipLaunchKernelGGL(k_select_exact, dim3(grid_blocks(n_tok, 4)), dim3(256), 0, cur_stream(), R, n_tok,
                               L->n_exp, L->top_k, ids, wts, logits);
            return launched();
        } else {  // batches: about 16 token groups, so that the rows are read that many times
            const int rt = max(1, n_tok / 16);
            hipLaunchKernelGGL(k_router_batch<F4>, dim3(grid_blocks(L->n_exp, BW), grid_blocks(n_tok, rt)),
                               dim3(BW * 64), 0, cur_stream(), L->router, x, n_tok, L->n_exp, rt, xf,
                               (double2 *)(ws + lay.stats), (int8_t *)(ws + lay.xq8), (float *)(ws + lay.xsc));
        }
        int rc = launched();
        if (rc || !select) return rc;
        hipLaunchKernelGGL(k_select<F4>, dim3(n_tok), dim3(SEL_WAVES * 64), 0, cur_stream(),
                           (const double2 *)(ws + lay.stats), L->router_bias, L->router, x, L->n_exp, L->top_k, xf,
                           (flags & RVM_EXACT_SELECT) ? 1 : 0, (uint32_t *)(ws + lay.ctl), ids, wts, logits);
        return launched();
    });
}

int launch_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of, int32_t *gstart,
                int32_t *tiles, int cap, int32_t *tiles2, int cap2) {
    RVM_CHECK(cap >= 1 && (!tiles2 || cap2 >= 1));
    // the tile counts' division (div_small) holds for groups below 2^20 pairs and tiles of <= 128
    RVM_CHECK(!tiles || (n_pairs < (1 << 20) && cap <= 128 && (!tiles2 || cap2 <= 128)));
    hipLaunchKernelGGL(k_plan, dim3(1), dim3(1024), 0, cur_stream(), ids, n_pairs, n_exp, order, pos_of, gstart,
                       tiles, cap, tiles2, cap2);
    return launched();
}

int phase_trace_router(void *host) {
#ifdef RVM_PHASE_TRACE
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_stamp), sizeof(g_stamp));
#else
    (void)host;
    return (int)hipErrorNotSupported;
#endif
}

}  // namespace rvm

using namespace rvm;

extern "C" {

int rvm_router_select(const rvm_layer *layer, const float *x, int n_tok, int flags, float eps, int32_t *ids,
                      float *weights, float *logits, void *ws, size_t ws_bytes) {
    RVM_CHECK(layer_ok(layer) && x && n_tok > 0 && n_tok <= MAX_TOKENS && ids && weights && ws);
    const WsLayout lay = ws_layout(layer, n_tok);
    RVM_CHECK(ws_bytes >= lay.total);
    return launch_router(layer, x, n_tok, flags, xform_of_flags(flags, eps), (uint8_t *)ws, lay, ids, weights, logits,
                         true);
}

int rvm_moe_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of, int32_t *group_start) {
    RVM_CHECK(ids && order && pos_of && group_start && n_pairs > 0 && n_exp > 0 && n_exp <= 256);
    return launch_plan(ids, n_pairs, n_exp, order, pos_of, group_start, nullptr, MTILE);
}

}  // extern "C"
