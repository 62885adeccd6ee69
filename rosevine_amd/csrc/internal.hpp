// internal.hpp - shared device helpers for the gfx950 MoE kernels.
//
// Arithmetic notes (reference paths relative to the reference root):
//  - Q4_0 x Q8_0 block dot (runtime/src/expert_kernel.rs:147-161): the packed nibble plane holds
//    qs XOR 0x88, so every nibble is the signed weight w = n - 8. An activation q (int8) is split
//    as q = 16*hi + lo' + 8 with hi = q >> 4 (the high nibble of the byte, signed) and
//    lo' = (q & 15) - 8 (the low nibble XOR 8, signed). Then
//        sum_j w_j q_j = 16 * sdot8(w, HI) + sdot8(w, LO) + 8 * sdot8(w, 0x11111111)
//    with three v_dot8_i32_i4 chains of four dwords: an exact int32 for every block.
//  - The f32 part is the reference's: term = (sumi as f32) * (d_w * d_x), folded sequentially in
//    block order from 0.0 with separate roundings, so every row equals dot_q8_scalar bit for bit;
//    the terms are computed in parallel and only the fold is sequential.
//  - Everything is compiled with -ffp-contract=off: no multiply-add is fused.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/rvmoe.h"

namespace rvm {

constexpr int QK = 32;
constexpr int Q4_BLOCK = 18;
constexpr int Q8_BLOCK = 34;
// A prepared activation block: HI[4], LO[4] nibble dwords in the weight-nibble order, then d_x
// (the f16-rounded scale as f32) and three spare dwords: 48 bytes, so that every block is three
// 16-byte-aligned vector loads from global memory or LDS.
constexpr int ACT_DW = 12;
constexpr uint32_t ONES4 = 0x11111111u;
constexpr int MAX_TOKENS = 65535;  // tokens per call (the router grid's y dimension)

// Library state (runtime.hip).
hipStream_t cur_stream();
inline int launched() { return (int)hipGetLastError(); }
inline int grid_blocks(size_t n, int per) { return (int)((n + per - 1) / per); }

#define RVM_CHECK(cond)                                  \
    do {                                                 \
        if (!(cond)) return (int)hipErrorInvalidValue;   \
    } while (0)
#define RVM_TRY(expr)                      \
    do {                                   \
        hipError_t e_ = (expr);            \
        if (e_ != hipSuccess) return (int)e_; \
    } while (0)

// IEEE binary16 bits -> f32, exact (same values as runtime/src/ops.rs:7-24).
__device__ __forceinline__ float h2f(uint16_t u) {
    _Float16 h;
    __builtin_memcpy(&h, &u, 2);
    return (float)h;
}

// f32 -> binary16 bits, round to nearest even, written out in integers so that the result is
// the reference's f32_to_f16 (runtime/src/ops.rs:27-59) bit for bit, NaN payload included.
__host__ __device__ __forceinline__ uint16_t f2h_rne(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man != 0 ? 0x200u : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t r = m >> shift;
        if (rem > half || (rem == half && (r & 1u))) r += 1;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1;
    return (uint16_t)(sign | r);
}

// Rust `f32 as i8`: saturate, NaN to 0.
__device__ __forceinline__ int sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int)v;
}

// expm1f and tanhf as the platform libm of the reference computes them: Rust's f32::tanh is the
// C library's tanhf, which on the reference's Linux hosts (glibc 2.35) is the fdlibm algorithm
// (Sun Microsystems; glibc sysdeps/ieee754/flt-32/s_tanhf.c and s_expm1f.c). The steps and
// constants below are that published algorithm, evaluated with the same single-precision
// operations, so the device result equals glibc's tanhf on every f32 input (compared over all
// 2^32 inputs on the host; the GPU tests compare the device against the host libm).
__host__ __device__ inline float fb_expm1f(float x) {
    const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = __builtin_bit_cast(uint32_t, x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (xsb == 0 && hx > 0x42b17217u) return huge * huge;
        }
        if (xsb != 0) return tiny - one;
    }
    if (hx > 0x3eb17218u) {  // |x| > ln2 / 2: argument reduction
        if (hx < 0x3F851592u) {
            if (xsb == 0) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {  // |x| < 2^-25
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : one + 2.0f * (x - e);
    if (k <= -2 || k > 56) {
        y = one - (e - x);
        y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
        return y - one;
    }
    if (k < 23) {
        t = __builtin_bit_cast(float, 0x3f800000u - (0x1000000u >> k));
        y = t - (e - x);
        y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
    } else {
        t = __builtin_bit_cast(float, (uint32_t)(0x7f - k) << 23);
        y = x - (e + t);
        y += one;
        y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
    }
    return y;
}

__host__ __device__ inline float fb_tanhf(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    const int32_t jx = __builtin_bit_cast(int32_t, x);
    const int32_t ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000) {  // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (one + x);  // |x| < 2^-55
        if (ix >= 0x3f800000) {
            t = fb_expm1f(two * fabsf(x));
            z = one - two / (t + two);
        } else {
            t = fb_expm1f(-two * fabsf(x));
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;
    }
    return jx >= 0 ? z : -z;
}

// tanh GELU in the reference's operation order (runtime/src/ops.rs:145-149).
__device__ __forceinline__ float gelu(float x) {
    const float A = 0.044715f;
    const float S = 0.7978846f;
    float inner = S * x * (1.0f + A * x * x);
    return 0.5f * x * (1.0f + fb_tanhf(inner));
}

// One block's term of the reference dot, (sumi as f32) * (d_w * d_x), each product rounded
// (runtime/src/expert_kernel.rs:158); the reference folds these terms in block order from 0.0.
__device__ __forceinline__ float block_term(int sumi, float dw, float dx) { return (float)sumi * (dw * dx); }

// Exact int32 sum of one 32-element block: w4 = this lane's 16 packed nibble bytes, a = HI[4], LO[4].
__device__ __forceinline__ int block_dot(uint4 w4, const uint32_t *a) {
    int hi = __builtin_amdgcn_sdot8((int)w4.x, (int)a[0], 0, false);
    hi = __builtin_amdgcn_sdot8((int)w4.y, (int)a[1], hi, false);
    hi = __builtin_amdgcn_sdot8((int)w4.z, (int)a[2], hi, false);
    hi = __builtin_amdgcn_sdot8((int)w4.w, (int)a[3], hi, false);
    int lo = __builtin_amdgcn_sdot8((int)w4.x, (int)a[4], 0, false);
    lo = __builtin_amdgcn_sdot8((int)w4.y, (int)a[5], lo, false);
    lo = __builtin_amdgcn_sdot8((int)w4.z, (int)a[6], lo, false);
    lo = __builtin_amdgcn_sdot8((int)w4.w, (int)a[7], lo, false);
    int s1 = __builtin_amdgcn_sdot8((int)w4.x, (int)ONES4, 0, false);
    s1 = __builtin_amdgcn_sdot8((int)w4.y, (int)ONES4, s1, false);
    s1 = __builtin_amdgcn_sdot8((int)w4.z, (int)ONES4, s1, false);
    s1 = __builtin_amdgcn_sdot8((int)w4.w, (int)ONES4, s1, false);
    return (hi << 4) + lo + (s1 << 3);
}

// Prepared activation dwords from a raw Q8_0 block's 32 quant bytes, given as 8 dwords q[0..7]
// (q[i] holds elements 4i..4i+3). Weight dword d pairs elements 4d..4d+3 (low nibbles) with
// 16+4d..16+4d+3 (high nibbles).
__device__ __forceinline__ void prep_from_q8(const uint32_t *q, uint32_t *a) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t lo = q[d], hi = q[4 + d];
        a[d] = ((lo >> 4) & 0x0f0f0f0fu) | (hi & 0xf0f0f0f0u);
        a[4 + d] = ((lo & 0x0f0f0f0fu) | ((hi & 0x0f0f0f0fu) << 4)) ^ 0x88888888u;
    }
}

// Q8_0 quantisation of one 32-value block held by a 32-lane half-wave (lane j of the half
// holds element j), as runtime/src/ops.rs:95-105: amax fold from 0 ignoring NaN, d = amax/127,
// id = 1/d (0 when d == 0), q = round-half-away(v * id) saturated. Returns q for this lane and
// the f16 bits of d in *dbits (same in every lane of the half).
__device__ __forceinline__ int quant_q8_half(float v, uint16_t *dbits) {
    float m = fmaxf(0.0f, fabsf(v));
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float d = m / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    *dbits = f2h_rne(d);
    return sat_i8(roundf(v * id));
}

// Build the prepared block from the 32 quants of a half-wave (lane j of the half holds q_j) and
// store it at dst (ACT_DW dwords) when ok. Element 4d+k (k < 4) sits in byte k, low nibble, of
// dword d; element 16+4d+k in byte k, high nibble. Every lane of the wave must call this.
__device__ __forceinline__ void store_prep_half(int q, uint16_t dbits, int j, uint32_t *dst, bool ok) {
    const int k = j & 3;
    const int sh = 8 * k + (j >= 16 ? 4 : 0);
    uint32_t ch = (uint32_t)((q >> 4) & 15) << sh;
    uint32_t cl = (uint32_t)((q & 15) ^ 8) << sh;
    ch |= __shfl_xor(ch, 1);
    cl |= __shfl_xor(cl, 1);
    ch |= __shfl_xor(ch, 2);
    cl |= __shfl_xor(cl, 2);
    ch |= __shfl_xor(ch, 16);
    cl |= __shfl_xor(cl, 16);
    if (!ok) return;
    if (j < 16 && k == 0) dst[j >> 2] = ch;
    if (j < 16 && k == 1) dst[4 + (j >> 2)] = cl;
    if (j == 16) dst[8] = __builtin_bit_cast(uint32_t, h2f(dbits));
    if (j >= 17 && j < 20) dst[j - 8] = 0u;
}

// Workspace layout for n_tok tokens through one layer (offsets in bytes, 256-aligned).
struct WsLayout {
    size_t ctl;     // u32[64]: [0] router-guard fallback count
    size_t stats;   // double2[n_tok][n_exp]: exact-sum estimate and error bound per logit
    size_t ids;     // i32[n_tok][top_k]
    size_t wts;     // f32[n_tok][top_k]
    size_t xact;    // u32[n_tok][d/32][ACT_DW]
    size_t hact;    // u32[pairs][ff/32][ACT_DW]
    size_t order;   // i32[pairs]
    size_t pos_of;  // i32[pairs]
    size_t gstart;  // i32[n_exp + 1]
    size_t y;       // f32[pairs][d]
    size_t total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline WsLayout ws_layout(const rvm_layer *L, int n_tok) {
    WsLayout w{};
    size_t o = 0;
    size_t pairs = (size_t)n_tok * L->top_k;
    auto take = [&](size_t bytes) {
        size_t at = o;
        o = align256(o + bytes);
        return at;
    };
    w.ctl = take(256);
    w.stats = take((size_t)n_tok * L->n_exp * 16);
    w.ids = take(pairs * 4);
    w.wts = take(pairs * 4);
    w.xact = take((size_t)n_tok * (L->d / QK) * ACT_DW * 4);
    w.hact = take(pairs * (L->ff / QK) * ACT_DW * 4);
    w.order = take(pairs * 4);
    w.pos_of = take(pairs * 4);
    w.gstart = take((size_t)(L->n_exp + 1) * 4);
    w.y = n_tok > 1 ? take(pairs * L->d * 4) : take(0);
    w.total = o;
    return w;
}

// The kernels are compiled for these per-lane step counts: d / 256 and ff / 64 must be one of
// them (d = 2816 and ff = 704 give 11).
__host__ __device__ constexpr bool steps_ok(int n) {
    return n == 1 || n == 2 || n == 4 || n == 8 || n == 11 || n == 16;
}

// Layer validation shared by the layer entry points.
inline bool layer_ok(const rvm_layer *L) {
    return L && L->router && L->gate_up && L->down && L->n_exp > 0 && L->n_exp <= 256 && L->top_k > 0 &&
           L->top_k <= 8 && L->top_k <= L->n_exp && L->d > 0 && L->d % 256 == 0 && steps_ok(L->d / 256) &&
           L->ff > 0 && L->ff % 64 == 0 && steps_ok(L->ff / 64);
}

// Calls f(std::integral_constant<int, n>) for a supported step count n (steps_ok).
template <class F>
inline int with_steps(int n, F &&f) {
    switch (n) {
        case 1: return f(std::integral_constant<int, 1>{});
        case 2: return f(std::integral_constant<int, 2>{});
        case 4: return f(std::integral_constant<int, 4>{});
        case 8: return f(std::integral_constant<int, 8>{});
        case 11: return f(std::integral_constant<int, 11>{});
        case 16: return f(std::integral_constant<int, 16>{});
        default: return (int)hipErrorInvalidValue;
    }
}

// Device limits read once per process (rvh_init).
int max_lds_per_block();

// Kernel launchers shared across translation units.
int launch_router(const rvm_layer *L, const float *x, int n_tok, int flags, float eps, uint8_t *ws,
                  const WsLayout &lay, int32_t *ids, float *wts, float *logits);
int launch_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of, int32_t *gstart);

}  // namespace rvm
