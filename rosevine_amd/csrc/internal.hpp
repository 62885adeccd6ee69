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
#include "tanhf.hpp"

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
constexpr int MAX_TOP_K = 8;       // experts per token
constexpr int MTILE = 16;          // pairs per MFMA m-tile
constexpr int MIN_TILE_PAIRS = 4;  // the smallest batched tile (quad tiles of small batches)

// Library state (runtime.hip).
hipStream_t cur_stream();
// The status of the launch just issued; every launch site calls it once, which also counts the
// launch in this thread's device-call counters (rvm_counters_get).
int launched();
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

// tanh GELU in the reference's operation order (runtime/src/ops.rs:145-149).
__device__ __forceinline__ float gelu(float x) {
    const float A = 0.044715f;
    const float S = 0.7978846f;
    float inner = S * x * (1.0f + A * x * x);
    return 0.5f * x * (1.0f + tanhf_select(inner));
}

// Expert weight loads, with the nontemporal hint when NT (weights read once in a stack of layers:
// they then do not push the router rows and the activations out of the caches).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ uint4 ld_weights(const uint4 *p) {
    if constexpr (NT) {
        const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *p;
    }
}
template <bool NT>
__device__ __forceinline__ uint32_t ld_weights(const uint16_t *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

// s_waitcnt with vmcnt = n and no wait on the other counters (gfx9 encoding)
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Copies to LDS (global_load_lds): lane l's 16 (4) bytes at src go to LDS address lds + 16 l (4 l),
// lds the same in every lane. Issued through asm, so the compiler adds no wait for them before LDS
// reads: the kernel waits for them itself (vmcnt).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" : : "v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p);
}

// A raw buffer descriptor over [p, p + bytes): loads through it take an SGPR base, a 32-bit VGPR
// offset and a wave-uniform offset, and read 0 at or past the end (no fault).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
typedef uint32_t u32v4 __attribute__((__vector_size__(16)));
// The whole vector is copied: a bit cast of one element of a vector type reads element 0's storage
// with this compiler.
__device__ __forceinline__ float4 buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const u32v4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    float4 f;
    __builtin_memcpy(&f, &v, 16);
    return f;
}
__device__ __forceinline__ uint4 buffer_load_u4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const u32v4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    uint4 u;
    __builtin_memcpy(&u, &v, 16);
    return u;
}
__device__ __forceinline__ uint32_t buffer_load_u32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint32_t buffer_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
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

// Cross-lane helpers; every lane of the wave must be active. DPP quad_perm [1,0,3,2] and
// [2,3,0,1] exchange lanes j ^ 1 and j ^ 2; row_half_mirror and row_mirror pair the quads and
// octets of a row of 16 lanes; ds_swizzle in bit-mask mode with xor 16 exchanges lanes j ^ 16
// within each half-wave.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t swz_xor16(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401f);
}
__device__ __forceinline__ float maxf_bits(float a, uint32_t b) { return fmaxf(a, __builtin_bit_cast(float, b)); }

// a & m, opaque to the optimiser: byte conversions of the result then map to v_cvt_f32_ubyte0..3,
// one instruction each, where knowing the bytes are nibbles makes the compiler extract each one
// first.
__device__ __forceinline__ uint32_t and_opaque(uint32_t a, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(m));
    return r;
}

// Sum over the wave in a fixed order: rows of 16 by DPP, then the four rows.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += __builtin_bit_cast(float, dpp<0xb1>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp<0x4e>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp<0x141>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp<0x140>(__builtin_bit_cast(uint32_t, v)));
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

// Orders LDS traffic between lanes of one wave (a wave's LDS operations complete in issue order).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Byte position of element j of a 32-element Q8_0 block in the batched path's activation rows.
// MFMA K group g (bytes 8g .. 8g+7) holds elements 4g .. 4g+3 and 16+4g .. 16+4g+3: the elements
// whose weights sit in the low and high nibbles of byte dword g of a packed Q4_0 entry, so that
// one dword of the entry is one lane's B operand. The block's int32 sum does not depend on the
// order of its 32 products.
__host__ __device__ constexpr int kperm(int j) { return 8 * ((j & 15) >> 2) + 4 * (j >> 4) + (j & 3); }

// Max over each 32-lane half-wave of non-NaN values, returned to every lane of the half.
__device__ __forceinline__ float half_max(float m) {
    m = maxf_bits(m, dpp<0xb1>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x4e>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x141>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x140>(__builtin_bit_cast(uint32_t, m)));
    return maxf_bits(m, swz_xor16(__builtin_bit_cast(uint32_t, m)));
}

// Q8_0 quantisation of one 32-value block held by a 32-lane half-wave (lane j of the half
// holds element j), as runtime/src/ops.rs:95-105: amax fold from 0 ignoring NaN, d = amax/127,
// id = 1/d (0 when d == 0), q = round-half-away(v * id) saturated. Returns q for this lane and
// the f16 bits of d in *dbits (same in every lane of the half). The block maximum does not
// depend on the order of the maxima (no value is NaN after fmaxf(0, |v|)).
__device__ __forceinline__ int quant_q8_half(float v, uint16_t *dbits) {
    const float m = half_max(fmaxf(0.0f, fabsf(v)));
    float d = m / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    *dbits = f2h_rne(d);
    return sat_i8(roundf(v * id));
}

// Build the prepared block from the 32 quants of a half-wave (lane j of the half holds q_j) and
// store it at dst (ACT_DW dwords) when ok. Element 4d+k (k < 4) sits in byte k, low nibble, of
// dword d; element 16+4d+k in byte k, high nibble. Every lane of the wave must call this.
__device__ __forceinline__ void store_prep_half(int q, uint16_t dbits, int j, uint32_t *dst, bool ok) {
    const uint32_t qp = swz_xor16((uint32_t)q);  // element j ^ 16 of the half
    const int k = j & 3;
    // lanes j < 16: byte k of dword j >> 2 from elements j (low nibble) and j + 16 (high nibble)
    uint32_t ch = ((((uint32_t)q >> 4) & 15u) | (((qp >> 4) & 15u) << 4)) << (8 * k);
    uint32_t cl = ((((uint32_t)q & 15u) ^ 8u) | (((qp & 15u) ^ 8u) << 4)) << (8 * k);
    ch |= dpp<0xb1>(ch);
    cl |= dpp<0xb1>(cl);
    ch |= dpp<0x4e>(ch);
    cl |= dpp<0x4e>(cl);
    if (!ok) return;
    if (j < 16 && k == 0) dst[j >> 2] = ch;
    if (j < 16 && k == 1) dst[4 + (j >> 2)] = cl;
    if (j == 16) dst[8] = __builtin_bit_cast(uint32_t, h2f(dbits));
    if (j >= 17 && j < 20) dst[j - 8] = 0u;
}

// Workspace layout for n_tok tokens through one layer (offsets in bytes, 256-aligned).
struct WsLayout {
    size_t ctl;     // u32[64]: [0] router fallback count; [16..24) decode: h row of each slot
    size_t stats;   // double2[n_tok][n_exp]: exact-sum estimate and error bound per logit
    size_t ids;     // i32[n_tok][top_k]
    size_t wts;     // f32[n_tok][top_k]
    size_t xact;    // u32[d/32][ACT_DW]: the decode token's prepared activation blocks
    size_t hact;    // u32[2 top_k][ff/32][ACT_DW]: decode h blocks per slot, then correction rows
    size_t order;   // i32[pairs]
    size_t pos_of;  // i32[pairs]
    size_t gstart;  // i32[n_exp + 1]
    size_t y;       // f32[pairs][d] (batched path)
    size_t dterm;   // f32[2 top_k][ff/32][d] (decode: down terms per slot and h block)
    size_t xq8;     // i8[n_tok][d]: plain Q8_0 values of the layer input (batched path)
    size_t xsc;     // f32[n_tok][d/32]: their scales
    size_t hq8;     // i8[pairs][ff]: plain Q8_0 values of h, in plan order (batched path)
    size_t hsc;     // f32[pairs][ff/32]
    size_t tiles;   // i32[1 + 2 max_tiles]: the plan's tiles (4 or 32 pairs)
    size_t tiles2;  // the same for the down kernel of the 16-pair MFMA path (48-pair tiles)
    size_t total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Upper bound on the plan's tiles of up to cap pairs: a group of n pairs takes ceil(n / cap) <=
// (n + cap - 1) / cap tiles, and there are at most min(n_exp, pairs) groups.
inline size_t max_tiles(const rvm_layer *L, int n_tok, int cap) {
    const size_t pairs = (size_t)n_tok * L->top_k, groups = pairs < (size_t)L->n_exp ? pairs : (size_t)L->n_exp;
    return (pairs + (size_t)(cap - 1) * groups) / cap;
}

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
    w.xact = take((size_t)(L->d / QK) * ACT_DW * 4);
    w.hact = take((size_t)2 * L->top_k * (L->ff / QK) * ACT_DW * 4);  // slots + correction rows
    w.order = take(pairs * 4);
    w.pos_of = take(pairs * 4);
    w.gstart = take((size_t)(L->n_exp + 1) * 4);
    w.y = n_tok > 1 ? take(pairs * L->d * 4) : take(0);
    // kept for every n_tok so that a workspace sized for a batch also serves rvm_moe_decode
    w.dterm = take((size_t)2 * L->top_k * (L->ff / QK) * L->d * 4);
    w.xq8 = take((size_t)n_tok * L->d);
    w.xsc = take((size_t)n_tok * (L->d / QK) * 4);
    w.hq8 = take(pairs * L->ff);
    w.hsc = take(pairs * (L->ff / QK) * 4);
    w.tiles = take((1 + 2 * max_tiles(L, n_tok, MIN_TILE_PAIRS)) * 4);
    w.tiles2 = take((1 + 2 * max_tiles(L, n_tok, MIN_TILE_PAIRS)) * 4);
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
           L->top_k <= MAX_TOP_K && L->top_k <= L->n_exp && L->d > 0 && L->d % 256 == 0 && steps_ok(L->d / 256) &&
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
// The per-device address of rvm_moe_decode_static's scratch array, taken once per device with
// that device current (decode.hip; rvh_init calls it).
int static_scratch_setup(int device);

// How a layer input row x becomes the router's input and the experts' input. Without pre_norm
// both are x. With it, s = 1 / sqrt(mean(x^2) + eps) (runtime/src/ops.rs:131-139) and
//   router input  r[i] = ((x[i] * s) * rpost) * rg[i]   (runtime/src/exec.rs:493-503;
//                                                         runtime/src/hip_exec.rs:786 with rvh_rms_norm)
//   expert input  e[i] = (x[i] * s) * eg[i]              (exec.rs:465-468; hip_exec.rs:796)
// each product rounded, with rg / eg absent meaning no factor (RVM_PRE_NORM alone: both x * s).
struct XForm {
    int pre_norm;
    float eps;
    float rpost;
    const float *rg;  // [d] or null
    const float *eg;  // [d] or null
};
inline XForm xform_of_flags(int flags, float eps) {
    return XForm{(flags & RVM_PRE_NORM) ? 1 : 0, eps, 1.0f, nullptr, nullptr};
}
// The router and expert inputs differ (a gain or a post factor is set).
__host__ __device__ inline bool xform_split(const XForm &xf) { return xf.rg || xf.eg || xf.rpost != 1.0f; }

// Span instrumentation of the session executor: when set, the layer call issued next records e on
// the current stream once its router work is issued (span_router_done), before its expert work.
void span_mark_after_router(hipEvent_t e);
int span_router_done();
// Records e on the current stream (an event node of the graph under capture); 0 or the error,
// which is also cleared from the thread's last error.
int record_event(hipEvent_t e);

// Kernel launchers shared across translation units.
// k_router (logit statistics and the Q8_0 input), then k_select unless select is false.
int launch_router(const rvm_layer *L, const float *x, int n_tok, int flags, const XForm &xf, uint8_t *ws,
                  const WsLayout &lay, int32_t *ids, float *wts, float *logits, bool select);
// One decode token (decode.hip) and n_tok tokens (grouped.hip) through the layer with input
// transform xf; flags carries RVM_EXACT_SELECT. stream: the decode kernel loads the expert weights
// with the nontemporal hint (a stack of layers, whose weights are read once per token and exceed
// the last-level cache); a single layer called token after token keeps plain loads, so that the
// experts it uses again can come from that cache.
int moe_decode(const rvm_layer *L, const float *x, float *out, int flags, const XForm &xf, void *ws,
               size_t ws_bytes, bool stream = false);
int moe_forward(const rvm_layer *L, const float *x, float *out, int n_tok, int flags, const XForm &xf, void *ws,
                size_t ws_bytes, bool stream = false);
// k_plan; with tiles set it also cuts every group into tiles of up to cap pairs: tiles[0] = count,
// then (expert, first position in order) per tile, the tiles with more m-tiles of 16 pairs first
// and in expert order within each such class; tiles2 likewise with cap2.
int launch_plan(const int32_t *ids, int n_pairs, int n_exp, int32_t *order, int32_t *pos_of, int32_t *gstart,
                int32_t *tiles, int cap, int32_t *tiles2 = nullptr, int cap2 = 0);

// Phase stamps of the decode kernels, in diagnostic builds only (-DRVM_PHASE_TRACE; other builds
// compile RVM_STAMP to nothing): thread 0 of each workgroup stores the 100 MHz realtime counter at
// point s of kernel k into its translation unit's array [k][workgroup][point] with a vector store,
// so that one decode call's phases can be read back across workgroups and XCDs.
constexpr int TRACE_WG = 4096, TRACE_PT = 8;
#ifdef RVM_PHASE_TRACE
#define RVM_STAMP(arr, k, s)                                                                              \
    do {                                                                                                  \
        if (threadIdx.x == 0 && blockIdx.x < (unsigned)rvm::TRACE_WG)                                     \
            (arr)[((k) * rvm::TRACE_WG + blockIdx.x) * rvm::TRACE_PT + (s)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
// the same after every memory operation issued so far has completed (a wait that only the
// diagnostic build has)
#define RVM_STAMP_LOADED(arr, k, s)       \
    do {                                  \
        __builtin_amdgcn_s_waitcnt(0);    \
        RVM_STAMP(arr, k, s);             \
    } while (0)
#else
#define RVM_STAMP(arr, k, s) ((void)0)
#define RVM_STAMP_LOADED(arr, k, s) ((void)0)
#endif
// Copy the stamps of k_router ([1][TRACE_WG][TRACE_PT]) and of k_gateup_decode, k_down_fold
// ([2][TRACE_WG][TRACE_PT]) to host memory; hipErrorNotSupported in other builds.
int phase_trace_router(void *host);
int phase_trace_decode(void *host);

}  // namespace rvm
