// grouped.hip - n_tok tokens through one MoE layer with device-side grouping (ragged decode
// batches and prefill; runtime/src/exec.rs:456-475 and 540-640, the reference's host dispatch is
// runtime/src/hip_exec.rs:822-843).
//
//   router (router.hip)   -> ids, weights, plain Q8_0 activation rows per token
//   k_plan (router.hip)   -> pairs stably grouped by expert, and the groups cut into 16-pair tiles
//   k_gateup_mfma         -> per (tile, 4 row tiles of 32 gate + 32 up rows): int8 MFMA
//                            (v_mfma_i32_16x16x32_i8, one 32-weight block per instruction) gives
//                            each block's exact int32 sum for 16 pairs x 16 rows; the f32 terms
//                            (sumi as f32) * (d_w * d_x) are folded in block order per output, as
//                            dot_q8_scalar does; GeGLU and the Q8_0 of h per pair finish the tile
//   k_down_mfma           -> per (tile, 4 row tiles of 32 down rows): the same on h, into y rows
//   k_combine_pairs       -> out[t] = sum_j (y[pos_of[t*k+j]] * scale) * weight, slot order
// Each output is the reference's sequential fold of exact block sums, so a token's result does not
// depend on the batch it arrives in and equals the decode path's.
#include "internal.hpp"

namespace rvm {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int MW = 4;  // waves (row tiles) per workgroup

// 8 int8 weights of one K group of a 32-weight block, from 8 of its 16 packed nibble bytes (each
// nibble the 4-bit two's complement weight): per byte, ((p ^ 8) + 0x78) ^ 0x80 = sign-extended p,
// with no carry between bytes. Groups 0 and 1 are the low nibbles of bytes 0-7 and 8-15 (elements
// 0-15), groups 2 and 3 their high nibbles (elements 16-31).
__device__ __forceinline__ uint32_t nib8(uint32_t p) {
    const uint32_t t = (p & 0x0F0F0F0Fu) ^ 0x08080808u;
    return (t + 0x78787878u) ^ 0x80808080u;
}
__device__ __forceinline__ long weights8(uint2 p, int shift) {
    return (long)(((uint64_t)nib8(p.y >> shift) << 32) | nib8(p.x >> shift));
}

// Max over each row of 16 lanes (the lanes of one MFMA K group) of non-NaN values.
__device__ __forceinline__ float row16_max(float m) {
    m = maxf_bits(m, dpp<0xb1>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x4e>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x141>(__builtin_bit_cast(uint32_t, m)));
    return maxf_bits(m, dpp<0x140>(__builtin_bit_cast(uint32_t, m)));
}

// Stages the tile's MTILE activation rows (Q8_0 values, row pitch `pitch` bytes, zeros for the
// tile's empty places) and their block scales transposed to [block][MTILE].
__device__ __forceinline__ void stage_rows(const int8_t *__restrict__ src, const float *__restrict__ ssrc, int width,
                                           const int *row_of, int cnt, int8_t *dst, int pitch, float *sdst) {
    const int n16 = width / 16, nb = width / QK;
    for (int i = threadIdx.x; i < MTILE * n16; i += blockDim.x) {
        const int r = i / n16, c = i - r * n16;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (r < cnt) v = ((const uint4 *)(src + (size_t)row_of[r] * width))[c];
        *(uint4 *)(dst + r * pitch + c * 16) = v;
    }
    for (int i = threadIdx.x; i < MTILE * nb; i += blockDim.x) {
        const int b = i / MTILE, r = i - b * MTILE;
        sdst[i] = r < cnt ? ssrc[(size_t)row_of[r] * nb + b] : 0.0f;
    }
}

// The f32 fold of one block into acc: acc[i] = acc[i] + (sumi as f32) * (d_w * d_x[i]).
__device__ __forceinline__ void fold_block(float (&acc)[4], v4i sumi, float dw, float4 dx) {
    acc[0] = acc[0] + (float)sumi[0] * (dw * dx.x);
    acc[1] = acc[1] + (float)sumi[1] * (dw * dx.y);
    acc[2] = acc[2] + (float)sumi[2] * (dw * dx.z);
    acc[3] = acc[3] + (float)sumi[3] * (dw * dx.w);
}

// Gate/up for one 16-pair tile: wave w takes row tile rt = 4 blockIdx.y + w (32 gate rows and the
// matching 32 up rows, one RVM_PACK_GATE_UP tile). Lane l = 16 g + m holds gate/up rows m and
// 16 + m for pairs 4g .. 4g + 3 (the MFMA output layout), so each lane folds 16 outputs.
__global__ __launch_bounds__(MW * 64) void k_gateup_mfma(const uint8_t *__restrict__ nib,
                                                         const uint16_t *__restrict__ scl,
                                                         const int32_t *__restrict__ tiles,
                                                         const int32_t *__restrict__ gstart,
                                                         const int32_t *__restrict__ order,
                                                         const int8_t *__restrict__ xq8,
                                                         const float *__restrict__ xsc, int8_t *__restrict__ hq8,
                                                         float *__restrict__ hsc, int d, int ff, int top_k) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int row_of[MTILE];
    const int tile = blockIdx.x;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(MTILE, gstart[e + 1] - k0);
    const int pitch = d + 32, nb = d / QK, Tg = ff / 32;
    int8_t *Xs = (int8_t *)smem;
    float *dxs = (float *)(smem + MTILE * pitch);
    if (threadIdx.x < MTILE) row_of[threadIdx.x] = threadIdx.x < (unsigned)cnt ? order[k0 + threadIdx.x] / top_k : 0;
    __syncthreads();
    stage_rows(xq8, xsc, d, row_of, cnt, Xs, pitch, dxs);
    __syncthreads();
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rt = blockIdx.y * MW + w;
    if (rt >= Tg) return;
    const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
    const int shift = (g >> 1) * 4;
    float acc[4][4] = {};  // gate rows m, 16 + m; up rows m, 16 + m
    const size_t tbase = ((size_t)e * Tg + rt) * nb * 64;
    for (int b = 0; b < nb; ++b) {
        const size_t eb = tbase + (size_t)b * 64;
        uint2 p[4];
        uint32_t sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const size_t ent = eb + 16 * r + m;  // plane lanes m, 16 + m (gate), 32 + m, 48 + m (up)
            p[r] = *(const uint2 *)(nib + ent * 16 + (g & 1) * 8);
            sc[r] = scl[ent];
        }
        const long a = *(const long *)(Xs + m * pitch + b * QK + g * 8);
        const float4 dx = *(const float4 *)(dxs + b * MTILE + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const v4i s = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, weights8(p[r], shift), v4i{0, 0, 0, 0}, 0, 0, 0);
            fold_block(acc[r], s, h2f((uint16_t)sc[r]), dx);
        }
    }
    // GeGLU, then Q8_0 of each pair's 32 h values (rows m and 16 + m over the 16 lanes of group g)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float h0 = gelu(acc[0][i]) * acc[2][i];
        const float h1 = gelu(acc[1][i]) * acc[3][i];
        const float amax = row16_max(fmaxf(fmaxf(0.0f, fabsf(h0)), fabsf(h1)));
        const float dq = amax / 127.0f;
        const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
        const uint16_t dbits = f2h_rne(dq);
        const int q0 = sat_i8(roundf(h0 * id)), q1 = sat_i8(roundf(h1 * id));
        const int pr = 4 * g + i;
        if (pr < cnt) {
            int8_t *hrow = hq8 + (size_t)(k0 + pr) * ff + rt * 32;
            hrow[m] = (int8_t)q0;
            hrow[16 + m] = (int8_t)q1;
            if (m == 0) hsc[(size_t)(k0 + pr) * Tg + rt] = h2f(dbits);
        }
    }
}

// Down for one 16-pair tile: wave w takes the 32-row down tile rt = 4 blockIdx.y + w
// (RVM_PACK_ROWS32: row r of the tile is plane lane r at block b < S, lane 32 + r at block S + b).
__global__ __launch_bounds__(MW * 64) void k_down_mfma(const uint8_t *__restrict__ nib,
                                                       const uint16_t *__restrict__ scl,
                                                       const int32_t *__restrict__ tiles,
                                                       const int32_t *__restrict__ gstart,
                                                       const int8_t *__restrict__ hq8, const float *__restrict__ hsc,
                                                       float *__restrict__ y, int d, int ff) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int row_of[MTILE];
    const int tile = blockIdx.x;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(MTILE, gstart[e + 1] - k0);
    const int pitch = ff + 32, nb = ff / QK, Sd = ff / 64, Td = d / 32;
    int8_t *Hs = (int8_t *)smem;
    float *dxs = (float *)(smem + MTILE * pitch);
    if (threadIdx.x < MTILE) row_of[threadIdx.x] = k0 + (threadIdx.x < (unsigned)cnt ? threadIdx.x : 0);
    __syncthreads();
    stage_rows(hq8, hsc, ff, row_of, cnt, Hs, pitch, dxs);
    __syncthreads();
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rt = blockIdx.y * MW + w;
    if (rt >= Td) return;
    const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
    const int shift = (g >> 1) * 4;
    float acc[2][4] = {};  // rows m, 16 + m
    const size_t tbase = ((size_t)e * Td + rt) * Sd * 64;
    for (int b = 0; b < nb; ++b) {
        const int half = b >= Sd ? 1 : 0, s = b - half * Sd;
        const size_t eb = tbase + (size_t)s * 64 + 32 * half;
        uint2 p[2];
        uint32_t sc[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const size_t ent = eb + 16 * r + m;
            p[r] = *(const uint2 *)(nib + ent * 16 + (g & 1) * 8);
            sc[r] = scl[ent];
        }
        const long a = *(const long *)(Hs + m * pitch + b * QK + g * 8);
        const float4 dx = *(const float4 *)(dxs + b * MTILE + 4 * g);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const v4i s4 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, weights8(p[r], shift), v4i{0, 0, 0, 0}, 0, 0, 0);
            fold_block(acc[r], s4, h2f((uint16_t)sc[r]), dx);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int pr = 4 * g + i;
        if (pr < cnt) {
            float *yrow = y + (size_t)(k0 + pr) * d + rt * 32;
            yrow[m] = acc[0][i];
            yrow[16 + m] = acc[1][i];
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
    int32_t *tiles = (int32_t *)(w + lay.tiles);
    float *y = (float *)(w + lay.y);
    int rc = launch_router(L, x, n_tok, flags, eps, w, lay, ids, wts, nullptr, true);
    if (rc) return rc;
    const int pairs = n_tok * L->top_k;
    if ((rc = launch_plan(ids, pairs, L->n_exp, order, pos_of, gstart, tiles))) return rc;
    const int nt = (int)max_tiles(L, n_tok);

    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint8_t *gnib = (const uint8_t *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)(gnib + gu_entries * 16);
    const int Tg = L->ff / 32;
    size_t smem = (size_t)MTILE * (L->d + 32) + (size_t)MTILE * (L->d / QK) * 4;
    RVM_CHECK(smem <= (size_t)max_lds_per_block());
    if (smem > 64 * 1024)
        RVM_TRY(hipFuncSetAttribute((const void *)k_gateup_mfma, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    hipLaunchKernelGGL(k_gateup_mfma, dim3(nt, grid_blocks(Tg, MW)), dim3(MW * 64), smem, cur_stream(), gnib, gscl,
                       tiles, gstart, order, (const int8_t *)(w + lay.xq8), (const float *)(w + lay.xsc),
                       (int8_t *)(w + lay.hq8), (float *)(w + lay.hsc), L->d, L->ff, L->top_k);
    if ((rc = launched())) return rc;

    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint8_t *dnib = (const uint8_t *)L->down;
    const uint16_t *dscl = (const uint16_t *)(dnib + dn_entries * 16);
    smem = (size_t)MTILE * (L->ff + 32) + (size_t)MTILE * (L->ff / QK) * 4;
    RVM_CHECK(smem <= (size_t)max_lds_per_block());
    hipLaunchKernelGGL(k_down_mfma, dim3(nt, grid_blocks(L->d / 32, MW)), dim3(MW * 64), smem, cur_stream(), dnib,
                       dscl, tiles, gstart, (const int8_t *)(w + lay.hq8), (const float *)(w + lay.hsc), y, L->d,
                       L->ff);
    if ((rc = launched())) return rc;

    hipLaunchKernelGGL(k_combine_pairs, dim3(n_tok), dim3(256), 0, cur_stream(), y, pos_of, ids, wts, L->down_scale,
                       out, L->top_k, L->d);
    return launched();
}
