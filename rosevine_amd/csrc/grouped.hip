// grouped.hip - n_tok tokens through one MoE layer with device-side grouping (ragged decode
// batches and prefill; runtime/src/exec.rs:456-475 and 540-640, the reference's host dispatch is
// runtime/src/hip_exec.rs:822-843).
//
//   router (router.hip)   -> ids, weights, Q8_0 activation rows per token (K order of kperm)
//   k_plan (router.hip)   -> pairs stably grouped by expert, each group cut into tiles of up to
//                            16 MT pairs
//   k_gateup_mfma         -> per (tile, 4 row tiles of 32 gate + 32 up rows): int8 MFMA
//                            (v_mfma_i32_16x16x32_i8, one 32-weight block per instruction) gives
//                            each block's exact int32 sum for 16 pairs x 16 rows; the f32 terms
//                            (sumi as f32) * (d_w * d_x) are folded in block order per output, as
//                            dot_q8_scalar does; GeGLU and the Q8_0 of h per pair finish the tile
//   k_down_mfma           -> per (tile, 4 row tiles of 32 down rows): the same on h, into y rows
//   k_combine_pairs       -> out[t] = sum_j (y[pos_of[t*k+j]] * scale) * weight, slot order
// Each output is the reference's sequential fold of exact block sums, so a token's result does not
// depend on the batch it arrives in and equals the decode path's.
//
// The tile loop walks the K blocks in chunks of KC: the tile's activation rows for a chunk are
// staged in LDS (double-buffered, one barrier per chunk), and each wave keeps the next chunk's
// weight dwords and scales in flight while it computes the current one.
#include "internal.hpp"

namespace rvm {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int MW = 4;  // waves (row tiles) per workgroup
// K blocks per chunk (a template parameter of the tile loop; 8 measured slower for one m-tile)
template <int MT>
constexpr int chunk_blocks() { return 4; }

// 8 int8 weights from one dword of a packed Q4_0 entry (bytes 4g .. 4g+3, each nibble the 4-bit
// two's complement weight): the low nibbles (elements 4g .. 4g+3) then the high nibbles
// (16+4g .. 16+4g+3), the K group order of kperm. Per byte, ((p ^ 8) + 0x78) ^ 0x80 is p
// sign-extended, with no carry between bytes.
__device__ __forceinline__ uint32_t nib8(uint32_t p) {
    const uint32_t t = (p & 0x0F0F0F0Fu) ^ 0x08080808u;
    return (t + 0x78787878u) ^ 0x80808080u;
}
__device__ __forceinline__ long weights8(uint32_t p) {
    return (long)(((uint64_t)nib8(p >> 4) << 32) | nib8(p));
}

// Max over each row of 16 lanes (the lanes of one MFMA K group) of non-NaN values.
__device__ __forceinline__ float row16_max(float m) {
    m = maxf_bits(m, dpp<0xb1>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x4e>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x141>(__builtin_bit_cast(uint32_t, m)));
    return maxf_bits(m, dpp<0x140>(__builtin_bit_cast(uint32_t, m)));
}

// The f32 fold of one block into acc: acc[i] = acc[i] + (sumi as f32) * (d_w * d_x[i]).
__device__ __forceinline__ void fold_block(float (&acc)[4], v4i sumi, float dw, float4 dx) {
    acc[0] = acc[0] + (float)sumi[0] * (dw * dx.x);
    acc[1] = acc[1] + (float)sumi[1] * (dw * dx.y);
    acc[2] = acc[2] + (float)sumi[2] * (dw * dx.z);
    acc[3] = acc[3] + (float)sumi[3] * (dw * dx.w);
}

template <int MT, int NR, int KC>
struct TileLds {
    static constexpr int R = 16 * MT, XP = KC * QK + 16;  // row pitch: conflict-free 8-byte reads
    alignas(16) int8_t xs[2][R * XP];           // activation rows of the chunk
    alignas(16) float ss[2][KC * R];            // their block scales, [block][row]
    alignas(16) uint16_t ws[MW][KC * 16 * NR];  // per wave: weight scales, [block][m][piece]
    int row_of[R];                              // source row of each tile place, -1 when empty
};

// The block sums of one tile: rows of the wave's row tile (entry groups tb .. tb+S-1, NR pieces of
// 16 plane lanes; block b uses group b mod S at lane offset 32 (b / S)) against the tile's R
// activation rows (K = width, nb = width / 32 blocks). acc[mt][r][i] is the output of pair
// 16 mt + 4 g + i and plane lane 16 r + m, for lane = 16 g + m. All waves take part in the staging
// and barriers; waves without a row tile (active false) skip the weights and MFMAs.
template <int MT, int NR, int KC>
__device__ __forceinline__ void tile_sums(const uint8_t *__restrict__ nib, const uint16_t *__restrict__ scl,
                                          size_t tb, int S, bool active, const int8_t *__restrict__ src,
                                          const float *__restrict__ ssrc, int width, TileLds<MT, NR, KC> &sh,
                                          float (&acc)[MT][NR][4]) {
    // Every global load below is issued unconditionally (addresses clamped into the buffers, the
    // values selected when stored), so that the compiler can count the loads in flight and wait
    // for exactly the ones it needs: the next chunk's loads stay outstanding while this one runs.
    constexpr int R = 16 * MT, NT = MW * 64, XP = TileLds<MT, NR, KC>::XP;
    constexpr int XU = KC * QK / 16;  // 16-byte pieces of a staged row chunk
    constexpr int XI = (R * XU + NT - 1) / NT, SI = (R * KC + NT - 1) / NT;
    constexpr int SPL = KC * 16 * NR / 64;  // weight scales per lane per chunk (2, 4 or 8)
    const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
    const int w = threadIdx.x >> 6;
    const int nb = width / QK, nch = (nb + KC - 1) / KC;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][r][i] = 0.0f;

    auto entry = [&](int b) {  // first plane entry of block b (clamped to the last block)
        b = min(b, nb - 1);
        const int half = b >= S ? 1 : 0;
        return (tb + (size_t)(b - half * S)) * 64 + 32 * half;
    };
    // this lane's share of a chunk's weight scales: block kb = lane / (64 / KC), entries
    // j .. j+SPL-1 of it
    constexpr int LPB = 64 / KC;
    const int skb = lane / LPB, sj = (lane % LPB) * SPL;
    // this thread's staging items, fixed over the chunks: activation piece q of tile place xrow[k],
    // and the scale of place srow[k] at chunk block skbx[k]
    const int8_t *xsrc[XI];
    int xq[XI], xdst[XI];
    bool xok[XI];
#pragma unroll
    for (int k = 0; k < XI; ++k) {
        const int i = threadIdx.x + k * NT, ii = min(i, R * XU - 1);
        const int row = ii / XU, q = ii - row * XU, from = sh.row_of[row];
        xok[k] = i < R * XU && from >= 0;
        xsrc[k] = src + (size_t)(from >= 0 ? from : 0) * width;
        xq[k] = q * 16;
        xdst[k] = i < R * XU ? row * XP + q * 16 : -1;
    }
    const float *ssp[SI];
    int skbx[SI];
    bool sok[SI];
#pragma unroll
    for (int k = 0; k < SI; ++k) {
        const int i = threadIdx.x + k * NT, ii = min(i, R * KC - 1);
        const int kb = ii / R, row = ii - kb * R, from = sh.row_of[row];
        sok[k] = i < R * KC && from >= 0;
        ssp[k] = ssrc + (size_t)(from >= 0 ? from : 0) * nb;
        skbx[k] = i < R * KC ? kb : -1;
    }

    auto load_w = [&](int c, uint32_t (&wn)[KC][NR], uint32_t (&wsc)[SPL / 2]) {
#pragma unroll
        for (int kb = 0; kb < KC; ++kb) {
            const size_t e0 = entry(c * KC + kb);
#pragma unroll
            for (int r = 0; r < NR; ++r) wn[kb][r] = *(const uint32_t *)(nib + (e0 + 16 * r + m) * 16 + 4 * g);
        }
        const uint16_t *sp = scl + entry(c * KC + skb) + sj;
        if constexpr (SPL == 8) {
            const uint4 v = *(const uint4 *)sp;
            wsc[0] = v.x;
            wsc[1] = v.y;
            wsc[2] = v.z;
            wsc[3] = v.w;
        } else if constexpr (SPL == 4) {
            const uint2 v = *(const uint2 *)sp;
            wsc[0] = v.x;
            wsc[1] = v.y;
        } else {
            wsc[0] = *(const uint32_t *)sp;
        }
    };
    auto load_x = [&](int c, uint4 (&xr)[XI], float (&sr)[SI]) {
#pragma unroll
        for (int k = 0; k < XI; ++k) xr[k] = *(const uint4 *)(xsrc[k] + min(c * KC * QK + xq[k], width - 16));
#pragma unroll
        for (int k = 0; k < SI; ++k) sr[k] = ssp[k][min(c * KC + max(skbx[k], 0), nb - 1)];
    };
    auto store_x = [&](int c, int buf, const uint4 (&xr)[XI], const float (&sr)[SI]) {
#pragma unroll
        for (int k = 0; k < XI; ++k) {
            const bool ok = xok[k] && c * KC * QK + xq[k] < width;
            if (xdst[k] >= 0) *(uint4 *)(sh.xs[buf] + xdst[k]) = ok ? xr[k] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int k = 0; k < SI; ++k) {
            const bool ok = sok[k] && c * KC + skbx[k] < nb;
            if (skbx[k] >= 0) sh.ss[buf][threadIdx.x + k * NT] = ok ? sr[k] : 0.0f;
        }
    };
    auto compute = [&](int c, int buf, const uint32_t (&wn)[KC][NR], const uint32_t (&wsc)[SPL / 2]) {
        if (!active) return;
        // the chunk's weight scales to [block][m][piece] in this wave's LDS
        uint16_t *wsw = sh.ws[w];
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
            const int j = sj + k;
            const uint32_t v = wsc[k >> 1] >> ((k & 1) * 16);
            wsw[(skb * 16 + (j & 15)) * NR + (j >> 4)] = (uint16_t)v;
        }
        wave_lds_sync();
#pragma unroll
        for (int kb = 0; kb < KC; ++kb) {
            const int b = c * KC + kb;
            if (b >= nb) break;
            float dw[NR];
            if constexpr (NR == 4) {
                const uint2 v = *(const uint2 *)(wsw + (kb * 16 + m) * NR);
                dw[0] = h2f((uint16_t)v.x);
                dw[1] = h2f((uint16_t)(v.x >> 16));
                dw[2] = h2f((uint16_t)v.y);
                dw[3] = h2f((uint16_t)(v.y >> 16));
            } else {
                const uint32_t v = *(const uint32_t *)(wsw + (kb * 16 + m) * NR);
                dw[0] = h2f((uint16_t)v);
                dw[1] = h2f((uint16_t)(v >> 16));
            }
            long a[MT];
            float4 dx[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                a[mt] = *(const long *)(sh.xs[buf] + (mt * 16 + m) * XP + kb * QK + g * 8);
                dx[mt] = *(const float4 *)(sh.ss[buf] + kb * R + mt * 16 + 4 * g);
            }
            // every MFMA of the block first, then the folds: no fold waits on the MFMA just issued
            v4i sm[MT][NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const long bw = weights8(wn[kb][r]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    sm[mt][r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[mt], bw, v4i{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) fold_block(acc[mt][r], sm[mt][r], dw[r], dx[mt]);
        }
        wave_lds_sync();  // the next chunk's scale stores stay behind these reads
    };

    uint32_t wn0[KC][NR], wn1[KC][NR];
    uint32_t ws0[SPL / 2], ws1[SPL / 2];
    uint4 xr[XI];
    float sr[SI];
    load_x(0, xr, sr);
    load_w(0, wn0, ws0);
    store_x(0, 0, xr, sr);
    __syncthreads();
    for (int c = 0; c < nch; c += 2) {
        {
            const bool more = c + 1 < nch;
            // staging loads first: store_x waits for them, and the in-order load counter then
            // leaves the weight loads behind them in flight; past the end both reload the last
            // block, unused
            load_x(c + 1, xr, sr);
            load_w(c + 1, wn1, ws1);
            compute(c, 0, wn0, ws0);
            if (more) store_x(c + 1, 1, xr, sr);
            __syncthreads();
        }
        if (c + 1 < nch) {
            const bool more = c + 2 < nch;
            load_x(c + 2, xr, sr);
            load_w(c + 2, wn0, ws0);
            compute(c + 1, 1, wn1, ws1);
            if (more) store_x(c + 2, 0, xr, sr);
            __syncthreads();
        }
    }
}

// Gate/up for one tile of up to 16 MT pairs of expert e: wave w takes row tile rt = 4 blockIdx.y + w
// (32 gate rows and the matching 32 up rows, one RVM_PACK_GATE_UP tile; pieces 0, 1 are gate rows
// m and 16 + m, pieces 2, 3 the up rows). h = gelu(gate) * up is quantised per pair to one Q8_0
// block of 32 (runtime/src/ops.rs:95-105) and stored in the K order of kperm.
template <int MT>
__global__ __launch_bounds__(MW * 64) void k_gateup_mfma(const uint8_t *__restrict__ nib,
                                                         const uint16_t *__restrict__ scl,
                                                         const int32_t *__restrict__ tiles,
                                                         const int32_t *__restrict__ gstart,
                                                         const int32_t *__restrict__ order,
                                                         const int8_t *__restrict__ xq8,
                                                         const float *__restrict__ xsc, int8_t *__restrict__ hq8,
                                                         float *__restrict__ hsc, int d, int ff, int top_k) {
    constexpr int R = 16 * MT, KC = chunk_blocks<MT>();
    __shared__ TileLds<MT, 4, KC> sh;
    const int tile = blockIdx.x;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(R, gstart[e + 1] - k0);
    const int nb = d / QK, Tg = ff / 32;
    if (threadIdx.x < R) sh.row_of[threadIdx.x] = (int)threadIdx.x < cnt ? order[k0 + threadIdx.x] / top_k : -1;
    __syncthreads();
    const int rt = blockIdx.y * MW + (threadIdx.x >> 6);
    const bool active = rt < Tg;
    float acc[MT][4][4];
    tile_sums<MT, 4, KC>(nib, scl, ((size_t)e * Tg + (active ? rt : 0)) * nb, nb, active, xq8, xsc, d, sh, acc);
    if (!active) return;
    const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (mt * 16 >= cnt) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float h0 = gelu(acc[mt][0][i]) * acc[mt][2][i];
            const float h1 = gelu(acc[mt][1][i]) * acc[mt][3][i];
            const float amax = row16_max(fmaxf(fmaxf(0.0f, fabsf(h0)), fabsf(h1)));
            const float dq = amax / 127.0f;
            const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
            const uint16_t dbits = f2h_rne(dq);
            const int q0 = sat_i8(roundf(h0 * id)), q1 = sat_i8(roundf(h1 * id));
            const int pr = mt * 16 + 4 * g + i;
            if (pr < cnt) {
                int8_t *hrow = hq8 + (size_t)(k0 + pr) * ff + rt * QK;
                hrow[kperm(m)] = (int8_t)q0;
                hrow[kperm(16 + m)] = (int8_t)q1;
                if (m == 0) hsc[(size_t)(k0 + pr) * Tg + rt] = h2f(dbits);
            }
        }
    }
}

// Down for one tile: wave w takes the 32-row down tile rt = 4 blockIdx.y + w (RVM_PACK_ROWS32:
// row r of the tile is plane lane r at block b < S, lane 32 + r at block S + b; pieces 0, 1 are
// rows m and 16 + m).
template <int MT>
__global__ __launch_bounds__(MW * 64) void k_down_mfma(const uint8_t *__restrict__ nib,
                                                       const uint16_t *__restrict__ scl,
                                                       const int32_t *__restrict__ tiles,
                                                       const int32_t *__restrict__ gstart,
                                                       const int8_t *__restrict__ hq8, const float *__restrict__ hsc,
                                                       float *__restrict__ y, int d, int ff) {
    constexpr int R = 16 * MT, KC = chunk_blocks<MT>();
    __shared__ TileLds<MT, 2, KC> sh;
    const int tile = blockIdx.x;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(R, gstart[e + 1] - k0);
    const int Sd = ff / 64, Td = d / 32;
    if (threadIdx.x < R) sh.row_of[threadIdx.x] = (int)threadIdx.x < cnt ? k0 + (int)threadIdx.x : -1;
    __syncthreads();
    const int rt = blockIdx.y * MW + (threadIdx.x >> 6);
    const bool active = rt < Td;
    float acc[MT][2][4];
    tile_sums<MT, 2, KC>(nib, scl, ((size_t)e * Td + (active ? rt : 0)) * Sd, Sd, active, hq8, hsc, ff, sh, acc);
    if (!active) return;
    const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int pr = mt * 16 + 4 * g + i;
            if (pr < cnt) {
                float *yrow = y + (size_t)(k0 + pr) * d + rt * 32;
                yrow[m] = acc[mt][0][i];
                yrow[16 + m] = acc[mt][1][i];
            }
        }
}

// out[t] = sum over slots j in order of (y[pos_of[t k + j]] * down_scale[e]) * weight, the first
// term taken as is (runtime/src/hip_ops.rs:421-439). One thread per 4 columns; the slot data is
// per token, so it is loaded once into LDS.
__global__ __launch_bounds__(256) void k_combine_pairs(const float *__restrict__ y, const int32_t *__restrict__ pos_of,
                                                       const int32_t *__restrict__ ids, const float *__restrict__ wts,
                                                       const float *__restrict__ dscale, float *__restrict__ out,
                                                       int top_k, int d) {
    __shared__ int pos[MAX_TOP_K];
    __shared__ float ds[MAX_TOP_K], wt[MAX_TOP_K];
    const int t = blockIdx.y;
    if ((int)threadIdx.x < top_k) {
        const int p = t * top_k + threadIdx.x;
        pos[threadIdx.x] = pos_of[p];
        ds[threadIdx.x] = dscale ? dscale[ids[p]] : 1.0f;
        wt[threadIdx.x] = wts[p];
    }
    __syncthreads();
    const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= d) return;
    float4 v[MAX_TOP_K];
#pragma unroll
    for (int j = 0; j < MAX_TOP_K; ++j)
        if (j < top_k) v[j] = *(const float4 *)(y + (size_t)pos[j] * d + c);
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < MAX_TOP_K; ++j) {
        if (j >= top_k) break;
        const float s = ds[j], wj = wt[j];
        const float4 q = make_float4(v[j].x * s * wj, v[j].y * s * wj, v[j].z * s * wj, v[j].w * s * wj);
        if (j == 0) {
            o = q;
        } else {
            o.x = o.x + q.x;
            o.y = o.y + q.y;
            o.z = o.z + q.z;
            o.w = o.w + q.w;
        }
    }
    *(float4 *)(out + (size_t)t * d + c) = o;
}

// Pairs per tile: enough m-tiles that a typical group fits one tile, so that its weights are
// streamed once.
inline int tile_mt(const rvm_layer *L, int n_tok) {
    const long pairs = (long)n_tok * L->top_k;
    if (pairs >= 8L * L->n_exp) return 2;
    return 1;
}

template <int MT>
int launch_experts(const rvm_layer *L, int n_tok, uint8_t *w, const WsLayout &lay) {
    const int32_t *tiles = (const int32_t *)(w + lay.tiles);
    const int32_t *gstart = (const int32_t *)(w + lay.gstart);
    const int nt = (int)max_tiles(L, n_tok, 16 * MT);
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint8_t *gnib = (const uint8_t *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)(gnib + gu_entries * 16);
    hipLaunchKernelGGL(k_gateup_mfma<MT>, dim3(nt, grid_blocks(L->ff / 32, MW)), dim3(MW * 64), 0, cur_stream(), gnib,
                       gscl, tiles, gstart, (const int32_t *)(w + lay.order), (const int8_t *)(w + lay.xq8),
                       (const float *)(w + lay.xsc), (int8_t *)(w + lay.hq8), (float *)(w + lay.hsc), L->d, L->ff,
                       L->top_k);
    int rc = launched();
    if (rc) return rc;
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint8_t *dnib = (const uint8_t *)L->down;
    const uint16_t *dscl = (const uint16_t *)(dnib + dn_entries * 16);
    hipLaunchKernelGGL(k_down_mfma<MT>, dim3(nt, grid_blocks(L->d / 32, MW)), dim3(MW * 64), 0, cur_stream(), dnib,
                       dscl, tiles, gstart, (const int8_t *)(w + lay.hq8), (const float *)(w + lay.hsc),
                       (float *)(w + lay.y), L->d, L->ff);
    return launched();
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
    int32_t *pos_of = (int32_t *)(w + lay.pos_of);
    int rc = launch_router(L, x, n_tok, flags, eps, w, lay, ids, wts, nullptr, true);
    if (rc) return rc;
    const int mt = tile_mt(L, n_tok);
    if ((rc = launch_plan(ids, n_tok * L->top_k, L->n_exp, (int32_t *)(w + lay.order), pos_of,
                          (int32_t *)(w + lay.gstart), (int32_t *)(w + lay.tiles), 16 * mt)))
        return rc;
    rc = mt == 4 ? launch_experts<4>(L, n_tok, w, lay)
                 : (mt == 2 ? launch_experts<2>(L, n_tok, w, lay) : launch_experts<1>(L, n_tok, w, lay));
    if (rc) return rc;
    hipLaunchKernelGGL(k_combine_pairs, dim3(grid_blocks(L->d / 4, 256), n_tok), dim3(256), 0, cur_stream(),
                       (const float *)(w + lay.y), pos_of, ids, wts, L->down_scale, out, L->top_k, L->d);
    return launched();
}
