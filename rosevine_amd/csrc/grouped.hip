// grouped.hip - n_tok tokens through one MoE layer with device-side grouping (ragged decode
// batches and prefill; runtime/src/exec.rs:456-475 and 540-640, the reference's host dispatch is
// runtime/src/hip_exec.rs:822-843).
//
//   router (router.hip)   -> ids, weights, Q8_0 activation rows per token (K order of kperm)
//   k_plan (router.hip)   -> pairs stably grouped by expert, each group cut into tiles of up to
//                            48 pairs (batches of 8+ pairs per expert on average), or 4 (smaller),
//                            listed with the tiles of the most m-tiles of 16 pairs first
//   k_gateup_quad,        -> 4-pair tiles: one wave per (tile, 64 weight rows); the 16-block
//   k_down_quad              v_mfma_i32_4x4x4_16b_i8 gives each lane its row's exact block sums
//                            for the 4 pairs, so the f32 fold spends nothing on empty pair places
//   k_gateup_mfma         -> per (tile, 2 row tiles of 32 gate + 32 up rows, half a tile a wave): int8 MFMA
//                            (v_mfma_i32_16x16x32_i8, one 32-weight block per instruction) gives
//                            each block's exact int32 sum for 16 pairs x 16 rows; the f32 terms
//                            (sumi as f32) * (d_w * d_x) are folded in block order per output, as
//                            dot_q8_scalar does; GeGLU and the Q8_0 of h per pair finish the tile
//   k_down_mfma           -> per (48-pair tile, 4 row tiles of 32 down rows): the same on h, into
//                            y rows
//   k_combine_pairs       -> out[t] = sum_j (y[pos_of[t*k+j]] * scale) * weight, slot order
// Each pair's gate/up, h and y rows are the reference's sequential folds of exact block sums, so
// they do not depend on the batch the pair arrives in. A token's output also carries its routing
// weights: below RVM_FOLD_MIN_TOKENS tokens they come from the certified estimates, as in decode,
// and the row equals the decode row bit for bit; from RVM_FOLD_MIN_TOKENS the weights are the
// reference's arithmetic on exact logits, and the row equals the oracle's bit for bit and the
// decode row within the f32 tolerance.
//
// The tile loop walks the K blocks in chunks of KC: the tile's activation rows for a chunk are
// staged in LDS (double-buffered, one barrier per chunk), and each wave keeps the next chunk's
// weight dwords and scales in flight while it computes the current one.
#include <cmath>

#include "internal.hpp"

namespace rvm {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int MW = 4;  // waves (row tiles) per workgroup

// Workgroups go to the 8 XCDs in turn, by linear index. A grid row of a multiple of 8 workgroups
// sends row tile x of every tile to the same XCD, so the tiles of one expert share its L2 there
// (the small-batch kernels, where a popular expert has several tiles; the arithmetic-bound batched
// kernels keep every XCD busy instead).
inline int xcd_rows(int n) { return (n + 7) & ~7; }
// K blocks per chunk of the tile loop: 4 for gate/up (d is a multiple of 256, so d / 32 blocks
// are whole chunks; 8 measured slower for one m-tile), 2 for down (ff is a multiple of 64)
constexpr int GU_KC = 4, DN_KC = 2;

// 16 times the int8 weights of one K slice of a packed Q4_0 entry's dword g (bytes 4g .. 4g+3,
// each nibble the 4-bit two's complement weight; byte k holds elements 4g + k in its low nibble and
// 16 + 4g + k in its high one): the low nibbles moved to the top of each byte, or the high nibbles
// in place. Products with these sum to 16 sumi, exactly (|16 sumi| < 2^20); the activation scales
// are staged divided by 16, which is exact for binary16 values, so the folds see the reference's
// terms: (16 sumi) * (d_w * d_x / 16) rounds the same real number as sumi * (d_w * d_x).
__device__ __forceinline__ int slice_lo16(uint32_t p) { return (int)((p << 4) & 0xF0F0F0F0u); }
__device__ __forceinline__ int slice_hi16(uint32_t p) { return (int)(p & 0xF0F0F0F0u); }
// The 8 weights of dword p for a 16x16x32 MFMA K group: elements 4g .. 4g+3, then 16+4g .. 16+4g+3
// (the K group order of kperm), each times 16.
__device__ __forceinline__ long weights16(uint32_t p) {
    return (long)(((uint64_t)(uint32_t)slice_hi16(p) << 32) | (uint32_t)slice_lo16(p));
}

// Max over each row of 16 lanes (the lanes of one MFMA K group) of non-NaN values.
__device__ __forceinline__ float row16_max(float m) {
    m = maxf_bits(m, dpp<0xb1>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x4e>(__builtin_bit_cast(uint32_t, m)));
    m = maxf_bits(m, dpp<0x141>(__builtin_bit_cast(uint32_t, m)));
    return maxf_bits(m, dpp<0x140>(__builtin_bit_cast(uint32_t, m)));
}

// The f32 fold of one block into acc: acc[i] = acc[i] + (16 sumi as f32) * (d_w * d_x[i] / 16),
// the reference's term sumi * (d_w * d_x[i]) (dx holds d_x / 16).
__device__ __forceinline__ void fold_block(float (&acc)[4], v4i sumi, float dw, float4 dx) {
    acc[0] = acc[0] + (float)sumi[0] * (dw * dx.x);
    acc[1] = acc[1] + (float)sumi[1] * (dw * dx.y);
    acc[2] = acc[2] + (float)sumi[2] * (dw * dx.z);
    acc[3] = acc[3] + (float)sumi[3] * (dw * dx.w);
}

template <int MT, int NR, int KC, int W = MW>
struct TileLds {
    static constexpr int R = 16 * MT, XP = KC * QK + 16;  // row pitch: conflict-free 8-byte reads
    alignas(16) int8_t xs[2][R * XP];           // activation rows of the chunk
    alignas(16) float ss[2][KC * R];            // their block scales, [block][row]
    alignas(16) float ws[W][KC * 16 * NR];      // per wave: weight scales, [block][m][piece]
    int row_of[R];                              // source row of each tile place, -1 when empty
};

// The block sums of one tile: rows of the wave's row tile (entry groups tb .. tb+S-1, NR pieces of
// 16 plane lanes, pieces p0, p0 + PS, ..., wave-uniform; block b uses group b mod S at lane offset
// 32 (b / S) when HALVES, group b otherwise) against the tile's R activation rows (K = width,
// nb = width / 32 blocks, a multiple of KC; src holds rows rows of width bytes, ssrc their nb block
// scales). acc[mt][r][i] is the output of pair 16 mt + 4 g + i and plane lane 16 r + m, for
// lane = 16 g + m. Only the first LIVE m-tiles are computed (the others hold no pair; their acc
// stays 0). All waves take part in the staging and barriers; waves without a row tile (active
// false) skip the MFMAs.
template <int MT, int NR, int KC, int LIVE, bool HALVES, int W = MW, int PS = 1>
__device__ __forceinline__ void tile_sums(const uint8_t *__restrict__ nib, const uint16_t *__restrict__ scl,
                                          size_t tb, int S, bool active, const int8_t *__restrict__ src,
                                          const float *__restrict__ ssrc, int width, int rows,
                                          TileLds<MT, NR, KC, W> &sh, float (&acc)[MT][NR][4], int p0 = 0) {
    // Every load goes through a buffer descriptor: the wave-uniform part of its offset (the chunk's)
    // sits in a scalar register, so the loads cost no vector address arithmetic, and an empty tile
    // place's loads take an offset past the end of the buffer, which reads 0. The loads of the chunk
    // after the last reload the last chunk (unused), so every load is issued unconditionally and the
    // compiler can count the loads in flight and wait for exactly the ones it needs: the next
    // chunk's loads stay outstanding while this one runs. Whole chunks only (no exit inside the
    // unrolled block loop, whose join would copy every accumulator).
    constexpr int R = 16 * MT, NT = W * 64, XP = TileLds<MT, NR, KC, W>::XP;
    constexpr int XU = KC * QK / 16;  // 16-byte pieces of a staged row chunk
    constexpr int XI = (R * XU + NT - 1) / NT, SI = (R * KC + NT - 1) / NT;
    constexpr int SPL = KC * 16 * NR / 64;  // weight scales per lane per chunk
    static_assert(NR == 2 && (SPL == 1 || SPL == 2), "two pieces of 16 rows per wave, at most one dword of scales per lane and chunk");
    const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = width / QK, nch = nb / KC;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][r][i] = 0.0f;

    // the row tile's plane entries (S groups of 64) and their scales; the activation rows and scales
    const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(nib + tb * 1024, (uint32_t)S * 1024u);
    const __amdgpu_buffer_rsrc_t sres = buffer_rsrc(scl + tb * 64, (uint32_t)S * 128u);
    const __amdgpu_buffer_rsrc_t xres = buffer_rsrc(src, (uint32_t)rows * (uint32_t)width);
    const __amdgpu_buffer_rsrc_t xsres = buffer_rsrc(ssrc, (uint32_t)rows * (uint32_t)nb * 4u);
    constexpr uint32_t EMPTY = 0x80000000u;  // an offset past the end of every buffer here
    auto eoff = [&](int b) {  // entry of block b from the row tile's first
        if constexpr (HALVES) {
            const int half = b >= S ? 1 : 0;
            return (b - half * S) * 64 + 32 * half;
        } else {
            return b * 64;
        }
    };
    // this lane's share of a chunk's weight scales: block kb = lane / (64 / KC), entries
    // j .. j+SPL-1 of it, plane lane 16 (p0 + PS (j / 16)) + j mod 16
    constexpr int LPB = 64 / KC;
    const int skb = lane / LPB, sj = (lane % LPB) * SPL;
    const int sjl = 16 * p0 + (sj & 15) + 16 * PS * (sj >> 4);
    // this thread's staging items, fixed over the chunks: activation piece q of tile place xrow[k],
    // and the scale of place srow[k] at chunk block skbx[k] (offsets at chunk 0)
    uint32_t xoff[XI];
    int xdst[XI];
#pragma unroll
    for (int k = 0; k < XI; ++k) {
        const int i = threadIdx.x + k * NT, ii = min(i, R * XU - 1);
        const int row = ii / XU, q = ii - row * XU, from = sh.row_of[row];
        xoff[k] = from >= 0 ? (uint32_t)from * (uint32_t)width + (uint32_t)(q * 16) : EMPTY;
        xdst[k] = i < R * XU ? row * XP + q * 16 : -1;
    }
    uint32_t soffx[SI];
    int sdst[SI];
#pragma unroll
    for (int k = 0; k < SI; ++k) {
        const int i = threadIdx.x + k * NT, ii = min(i, R * KC - 1);
        const int kb = ii / R, row = ii - kb * R, from = sh.row_of[row];
        soffx[k] = from >= 0 ? ((uint32_t)from * (uint32_t)nb + (uint32_t)kb) * 4u : EMPTY;
        sdst[k] = i < R * KC ? i : -1;  // [block][row]
    }

    const int loff = m * 16 + 4 * g;  // this lane's byte in a piece of 16 plane entries
    auto load_w = [&](int c, uint32_t (&wn)[KC][NR], uint32_t &wsc) {
        const int cc = min(c, nch - 1);
#pragma unroll
        for (int kb = 0; kb < KC; ++kb) {
            const uint32_t so = (uint32_t)eoff(cc * KC + kb) * 16u;  // wave-uniform
#pragma unroll
            for (int r = 0; r < NR; ++r) wn[kb][r] = buffer_load_u32(wres, (uint32_t)(256 * (p0 + PS * r) + loff), so);
        }
        if constexpr (HALVES) {
            const uint32_t vo = (uint32_t)(eoff(cc * KC + skb) + sjl) * 2u;
            wsc = SPL == 2 ? buffer_load_u32(sres, vo, 0) : buffer_load_u16(sres, vo, 0);
        } else {
            const uint32_t vo = (uint32_t)(skb * 64 + sjl) * 2u, so = (uint32_t)(cc * KC) * 128u;
            wsc = SPL == 2 ? buffer_load_u32(sres, vo, so) : buffer_load_u16(sres, vo, so);
        }
    };
    auto load_x = [&](int c, uint4 (&xr)[XI], float (&sr)[SI]) {
        const uint32_t cc = (uint32_t)min(c, nch - 1);
#pragma unroll
        for (int k = 0; k < XI; ++k) xr[k] = buffer_load_u4(xres, xoff[k], cc * (KC * QK));
#pragma unroll
        for (int k = 0; k < SI; ++k) sr[k] = buffer_load_f32(xsres, soffx[k], cc * (KC * 4));
    };
    auto store_x = [&](int buf, const uint4 (&xr)[XI], const float (&sr)[SI]) {
#pragma unroll
        for (int k = 0; k < XI; ++k)
            if (xdst[k] >= 0) *(uint4 *)(sh.xs[buf] + xdst[k]) = xr[k];
#pragma unroll
        for (int k = 0; k < SI; ++k)
            if (sdst[k] >= 0) sh.ss[buf][sdst[k]] = sr[k] * 0.0625f;  // d_x / 16
    };
    auto compute = [&](int buf, const uint32_t (&wn)[KC][NR], uint32_t wsc) {
        if (!active) return;
        // the chunk's weight scales as f32 to [block][m][piece] in this wave's LDS
        float *wsw = sh.ws[w];
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
            const int j = sj + k;
            wsw[(skb * 16 + (j & 15)) * NR + (j >> 4)] = h2f((uint16_t)(wsc >> (16 * k)));
        }
        wave_lds_sync();
#pragma unroll
        for (int kb = 0; kb < KC; ++kb) {
            const float2 v = *(const float2 *)(wsw + (kb * 16 + m) * NR);
            const float dw[NR] = {v.x, v.y};
            long a[MT];
            float4 dx[MT];
#pragma unroll
            for (int mt = 0; mt < LIVE; ++mt) {
                a[mt] = *(const long *)(sh.xs[buf] + (mt * 16 + m) * XP + kb * QK + g * 8);
                dx[mt] = *(const float4 *)(sh.ss[buf] + kb * R + mt * 16 + 4 * g);
            }
            // every MFMA of the block first, then the folds: no fold waits on the MFMA just issued
            v4i sm[MT][NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const long bw = weights16(wn[kb][r]);
#pragma unroll
                for (int mt = 0; mt < LIVE; ++mt)
                    sm[mt][r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[mt], bw, v4i{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int mt = 0; mt < LIVE; ++mt) fold_block(acc[mt][r], sm[mt][r], dw[r], dx[mt]);
        }
        wave_lds_sync();  // the next chunk's scale stores stay behind these reads
    };

    uint32_t wn0[KC][NR], wn1[KC][NR];
    uint32_t ws0, ws1;
    uint4 xr[XI];
    float sr[SI];
    load_x(0, xr, sr);
    load_w(0, wn0, ws0);
    store_x(0, xr, sr);
    __syncthreads();
    for (int c = 0; c < nch; c += 2) {
        {
            const bool more = c + 1 < nch;
            // staging loads first: store_x waits for them, and the in-order load counter then
            // leaves the weight loads behind them in flight
            load_x(c + 1, xr, sr);
            load_w(c + 1, wn1, ws1);
            compute(0, wn0, ws0);
            if (more) store_x(1, xr, sr);
            __syncthreads();
        }
        if (c + 1 < nch) {
            const bool more = c + 2 < nch;
            load_x(c + 2, xr, sr);
            load_w(c + 2, wn0, ws0);
            compute(1, wn1, ws1);
            if (more) store_x(0, xr, sr);
            __syncthreads();
        }
    }
}

// The tile's pair at place 16 mt + 4 g + i (MFMA row 4 g + i of m-tile mt, output register i of lane
// group g): pairs fill register (mt, i) of all four lane groups before the next, so a tile of cnt
// pairs occupies the first ceil(cnt / 4) registers and the epilogue skips the others (the pairs of
// one register are the same MFMA rows for every lane, so the skip is wave-uniform).
__device__ __forceinline__ int place_pair(int mt, int g, int i) { return 4 * (4 * mt + i) + g; }

// Gate/up for one tile (blockIdx.y) of up to 16 MT pairs of expert e, TW row tiles per workgroup
// (32 gate rows and the matching 32 up rows each, one RVM_PACK_GATE_UP tile), half a row tile per
// wave: wave w takes row tile rt = TW blockIdx.x + w / 2, gate rows 16 h + m (piece h = w mod 2) and
// the matching up rows (piece h + 2). Half-tile waves are twice as many, each half as long, at four
// waves per SIMD (against three for whole row tiles): the grid's last partial round of workgroups
// leaves fewer SIMDs short of waves (512 tokens: 297 -> 275 us per call). A tile runs the loop of
// its occupied m-tiles only. Four waves per SIMD are asked for: 48-pair tiles need 145 VGPRs
// otherwise (three waves); at 128 a few values outside the tile loop go to scratch.
// h = gelu(gate) * up is quantised per pair to one Q8_0 block of 32 (runtime/src/ops.rs:95-105) and
// stored in the K order of kperm; the block spans both waves' rows, so they exchange their maxima of
// |h| in LDS (a maximum of non-negative values, the same bits in any order).
template <int MT, int TW>
__global__ __launch_bounds__(128 * TW) __attribute__((amdgpu_waves_per_eu(4))) void k_gateup_mfma(const uint8_t *__restrict__ nib,
                                                          const uint16_t *__restrict__ scl,
                                                          const int32_t *__restrict__ tiles,
                                                          const int32_t *__restrict__ gstart,
                                                          const int32_t *__restrict__ order,
                                                          const int8_t *__restrict__ xq8,
                                                          const float *__restrict__ xsc, int8_t *__restrict__ hq8,
                                                          float *__restrict__ hsc, int d, int ff, int top_k,
                                                          int n_tok) {
    constexpr int R = 16 * MT, KC = GU_KC;
    __shared__ TileLds<MT, 2, KC, 2 * TW> sh;
    __shared__ float hmax[2 * TW][MT][4][4];  // [wave][m-tile][i][g]: max of |h| over the wave's 16 rows
    __shared__ alignas(8) float qsc[TW][R][2];  // [row tile][tile place]: the Q8_0 block's d and 1/d
    const int tile = blockIdx.y;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(R, gstart[e + 1] - k0);
    const int nb = d / QK, Tg = ff / 32;
    if (threadIdx.x < R) {  // tile place 16 mt + 4 g + i holds pair place_pair(...) of the tile
        const int p = threadIdx.x, pr = place_pair(p >> 4, (p >> 2) & 3, p & 3);
        sh.row_of[p] = pr < cnt ? order[k0 + pr] / top_k : -1;
    }
    __syncthreads();
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = wv & 1;
    const int rt = blockIdx.x * TW + (wv >> 1);
    const bool active = rt < Tg;
    float acc[MT][2][4];
    const size_t tb = ((size_t)e * Tg + (active ? rt : 0)) * nb;
    if (MT > 1 && cnt <= 16)  // a tile of at most 16 pairs runs the loop of its one occupied m-tile
        tile_sums<MT, 2, KC, 1, false, 2 * TW, 2>(nib, scl, tb, nb, active, xq8, xsc, d, n_tok, sh, acc, h);
    else if (MT > 2 && cnt <= 32)
        tile_sums<MT, 2, KC, (MT > 2 ? 2 : MT), false, 2 * TW, 2>(nib, scl, tb, nb, active, xq8, xsc, d, n_tok, sh, acc, h);
    else
        tile_sums<MT, 2, KC, MT, false, 2 * TW, 2>(nib, scl, tb, nb, active, xq8, xsc, d, n_tok, sh, acc, h);
    const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
    float hv[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (place_pair(mt, 0, i) >= cnt) break;  // wave-uniform: no pair in this register
            hv[mt][i] = gelu(acc[mt][0][i]) * acc[mt][1][i];
            const float mx = row16_max(fmaxf(0.0f, fabsf(hv[mt][i])));
            if (m == 0) hmax[wv][mt][i][g] = mx;
        }
    }
    __syncthreads();
    // each block's scale d = amax / 127 and 1/d once, by one thread per (row tile, tile place),
    // instead of in every lane of the block's 16 rows in both waves (places without a pair
    // compute from maxima that were not written: unused)
    if ((int)threadIdx.x < TW * R) {
        const int rtl = threadIdx.x / R, p = threadIdx.x - rtl * R;
        const int pm = p >> 4, pg = (p >> 2) & 3, pi = p & 3;
        const float amax = fmaxf(hmax[2 * rtl][pm][pi][pg], hmax[2 * rtl + 1][pm][pi][pg]);
        const float dq = amax / 127.0f;
        qsc[rtl][p][0] = dq;
        qsc[rtl][p][1] = dq != 0.0f ? 1.0f / dq : 0.0f;
    }
    __syncthreads();
    if (!active) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (place_pair(mt, 0, i) >= cnt) break;
            const float2 dqi = *(const float2 *)qsc[wv >> 1][16 * mt + 4 * g + i];
            const int q = sat_i8(roundf(hv[mt][i] * dqi.y));
            const int pr = place_pair(mt, g, i);
            if (pr < cnt) {
                int8_t *hrow = hq8 + (size_t)(k0 + pr) * ff + rt * QK;
                hrow[kperm(16 * h + m)] = (int8_t)q;
                if (h == 0 && m == 0) hsc[(size_t)(k0 + pr) * Tg + rt] = h2f(f2h_rne(dqi.x));
            }
        }
    }
}

// Down for one tile (blockIdx.y): wave w takes the 32-row down tile rt = 4 blockIdx.x + w (RVM_PACK_ROWS32:
// row r of the tile is plane lane r at block b < S, lane 32 + r at block S + b; pieces 0, 1 are
// rows m and 16 + m).
template <int MT>
__global__ __launch_bounds__(MW * 64) void k_down_mfma(const uint8_t *__restrict__ nib,
                                                       const uint16_t *__restrict__ scl,
                                                       const int32_t *__restrict__ tiles,
                                                       const int32_t *__restrict__ gstart,
                                                       const int8_t *__restrict__ hq8, const float *__restrict__ hsc,
                                                       float *__restrict__ y, int d, int ff, int n_pairs) {
    constexpr int R = 16 * MT, KC = DN_KC;
    __shared__ TileLds<MT, 2, KC> sh;
    const int tile = blockIdx.y;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(R, gstart[e + 1] - k0);
    const int Sd = ff / 64, Td = d / 32;
    if (threadIdx.x < R) sh.row_of[threadIdx.x] = (int)threadIdx.x < cnt ? k0 + (int)threadIdx.x : -1;
    __syncthreads();
    const int rt = blockIdx.x * MW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const bool active = rt < Td;
    float acc[MT][2][4];
    // a tile runs the loop of its occupied m-tiles only (half row tiles per wave, as in the gate/up
    // kernel, measured slower here: 282 against 276.5 us for 512 tokens)
    const size_t tb = ((size_t)e * Td + (active ? rt : 0)) * Sd;
    if (MT > 1 && cnt <= 16)
        tile_sums<MT, 2, KC, 1, true>(nib, scl, tb, Sd, active, hq8, hsc, ff, n_pairs, sh, acc);
    else if (MT > 2 && cnt <= 32)
        tile_sums<MT, 2, KC, (MT > 2 ? 2 : MT), true>(nib, scl, tb, Sd, active, hq8, hsc, ff, n_pairs, sh, acc);
    else
        tile_sums<MT, 2, KC, MT, true>(nib, scl, tb, Sd, active, hq8, hsc, ff, n_pairs, sh, acc);
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

// ---- Quad tiles: up to 4 pairs of one expert (small batches, where most groups hold a few
// pairs and a 16-pair m-tile would spend most of its arithmetic on empty places) ----
//
// v_mfma_i32_4x4x4_16b_i8 computes 16 independent 4x4x4 products. In block q (lanes 4q .. 4q+3),
// lane 4q + i gives row i of A and lane 4q + j column j of B (4 int8 each), and register i of
// lane 4q + j receives D[i][j]. With row i of A = 4 activations of pair i (the same in every block)
// and column j of block q = the 4 weights of row 4q + j, lane l accumulates the four pairs' sums
// of weight row l: eight instructions cover one 32-weight block, and the f32 fold takes four
// outputs per lane.
constexpr int QUAD = MIN_TILE_PAIRS;  // pairs per quad tile

// 16 times the block sums of this lane's weight row (entry w) with the four pairs' activations
// (x0, x1: the 32 bytes of the block in the K order of kperm, dwords 2g and 2g + 1 holding the
// elements of weight dword g's low and high nibbles).
__device__ __forceinline__ v4i quad_sums16(uint4 w, uint4 x0, uint4 x1) {
    v4i s = {0, 0, 0, 0};
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x0.x, slice_lo16(w.x), s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x0.y, slice_hi16(w.x), s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x0.z, slice_lo16(w.y), s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x0.w, slice_hi16(w.y), s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x1.x, slice_lo16(w.z), s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x1.y, slice_hi16(w.z), s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x1.z, slice_lo16(w.w), s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_i32_4x4x4i8((int)x1.w, slice_hi16(w.w), s, 0, 0, 0);
    return s;
}

// acc[i] = acc[i] + (16 sumi_i as f32) * (d_w / 16 * d_x_i), the reference's term (dw holds d_w / 16,
// dx the four pairs' d_x: d_w * d_x is exact in f32 for binary16 scales, and so is its sixteenth).
// Only the first NP pairs are folded (the MFMA forms all four sums either way).
template <int NP>
__device__ __forceinline__ void quad_fold(float (&acc)[4], v4i s16, float dw, float4 dx) {
    const float dxi[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
    for (int i = 0; i < NP; ++i) acc[i] = acc[i] + (float)s16[i] * (dw * dxi[i]);
}

// The wave's LDS region: the four pairs' activation rows (K order of kperm) at a pitch of
// width + 16 bytes, so that the four rows start on different LDS banks, then their block scales,
// [block][pair].
__host__ __device__ constexpr int quad_pitch(int width) { return width + 16; }
__host__ __device__ constexpr int quad_lds_bytes(int width) { return 4 * quad_pitch(width) + 4 * (width / QK) * 4; }

// Copies the rows src_r = src + row_r * width (and scales ssrc + row_r * nb) of the wave's four
// pairs into its LDS region; row_r comes from lane r of rowv. The copies go from memory straight
// to LDS (64 pieces of 16 bytes of one row, or 64 scales, per instruction), all issued before one
// wait: one memory round trip, where register copies had one per piece.
__device__ __forceinline__ void stage_quad_rows(const int8_t *__restrict__ src, const float *__restrict__ ssrc,
                                                int rowv, int width, uint8_t *lds) {
    const int lane = threadIdx.x & 63, nb = width / QK, pcs = width / 16, P = quad_pitch(width);
    const uint32_t base = lds_addr(lds);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int8_t *rowp = src + (size_t)__builtin_amdgcn_readfirstlane(__shfl(rowv, r)) * width;
        for (int c0 = 0; c0 < pcs; c0 += 64)
            if (c0 + lane < pcs) lds_copy16(rowp + (size_t)(c0 + lane) * 16, base + r * P + c0 * 16);
    }
    // scale q = 4 b + r at [b][r]: lane l of a 64-scale copy is pair l mod 4
    const float *srow = ssrc + (size_t)__shfl(rowv, lane & 3) * nb;
    for (int q0 = 0; q0 < 4 * nb; q0 += 64)
        if (q0 + lane < 4 * nb) lds_copy4(srow + (q0 + lane) / 4, base + 4 * P + q0 * 4);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    wave_lds_sync();
}

// The four pairs' sequential folds of this lane's weight row over blocks 0 .. nb-1 (a multiple of
// QD). The lane's 16-byte weight entry of block b is entry lane_entry + boff(b) of the planes from
// nib and scl (its scale has the same index; entries: the planes' extent there, in entries), with
// boff(b) wave-uniform: the loads go through buffer descriptors with boff in a scalar register, so
// they cost no vector address arithmetic. stage(): fills lds, the wave's staged rows (the lane's
// pair is lane & 3). The weight loads run QD blocks ahead in a ring of registers.
template <int QD, int NP, class BlockOff, class Stage>
__device__ __forceinline__ void quad_row_sums(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl,
                                              uint32_t entries, uint32_t lane_entry, BlockOff boff, Stage stage,
                                              const uint8_t *lds, int width, float (&acc)[4]) {
    const int nb = width / QK, i = threadIdx.x & 3;
    const uint8_t *xl = lds + i * quad_pitch(width);
    const float4 *sl = (const float4 *)(lds + 4 * quad_pitch(width));
    const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(nib, entries * 16u), sres = buffer_rsrc(scl, entries * 2u);
    uint4 w[QD];
    uint32_t s[QD];
    auto load = [&](int u, int b) {
        const uint32_t so = (uint32_t)boff(b);
        w[u] = buffer_load_u4(wres, lane_entry * 16u, so * 16u);
        s[u] = buffer_load_u16(sres, lane_entry * 2u, so * 2u);
    };
    auto compute = [&](int u, int b) {
        const uint4 x0 = *(const uint4 *)(xl + 32 * b), x1 = *(const uint4 *)(xl + 32 * b + 16);
        quad_fold<NP>(acc, quad_sums16(w[u], x0, x1), h2f((uint16_t)s[u]) * 0.0625f, sl[b]);
    };
    // The first round only loads (and then stages the activation rows, their loads behind the
    // weights'): it is the same code as the later rounds, so the loads are issued in the same order
    // (one block's loads after each block's arithmetic) and each block waits for its own loads only.
    // The last round, blocks nb - QD .. nb - 1, loads nothing.
#pragma clang loop unroll(disable)
    for (int b0 = -QD; b0 < nb - QD; b0 += QD) {
#pragma unroll
        for (int u = 0; u < QD; ++u) {
            if (b0 >= 0) compute(u, b0 + u);
            load(u, b0 + u + QD);
        }
        if (b0 < 0) stage();
    }
#pragma unroll
    for (int u = 0; u < QD; ++u) compute(u, nb - QD + u);
}

// Ring depth for nb blocks, a divisor of nb (nb is even), so that the loop has no partial round:
// 8 for the long gate/up rows; 2 for short rows (the down rows, 22 blocks at ff = 704, measured
// faster at 2 than at 11).
inline int quad_depth(int nb) { return nb >= 64 && nb % 8 == 0 ? 8 : 2; }

// Gate/up for one quad tile (up to 4 pairs of expert e) and one 64-row tile rt
// (RVM_PACK_GATE_UP: lane l < 32 is gate row 32 rt + l, lane l >= 32 the matching up row), one
// wave per workgroup. Lanes < 32 then form h of pairs 0 and 1, lanes >= 32 those of pairs 2 and 3 (gelu(gate) * up, runtime/src/exec.rs:626-630), each half-wave
// quantising its pair's 32 values to one Q8_0 block (runtime/src/ops.rs:95-105) stored in the K
// order of kperm.
template <int QD>
__global__ __launch_bounds__(64) void k_gateup_quad(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl,
                                                     const int32_t *__restrict__ tiles,
                                                     const int32_t *__restrict__ gstart,
                                                     const int32_t *__restrict__ order,
                                                     const int8_t *__restrict__ xq8, const float *__restrict__ xsc,
                                                     int8_t *__restrict__ hq8, float *__restrict__ hsc, int d, int ff,
                                                     int top_k) {
    extern __shared__ uint4 quad_lds[];
    const int tile = blockIdx.y;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(QUAD, gstart[e + 1] - k0);
    const int lane = threadIdx.x, rt = blockIdx.x, nb = d / QK, Tg = ff / 32;
    if (rt >= Tg) return;  // the padding of the grid's rows
    uint8_t *lds = (uint8_t *)quad_lds;
    // the rows of the quad's pairs; a missing pair takes pair 0's row and is not stored
    const int tok = lane < 4 ? order[k0 + (lane < cnt ? lane : 0)] / top_k : 0;
    const size_t tb = ((size_t)e * Tg + rt) * nb;  // the row tile's first entry group
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto rows = [&](auto np) {
        quad_row_sums<QD, decltype(np)::value>(
            nib + tb * 64, scl + tb * 64, (uint32_t)nb * 64u, (uint32_t)lane, [&](int b) { return b * 64; },
            [&]() { stage_quad_rows(xq8, xsc, tok, d, lds); }, lds, d, acc);
    };
    if (cnt <= 2) rows(std::integral_constant<int, 2>{});  // a tile of one or two pairs folds two
    else rows(std::integral_constant<int, 4>{});
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __shfl_xor(acc[i], 32);
    const bool lo = lane < 32;
    const float hA = gelu(lo ? acc[0] : o[2]) * (lo ? o[0] : acc[2]);
    const float hB = gelu(lo ? acc[1] : o[3]) * (lo ? o[1] : acc[3]);
    uint16_t dA, dB;
    const int qA = quant_q8_half(hA, &dA), qB = quant_q8_half(hB, &dB);
    const int j = lane & 31, pA = lo ? 0 : 2;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int pr = pA + k;
        if (pr < cnt) {
            hq8[(size_t)(k0 + pr) * ff + rt * QK + kperm(j)] = (int8_t)(k ? qB : qA);
            if (j == 0) hsc[(size_t)(k0 + pr) * Tg + rt] = h2f(k ? dB : dA);
        }
    }
}

// Down for one quad tile and 64 rows (two RVM_PACK_ROWS32 tiles: lane l is row 64 x + l, in tile
// 2 x + l / 32 at place l & 31, block b at step b mod S, half b / S), one wave per workgroup.
template <int QD>
__global__ __launch_bounds__(64) void k_down_quad(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl,
                                                   const int32_t *__restrict__ tiles,
                                                   const int32_t *__restrict__ gstart, const int8_t *__restrict__ hq8,
                                                   const float *__restrict__ hsc, float *__restrict__ y, int d,
                                                   int ff) {
    extern __shared__ uint4 quad_lds[];
    const int tile = blockIdx.y;
    if (tile >= tiles[0]) return;
    const int e = tiles[1 + 2 * tile], k0 = tiles[2 + 2 * tile];
    const int cnt = min(QUAD, gstart[e + 1] - k0);
    const int lane = threadIdx.x, S = ff / 64, Td = d / 32;
    if ((int)blockIdx.x >= d / 64) return;  // the padding of the grid's rows
    uint8_t *lds = (uint8_t *)quad_lds;
    const size_t tb = ((size_t)e * Td + 2 * blockIdx.x) * S;  // the two row tiles' first entry group
    const int place = lane & 31;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto rows = [&](auto np) {
        quad_row_sums<QD, decltype(np)::value>(
            nib + tb * 64, scl + tb * 64, 2u * (uint32_t)S * 64u, (uint32_t)((lane >> 5) * S * 64 + place),
            [&](int b) {
                const int half = b >= S ? 1 : 0;
                return (b - half * S) * 64 + 32 * half;
            },
            [&]() { stage_quad_rows(hq8, hsc, k0 + (lane < cnt ? lane : 0), ff, lds); }, lds, ff, acc);
    };
    if (cnt <= 2) rows(std::integral_constant<int, 2>{});
    else rows(std::integral_constant<int, 4>{});
    const int row = 64 * blockIdx.x + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < cnt) y[(size_t)(k0 + i) * d + row] = acc[i];
}

template <class F>
int with_quad_depth(int nb, F &&f) {
    if (quad_depth(nb) == 8) return f(std::integral_constant<int, 8>{});
    return f(std::integral_constant<int, 2>{});
}

int launch_experts_quad(const rvm_layer *L, int n_tok, uint8_t *w, const WsLayout &lay) {
    const int32_t *tiles = (const int32_t *)(w + lay.tiles);
    const int32_t *gstart = (const int32_t *)(w + lay.gstart);
    const int nt = (int)max_tiles(L, n_tok, QUAD);
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint4 *gnib = (const uint4 *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)((const uint8_t *)L->gate_up + gu_entries * 16);
    int rc = with_quad_depth(L->d / QK, [&](auto qd) {
        hipLaunchKernelGGL(k_gateup_quad<decltype(qd)::value>, dim3(xcd_rows(L->ff / 32), nt), dim3(64), quad_lds_bytes(L->d),
                           cur_stream(),
                           gnib, gscl, tiles, gstart,
                           (const int32_t *)(w + lay.order), (const int8_t *)(w + lay.xq8),
                           (const float *)(w + lay.xsc), (int8_t *)(w + lay.hq8), (float *)(w + lay.hsc), L->d, L->ff,
                           L->top_k);
        return launched();
    });
    if (rc) return rc;
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint4 *dnib = (const uint4 *)L->down;
    const uint16_t *dscl = (const uint16_t *)((const uint8_t *)L->down + dn_entries * 16);
    return with_quad_depth(L->ff / QK, [&](auto qd) {
        hipLaunchKernelGGL(k_down_quad<decltype(qd)::value>, dim3(xcd_rows(L->d / 64), nt), dim3(64), quad_lds_bytes(L->ff),
                           cur_stream(), dnib, dscl, tiles, gstart,
                           (const int8_t *)(w + lay.hq8), (const float *)(w + lay.hsc), (float *)(w + lay.y), L->d,
                           L->ff);
        return launched();
    });
}

// Pairs per tile: quads while the groups are small (fewer pairs than 8 per expert on average),
// else the MFMA tiles (48 pairs for gate/up and down), so that a typical group fits one tile
// and its weights are streamed once.
inline int tile_pairs(const rvm_layer *L, int n_tok) {
    const long pairs = (long)n_tok * L->top_k;
    return pairs >= 8L * L->n_exp ? 48 : QUAD;
}

// The 16x16 MFMA kernels: gate/up on tiles of 16 MT pairs (lay.tiles), down on tiles of 16 MD pairs
// (lay.tiles2). Both take three m-tiles: 48-pair tiles split fewer experts' pairs over two tiles,
// whose weights are then streamed twice (gate/up 512 tokens: 241.5-243.6 against 244.6-246.3 us
// with 32-pair tiles; down 73 against 82.5 us), each tile through the loop of only its occupied
// m-tiles.
template <int MT, int MD>
int launch_experts(const rvm_layer *L, int n_tok, uint8_t *w, const WsLayout &lay) {
    const int32_t *tiles = (const int32_t *)(w + lay.tiles);
    const int32_t *tiles2 = (const int32_t *)(w + lay.tiles2);
    const int32_t *gstart = (const int32_t *)(w + lay.gstart);
    const int nt = (int)max_tiles(L, n_tok, 16 * MT), nd = (int)max_tiles(L, n_tok, 16 * MD);
    const size_t gu_entries = (size_t)L->n_exp * 2 * L->ff * (L->d / QK);
    const uint8_t *gnib = (const uint8_t *)L->gate_up;
    const uint16_t *gscl = (const uint16_t *)(gnib + gu_entries * 16);
    constexpr int TW = 2;  // row tiles per gate/up workgroup (one: 280 against 275 us for 512 tokens)
    auto *gkern = k_gateup_mfma<MT, TW>;
    hipLaunchKernelGGL(gkern, dim3(grid_blocks(L->ff / 32, TW), nt), dim3(128 * TW), 0, cur_stream(), gnib, gscl, tiles,
                       gstart, (const int32_t *)(w + lay.order), (const int8_t *)(w + lay.xq8),
                       (const float *)(w + lay.xsc), (int8_t *)(w + lay.hq8), (float *)(w + lay.hsc), L->d, L->ff,
                       L->top_k, n_tok);
    int rc = launched();
    if (rc) return rc;
    const size_t dn_entries = (size_t)L->n_exp * L->d * (L->ff / QK);
    const uint8_t *dnib = (const uint8_t *)L->down;
    const uint16_t *dscl = (const uint16_t *)(dnib + dn_entries * 16);
    hipLaunchKernelGGL(k_down_mfma<MD>, dim3(grid_blocks(L->d / 32, MW), nd), dim3(MW * 64), 0, cur_stream(), dnib,
                       dscl, tiles2, gstart, (const int8_t *)(w + lay.hq8), (const float *)(w + lay.hsc),
                       (float *)(w + lay.y), L->d, L->ff, n_tok * L->top_k);
    return launched();
}

int moe_forward(const rvm_layer *L, const float *x, float *out, int n_tok, int flags, const XForm &xf, void *ws,
                size_t ws_bytes, bool stream) {
    RVM_CHECK(layer_ok(L) && x && out && ws && n_tok > 0 && n_tok <= MAX_TOKENS);
    if (n_tok == 1) return moe_decode(L, x, out, flags, xf, ws, ws_bytes, stream);
    const WsLayout lay = ws_layout(L, n_tok);
    RVM_CHECK(ws_bytes >= lay.total);
    uint8_t *w = (uint8_t *)ws;
    int32_t *ids = (int32_t *)(w + lay.ids);
    float *wts = (float *)(w + lay.wts);
    int32_t *pos_of = (int32_t *)(w + lay.pos_of);
    int rc = launch_router(L, x, n_tok, flags, xf, w, lay, ids, wts, nullptr, true);
    if (rc || (rc = span_router_done())) return rc;
    constexpr int GU_MT = 3, DN_MT = 3;  // m-tiles per tile of the two MFMA kernels
    const int cap = tile_pairs(L, n_tok);
    const bool quad = cap == QUAD;
    if ((rc = launch_plan(ids, n_tok * L->top_k, L->n_exp, (int32_t *)(w + lay.order), pos_of,
                          (int32_t *)(w + lay.gstart), (int32_t *)(w + lay.tiles), quad ? QUAD : 16 * GU_MT,
                          quad ? nullptr : (int32_t *)(w + lay.tiles2), 16 * DN_MT)))
        return rc;
    rc = quad ? launch_experts_quad(L, n_tok, w, lay) : launch_experts<GU_MT, DN_MT>(L, n_tok, w, lay);
    if (rc) return rc;
    hipLaunchKernelGGL(k_combine_pairs, dim3(grid_blocks(L->d / 4, 256), n_tok), dim3(256), 0, cur_stream(),
                       (const float *)(w + lay.y), pos_of, ids, wts, L->down_scale, out, L->top_k, L->d);
    return launched();
}

}  // namespace rvm

using namespace rvm;

extern "C" int rvm_moe_forward(const rvm_layer *L, const float *x, float *out, int n_tok, int flags, float eps,
                               void *ws, size_t ws_bytes) {
    return moe_forward(L, x, out, n_tok, flags, xform_of_flags(flags, eps), ws, ws_bytes);
}

namespace {

// The block entries' input transform: always normed, with the router's and the experts' factors.
bool block_xform(const rvm_block_norms *nm, int flags, XForm *xf) {
    if (!nm || !(nm->eps >= 0.0f) || !std::isfinite(nm->router_post) || (flags & ~RVM_EXACT_SELECT) != 0)
        return false;
    *xf = XForm{1, nm->eps, nm->router_post, nm->router_scale, nm->expert_scale};
    return true;
}

}  // namespace

extern "C" int rvm_moe_block_decode(const rvm_layer *L, const rvm_block_norms *norms, const float *o, float *out,
                                    int flags, void *ws, size_t ws_bytes) {
    XForm xf;
    RVM_CHECK(block_xform(norms, flags, &xf));
    return moe_decode(L, o, out, flags, xf, ws, ws_bytes);
}

extern "C" int rvm_moe_block_forward(const rvm_layer *L, const rvm_block_norms *norms, const float *o, float *out,
                                     int n_tok, int flags, void *ws, size_t ws_bytes) {
    XForm xf;
    RVM_CHECK(block_xform(norms, flags, &xf));
    return moe_forward(L, o, out, n_tok, flags, xf, ws, ws_bytes);
}
