// attention.hip - decode attention over a Q8_0 key/value ring with the reference's operator ABI
// (runtime/hip/rvhip.h:55-67): rvh_kv_store, rvh_attention, rvh_attn_split, rvh_attn_combine.
// The reference's kernels are runtime/hip/rvhip.hip:214-394, its host side runtime/src/hip.rs:423-530.
//
// Semantics (the reference's): query t of a call sits at position pos = p0 + t and attends, with
// scale 1.0, to keys lo .. pos, lo = max(0, pos + 1 - window) when window > 0, else 0. Key p is ring
// slot p % cap: row (slot * n_kv + g) of hd/32 Q8_0 blocks, g = h / (n_head / n_kv). Split-K cuts a
// query's keys into n_chunks contiguous chunks of ceil(len / n_chunks) keys; with more than one
// chunk each (query head, chunk) leaves an unnormalised partial {max, sum, acc[hd]} that
// rvh_attn_combine merges. Results match the CPU ops (runtime/tests/hip_ops.rs:245-271) to the
// reference's relative L2 bound of 1e-5; only summation orders differ.
//
// Work layout. A workgroup of 4 waves takes one tile (token, kv head, chunk) and G query heads that
// share the kv head (G up to the heads per kv head: fewer when the call has few tiles, to spread
// them over more CUs; the head groups of one tile run on one XCD). Keys go in tiles of 64:
//  - loads: wave w reads keys 16 w .. 16 w + 15 of the tile, key and value rows whole and
//    coalesced (lane l the quants of its DPL dimensions); the key quants go through LDS.
//  - scores: MFMA, heads x keys over one Q8_0 block (see k_attn_split); wave w takes the blocks
//    w, w + 4, ... of every key, and the four partial scores meet in LDS.
//  - softmax: wave w keeps its own online softmax over its 16 keys, the maxima and sums running
//    over the 16 lanes of a row.
//  - values: wave w accumulates its 16 keys into every dimension of every head (lane l owns
//    dimensions DPL l .. DPL l + DPL - 1), each key's weight read from the lane that scored it.
//  - merge: the four waves' (max, sum, values) combine in LDS after one barrier.
// Every workgroup is a short serial chain of loads; the grid fits the GPU in one round.
#include "internal.hpp"

namespace rvm {

constexpr int AT_WAVES = 4;
constexpr int AT_TILE = 64;    // keys per tile
constexpr int AT_MAXHD = 512;  // dimensions per head (8 per lane)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int v2i_t __attribute__((ext_vector_type(2)));

struct __attribute__((packed, aligned(2))) Q8Half {  // 8 quants of a Q8_0 block
    uint32_t q[2];
};
struct __attribute__((packed, aligned(2))) Q8Word {
    uint32_t q;
};

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Max over the wave (NaN ignored), the same in every lane.
__device__ __forceinline__ float wave_max_f(float m) {
    m = half_max(m);
    return fmaxf(readlane_f(m, 0), readlane_f(m, 32));
}

__device__ __forceinline__ float q8_at(uint32_t u, int e) { return (float)(int8_t)(uint8_t)(u >> (8 * e)); }

// Max and sum over each row of 16 lanes (xor-pattern exchanges, so that every lane of the row ends
// with the same bits).
__device__ __forceinline__ float row16_max_f(float v) {
    v = maxf_bits(v, dpp<0xb1>(__builtin_bit_cast(uint32_t, v)));
    v = maxf_bits(v, dpp<0x4e>(__builtin_bit_cast(uint32_t, v)));
    v = maxf_bits(v, dpp<0x141>(__builtin_bit_cast(uint32_t, v)));
    return maxf_bits(v, dpp<0x140>(__builtin_bit_cast(uint32_t, v)));
}
__device__ __forceinline__ float row16_sum_f(float v) {
    v += __builtin_bit_cast(float, dpp<0xb1>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp<0x4e>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp<0x141>(__builtin_bit_cast(uint32_t, v)));
    return v + __builtin_bit_cast(float, dpp<0x140>(__builtin_bit_cast(uint32_t, v)));
}

// Four int8 quants as bf16 pairs (exact: |q| <= 128 has at most 8 significant bits): the f32
// value's high half is its bf16.
__device__ __forceinline__ void q8_bf16(uint32_t u, uint32_t &lo, uint32_t &hi) {
    const uint32_t f0 = __builtin_bit_cast(uint32_t, q8_at(u, 0)), f1 = __builtin_bit_cast(uint32_t, q8_at(u, 1));
    const uint32_t f2 = __builtin_bit_cast(uint32_t, q8_at(u, 2)), f3 = __builtin_bit_cast(uint32_t, q8_at(u, 3));
    lo = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    hi = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
}

template <int DPL>
struct AttnTile {              // the wave's 16 keys of a tile, as loaded: row by row, coalesced
    uint32_t kq[16][DPL / 4];  // key rows: the lane's DPL quants (dimensions DPL l ..)
    uint16_t kd[16];           // and their block scale
    uint32_t vq[16][DPL / 4];  // value rows, likewise
    uint16_t vd[16];
};

// G query heads per workgroup; DPL contiguous value dimensions per lane (4 for hd <= 256, 8 for
// hd <= 512): lane l owns dimensions DPL l .. DPL l + DPL - 1, inside one Q8_0 block.
//
// Rows are read whole and coalesced (wave w reads keys 16 w .. 16 w + 15 of a tile, lane l the
// quants of its dimensions); the key quants then go through LDS into the MFMA layout.
//
// Scores run on v_mfma_f32_16x16x32_bf16 with the heads as rows (A = q), the keys as columns
// (B = key quants) and one Q8_0 block as the 32-long reduction: q is held exactly as the sum of
// three bf16 parts (8 + 8 + 8 significant bits), each a separate product accumulated in f32, and
// int8 quants are exact in bf16, so a block's partial is the f32 sum of exact products; the
// lane then scales its own key's partial by the block scale. Wave w takes blocks w, w + 4, ... of
// every key in the tile; lane l of the MFMA output holds heads 4 (l / 16) .. + 3 of key l % 16.
template <int G, int DPL>
__global__ __launch_bounds__(AT_WAVES * 64) void k_attn_split(
    const float *__restrict__ q, const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc,
    float *__restrict__ out, float *__restrict__ part, int n_tok, int n_head, int n_kv, int hd, int p0, int cap,
    int window, int n_chunks) {
    constexpr int NBW = DPL / 2;
    // LDS: partial scores [2][wave][key][head]; the tile's key quants [key][KROW bytes] and block
    // scales [key][16], whose space the waves' value sums [wave][head][dimension][lane] reuse
    constexpr int KROW = 64 * DPL + 16;  // padded: the 16 keys of a fragment read hit distinct banks
    constexpr int KBYTES = AT_TILE * KROW + AT_TILE * 16 * 2;
    constexpr int MBYTES = AT_WAVES * G * DPL * 64 * 4;
    __shared__ float red_lds[2 * AT_WAVES * AT_TILE * G];
    __shared__ __attribute__((aligned(16))) uint8_t kt_lds[KBYTES > MBYTES ? KBYTES : MBYTES];
    uint8_t *const kt_q = kt_lds;
    uint16_t *const kt_d = (uint16_t *)(kt_lds + AT_TILE * KROW);
    const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroup -> (tile, head group): a tile is (token t, kv head g, chunk c); its S head groups
    // get workgroup numbers equal mod 8, so that they run on one XCD and share its L2 for the
    // tile's key and value rows
    const int S = (n_head / n_kv) / G;
    const int xcd = blockIdx.x & 7, rest = blockIdx.x >> 3;
    const int sg = rest % S;
    const long T = (long)(rest / S) * 8 + xcd;
    if (T >= (long)n_tok * n_kv * n_chunks) return;
    const int c = (int)(T % n_chunks);
    const int tg = (int)(T / n_chunks);
    const int g = tg % n_kv, t = tg / n_kv;
    const int h0 = g * (n_head / n_kv) + sg * G;
    const int pos = p0 + t;
    const int lo = window > 0 ? max(0, pos + 1 - window) : 0;
    const int len = pos - lo + 1;
    const int per = (len + n_chunks - 1) / n_chunks;
    const int k0 = lo + c * per, k1 = min(pos + 1, k0 + per);  // this chunk's keys [k0, k1)
    const int nb = hd / QK, row = nb * Q8_BLOCK;
    const size_t slot_bytes = (size_t)n_kv * row;
    const uint8_t *kg = kc + (size_t)g * row, *vg = vc + (size_t)g * row;

    // this lane's value dimensions DPL lane .. + DPL - 1, when below hd (hd is a multiple of 32)
    const bool vok = DPL * lane < hd;
    const int vd0 = vok ? DPL * lane : 0;
    const int vblk = (vd0 / QK) * Q8_BLOCK, vq_off = vblk + 2 + vd0 % QK;

    // ---- every first load at once: the q fragments (q[head lr][block b, elements 8 lg .. + 7]),
    // then the first tile's key and value rows. Loads are unconditional (clamped addresses, the
    // values selected afterwards) so that each wait counts only what it needs.
    float qx[NBW][8];
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
        const int b = w + AT_WAVES * i;
        const bool qok = b < nb && lr < G;
        const float *qr = q + ((size_t)t * n_head + h0 + (qok ? lr : 0)) * hd + (qok ? b : 0) * QK + 8 * lg;
#pragma unroll
        for (int e = 0; e < 8; ++e) qx[i][e] = qr[e];
    }
    AttnTile<DPL> tl;
    const int j0 = 16 * w;  // the wave's keys in the value phase
    // the tile at `base` (ring slot `bslot`; later slots follow by increments, no division per key):
    // the wave's 16 keys, key and value rows; keys past the chunk read the tile's first key
    auto row_offsets = [&](int base, int bslot, size_t *off) {
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            int s = bslot + j0 + jj;
            s = s >= cap ? s - cap : s;
            off[jj] = (size_t)(base + j0 + jj < k1 ? s : bslot) * slot_bytes;
        }
    };
    auto load_keys = [&](int base, int bslot) {
        size_t off[16];
        row_offsets(base, bslot, off);
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            const uint8_t *kr = kg + off[jj];
            tl.kd[jj] = *(const uint16_t *)(kr + vblk);
            if constexpr (DPL == 8) {
                const Q8Half k8 = *(const Q8Half *)(kr + vq_off);
                tl.kq[jj][0] = k8.q[0];
                tl.kq[jj][1] = k8.q[1];
            } else {
                tl.kq[jj][0] = ((const Q8Word *)(kr + vq_off))->q;
            }
        }
    };
    auto load_values = [&](int base, int bslot) {
        size_t off[16];
        row_offsets(base, bslot, off);
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            const uint8_t *vr = vg + off[jj];
            tl.vd[jj] = *(const uint16_t *)(vr + vblk);
            if constexpr (DPL == 8) {
                const Q8Half v8 = *(const Q8Half *)(vr + vq_off);
                tl.vq[jj][0] = v8.q[0];
                tl.vq[jj][1] = v8.q[1];
            } else {
                tl.vq[jj][0] = ((const Q8Word *)(vr + vq_off))->q;
            }
        }
    };
    // order: q and the first keys, then (once q is in) the first values; a wave holds at most 63
    // loads in flight, and the q conversion must not wait behind the value rows
    const int slot0 = k0 % cap;
    load_keys(k0, slot0);  // an empty chunk reads slot0 and uses nothing
    __builtin_amdgcn_sched_barrier(0);

    // ---- q as three bf16 parts (A fragments; heads past G and blocks past hd are zero)
    bf16x8 qa[NBW][3];
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
        const bool qok = w + AT_WAVES * i < nb && lr < G;
        uint32_t pk[3][4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            f32x2 r = {qok ? qx[i][e] : 0.0f, qok ? qx[i][e + 1] : 0.0f};
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                const bf16x2 b = __builtin_convertvector(r, bf16x2);
                pk[k][e / 2] = __builtin_bit_cast(uint32_t, b);
                r -= __builtin_convertvector(b, f32x2);  // exact: the rounding's residual
            }
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            uint4 v = {pk[k][0], pk[k][1], pk[k][2], pk[k][3]};
            qa[i][k] = __builtin_bit_cast(bf16x8, v);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_values(k0, slot0);

    // softmax statistics: each wave keeps its own over its keys; lane (j, r) = (lane % 16,
    // lane / 16) holds heads r HPL .. r HPL + HPL - 1 (rows r < RU)
    constexpr int HPL = G >= 4 ? G / 4 : 1, RU = G >= 4 ? 4 : G;
    float m[HPL], l[HPL], acc[G][DPL];
#pragma unroll
    for (int u = 0; u < HPL; ++u) {
        m[u] = -INFINITY;
        l[u] = 0.0f;
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[h][e] = 0.0f;

    int buf = 0;
    for (int base = k0, bslot = slot0; base < k1;) {
        // ---- the wave's key rows into LDS (dimensions past hd are never read)
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            uint8_t *dst = kt_q + (j0 + jj) * KROW + DPL * lane;
            if constexpr (DPL == 8)
                *(uint2 *)dst = uint2{tl.kq[jj][0], tl.kq[jj][1]};
            else
                *(uint32_t *)dst = tl.kq[jj][0];
            if ((DPL * lane) % QK == 0) kt_d[(j0 + jj) * 16 + DPL * lane / QK] = tl.kd[jj];
        }
        __syncthreads();

        // ---- scores on MFMA: s[kg][r] = head 4 lg + r, key 16 kg + lr, over the wave's blocks
        f32x4 s[4];
#pragma unroll
        for (int kgp = 0; kgp < 4; ++kgp) s[kgp] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < NBW; ++i) {
            const int b = w + AT_WAVES * i;
            if (b >= nb) break;
#pragma unroll
            for (int kgp = 0; kgp < 4; ++kgp) {
                const uint2 kw = *(const uint2 *)(kt_q + (16 * kgp + lr) * KROW + QK * b + 8 * lg);
                uint32_t kb[4];
                q8_bf16(kw.x, kb[0], kb[1]);
                q8_bf16(kw.y, kb[2], kb[3]);
                const bf16x8 bk = __builtin_bit_cast(bf16x8, uint4{kb[0], kb[1], kb[2], kb[3]});
                f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i][0], bk, f32x4{0, 0, 0, 0}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i][1], bk, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i][2], bk, d, 0, 0, 0);
                const float dk = h2f(kt_d[(16 * kgp + lr) * 16 + b]);
#pragma unroll
                for (int r = 0; r < 4; ++r) s[kgp][r] = fmaf(dk, d[r], s[kgp][r]);
            }
        }
        float *red = red_lds + buf * (AT_WAVES * AT_TILE * G);
#pragma unroll
        for (int kgp = 0; kgp < 4; ++kgp)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (4 * lg + r < G) red[(w * AT_TILE + 16 * kgp + lr) * G + 4 * lg + r] = s[kgp][r];
        __syncthreads();

        // ---- online softmax of the wave's keys 16 w .. 16 w + 15: lane (j, r) scores key 16 w + j
        // for its heads; maxima and sums run over the 16 lanes of each row
        const bool live = base + j0 + lr < k1;
        float p[HPL], corr[HPL];
#pragma unroll
        for (int u = 0; u < HPL; ++u) {
            const int h = (lg < RU ? lg : 0) * HPL + u;
            const int kk = j0 + lr;
            const float sc = ((red[kk * G + h] + red[(AT_TILE + kk) * G + h]) + red[(2 * AT_TILE + kk) * G + h]) +
                             red[(3 * AT_TILE + kk) * G + h];
            const float mn = fmaxf(m[u], row16_max_f(live ? sc : -INFINITY));
            corr[u] = m[u] == -INFINITY ? 0.0f : expf(m[u] - mn);
            p[u] = live ? expf(sc - mn) : 0.0f;
            l[u] = l[u] * corr[u] + row16_sum_f(p[u]);
            m[u] = mn;
        }

        // ---- values: the wave's 16 keys; dead keys weigh 0
        if (base + j0 < k1) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float ch = readlane_f(corr[h % HPL], 16 * (h / HPL));
#pragma unroll
                for (int e = 0; e < DPL; ++e) acc[h][e] *= ch;
            }
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                float x[DPL];
                const float d = h2f(tl.vd[jj]);
#pragma unroll
                for (int e = 0; e < DPL; ++e) x[e] = d * q8_at(tl.vq[jj][e / 4], e % 4);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float ph = readlane_f(p[h % HPL], 16 * (h / HPL) + jj);
#pragma unroll
                    for (int e = 0; e < DPL; ++e) acc[h][e] = fmaf(ph, x[e], acc[h][e]);
                }
            }
        }

        // ---- the next tile's rows, when there is one (issued last, so that no wait above counts them)
        const int next = base + AT_TILE;
        int nslot = bslot + AT_TILE;
        while (nslot >= cap) nslot -= cap;
        if (next < k1) {
            load_keys(next, nslot);
            load_values(next, nslot);
        }
        buf ^= 1;
        base = next;
        bslot = nslot;
    }

    // ---- merge the four waves: M = max of their maxima, their sums weighted by e^(m_w - M) and
    // added in wave order; one barrier, then each wave finishes a share of the (head, 4 dimensions)
    // groups. The value sums reuse the key tile's LDS, which the last tile's barrier has released.
    __shared__ float wm[AT_WAVES][G], wl[AT_WAVES][G];
    float *mrg = (float *)kt_lds;  // [wave][head * DPL + e][lane]
    __syncthreads();  // every wave is done with the last key tile
    if (lr == 0 && lg < RU)
#pragma unroll
        for (int u = 0; u < HPL; ++u) {
            wm[w][lg * HPL + u] = m[u];
            wl[w][lg * HPL + u] = l[u];
        }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < DPL; ++e) mrg[((size_t)w * G * DPL + h * DPL + e) * 64 + lane] = acc[h][e];
    __syncthreads();
    const size_t r0 = (size_t)t * n_head + h0;
    constexpr int NQ = G * DPL / 4;  // (head, 4 dimensions) groups
#pragma unroll
    for (int g0 = 0; g0 < NQ; g0 += AT_WAVES) {
        const int gi = g0 + w;
        if (NQ % AT_WAVES != 0 && gi >= NQ) break;
        const int h = gi / (DPL / 4), e0 = 4 * (gi % (DPL / 4));
        const float Mh = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
        float f[AT_WAVES], den = 0.0f;
#pragma unroll
        for (int u = 0; u < AT_WAVES; ++u) {
            f[u] = wm[u][h] == -INFINITY ? 0.0f : expf(wm[u][h] - Mh);
            den = fmaf(f[u], wl[u][h], den);
        }
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float num = 0.0f;
#pragma unroll
            for (int u = 0; u < AT_WAVES; ++u) num = fmaf(f[u], mrg[((size_t)u * G * DPL + h * DPL + e0 + e) * 64 + lane], num);
            v[e] = num;
        }
        if (n_chunks == 1) {
            const float inv = 1.0f / den;
            if (vok)
#pragma unroll
                for (int e = 0; e < 4; ++e) out[(r0 + h) * hd + vd0 + e0 + e] = v[e] * inv;
        } else {
            float *pp = part + ((r0 + h) * n_chunks + c) * (size_t)(hd + 2);
            if (e0 == 0 && lane == 0) {
                pp[0] = Mh;
                pp[1] = den;
            }
            if (vok)
#pragma unroll
                for (int e = 0; e < 4; ++e) pp[2 + vd0 + e0 + e] = v[e];
        }
    }
}

// ---- Streaming split-K for head dimensions 256 and 512 (nb = 8 or 16 Q8_0 blocks per row) ----
// A workgroup of 8 waves takes one tile (token, kv head, chunk) with up to 16 query heads of that kv
// head, so that every key and value row of the tile is read once. The tile's keys go in stages of
// 32, copied from HBM straight into LDS (global_load_lds, 1 KB of two or four whole rows per
// instruction) through a ring of ST_RING stages: ST_RING - 1 stages are in flight while one is
// computed, and each wave waits (vmcnt) only for the copies of the stage it needs next. A stage
// sits in LDS as [K/V][key][16-byte piece p ^ key] (piece p holds half of block p / 2's quants, read
// from the ring rows at 2-byte alignment; the XOR puts the same piece of 16 keys on distinct banks)
// and the block scales as the dwords that start at them (low half), [K/V][key][block].
//  - scores: v_mfma_f32_16x16x32_bf16, heads x 16 keys over one block (q as three exact bf16 parts,
//    the key quants exact in bf16), scaled by the key's block scale; wave w takes key group w & 1
//    and a quarter of the blocks, and the four partial scores meet in LDS;
//  - softmax: wave w keeps heads 2 w and 2 w + 1 (lane = head parity, key): their running max and
//    sum, and writes the stage's p and the rescale factor to LDS;
//  - values: v_mfma_f32_16x16x32_bf16 with A = p * d_v (heads x 32 keys, three exact bf16 parts)
//    and B = the value quants of 32 keys x 16 dimensions, read transposed out of LDS
//    (ds_read_b64_tr_b8: each 16-lane group turns 8 keys x 8 bytes into 8 dimensions x 8 keys);
//    wave w owns the dimensions of blocks w, w + 8, so no merge is needed.
constexpr int ST_WAVES = 8;
constexpr int ST_KEYS = 32;  // keys per stage
constexpr int ST_RING = 4;   // stages resident in LDS
constexpr int ST_PP = 36;    // row pitch of the p rows in LDS (floats)

template <int NB>
struct StreamShape {
    static constexpr int HD = 32 * NB;
    static constexpr int ROW = NB * Q8_BLOCK;
    static constexpr int QBYTES = 2 * ST_KEYS * HD;      // quants of a stage, K then V
    static constexpr int SBYTES = 2 * NB * ST_KEYS * 4;  // scale dwords of a stage
    static constexpr int STAGE = QBYTES + SBYTES;
    static constexpr int NQ = NB / 4;  // 16-byte copies per wave and stage
    static constexpr int NS = NB / 8;  // 4-byte copies per wave and stage
    static constexpr int NI = NQ + NS;
    static constexpr int SBW = NB / 4;  // blocks per wave in the scores
    static constexpr int VBW = NB / 8;  // blocks per wave in the values
    static constexpr int LDS = ST_RING * STAGE + (4 * 16 * ST_KEYS + 16 * ST_PP + 2 * 16) * 4;
    static_assert(LDS <= 163840, "LDS");
};

typedef __attribute__((address_space(3))) v2i_t lds_v2i_t;


__device__ __forceinline__ bf16x8 q8x8_bf16(uint32_t a, uint32_t b) {
    uint32_t k[4];
    q8_bf16(a, k[0], k[1]);
    q8_bf16(b, k[2], k[3]);
    return __builtin_bit_cast(bf16x8, uint4{k[0], k[1], k[2], k[3]});
}

// x as three bf16 parts whose sum is x exactly (each part the rounding of the residual before it)
__device__ __forceinline__ void split3_bf16(const float (&x)[8], bf16x8 (&a)[3]) {
    uint32_t pk[3][4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        f32x2 r = {x[e], x[e + 1]};
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const bf16x2 b = __builtin_convertvector(r, bf16x2);
            pk[k][e / 2] = __builtin_bit_cast(uint32_t, b);
            r -= __builtin_convertvector(b, f32x2);
        }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) a[k] = __builtin_bit_cast(bf16x8, uint4{pk[k][0], pk[k][1], pk[k][2], pk[k][3]});
}

// e^d for d <= 0 as 2^(d log2 e) on the hardware exp2 (0 for d = -inf)
__device__ __forceinline__ float exp_le0(float d) { return __builtin_amdgcn_exp2f(d * 1.44269504088896341f); }

// max and sum over the 32 lanes of a half-wave: the 16-lane DPP exchanges, then the other row's
// result through a swizzle (every lane ends with the same bits)
__device__ __forceinline__ float half32_max(float v) {
    v = row16_max_f(v);
    return maxf_bits(v, swz_xor16(__builtin_bit_cast(uint32_t, v)));
}
__device__ __forceinline__ float half32_sum(float v) {
    v = row16_sum_f(v);
    return v + __builtin_bit_cast(float, swz_xor16(__builtin_bit_cast(uint32_t, v)));
}

//
// With kin / vin set (one decode token, n_tok = 1) the kernel also stores that token's key and value
// rows: the workgroups whose chunk holds position p0 quantise them (bit for bit k_kv_store's Q8_0),
// head group 0 writes them to ring slot p0 % cap, and each writes them over the stale slot's copy
// in its LDS stage before computing it (the value scales of the stage's later keys, copies of that
// slot, are set to 0: those keys weigh 0).
template <int NB>
__global__ __launch_bounds__(ST_WAVES * 64) void k_attn_stream(
    const float *__restrict__ q, uint8_t *__restrict__ kc, uint8_t *__restrict__ vc, float *__restrict__ out,
    float *__restrict__ part, int n_tok, int n_head, int n_kv, int G, int p0, int cap, int window, int n_chunks,
    const float *__restrict__ kin, const float *__restrict__ vin) {
    using Sh = StreamShape<NB>;
    constexpr int HD = Sh::HD, SBW = Sh::SBW, VBW = Sh::VBW, PMASK = 2 * NB - 1;
    __shared__ __attribute__((aligned(16))) uint8_t ring[ST_RING * Sh::STAGE];
    __shared__ __attribute__((aligned(16))) float red[4 * 16 * ST_KEYS];  // [block quarter][head][key]
    __shared__ __attribute__((aligned(16))) float pl[16 * ST_PP];          // [head][key]: the stage's p
    __shared__ __attribute__((aligned(16))) float hcorr[16], hsum[16];
    const int lane = threadIdx.x & 63, lr = lane & 15, jg = lane >> 4, lk = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroup -> (tile, head group) as in k_attn_split
    const int S = (n_head / n_kv) / G;
    const int xcd = blockIdx.x & 7, rest = blockIdx.x >> 3;
    const int sg = rest % S;
    const long T = (long)(rest / S) * 8 + xcd;
    if (T >= (long)n_tok * n_kv * n_chunks) return;
    const int c = (int)(T % n_chunks);
    const int tg = (int)(T / n_chunks);
    const int g = tg % n_kv, t = tg / n_kv;
    const int h0 = g * (n_head / n_kv) + sg * G;
    const int pos = p0 + t;
    const int lo = window > 0 ? max(0, pos + 1 - window) : 0;
    const int len = pos - lo + 1;
    const int per = (len + n_chunks - 1) / n_chunks;
    const int k0 = lo + c * per, k1 = min(pos + 1, k0 + per);
    const int nkeys = max(0, k1 - k0), nst = (nkeys + ST_KEYS - 1) / ST_KEYS;
    const size_t slot_bytes = (size_t)n_kv * Sh::ROW;
    const int slot0 = k0 % cap;
    const uint8_t *kg = kc + (size_t)g * Sh::ROW, *vg = vc + (size_t)g * Sh::ROW;

    // the copies of stage s into its ring slot. Every wave issues exactly NI copy instructions per
    // stage, stages past the tile included (those repeat one row, which stays in the caches), so that
    // the waits count stages; keys past the tile repeat its last key. Copy i of this lane: the key,
    // K or V, and the byte offset in the row are the same in every stage.
    int ckey[Sh::NI];
    const uint8_t *crow[Sh::NI];  // row base of the key's slot in stage 0, K or V
    uint32_t coff[Sh::NI];
#pragma unroll
    for (int i = 0; i < Sh::NQ; ++i) {
        const int P = (w * Sh::NQ + i) * 64 + lane;  // 16-byte slot of the stage: [K/V][key][slot]
        const int key = (P / (2 * NB)) % ST_KEYS, j = (P & PMASK) ^ (key & PMASK);  // the piece it holds
        ckey[i] = key;
        crow[i] = P / (64 * NB) ? vg : kg;
        coff[i] = Q8_BLOCK * (j >> 1) + 2 + 16 * (j & 1);
    }
#pragma unroll
    for (int i = 0; i < Sh::NS; ++i) {
        const int P = (w * Sh::NS + i) * 64 + lane;  // scale dword of the stage: [K/V][key][block]
        ckey[Sh::NQ + i] = (P / NB) % ST_KEYS;
        crow[Sh::NQ + i] = P / (32 * NB) ? vg : kg;
        coff[Sh::NQ + i] = Q8_BLOCK * (P % NB);  // the dword starting at the block's scale
    }
    const uint32_t ring0 = lds_addr(ring);
    auto issue = [&](int s) {
        const uint32_t base = ring0 + (s % ST_RING) * Sh::STAGE;
        const int kb = s * ST_KEYS;
        const uint8_t *src[Sh::NI];
        if (kb + ST_KEYS <= nkeys && slot0 + kb + ST_KEYS <= cap) {  // whole stage, no wrap
            const size_t adv = (size_t)(slot0 + kb) * slot_bytes;
#pragma unroll
            for (int i = 0; i < Sh::NI; ++i) src[i] = crow[i] + adv + ((size_t)ckey[i] * slot_bytes + coff[i]);
        } else {
            const bool real = s < nst;
            const int last = real ? min(ST_KEYS, nkeys - kb) - 1 : 0;
#pragma unroll
            for (int i = 0; i < Sh::NI; ++i) {
                int sl = slot0 + (real ? kb + min(ckey[i], last) : 0);
                sl = sl >= cap ? sl - cap : sl;
                src[i] = crow[i] + (size_t)sl * slot_bytes + coff[i];
            }
        }
#pragma unroll
        for (int i = 0; i < Sh::NQ; ++i) lds_copy16(src[i], base + (w * Sh::NQ + i) * 1024);
#pragma unroll
        for (int i = 0; i < Sh::NS; ++i)
            lds_copy4(src[Sh::NQ + i], base + Sh::QBYTES + (w * Sh::NS + i) * 256);
    };

    // the new token's key and value (fused store): half-wave (w, lane / 32) quantises blocks
    // 16 i + 2 w + lane / 32 of [K blocks, V blocks], element lane % 32
    constexpr int NPASS = NB / 8;
    const bool fuse = kin != nullptr && k0 <= pos && pos < k1;
    float fx[NPASS];
    if (fuse) {
#pragma unroll
        for (int i = 0; i < NPASS; ++i) {
            const int B = 16 * i + 2 * w + (lane >> 5);
            fx[i] = (B < NB ? kin : vin)[(size_t)g * HD + QK * (B % NB) + lk];
        }
    }

    // the queries and stage 0 first: 16 rows of HD floats (heads past G repeat head h0) into the last
    // ring slot, which the first stages leave free; stages 1 and 2 once those have landed, so that the
    // first stage of every workgroup is not queued behind the next ones
    {
        const uint32_t qbase = ring0 + (ST_RING - 1) * Sh::STAGE;
        const float *qrow = q + ((size_t)t * n_head + h0) * HD;
#pragma unroll
        for (int i = 0; i < Sh::NQ; ++i) {
            const int P = (w * Sh::NQ + i) * 64 + lane;  // 16-byte piece of the 16 x HD floats
            const int hh = P / (HD / 4), e = P % (HD / 4);
            lds_copy16(qrow + (size_t)(hh < G ? hh : 0) * HD + 4 * e, qbase + (w * Sh::NQ + i) * 1024);
        }
    }
    issue(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __syncthreads();
#pragma unroll
    for (int s = 1; s < ST_RING - 1; ++s) issue(s);
    // the fused token's row (its stores come after the copies of stages 1 and 2; the waits below
    // count loads, which complete in order, so a store still in flight only delays them)
    int fq[NPASS];
    uint16_t fd[NPASS];
    if (fuse) {
        uint8_t *slotp = nullptr;
        const int sp = p0 % cap;
#pragma unroll
        for (int i = 0; i < NPASS; ++i) {
            const int B = 16 * i + 2 * w + (lane >> 5);
            fq[i] = quant_q8_half(fx[i], &fd[i]);
            if (sg == 0) {  // the ring row, as k_kv_store writes it
                slotp = (B < NB ? kc : vc) + ((size_t)sp * n_kv + g) * Sh::ROW + Q8_BLOCK * (B % NB);
                slotp[2 + lk] = (uint8_t)(int8_t)fq[i];
                if (lk == 0) {
                    slotp[0] = (uint8_t)(fd[i] & 0xff);
                    slotp[1] = (uint8_t)(fd[i] >> 8);
                }
            }
        }
    }

    // the scores' share of this wave: key group kq, blocks SBW bq .. SBW bq + SBW - 1; q fragments
    // (A: head lr, elements 8 jg .. + 7 of each block) as three bf16 parts
    const int kq = w & 1, bq = w >> 1;
    bf16x8 qa[SBW][3];
    {
        const float *qs = (const float *)(ring + (ST_RING - 1) * Sh::STAGE);
#pragma unroll
        for (int i = 0; i < SBW; ++i) {
            const int b = SBW * bq + i;
            const bool qok = lr < G;
            const float4 *qr = (const float4 *)(qs + lr * HD + b * QK + 8 * jg);
            const float4 x0 = qr[0], x1 = qr[1];
            const float x[8] = {qok ? x0.x : 0.0f, qok ? x0.y : 0.0f, qok ? x0.z : 0.0f, qok ? x0.w : 0.0f,
                                qok ? x1.x : 0.0f, qok ? x1.y : 0.0f, qok ? x1.z : 0.0f, qok ? x1.w : 0.0f};
            split3_bf16(x, qa[i]);
        }
    }

    // the softmax of heads hw = 2 w + lane / 32, key lk: running max and sum
    const int hw = 2 * w + (lane >> 5);
    float m = -INFINITY, lsum = 0.0f;
    f32x4 acc[VBW][2];
#pragma unroll
    for (int i = 0; i < VBW; ++i) acc[i][0] = acc[i][1] = f32x4{0, 0, 0, 0};

    for (int s = 0; s < nst; ++s) {
        if (s > 0) {  // stage s + 1 stays in flight; stage 0 was waited for with the queries
            __builtin_amdgcn_s_waitcnt(vmcnt_only((ST_RING - 3) * Sh::NI));
            __syncthreads();  // the stage is in LDS for every wave; the slot of stage s - 2 is free
            issue(s + ST_RING - 2);
        }
        const uint8_t *sb = ring + (s % ST_RING) * Sh::STAGE;
        const uint32_t *scl = (const uint32_t *)(sb + Sh::QBYTES);
        const int nk = min(ST_KEYS, nkeys - s * ST_KEYS);
        if (fuse && s == (pos - k0) / ST_KEYS) {  // the stage holding the new token: its row into LDS
            uint8_t *st = ring + (s % ST_RING) * Sh::STAGE;
            uint32_t *stsc = (uint32_t *)(st + Sh::QBYTES);
            const int kp = (pos - k0) % ST_KEYS;
#pragma unroll
            for (int i = 0; i < NPASS; ++i) {
                const int B = 16 * i + 2 * w + (lane >> 5), which = B / NB, b = B % NB;
                const int slot = (2 * b + (lk >> 4)) ^ (kp & PMASK);
                st[((which * ST_KEYS + kp) * 2 * NB + slot) * 16 + (lk & 15)] = (uint8_t)(int8_t)fq[i];
                if (lk == 0) stsc[(which * ST_KEYS + kp) * NB + b] = fd[i];
            }
            // the later keys of the stage repeat the stale slot: a value scale of 0 keeps them finite
            const int dk = kp + 1 + (int)threadIdx.x / NB, db = (int)threadIdx.x % NB;
            if (dk < ST_KEYS) stsc[(ST_KEYS + dk) * NB + db] = 0u;
            __syncthreads();
        }

        // ---- scores: heads x keys 16 kq .. 16 kq + 15 over this wave's blocks
        if (kq == 0 || nk > 16) {
            const int kl = 16 * kq + lr;
            f32x4 s4 = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < SBW; ++i) {
                const int b = SBW * bq + i;
                const int slot = (2 * b + (jg >> 1)) ^ (kl & PMASK);
                const uint2 kw = *(const uint2 *)(sb + (kl * 2 * NB + slot) * 16 + 8 * (jg & 1));
                const bf16x8 bk = q8x8_bf16(kw.x, kw.y);
                f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i][0], bk, f32x4{0, 0, 0, 0}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i][1], bk, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i][2], bk, d, 0, 0, 0);
                const float dk = h2f((uint16_t)scl[kl * NB + b]);
#pragma unroll
                for (int r = 0; r < 4; ++r) s4[r] = fmaf(dk, d[r], s4[r]);
            }
            float *rw = red + bq * 16 * ST_KEYS;
#pragma unroll
            for (int r = 0; r < 4; ++r) rw[(4 * jg + r) * ST_KEYS + kl] = s4[r];
        }
        __syncthreads();

        // ---- online softmax of heads 2 w, 2 w + 1 over the stage's keys (one key per lane)
        {
            const int hh = hw < 16 ? hw : 0;
            float sv = ((red[hh * ST_KEYS + lk] + red[(16 + hh) * ST_KEYS + lk]) + red[(32 + hh) * ST_KEYS + lk]) +
                       red[(48 + hh) * ST_KEYS + lk];
            sv = lk < nk ? sv : -INFINITY;
            const float mn = fmaxf(m, half32_max(sv));
            const float corr = exp_le0(m - mn);  // 0 while m = -inf
            const float p = exp_le0(sv - mn);    // 0 for keys past the stage
            lsum = lsum * corr + half32_sum(p);
            m = mn;
            if (hw < 16) {
                pl[hw * ST_PP + lk] = hw < G ? p : 0.0f;
                if (lk == 0) hcorr[hw] = corr;
            }
        }
        __syncthreads();

        // ---- values: heads x the 32 dimensions of each of the wave's blocks
        {
            const float4 *pr = (const float4 *)(pl + lr * ST_PP + 8 * jg);
            const float4 pa = pr[0], pb = pr[1];
            const float p[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
            const float4 cr = *(const float4 *)(hcorr + 4 * jg);  // rows 4 jg .. 4 jg + 3 of the MFMA output
#pragma unroll
            for (int i = 0; i < VBW; ++i)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    acc[i][tt][0] *= cr.x;
                    acc[i][tt][1] *= cr.y;
                    acc[i][tt][2] *= cr.z;
                    acc[i][tt][3] *= cr.w;
                }
#pragma unroll
            for (int i = 0; i < VBW; ++i) {
                const int b = w + ST_WAVES * i;
                float x[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    x[e] = p[e] * h2f((uint16_t)scl[(ST_KEYS + 8 * jg + e) * NB + b]);
                bf16x8 a[3];
                split3_bf16(x, a);
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    // source row of this lane: key 8 jg + lr / 2, dimensions 32 b + 16 tt + 8 (lr & 1) .. + 7
                    const int kl = 8 * jg + (lr >> 1);
                    const int slot = (2 * b + tt) ^ (kl & PMASK);
                    const uint8_t *src = sb + ((ST_KEYS + kl) * 2 * NB + slot) * 16 + 8 * (lr & 1);
                    const v2i_t vt = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t *)src);
                    const bf16x8 bv = q8x8_bf16((uint32_t)vt.x, (uint32_t)vt.y);
                    acc[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], bv, acc[i][tt], 0, 0, 0);
                    acc[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], bv, acc[i][tt], 0, 0, 0);
                    acc[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], bv, acc[i][tt], 0, 0, 0);
                }
            }
        }
    }

    // the copies past the last stage land in LDS: none may be in flight when the workgroup ends
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));

    // ---- results: lane (lr, jg) holds heads 4 jg + r, dimension 32 b + 16 tt + lr of each block
    const size_t r0 = (size_t)t * n_head + h0;
    if (hw < 16 && lk == 0) hsum[hw] = lsum;
    __syncthreads();
    if (n_chunks == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * jg + r;
            const float inv = 1.0f / hsum[h];
            if (h < G)
#pragma unroll
                for (int i = 0; i < VBW; ++i)
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt)
                        out[(r0 + h) * HD + 32 * (w + ST_WAVES * i) + 16 * tt + lr] = acc[i][tt][r] * inv;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * jg + r;
            if (h < G) {
                float *pp = part + ((r0 + h) * n_chunks + c) * (size_t)(HD + 2);
#pragma unroll
                for (int i = 0; i < VBW; ++i)
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) pp[2 + 32 * (w + ST_WAVES * i) + 16 * tt + lr] = acc[i][tt][r];
            }
        }
        if (hw < G && lk == 0) {
            float *pp = part + ((r0 + hw) * n_chunks + c) * (size_t)(HD + 2);
            pp[0] = m;
            pp[1] = lsum;
        }
    }
}

// out[i][d] = sum_c e^(m_c - M) acc_c[d] / sum_c e^(m_c - M) l_c with M = max_c m_c; an empty chunk
// (m = -inf, l = 0) adds nothing (the reference's merge, runtime/hip/rvhip.hip:376-394).
// Workgroup (row, 64 dimensions), lane = dimension: wave w folds chunks w, w + 4, ... in one pass
// with a running maximum (rescaling what it holds when the maximum grows), eight chunks per load
// batch with the next batch in flight; the four waves' (max, sum, acc) then merge in a fixed order.
constexpr int CB_B = 8;  // chunks per load batch and wave
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part, float *__restrict__ out,
                                                      int hd, int n_chunks) {
    __shared__ float wm[AT_WAVES], wl[AT_WAVES], wo[AT_WAVES][64];
    const int i = blockIdx.x, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int d = blockIdx.y * 64 + lane;
    const int dd = d < hd ? d : 0;
    const size_t stride = (size_t)hd + 2;
    const float *pp = part + (size_t)i * n_chunks * stride;
    const int nw = n_chunks > w ? (n_chunks - w + AT_WAVES - 1) / AT_WAVES : 0;  // this wave's chunks
    // clamped, always valid: past the wave's chunks its first one, or the row's last one if it has none
    auto chunk = [&](int j) { return j < nw ? w + AT_WAVES * j : min(w, n_chunks - 1); };
    // batch j: lane k < CB_B loads (m, l) of the wave's chunk j + k; every lane loads its dimension
    // of each of the CB_B chunks
    const int kl = lane < CB_B ? lane : 0;
    float a[CB_B], ml, ll;
    {
        const float *pc = pp + (size_t)chunk(kl) * stride;
        ml = pc[0];
        ll = pc[1];
#pragma unroll
        for (int k = 0; k < CB_B; ++k) a[k] = pp[(size_t)chunk(k) * stride + 2 + dd];
    }
    float M = -INFINITY, den = 0.0f, o = 0.0f;
    for (int j = 0; j < nw; j += CB_B) {
        float an[CB_B], mln, lln;
        {
            const float *pc = pp + (size_t)chunk(j + CB_B + kl) * stride;
            mln = pc[0];
            lln = pc[1];
#pragma unroll
            for (int k = 0; k < CB_B; ++k) an[k] = pp[(size_t)chunk(j + CB_B + k) * stride + 2 + dd];
        }
        float mc[CB_B], lc[CB_B];
        float bm = -INFINITY;
#pragma unroll
        for (int k = 0; k < CB_B; ++k) {
            mc[k] = readlane_f(ml, k);
            lc[k] = readlane_f(ll, k);
            if (j + k < nw) bm = fmaxf(bm, mc[k]);
        }
        const float Mn = fmaxf(M, bm);
        if (Mn != -INFINITY) {
            const float sc = M == -INFINITY ? 0.0f : expf(M - Mn);
            o *= sc;
            den *= sc;
#pragma unroll
            for (int k = 0; k < CB_B; ++k) {
                const float e = (j + k < nw && mc[k] != -INFINITY) ? expf(mc[k] - Mn) : 0.0f;
                o = fmaf(e, a[k], o);
                den = fmaf(e, lc[k], den);
            }
            M = Mn;
        }
#pragma unroll
        for (int k = 0; k < CB_B; ++k) a[k] = an[k];
        ml = mln;
        ll = lln;
    }
    if (lane == 0) {
        wm[w] = M;
        wl[w] = den;
    }
    wo[w][lane] = o;
    __syncthreads();
    if (w != 0 || d >= hd) return;
    const float Mx = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    float num = 0.0f, dsum = 0.0f;
#pragma unroll
    for (int u = 0; u < AT_WAVES; ++u) {
        const float e = wm[u] == -INFINITY ? 0.0f : expf(wm[u] - Mx);
        num = fmaf(e, wo[u][lane], num);
        dsum = fmaf(e, wl[u], dsum);
    }
    out[(size_t)i * hd + d] = num * (1.0f / dsum);
}

// The same merge for up to NW * CW chunks in one round of loads: wave w takes chunks w, w + NW, ..
// (at most CW), every value and lane k's (max, sum) of its k-th chunk loaded at once; the wave's
// maximum M_w, then o_w = sum_k e^(m_k - M_w) acc_k and l_w likewise in chunk order, and the NW
// waves' (M, l, o) merge in wave order as in k_attn_combine. Four waves of 32 chunks take up to
// 128 chunks, eight of 40 up to 320 (a global layer split into chunks of 64 keys at depth 16384).
template <int NW, int CW>
__global__ __launch_bounds__(NW * 64) void k_attn_merge(const float *__restrict__ part, float *__restrict__ out, int hd,
                                                        int n_chunks) {
    static_assert(CW <= 64, "one chunk's (max, sum) per lane");
    __shared__ float wm[NW], wl[NW], wo[NW][64];
    const int i = blockIdx.x, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int d = blockIdx.y * 64 + lane;
    const int dd = d < hd ? d : 0;
    const size_t stride = (size_t)hd + 2;
    const float *pp = part + (size_t)i * n_chunks * stride;
    const int nw = n_chunks > w ? (n_chunks - w + NW - 1) / NW : 0;  // this wave's chunks
    // clamped, always valid: past the wave's chunks its first one, or the row's last one if it has none
    auto chunk = [&](int k) { return k < nw ? w + NW * k : min(w, n_chunks - 1); };
    float a[CW];
#pragma unroll
    for (int k = 0; k < CW; ++k) a[k] = pp[(size_t)chunk(k) * stride + 2 + dd];
    const int kl = lane < CW ? lane : 0;
    const float ml = pp[(size_t)chunk(kl) * stride], ll = pp[(size_t)chunk(kl) * stride + 1];
    const float mk = lane < nw ? ml : -INFINITY;
    float M = mk;
#pragma unroll
    for (int k = 0; k < CW; ++k) M = fmaxf(M, readlane_f(mk, k));
    const float e = mk == -INFINITY ? 0.0f : expf(mk - M);  // 0 past the wave's chunks and for empty ones
    float o = 0.0f, den = 0.0f;
#pragma unroll
    for (int k = 0; k < CW; ++k) {
        const float ek = readlane_f(e, k);
        o = fmaf(ek, a[k], o);
        den = fmaf(ek, readlane_f(ll, k), den);
    }
    if (lane == 0) {
        wm[w] = M;
        wl[w] = den;
    }
    wo[w][lane] = o;
    __syncthreads();
    if (w != 0 || d >= hd) return;
    float Mx = wm[0];
#pragma unroll
    for (int u = 1; u < NW; ++u) Mx = fmaxf(Mx, wm[u]);
    float num = 0.0f, dsum = 0.0f;
#pragma unroll
    for (int u = 0; u < NW; ++u) {
        const float eu = wm[u] == -INFINITY ? 0.0f : expf(wm[u] - Mx);
        num = fmaf(eu, wo[u][lane], num);
        dsum = fmaf(eu, wl[u], dsum);
    }
    out[(size_t)i * hd + d] = num * (1.0f / dsum);
}

// Q8_0 of the keys and values of tokens p0 .. p0 + n_tok - 1 into ring slots p % cap, bit for bit
// the CPU quantiser (runtime/src/ops.rs:95-105; the reference kernel is rvhip.hip:214-239): one
// 32-value block per half-wave, workgroup (token, kv head).
__global__ __launch_bounds__(256) void k_kv_store(const float *__restrict__ k, const float *__restrict__ v,
                                                  uint8_t *__restrict__ kc, uint8_t *__restrict__ vc, int n_kv,
                                                  int hd, int p0, int cap) {
    const int t = blockIdx.x / n_kv, h = blockIdx.x - t * n_kv;
    const int nb = hd / QK, row = nb * Q8_BLOCK;
    const size_t slot = (size_t)((p0 + t) % cap);
    const int half = threadIdx.x >> 5, j = threadIdx.x & 31;
    for (int which = 0; which < 2; ++which) {
        const float *src = (which ? v : k) + ((size_t)t * n_kv + h) * hd;
        uint8_t *dst = (which ? vc : kc) + (slot * n_kv + h) * row;
        for (int b0 = 0; b0 < nb; b0 += 8) {
            const int b = b0 + half;
            const bool ok = b < nb;
            uint16_t dbits;
            const int qv = quant_q8_half(ok ? src[b * QK + j] : 0.0f, &dbits);
            if (ok) {
                dst[b * Q8_BLOCK + 2 + j] = (uint8_t)(int8_t)qv;
                if (j == 0) {
                    dst[b * Q8_BLOCK] = (uint8_t)(dbits & 0xff);
                    dst[b * Q8_BLOCK + 1] = (uint8_t)(dbits >> 8);
                }
            }
        }
    }
}

// The longest key range of a call (the last query's): it must fit the ring.
inline long attn_longest(int n_tok, int p0, int window) {
    const long last = (long)p0 + n_tok;
    return window > 0 && window < last ? (long)window : last;
}

// Heads per workgroup: the largest of 16, 8, 4, 2, 1 (8 for hd > 256) that divides the query heads
// of a kv head, halved while the smaller group's grid still fits the GPU in one round (workgroups
// resident per CU, from the runtime's occupancy for that kernel, times the CUs). Decode at depth
// has few tiles: a smaller head group spreads each tile's work over more CUs, which re-read its
// key and value rows from their XCD's L2; more workgroups than fit at once would only queue, as
// each is a serial chain of loads, scores, values and a merge.
template <int G, int DPL>
void launch_g(long wgs, const float *q, const uint8_t *kc, const uint8_t *vc, float *out, float *part, int n_tok,
              int n_head, int n_kv, int hd, int p0, int cap, int window, int n_chunks) {
    hipLaunchKernelGGL((k_attn_split<G, DPL>), dim3((unsigned)wgs), dim3(AT_WAVES * 64), 0, cur_stream(), q, kc, vc,
                       out, part, n_tok, n_head, n_kv, hd, p0, cap, window, n_chunks);
}

template <int G, int DPL>
long resident_wgs() {  // per GPU, for this kernel; cached per device
    static long cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_attn_split<G, DPL>, AT_WAVES * 64, 0) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 ||
            cus < 1)
            return 256;
        cache[dev] = (long)per_cu * cus;
    }
    return cache[dev];
}

template <int DPL>
long resident_for(int gt) {
    switch (gt) {
        case 16: return DPL == 4 ? resident_wgs<16, 4>() : 0;
        case 8: return resident_wgs<8, DPL>();
        case 4: return resident_wgs<4, DPL>();
        case 2: return resident_wgs<2, DPL>();
        default: return resident_wgs<1, DPL>();
    }
}

inline long attn_wgs(int n_tok, int n_head, int n_kv, int n_chunks, int gt) {
    const long tiles = (long)n_tok * n_kv * n_chunks;
    return (tiles + 7) / 8 * 8 * ((n_head / n_kv) / gt);  // see the workgroup mapping
}

template <int DPL>
int attn_group(int n_tok, int n_head, int n_kv, int n_chunks) {
    const int per_kv = n_head / n_kv;
    int gt = 1;
    for (int c = DPL == 8 ? 8 : 16; c > 1; c >>= 1)
        if (per_kv % c == 0) {
            gt = c;
            break;
        }
    while (gt > 1 && attn_wgs(n_tok, n_head, n_kv, n_chunks, gt / 2) <= resident_for<DPL>(gt / 2)) gt >>= 1;
    return gt;
}

// The streaming kernel's head group: every query head of a kv head, or groups of 16 when there are
// more (0 when it does not apply: another head dimension, or a count of heads 16 does not divide).
inline int stream_group(int n_head, int n_kv, int hd) {
    if (hd != 256 && hd != 512) return 0;
    const int per_kv = n_head / n_kv;
    return per_kv <= 16 ? per_kv : (per_kv % 16 == 0 ? 16 : 0);
}

int launch_stream(const float *q, const void *kc, const void *vc, float *out, float *part, int n_tok, int n_head,
                  int n_kv, int hd, int p0, int cap, int window, int n_chunks, int G, const float *kin,
                  const float *vin) {
    const long wgs = attn_wgs(n_tok, n_head, n_kv, n_chunks, G);
    RVM_CHECK(wgs <= 0x7fffffffL);
    // the rings are written only with kin / vin set (rvm_attn_decode, whose rings are writable)
    uint8_t *k8 = (uint8_t *)kc, *v8 = (uint8_t *)vc;
    if (hd == 512)
        hipLaunchKernelGGL(k_attn_stream<16>, dim3((unsigned)wgs), dim3(ST_WAVES * 64), 0, cur_stream(), q, k8, v8, out,
                           part, n_tok, n_head, n_kv, G, p0, cap, window, n_chunks, kin, vin);
    else
        hipLaunchKernelGGL(k_attn_stream<8>, dim3((unsigned)wgs), dim3(ST_WAVES * 64), 0, cur_stream(), q, k8, v8, out,
                           part, n_tok, n_head, n_kv, G, p0, cap, window, n_chunks, kin, vin);
    return launched();
}

int launch_attn(const float *q, const void *kc, const void *vc, float *out, float *part, int n_tok, int n_head,
                int n_kv, int hd, int p0, int cap, int window, int n_chunks) {
    if (const int G = stream_group(n_head, n_kv, hd))
        return launch_stream(q, kc, vc, out, part, n_tok, n_head, n_kv, hd, p0, cap, window, n_chunks, G, nullptr,
                             nullptr);
    // heads per workgroup times dimensions per lane at most 64: the merge buffer's LDS
    const bool wide = hd > 256;
    const int gt = wide ? attn_group<8>(n_tok, n_head, n_kv, n_chunks) : attn_group<4>(n_tok, n_head, n_kv, n_chunks);
    const long wgs = attn_wgs(n_tok, n_head, n_kv, n_chunks, gt);
    RVM_CHECK(wgs <= 0x7fffffffL);
    const uint8_t *k8 = (const uint8_t *)kc, *v8 = (const uint8_t *)vc;
#define RVM_ATTN_ARGS wgs, q, k8, v8, out, part, n_tok, n_head, n_kv, hd, p0, cap, window, n_chunks
    if (wide) {
        switch (gt) {
            case 8: launch_g<8, 8>(RVM_ATTN_ARGS); break;
            case 4: launch_g<4, 8>(RVM_ATTN_ARGS); break;
            case 2: launch_g<2, 8>(RVM_ATTN_ARGS); break;
            default: launch_g<1, 8>(RVM_ATTN_ARGS); break;
        }
    } else {
        switch (gt) {
            case 16: launch_g<16, 4>(RVM_ATTN_ARGS); break;
            case 8: launch_g<8, 4>(RVM_ATTN_ARGS); break;
            case 4: launch_g<4, 4>(RVM_ATTN_ARGS); break;
            case 2: launch_g<2, 4>(RVM_ATTN_ARGS); break;
            default: launch_g<1, 4>(RVM_ATTN_ARGS); break;
        }
    }
#undef RVM_ATTN_ARGS
    return launched();
}

}  // namespace rvm

using namespace rvm;

extern "C" {

int rvh_kv_store(const float *k, const float *v, void *kc, void *vc, int n_tok, int n_kv, int hd, int p0, int cap) {
    RVM_CHECK(k && v && kc && vc && n_tok > 0 && n_kv > 0 && hd > 0 && hd % QK == 0 && p0 >= 0 && cap > 0);
    RVM_CHECK((long)n_tok * n_kv <= 0x7fffffffL);
    hipLaunchKernelGGL(k_kv_store, dim3(n_tok * n_kv), dim3(256), 0, cur_stream(), k, v, (uint8_t *)kc, (uint8_t *)vc,
                       n_kv, hd, p0, cap);
    return launched();
}

int rvh_attn_split(const float *q, const void *kc, const void *vc, float *out, float *part, int n_tok, int n_head,
                   int n_kv, int hd, int p0, int cap, int window, int n_chunks) {
    RVM_CHECK(q && kc && vc && out && n_tok > 0 && n_kv > 0 && n_head > 0 && n_head % n_kv == 0 && hd > 0 &&
              hd % QK == 0 && hd <= AT_MAXHD && p0 >= 0 && cap > 0 && window >= 0 && n_chunks > 0 &&
              (n_chunks == 1 || part));
    RVM_CHECK(attn_longest(n_tok, p0, window) <= cap);
    return launch_attn(q, kc, vc, out, part, n_tok, n_head, n_kv, hd, p0, cap, window, n_chunks);
}

int rvh_attn_combine(const float *part, float *out, int rows, int hd, int n_chunks) {
    RVM_CHECK(part && out && rows > 0 && hd > 0 && n_chunks > 1);
    if (n_chunks > AT_WAVES * CB_B && n_chunks <= 4 * 32)  // more than one batch of k_attn_combine
        hipLaunchKernelGGL((k_attn_merge<4, 32>), dim3(rows, (hd + 63) / 64), dim3(4 * 64), 0, cur_stream(), part,
                           out, hd, n_chunks);
    else if (n_chunks > 4 * 32 && n_chunks <= 8 * 40)
        hipLaunchKernelGGL((k_attn_merge<8, 40>), dim3(rows, (hd + 63) / 64), dim3(8 * 64), 0, cur_stream(), part,
                           out, hd, n_chunks);
    else
        hipLaunchKernelGGL(k_attn_combine, dim3(rows, (hd + 63) / 64), dim3(AT_WAVES * 64), 0, cur_stream(), part,
                           out, hd, n_chunks);
    return launched();
}

int rvm_attn_decode(const float *q, const float *k, const float *v, void *kc, void *vc, float *out, float *part,
                    int n_head, int n_kv, int hd, int pos, int cap, int window, int n_chunks) {
    RVM_CHECK(q && k && v && kc && vc && out && n_kv > 0 && n_head > 0 && n_head % n_kv == 0 && hd > 0 &&
              hd % QK == 0 && hd <= AT_MAXHD && pos >= 0 && cap > 0 && window >= 0 && n_chunks > 0 &&
              (n_chunks == 1 || part));
    RVM_CHECK(attn_longest(1, pos, window) <= cap);
    const int G = stream_group(n_head, n_kv, hd);
    if (!G) {  // other shapes: the three reference operations in sequence
        if (int rc = rvh_kv_store(k, v, kc, vc, 1, n_kv, hd, pos, cap)) return rc;
        if (int rc = launch_attn(q, kc, vc, out, part, 1, n_head, n_kv, hd, pos, cap, window, n_chunks)) return rc;
    } else if (int rc = launch_stream(q, kc, vc, out, part, 1, n_head, n_kv, hd, pos, cap, window, n_chunks, G, k, v)) {
        return rc;
    }
    return n_chunks > 1 ? rvh_attn_combine(part, out, n_head, hd, n_chunks) : 0;
}

int rvh_attention(const float *q, const void *kc, const void *vc, float *out, float *scores, int n_tok, int n_head,
                  int n_kv, int hd, int p0, int cap, int window, int max_keys) {
    RVM_CHECK(q && kc && vc && out && scores && n_tok > 0 && n_kv > 0 && n_head > 0 && n_head % n_kv == 0 &&
              hd > 0 && hd % QK == 0 && hd <= AT_MAXHD && p0 >= 0 && cap > 0 && window >= 0);
    const long longest = attn_longest(n_tok, p0, window);
    RVM_CHECK(longest <= max_keys && longest <= cap);
    return launch_attn(q, kc, vc, out, nullptr, n_tok, n_head, n_kv, hd, p0, cap, window, 1);
}

}  // extern "C"
