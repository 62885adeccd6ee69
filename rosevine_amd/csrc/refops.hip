// refops.hip - the reference's per-operation expert-path operators with their rvhip.h signatures
// (runtime/hip/rvhip.h:42-80), written for wave64: a caller of the reference ABI (its
// runtime/src/hip_exec.rs:780-843 dispatch) can bind these symbols unchanged. The fused
// rvm_moe_* entry points are the fast path; these keep the per-operation contract.
//
// The element-wise operators (rms_norm, geglu_split, gather_rows, moe_combine) compute every
// element with the operations, and in the order, that the reference's operator contract fixes
// (runtime/tests/hip_ops.rs:402-439: rms_norm and geglu_split within a relative 1e-6, gather_rows
// and moe_combine bit for bit; runtime/src/ops.rs:131-149 and runtime/src/exec.rs:626-638 state
// the arithmetic); their kernels are this library's: 16-byte columns wherever the rows allow,
// a flat grid of (row, column chunk) workgroups, and per-row scalars read once per workgroup.
#include <initializer_list>

#include "internal.hpp"

namespace rvm {

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// ---- Element-wise operators: V floats per thread and column chunk (V = 4 where every row
// starts 16-byte aligned and the width is a multiple of 4, else 1) ----
template <int V>
struct Cols;
template <>
struct Cols<4> {
    float v[4];
    __device__ __forceinline__ void load(const float *p) {
        const float4 q = *(const float4 *)p;
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    }
    __device__ __forceinline__ void store(float *p) const { *(float4 *)p = make_float4(v[0], v[1], v[2], v[3]); }
};
template <>
struct Cols<1> {
    float v[1];
    __device__ __forceinline__ void load(const float *p) { v[0] = *p; }
    __device__ __forceinline__ void store(float *p) const { *p = v[0]; }
};
// The rows' 16-byte columns are usable: base pointers 16-byte aligned and width a multiple of 4.
inline bool cols4(int width, std::initializer_list<const void *> ptrs) {
    if (width % 4) return false;
    for (const void *p : ptrs)
        if (p && ((uintptr_t)p & 15)) return false;
    return true;
}
constexpr int EW_THREADS = 256;

// rms_norm of row blockIdx.x: s = 1 / sqrt(mean(x^2) + eps) with the sum of squares in f64 (each
// wave's partial sums joined in a fixed order), then ((x * s) * post) * w[i] per element, each
// product rounded (runtime/src/ops.rs:131-139; the post factor and the weight only when set).
// x may be out: every element is read before the barrier that precedes the first store.
template <int V>
__global__ __launch_bounds__(EW_THREADS) void k_rms_norm(const float *x, float *out, const float *__restrict__ w,
                                                         int width, float eps, float post) {
    __shared__ double part[EW_THREADS / 64];
    const float *xr = x + (size_t)blockIdx.x * width;
    float *o = out + (size_t)blockIdx.x * width;
    double s = 0.0;
    for (int c = threadIdx.x * V; c < width; c += EW_THREADS * V) {
        Cols<V> a;
        a.load(xr + c);
#pragma unroll
        for (int k = 0; k < V; ++k) s += (double)a.v[k] * (double)a.v[k];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = 1.0f / sqrtf((float)(tot / (double)width) + eps);
    for (int c = threadIdx.x * V; c < width; c += EW_THREADS * V) {
        Cols<V> a;
        a.load(xr + c);
        Cols<V> g;
        if (w) g.load(w + c);
#pragma unroll
        for (int k = 0; k < V; ++k) {
            float v = a.v[k] * scale;
            if (post != 1.0f) v = v * post;
            if (w) v = v * g.v[k];
            a.v[k] = v;
        }
        a.store(o + c);
    }
}

// One wave per output row and token.
__global__ __launch_bounds__(256) void k_f32_mm(const float *__restrict__ w, const float *__restrict__ x,
                                                float *__restrict__ y, int n_out, int k) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y, lane = threadIdx.x & 63;
    if (r >= n_out) return;
    const float *wr = w + (size_t)r * k, *xr = x + (size_t)t * k;
    float s = 0.0f;
    for (int i = lane; i < k; i += 64) s += wr[i] * xr[i];
    s = wave_sum_f(s);
    if (lane == 0) y[(size_t)t * n_out + r] = s;
}

// Q4_0 rows in the reference layout (18-byte blocks: f16 d, 16 nibble bytes; runtime/src/ops.rs:83-92)
// times f32 activations, the dense GEMV/GEMM family behind rvh_q4_mm (runtime/hip/rvhip.hip; the
// reference's k_q4_mm). Workgroup (one wave) w takes rows QRW w .. QRW w + QRW-1 (1 to 8, so that
// there are about 2048 waves) and lane l item columns l, l + 64, ... (an item is a block or half of
// one): each row's items are read as one contiguous run per wave, through dword-aligned loads where
// the rows start on dwords (q4_load_items; 2-byte-aligned loads read the same bytes a third slower),
// and a lane's activations are loaded once for the wave's rows. Matrices of 16384 rows or more take
// k_q4_mm_i8 (int8 digits of the activations on the matrix cores) instead.
// An item adds d * (sum_j n_j x_j - 8 sum_j x_j) with n_j its unsigned nibbles (one byte convert
// and one fused multiply-add per element), which is sum_j ((n_j - 8) d) x_j up to rounding; the
// reference's CPU ops are the tolerance target (runtime/tests/hip_ops.rs:56-81). Each output is
// summed in a fixed order (items per lane in column order, then a fixed wave reduction), so a
// token's result does not depend on the other tokens of the call.
constexpr int QTT = 8;  // tokens per pass (calls with one token use a one-token variant)
template <int NW>
struct __attribute__((packed, aligned(2))) Q4Nibbles {
    uint32_t q[NW];
};
template <int N>
struct __attribute__((packed, aligned(4))) Dwords {
    uint32_t q[N];
};

// An item is a whole block (SUB 1) or half of one (SUB 2: nibble bytes 8h .. 8h+7, elements
// 8h .. 8h+7 and 16+8h .. 16+8h+7, with the block's d). Half blocks keep more lanes busy where a
// row's blocks leave the last column of lanes mostly idle: 88 blocks of a 2816-wide row fill 2 x 64
// lanes to 69%, its 176 halves fill 3 x 64 lanes to 92% at half the work per item.
// Loads QRW rows from r0 x NCOL item columns from cg of one matrix (rows and columns past the end
// clamped): each (item, row)'s d and nibble dwords, and each item's first activation within a row of x.
template <int SUB, int NCOL, int QRW>
__device__ __forceinline__ void q4_load_items(const uint8_t *__restrict__ w, size_t rb, int n_out, int r0, int cg,
                                              int ni, bool aligned, float (&d)[NCOL][QRW],
                                              uint32_t (&q)[NCOL][QRW][4 / SUB], uint32_t (&xo)[NCOL]) {
    constexpr int NW = 4 / SUB, NB = 4 * NW;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
        const uint32_t it = min(cg + lane + 64 * c, ni - 1), b = it / SUB, h = it % SUB;
        xo[c] = b * QK + h * NB;
        if (aligned) {
            // Dword-aligned loads that cover the item: a block starts on a dword (even b) or 2 bytes
            // past one (odd b), so the load starts at 18 b + 8 h, 2 bytes earlier for odd b, and a
            // byte permute picks the nibble dwords. Every load stays inside the matrix: an odd
            // block's loads start 2 bytes into the block before it, an even block's whole-block
            // load ends 2 bytes into the block after it, and a row's last block is odd.
            const uint32_t odd = b & 1, a = b * Q4_BLOCK + h * 8 - 2 * odd;
            const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
#pragma unroll
            for (int r = 0; r < QRW; ++r) {
                const uint8_t *row = w + (size_t)__builtin_amdgcn_readfirstlane(min(r0 + r, n_out - 1)) * rb;
                uint32_t v[NW + 1];
                if constexpr (SUB == 2) {
                    const Dwords<3> u = *(const Dwords<3> *)(row + a);
                    v[0] = u.q[0];
                    v[1] = u.q[1];
                    v[2] = u.q[2];
                } else {
                    const Dwords<4> u = *(const Dwords<4> *)(row + a);
                    v[0] = u.q[0];
                    v[1] = u.q[1];
                    v[2] = u.q[2];
                    v[3] = u.q[3];
                    v[4] = *(const uint32_t *)(row + a + 16);
                }
#pragma unroll
                for (int j = 0; j < NW; ++j) q[c][r][j] = __builtin_amdgcn_perm(v[j + 1], v[j], sel);
                uint32_t dbits = v[0] >> (16 * odd);
                // the second half of a block takes d from the first half's lane (lane ^ 1)
                if constexpr (SUB == 2) dbits = __builtin_amdgcn_mov_dpp(dbits, 0xA0, 0xF, 0xF, false);
                d[c][r] = h2f((uint16_t)dbits);
            }
        } else {
            const uint32_t bo = b * Q4_BLOCK, qo = bo + 2 + h * NB;
#pragma unroll
            for (int r = 0; r < QRW; ++r) {
                // the row's start is the same for the whole wave; lanes add a 32-bit offset
                const uint8_t *row = w + (size_t)__builtin_amdgcn_readfirstlane(min(r0 + r, n_out - 1)) * rb;
                d[c][r] = h2f(*(const uint16_t *)(row + bo));
                const Q4Nibbles<NW> v = *(const Q4Nibbles<NW> *)(row + qo);
#pragma unroll
                for (int j = 0; j < NW; ++j) q[c][r][j] = v.q[j];
            }
        }
    }
}

// An item's activations (its low-nibble elements, then its high-nibble ones); returns their sum.
template <int SUB>
__device__ __forceinline__ float q4_item_x(const float *__restrict__ xb, float (&xv)[32 / SUB]) {
    constexpr int NB = 16 / SUB;
#pragma unroll
    for (int i = 0; i < NB / 4; ++i) {
        const float4 lo = ((const float4 *)xb)[i], hi = ((const float4 *)(xb + 16))[i];
        xv[4 * i] = lo.x;
        xv[4 * i + 1] = lo.y;
        xv[4 * i + 2] = lo.z;
        xv[4 * i + 3] = lo.w;
        xv[NB + 4 * i] = hi.x;
        xv[NB + 4 * i + 1] = hi.y;
        xv[NB + 4 * i + 2] = hi.z;
        xv[NB + 4 * i + 3] = hi.w;
    }
    float xs = 0.0f;
#pragma unroll
    for (int i = 0; i < 2 * NB; ++i) xs += xv[i];
    return xs;
}

// acc + d (sum_j n_j x_j - 8 sum_j x_j) over one item: low nibbles as they lie, high nibbles in place
// (16 n, scaled back once)
template <int SUB>
__device__ __forceinline__ float q4_item_dot(const uint32_t (&q)[4 / SUB], const float (&xv)[32 / SUB], float d,
                                             float xs, float acc) {
    constexpr int NW = 4 / SUB, NB = 4 * NW;
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const uint32_t lo = and_opaque(q[j], 0x0F0F0F0Fu);
        const uint32_t hi = and_opaque(q[j], 0xF0F0F0F0u);
        sl = fmaf((float)(lo & 0xFF), xv[4 * j], sl);
        sh = fmaf((float)(hi & 0xFF), xv[NB + 4 * j], sh);
        sl = fmaf((float)((lo >> 8) & 0xFF), xv[4 * j + 1], sl);
        sh = fmaf((float)((hi >> 8) & 0xFF), xv[NB + 4 * j + 1], sh);
        sl = fmaf((float)((lo >> 16) & 0xFF), xv[4 * j + 2], sl);
        sh = fmaf((float)((hi >> 16) & 0xFF), xv[NB + 4 * j + 2], sh);
        sl = fmaf((float)(lo >> 24), xv[4 * j + 3], sl);
        sh = fmaf((float)(hi >> 24), xv[NB + 4 * j + 3], sh);
    }
    return fmaf(d, fmaf(sh, 0.0625f, sl) - 8.0f * xs, acc);
}

// rows of an even block count on a 4-byte aligned matrix: every row starts on a dword
__host__ __device__ __forceinline__ bool q4_rows_aligned(const uint8_t *w, int nb) {
    return (nb & 1) == 0 && ((uintptr_t)w & 3) == 0;
}

// The rows of workgroup bx (one wave) of one matrix (blockIdx.y picks the tokens). One-wave
// workgroups spread the rows over the CUs within a wave's rows of each other: with four waves per
// workgroup, 2112 rows made 528 workgroups, three on some CUs and two on most (a third slower).
template <int SUB, int NCOL, int QRW, int TT>  // items per block; item columns per lane; rows per wave; tokens
__device__ __forceinline__ void q4_mm_rows(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                           float *__restrict__ y, int n_out, int k, int n_in, int bx) {
    constexpr int NW = 4 / SUB, NE = 32 / SUB;
    const int r0 = bx * QRW, lane = threadIdx.x & 63;
    if (r0 >= n_out) return;
    const int t0 = blockIdx.y * TT, nt = min(TT, n_in - t0);
    const int nb = k / QK, ni = nb * SUB;
    const size_t rb = (size_t)nb * Q4_BLOCK;
    const bool aligned = q4_rows_aligned(w, nb);
    float acc[QRW][TT];
#pragma unroll
    for (int r = 0; r < QRW; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = 0.0f;
    for (int cg = 0; cg < ni; cg += 64 * NCOL) {  // one pass unless a row has more than 64 NCOL items
        // the group's weight loads first
        float d[NCOL][QRW];
        uint32_t q[NCOL][QRW][NW];
        uint32_t xo[NCOL];
        q4_load_items<SUB, NCOL, QRW>(w, rb, n_out, r0, cg, ni, aligned, d, q, xo);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (t >= nt) break;
            const float *xt = x + (size_t)(t0 + t) * k;
#pragma unroll
            for (int c = 0; c < NCOL; ++c) {
                if (cg + lane + 64 * c >= ni) break;
                float xv[NE];
                const float xs = q4_item_x<SUB>(xt + xo[c], xv);
#pragma unroll
                for (int r = 0; r < QRW; ++r) acc[r][t] = q4_item_dot<SUB>(q[c][r], xv, d[c][r], xs, acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if (t >= nt) break;
#pragma unroll
        for (int r = 0; r < QRW; ++r) {
            const float v = wave_sum_dpp(acc[r][t]);
            if (lane == 0 && r0 + r < n_out) y[(size_t)(t0 + t) * n_out + r0 + r] = v;
        }
    }
}

// Many rows (a vocabulary head): exact int8 block sums on the matrix cores. The token's activations
// become, per block b, four int8 digits D_p (|D_p| <= 64) with
//   x_k 2^(132 - E_b) = D_0k + D_1k 2^-7 + D_2k 2^-14 + D_3k 2^-21 (+ less than 2^-22),
// E_b the largest biased exponent of the block's |x| (so |x_k| 2^(132 - E_b) < 64): exact for every
// element within 2^-3 of the block's largest, and within 2^-28 of that largest for the rest. Each
// v_mfma_i32_16x16x32_i8 then sums 16 (n - 8) D over one block's 8 elements exactly, with the
// weights 16 (n - 8) = ((n ^ 8) << 4) as signed bytes. A step covers 16 rows x 4 blocks: K group g of
// the instruction carries one block of each row (B, from lane (row j, group g)), and A row 4g + p
// carries digit p of that block (zero in the other groups), so lane (j, g) receives C[4g + p][j], the
// four digit sums of its own row and block, which it folds with its own d:
//   acc += d * ((((C_3 2^-7 + C_2) 2^-7 + C_1) 2^-7 + C_0) * 2^(E_b - 136)),
// the block's term d sum_k (n_k - 8) x_k up to f32 rounding. The lanes of a row add their sums in
// a fixed order, and the tokens of a pass (up to 4 per blockIdx.y) share only the weight loads, so
// a token's result does not depend on the other tokens of the call. A block with a non-finite
// activation gives NaN rows.
typedef int qi_v4i __attribute__((ext_vector_type(4)));
constexpr int QI_WAVES = 8, QI_ROWS = 16, QI_CH = 4;  // waves, rows per wave, step pairs per load chunk
constexpr int QI_BUF = 1;                               // chunks in registers
constexpr int QI_MIN_ROWS = 16384, QI_MAX_NB = 256;    // rvh_q4_mm takes this kernel from 16384 rows, k <= 8192
// dynamic LDS for tt tokens: digits [tt][nb][4 digits][8 dwords], 8 zero dwords, then the block
// scales [tt][nb]; passes take 4, 2 or 1 tokens, as many as fit 64 KB
inline size_t qi_lds_bytes(int nb, int tt) { return (size_t)tt * nb * (128 + 4) + 32; }
inline int qi_tokens(int nb, int n_in) {
    const int tt = qi_lds_bytes(nb, 4) <= 65536 ? 4 : (qi_lds_bytes(nb, 2) <= 65536 ? 2 : 1);
    return n_in >= tt ? tt : (n_in >= 2 && tt >= 2 ? 2 : 1);
}

// ALN: rows of an even block count on a 4-byte aligned matrix (q4_rows_aligned). TT: tokens per
// pass (blockIdx.y), which share the weight loads; each has its own digits, MFMAs and folds, the
// same operations as a pass of one token, so the same bits.
template <bool ALN, int TT>
__global__ __launch_bounds__(QI_WAVES * 64) void k_q4_mm_i8(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                  float *__restrict__ y, int n_out, int k, int n_in) {
    extern __shared__ __align__(16) uint32_t qi_sh[];
    const int nb = k / QK, tid = threadIdx.x;
    const int t0 = blockIdx.y * TT, nt = min(TT, n_in - t0);
    // token t's digits at dig + t nb 32, its block scales at xsc + t nb, one zero area after them
    uint32_t *dig = qi_sh, *zero = qi_sh + TT * nb * 32;
    float *xsc = (float *)(qi_sh + TT * nb * 32 + 8);
    const int lane = tid & 63, j = lane & 15, g = lane >> 4;
    const int r0 = (blockIdx.x * QI_WAVES + (tid >> 6)) * QI_ROWS;
    const size_t rb = (size_t)nb * Q4_BLOCK;
    const uint8_t *wr = w + (size_t)min(r0 + j, n_out - 1) * rb;
    // Steps go in pairs: K group g of pair p carries block 8p + 2g in the pair's first step and
    // block 8p + 2g + 1 in its second, so each lane loads two adjacent blocks, 36 bytes of its row.
    // This lane's A operand: digit j & 3 of its K group's block when j >> 2 == g, zeros otherwise.
    const bool adig = (j >> 2) == g;
    const int pairs = (nb + 7) >> 3, nch = (pairs + QI_CH - 1) / QI_CH;
    // a pair's weights: aligned rows, its 9 dwords as loaded (d0 in the low half of v[0], nibbles of
    // the first block from byte 2, d1 in the high half of v[4], nibbles of the second in v[5 .. 8]);
    // otherwise v = {d0, n0[4], d1, n1[4]}
    auto load = [&](int c, uint32_t (&v)[QI_CH][10]) {
#pragma unroll
        for (int u = 0; u < QI_CH; ++u) {
            const int b0 = (c * QI_CH + u) * 8 + 2 * g;
            if constexpr (ALN) {
                // blocks 2i and 2i + 1 are the 9 dwords from byte 36 i (rows of an even block count)
                const Dwords<4> a = *(const Dwords<4> *)(wr + min(b0, nb - 2) * Q4_BLOCK);
                const Dwords<4> e = *(const Dwords<4> *)(wr + min(b0, nb - 2) * Q4_BLOCK + 16);
                const uint32_t f = *(const uint32_t *)(wr + min(b0, nb - 2) * Q4_BLOCK + 32);
                // the dwords as loaded: compute() picks the fields, so nothing here waits for them
                const uint32_t dw[9] = {a.q[0], a.q[1], a.q[2], a.q[3], e.q[0], e.q[1], e.q[2], e.q[3], f};
#pragma unroll
                for (int i = 0; i < 9; ++i) v[u][i] = dw[i];
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint8_t *p = wr + min(b0 + h, nb - 1) * Q4_BLOCK;
                    v[u][5 * h] = *(const uint16_t *)p;
                    const Q4Nibbles<4> q = *(const Q4Nibbles<4> *)(p + 2);
#pragma unroll
                    for (int m = 0; m < 4; ++m) v[u][5 * h + 1 + m] = q.q[m];
                }
            }
        }
    };
    // The token's activations first (a thread per 4 elements, 8 threads per block), then the first
    // QI_BUF chunks of weights, in flight while the activation digits are built; chunk c + QI_BUF is
    // loaded into chunk c's registers once chunk c is computed. (Loads past the last chunk would
    // re-read it; with more than one chunk in registers, skipping them under a branch makes the
    // compiler's waits on the other path wait for the newer loads too.)
    constexpr int XPT = QI_MAX_NB * 8 / (QI_WAVES * 64);  // float4s per thread and token at most
    float4 xq[TT][XPT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const float4 *xt = (const float4 *)(x + (size_t)(t0 + min(t, nt - 1)) * k);
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
            const int f = tid + i * QI_WAVES * 64;
            xq[t][i] = f < nb * 8 ? xt[f] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    const bool rows_live = r0 < n_out;
    uint32_t vb[QI_BUF][QI_CH][10];
#pragma unroll
    for (int i = 0; i < QI_BUF; ++i)
        if (i < nch) load(i, vb[i]);
    // the digits
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const int f = tid + i * QI_WAVES * 64;
        if (t >= nt || f >= nb * 8) break;
        const int blk = t * nb + (f >> 3), q = f & 7;
        const float4 v = xq[t][i];
        const float e4[4] = {v.x, v.y, v.z, v.w};
        int e = 0;
#pragma unroll
        for (int el = 0; el < 4; ++el) e = max(e, (int)((__float_as_uint(e4[el]) >> 23) & 0xFF));
        e = max(e, __shfl_xor(e, 1));
        e = max(e, __shfl_xor(e, 2));
        e = max(e, __shfl_xor(e, 4));
        uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int el = 0; el < 4; ++el) {
            float u = ldexpf(e4[el], 132 - e);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const float dp = rintf(u);
                pk[p] |= ((uint32_t)(int)dp & 0xFFu) << (8 * el);
                u = (u - dp) * 128.0f;
            }
        }
        // elements 4q .. 4q+3 are bytes 8q .. 8q+3 of a digit's 32 (q < 4); 16 + 4m .. are 8m+4 ..
        const int dw = q < 4 ? 2 * q : 2 * (q - 4) + 1;
#pragma unroll
        for (int p = 0; p < 4; ++p) dig[(blk * 4 + p) * 8 + dw] = pk[p];
        if (q == 0) xsc[blk] = e == 255 ? __uint_as_float(0x7FC00000u) : ldexpf(1.0f, e - 136);
    }
    if (tid < 8) zero[tid] = 0u;
    __syncthreads();
    if (!rows_live) return;

    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = 0.0f;
    auto compute = [&](int c, const uint32_t (&v)[QI_CH][10]) {
#pragma unroll
        for (int u = 0; u < QI_CH; ++u) {
            if (c * QI_CH + u >= pairs) break;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int blk = (c * QI_CH + u) * 8 + 2 * g + h;
                const bool live = blk < nb;
                uint32_t nib[4], dbits;
                if constexpr (ALN) {
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        nib[m] = h ? v[u][5 + m] : __builtin_amdgcn_perm(v[u][m + 1], v[u][m], 0x05040302u);
                    dbits = h ? v[u][4] >> 16 : v[u][0] & 0xFFFFu;
                } else {
#pragma unroll
                    for (int m = 0; m < 4; ++m) nib[m] = v[u][5 * h + 1 + m];
                    dbits = v[u][5 * h];
                }
                long bw[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t n8 = nib[m] ^ 0x88888888u;
                    bw[m] = (long)(((uint64_t)(n8 & 0xF0F0F0F0u) << 32) | ((n8 << 4) & 0xF0F0F0F0u));
                }
                const float dv = h2f((uint16_t)dbits);
#pragma unroll
                for (int tk = 0; tk < TT; ++tk) {
                    if (tk >= nt) break;
                    const uint32_t *ap = adig && live ? dig + ((tk * nb + blk) * 4 + (j & 3)) * 8 : zero;
                    const uint4 a0 = *(const uint4 *)ap, a1 = *(const uint4 *)(ap + 4);
                    const uint32_t ad[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    qi_v4i cm = {0, 0, 0, 0};
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const long aw = (long)(((uint64_t)ad[2 * m + 1] << 32) | ad[2 * m]);
                        cm = __builtin_amdgcn_mfma_i32_16x16x32_i8(aw, bw[m], cm, 0, 0, 0);
                    }
                    const float t = fmaf(fmaf(fmaf((float)cm[3], 0.0078125f, (float)cm[2]), 0.0078125f,
                                              (float)cm[1]),
                                         0.0078125f, (float)cm[0]);
                    // past the row's last block the lane adds nothing (its loaded d is another block's)
                    if (live) acc[tk] = fmaf(dv, t * xsc[tk * nb + blk], acc[tk]);
                }
            }
        }
    };
    for (int c0 = 0; c0 < nch; c0 += QI_BUF) {
#pragma unroll
        for (int b = 0; b < QI_BUF; ++b) {
            const int c = c0 + b;
            if (c >= nch) break;
            compute(c, vb[b]);
            if (c + QI_BUF < nch) load(c + QI_BUF, vb[b]);
        }
    }
    // the four lanes of row j, groups (0 + 2) + (1 + 3)
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if (t >= nt) break;
        float r = acc[t] + __shfl_xor(acc[t], 32);
        r = r + __shfl_xor(r, 16);
        if (g == 0 && r0 + j < n_out) y[(size_t)(t0 + t) * n_out + r0 + j] = r;
    }
}

template <int SUB, int NCOL, int QRW, int TT>
__global__ __launch_bounds__(64) void k_q4_mm(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                              float *__restrict__ y, int n_out, int k, int n_in) {
    q4_mm_rows<SUB, NCOL, QRW, TT>(w, x, y, n_out, k, n_in, blockIdx.x);
}

// Up to four matrices on one input in one launch: workgroups start[m] .. start[m + 1] - 1 take
// matrix m, each row as k_q4_mm computes it (the same bits as one rvh_q4_mm call per matrix).
constexpr int Q4_NMAT = 4;
struct Q4Mats {
    const uint8_t *w[Q4_NMAT];
    float *y[Q4_NMAT];
    int n_out[Q4_NMAT];
    int start[Q4_NMAT];
    int n;
};

template <int SUB, int NCOL, int QRW, int TT>
__global__ __launch_bounds__(64) void k_q4_mm_n(Q4Mats mats, const float *__restrict__ x, int k, int n_in) {
    int m = 0;
#pragma unroll
    for (int i = 1; i < Q4_NMAT; ++i)
        if (i < mats.n && (int)blockIdx.x >= mats.start[i]) m = i;
    q4_mm_rows<SUB, NCOL, QRW, TT>(mats.w[m], x, mats.y[m], mats.n_out[m], k, n_in, blockIdx.x - mats.start[m]);
}

// Workgroup b takes row b / chunks, columns of chunk b % chunks (EW_THREADS V columns each).
struct EwTile {
    size_t row;
    int col;
    __device__ __forceinline__ EwTile(int chunks, int V) {
        row = blockIdx.x / (unsigned)chunks;
        col = ((int)(blockIdx.x % (unsigned)chunks) * EW_THREADS + (int)threadIdx.x) * V;
    }
};

// out[r][j] = gelu(gu[r][j]) * gu[r][ff + j]: the gate half, then the up half of each row of gu
// (runtime/src/ops.rs:145-149; gelu is the reference's tanh form with the reference hosts' tanhf).
template <int V>
__global__ __launch_bounds__(EW_THREADS) void k_geglu_split(const float *__restrict__ gu, float *__restrict__ out,
                                                            int ff, int chunks) {
    const EwTile at(chunks, V);
    if (at.col >= ff) return;
    Cols<V> g, u;
    g.load(gu + at.row * 2 * ff + at.col);
    u.load(gu + at.row * 2 * ff + ff + at.col);
#pragma unroll
    for (int k = 0; k < V; ++k) g.v[k] = gelu(g.v[k]) * u.v[k];
    g.store(out + at.row * ff + at.col);
}

// dst[r] = src[idx[r]], row by row.
template <int V>
__global__ __launch_bounds__(EW_THREADS) void k_gather_rows(const float *__restrict__ src, const int32_t *__restrict__ idx,
                                                            float *__restrict__ dst, int width, int chunks) {
    const EwTile at(chunks, V);
    if (at.col >= width) return;
    Cols<V> a;
    a.load(src + (size_t)idx[at.row] * width + at.col);
    a.store(dst + at.row * width + at.col);
}

// out[t] = sum over the token's slots j in order of (y[pos[p]] * scale[p]) * weight[p], p = t used + j,
// the first term assigned (runtime/src/exec.rs:626-638; runtime/tests/hip_ops.rs:421-439 checks it
// bit for bit). The slot's position, scale and weight are the same for the whole workgroup.
template <int V>
__global__ __launch_bounds__(EW_THREADS) void k_moe_combine(const float *__restrict__ y, const int32_t *__restrict__ pos,
                                                            const float *__restrict__ scale,
                                                            const float *__restrict__ weight, float *__restrict__ out,
                                                            int used, int width, int chunks) {
    const EwTile at(chunks, V);
    if (at.col >= width) return;
    Cols<V> acc;
    for (int j = 0; j < used; ++j) {
        const size_t p = at.row * used + j;
        const float sc = scale[p], wt = weight[p];
        Cols<V> a;
        a.load(y + (size_t)pos[p] * width + at.col);
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const float v = a.v[k] * sc * wt;
            acc.v[k] = j == 0 ? v : acc.v[k] + v;
        }
    }
    acc.store(out + at.row * width + at.col);
}

// a matrix of n_out rows of k goes through k_q4_mm_i8 (whatever the token count)
inline bool q4_uses_i8(int n_out, int k) { return n_out >= QI_MIN_ROWS && k / QK <= QI_MAX_NB; }

// rows per wave for n_out rows in all: 1024 to 2048 waves, each with as many rows' bytes in flight
// as that allows (two rows from 2048: one activation read serves both, 2816 x 4096 took 4.2 against
// 5.2 us with one)
inline int q4_rows_per_wave(long n_out) { return n_out >= 16384 ? 8 : (n_out >= 8192 ? 4 : (n_out >= 2048 ? 2 : 1)); }

// Calls go(kernel template instance) with the instance for (k, rows per wave rw, n_in). Half-block
// items up to 128 blocks: 1 .. 32 blocks (one column of halves against one of blocks at twice the
// work), 65 .. 96 (three columns of halves against two of blocks) and 97 .. 128 (four columns of
// halves, the same lane passes as two of blocks, at half each lane's dependent chain: 2816 x 4096
// took 5.2 against 7.0 us). The choice depends on k alone, so every token of a batch sums in the
// same order.
template <template <int, int, int, int> class K, typename Go>
void q4_dispatch(int k, int rw, int n_in, Go &&go) {
    const int nb = k / QK, ncol = min(grid_blocks(nb, 64), 4);
    const bool halves = nb <= 32 || (nb > 64 && nb <= 128);
    auto by_cols = [&](auto rwc, auto ttc) {
        constexpr int RW = decltype(rwc)::value, T = decltype(ttc)::value;
        if (halves) {
            if (nb <= 32) go(K<2, 1, RW, T>::fn);
            else if (nb <= 96) go(K<2, 3, RW, T>::fn);
            else go(K<2, 4, RW, T>::fn);
        } else if (ncol == 1) go(K<1, 1, RW, T>::fn);
        else if (ncol == 2) go(K<1, 2, RW, T>::fn);
        else if (ncol == 3) go(K<1, 3, RW, T>::fn);
        else go(K<1, 4, RW, T>::fn);
    };
    auto by_rows = [&](auto ttc) {
        if (rw == 8) by_cols(std::integral_constant<int, 8>{}, ttc);
        else if (rw == 4) by_cols(std::integral_constant<int, 4>{}, ttc);
        else if (rw == 2) by_cols(std::integral_constant<int, 2>{}, ttc);
        else by_cols(std::integral_constant<int, 1>{}, ttc);
    };
    if (n_in == 1) by_rows(std::integral_constant<int, 1>{});
    else by_rows(std::integral_constant<int, QTT>{});
}
template <int S, int C, int R, int T>
struct Q4One {
    static constexpr auto fn = k_q4_mm<S, C, R, T>;
};
template <int S, int C, int R, int T>
struct Q4Many {
    static constexpr auto fn = k_q4_mm_n<S, C, R, T>;
};

}  // namespace rvm

using namespace rvm;

extern "C" {

int rvh_rms_norm(const float *x, float *out, const float *weight, int rows, int width, float eps, float post) {
    RVM_CHECK(x && out && rows > 0 && width > 0);
    if (cols4(width, {x, out, weight}))
        hipLaunchKernelGGL(k_rms_norm<4>, dim3(rows), dim3(EW_THREADS), 0, cur_stream(), x, out, weight, width, eps, post);
    else
        hipLaunchKernelGGL(k_rms_norm<1>, dim3(rows), dim3(EW_THREADS), 0, cur_stream(), x, out, weight, width, eps, post);
    return launched();
}

int rvh_f32_mm(const float *w, const float *x, float *y, int n_out, int k, int n_in) {
    RVM_CHECK(w && x && y && n_out > 0 && n_in > 0 && n_in <= 65535 && k > 0);
    hipLaunchKernelGGL(k_f32_mm, dim3(grid_blocks(n_out, 4), n_in), dim3(256), 0, cur_stream(), w, x, y, n_out, k);
    return launched();
}

int rvh_q4_mm(const void *w, const float *x, float *y, int n_out, int k, int n_in) {
    RVM_CHECK(w && x && y && n_out > 0 && n_in > 0 && k > 0 && k % QK == 0 && ((uintptr_t)w & 1) == 0);
    RVM_CHECK(grid_blocks(n_in, QTT) <= 65535);
    if (q4_uses_i8(n_out, k)) {
        const int nb = k / QK, tt = qi_tokens(nb, n_in);
        RVM_CHECK(grid_blocks(n_in, tt) <= 65535);
        const dim3 grid(grid_blocks(n_out, QI_WAVES * QI_ROWS), grid_blocks(n_in, tt));
        const bool aln = q4_rows_aligned((const uint8_t *)w, nb);
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(QI_WAVES * 64), qi_lds_bytes(nb, tt), cur_stream(), (const uint8_t *)w,
                               x, y, n_out, k, n_in);
        };
        if (tt == 4) aln ? go(k_q4_mm_i8<true, 4>) : go(k_q4_mm_i8<false, 4>);
        else if (tt == 2) aln ? go(k_q4_mm_i8<true, 2>) : go(k_q4_mm_i8<false, 2>);
        else aln ? go(k_q4_mm_i8<true, 1>) : go(k_q4_mm_i8<false, 1>);
        return launched();
    }
    const int rw = q4_rows_per_wave(n_out);
    const dim3 grid(grid_blocks(n_out, rw), grid_blocks(n_in, n_in == 1 ? 1 : QTT));
    q4_dispatch<Q4One>(k, rw, n_in, [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(64), 0, cur_stream(), (const uint8_t *)w, x, y, n_out, k, n_in);
    });
    return launched();
}

int rvm_q4_mm_n(int n_mat, const void *const *w, const int *n_out, float *const *y, const float *x, int k, int n_in) {
    RVM_CHECK(n_mat >= 1 && n_mat <= Q4_NMAT && w && n_out && y && x && n_in > 0 && k > 0 && k % QK == 0);
    RVM_CHECK(grid_blocks(n_in, QTT) <= 65535);
    for (int m = 0; m < n_mat; ++m) RVM_CHECK(w[m] && y[m] && n_out[m] > 0 && ((uintptr_t)w[m] & 1) == 0);
    // matrices that rvh_q4_mm sends to k_q4_mm_i8 go there (their own launches), the rest together
    Q4Mats mats{};
    long rows = 0;
    for (int m = 0; m < n_mat; ++m) {
        if (q4_uses_i8(n_out[m], k)) continue;
        mats.w[mats.n] = (const uint8_t *)w[m];
        mats.y[mats.n] = y[m];
        mats.n_out[mats.n] = n_out[m];
        rows += n_out[m];
        ++mats.n;
    }
    for (int m = 0; m < n_mat; ++m)
        if (q4_uses_i8(n_out[m], k)) {
            const int rc = rvh_q4_mm(w[m], x, y[m], n_out[m], k, n_in);
            if (rc) return rc;
        }
    if (mats.n == 0) return 0;
    const int rw = q4_rows_per_wave(rows);
    long blocks = 0;
    for (int m = 0; m < mats.n; ++m) {
        mats.start[m] = (int)blocks;
        blocks += grid_blocks(mats.n_out[m], rw);
    }
    RVM_CHECK(blocks <= 0x7fffffffL);
    const dim3 grid((unsigned)blocks, grid_blocks(n_in, n_in == 1 ? 1 : QTT));
    q4_dispatch<Q4Many>(k, rw, n_in, [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(64), 0, cur_stream(), mats, x, k, n_in);
    });
    return launched();
}

// The reference's K2 variant (rvhip.h:46-48) has rvh_q4_mm's result up to summation order and asks
// for 16-byte aligned x and 2-byte aligned w; here it is the same kernel.
int rvh_q4_mv(const void *w, const float *x, float *y, int n_out, int k, int n_in) {
    RVM_CHECK(((uintptr_t)x & 15) == 0);
    return rvh_q4_mm(w, x, y, n_out, k, n_in);
}

// The flat grid of the element-wise operators: rows x column chunks workgroups (at most 2^31 - 1).
inline int ew_chunks(int width, int V) { return grid_blocks(width, EW_THREADS * V); }
inline bool ew_grid_ok(int rows, int chunks) { return (long)rows * chunks <= 0x7fffffffL; }

int rvh_geglu_split(const float *gu, float *out, int rows, int ff) {
    RVM_CHECK(gu && out && rows > 0 && ff > 0);
    const int V = cols4(ff, {gu, out}) ? 4 : 1, chunks = ew_chunks(ff, V);
    RVM_CHECK(ew_grid_ok(rows, chunks));
    const dim3 grid((unsigned)((long)rows * chunks));
    if (V == 4)
        hipLaunchKernelGGL(k_geglu_split<4>, grid, dim3(EW_THREADS), 0, cur_stream(), gu, out, ff, chunks);
    else
        hipLaunchKernelGGL(k_geglu_split<1>, grid, dim3(EW_THREADS), 0, cur_stream(), gu, out, ff, chunks);
    return launched();
}

int rvh_gather_rows(const float *src, const int32_t *idx, float *dst, int n, int width) {
    RVM_CHECK(src && idx && dst && n > 0 && width > 0);
    const int V = cols4(width, {src, dst}) ? 4 : 1, chunks = ew_chunks(width, V);
    RVM_CHECK(ew_grid_ok(n, chunks));
    const dim3 grid((unsigned)((long)n * chunks));
    if (V == 4)
        hipLaunchKernelGGL(k_gather_rows<4>, grid, dim3(EW_THREADS), 0, cur_stream(), src, idx, dst, width, chunks);
    else
        hipLaunchKernelGGL(k_gather_rows<1>, grid, dim3(EW_THREADS), 0, cur_stream(), src, idx, dst, width, chunks);
    return launched();
}

int rvh_moe_combine(const float *y, const int32_t *pos, const float *scale, const float *weight, float *out,
                    int n_tok, int used, int width) {
    RVM_CHECK(y && pos && scale && weight && out && n_tok > 0 && used > 0 && width > 0);
    const int V = cols4(width, {y, out}) ? 4 : 1, chunks = ew_chunks(width, V);
    RVM_CHECK(ew_grid_ok(n_tok, chunks));
    const dim3 grid((unsigned)((long)n_tok * chunks));
    if (V == 4)
        hipLaunchKernelGGL(k_moe_combine<4>, grid, dim3(EW_THREADS), 0, cur_stream(), y, pos, scale, weight, out, used,
                           width, chunks);
    else
        hipLaunchKernelGGL(k_moe_combine<1>, grid, dim3(EW_THREADS), 0, cur_stream(), y, pos, scale, weight, out, used,
                           width, chunks);
    return launched();
}

}  // extern "C"
