// SPDX-License-Identifier: GPL-3.0-only
// refops.hip - the reference's per-operation expert-path kernels with their rvhip.h signatures
// (runtime/hip/rvhip.h:42-80), written for wave64: a caller of the reference ABI (its
// runtime/src/hip_exec.rs:780-843 dispatch) can bind these symbols unchanged. The fused
// rvm_moe_* entry points are the fast path; these keep the per-operation contract.
//
// Attribution: k_rms_norm, k_geglu_split, k_gather_rows and k_moe_combine follow the reference's
// kernels of the same operators (Rowanjgc/Rosevine runtime/hip/rvhip.hip:75-90 and 401-436,
// GPL-3.0-only) statement for statement where the bitwise contract of those operators
// (runtime/tests/hip_ops.rs:421-439) fixes every operation; this file is therefore distributed
// under the reference's licence. k_f32_mm and k_q4_mm are this project's own designs.
#include "internal.hpp"

namespace rvm {

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// out = ((x * 1/sqrt(mean(x^2) + eps)) * post) * weight, f64 sum of squares
// (runtime/hip/rvhip.hip:75-90 semantics; runtime/src/ops.rs:131-139).
__global__ __launch_bounds__(256) void k_rms_norm(const float *x, float *out, const float *__restrict__ w,
                                                  int width, float eps, float post) {
    __shared__ double sh[4];
    const float *xr = x + (size_t)blockIdx.x * width;
    float *o = out + (size_t)blockIdx.x * width;
    double s = 0.0;
    for (int i = threadIdx.x; i < width; i += 256) s += (double)xr[i] * (double)xr[i];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    const double tot = ((sh[0] + sh[1]) + sh[2]) + sh[3];
    const float mean = (float)(tot / (double)width);
    const float scale = 1.0f / sqrtf(mean + eps);
    __syncthreads();  // x may alias out
    for (int i = threadIdx.x; i < width; i += 256) {
        float v = xr[i] * scale;
        if (post != 1.0f) v = v * post;
        if (w) v = v * w[i];
        o[i] = v;
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
// one): each row's items are read as one contiguous run per wave (a 16- or 8-byte nibble load per
// lane, at the block's 2-byte alignment), and a lane's activations are loaded once for the wave's rows.
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

// An item is a whole block (SUB 1) or half of one (SUB 2: nibble bytes 8h .. 8h+7, elements
// 8h .. 8h+7 and 16+8h .. 16+8h+7, with the block's d). Half blocks keep more lanes busy where a
// row's blocks leave the last column of lanes mostly idle: 88 blocks of a 2816-wide row fill 2 x 64
// lanes to 69%, its 176 halves fill 3 x 64 lanes to 92% at half the work per item.
// The rows of workgroup bx (one wave) of one matrix (blockIdx.y picks the tokens). One-wave
// workgroups spread the rows over the CUs within a wave's rows of each other: with four waves per
// workgroup, 2112 rows made 528 workgroups, three on some CUs and two on most (a third slower).
template <int SUB, int NCOL, int QRW, int TT>  // items per block; item columns per lane; rows per wave; tokens
__device__ __forceinline__ void q4_mm_rows(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                           float *__restrict__ y, int n_out, int k, int n_in, int bx) {
    constexpr int NW = 4 / SUB, NB = 4 * NW, NE = 2 * NB;  // nibble dwords, bytes and elements per item
    const int r0 = bx * QRW, lane = threadIdx.x & 63;
    if (r0 >= n_out) return;
    const int t0 = blockIdx.y * TT, nt = min(TT, n_in - t0);
    const int nb = k / QK, ni = nb * SUB;
    const size_t rb = (size_t)nb * Q4_BLOCK;
    float acc[QRW][TT];
#pragma unroll
    for (int r = 0; r < QRW; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = 0.0f;
    for (int cg = 0; cg < ni; cg += 64 * NCOL) {  // one pass unless a row has more than 64 NCOL items
        // the group's weight loads first: QRW rows x NCOL columns (rows and columns past the end clamped)
        float d[NCOL][QRW];
        uint32_t q[NCOL][QRW][NW];
        uint32_t xo[NCOL];  // the item's first activation within a token's row
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
            const uint32_t it = min(cg + lane + 64 * c, ni - 1), bo = it / SUB * Q4_BLOCK;
            const uint32_t qo = bo + 2 + it % SUB * NB;
            xo[c] = it / SUB * QK + it % SUB * NB;
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
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (t >= nt) break;
            const float *xt = x + (size_t)(t0 + t) * k;
#pragma unroll
            for (int c = 0; c < NCOL; ++c) {
                if (cg + lane + 64 * c >= ni) break;
                const float *xb = xt + xo[c];
                float xv[NE];  // the item's low-nibble elements, then its high-nibble ones
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
                for (int i = 0; i < NE; ++i) xs += xv[i];
#pragma unroll
                for (int r = 0; r < QRW; ++r) {
                    // low nibbles as they lie, high nibbles in place (16 n, scaled back once)
                    float sl = 0.0f, sh = 0.0f;
#pragma unroll
                    for (int j = 0; j < NW; ++j) {
                        const uint32_t lo = and_opaque(q[c][r][j], 0x0F0F0F0Fu);
                        const uint32_t hi = and_opaque(q[c][r][j], 0xF0F0F0F0u);
                        sl = fmaf((float)(lo & 0xFF), xv[4 * j], sl);
                        sh = fmaf((float)(hi & 0xFF), xv[NB + 4 * j], sh);
                        sl = fmaf((float)((lo >> 8) & 0xFF), xv[4 * j + 1], sl);
                        sh = fmaf((float)((hi >> 8) & 0xFF), xv[NB + 4 * j + 1], sh);
                        sl = fmaf((float)((lo >> 16) & 0xFF), xv[4 * j + 2], sl);
                        sh = fmaf((float)((hi >> 16) & 0xFF), xv[NB + 4 * j + 2], sh);
                        sl = fmaf((float)(lo >> 24), xv[4 * j + 3], sl);
                        sh = fmaf((float)(hi >> 24), xv[NB + 4 * j + 3], sh);
                    }
                    acc[r][t] = fmaf(d[c][r], fmaf(sh, 0.0625f, sl) - 8.0f * xs, acc[r][t]);
                }
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

__global__ void k_geglu_split(const float *__restrict__ gu, float *__restrict__ out, size_t n, int ff) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const size_t r = i / ff, j = i % ff;
    out[i] = gelu(gu[r * 2 * ff + j]) * gu[r * 2 * ff + ff + j];
}

__global__ void k_gather_rows(const float *__restrict__ src, const int32_t *__restrict__ idx, float *__restrict__ dst,
                              int width) {
    const float *s = src + (size_t)idx[blockIdx.x] * width;
    float *d = dst + (size_t)blockIdx.x * width;
    for (int i = threadIdx.x; i < width; i += blockDim.x) d[i] = s[i];
}

// Slot order, (y * scale) * weight, first term assigned: bitwise the CPU combine
// (runtime/src/exec.rs:626-638; runtime/tests/hip_ops.rs:421-439).
__global__ void k_moe_combine(const float *__restrict__ y, const int32_t *__restrict__ pos,
                              const float *__restrict__ scale, const float *__restrict__ weight,
                              float *__restrict__ out, int used, int width) {
    const int t = blockIdx.x;
    for (int i = threadIdx.x; i < width; i += blockDim.x) {
        float acc = 0.0f;
        for (int j = 0; j < used; ++j) {
            const int p = t * used + j;
            const float v = y[(size_t)pos[p] * width + i] * scale[p] * weight[p];
            acc = j == 0 ? v : acc + v;
        }
        out[(size_t)t * width + i] = acc;
    }
}

// rows per wave for n_out rows in all: about 2048 waves, each with as many rows' bytes in flight as
// that allows
inline int q4_rows_per_wave(long n_out) { return n_out >= 16384 ? 8 : (n_out >= 8192 ? 4 : (n_out >= 4096 ? 2 : 1)); }

// Calls go(kernel template instance) with the instance for (k, rows per wave rw, n_in). Half-block
// items where they take fewer lane passes than whole blocks: 1 .. 32 blocks (one column of halves
// against one of blocks at twice the work) and 65 .. 96 (three columns of halves against two of
// blocks). The choice depends on k alone, so every token of a batch sums in the same order.
template <template <int, int, int, int> class K, typename Go>
void q4_dispatch(int k, int rw, int n_in, Go &&go) {
    const int nb = k / QK, ncol = min(grid_blocks(nb, 64), 4);
    const bool halves = nb <= 32 || (nb > 64 && nb <= 96);
    auto by_cols = [&](auto rwc, auto ttc) {
        constexpr int RW = decltype(rwc)::value, T = decltype(ttc)::value;
        if (halves) {
            if (nb <= 32) go(K<2, 1, RW, T>::fn);
            else go(K<2, 3, RW, T>::fn);
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
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(256), 0, cur_stream(), x, out, weight, width, eps, post);
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
    long rows = 0;
    for (int m = 0; m < n_mat; ++m) {
        RVM_CHECK(w[m] && y[m] && n_out[m] > 0 && ((uintptr_t)w[m] & 1) == 0);
        rows += n_out[m];
    }
    const int rw = q4_rows_per_wave(rows);
    Q4Mats mats{};
    long blocks = 0;
    for (int m = 0; m < n_mat; ++m) {
        mats.w[m] = (const uint8_t *)w[m];
        mats.y[m] = y[m];
        mats.n_out[m] = n_out[m];
        mats.start[m] = (int)blocks;
        blocks += grid_blocks(n_out[m], rw);
    }
    RVM_CHECK(blocks <= 0x7fffffffL);
    mats.n = n_mat;
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

int rvh_geglu_split(const float *gu, float *out, int rows, int ff) {
    RVM_CHECK(gu && out && rows > 0 && ff > 0);
    const size_t n = (size_t)rows * ff;
    hipLaunchKernelGGL(k_geglu_split, dim3(grid_blocks(n, 256)), dim3(256), 0, cur_stream(), gu, out, n, ff);
    return launched();
}

int rvh_gather_rows(const float *src, const int32_t *idx, float *dst, int n, int width) {
    RVM_CHECK(src && idx && dst && n > 0 && width > 0);
    hipLaunchKernelGGL(k_gather_rows, dim3(n), dim3(256), 0, cur_stream(), src, idx, dst, width);
    return launched();
}

int rvh_moe_combine(const float *y, const int32_t *pos, const float *scale, const float *weight, float *out,
                    int n_tok, int used, int width) {
    RVM_CHECK(y && pos && scale && weight && out && n_tok > 0 && used > 0 && width > 0);
    hipLaunchKernelGGL(k_moe_combine, dim3(n_tok), dim3(256), 0, cur_stream(), y, pos, scale, weight, out, used,
                       width);
    return launched();
}

}  // extern "C"
