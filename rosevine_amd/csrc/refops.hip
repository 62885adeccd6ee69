// refops.hip - the reference's per-operation expert-path kernels with their rvhip.h signatures
// (runtime/hip/rvhip.h:42-80), written for wave64: a caller of the reference ABI (its
// runtime/src/hip_exec.rs:780-843 dispatch) can bind these symbols unchanged. The fused
// rvm_moe_* entry points are the fast path; these keep the per-operation contract.
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

// Q4_0 rows (reference layout) x f32 activations: one wave per row, lanes over blocks, up to
// 8 tokens per pass; each element dequantised as ((q - 8) as f32) * d, as ops.rs:83-92.
constexpr int QTT = 8;
__global__ __launch_bounds__(256) void k_q4_mm(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                               float *__restrict__ y, int n_out, int k, int n_in) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int t0 = blockIdx.y * QTT;
    if (r >= n_out) return;
    const int nb = k / QK, nt = min(QTT, n_in - t0);
    const uint8_t *row = w + (size_t)r * nb * Q4_BLOCK;
    float acc[QTT];
#pragma unroll
    for (int i = 0; i < QTT; ++i) acc[i] = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const uint16_t *h = (const uint16_t *)(row + (size_t)b * Q4_BLOCK);
        const float d = h2f(h[0]);
        float v[QK];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t u = h[1 + j];
            v[2 * j] = (float)((int)(u & 15) - 8) * d;
            v[2 * j + 1] = (float)((int)((u >> 8) & 15) - 8) * d;
            v[16 + 2 * j] = (float)((int)((u >> 4) & 15) - 8) * d;
            v[16 + 2 * j + 1] = (float)((int)((u >> 12) & 15) - 8) * d;
        }
#pragma unroll
        for (int i = 0; i < QTT; ++i)
            if (i < nt) {
                const float *xs = x + (size_t)(t0 + i) * k + (size_t)b * QK;
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < QK; ++j) s += v[j] * xs[j];
                acc[i] += s;
            }
    }
#pragma unroll
    for (int i = 0; i < QTT; ++i) {
        const float s = wave_sum_f(acc[i]);
        if (i < nt && lane == 0) y[(size_t)(t0 + i) * n_out + r] = s;
    }
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
    hipLaunchKernelGGL(k_q4_mm, dim3(grid_blocks(n_out, 4), grid_blocks(n_in, QTT)), dim3(256), 0, cur_stream(),
                       (const uint8_t *)w, x, y, n_out, k, n_in);
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
