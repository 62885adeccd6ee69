// quant.hip - Q8_0 activation quantisation, GeGLU + Q8_0, and the generic packed Q4_0 x Q8_0
// GEMV/GEMM with its per-block integer sums (runtime/src/ops.rs:95-105,
// runtime/src/expert_kernel.rs:147-161, runtime/src/exec.rs:606-611). All of them reproduce the
// reference bit for bit on the same inputs.
#include "internal.hpp"

namespace rvm {

// One Q8_0 block per 32-lane half-wave.
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, uint8_t *__restrict__ xq,
                                                       size_t nblocks) {
    const size_t gb = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    const bool ok = gb < nblocks;
    float v = ok ? x[gb * QK + j] : 0.0f;
    uint16_t dbits;
    int q = quant_q8_half(v, &dbits);
    if (ok) {
        uint8_t *blk = xq + gb * Q8_BLOCK;
        blk[2 + j] = (uint8_t)q;
        if (j == 0) {
            blk[0] = (uint8_t)(dbits & 0xff);
            blk[1] = (uint8_t)(dbits >> 8);
        }
    }
}

// h = gelu(gate) * up for rows of 2*ff, then Q8_0 per 32-block: one block per half-wave.
__global__ __launch_bounds__(256) void k_geglu_q8_0(const float *__restrict__ gu, uint8_t *__restrict__ hq,
                                                    size_t nblocks, int ff) {
    const size_t gb = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    const bool ok = gb < nblocks;
    const int nbf = ff / QK;
    float h = 0.0f;
    if (ok) {
        size_t r = gb / nbf, b = gb % nbf;
        const float *row = gu + r * 2 * (size_t)ff;
        h = gelu(row[b * QK + j]) * row[ff + b * QK + j];
    }
    uint16_t dbits;
    int q = quant_q8_half(h, &dbits);
    if (ok) {
        uint8_t *blk = hq + gb * Q8_BLOCK;
        blk[2 + j] = (uint8_t)q;
        if (j == 0) {
            blk[0] = (uint8_t)(dbits & 0xff);
            blk[1] = (uint8_t)(dbits >> 8);
        }
    }
}

// Load the 32 quant bytes (8 dwords) and the scale of a Q8_0 block (2-byte aligned).
__device__ __forceinline__ float load_q8_block(const uint8_t *blk, uint32_t *q) {
    const uint16_t *h = (const uint16_t *)blk;
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = (uint32_t)h[1 + 2 * i] | ((uint32_t)h[2 + 2 * i] << 16);
    return h2f(h[0]);
}

// Generic packed GEMV/GEMM: one wave per (tile, token), each row's block terms folded in block
// order as the reference's dot_q8_scalar. RVM_PACK_GATE_UP lanes own whole rows; for
// RVM_PACK_ROWS32 the two half-waves own the two halves of each row's blocks, and their terms meet
// in LDS (terms[32][nb + 1], dynamic) for the fold. When sums != nullptr (n_in == 1) the per-block
// int32 sums are stored instead of y.
__global__ __launch_bounds__(64) void k_q4q8_generic(const uint4 *__restrict__ nib, const uint16_t *__restrict__ scl,
                                                     const uint8_t *__restrict__ xq, float *__restrict__ y,
                                                     int32_t *__restrict__ sums, int n_out, int nb, int T, int S,
                                                     int format) {
    extern __shared__ float terms[];
    const int t = blockIdx.x, tok = blockIdx.y, l = threadIdx.x;
    const uint8_t *xrow = xq + (size_t)tok * nb * Q8_BLOCK;
    float acc = 0.0f;
    int row = 0;
    for (int s = 0; s < S; ++s) {
        int b;
        if (format == RVM_PACK_GATE_UP) {
            row = l < 32 ? 32 * t + l : n_out / 2 + 32 * t + (l - 32);
            b = s;
        } else {
            row = 32 * t + (l & 31);
            b = (l >> 5) * S + s;
        }
        const size_t e = ((size_t)t * S + s) * 64 + l;
        uint32_t q[8], a[8];
        const float dx = load_q8_block(xrow + (size_t)b * Q8_BLOCK, q);
        prep_from_q8(q, a);
        const int sumi = block_dot(nib[e], a);
        if (sums) sums[(size_t)row * nb + b] = sumi;
        const float term = block_term(sumi, h2f(scl[e]), dx);
        if (format == RVM_PACK_GATE_UP)
            acc = acc + term;
        else
            terms[(l & 31) * (nb + 1) + b] = term;
    }
    if (sums) return;
    if (format == RVM_PACK_ROWS32) {
        __syncthreads();
        if (l < 32) {
            for (int b = 0; b < nb; ++b) acc = acc + terms[l * (nb + 1) + b];
            y[(size_t)tok * n_out + row] = acc;
        }
    } else {
        y[(size_t)tok * n_out + row] = acc;
    }
}

static bool geo(int n_out, int k, int format, int *T, int *S) {
    if (n_out <= 0 || k <= 0 || k % QK) return false;
    const int nb = k / QK;
    if (format == RVM_PACK_GATE_UP) {
        if (n_out % 64) return false;
        *T = n_out / 64;
        *S = nb;
        return true;
    }
    if (format == RVM_PACK_ROWS32) {
        if (n_out % 32 || nb % 2 || nb > 256) return false;
        *T = n_out / 32;
        *S = nb / 2;
        return true;
    }
    return false;
}

}  // namespace rvm

using namespace rvm;

extern "C" {

int rvm_quantize_q8_0(const float *x, void *xq, int rows, int k) {
    RVM_CHECK(x && xq && rows > 0 && k > 0 && k % QK == 0);
    size_t nblocks = (size_t)rows * (k / QK);
    hipLaunchKernelGGL(k_quantize_q8_0, dim3(grid_blocks(nblocks, 8)), dim3(256), 0, cur_stream(), x, (uint8_t *)xq,
                       nblocks);
    return launched();
}

int rvm_geglu_q8_0(const float *gu, void *hq, int rows, int ff) {
    RVM_CHECK(gu && hq && rows > 0 && ff > 0 && ff % QK == 0);
    size_t nblocks = (size_t)rows * (ff / QK);
    hipLaunchKernelGGL(k_geglu_q8_0, dim3(grid_blocks(nblocks, 8)), dim3(256), 0, cur_stream(), gu, (uint8_t *)hq,
                       nblocks, ff);
    return launched();
}

int rvm_q4q8_mm(const void *w_packed, int format, const void *xq, float *y, int n_out, int k, int n_in) {
    int T, S;
    RVM_CHECK(w_packed && xq && y && n_in > 0 && n_in <= 65535 && geo(n_out, k, format, &T, &S));
    const size_t entries = (size_t)n_out * (k / QK);
    const uint4 *nib = (const uint4 *)w_packed;
    const uint16_t *scl = (const uint16_t *)((const uint8_t *)w_packed + entries * 16);
    const size_t smem = format == RVM_PACK_ROWS32 ? (size_t)32 * (k / QK + 1) * 4 : 0;
    hipLaunchKernelGGL(k_q4q8_generic, dim3(T, n_in), dim3(64), smem, cur_stream(), nib, scl, (const uint8_t *)xq, y,
                       (int32_t *)nullptr, n_out, k / QK, T, S, format);
    return launched();
}

int rvm_q4q8_block_sums(const void *w_packed, int format, const void *xq, int32_t *sums, int n_out, int k) {
    int T, S;
    RVM_CHECK(w_packed && xq && sums && geo(n_out, k, format, &T, &S));
    const size_t entries = (size_t)n_out * (k / QK);
    const uint4 *nib = (const uint4 *)w_packed;
    const uint16_t *scl = (const uint16_t *)((const uint8_t *)w_packed + entries * 16);
    const size_t smem = format == RVM_PACK_ROWS32 ? (size_t)32 * (k / QK + 1) * 4 : 0;
    hipLaunchKernelGGL(k_q4q8_generic, dim3(T, 1), dim3(64), smem, cur_stream(), nib, scl, (const uint8_t *)xq,
                       (float *)nullptr, sums, n_out, k / QK, T, S, format);
    return launched();
}

}  // extern "C"
