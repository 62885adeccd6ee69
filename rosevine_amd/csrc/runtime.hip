// runtime.hip - runtime, memory, events, streams/graphs, weight packing and synthetic weights.
// The rvh_* symbols keep the meaning of the reference's runtime/hip/rvhip.h:22-38
// (runtime/hip/rvhip.hip:449-509); transfers and events use the library's current stream so that
// they stay ordered with the kernels issued there.
#include "internal.hpp"

namespace rvm {

static thread_local hipStream_t g_stream = nullptr;
// Device calls issued by this thread (the reference's per-thread Counters, runtime/src/hip.rs:167-187).
static thread_local rvm_counters g_count{};

hipStream_t cur_stream() { return g_stream; }

static thread_local hipEvent_t g_span = nullptr;

// A failed runtime call leaves its code as the thread's last error, which the next launch check
// (hipGetLastError in launched()) would report as its own: return the code and clear it.
int api_status(hipError_t e) {
    if (e != hipSuccess) (void)hipGetLastError();
    return (int)e;
}

// Records e on the current stream; under stream capture as an event node of the graph (the
// external-event form, whose timestamps hipEventElapsedTime reads after a replay).
int record_event(hipEvent_t e) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (int rc = api_status(hipStreamIsCapturing(g_stream, &st))) return rc;
    const unsigned flags = st == hipStreamCaptureStatusActive ? hipEventRecordExternal : 0u;
    return api_status(hipEventRecordWithFlags(e, g_stream, flags));
}

void span_mark_after_router(hipEvent_t e) { g_span = e; }

int span_router_done() {
    if (!g_span) return 0;
    const hipEvent_t e = g_span;
    g_span = nullptr;
    return record_event(e);
}

int launched() {
    ++g_count.launches;
    return (int)hipGetLastError();
}

// LDS a workgroup may allocate on the current device, capped at the 64 KiB that needs no
// per-kernel attribute.
int max_lds_per_block() {
    static int v = 0;
    if (!v) {
        int dev = 0, x = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&x, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || x <= 0)
            x = 65536;
        v = x < 65536 ? x : 65536;
    }
    return v;
}

// ---- synthetic Q4_0 weights: a counter-based generator, identical on host and device ----

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t synth_key(uint64_t seed, uint64_t stream) {
    return splitmix64(splitmix64(seed) ^ splitmix64(stream ^ 0xD1B54A32D192ED03ull));
}

// Block i of a stream: scale f16(0.005 + 0.015 * u), u a 24-bit uniform in [0, 1) (the multiply
// and the add each round once: the build uses -ffp-contract=off), then 16 uniform nibble bytes.
__host__ __device__ __forceinline__ void synth_block(uint64_t key, uint64_t i, uint8_t *out) {
    uint64_t r0 = splitmix64(key + 3 * i), r1 = splitmix64(key + 3 * i + 1), r2 = splitmix64(key + 3 * i + 2);
    float u = (float)(uint32_t)(r2 >> 40) * 0x1p-24f;
    float scaled = 0.015f * u;
    float d = 0.005f + scaled;
    uint16_t h = f2h_rne(d);
    out[0] = (uint8_t)(h & 0xff);
    out[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 8; ++j) {
        out[2 + j] = (uint8_t)(r0 >> (8 * j));
        out[10 + j] = (uint8_t)(r1 >> (8 * j));
    }
}

__global__ void k_synth_q4(uint8_t *dst, size_t blocks_per_mat, size_t n_blocks, uint64_t seed, uint64_t stream0) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    size_t m = i / blocks_per_mat, b = i % blocks_per_mat;
    uint8_t blk[18];
    synth_block(synth_key(seed, stream0 + m), b, blk);
    uint16_t *o = (uint16_t *)(dst + i * Q4_BLOCK);  // blocks are 18 B: 2-byte aligned
    for (int j = 0; j < 9; ++j) o[j] = (uint16_t)(blk[2 * j] | (blk[2 * j + 1] << 8));
}

// ---- packing: Q4_0 rows -> wave-interleaved nibble and scale planes ----

struct PackGeo {
    int rt;  // rows per tile
    int T;   // tiles per matrix
    int S;   // steps per lane
    int nb;  // blocks per row
};

static bool pack_geo(int n_out, int k, int format, PackGeo *g) {
    if (n_out <= 0 || k <= 0 || k % QK) return false;
    g->nb = k / QK;
    if (format == RVM_PACK_GATE_UP) {
        if (n_out % 64) return false;
        g->rt = 64;
        g->S = g->nb;
    } else if (format == RVM_PACK_ROWS32) {
        if (n_out % 32 || g->nb % 2) return false;
        g->rt = 32;
        g->S = g->nb / 2;
    } else {
        return false;
    }
    g->T = n_out / g->rt;
    return true;
}

// Source row and block of plane entry (tile t, step s, lane l) within one matrix.
__device__ __forceinline__ void pack_src(int format, int n_out, int t, int s, int l, int S, int *row, int *blk) {
    if (format == RVM_PACK_GATE_UP) {
        *row = l < 32 ? 32 * t + l : n_out / 2 + 32 * t + (l - 32);
        *blk = s;
    } else {
        *row = 32 * t + (l & 31);
        *blk = (l >> 5) * S + s;
    }
}

__global__ void k_pack_q4(const uint8_t *src, uint4 *nib, uint16_t *scl, size_t entries, int n_out, int nb, int T,
                          int S, int format) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= entries) return;
    int l = (int)(i & 63);
    size_t ts = i >> 6;  // (m * T + t) * S + s
    int s = (int)(ts % S);
    size_t mt = ts / S;
    int t = (int)(mt % T);
    size_t m = mt / T;
    int row, blk;
    pack_src(format, n_out, t, s, l, S, &row, &blk);
    const uint8_t *b = src + ((m * n_out + row) * (size_t)nb + blk) * Q4_BLOCK;
    const uint16_t *h = (const uint16_t *)b;  // 2-byte aligned
    uint32_t q[4];
    for (int j = 0; j < 4; ++j) q[j] = ((uint32_t)h[1 + 2 * j] | ((uint32_t)h[2 + 2 * j] << 16)) ^ 0x88888888u;
    nib[i] = make_uint4(q[0], q[1], q[2], q[3]);
    scl[i] = h[0];
}

__global__ void k_fill_u32(uint32_t *p, size_t n, uint32_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace rvm

using namespace rvm;

extern "C" {

int rvh_init(int device) {
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return (int)e;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return (int)e;
    // The kernels are wave64 code for CDNA: refuse any other wave size instead of misbehaving.
    if (prop.warpSize != 64) return (int)hipErrorInvalidDevice;
    return rvm::static_scratch_setup(device);
}

int rvh_mem_info(size_t *free_bytes, size_t *total_bytes) {
    RVM_CHECK(free_bytes && total_bytes);
    return (int)hipMemGetInfo(free_bytes, total_bytes);
}

int rvh_alloc(size_t bytes, void **out) {
    RVM_CHECK(out);
    *out = nullptr;
    return (int)hipMalloc(out, bytes ? bytes : 1);
}

int rvh_free(void *ptr) { return ptr ? (int)hipFree(ptr) : 0; }

int rvh_upload(void *dst, const void *src, size_t bytes) {
    RVM_CHECK(dst && src);
    ++g_count.h2d;  // a transfer, not a counted sync (the reference counts only explicit syncs)
    RVM_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, cur_stream()));
    return (int)hipStreamSynchronize(cur_stream());
}

int rvh_download(void *dst, const void *src, size_t bytes) {
    RVM_CHECK(dst && src);
    ++g_count.d2h;
    RVM_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, cur_stream()));
    return (int)hipStreamSynchronize(cur_stream());
}

int rvh_copy(void *dst, const void *src, size_t bytes) {
    RVM_CHECK(dst && src);
    ++g_count.d2d;
    return (int)hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, cur_stream());
}

int rvh_sync(void) {
    ++g_count.syncs;
    return (int)hipDeviceSynchronize();
}

int rvm_counters_get(rvm_counters *c) {
    RVM_CHECK(c);
    *c = g_count;
    return 0;
}

int rvm_counters_reset(void) {
    g_count = rvm_counters{};
    return 0;
}

int rvm_phase_trace(void *host, size_t bytes) {
    constexpr size_t per = (size_t)TRACE_WG * TRACE_PT * sizeof(uint64_t);
    RVM_CHECK(host && bytes >= 3 * per);
    if (int rc = phase_trace_router(host)) return rc;
    return phase_trace_decode((uint8_t *)host + per);
}

const char *rvh_error_string(int code) { return hipGetErrorString((hipError_t)code); }

int rvh_event_create(void **out) {
    RVM_CHECK(out);
    hipEvent_t e = nullptr;
    hipError_t r = hipEventCreate(&e);
    *out = (void *)e;
    return (int)r;
}

int rvh_event_destroy(void *ev) { return ev ? (int)hipEventDestroy((hipEvent_t)ev) : 0; }

int rvh_event_record(void *ev) {
    RVM_CHECK(ev);
    return record_event((hipEvent_t)ev);
}

int rvh_event_sync(void *ev) {
    RVM_CHECK(ev);
    ++g_count.syncs;
    return (int)hipEventSynchronize((hipEvent_t)ev);
}

int rvh_event_elapsed(void *start, void *end, float *ms) {
    RVM_CHECK(start && end && ms);
    return (int)hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end);
}

int rvm_set_stream(void *stream) {
    g_stream = (hipStream_t)stream;
    return 0;
}

int rvm_stream_create(void **out) {
    RVM_CHECK(out);
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);  // default priority
    *out = (void *)s;
    return (int)e;
}

int rvm_stream_destroy(void *stream) { return stream ? (int)hipStreamDestroy((hipStream_t)stream) : 0; }

int rvm_graph_begin(void) {
    RVM_CHECK(cur_stream() != nullptr);
    return api_status(hipStreamBeginCapture(cur_stream(), hipStreamCaptureModeThreadLocal));
}

int rvm_graph_end(void **graph_exec) {
    RVM_CHECK(graph_exec && cur_stream() != nullptr);
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    if (int rc = api_status(hipStreamEndCapture(cur_stream(), &g))) return rc;
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return api_status(e);
    *graph_exec = (void *)ex;
    return 0;
}

int rvm_graph_launch(void *graph_exec) {
    RVM_CHECK(graph_exec);
    ++g_count.graphs;
    return api_status(hipGraphLaunch((hipGraphExec_t)graph_exec, cur_stream()));
}

int rvm_graph_destroy(void *graph_exec) {
    return graph_exec ? (int)hipGraphExecDestroy((hipGraphExec_t)graph_exec) : 0;
}

int rvm_q4_packed_bytes(int n_mat, int n_out, int k, int format, size_t *bytes) {
    PackGeo g;
    RVM_CHECK(bytes && n_mat > 0 && pack_geo(n_out, k, format, &g));
    *bytes = (size_t)n_mat * n_out * g.nb * Q4_BLOCK;
    return 0;
}

int rvm_pack_q4(const void *src, void *dst, int n_mat, int n_out, int k, int format) {
    PackGeo g;
    RVM_CHECK(src && dst && src != dst && n_mat > 0 && pack_geo(n_out, k, format, &g));
    size_t entries = (size_t)n_mat * n_out * g.nb;  // one per (row, block)
    uint4 *nib = (uint4 *)dst;
    uint16_t *scl = (uint16_t *)((uint8_t *)dst + entries * 16);
    hipLaunchKernelGGL(k_pack_q4, dim3(grid_blocks(entries, 256)), dim3(256), 0, cur_stream(), (const uint8_t *)src,
                       nib, scl, entries, n_out, g.nb, g.T, g.S, format);
    return launched();
}

int rvm_synth_q4(void *dst, int n_mat, int n_out, int k, uint64_t seed, uint64_t stream0) {
    RVM_CHECK(dst && n_mat > 0 && n_out > 0 && k > 0 && k % QK == 0);
    size_t per = (size_t)n_out * (k / QK), n = per * n_mat;
    hipLaunchKernelGGL(k_synth_q4, dim3(grid_blocks(n, 256)), dim3(256), 0, cur_stream(), (uint8_t *)dst, per, n,
                       seed, stream0);
    return launched();
}

int rvm_synth_q4_host(void *dst, int n_mat, int n_out, int k, uint64_t seed, uint64_t stream0) {
    RVM_CHECK(dst && n_mat > 0 && n_out > 0 && k > 0 && k % QK == 0);
    size_t per = (size_t)n_out * (k / QK);
    uint8_t *o = (uint8_t *)dst;
    for (int m = 0; m < n_mat; ++m) {
        uint64_t key = synth_key(seed, stream0 + (uint64_t)m);
        for (size_t b = 0; b < per; ++b) synth_block(key, b, o + ((size_t)m * per + b) * Q4_BLOCK);
    }
    return 0;
}

int rvm_moe_workspace_bytes(const rvm_layer *layer, int n_tok, size_t *bytes) {
    RVM_CHECK(bytes && layer_ok(layer) && n_tok > 0);
    *bytes = ws_layout(layer, n_tok).total;
    return 0;
}

int rvm_workspace_init(void *ws, size_t bytes) {
    RVM_CHECK(ws && bytes % 4 == 0);
    size_t n = bytes / 4;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_blocks(n, 256)), dim3(256), 0, cur_stream(), (uint32_t *)ws, n, 0u);
    return launched();
}

int rvm_workspace_fallbacks(const void *ws, uint32_t *count) {
    RVM_CHECK(ws && count);
    return rvh_download(count, ws, 4);
}

int rvm_workspace_selection(const rvm_layer *layer, int n_tok, const void *ws, int32_t *ids, float *weights) {
    RVM_CHECK(layer_ok(layer) && n_tok > 0 && ws && ids && weights);
    const WsLayout lay = ws_layout(layer, n_tok);
    const size_t n = (size_t)n_tok * layer->top_k * 4;
    int rc = rvh_download(ids, (const uint8_t *)ws + lay.ids, n);
    return rc ? rc : rvh_download(weights, (const uint8_t *)ws + lay.wts, n);
}

}  // extern "C"
