// session.hip - a stack of MoE layers evaluated on the device with no host round trip.
//
// The reference's executor runs each layer's MoE block with a blocking router-logits download, host
// selection and four metadata uploads per layer (runtime/src/hip_exec.rs:780-843; its device calls
// are counted by hand in runtime/tests/exec.rs:521-543). A session here owns one workspace and two
// activation buffers for n layers of one shape and issues, per layer, only the kernels of one
// rvm_moe_* call: layer l reads the previous layer's output from device memory, so a token crosses
// the whole stack without a synchronisation, a transfer or a host decision, and the whole evaluation
// can be captured in one graph.
//
// Between layers the session applies either the synthetic stack's RMSNorm (eps; layer 0 takes its
// input as is) or, with per-layer block norms, each layer's own router and expert norms of the
// reference's MoE block (rvm_moe_block_*).
#include <cmath>
#include <vector>

#include "internal.hpp"

struct rvm_session {
    std::vector<rvm_layer> layers;
    std::vector<rvm_block_norms> norms;  // empty: the RMSNorm stack
    int max_tokens = 0;
    float eps = 0.0f;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    float *buf[2] = {nullptr, nullptr};
};

namespace {

bool same_shape(const rvm_layer &a, const rvm_layer &b) {
    return a.n_exp == b.n_exp && a.top_k == b.top_k && a.d == b.d && a.ff == b.ff;
}

void release(rvm_session *s) {
    if (!s) return;
    if (s->ws) (void)hipFree(s->ws);
    for (float *b : s->buf)
        if (b) (void)hipFree(b);
    delete s;
}

}  // namespace

using namespace rvm;

extern "C" {

int rvm_session_create(const rvm_layer *layers, int n_layers, const rvm_block_norms *norms, int max_tokens,
                       float eps, rvm_session **out) {
    RVM_CHECK(out && layers && n_layers > 0 && max_tokens > 0 && max_tokens <= MAX_TOKENS && eps >= 0.0f);
    *out = nullptr;
    for (int l = 0; l < n_layers; ++l) RVM_CHECK(layer_ok(&layers[l]) && same_shape(layers[l], layers[0]));
    if (norms)
        for (int l = 0; l < n_layers; ++l) RVM_CHECK(norms[l].eps >= 0.0f && std::isfinite(norms[l].router_post));
    rvm_session *s = new (std::nothrow) rvm_session;
    if (!s) return (int)hipErrorOutOfMemory;
    s->layers.assign(layers, layers + n_layers);
    if (norms) s->norms.assign(norms, norms + n_layers);
    s->max_tokens = max_tokens;
    s->eps = eps;
    s->ws_bytes = ws_layout(&layers[0], max_tokens).total;
    const size_t act = (size_t)max_tokens * layers[0].d * sizeof(float);
    int rc = (int)hipMalloc(&s->ws, s->ws_bytes);
    if (!rc) rc = (int)hipMalloc((void **)&s->buf[0], act);
    if (!rc) rc = (int)hipMalloc((void **)&s->buf[1], act);
    if (!rc) rc = rvm_workspace_init(s->ws, s->ws_bytes);
    if (!rc) rc = (int)hipStreamSynchronize(cur_stream());
    if (rc) {
        release(s);
        return rc;
    }
    *out = s;
    return 0;
}

int rvm_session_destroy(rvm_session *s) {
    if (s) (void)hipStreamSynchronize(cur_stream());
    release(s);
    return 0;
}

int rvm_session_workspace(const rvm_session *s, const void **ws) {
    RVM_CHECK(s && ws);
    *ws = s->ws;
    return 0;
}

int rvm_session_eval(rvm_session *s, const float *x, float *out, int n_tok, int flags) {
    RVM_CHECK(s && x && out && n_tok > 0 && n_tok <= s->max_tokens);
    RVM_CHECK((flags & ~RVM_EXACT_SELECT) == 0);
    const int n = (int)s->layers.size();
    for (int l = 0; l < n; ++l) {
        const float *in = l == 0 ? x : s->buf[(l - 1) & 1];
        float *dst = l == n - 1 ? out : s->buf[l & 1];
        const rvm_layer *L = &s->layers[l];
        int rc;
        if (!s->norms.empty()) {
            const rvm_block_norms &nm = s->norms[l];
            const XForm xf{1, nm.eps, nm.router_post, nm.router_scale, nm.expert_scale};
            rc = moe_forward(L, in, dst, n_tok, flags, xf, s->ws, s->ws_bytes);
        } else {
            const int f = flags | (l > 0 ? RVM_PRE_NORM : 0);
            rc = moe_forward(L, in, dst, n_tok, f, xform_of_flags(f, s->eps), s->ws, s->ws_bytes);
        }
        if (rc) return rc;
    }
    return 0;
}

}  // extern "C"
