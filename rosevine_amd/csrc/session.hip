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
    // Range evaluation: the layer the next range must start at (0: a new evaluation) and the token
    // count of the evaluation in progress.
    int next = 0, n_tok = 0;
    // Span events (instrumentation, off when empty): 2 per layer, recorded on the current stream
    // before the layer's router work and before its expert work, then one after the last layer.
    std::vector<hipEvent_t> probe;
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

int rvm_session_eval_range(rvm_session *s, const float *x, float *out, int n_tok, int flags, int l0, int l1) {
    RVM_CHECK(s && n_tok > 0 && n_tok <= s->max_tokens);
    RVM_CHECK((flags & ~RVM_EXACT_SELECT) == 0);
    const int n = (int)s->layers.size();
    RVM_CHECK(l0 >= 0 && l0 < l1 && l1 <= n);
    // A range continues the evaluation in progress: it starts where the previous range ended, with
    // the same tokens; only a range from layer 0 starts a new one (and needs x), and only the range
    // that ends at the last layer writes out.
    RVM_CHECK(l0 == 0 ? x != nullptr : (l0 == s->next && n_tok == s->n_tok));
    RVM_CHECK(l1 < n || out != nullptr);
    const bool probe = !s->probe.empty();
    for (int l = l0; l < l1; ++l) {
        const float *in = l == 0 ? x : s->buf[(l - 1) & 1];
        float *dst = l == n - 1 ? out : s->buf[l & 1];
        const rvm_layer *L = &s->layers[l];
        if (probe) {
            if (int rc = record_event(s->probe[2 * l])) return rc;
            span_mark_after_router(s->probe[2 * l + 1]);
        }
        int rc;
        if (!s->norms.empty()) {
            const rvm_block_norms &nm = s->norms[l];
            const XForm xf{1, nm.eps, nm.router_post, nm.router_scale, nm.expert_scale};
            rc = moe_forward(L, in, dst, n_tok, flags, xf, s->ws, s->ws_bytes, true);
        } else {
            const int f = flags | (l > 0 ? RVM_PRE_NORM : 0);
            rc = moe_forward(L, in, dst, n_tok, f, xform_of_flags(f, s->eps), s->ws, s->ws_bytes, true);
        }
        span_mark_after_router(nullptr);
        if (rc) {
            s->next = 0;
            return rc;
        }
    }
    if (probe && l1 == n)
        if (int rc = record_event(s->probe[2 * n])) return rc;
    s->next = l1 == n ? 0 : l1;
    s->n_tok = n_tok;
    return 0;
}

int rvm_session_eval(rvm_session *s, const float *x, float *out, int n_tok, int flags) {
    RVM_CHECK(s && x && out);
    return rvm_session_eval_range(s, x, out, n_tok, flags, 0, (int)s->layers.size());
}

int rvm_session_probe(rvm_session *s, void *const *events, int n_events) {
    RVM_CHECK(s);
    if (!events) {
        s->probe.clear();
        return 0;
    }
    RVM_CHECK(n_events == 2 * (int)s->layers.size() + 1);
    for (int i = 0; i < n_events; ++i) RVM_CHECK(events[i] != nullptr);
    s->probe.assign((hipEvent_t const *)events, (hipEvent_t const *)events + n_events);
    return 0;
}

}  // extern "C"
