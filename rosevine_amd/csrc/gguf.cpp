// gguf.cpp - GGUF v3 reading and the device binding of a layer's MoE tensors (host code).
//
// The reader follows the reference's bounded, zero-copy parser (runtime/src/gguf.rs:21-41,
// 217-340): a little-endian header, metadata key/value pairs, tensor descriptors, then a data
// section aligned to general.alignment (32 by default). Every size read from the file is bounded
// before use, every length and offset addition is checked for overflow, only F32 and Q4_0 tensors
// are accepted, and a malformed image is refused with the reference's own message for the same
// fault (its Error::Malformed strings), readable through rvm_gguf_last_error. Tensor views point
// into the caller's image; nothing is copied.
//
// The binding takes blk.L.ffn_gate_up_exps.weight [d, 2ff, n_exp] and blk.L.ffn_down_exps.weight
// [ff, d, n_exp] (ggml order, dimension 0 contiguous: n_exp matrices of Q4_0 rows; contract.rs:
// 66-70, model.rs:33-40), uploads each through a staging buffer and repacks it into the layer's
// planar layout (rvm_pack_q4), and copies the F32 router blk.L.ffn_gate_inp.weight [d, n_exp]
// (rows of d, one per expert) and, when the layer has a down-scale buffer, ffn_down_exps.scale.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/rvmoe.h"

namespace {

constexpr uint64_t MAX_KV = 65536, MAX_TENSORS = 65536, MAX_ARRAY_LEN = 4194304;
constexpr uint64_t MAX_STRING_LEN = 16ull << 20;
constexpr uint32_t MAX_ALIGNMENT = 1u << 20, DEFAULT_ALIGNMENT = 32;
constexpr uint32_t T_F32 = 0, T_Q4_0 = 2;

thread_local std::string g_last_error;

struct Fail {
    const char *msg;
};

struct TensorView {
    uint32_t type;
    std::vector<uint64_t> shape;
    uint64_t offset, bytes;
    const uint8_t *data;
};

// Reads from [buf, buf + size) with every bound checked (a Fail names the reference's message).
struct Reader {
    const uint8_t *buf;
    uint64_t size, pos = 0;
    const uint8_t *take(uint64_t n) {
        if (n > size - pos) throw Fail{n > (uint64_t)-1 - pos ? "length overflow" : "truncated header"};
        const uint8_t *p = buf + pos;
        pos += n;
        return p;
    }
    template <class T>
    T num() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));  // little-endian host
        return v;
    }
    std::string str() {
        const uint64_t n = num<uint64_t>();
        if (n > MAX_STRING_LEN) throw Fail{"string length limit exceeded"};
        const uint8_t *p = take(n);
        if (!utf8_ok(p, n)) throw Fail{"string is not UTF-8"};
        return std::string((const char *)p, n);
    }
    static bool utf8_ok(const uint8_t *s, uint64_t n) {
        for (uint64_t i = 0; i < n;) {
            const uint8_t c = s[i];
            int len;
            uint32_t cp;
            if (c < 0x80) {
                ++i;
                continue;
            } else if ((c & 0xE0) == 0xC0) {
                len = 2, cp = c & 0x1F;
            } else if ((c & 0xF0) == 0xE0) {
                len = 3, cp = c & 0x0F;
            } else if ((c & 0xF8) == 0xF0) {
                len = 4, cp = c & 0x07;
            } else {
                return false;
            }
            if (n - i < (uint64_t)len) return false;
            for (int k = 1; k < len; ++k) {
                if ((s[i + k] & 0xC0) != 0x80) return false;
                cp = (cp << 6) | (s[i + k] & 0x3F);
            }
            // no overlong forms, no surrogates, nothing past U+10FFFF
            if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
                (cp >= 0xD800 && cp <= 0xDFFF) || cp > 0x10FFFF)
                return false;
            i += len;
        }
        return true;
    }
};

// Bytes of a scalar metadata type (0 when the id is not a scalar).
uint64_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;   // u8 i8 bool
        case 2: case 3: return 2;           // u16 i16
        case 4: case 5: case 6: return 4;   // u32 i32 f32
        case 10: case 11: case 12: return 8;  // u64 i64 f64
        default: return 0;
    }
}

struct Meta {
    uint32_t type;
    bool is_int = false;
    __int128 ival = 0;  // integer scalars
    std::string sval;   // strings
};

Meta read_value(Reader &r, uint32_t t) {
    Meta m;
    m.type = t;
    if (const uint64_t sz = scalar_size(t)) {
        const uint8_t *p = r.take(sz);
        switch (t) {
            case 0: m.ival = p[0]; m.is_int = true; break;
            case 1: m.ival = (int8_t)p[0]; m.is_int = true; break;
            case 2: { uint16_t v; std::memcpy(&v, p, 2); m.ival = v; m.is_int = true; break; }
            case 3: { int16_t v; std::memcpy(&v, p, 2); m.ival = v; m.is_int = true; break; }
            case 4: { uint32_t v; std::memcpy(&v, p, 4); m.ival = v; m.is_int = true; break; }
            case 5: { int32_t v; std::memcpy(&v, p, 4); m.ival = v; m.is_int = true; break; }
            case 10: { uint64_t v; std::memcpy(&v, p, 8); m.ival = v; m.is_int = true; break; }
            case 11: { int64_t v; std::memcpy(&v, p, 8); m.ival = v; m.is_int = true; break; }
            case 7: if (p[0] > 1) throw Fail{"invalid bool"}; break;
            default: break;  // f32, f64
        }
        return m;
    }
    if (t == 8) {
        m.sval = r.str();
        return m;
    }
    if (t == 9) {
        const uint32_t elem = r.num<uint32_t>();
        const uint64_t count = r.num<uint64_t>();
        if (count > MAX_ARRAY_LEN) throw Fail{"array length limit exceeded"};
        if (const uint64_t sz = scalar_size(elem)) {
            const uint8_t *p = r.take(count * sz);  // count * sz < 2^26: no overflow
            if (elem == 7)
                for (uint64_t i = 0; i < count; ++i)
                    if (p[i] > 1) throw Fail{"invalid bool"};
        } else if (elem == 8) {
            // each string takes at least its 8-byte length: bound the count by what is left
            if (count > (r.size - r.pos) / 8) throw Fail{"truncated header"};
            for (uint64_t i = 0; i < count; ++i) r.str();
        } else {
            throw Fail{"unsupported array element type"};
        }
        return m;
    }
    throw Fail{"unsupported metadata type"};
}

}  // namespace

struct rvm_gguf {
    uint32_t version = 0, alignment = DEFAULT_ALIGNMENT;
    uint64_t data_offset = 0;
    std::map<std::string, Meta> meta;
    std::vector<std::pair<std::string, TensorView>> tensors;  // file order
    std::map<std::string, size_t> index;
};

namespace {

void parse(const uint8_t *buf, uint64_t size, rvm_gguf &g) {
    Reader r{buf, size};
    if (std::memcmp(r.take(4), "GGUF", 4) != 0) throw Fail{"bad magic"};
    g.version = r.num<uint32_t>();
    if (g.version != 3) throw Fail{"expected GGUF version 3"};
    const uint64_t n_tensors = r.num<uint64_t>(), n_kv = r.num<uint64_t>();
    if (n_tensors == 0 || n_tensors > MAX_TENSORS || n_kv > MAX_KV) throw Fail{"descriptor count limit exceeded"};
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.str();
        if (key.empty()) throw Fail{"empty metadata key"};
        const uint32_t t = r.num<uint32_t>();
        Meta v = read_value(r, t);
        if (!g.meta.emplace(std::move(key), std::move(v)).second) throw Fail{"duplicate metadata key"};
    }
    if (auto it = g.meta.find("general.alignment"); it != g.meta.end()) {
        const Meta &a = it->second;
        if (!a.is_int || a.ival < 1 || a.ival > MAX_ALIGNMENT || (a.ival & (a.ival - 1)) != 0)
            throw Fail{"invalid alignment"};
        g.alignment = (uint32_t)a.ival;
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        std::string name = r.str();
        if (name.empty() || g.index.count(name)) throw Fail{"empty or duplicate tensor name"};
        const uint32_t n_dims = r.num<uint32_t>();
        if (n_dims < 1 || n_dims > 4) throw Fail{"invalid tensor rank"};
        TensorView tv;
        for (uint32_t k = 0; k < n_dims; ++k) tv.shape.push_back(r.num<uint64_t>());
        tv.type = r.num<uint32_t>();
        if (tv.type != T_F32 && tv.type != T_Q4_0) throw Fail{"unsupported tensor type"};
        tv.offset = r.num<uint64_t>();
        const uint64_t block = tv.type == T_Q4_0 ? 32 : 1, block_bytes = tv.type == T_Q4_0 ? 18 : 4;
        if (std::find(tv.shape.begin(), tv.shape.end(), 0ull) != tv.shape.end() || tv.shape[0] % block != 0)
            throw Fail{"invalid tensor shape"};
        uint64_t elems = 1;
        for (uint64_t dim : tv.shape) {
            if (__builtin_mul_overflow(elems, dim, &elems)) throw Fail{"tensor element count overflow"};
        }
        if (elems >= (1ull << 62)) throw Fail{"tensor element count overflow"};
        if (__builtin_mul_overflow(elems / block, block_bytes, &tv.bytes)) throw Fail{"tensor size overflow"};
        if (tv.offset % g.alignment != 0) throw Fail{"misaligned tensor offset"};
        g.index.emplace(name, g.tensors.size());
        g.tensors.emplace_back(std::move(name), std::move(tv));
    }
    const uint64_t a = g.alignment;
    if (r.pos > (uint64_t)-1 - (a - 1)) throw Fail{"length overflow"};
    g.data_offset = (r.pos + a - 1) / a * a;
    if (g.data_offset > size) throw Fail{"truncated before data section"};
    std::vector<size_t> order(g.tensors.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = i;
    std::sort(order.begin(), order.end(),
              [&](size_t x, size_t y) { return g.tensors[x].second.offset < g.tensors[y].second.offset; });
    uint64_t end = 0;
    for (size_t i : order) {
        TensorView &t = g.tensors[i].second;
        uint64_t stop, abs;
        if (__builtin_add_overflow(t.offset, t.bytes, &stop)) throw Fail{"tensor range overflow"};
        if (t.offset < end || __builtin_add_overflow(g.data_offset, stop, &abs) || abs > size)
            throw Fail{"overlapping or out-of-file tensor range"};
        end = stop;
        t.data = buf + g.data_offset + t.offset;
    }
}

int fail(const char *msg) {
    g_last_error = msg;
    return (int)hipErrorInvalidValue;
}

const TensorView *find(const rvm_gguf *g, const std::string &name) {
    auto it = g->index.find(name);
    return it == g->index.end() ? nullptr : &g->tensors[it->second].second;
}

}  // namespace

extern "C" {

int rvm_gguf_open(const void *data, size_t size, rvm_gguf **out) {
    if (!out) return fail("null argument");
    *out = nullptr;
    if (!data && size) return fail("null argument");
    rvm_gguf *g = new (std::nothrow) rvm_gguf;
    if (!g) return (int)hipErrorOutOfMemory;
    try {
        parse((const uint8_t *)data, size, *g);
    } catch (const Fail &f) {
        delete g;
        return fail(f.msg);
    } catch (const std::bad_alloc &) {
        delete g;
        return (int)hipErrorOutOfMemory;
    }
    *out = g;
    return 0;
}

int rvm_gguf_close(rvm_gguf *g) {
    delete g;
    return 0;
}

const char *rvm_gguf_last_error(void) { return g_last_error.c_str(); }

int rvm_gguf_info(const rvm_gguf *g, uint32_t *version, uint32_t *alignment, uint64_t *data_offset,
                  uint64_t *n_tensors) {
    if (!g || !version || !alignment || !data_offset || !n_tensors) return fail("null argument");
    *version = g->version;
    *alignment = g->alignment;
    *data_offset = g->data_offset;
    *n_tensors = g->tensors.size();
    return 0;
}

int rvm_gguf_meta_str(const rvm_gguf *g, const char *key, const char **value) {
    if (!g || !key || !value) return fail("null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end() || it->second.type != 8) return fail("missing string metadata");
    *value = it->second.sval.c_str();
    return 0;
}

int rvm_gguf_tensor(const rvm_gguf *g, const char *name, uint32_t *type, uint32_t *n_dims, uint64_t shape[4],
                    const void **data, size_t *bytes) {
    if (!g || !name || !type || !n_dims || !shape || !data || !bytes) return fail("null argument");
    const TensorView *t = find(g, name);
    if (!t) return fail("missing tensor");
    *type = t->type;
    *n_dims = (uint32_t)t->shape.size();
    for (int k = 0; k < 4; ++k) shape[k] = k < (int)t->shape.size() ? t->shape[k] : 1;
    *data = t->data;
    *bytes = (size_t)t->bytes;
    return 0;
}

int rvm_gguf_bind_moe(const rvm_gguf *g, int layer, const rvm_layer *dst, void *staging, size_t staging_bytes) {
    if (!g || !dst || !staging || layer < 0 || !dst->gate_up || !dst->down || !dst->router)
        return fail("null argument");
    const uint64_t E = (uint64_t)dst->n_exp, d = (uint64_t)dst->d, ff = (uint64_t)dst->ff;
    const std::string p = "blk." + std::to_string(layer) + ".";
    struct Want {
        const char *name;
        uint32_t type;
        std::vector<uint64_t> shape;
    };
    const Want gu{"ffn_gate_up_exps.weight", T_Q4_0, {d, 2 * ff, E}};
    const Want dn{"ffn_down_exps.weight", T_Q4_0, {ff, d, E}};
    const Want rt{"ffn_gate_inp.weight", T_F32, {d, E}};
    const Want sc{"ffn_down_exps.scale", T_F32, {E}};
    auto get = [&](const Want &w) -> const TensorView * {
        const TensorView *t = find(g, p + w.name);
        if (!t) throw Fail{"missing tensor"};
        if (t->type != w.type || t->shape != w.shape) throw Fail{"tensor shape or type mismatch"};
        return t;
    };
    try {
        const TensorView *tg = get(gu), *td = get(dn), *tr = get(rt);
        const TensorView *ts = dst->down_scale ? get(sc) : nullptr;
        if (staging_bytes < std::max(tg->bytes, td->bytes)) throw Fail{"staging buffer too small"};
        // one expert tensor at a time: upload, repack (in stream order), then the next upload
        int rc = rvh_upload(staging, tg->data, tg->bytes);
        if (!rc) rc = rvm_pack_q4(staging, (void *)dst->gate_up, dst->n_exp, 2 * dst->ff, dst->d, RVM_PACK_GATE_UP);
        if (!rc) rc = rvh_sync();
        if (!rc) rc = rvh_upload(staging, td->data, td->bytes);
        if (!rc) rc = rvm_pack_q4(staging, (void *)dst->down, dst->n_exp, dst->d, dst->ff, RVM_PACK_ROWS32);
        if (!rc) rc = rvh_upload((void *)dst->router, tr->data, tr->bytes);
        if (!rc && ts) rc = rvh_upload((void *)dst->down_scale, ts->data, ts->bytes);
        if (!rc) rc = rvh_sync();
        return rc;
    } catch (const Fail &f) {
        return fail(f.msg);
    }
}

}  // extern "C"
