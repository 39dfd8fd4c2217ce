// GGUF v3 model files (crates/model-formats/src/gguf.rs) behind the C ABI: the header index with
// the reference reader's validation, metadata and tensor lookups, tensor reads, and a generation
// session opened straight from a Gemma 4 file with the reference's layer assembly
// (crates/application/src/stack.rs:26-107, lib.rs:351-383, 661-709).  Host code only: tensors are
// read from a read-only memory mapping and copied to the device by af_session_open.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../../include/af.h"
#include "af_internal.h"

namespace {

using af::set_error;

// GGUF metadata value types
enum : uint32_t {
    T_U8 = 0, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64, T_F64, T_LAST = 12
};

struct Value {
    int32_t kind = AF_GGUF_UNSIGNED;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string text;
    uint32_t element_type = 0;
    uint64_t length = 0;
    std::vector<Value> items;  // AF_GGUF_ARRAY: arrays of at most kKeptArray elements are kept
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> dims;
    uint64_t offset = 0, bytes = 0;  // absolute file offset
};

constexpr uint64_t kHeaderBudget = 256ull << 20;   // bytes of header the reader accepts
constexpr uint64_t kMaxString = 16ull << 20;
constexpr uint64_t kMaxArray = 4000000;
constexpr uint64_t kKeptArray = 4096;               // larger arrays (the vocabulary) are summarised
constexpr uint64_t kMaxEntries = 100000;

// Weight types the reader knows, with (elements, bytes) per block (crates/domain/src/lib.rs:12-20).
bool block_layout(uint32_t type, uint64_t& block, uint64_t& bytes) {
    switch (type) {
        case AF_GGUF_F32: block = 1, bytes = 4; return true;
        case AF_GGUF_F16: block = 1, bytes = 2; return true;
        case AF_GGUF_Q4_0: block = 32, bytes = 18; return true;
        case AF_GGUF_Q8_0: block = 32, bytes = 34; return true;
        case AF_GGUF_Q6_K: block = 256, bytes = 210; return true;
        case AF_GGUF_BF16: block = 1, bytes = 2; return true;
        default: return false;
    }
}

bool valid_utf8(const std::string& s) {
    const size_t n = s.size();
    for (size_t i = 0; i < n;) {
        const unsigned char c = (unsigned char)s[i];
        size_t k;
        if (c < 0x80) k = 0;
        else if ((c >> 5) == 6) k = 1;
        else if ((c >> 4) == 14) k = 2;
        else if ((c >> 3) == 30) k = 3;
        else return false;
        if (n - i <= k) return false;
        for (size_t j = 1; j <= k; ++j)
            if (((unsigned char)s[i + j] >> 6) != 2) return false;
        i += k + 1;
    }
    return true;
}

// Sequential header reader over the mapped file, every read bounded by the file size and by the
// header budget.
struct Cursor {
    const uint8_t* base;
    uint64_t size, pos = 0, budget = kHeaderBudget;
    std::string err;

    bool take(uint64_t n) {
        if (!err.empty()) return false;
        if (n > budget) return fail("header above the 256 MiB limit");
        if (n > size - pos) return fail("file truncated");
        budget -= n;
        return true;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    template <typename T>
    bool get(T& v) {
        if (!take(sizeof(T))) return false;
        std::memcpy(&v, base + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool string(std::string& s, bool keep = true) {
        uint64_t n = 0;
        if (!get(n)) return false;
        if (n > kMaxString) return fail("invalid or excessive string length");
        if (!take(n)) return false;
        if (keep) s.assign(reinterpret_cast<const char*>(base + pos), n);
        pos += n;
        if (keep && !valid_utf8(s)) return fail("invalid UTF-8 string");
        return true;
    }
    bool value(uint32_t type, Value& v, bool keep) {
        switch (type) {
            case T_U8: { uint8_t x; if (!get(x)) return false; v.kind = AF_GGUF_UNSIGNED; v.u = x; return true; }
            case T_I8: { int8_t x; if (!get(x)) return false; v.kind = AF_GGUF_SIGNED; v.i = x; return true; }
            case T_U16: { uint16_t x; if (!get(x)) return false; v.kind = AF_GGUF_UNSIGNED; v.u = x; return true; }
            case T_I16: { int16_t x; if (!get(x)) return false; v.kind = AF_GGUF_SIGNED; v.i = x; return true; }
            case T_U32: { uint32_t x; if (!get(x)) return false; v.kind = AF_GGUF_UNSIGNED; v.u = x; return true; }
            case T_I32: { int32_t x; if (!get(x)) return false; v.kind = AF_GGUF_SIGNED; v.i = x; return true; }
            case T_F32: { float x; if (!get(x)) return false; v.kind = AF_GGUF_FLOAT; v.f = x; return true; }
            case T_BOOL: {
                uint8_t x;
                if (!get(x)) return false;
                if (x > 1) return fail("invalid boolean");
                v.kind = AF_GGUF_BOOL;
                v.u = x;
                return true;
            }
            case T_STRING: v.kind = AF_GGUF_TEXT; return string(v.text, keep);
            case T_ARRAY: {
                uint32_t et = 0;
                uint64_t n = 0;
                if (!get(et) || !get(n)) return false;
                if (et > T_LAST || et == T_ARRAY || n > kMaxArray) return fail("unsupported array type or size");
                const bool collect = keep && n <= kKeptArray;
                v.kind = collect ? AF_GGUF_ARRAY : AF_GGUF_ARRAY_SUMMARY;
                v.element_type = et;
                v.length = n;
                for (uint64_t k = 0; k < n; ++k) {
                    Value e;
                    if (!value(et, e, collect)) return false;
                    if (collect) v.items.push_back(std::move(e));
                }
                return true;
            }
            case T_U64: { uint64_t x; if (!get(x)) return false; v.kind = AF_GGUF_UNSIGNED; v.u = x; return true; }
            case T_I64: { int64_t x; if (!get(x)) return false; v.kind = AF_GGUF_SIGNED; v.i = x; return true; }
            case T_F64: { double x; if (!get(x)) return false; v.kind = AF_GGUF_FLOAT; v.f = x; return true; }
            default: return fail("unknown metadata type");
        }
    }
};

}  // namespace

struct af_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    uint64_t size = 0, data_offset = 0;
    uint32_t version = 0;
    std::map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> by_name;
    ~af_gguf() {
        if (map) munmap(const_cast<uint8_t*>(map), size);
        if (fd >= 0) close(fd);
    }
    const Tensor* find(const char* name) const {
        auto it = by_name.find(name);
        return it == by_name.end() ? nullptr : &tensors[it->second];
    }
    const Value* value(const std::string& key) const {
        auto it = meta.find(key);
        return it == meta.end() ? nullptr : &it->second;
    }
};

namespace {

// The header parse (gguf.rs:419-540 rules): signature, version 3, bounded counts, unique keys and
// tensor names, alignment, known types with whole blocks per row, aligned offsets, every tensor
// inside the file and no two overlapping.
int parse(af_gguf& g) {
    Cursor c{g.map, g.size};
    char magic[4] = {};
    for (char& m : magic)
        if (!c.get(m)) break;
    if (c.err.empty() && std::memcmp(magic, "GGUF", 4) != 0) c.fail("GGUF signature missing");
    uint32_t version = 0;
    uint64_t nt = 0, nk = 0;
    if (c.get(version) && version != 3) c.fail("only little-endian GGUF v3 is supported");
    if (c.get(nt) && c.get(nk) && (nt > kMaxEntries || nk > kMaxEntries)) c.fail("too many entries");
    for (uint64_t k = 0; c.err.empty() && k < nk; ++k) {
        std::string key;
        uint32_t type = 0;
        Value v;
        if (!c.string(key) || !c.get(type) || !c.value(type, v, true)) break;
        if (!g.meta.emplace(key, std::move(v)).second) c.fail("duplicate metadata key");
    }
    uint64_t alignment = 32;
    if (c.err.empty()) {
        if (const Value* a = g.value("general.alignment")) {
            alignment = a->kind == AF_GGUF_UNSIGNED ? a->u : 0;
            if (alignment == 0 || (alignment & (alignment - 1)) || alignment > (1u << 20)) c.fail("invalid alignment");
        }
    }
    std::set<std::string> names;
    for (uint64_t k = 0; c.err.empty() && k < nt; ++k) {
        Tensor t;
        uint32_t nd = 0;
        if (!c.string(t.name) || !c.get(nd)) break;
        if (t.name.empty() || !names.insert(t.name).second) { c.fail("empty or duplicate tensor name"); break; }
        if (nd < 1 || nd > 4) { c.fail("invalid number of dimensions"); break; }
        unsigned __int128 elements = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            uint64_t n = 0;
            if (!c.get(n)) break;
            if (n == 0) { c.fail("zero dimension"); break; }
            elements *= n;
            if (elements >> 64) { c.fail("dimensions too large"); break; }
            t.dims.push_back(n);
        }
        if (!c.err.empty() || !c.get(t.type)) break;
        uint64_t block = 0, bytes = 0;
        if (!block_layout(t.type, block, bytes)) { c.fail("unsupported weight type"); break; }
        if (t.dims[0] % block) { c.fail("row not a whole number of quantisation blocks"); break; }
        const unsigned __int128 len = elements / block * bytes;
        if (len >> 64) { c.fail("tensor too large"); break; }
        t.bytes = (uint64_t)len;
        if (!c.get(t.offset)) break;
        if (t.offset % alignment) { c.fail("tensor offset not aligned"); break; }
        g.tensors.push_back(std::move(t));
    }
    if (!c.err.empty()) return set_error(AF_ERR_INVALID, "GGUF: " + c.err);
    const uint64_t data = (c.pos + alignment - 1) / alignment * alignment;
    if (data > g.size) return set_error(AF_ERR_INVALID, "GGUF: data section missing");
    std::vector<std::pair<uint64_t, uint64_t>> ranges;
    for (size_t i = 0; i < g.tensors.size(); ++i) {
        Tensor& t = g.tensors[i];
        if (t.offset > g.size - data || t.bytes > g.size - data - t.offset)
            return set_error(AF_ERR_INVALID, "GGUF: tensor outside the file (truncated file)");
        t.offset += data;
        ranges.emplace_back(t.offset, t.offset + t.bytes);
        g.by_name[t.name] = i;
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); ++i)
        if (ranges[i - 1].second > ranges[i].first) return set_error(AF_ERR_INVALID, "GGUF: overlapping tensors");
    g.version = version;
    g.data_offset = data;
    return AF_OK;
}

void fill_tensor(const Tensor& t, af_gguf_tensor_info* out) {
    std::memset(out, 0, sizeof(*out));
    out->type = t.type;
    out->n_dims = (uint32_t)t.dims.size();
    for (size_t d = 0; d < t.dims.size(); ++d) out->dims[d] = t.dims[d];
    out->offset = t.offset;
    out->bytes = t.bytes;
}

void fill_value(const Value& v, af_gguf_value* out) {
    std::memset(out, 0, sizeof(*out));
    out->kind = v.kind;
    out->u = v.u;
    out->i = v.i;
    out->f = v.f;
    out->text = v.kind == AF_GGUF_TEXT ? v.text.c_str() : nullptr;
    out->length = v.kind == AF_GGUF_TEXT ? v.text.size() : v.length;
    out->element_type = v.element_type;
}

// ---- Gemma 4 layer assembly ---------------------------------------------------------------------

struct Loader {
    const af_gguf& g;
    std::string err;
    std::vector<std::vector<float>> keep;  // RoPE factors of local layers (ones)

    bool fail(const std::string& m) {
        if (err.empty()) err = m;
        return false;
    }
    const Tensor* tensor(const std::string& name, uint32_t type, uint32_t nd) {
        const Tensor* t = g.find(name.c_str());
        if (!t) return fail("tensor " + name + " missing"), nullptr;
        if (t->type != type || t->dims.size() != nd) return fail("tensor " + name + " has an unexpected type or rank"), nullptr;
        return t;
    }
    bool matrix(const std::string& name, uint32_t type, af_matrix& m) {
        const Tensor* t = tensor(name, type, 2);
        if (!t) return false;
        if (t->dims[0] > 0xFFFFFFFFull || t->dims[1] > 0xFFFFFFFFull) return fail("tensor " + name + " too large");
        m = af_matrix{g.map + t->offset, (size_t)t->bytes, (uint32_t)t->dims[0], (uint32_t)t->dims[1]};
        return true;
    }
    const float* vector(const std::string& name, uint32_t& len) {
        const Tensor* t = tensor(name, AF_GGUF_F32, 1);
        if (!t) return nullptr;
        if (t->dims[0] == 0 || t->dims[0] > 65536) return fail("vector " + name + " must hold 1..65536 floats"), nullptr;
        len = (uint32_t)t->dims[0];
        return reinterpret_cast<const float*>(g.map + t->offset);
    }
    bool norm(const std::string& name, float eps, af_rms_norm& n) {
        uint32_t len = 0;
        const float* w = vector(name, len);
        if (!w) return false;
        n = af_rms_norm{w, len, eps};
        return true;
    }
    bool unsigned_meta(const std::string& key, uint64_t& v) {
        const Value* x = g.value(key);
        if (!x || x->kind != AF_GGUF_UNSIGNED) return fail("metadata " + key + " missing or not an unsigned integer");
        v = x->u;
        return true;
    }
    bool float_meta(const std::string& key, double& v) {
        const Value* x = g.value(key);
        if (!x || x->kind != AF_GGUF_FLOAT) return fail("metadata " + key + " missing or not a float");
        v = x->f;
        return true;
    }
};

}  // namespace

namespace af {

// One layer of a Gemma 4 file as crates/application/src/stack.rs:26-107 assembles it: Q/K (V when
// present, else K's weights, lib.rs:351-383), per-head norms, RoPE from the metadata (local layers
// base freq_base_swa and unit factors, global layers freq_base and rope_freqs, lib.rs:661-709),
// scale 1.0, the sliding window of local layers, the output branch and the FFN with its optional
// scalar layer_output_scale; unit-weight V RMSNorm on every layer (stack.rs:687-688).
int gguf_layer(const af_gguf& g, uint32_t layer, std::vector<std::vector<float>>& factors, af_layer_weights& w) {
    Loader L{g};
    const std::string p = "blk." + std::to_string(layer) + ".";
    std::memset(&w, 0, sizeof(w));
    double eps = 0;
    L.float_meta("gemma4.attention.layer_norm_rms_epsilon", eps);
    const float e = (float)eps;
    L.norm(p + "attn_norm.weight", e, w.input_norm);
    L.matrix(p + "attn_q.weight", AF_GGUF_Q4_0, w.matrices[0]);
    L.matrix(p + "attn_k.weight", AF_GGUF_Q4_0, w.matrices[1]);
    if (g.find((p + "attn_v.weight").c_str())) L.matrix(p + "attn_v.weight", AF_GGUF_Q4_0, w.matrices[2]);
    else w.matrices[2] = w.matrices[1];  // V computed with K's weights (pointer equality, stack.rs:172)
    L.norm(p + "attn_q_norm.weight", e, w.head_norms[0]);
    L.norm(p + "attn_k_norm.weight", e, w.head_norms[1]);
    if (!L.err.empty()) return set_error(AF_ERR_INVALID, "GGUF layer " + std::to_string(layer) + ": " + L.err);
    const uint32_t width = w.head_norms[0].len;
    const Value* pattern = g.value("gemma4.attention.sliding_window_pattern");
    if (!pattern || pattern->kind != AF_GGUF_ARRAY || layer >= pattern->items.size() ||
        pattern->items[layer].kind != AF_GGUF_BOOL)
        return set_error(AF_ERR_INVALID, "GGUF: RoPE metadata missing or incompatible");
    const bool local = pattern->items[layer].u != 0;
    const std::string sfx = local ? "_swa" : "";
    double base = 0;
    uint64_t dim = 0, context = 0, window = 0;
    L.float_meta("gemma4.rope.freq_base" + sfx, base);
    L.unsigned_meta("gemma4.rope.dimension_count" + sfx, dim);
    L.unsigned_meta("gemma4.context_length", context);
    if (local) L.unsigned_meta("gemma4.attention.sliding_window", window);
    if (!L.err.empty()) return set_error(AF_ERR_INVALID, "GGUF layer " + std::to_string(layer) + ": " + L.err);
    if (dim != width)
        return set_error(AF_ERR_INVALID, "GGUF: partial RoPE is not supported (dimension_count must equal the head width)");
    if (context > 0xFFFFFFFFull || window > 0xFFFFFFFFull) return set_error(AF_ERR_INVALID, "GGUF: context out of range");
    const float* f = nullptr;
    if (local) {
        factors.emplace_back(width / 2, 1.0f);
        f = factors.back().data();
    } else {
        const std::string own = p + "rope_freqs.weight";
        uint32_t n = 0;
        f = L.vector(g.find(own.c_str()) ? own : std::string("rope_freqs.weight"), n);
        if (f && n != width / 2) return set_error(AF_ERR_INVALID, "GGUF: rope_freqs length differs from width / 2");
    }
    w.rope = af_rope_params{width, base, f, (uint32_t)context};
    if (width == 0 || w.matrices[0].rows % width || w.matrices[1].rows % width)
        return set_error(AF_ERR_INVALID, "GGUF: incompatible head dimensions");
    w.attention = af_attention_config{w.matrices[0].rows / width, w.matrices[1].rows / width, width,
                                      local ? (uint32_t)window : 0u, 1.0f};
    L.matrix(p + "attn_output.weight", AF_GGUF_Q4_0, w.output);
    L.norm(p + "post_attention_norm.weight", e, w.output_norm);
    // dense layers only (stack.rs:71-83)
    for (const auto& t : g.tensors)
        if (t.name.rfind(p + "ffn_gate_inp", 0) == 0) return set_error(AF_ERR_INVALID, "GGUF: MoE layers are not supported");
    const Value* ple = g.value("gemma4.embedding_length_per_layer_input");
    if (!ple || ple->kind != AF_GGUF_UNSIGNED || ple->u != 0)
        return set_error(AF_ERR_INVALID, "GGUF: per-layer embeddings are not supported");
    float scale = 1.0f;
    if (g.find((p + "layer_output_scale.weight").c_str())) {
        uint32_t n = 0;
        const float* s = L.vector(p + "layer_output_scale.weight", n);
        if (s && n != 1) return set_error(AF_ERR_INVALID, "GGUF: layer scale is not a scalar");
        if (s) scale = s[0];
    }
    L.norm(p + "ffn_norm.weight", e, w.ffn.pre);
    L.matrix(p + "ffn_gate.weight", AF_GGUF_Q4_0, w.ffn.gate);
    L.matrix(p + "ffn_up.weight", AF_GGUF_Q4_0, w.ffn.up);
    L.matrix(p + "ffn_down.weight", AF_GGUF_Q4_0, w.ffn.down);
    L.norm(p + "post_ffw_norm.weight", e, w.ffn.post);
    w.ffn.layer_scale = scale;
    w.flags = AF_LAYER_V_NORM;
    if (!L.err.empty()) return set_error(AF_ERR_INVALID, "GGUF layer " + std::to_string(layer) + ": " + L.err);
    return AF_OK;
}

}  // namespace af

extern "C" {

int af_gguf_open(const char* path, af_gguf** out) {
    if (!path || !out) return set_error(AF_ERR_INVALID, "null argument");
    *out = nullptr;
    auto g = std::make_unique<af_gguf>();
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) return set_error(AF_ERR_INVALID, std::string(path) + ": " + std::strerror(errno));
    struct stat st {};
    if (fstat(g->fd, &st) != 0) return set_error(AF_ERR_INVALID, std::string(path) + ": " + std::strerror(errno));
    g->size = (uint64_t)st.st_size;
    if (g->size == 0) return set_error(AF_ERR_INVALID, "GGUF: file truncated");
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return set_error(AF_ERR_INVALID, std::string(path) + ": mmap: " + std::strerror(errno));
    g->map = static_cast<const uint8_t*>(m);
    int rc = parse(*g);
    if (rc) return rc;
    *out = g.release();
    return AF_OK;
}

void af_gguf_close(af_gguf* g) { delete g; }

int af_gguf_info(const af_gguf* g, af_gguf_file* out) {
    if (!g || !out) return set_error(AF_ERR_INVALID, "null argument");
    out->version = g->version;
    out->tensors = g->tensors.size();
    out->metadata = g->meta.size();
    out->data_offset = g->data_offset;
    out->file_bytes = g->size;
    return AF_OK;
}

int af_gguf_tensor_at(const af_gguf* g, uint64_t index, const char** name, af_gguf_tensor_info* out) {
    if (!g || !out || !name || index >= g->tensors.size()) return set_error(AF_ERR_INVALID, "tensor index out of range");
    *name = g->tensors[index].name.c_str();
    fill_tensor(g->tensors[index], out);
    return AF_OK;
}

int af_gguf_tensor(const af_gguf* g, const char* name, af_gguf_tensor_info* out) {
    if (!g || !name || !out) return set_error(AF_ERR_INVALID, "null argument");
    const Tensor* t = g->find(name);
    if (!t) return set_error(AF_ERR_INVALID, std::string("tensor ") + name + " missing");
    fill_tensor(*t, out);
    return AF_OK;
}

int af_gguf_read(const af_gguf* g, const char* name, uint64_t offset, void* dst, uint64_t len) {
    if (!g || !name || (!dst && len)) return set_error(AF_ERR_INVALID, "null argument");
    const Tensor* t = g->find(name);
    if (!t) return set_error(AF_ERR_INVALID, std::string("tensor ") + name + " missing");
    if (offset > t->bytes || len > t->bytes - offset) return set_error(AF_ERR_INVALID, "read outside the tensor");
    std::memcpy(dst, g->map + t->offset + offset, len);
    return AF_OK;
}

int af_gguf_meta_at(const af_gguf* g, uint64_t index, const char** key, af_gguf_value* out) {
    if (!g || !key || !out || index >= g->meta.size()) return set_error(AF_ERR_INVALID, "metadata index out of range");
    auto it = g->meta.begin();
    std::advance(it, (long)index);
    *key = it->first.c_str();
    fill_value(it->second, out);
    return AF_OK;
}

int af_gguf_meta(const af_gguf* g, const char* key, uint64_t element, af_gguf_value* out) {
    if (!g || !key || !out) return set_error(AF_ERR_INVALID, "null argument");
    const Value* v = g->value(key);
    if (!v) return set_error(AF_ERR_INVALID, std::string("metadata ") + key + " missing");
    if (element == AF_GGUF_WHOLE) {
        fill_value(*v, out);
        return AF_OK;
    }
    if (v->kind != AF_GGUF_ARRAY || element >= v->items.size())
        return set_error(AF_ERR_INVALID, std::string("metadata ") + key + ": element out of range or array not kept");
    fill_value(v->items[element], out);
    return AF_OK;
}

int af_gguf_session_open(const af_gguf* g, uint32_t capacity, af_session** out) {
    if (!g || !out) return set_error(AF_ERR_INVALID, "null argument");
    *out = nullptr;
    const Value* arch = g->value("general.architecture");
    if (!arch || arch->kind != AF_GGUF_TEXT || arch->text != "gemma4")
        return set_error(AF_ERR_INVALID, "GGUF: a Gemma 4 model is required");
    const Value* blocks = g->value("gemma4.block_count");
    if (!blocks || blocks->kind != AF_GGUF_UNSIGNED || blocks->u == 0 || blocks->u > 1024)
        return set_error(AF_ERR_INVALID, "GGUF: block count missing or invalid");
    const Value* cap = g->value("gemma4.final_logit_softcapping");
    if (!cap || cap->kind != AF_GGUF_FLOAT || !std::isfinite(cap->f) || cap->f <= 0)
        return set_error(AF_ERR_INVALID, "GGUF: softcap missing or invalid");
    // the session embeds tokens from the head's table (crates/application/src/stack.rs:333-339
    // requires tied output weights for generation)
    if (g->find("output.weight"))
        return set_error(AF_ERR_INVALID, "GGUF: output weights separate from the embeddings are not supported");
    const uint32_t n = (uint32_t)blocks->u;
    std::vector<af_layer_weights> layers(n);
    std::vector<std::vector<float>> factors;
    factors.reserve(n);
    for (uint32_t l = 0; l < n; ++l) {
        int rc = af::gguf_layer(*g, l, factors, layers[l]);
        if (rc) return rc;
    }
    Loader L{*g};
    double eps = 0;
    L.float_meta("gemma4.attention.layer_norm_rms_epsilon", eps);
    af_output_head head{};
    L.norm("output_norm.weight", (float)eps, head.norm);
    L.matrix("token_embd.weight", AF_GGUF_Q6_K, head.matrix);  // tied embedding / lm-head
    if (!L.err.empty()) return set_error(AF_ERR_INVALID, "GGUF head: " + L.err);
    head.cap = (float)cap->f;
    return af_session_open(layers.data(), n, &head, capacity, out);
}

}  // extern "C"
