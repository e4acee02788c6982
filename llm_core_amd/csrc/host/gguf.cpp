// gguf.cpp — GGUF v2/v3 file access and the file → device-resident decoder
// load, the `-b hip` counterparts of GgufReader (src/loader/gguf_reader.hpp,
// gguf_loader.cpp:49-163), Engine::from_gguf (src/engine.cpp:79-183) and the
// weight table of build_weights (src/models/llama_model.cpp:975-1006).
//
// The file is mmap'd read-only and parsed once; tensors are device-uploaded
// straight from the mapping (no host copy of the weights), in native GGUF
// block layout.  Format errors carry the reference's messages; where the
// reference would read out of bounds or divide by zero on a corrupt file
// (a tensor whose data range leaves the file, general.alignment == 0, counts
// beyond the file) this code reports an error instead.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

#include "../capi_internal.hpp"

using namespace axf;

namespace {

struct GgufArray {
    int32_t elem_type = 0;
    uint64_t count = 0;
    std::vector<uint8_t> data;         // POD elements
    std::vector<std::string> strings;  // elem_type 8
};

// index = GGUF value type tag: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32,
// 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64
using GgufValue = std::variant<uint8_t, int8_t, uint16_t, int16_t, uint32_t, int32_t, float, bool,
                               std::string, GgufArray, uint64_t, int64_t, double>;

struct TensorInfo {
    std::string name;
    std::vector<int64_t> shape;  // GGML order, ne[0] innermost
    int32_t ggml_type = 0;
    uint64_t offset = 0;  // within the data blob
    uint64_t nbytes = 0;  // 0 for types without a known size
};

struct ParseError {
    std::string msg;
};

}  // namespace

struct axf_gguf {
    int fd = -1;
    void* map = nullptr;
    size_t size = 0;
    const uint8_t* begin = nullptr;
    const uint8_t* cur = nullptr;
    const uint8_t* end = nullptr;

    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_base = 0;
    int64_t n_kv = 0;
    std::unordered_map<std::string, GgufValue> kv;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, size_t> index;

    ~axf_gguf() {
        if (map && map != MAP_FAILED) munmap(map, size);
        if (fd >= 0) ::close(fd);
    }

    size_t left() const { return (size_t)(end - cur); }
    void need(uint64_t n) const {
        if (n > left()) throw ParseError{"GgufReader: unexpected end of file (truncated)"};
    }
    template <typename T>
    T pod() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, cur, sizeof(T));
        cur += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = pod<uint64_t>();
        need(n);
        std::string s(reinterpret_cast<const char*>(cur), (size_t)n);
        cur += n;
        return s;
    }
    GgufArray array();
    GgufValue value(int32_t tag);
    void parse();

    const TensorInfo* tensor(int64_t i) const {
        return i >= 0 && (size_t)i < tensors.size() ? &tensors[(size_t)i] : nullptr;
    }
    // the tensor's bytes, or nullptr when its data range leaves the file
    const uint8_t* data(const TensorInfo& t) const {
        const uint64_t a = data_base + t.offset;
        if (a < data_base || a > size || t.nbytes > size - a) return nullptr;
        return begin + a;
    }
    const GgufValue* find(const char* key) const {
        if (!key) return nullptr;
        auto it = kv.find(key);
        return it == kv.end() ? nullptr : &it->second;
    }
};

namespace {

// gguf_type_pod_size (include/axonforge/dtype.hpp:87-104)
size_t pod_size(int32_t tag) {
    switch (tag) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

// gguf_tensor_nbytes over ggml_type_to_dtype (dtype.hpp:107-155): block types
// round up to whole blocks; 0 for types the reference does not size
uint64_t type_nbytes(int32_t ggml_type, int64_t numel) {
    if (numel <= 0) return 0;
    const uint64_t n = (uint64_t)numel;
    switch (ggml_type) {
    case 0: return n * 4;                     // F32
    case 1: case 30: return n * 2;            // F16, BF16
    case 24: return n;                        // I8
    case 25: return n * 2;                    // I16
    case 26: return n * 4;                    // I32
    case 8: return (n + 31) / 32 * 34;        // Q8_0
    case 2: return (n + 31) / 32 * 18;        // Q4_0
    case 6: return (n + 31) / 32 * 22;        // Q5_0
    case 12: return (n + 255) / 256 * 144;    // Q4_K
    case 11: return (n + 255) / 256 * 110;    // Q3_K
    case 10: return (n + 255) / 256 * 84;     // Q2_K
    case 14: return (n + 255) / 256 * 210;    // Q6_K
    default: return 0;
    }
}

}  // namespace

GgufArray axf_gguf::array() {
    GgufArray a;
    a.elem_type = pod<int32_t>();
    a.count = pod<uint64_t>();
    if (a.elem_type == 8) {
        if (a.count > left() / 8) throw ParseError{"GgufReader: unexpected end of file (truncated)"};
        a.strings.reserve((size_t)a.count);
        for (uint64_t i = 0; i < a.count; i++) a.strings.push_back(str());
        return a;
    }
    const size_t esz = pod_size(a.elem_type);
    if (esz == 0) throw ParseError{"GgufReader: nested ARRAY or unknown type in array"};
    if (a.count > left() / esz) throw ParseError{"GgufReader: unexpected end of file (truncated)"};
    const size_t total = (size_t)a.count * esz;
    a.data.assign(cur, cur + total);
    cur += total;
    return a;
}

GgufValue axf_gguf::value(int32_t tag) {
    switch (tag) {
    case 0: return pod<uint8_t>();
    case 1: return pod<int8_t>();
    case 2: return pod<uint16_t>();
    case 3: return pod<int16_t>();
    case 4: return pod<uint32_t>();
    case 5: return pod<int32_t>();
    case 6: return pod<float>();
    case 7: return pod<int8_t>() != 0;
    case 8: return str();
    case 9: return array();
    case 10: return pod<uint64_t>();
    case 11: return pod<int64_t>();
    case 12: return pod<double>();
    default: throw ParseError{"GgufReader: unknown KV type tag " + std::to_string(tag)};
    }
}

// Header, KV pairs, tensor infos, aligned data base (gguf_loader.cpp:84-163).
void axf_gguf::parse() {
    need(4);
    if (std::memcmp(cur, "GGUF", 4) != 0)
        throw ParseError{"GgufReader: invalid magic (not a GGUF file)"};
    cur += 4;
    version = pod<uint32_t>();
    if (version < 2 || version > 3)
        throw ParseError{"GgufReader: unsupported GGUF version " + std::to_string(version) +
                         " (supported: 2, 3)"};
    const int64_t nt = pod<int64_t>();
    const int64_t nk = pod<int64_t>();
    if (nt < 0 || nk < 0) throw ParseError{"GgufReader: negative tensor/kv counts"};
    n_kv = nk;
    for (int64_t i = 0; i < nk; i++) {
        std::string key = str();
        const int32_t tag = pod<int32_t>();
        GgufValue v = value(tag);
        kv.emplace(std::move(key), std::move(v));  // the first of duplicate keys is kept
    }
    if (const GgufValue* a = find("general.alignment")) {
        if (const auto* u = std::get_if<uint32_t>(a)) {
            if (*u == 0) throw ParseError{"GgufReader: general.alignment must be non-zero"};
            alignment = *u;
        }
    }
    for (int64_t i = 0; i < nt; i++) {
        TensorInfo t;
        t.name = str();
        const uint32_t nd = pod<uint32_t>();
        if (nd > 4)
            throw ParseError{"GgufReader: tensor '" + t.name + "' has more than 4 dimensions (" +
                             std::to_string(nd) + ")"};
        t.shape.resize(nd);
        for (uint32_t d = 0; d < nd; d++) {
            t.shape[d] = pod<int64_t>();
            if (t.shape[d] < 0)
                throw ParseError{"GgufReader: tensor '" + t.name + "' has negative dimension"};
        }
        t.ggml_type = pod<int32_t>();
        t.offset = pod<uint64_t>();
        int64_t ne = 1;
        bool ovf = false;
        for (int64_t d : t.shape) {
            if (d != 0 && ne > INT64_MAX / d) ovf = true;
            ne = ovf ? 0 : ne * d;
        }
        t.nbytes = ovf ? 0 : type_nbytes(t.ggml_type, ne);
        index[t.name] = tensors.size();  // a later duplicate name wins the lookup
        tensors.push_back(std::move(t));
    }
    const uint64_t pos = (uint64_t)(cur - begin);
    data_base = (pos + alignment - 1) / alignment * alignment;
}

namespace {

uint64_t coerce_u64(const GgufValue& v, uint64_t def) {
    if (auto* p = std::get_if<uint64_t>(&v)) return *p;
    if (auto* p = std::get_if<uint32_t>(&v)) return *p;
    if (auto* p = std::get_if<int64_t>(&v)) return (uint64_t)*p;
    if (auto* p = std::get_if<int32_t>(&v)) return (uint64_t)*p;
    if (auto* p = std::get_if<uint16_t>(&v)) return *p;
    if (auto* p = std::get_if<int16_t>(&v)) return (uint64_t)*p;
    if (auto* p = std::get_if<uint8_t>(&v)) return *p;
    if (auto* p = std::get_if<int8_t>(&v)) return (uint64_t)*p;
    return def;
}

uint64_t get_u64(const axf_gguf* g, const std::string& key, uint64_t def) {
    const GgufValue* v = g->find(key.c_str());
    return v ? coerce_u64(*v, def) : def;
}

int32_t get_i32(const axf_gguf* g, const char* key, int32_t def) {
    const GgufValue* v = g->find(key);
    if (!v) return def;
    if (auto* p = std::get_if<int32_t>(v)) return *p;
    if (auto* p = std::get_if<uint32_t>(v)) return (int32_t)*p;
    if (auto* p = std::get_if<int64_t>(v)) return (int32_t)*p;
    if (auto* p = std::get_if<uint64_t>(v)) return (int32_t)*p;
    return def;
}

float get_f32(const axf_gguf* g, const std::string& key, float def) {
    const GgufValue* v = g->find(key.c_str());
    if (!v) return def;
    if (auto* p = std::get_if<float>(v)) return *p;
    if (auto* p = std::get_if<double>(v)) return (float)*p;
    return def;
}

const GgufArray* get_array(const axf_gguf* g, const char* key) {
    const GgufValue* v = g->find(key);
    return v ? std::get_if<GgufArray>(v) : nullptr;
}

#define GG_CHECK(g)                                                                        \
    if (!(g)) return fail(AXF_ERR_INVALID_ARG, std::string(__func__) + ": null file")

}  // namespace

extern "C" {

int axf_gguf_open(const char* path, axf_gguf** out) {
    if (!path || !out) return fail(AXF_ERR_INVALID_ARG, "axf_gguf_open: null argument");
    *out = nullptr;
    const std::string p(path);
    auto* g = new axf_gguf();
    g->fd = ::open(p.c_str(), O_RDONLY);
    if (g->fd < 0) {
        delete g;
        return fail(AXF_ERR_INVALID_ARG, "GgufReader: cannot open '" + p + "'");
    }
    struct stat st {};
    if (fstat(g->fd, &st) != 0) {
        delete g;
        return fail(AXF_ERR_INVALID_ARG, "GgufReader: fstat failed for '" + p + "'");
    }
    g->size = (size_t)st.st_size;
    if (g->size < 16) {
        delete g;
        return fail(AXF_ERR_INVALID_ARG, "GgufReader: file too small (< 16 bytes)");
    }
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->map == MAP_FAILED) {
        g->map = nullptr;
        delete g;
        return fail(AXF_ERR_INVALID_ARG, "GgufReader: mmap failed for '" + p + "'");
    }
    g->begin = g->cur = static_cast<const uint8_t*>(g->map);
    g->end = g->begin + g->size;
    try {
        g->parse();
    } catch (const ParseError& e) {
        delete g;
        return fail(AXF_ERR_INVALID_ARG, e.msg);
    } catch (const std::bad_alloc&) {
        delete g;
        return fail(AXF_ERR_INVALID_ARG, "GgufReader: out of host memory while parsing");
    }
    *out = g;
    return AXF_OK;
}

int axf_gguf_close(axf_gguf* g) {
    delete g;
    return AXF_OK;
}

uint32_t axf_gguf_version(const axf_gguf* g) { return g ? g->version : 0; }
uint64_t axf_gguf_alignment(const axf_gguf* g) { return g ? g->alignment : 0; }
uint64_t axf_gguf_data_offset(const axf_gguf* g) { return g ? g->data_base : 0; }
uint64_t axf_gguf_file_size(const axf_gguf* g) { return g ? g->size : 0; }
int64_t axf_gguf_n_kv(const axf_gguf* g) { return g ? g->n_kv : 0; }
int64_t axf_gguf_n_tensors(const axf_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }

int axf_gguf_kv_type(const axf_gguf* g, const char* key) {
    const GgufValue* v = g ? g->find(key) : nullptr;
    return v ? (int)v->index() : -1;
}

uint64_t axf_gguf_get_u64(const axf_gguf* g, const char* key, uint64_t def) {
    return g && key ? get_u64(g, key, def) : def;
}
uint32_t axf_gguf_get_u32(const axf_gguf* g, const char* key, uint32_t def) {
    return (uint32_t)axf_gguf_get_u64(g, key, def);
}
int32_t axf_gguf_get_i32(const axf_gguf* g, const char* key, int32_t def) {
    return g && key ? get_i32(g, key, def) : def;
}
float axf_gguf_get_f32(const axf_gguf* g, const char* key, float def) {
    return g && key ? get_f32(g, key, def) : def;
}
int axf_gguf_get_bool(const axf_gguf* g, const char* key, int def) {
    const GgufValue* v = g ? g->find(key) : nullptr;
    if (!v) return def;
    if (auto* p = std::get_if<bool>(v)) return *p ? 1 : 0;
    return def;
}

int axf_gguf_get_str(const axf_gguf* g, const char* key, const char** s, size_t* len) {
    GG_CHECK(g);
    if (!key || !s) return fail(AXF_ERR_INVALID_ARG, "axf_gguf_get_str: null argument");
    const GgufValue* v = g->find(key);
    const std::string* p = v ? std::get_if<std::string>(v) : nullptr;
    if (!p) return fail(AXF_ERR_INVALID_ARG, std::string("axf_gguf_get_str: no string key ") + key);
    *s = p->c_str();
    if (len) *len = p->size();
    return AXF_OK;
}

uint64_t axf_gguf_get_array_count(const axf_gguf* g, const char* key) {
    const GgufArray* a = g ? get_array(g, key) : nullptr;
    return a ? a->count : 0;
}

int axf_gguf_get_array_type(const axf_gguf* g, const char* key) {
    const GgufArray* a = g ? get_array(g, key) : nullptr;
    return a ? a->elem_type : -1;
}

int axf_gguf_get_array_str(const axf_gguf* g, const char* key, uint64_t i, const char** s,
                           size_t* len) {
    GG_CHECK(g);
    const GgufArray* a = get_array(g, key);
    if (!a || a->elem_type != 8 || i >= a->count || !s)
        return fail(AXF_ERR_INVALID_ARG, "axf_gguf_get_array_str: no such string element");
    *s = a->strings[(size_t)i].c_str();
    if (len) *len = a->strings[(size_t)i].size();
    return AXF_OK;
}

int axf_gguf_get_array_data(const axf_gguf* g, const char* key, const void** data,
                            size_t* bytes) {
    GG_CHECK(g);
    const GgufArray* a = get_array(g, key);
    if (!a || a->elem_type == 8 || !data || !bytes)
        return fail(AXF_ERR_INVALID_ARG, "axf_gguf_get_array_data: no such POD array");
    *data = a->data.data();
    *bytes = a->data.size();
    return AXF_OK;
}

int64_t axf_gguf_find_tensor(const axf_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->index.find(name);
    return it == g->index.end() ? -1 : (int64_t)it->second;
}

int axf_gguf_tensor_info(const axf_gguf* g, int64_t i, axf_gguf_tensor* out) {
    GG_CHECK(g);
    const TensorInfo* t = g->tensor(i);
    if (!t || !out) return fail(AXF_ERR_INVALID_ARG, "axf_gguf_tensor_info: bad index");
    std::memset(out, 0, sizeof(*out));
    out->name = t->name.c_str();
    out->n_dims = (int)t->shape.size();
    for (size_t d = 0; d < t->shape.size(); d++) out->shape[d] = t->shape[d];
    out->ggml_type = t->ggml_type;
    out->offset = t->offset;
    out->nbytes = t->nbytes;
    out->data = g->data(*t);
    return AXF_OK;
}

size_t axf_gguf_type_nbytes(int ggml_type, int64_t numel) {
    return (size_t)type_nbytes(ggml_type, numel);
}

size_t axf_gguf_pod_size(int type_tag) { return pod_size(type_tag); }

// ModelConfig extraction of Engine::from_gguf (engine.cpp:79-118).
int axf_gguf_read_model_config(const axf_gguf* g, axf_gguf_model_config* c) {
    GG_CHECK(g);
    if (!c) return fail(AXF_ERR_INVALID_ARG, "axf_gguf_read_model_config: null argument");
    std::memset(c, 0, sizeof(*c));
    std::string arch = "unknown";
    if (const GgufValue* v = g->find("general.architecture"))
        if (auto* p = std::get_if<std::string>(v)) arch = *p;
    std::snprintf(c->arch, sizeof(c->arch), "%s", arch.c_str());
    c->n_layer = (int)get_u64(g, arch + ".block_count", 0);
    c->n_embd = (int)get_u64(g, arch + ".embedding_length", 0);
    c->ffn_dim = (int)get_u64(g, arch + ".feed_forward_length", 0);
    c->n_heads = (int)get_u64(g, arch + ".attention.head_count", 0);
    c->n_kv_heads = (int)get_u64(g, arch + ".attention.head_count_kv", (uint64_t)c->n_heads);
    c->max_seq_len = (int)get_u64(g, arch + ".context_length", 4096);
    c->rms_eps = get_f32(g, arch + ".attention.layer_norm_rms_epsilon", 1e-5f);
    c->rope_theta = get_f32(g, arch + ".rope.freq_base", 10000.0f);
    c->rope_scaling_alpha = get_f32(g, arch + ".rope.scaling.alpha", 0.0f);
    if (c->n_heads > 0 && c->n_embd > 0) c->head_dim = c->n_embd / c->n_heads;
    if (arch == "hunyuan-dense" && c->rope_scaling_alpha > 0.0f && c->head_dim > 2)
        c->rope_theta *= std::pow(c->rope_scaling_alpha,
                                  (float)c->head_dim / (float)(c->head_dim - 2));
    c->n_vocab = (int)axf_gguf_get_array_count(g, "tokenizer.ggml.tokens");
    c->weight_type = g->tensors.empty() ? -1 : g->tensors[0].ggml_type;
    c->bos_id = get_i32(g, "tokenizer.ggml.bos_token_id", 1);
    c->eos_id = get_i32(g, "tokenizer.ggml.eos_token_id", 2);
    return AXF_OK;
}

// Register every tensor the decoder reads (the names of build_weights,
// llama_model.cpp:975-1006) straight from the mapping, then upload.
int axf_llama_load_gguf(axf_llama* m, const axf_gguf* g) {
    GG_CHECK(g);
    if (!m) return fail(AXF_ERR_INVALID_ARG, "axf_llama_load_gguf: null model");
    for (const TensorInfo& t : g->tensors) {
        const bool model_tensor = t.name == "token_embd.weight" || t.name == "output.weight" ||
                                  t.name == "output_norm.weight" ||
                                  t.name.compare(0, 4, "blk.") == 0;
        if (!model_tensor) continue;
        // the weight types of the reference's gemv_wt / gemv_wt_q8 dispatch
        // (llama_model.cpp:670-831); axf_llama_load checks each tensor's shape
        if (t.ggml_type != AXF_TYPE_F32 && t.ggml_type != AXF_TYPE_Q4_K &&
            t.ggml_type != AXF_TYPE_Q6_K && t.ggml_type != AXF_TYPE_Q8_0 &&
            t.ggml_type != AXF_TYPE_Q5_0 && t.ggml_type != AXF_TYPE_F16)
            return fail(AXF_ERR_UNSUPPORTED, "axf_llama_load_gguf: " + t.name + " has GGML type " +
                                                 std::to_string(t.ggml_type) +
                                                 " (supported: F32, F16, Q8_0, Q5_0, Q4_K, Q6_K)");
        const uint8_t* p = g->data(t);
        if (!p || t.nbytes == 0)
            return fail(AXF_ERR_INVALID_ARG,
                        "axf_llama_load_gguf: tensor '" + t.name + "' data lies outside the file");
        int rc = axf_llama_set_tensor(m, t.name.c_str(), t.ggml_type, p, (size_t)t.nbytes);
        if (rc) return rc;
    }
    return axf_llama_load(m);
}

// Engine::from_gguf followed by llama_generate_cpu_impl's hyperparameter
// defaults (llama_model.cpp:1508-1518): KV heads default to the heads, the
// context is min(context_length, max_context_len), and zero eps / theta / FFN
// fall back to 1e-5 / 10000 / 4*E.  The vocabulary is the token-array length,
// or token_embd's rows when the file has no token array.
int axf_llama_from_gguf(axf_ctx* ctx, const char* path, int max_context_len, axf_llama** out) {
    if (!ctx || !path || !out) return fail(AXF_ERR_INVALID_ARG, "axf_llama_from_gguf: null argument");
    *out = nullptr;
    axf_gguf* g = nullptr;
    int rc = axf_gguf_open(path, &g);
    if (rc) return rc;
    axf_gguf_model_config c;
    axf_gguf_read_model_config(g, &c);
    axf_llama_hparams hp{};
    hp.n_layer = c.n_layer;
    hp.n_embd = c.n_embd;
    hp.n_heads = c.n_heads;
    hp.n_kv_heads = c.n_kv_heads > 0 ? c.n_kv_heads : c.n_heads;
    hp.ffn_dim = c.ffn_dim > 0 ? c.ffn_dim : 4 * c.n_embd;
    const int cap = max_context_len > 0 ? max_context_len : 4096;
    hp.n_ctx = c.max_seq_len < cap ? c.max_seq_len : cap;
    hp.rms_eps = c.rms_eps > 0.f ? c.rms_eps : 1e-5f;
    hp.rope_theta = c.rope_theta > 0.f ? c.rope_theta : 10000.f;
    const int64_t te = axf_gguf_find_tensor(g, "token_embd.weight");
    const int embd_rows = te >= 0 && g->tensors[(size_t)te].shape.size() == 2
                              ? (int)g->tensors[(size_t)te].shape[1]
                              : 0;
    hp.n_vocab = c.n_vocab > 0 ? c.n_vocab : embd_rows;
    if (c.n_vocab > 0 && embd_rows > 0 && c.n_vocab != embd_rows) {
        axf_gguf_close(g);
        return fail(AXF_ERR_INVALID_ARG, "axf_llama_from_gguf: tokenizer.ggml.tokens has " +
                                             std::to_string(c.n_vocab) + " entries, token_embd " +
                                             std::to_string(embd_rows) + " rows");
    }
    // QkNormOrder from the architecture (llama_model.cpp:1520-1522)
    hp.qk_norm_order = std::strcmp(c.arch, "hunyuan-dense") == 0 ? 2
                       : std::strcmp(c.arch, "qwen3") == 0     ? 1
                                                                : 0;
    axf_llama* m = nullptr;
    rc = axf_llama_create(ctx, &hp, &m);
    if (!rc) rc = axf_llama_load_gguf(m, g);
    axf_gguf_close(g);  // the weights are on the device now
    if (rc) {
        axf_llama_destroy(m);
        return rc;
    }
    *out = m;
    return AXF_OK;
}

}  // extern "C"
