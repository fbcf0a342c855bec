// Checkpoint reading on the host: safetensors files (one, or the shards an
// index names), config.json, and the fp32 tensors a WPC model takes from the
// dense checkpoint. Mirrors the reference's readers:
//   SafetensorsFile::{open, names, shape, read_f32}   weights.rs:125-178
//   ShardedSafetensors::{open, read_f32, shape}        weights.rs:180-264
//   Config::{load, from_json_str, head_dim}, moe_dims  config.rs:8-106,
//                                                      qwen3_moe_model.rs:121-135
//   (the norms and routers build_layers / load_wpc_v4 read from the
//   checkpoint are loaded by wpcg_model_load_safetensors in capi_model.cpp)
// Where the reference panics (an invalid file, a missing tensor, an
// unsupported dtype) these return status codes, and every file is
// validated when it is opened rather than at its first read.
//
// The safetensors format (the `safetensors` crate 0.4.5, which the
// reference deserializes every file with): an 8-byte little-endian header
// length n (at most 100,000,000), n bytes of JSON starting with '{' mapping
// each tensor name to {dtype, shape, data_offsets: [begin, end)} (plus an
// optional "__metadata__" map of strings), then the data. The offsets,
// relative to the data, must tile it exactly in offset order from 0, each
// span holding exactly product(shape) elements of the dtype.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <new>
#include <sstream>

#include "wpcg_internal.hpp"

namespace {

using wpcg::JsonValue;
using wpcg::fail;

struct StTensor {
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0;
};

struct StFile {
    std::string path;
    const uint8_t* map = nullptr;
    size_t size = 0;
    const uint8_t* data = nullptr;  // the byte buffer after the header
    std::unordered_map<std::string, StTensor> tensors;
    std::vector<std::string> names;  // header order
    ~StFile()
    {
        if (map) munmap(const_cast<uint8_t*>(map), size);
    }
};

uint64_t dtype_size(const std::string& d)
{
    if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E5M2" || d == "F8_E4M3") return 1;
    if (d == "I16" || d == "U16" || d == "F16" || d == "BF16") return 2;
    if (d == "I32" || d == "U32" || d == "F32") return 4;
    if (d == "I64" || d == "U64" || d == "F64") return 8;
    return 0;
}

int bad_file(const std::string& path, const std::string& why)
{
    return fail(WPCG_E_FORMAT, "invalid safetensors file " + path + ": " + why);
}

// Maps and validates one file (SafeTensors::deserialize's checks).
int open_file(const std::string& path, std::unique_ptr<StFile>& out)
{
    auto f = std::make_unique<StFile>();
    f->path = path;
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail(WPCG_E_IO, "cannot open " + path);
    struct stat stt;
    if (fstat(fd, &stt) != 0) {
        ::close(fd);
        return fail(WPCG_E_IO, "cannot stat " + path);
    }
    f->size = (size_t)stt.st_size;
    if (f->size) {
        void* p = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            ::close(fd);
            return fail(WPCG_E_IO, "cannot mmap " + path);
        }
        f->map = static_cast<const uint8_t*>(p);
    }
    ::close(fd);
    if (f->size < 8) return bad_file(path, "header too small");
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | f->map[i];
    if (n > 100000000ull) return bad_file(path, "header too large");
    if (n > f->size - 8) return bad_file(path, "header length past the end of the file");
    const char* h = reinterpret_cast<const char*>(f->map + 8);
    if (n == 0 || h[0] != '{') return bad_file(path, "header does not start with '{'");
    JsonValue root;
    std::string err;
    if (!wpcg::json_parse(h, (size_t)n, root, err)) return bad_file(path, "header: " + err);
    if (root.kind != JsonValue::OBJ) return bad_file(path, "header is not an object");
    struct Span {
        uint64_t b, e;
        const std::string* name;
    };
    std::vector<Span> spans;
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") {
            if (kv.second.kind == JsonValue::NUL) continue;
            if (kv.second.kind != JsonValue::OBJ) return bad_file(path, "__metadata__ is not a map");
            for (const auto& m : kv.second.obj)
                if (m.second.kind != JsonValue::STR) return bad_file(path, "__metadata__ value is not a string");
            continue;
        }
        const JsonValue& t = kv.second;
        const JsonValue* dt = t.get("dtype");
        const JsonValue* sh = t.get("shape");
        const JsonValue* off = t.get("data_offsets");
        if (t.kind != JsonValue::OBJ || !dt || !sh || !off) return bad_file(path, "tensor " + kv.first + " lacks dtype/shape/data_offsets");
        if (dt->kind != JsonValue::STR || !dtype_size(dt->str)) return bad_file(path, "tensor " + kv.first + ": unknown dtype");
        if (sh->kind != JsonValue::ARR) return bad_file(path, "tensor " + kv.first + ": shape is not a list");
        if (off->kind != JsonValue::ARR || off->arr.size() != 2 || !off->arr[0].is_uint || !off->arr[1].is_uint)
            return bad_file(path, "tensor " + kv.first + ": data_offsets is not [begin, end]");
        StTensor st;
        st.dtype = dt->str;
        for (const JsonValue& d : sh->arr) {
            if (!d.is_uint) return bad_file(path, "tensor " + kv.first + ": shape entry is not a size");
            st.shape.push_back(d.u);
        }
        st.begin = off->arr[0].u;
        st.end = off->arr[1].u;
        if (!f->tensors.count(kv.first)) f->names.push_back(kv.first);
        f->tensors[kv.first] = st;  // a repeated key keeps its last value, as the map does
    }
    for (const auto& kv : f->tensors) spans.push_back({kv.second.begin, kv.second.end, &kv.first});
    std::sort(spans.begin(), spans.end(), [](const Span& a, const Span& b) {
        return a.b != b.b ? a.b < b.b : a.e < b.e;
    });
    uint64_t at = 0;
    for (const Span& s : spans) {
        const StTensor& t = f->tensors[*s.name];
        if (s.b != at || s.e < s.b) return bad_file(path, "invalid offset for tensor " + *s.name);
        uint64_t count = 1;
        for (uint64_t d : t.shape) {
            if (d && count > UINT64_MAX / d) return bad_file(path, "size overflow in tensor " + *s.name);
            count *= d;
        }
        const uint64_t es = dtype_size(t.dtype);
        if (count > UINT64_MAX / es) return bad_file(path, "size overflow in tensor " + *s.name);
        if (s.e - s.b != count * es) return bad_file(path, "tensor " + *s.name + ": data_offsets disagree with shape and dtype");
        at = s.e;
    }
    if (at != f->size - 8 - n) return bad_file(path, "data length disagrees with the header");
    f->data = f->map + 8 + n;
    out = std::move(f);
    return WPCG_OK;
}

// f16 -> f32 exactly, as half 2.7.1's f16::to_f32 (a NaN keeps its payload
// with the quiet bit set).
float f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m ? (0x00400000u | (m << 13)) : 0u);
    } else if (e) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (!m) {
        bits = sign;
    } else {  // subnormal: m * 2^-24, exact in binary32
        const float v = (float)m * 0x1p-24f;
        float r = sign ? -v : v;
        return r;
    }
    float r;
    std::memcpy(&r, &bits, 4);
    return r;
}

}  // namespace

struct wpcg_safetensors {
    std::vector<std::unique_ptr<StFile>> shards;
    std::unordered_map<std::string, size_t> index;  // empty: one file serves every name
    std::vector<std::string> names;                 // names(): every tensor, shard by shard
};

namespace {

// The shard holding `name` (ShardedSafetensors::read_f32's lookup) and its
// entry; E_NOTFOUND where the reference panics.
int find(wpcg_safetensors* st, const char* name, const StFile** f, const StTensor** t)
{
    if (!st || !name) return fail(WPCG_E_ARG, "null argument");
    size_t slot = 0;
    auto it = st->index.find(name);
    if (it != st->index.end()) slot = it->second;
    else if (!st->index.empty()) return fail(WPCG_E_NOTFOUND, std::string("missing tensor ") + name + " (not in safetensors index)");
    const StFile* file = st->shards[slot].get();
    auto jt = file->tensors.find(name);
    if (jt == file->tensors.end()) return fail(WPCG_E_NOTFOUND, std::string("missing tensor ") + name);
    *f = file;
    *t = &jt->second;
    return WPCG_OK;
}

uint64_t count_of(const StTensor& t)
{
    uint64_t c = 1;
    for (uint64_t d : t.shape) c *= d;
    return c;
}

bool file_exists(const std::string& p)
{
    struct stat s;
    return ::stat(p.c_str(), &s) == 0 && S_ISREG(s.st_mode);
}

// ---- config.json ------------------------------------------------------------
int cfg_fail(const std::string& why) { return fail(WPCG_E_FORMAT, "config.json: " + why); }

// serde's usize / u32 / bool / f64 / Option<...> rules for the fields read.
int need_size(const JsonValue& root, const char* key, uint64_t& v)
{
    const JsonValue* x = root.get(key);
    if (!x) return cfg_fail(std::string("missing field `") + key + "`");
    if (!x->is_uint) return cfg_fail(std::string("`") + key + "` is not a non-negative integer");
    v = x->u;
    return WPCG_OK;
}
int need_f64(const JsonValue& root, const char* key, double& v)
{
    const JsonValue* x = root.get(key);
    if (!x) return cfg_fail(std::string("missing field `") + key + "`");
    if (x->kind != JsonValue::NUM) return cfg_fail(std::string("`") + key + "` is not a number");
    v = x->num;
    return WPCG_OK;
}
// Option<usize>: absent or null -> has = false
int opt_size(const JsonValue& root, const char* key, bool& has, uint64_t& v)
{
    const JsonValue* x = root.get(key);
    has = false;
    if (!x || x->kind == JsonValue::NUL) return WPCG_OK;
    if (!x->is_uint) return cfg_fail(std::string("`") + key + "` is not a non-negative integer");
    has = true;
    v = x->u;
    return WPCG_OK;
}
int opt_bool(const JsonValue& root, const char* key, bool& has, bool& v)
{
    const JsonValue* x = root.get(key);
    has = false;
    if (!x || x->kind == JsonValue::NUL) return WPCG_OK;
    if (x->kind != JsonValue::BOOL) return cfg_fail(std::string("`") + key + "` is not a boolean");
    has = true;
    v = x->b;
    return WPCG_OK;
}

int parse_config(const char* text, size_t n, uint32_t max_pos, wpcg_model_config* out)
{
    JsonValue root;
    std::string err;
    if (!wpcg::json_parse(text, n, root, err)) return cfg_fail(err);
    if (root.kind != JsonValue::OBJ) return cfg_fail("not an object");
    uint64_t vocab, hidden, layers, heads, kv_heads, inter;
    double theta, eps;
    for (auto [key, dst] : {std::pair<const char*, uint64_t*>{"vocab_size", &vocab}, {"hidden_size", &hidden},
                            {"num_hidden_layers", &layers}, {"num_attention_heads", &heads},
                            {"num_key_value_heads", &kv_heads}, {"intermediate_size", &inter}})
        if (int rc = need_size(root, key, *dst)) return rc;
    if (int rc = need_f64(root, "rope_theta", theta)) return rc;
    if (int rc = need_f64(root, "rms_norm_eps", eps)) return rc;
    // Config::tie_word_embeddings is parsed (a non-boolean fails as serde
    // fails) but never decides the head: the reference's loaders choose it by
    // model kind (below).
    if (const JsonValue* t = root.get("tie_word_embeddings"))
        if (t->kind != JsonValue::BOOL) return cfg_fail("`tie_word_embeddings` is not a boolean");
    for (const char* key : {"eos_token_id", "bos_token_id"}) {  // Option<u32>: type-checked only
        bool has;
        uint64_t v;
        if (int rc = opt_size(root, key, has, v)) return rc;
        if (has && v > 0xFFFFFFFFull) return cfg_fail(std::string("`") + key + "` does not fit u32");
    }
    std::string model_type;
    if (const JsonValue* t = root.get("model_type")) {
        if (t->kind == JsonValue::STR) model_type = t->str;
        else if (t->kind != JsonValue::NUL) return cfg_fail("`model_type` is not a string");
    }
    bool has_hd, has_ne, has_k, has_mi, has_nt, nt = true;
    uint64_t hd, ne, k, mi;
    if (int rc = opt_size(root, "head_dim", has_hd, hd)) return rc;
    if (int rc = opt_size(root, "num_experts", has_ne, ne)) return rc;
    if (int rc = opt_size(root, "num_experts_per_tok", has_k, k)) return rc;
    if (int rc = opt_size(root, "moe_intermediate_size", has_mi, mi)) return rc;
    if (int rc = opt_bool(root, "norm_topk_prob", has_nt, nt)) return rc;
    if (!heads) return cfg_fail("num_attention_heads is 0");
    wpcg_model_config c{};
    c.n_layers = (uint32_t)layers;
    c.hidden = (uint32_t)hidden;
    c.n_heads = (uint32_t)heads;
    c.n_kv_heads = (uint32_t)kv_heads;
    c.head_dim = (uint32_t)(has_hd ? hd : hidden / heads);  // Config::head_dim
    c.inter = (uint32_t)inter;
    c.vocab = (uint32_t)vocab;
    c.eps = (float)eps;
    c.rope_theta = theta;
    c.max_pos = max_pos;
    // The reference runs the MoE decoder exactly when model_type is
    // "qwen3_moe" (main.rs:73-77) and takes its dimensions from moe_dims.
    if (model_type == "qwen3_moe") {
        if (!has_ne) return cfg_fail("config.json has no `num_experts`; not a Qwen3-MoE model");
        if (!has_k) return cfg_fail("config.json has no `num_experts_per_tok`; cannot route");
        if (!has_mi) return cfg_fail("config.json has no `moe_intermediate_size`; expert width unknown");
        if (k == 0 || k > ne)
            return cfg_fail("num_experts_per_tok = " + std::to_string(k) + " is not in 1..=" + std::to_string(ne));
        c.n_experts = (uint32_t)ne;
        c.top_k = (uint32_t)k;
        c.moe_inter = (uint32_t)mi;
        c.norm_topk = (has_nt ? nt : true) ? 1 : 0;
    } else {
        c.norm_topk = 1;
    }
    // The logits head as the reference's loaders take it, whatever
    // tie_word_embeddings says: the dense decoder always multiplies by the
    // embedding table (qwen3_model.rs:187-206 builds no lm_head; model.rs:545
    // calls embed.logits), Qwen3-MoE always by lm_head.weight
    // (qwen3_moe_model.rs:337-343, 540).
    c.tied = c.n_experts == 0 ? 1 : 0;
    for (uint64_t v : {layers, hidden, heads, kv_heads, inter, vocab, has_hd ? hd : 0, has_ne ? ne : 0,
                       has_k ? k : 0, has_mi ? mi : 0})
        if (v > 0xFFFFFFFFull) return cfg_fail("a size does not fit 32 bits");
    *out = c;
    return WPCG_OK;
}

}  // namespace

using namespace wpcg;

extern "C" {

int wpcg_safetensors_open_file(const char* path, wpcg_safetensors** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (!path) return fail(WPCG_E_ARG, "null path");
    std::unique_ptr<wpcg_safetensors> st(new (std::nothrow) wpcg_safetensors);
    if (!st) return fail(WPCG_E_NOMEM, "safetensors");
    std::unique_ptr<StFile> f;
    if (int rc = open_file(path, f)) return rc;
    st->names = f->names;
    st->shards.push_back(std::move(f));
    *out = st.release();
    return WPCG_OK;
}

int wpcg_safetensors_open(const char* model_dir, wpcg_safetensors** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (!model_dir) return fail(WPCG_E_ARG, "null directory");
    const std::string dir(model_dir);
    const std::string single = dir + "/model.safetensors";
    if (file_exists(single)) return wpcg_safetensors_open_file(single.c_str(), out);
    const std::string index_path = dir + "/model.safetensors.index.json";
    std::ifstream in(index_path, std::ios::binary);
    if (!in) return fail(WPCG_E_IO, dir + ": contains neither model.safetensors nor model.safetensors.index.json");
    std::stringstream ss;
    ss << in.rdbuf();
    const std::string text = ss.str();
    JsonValue root;
    std::string err;
    if (!json_parse(text.data(), text.size(), root, err)) return fail(WPCG_E_FORMAT, index_path + ": " + err);
    const JsonValue* wm = root.get("weight_map");
    if (!wm || wm->kind != JsonValue::OBJ) return fail(WPCG_E_FORMAT, index_path + ": no `weight_map` object");
    std::unique_ptr<wpcg_safetensors> st(new (std::nothrow) wpcg_safetensors);
    if (!st) return fail(WPCG_E_NOMEM, "safetensors");
    // The reference walks serde_json's map: keys in sorted order, a repeated
    // key keeping its last value; shards open in that order.
    std::map<std::string, const JsonValue*> entries;
    for (const auto& kv : wm->obj) entries[kv.first] = &kv.second;
    std::unordered_map<std::string, size_t> shard_of_file;
    for (const auto& kv : entries) {
        if (kv.second->kind != JsonValue::STR) continue;  // a non-string entry is skipped
        const std::string& file = kv.second->str;
        size_t slot;
        auto it = shard_of_file.find(file);
        if (it != shard_of_file.end()) {
            slot = it->second;
        } else {
            std::unique_ptr<StFile> f;
            if (int rc = open_file(dir + "/" + file, f)) return rc;
            st->shards.push_back(std::move(f));
            slot = st->shards.size() - 1;
            shard_of_file[file] = slot;
        }
        st->index[kv.first] = slot;
    }
    if (st->shards.empty()) return fail(WPCG_E_FORMAT, index_path + ": the weight map names no shard");
    for (const auto& f : st->shards) st->names.insert(st->names.end(), f->names.begin(), f->names.end());
    *out = st.release();
    return WPCG_OK;
}

int wpcg_safetensors_close(wpcg_safetensors* st)
{
    delete st;
    return WPCG_OK;
}

int wpcg_safetensors_tensor_count(wpcg_safetensors* st, uint64_t* n)
{
    if (!st || !n) return fail(WPCG_E_ARG, "null argument");
    *n = st->names.size();
    return WPCG_OK;
}

int wpcg_safetensors_name(wpcg_safetensors* st, uint64_t i, const char** name)
{
    if (!st || !name) return fail(WPCG_E_ARG, "null argument");
    if (i >= st->names.size()) return fail(WPCG_E_ARG, "tensor index out of range");
    *name = st->names[i].c_str();
    return WPCG_OK;
}

int wpcg_safetensors_shape(wpcg_safetensors* st, const char* name, uint32_t* ndim, uint64_t* dims,
                           uint32_t max_dims)
{
    if (!ndim) return fail(WPCG_E_ARG, "null argument");
    const StFile* f;
    const StTensor* t;
    if (int rc = find(st, name, &f, &t)) return rc;
    *ndim = (uint32_t)t->shape.size();
    if (t->shape.size() > max_dims) return fail(WPCG_E_ARG, "tensor has more dimensions than dims holds");
    if (!dims && !t->shape.empty()) return fail(WPCG_E_ARG, "null dims");
    for (size_t i = 0; i < t->shape.size(); i++) dims[i] = t->shape[i];
    return WPCG_OK;
}

int wpcg_safetensors_dtype(wpcg_safetensors* st, const char* name, const char** dtype)
{
    if (!dtype) return fail(WPCG_E_ARG, "null argument");
    const StFile* f;
    const StTensor* t;
    if (int rc = find(st, name, &f, &t)) return rc;
    *dtype = t->dtype.c_str();
    return WPCG_OK;
}

int wpcg_safetensors_read_f32(wpcg_safetensors* st, const char* name, float* out, uint64_t n)
{
    const StFile* f;
    const StTensor* t;
    if (int rc = find(st, name, &f, &t)) return rc;
    const uint64_t c = count_of(*t);
    if (n != c) return fail(WPCG_E_SHAPE, std::string("tensor ") + name + " holds " + std::to_string(c) + " values");
    if (c && !out) return fail(WPCG_E_ARG, "null output");
    const uint8_t* p = f->data + t->begin;
    if (t->dtype == "F32") {
        std::memcpy(out, p, c * 4);  // little-endian host
    } else if (t->dtype == "F16") {
        for (uint64_t i = 0; i < c; i++) out[i] = f16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
    } else if (t->dtype == "BF16") {
        for (uint64_t i = 0; i < c; i++) {
            const uint32_t bits = ((uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 8)) << 16;
            std::memcpy(out + i, &bits, 4);
        }
    } else {
        return fail(WPCG_E_UNSUPPORTED, "unsupported dtype " + t->dtype + " for tensor " + name);
    }
    return WPCG_OK;
}

int wpcg_config_parse(const char* json_text, uint32_t max_pos, wpcg_model_config* out)
{
    if (!json_text || !out) return fail(WPCG_E_ARG, "null argument");
    return parse_config(json_text, std::strlen(json_text), max_pos, out);
}

int wpcg_config_load(const char* path, uint32_t max_pos, wpcg_model_config* out)
{
    if (!path || !out) return fail(WPCG_E_ARG, "null argument");
    std::ifstream in(path, std::ios::binary);
    if (!in) return fail(WPCG_E_IO, std::string("cannot read ") + path);
    std::stringstream ss;
    ss << in.rdbuf();
    const std::string text = ss.str();
    return parse_config(text.data(), text.size(), max_pos, out);
}

}  // extern "C"
