// gguf.cpp -- GGUF (v2/v3) reader and writer, and the loader that turns a
// Llama/Qwen3 GGUF into the decoder's weights.
//
// Format (the reference's parser: src/engine/model.cpp:445-657, doc
// docs/gguf.md): header {u32 magic "GGUF", u32 version, u64 n_tensors,
// u64 n_kv}; n_kv metadata pairs {string key, u32 type, value}; n_tensors
// infos {string name, u32 n_dims, u64 dims[n_dims] (dims[0] fastest), u32
// ggml type, u64 offset}; padding to `general.alignment` (default 32); the
// tensor data, each tensor at data_start + offset.  Strings are {u64 len,
// bytes}.  Value types 0..12: u8 i8 u16 i16 u32 i32 f32 bool string array
// u64 i64 f64; arrays are {u32 elem type, u64 count, elems}.
//
// The reader maps the file read-only and bounds-checks every field, so a
// truncated or malformed file is reported instead of read past its end.
// Config keys and tensor names follow the reference's loader
// (model.cpp:150-345 config, :675-810 tensor mapping, tied output fallback).
#include <hip/hip_runtime.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <math.h>
#include <new>
#include <string>
#include <vector>
#include "../../include/jllm_hip.h"
#include "capi_common.h"

namespace {

constexpr uint32_t GGUF_MAGIC = 0x46554747u;   // "GGUF" little-endian

struct KV {
    std::string key;
    uint32_t type = 0;
    uint64_t u = 0;          // integer / bool value (types 0-5, 7, 10, 11)
    double f = 0.0;          // float value (types 6, 12)
    std::string s;           // string value (type 8)
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;
    int64_t bytes = 0;
};

int64_t block_elems(uint32_t t) {
    switch (t) {
    case 0: case 1: case 30: return 1;                 // F32, F16, BF16
    case 2: case 3: case 6: case 7: case 8: case 9: return 32;
    case 10: case 11: case 12: case 13: case 14: return 256;
    default: return 0;
    }
}
int64_t block_bytes(uint32_t t) {
    switch (t) {
    case 0: return 4;  case 1: return 2;  case 30: return 2;
    case 2: return 18; case 3: return 20; case 6: return 22; case 7: return 24; case 8: return 34; case 9: return 36;
    case 10: return 84; case 11: return 110; case 12: return 144; case 13: return 176; case 14: return 210;
    default: return 0;
    }
}
int64_t tensor_bytes(uint32_t type, int64_t n) {
    const int64_t be = block_elems(type), bb = block_bytes(type);
    if (be <= 0 || n % be != 0) return -1;
    return n / be * bb;
}
int scalar_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

struct Cursor {
    const uint8_t* p;
    size_t n, off = 0;
    bool ok = true;
    bool take(void* dst, size_t k) {
        if (!ok || k > n - off) { ok = false; return false; }
        memcpy(dst, p + off, k);
        off += k;
        return true;
    }
    bool skip(uint64_t k) {
        if (!ok || k > n - off) { ok = false; return false; }
        off += k;
        return true;
    }
    bool str(std::string& s) {
        uint64_t len = 0;
        if (!take(&len, 8) || len > n - off) { ok = false; return false; }
        s.assign((const char*)p + off, len);
        off += len;
        return true;
    }
};

}  // namespace

struct jllm_hip_gguf {
    void* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    std::vector<KV> kv;
    std::vector<Tensor> tensors;
    size_t data_start = 0;
    const KV* find(const char* key) const {
        for (const auto& e : kv) if (e.key == key) return &e;
        return nullptr;
    }
    // first key ending in `suffix` (the architecture prefix varies: qwen3., llama. ...)
    const KV* find_suffix(const char* suffix) const {
        const size_t ls = strlen(suffix);
        for (const auto& e : kv)
            if (e.key.size() >= ls && e.key.compare(e.key.size() - ls, ls, suffix) == 0) return &e;
        return nullptr;
    }
};

struct jllm_hip_gguf_writer {
    std::vector<KV> kv;
    std::vector<Tensor> tensors;
    std::vector<std::vector<uint8_t>> data;
};

struct jllm_hip_gguf_model {
    void* arena = nullptr;
    jllm_hip_model_weights mw{};
    std::vector<jllm_hip_layer_weights> lw;
};

namespace {

bool parse(jllm_hip_gguf* g) {
    Cursor c{(const uint8_t*)g->map, g->size};
    uint32_t magic = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    c.take(&magic, 4);
    c.take(&g->version, 4);
    c.take(&n_tensors, 8);
    c.take(&n_kv, 8);
    if (!c.ok || magic != GGUF_MAGIC || g->version < 2 || g->version > 3) {
        fprintf(stderr, "[gguf] not a GGUF v2/v3 file\n");
        return false;
    }
    if (n_kv > (1u << 24) || n_tensors > (1u << 24)) { fprintf(stderr, "[gguf] implausible counts\n"); return false; }
    for (uint64_t i = 0; i < n_kv && c.ok; i++) {
        KV e;
        c.str(e.key);
        c.take(&e.type, 4);
        const int sz = scalar_size(e.type);
        if (sz > 0) {
            uint8_t b[8] = {};
            c.take(b, sz);
            if (e.type == 6) { float v; memcpy(&v, b, 4); e.f = v; }
            else if (e.type == 12) { double v; memcpy(&v, b, 8); e.f = v; }
            else if (e.type == 1) e.u = (uint64_t)(int64_t)(int8_t)b[0];
            else if (e.type == 3) { int16_t v; memcpy(&v, b, 2); e.u = (uint64_t)(int64_t)v; }
            else if (e.type == 5) { int32_t v; memcpy(&v, b, 4); e.u = (uint64_t)(int64_t)v; }
            else memcpy(&e.u, b, sz);
        } else if (e.type == 8) {
            c.str(e.s);
        } else if (e.type == 9) {
            uint32_t at = 0;
            uint64_t an = 0;
            c.take(&at, 4);
            c.take(&an, 8);
            e.u = an;
            const int esz = scalar_size(at);
            if (esz > 0) {
                if (an > (c.n - c.off) / esz) { c.ok = false; break; }
                c.skip(an * esz);
            } else if (at == 8) {
                for (uint64_t a = 0; a < an && c.ok; a++) { std::string s; c.str(s); }
            } else {
                fprintf(stderr, "[gguf] nested array in '%s' not supported\n", e.key.c_str());
                return false;
            }
        } else {
            fprintf(stderr, "[gguf] unknown value type %u for '%s'\n", e.type, e.key.c_str());
            return false;
        }
        g->kv.push_back(std::move(e));
    }
    for (uint64_t i = 0; i < n_tensors && c.ok; i++) {
        Tensor t;
        c.str(t.name);
        c.take(&t.n_dims, 4);
        if (!c.ok || t.n_dims < 1 || t.n_dims > 4) { fprintf(stderr, "[gguf] bad tensor rank\n"); return false; }
        int64_t n = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            uint64_t v = 0;
            c.take(&v, 8);
            if (v == 0 || v > ((uint64_t)1 << 40) || n > ((int64_t)1 << 50) / (int64_t)v) { c.ok = false; break; }
            t.dims[d] = (int64_t)v;
            n *= (int64_t)v;
        }
        c.take(&t.type, 4);
        c.take(&t.offset, 8);
        t.bytes = tensor_bytes(t.type, n);
        if (!c.ok || t.bytes < 0) {
            fprintf(stderr, "[gguf] tensor '%s': unsupported type %u or size\n", t.name.c_str(), t.type);
            return false;
        }
        g->tensors.push_back(std::move(t));
    }
    if (!c.ok) { fprintf(stderr, "[gguf] truncated file\n"); return false; }
    uint64_t align = 32;
    if (const KV* a = g->find("general.alignment")) {
        // the spec's alignment is a power of two (a u32); anything else would
        // misplace every tensor
        if (scalar_size(a->type) == 0 || a->type == 6 || a->type == 12 || a->u == 0 || a->u > 65536 ||
            (a->u & (a->u - 1)) != 0) {
            fprintf(stderr, "[gguf] general.alignment must be a power of two <= 65536\n");
            return false;
        }
        align = a->u;
    }
    g->data_start = (c.off + align - 1) / align * align;
    for (const auto& t : g->tensors) {
        if (t.offset % align != 0 || t.offset > g->size || (uint64_t)t.bytes > g->size ||
            g->data_start + t.offset + (uint64_t)t.bytes > g->size) {
            fprintf(stderr, "[gguf] tensor '%s' lies outside the file or is misaligned\n", t.name.c_str());
            return false;
        }
    }
    return true;
}

bool wr(FILE* f, const void* p, size_t n) { return fwrite(p, 1, n, f) == n; }
bool wr_str(FILE* f, const std::string& s) {
    const uint64_t n = s.size();
    return wr(f, &n, 8) && wr(f, s.data(), n);
}

}  // namespace

extern "C" {

jllm_hip_gguf* jllm_hip_gguf_open(const char* path) {
    if (!path) return nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { fprintf(stderr, "[gguf] cannot open %s\n", path); return nullptr; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) { close(fd); fprintf(stderr, "[gguf] %s: too small\n", path); return nullptr; }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) { fprintf(stderr, "[gguf] mmap of %s failed\n", path); return nullptr; }
    jllm_hip_gguf* g = new (std::nothrow) jllm_hip_gguf();
    if (!g) { munmap(m, (size_t)st.st_size); return nullptr; }
    g->map = m;
    g->size = (size_t)st.st_size;
    if (!parse(g)) { jllm_hip_gguf_close(g); return nullptr; }
    return g;
}

void jllm_hip_gguf_close(jllm_hip_gguf* g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    delete g;
}

int64_t jllm_hip_gguf_n_tensors(const jllm_hip_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int64_t jllm_hip_gguf_find_tensor(const jllm_hip_gguf* g, const char* name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); i++) if (g->tensors[i].name == name) return (int64_t)i;
    return -1;
}

int jllm_hip_gguf_tensor(const jllm_hip_gguf* g, int64_t i, const char** name, int* ggml_type, int* n_dims,
                         int64_t* dims, const void** data, int64_t* bytes) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return JLLM_ERR_INVALID;
    const Tensor& t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = (int)t.type;
    if (n_dims) *n_dims = (int)t.n_dims;
    if (dims) for (int d = 0; d < 4; d++) dims[d] = t.dims[d];
    if (data) *data = (const uint8_t*)g->map + g->data_start + t.offset;
    if (bytes) *bytes = t.bytes;
    return JLLM_OK;
}

int jllm_hip_gguf_get_u64(const jllm_hip_gguf* g, const char* key, uint64_t* out) {
    const KV* e = g && key ? g->find(key) : nullptr;
    if (!e || !out || scalar_size(e->type) == 0 || e->type == 6 || e->type == 12) return JLLM_ERR_INVALID;
    *out = e->u;
    return JLLM_OK;
}

int jllm_hip_gguf_get_f64(const jllm_hip_gguf* g, const char* key, double* out) {
    const KV* e = g && key ? g->find(key) : nullptr;
    if (!e || !out || (e->type != 6 && e->type != 12)) return JLLM_ERR_INVALID;
    *out = e->f;
    return JLLM_OK;
}

const char* jllm_hip_gguf_get_str(const jllm_hip_gguf* g, const char* key) {
    const KV* e = g && key ? g->find(key) : nullptr;
    return e && e->type == 8 ? e->s.c_str() : nullptr;
}

int jllm_hip_gguf_config(const jllm_hip_gguf* g, jllm_hip_decoder_config* cfg) {
    if (!g || !cfg) return JLLM_ERR_INVALID;
    jllm_hip_decoder_config c{};
    auto u = [&](const char* suffix, int def) -> int {
        const KV* e = g->find_suffix(suffix);
        return e && scalar_size(e->type) > 0 && e->type != 6 && e->type != 12 ? (int)e->u : def;
    };
    auto f = [&](const char* suffix, float def) -> float {
        const KV* e = g->find_suffix(suffix);
        return e && (e->type == 6 || e->type == 12) ? (float)e->f : def;
    };
    c.n_layers = u(".block_count", 0);
    c.hidden_dim = u(".embedding_length", 0);
    c.n_heads = u(".attention.head_count", 0);
    c.n_kv_heads = u(".attention.head_count_kv", c.n_heads);
    c.head_dim = u(".attention.key_length", c.n_heads > 0 ? c.hidden_dim / c.n_heads : 0);
    c.intermediate_dim = u(".feed_forward_length", 0);
    c.vocab_size = u(".vocab_size", 0);
    c.max_seq = u(".context_length", 4096);
    c.rms_eps = f(".attention.layer_norm_rms_epsilon", 1e-6f);
    c.rope_theta = f(".rope.freq_base", 10000.0f);
    const char* arch = jllm_hip_gguf_get_str(g, "general.architecture");
    const std::string a = arch ? arch : "";
    c.rope_neox = (a == "qwen" || a == "qwen2" || a == "qwen3" || a == "qwen2moe" || a == "qwen3moe" ||
                   a == "gemma" || a == "gemma2" || a == "gemma3" || a == "phi2" || a == "phi3" ||
                   a == "gptneox" || a == "olmo" || a == "olmo2") ? 1 : 0;
    const int64_t te = jllm_hip_gguf_find_tensor(g, "token_embd.weight");
    if (c.vocab_size == 0 && te >= 0) c.vocab_size = (int)g->tensors[(size_t)te].dims[1];
    auto type_of = [&](const char* name, int def) {
        const int64_t i = jllm_hip_gguf_find_tensor(g, name);
        return i >= 0 ? (int)g->tensors[(size_t)i].type : def;
    };
    c.norm_fp32 = type_of("blk.0.attn_norm.weight", 0) == 0;
    c.qk_norm_fp32 = type_of("blk.0.attn_q_norm.weight", 0) == 0;
    c.output_norm_fp32 = type_of("output_norm.weight", 0) == 0;
    c.kv_int8 = 1;
    if (c.n_layers <= 0 || c.hidden_dim <= 0 || c.n_heads <= 0 || c.vocab_size <= 0 || c.intermediate_dim <= 0) {
        fprintf(stderr, "[gguf] metadata lacks the model shape\n");
        return JLLM_ERR_INVALID;
    }
    if (!jllm_hip::decoder_config_ok(c)) return JLLM_ERR_UNSUPPORTED;
    *cfg = c;
    return JLLM_OK;
}

jllm_hip_gguf_model* jllm_hip_gguf_model_load(const jllm_hip_gguf* g, const jllm_hip_decoder_config* cfg) {
    if (!g || !cfg || cfg->n_layers <= 0) return nullptr;
    jllm_hip_gguf_model* m = new (std::nothrow) jllm_hip_gguf_model();
    if (!m) return nullptr;
    m->lw.assign((size_t)cfg->n_layers, jllm_hip_layer_weights{});
    // one device allocation for every tensor the decoder uses (256-byte aligned)
    struct Use { const Tensor* t; const void** dst; int* type; };
    std::vector<Use> uses;
    bool shape_ok = true;
    // a used tensor must have the shape the kernels will index with: a K-quant
    // matrix [K, M] (dims[0] fastest) of type 12-14, a norm vector [n] of F32
    // (type 0) when fp32 is 1, else F16 (type 1); anything else would make
    // the kernels read past the tensor's slot in the arena
    auto check = [&](const Tensor& t, int64_t d0, int64_t d1, int fp32) {
        bool good;
        if (d1 > 0) good = t.n_dims == 2 && t.dims[0] == d0 && t.dims[1] == d1 && t.type >= 12 && t.type <= 14;
        else good = t.n_dims == 1 && t.dims[0] == d0 && t.type == (fp32 ? 0u : 1u);
        if (!good) {
            fprintf(stderr, "[gguf] tensor '%s': type %u, %u dims [%lld, %lld]; the configuration needs ",
                    t.name.c_str(), t.type, t.n_dims, (long long)t.dims[0], (long long)(t.n_dims > 1 ? t.dims[1] : 0));
            if (d1 > 0) fprintf(stderr, "a Q4_K/Q5_K/Q6_K matrix [%lld, %lld]\n", (long long)d0, (long long)d1);
            else fprintf(stderr, "an %s vector [%lld]\n", fp32 ? "F32" : "F16", (long long)d0);
            shape_ok = false;
        }
    };
    auto want = [&](const std::string& name, const void** dst, int* type, int64_t d0, int64_t d1, int fp32) {
        const int64_t i = jllm_hip_gguf_find_tensor(g, name.c_str());
        if (i >= 0) {
            check(g->tensors[(size_t)i], d0, d1, fp32);
            uses.push_back({&g->tensors[(size_t)i], dst, type});
        }
        return i >= 0;
    };
    const int64_t H = cfg->hidden_dim, QD = (int64_t)cfg->n_heads * cfg->head_dim,
                  KVD = (int64_t)cfg->n_kv_heads * cfg->head_dim, I = cfg->intermediate_dim, V = cfg->vocab_size;
    bool ok = want("token_embd.weight", &m->mw.tok_embd, &m->mw.embd_type, H, V, 0);
    ok &= want("output_norm.weight", &m->mw.output_norm, nullptr, H, 0, cfg->output_norm_fp32);
    // tied embeddings: without output.weight the output projection re-uses
    // token_embd (model.cpp:791-806)
    const bool tied = !want("output.weight", &m->mw.output, &m->mw.output_type, H, V, 0);
    for (int l = 0; l < cfg->n_layers; l++) {
        jllm_hip_layer_weights& w = m->lw[(size_t)l];
        const std::string p = "blk." + std::to_string(l) + ".";
        ok &= want(p + "attn_q.weight", &w.wq, &w.type_wq, H, QD, 0);
        ok &= want(p + "attn_k.weight", &w.wk, &w.type_wk, H, KVD, 0);
        ok &= want(p + "attn_v.weight", &w.wv, &w.type_wv, H, KVD, 0);
        ok &= want(p + "attn_output.weight", &w.wo, &w.type_wo, QD, H, 0);
        ok &= want(p + "ffn_gate.weight", &w.w_gate, &w.type_w_gate, H, I, 0);
        ok &= want(p + "ffn_up.weight", &w.w_up, &w.type_w_up, H, I, 0);
        ok &= want(p + "ffn_down.weight", &w.w_down, &w.type_w_down, I, H, 0);
        ok &= want(p + "attn_norm.weight", &w.rms_attn, nullptr, H, 0, cfg->norm_fp32);
        ok &= want(p + "ffn_norm.weight", &w.rms_ffn, nullptr, H, 0, cfg->norm_fp32);
        const bool qn = want(p + "attn_q_norm.weight", &w.q_norm, nullptr, cfg->head_dim, 0, cfg->qk_norm_fp32);
        const bool kn = want(p + "attn_k_norm.weight", &w.k_norm, nullptr, cfg->head_dim, 0, cfg->qk_norm_fp32);
        if (qn != kn) {
            fprintf(stderr, "[gguf] layer %d has only one of attn_q_norm / attn_k_norm\n", l);
            shape_ok = false;
        }
    }
    if (!ok) {
        fprintf(stderr, "[gguf] the file lacks tensors of the Llama/Qwen3 decoder\n");
        delete m;
        return nullptr;
    }
    if (!shape_ok) {
        delete m;
        return nullptr;
    }
    size_t total = 0;
    std::vector<size_t> off(uses.size());
    for (size_t i = 0; i < uses.size(); i++) { off[i] = total; total += ((size_t)uses[i].t->bytes + 255) & ~(size_t)255; }
    if (hipMalloc(&m->arena, total) != hipSuccess) {
        fprintf(stderr, "[gguf] hipMalloc of %zu bytes failed\n", total);
        delete m;
        return nullptr;
    }
    for (size_t i = 0; i < uses.size(); i++) {
        uint8_t* d = (uint8_t*)m->arena + off[i];
        const uint8_t* s = (const uint8_t*)g->map + g->data_start + uses[i].t->offset;
        if (hipMemcpy(d, s, (size_t)uses[i].t->bytes, hipMemcpyHostToDevice) != hipSuccess) {
            fprintf(stderr, "[gguf] upload of '%s' failed\n", uses[i].t->name.c_str());
            jllm_hip_gguf_model_free(m);
            return nullptr;
        }
        *uses[i].dst = d;
        if (uses[i].type) *uses[i].type = (int)uses[i].t->type;
    }
    if (tied) { m->mw.output = m->mw.tok_embd; m->mw.output_type = m->mw.embd_type; }
    return m;
}

const jllm_hip_model_weights* jllm_hip_gguf_model_weights(const jllm_hip_gguf_model* m) { return m ? &m->mw : nullptr; }
const jllm_hip_layer_weights* jllm_hip_gguf_layer_weights(const jllm_hip_gguf_model* m) {
    return m && !m->lw.empty() ? m->lw.data() : nullptr;
}

void jllm_hip_gguf_model_free(jllm_hip_gguf_model* m) {
    if (!m) return;
    if (m->arena) (void)hipFree(m->arena);
    delete m;
}

jllm_hip_gguf_writer* jllm_hip_gguf_writer_create(void) { return new (std::nothrow) jllm_hip_gguf_writer(); }
void jllm_hip_gguf_writer_free(jllm_hip_gguf_writer* w) { delete w; }

int jllm_hip_gguf_writer_set_u32(jllm_hip_gguf_writer* w, const char* key, uint32_t v) {
    if (!w || !key) return JLLM_ERR_INVALID;
    KV e; e.key = key; e.type = 4; e.u = v;
    w->kv.push_back(e);
    return JLLM_OK;
}
int jllm_hip_gguf_writer_set_f32(jllm_hip_gguf_writer* w, const char* key, float v) {
    if (!w || !key) return JLLM_ERR_INVALID;
    KV e; e.key = key; e.type = 6; e.f = v;
    w->kv.push_back(e);
    return JLLM_OK;
}
int jllm_hip_gguf_writer_set_str(jllm_hip_gguf_writer* w, const char* key, const char* v) {
    if (!w || !key || !v) return JLLM_ERR_INVALID;
    KV e; e.key = key; e.type = 8; e.s = v;
    w->kv.push_back(e);
    return JLLM_OK;
}

int jllm_hip_gguf_writer_add_tensor(jllm_hip_gguf_writer* w, const char* name, int ggml_type, int n_dims,
                                    const int64_t* dims, const void* data, int64_t bytes) {
    if (!w || !name || !dims || !data || n_dims < 1 || n_dims > 4) return JLLM_ERR_INVALID;
    Tensor t;
    t.name = name; t.type = (uint32_t)ggml_type; t.n_dims = (uint32_t)n_dims;
    int64_t n = 1;
    for (int d = 0; d < n_dims; d++) { if (dims[d] <= 0) return JLLM_ERR_INVALID; t.dims[d] = dims[d]; n *= dims[d]; }
    t.bytes = tensor_bytes(t.type, n);
    if (t.bytes != bytes) return JLLM_ERR_INVALID;
    w->tensors.push_back(t);
    w->data.emplace_back((const uint8_t*)data, (const uint8_t*)data + bytes);
    return JLLM_OK;
}

int jllm_hip_gguf_writer_write(const jllm_hip_gguf_writer* w, const char* path) {
    if (!w || !path) return JLLM_ERR_INVALID;
    // the alignment the file declares (general.alignment), else the spec's 32
    uint64_t align = 32;
    for (const auto& e : w->kv)
        if (e.key == "general.alignment") {
            if (e.type != 4 || e.u == 0 || e.u > 65536 || (e.u & (e.u - 1)) != 0) return JLLM_ERR_INVALID;
            align = e.u;
        }
    FILE* f = fopen(path, "wb");
    if (!f) return JLLM_ERR_INVALID;
    bool ok = true;
    const uint32_t magic = GGUF_MAGIC, version = 3;
    const uint64_t nt = w->tensors.size(), nkv = w->kv.size();
    ok &= wr(f, &magic, 4) && wr(f, &version, 4) && wr(f, &nt, 8) && wr(f, &nkv, 8);
    for (const auto& e : w->kv) {
        ok &= wr_str(f, e.key) && wr(f, &e.type, 4);
        if (e.type == 4) { const uint32_t v = (uint32_t)e.u; ok &= wr(f, &v, 4); }
        else if (e.type == 6) { const float v = (float)e.f; ok &= wr(f, &v, 4); }
        else ok &= wr_str(f, e.s);
    }
    uint64_t off = 0;
    for (const auto& t : w->tensors) {
        ok &= wr_str(f, t.name) && wr(f, &t.n_dims, 4);
        for (uint32_t d = 0; d < t.n_dims; d++) { const uint64_t v = (uint64_t)t.dims[d]; ok &= wr(f, &v, 8); }
        ok &= wr(f, &t.type, 4) && wr(f, &off, 8);
        off += ((uint64_t)t.bytes + align - 1) / align * align;
    }
    const uint8_t zeros[256] = {};
    auto pad_to = [&](uint64_t n) {          // n zero bytes
        while (ok && n > 0) {
            const size_t k = n < sizeof(zeros) ? (size_t)n : sizeof(zeros);
            ok &= wr(f, zeros, k);
            n -= k;
        }
    };
    long pos = ftell(f);
    ok &= pos >= 0;
    if (ok) pad_to(((uint64_t)pos + align - 1) / align * align - (uint64_t)pos);
    for (size_t i = 0; i < w->tensors.size(); i++) {
        const size_t b = w->data[i].size();
        ok &= wr(f, w->data[i].data(), b);
        pad_to(((uint64_t)b + align - 1) / align * align - b);
    }
    ok &= fclose(f) == 0;
    return ok ? JLLM_OK : JLLM_ERR_INVALID;
}

}  // extern "C"
