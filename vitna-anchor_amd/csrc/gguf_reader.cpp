/**
 * gguf_reader.cpp - A GGUF checkpoint read into the engine's vitna_llama_t
 * (include/vitna_gguf.h), host code only.
 *
 * Reference counterparts:
 *   vitna_hip_gguf_open   engine/src/gguf.c:229-478 (vitna_gguf_open, one unsplit file)
 *   name map              engine/src/gguf.c:160-214 (LAYER_PARTS, MODEL_PARTS, hf_name)
 *   vitna_hip_gguf_llama  engine/src/model.c:160-175 (gguf_disagrees), :259-305 (bind,
 *                         norm_weights), :302-410 (vitna_llama_load_ex)
 *
 * The file format, little-endian: "GGUF", u32 version, u64 tensor count, u64
 * metadata count; each metadata entry a string key, a u32 type and a value
 * (scalars, strings, arrays of either); each tensor a string name, u32 dims,
 * u64 extents (fastest first), u32 ggml type, u64 offset; the data section
 * at the next multiple of general.alignment (32 when absent). Every read is
 * checked against the bytes left in the mapping before it is made.
 */

#include "../../include/vitna_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

bool say(char* err, size_t len, const char* fmt, ...) {
    if (err && len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, len, fmt, ap);
        va_end(ap);
    }
    return false;
}

/* ggml type ids (ggml.h's enum ggml_type) of the formats the engine computes with. */
vitna_dtype_t dtype_of_ggml(uint32_t t) {
    switch (t) {
        case 0: return VITNA_DTYPE_F32;
        case 1: return VITNA_DTYPE_F16;
        case 8: return VITNA_DTYPE_Q8_0;
        case 10: return VITNA_DTYPE_Q2_K;
        case 11: return VITNA_DTYPE_Q3_K;
        case 12: return VITNA_DTYPE_Q4_K;
        case 13: return VITNA_DTYPE_Q5_K;
        case 14: return VITNA_DTYPE_Q6_K;
        case 30: return VITNA_DTYPE_BF16;
        default: return VITNA_DTYPE_UNKNOWN;
    }
}

const char* dtype_text(vitna_dtype_t t) {
    switch (t) {
        case VITNA_DTYPE_F32: return "F32";
        case VITNA_DTYPE_F16: return "F16";
        case VITNA_DTYPE_BF16: return "BF16";
        case VITNA_DTYPE_Q8_0: return "Q8_0";
        case VITNA_DTYPE_Q2_K: return "Q2_K";
        case VITNA_DTYPE_Q3_K: return "Q3_K";
        case VITNA_DTYPE_Q4_K: return "Q4_K";
        case VITNA_DTYPE_Q5_K: return "Q5_K";
        case VITNA_DTYPE_Q6_K: return "Q6_K";
        default: return "an unsupported type";
    }
}

/* Metadata value types of the format. */
enum : uint32_t { M_U8, M_I8, M_U16, M_I16, M_U32, M_I32, M_F32, M_BOOL, M_STR, M_ARR, M_U64, M_I64, M_F64 };

size_t scalar_bytes(uint32_t t) {
    switch (t) {
        case M_U8: case M_I8: case M_BOOL: return 1;
        case M_U16: case M_I16: return 2;
        case M_U32: case M_I32: case M_F32: return 4;
        case M_U64: case M_I64: case M_F64: return 8;
        default: return 0;
    }
}

/* A bounds-checked reader over the mapping; any short read clears ok and every later read returns zero. */
struct reader {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;

    bool has(uint64_t n) {
        if (ok && (uint64_t)(end - p) < n) ok = false;
        return ok;
    }
    uint64_t le(int n) {
        if (!has((uint64_t)n)) return 0;
        uint64_t v = 0;
        for (int i = n - 1; i >= 0; i--) v = v << 8 | p[i];
        p += n;
        return v;
    }
    bool str(std::string* s) {
        const uint64_t n = le(8);
        if (!has(n)) return false;
        if (s) s->assign((const char*)p, (size_t)n);
        p += n;
        return true;
    }
    double number(uint32_t t) {
        const uint64_t u = le((int)scalar_bytes(t));
        switch (t) {
            case M_I8: return (double)(int8_t)u;
            case M_I16: return (double)(int16_t)u;
            case M_I32: return (double)(int32_t)u;
            case M_I64: return (double)(int64_t)u;
            case M_F32: { const uint32_t b = (uint32_t)u; float f; memcpy(&f, &b, 4); return (double)f; }
            case M_F64: { double d; memcpy(&d, &u, 8); return d; }
            default: return (double)u;
        }
    }
    /* step over a value: a scalar, a string, or an array (nested up to four deep) */
    bool skip(uint32_t t, int depth) {
        if (scalar_bytes(t)) return has(scalar_bytes(t)) && (p += scalar_bytes(t), true);
        if (t == M_STR) return str(nullptr);
        if (t != M_ARR || depth >= 4) return ok = false;
        const uint32_t et = (uint32_t)le(4);
        const uint64_t n = le(8);
        if (!ok) return false;
        if (scalar_bytes(et)) {
            if (n > (uint64_t)(end - p) / scalar_bytes(et)) return ok = false;
            p += n * scalar_bytes(et);
            return true;
        }
        for (uint64_t i = 0; i < n && ok; i++) skip(et, depth + 1);
        return ok;
    }
};

/* Where a llama.cpp tensor name goes under the Hugging Face names (the format's mapping, engine/src/gguf.c:160-183):
   per-layer parts, and whether the tensor is a stack of experts split one tensor per expert. */
struct part_map {
    const char* gguf;
    const char* hf;
    bool stack;
};
const part_map k_layer_parts[] = {
    {"attn_norm", "input_layernorm", false},      {"attn_q", "self_attn.q_proj", false},
    {"attn_k", "self_attn.k_proj", false},        {"attn_v", "self_attn.v_proj", false},
    {"attn_output", "self_attn.o_proj", false},   {"attn_q_norm", "self_attn.q_norm", false},
    {"attn_k_norm", "self_attn.k_norm", false},   {"ffn_norm", "post_attention_layernorm", false},
    {"ffn_gate_inp", "mlp.gate", false},          {"ffn_gate", "mlp.gate_proj", false},
    {"ffn_up", "mlp.up_proj", false},             {"ffn_down", "mlp.down_proj", false},
    {"ffn_gate_exps", "gate_proj", true},         {"ffn_up_exps", "up_proj", true},
    {"ffn_down_exps", "down_proj", true},
};
const part_map k_model_parts[] = {
    {"token_embd.weight", "model.embed_tokens.weight", false},
    {"output_norm.weight", "model.norm.weight", false},
    {"output.weight", "lm_head.weight", false},
};

/* name -> (Hugging Face name or, for a stack, the per-expert part), layer. */
bool map_name(const std::string& name, std::string* hf, bool* stack, size_t* layer, const char** stack_part) {
    *stack = false;
    for (const part_map& m : k_model_parts)
        if (name == m.gguf) {
            *hf = m.hf;
            return true;
        }
    if (name.compare(0, 4, "blk.") != 0 || name.size() < 6 || !isdigit((unsigned char)name[4])) return false;
    size_t i = 4;
    unsigned long l = 0;
    while (i < name.size() && isdigit((unsigned char)name[i])) {
        l = l * 10 + (unsigned long)(name[i] - '0');
        if (l > 100000) return false;
        i++;
    }
    if (i >= name.size() || name[i] != '.') return false;
    const std::string rest = name.substr(i + 1);
    const size_t dot = rest.rfind('.');
    if (dot == std::string::npos || rest.substr(dot) != ".weight") return false;
    const std::string part = rest.substr(0, dot);
    for (const part_map& m : k_layer_parts)
        if (part == m.gguf) {
            *layer = (size_t)l;
            *stack = m.stack;
            *stack_part = m.hf;
            if (!m.stack) *hf = "model.layers." + std::to_string(l) + "." + m.hf + ".weight";
            return true;
        }
    return false;
}

/* Bytes of one row of cols weights, or 0 for a width the dtype does not take. Widths of 2^40 weights and more
   are refused before any multiplication, so a hostile shape cannot wrap the product to a small row. */
uint64_t row_bytes_of(vitna_dtype_t t, uint64_t cols) {
    if (cols >= ((uint64_t)1 << 40)) return 0;
    switch (t) {
        case VITNA_DTYPE_F32: return cols * 4;
        case VITNA_DTYPE_F16: case VITNA_DTYPE_BF16: return cols * 2;
        case VITNA_DTYPE_Q8_0: return cols % 32 ? 0 : cols / 32 * 34;
        case VITNA_DTYPE_Q2_K: return cols % 256 ? 0 : cols / 256 * 84;
        case VITNA_DTYPE_Q3_K: return cols % 256 ? 0 : cols / 256 * 110;
        case VITNA_DTYPE_Q4_K: return cols % 256 ? 0 : cols / 256 * 144;
        case VITNA_DTYPE_Q5_K: return cols % 256 ? 0 : cols / 256 * 176;
        case VITNA_DTYPE_Q6_K: return cols % 256 ? 0 : cols / 256 * 210;
        default: return 0;
    }
}

float half_value(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, f = h & 1023;
    uint32_t bits;
    if (e == 0) {
        if (f == 0) {
            bits = s;
        } else { /* subnormal: normalize */
            int sh = 0;
            uint32_t m = f;
            while (!(m & 1024)) { m <<= 1; sh++; }
            bits = s | (uint32_t)(127 - 15 + 1 - sh) << 23 | (m & 1023) << 13;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | f << 13;
    } else {
        bits = s | (e + 127 - 15) << 23 | f << 13;
    }
    float v;
    memcpy(&v, &bits, 4);
    return v;
}

}  // namespace

struct vitna_hip_gguf {
    void* map = nullptr;
    size_t size = 0;
    uint64_t data_offset = 0;
    vitna_hip_gguf_info_t info{};
    std::vector<vitna_hip_gguf_tensor_t> tensors;

    const vitna_hip_gguf_tensor_t* find(const std::string& name) const {
        for (const vitna_hip_gguf_tensor_t& t : tensors)
            if (name == t.name) return &t;
        return nullptr;
    }
};

extern "C" vitna_hip_gguf_t* vitna_hip_gguf_open(const char* path, vitna_hip_gguf_info_t* info_out, char* err, size_t err_len) {
    if (err && err_len) err[0] = 0;
    if (!path) { say(err, err_len, "no path"); return nullptr; }
    const int fd = open(path, O_RDONLY);
    struct stat st;
    if (fd < 0 || fstat(fd, &st) != 0 || st.st_size <= 0) {
        if (fd >= 0) close(fd);
        say(err, err_len, "cannot open or map %s", path);
        return nullptr;
    }
    void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) { say(err, err_len, "cannot open or map %s", path); return nullptr; }
    vitna_hip_gguf* g = new vitna_hip_gguf();
    g->map = map;
    g->size = (size_t)st.st_size;
    auto bad = [&](const char* fmt, ...) -> vitna_hip_gguf_t* {
        if (err && err_len) {
            char msg[400];
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(msg, sizeof(msg), fmt, ap);
            va_end(ap);
            snprintf(err, err_len, "%s: %s", path, msg);
        }
        vitna_hip_gguf_close(g);
        return nullptr;
    };
    vitna_hip_gguf_info_t& info = g->info;
    reader r{(const uint8_t*)map, (const uint8_t*)map + g->size};
    const uint32_t magic = (uint32_t)r.le(4);
    info.version = (uint32_t)r.le(4);
    const uint64_t n_tensors = r.le(8), n_meta = r.le(8);
    if (!r.ok || magic != 0x46554747u) return bad("not a GGUF file");
    if (info.version != 2 && info.version != 3) return bad("GGUF version %u; versions 2 and 3 are read", info.version);
    if (n_meta > g->size / 16 || n_tensors > g->size / 16) return bad("more metadata or tensors than the file could hold");

    /* metadata: the architecture, the alignment, and every scalar kept by key */
    std::vector<std::pair<std::string, double>> nums;
    info.alignment = 32;
    for (uint64_t i = 0; i < n_meta && r.ok; i++) {
        std::string key;
        if (!r.str(&key)) break;
        const uint32_t t = (uint32_t)r.le(4);
        if (!r.ok) break;
        if (t == M_STR && key == "general.architecture") {
            std::string a;
            if (!r.str(&a)) break;
            if (a.size() >= sizeof(info.arch)) return bad("general.architecture is too long");
            memcpy(info.arch, a.data(), a.size());
            info.arch[a.size()] = 0;
        } else if (scalar_bytes(t)) {
            const double v = r.number(t);
            if (key == "general.alignment") info.alignment = (uint64_t)v;
            nums.emplace_back(key, v);
        } else {
            r.skip(t, 0);
        }
    }
    if (!r.ok) return bad("its metadata runs past the end of the file, or holds a type GGUF does not have");
    auto meta = [&](const std::string& key, double* v) {
        for (const auto& kv : nums)
            if (kv.first == key) { *v = kv.second; return true; }
        return false;
    };
    double sno = 0, scnt = 0, stc = 0;
    meta("split.no", &sno);
    meta("split.count", &scnt);
    meta("split.tensors.count", &stc);
    if (!(sno >= 0 && sno <= 4096 && sno == (double)(uint16_t)sno) || !(scnt >= 0 && scnt <= 4096 && scnt == (double)(uint16_t)scnt) ||
        !(stc >= 0 && stc <= 1e12 && stc == (double)(uint64_t)stc))
        return bad("invalid split metadata");
    info.split_no = (uint16_t)sno;
    info.split_count = (uint16_t)scnt;
    info.split_tensors_count = (uint64_t)stc;
    if (info.split_count > 1) return bad("one shard of %u: this reader takes a checkpoint in one file", (unsigned)info.split_count);
    if (info.split_no != 0) return bad("split.no (%u) set without split.count > 1", (unsigned)info.split_no);
    if (!info.arch[0]) return bad("no general.architecture");
    if (strcmp(info.arch, "llama") == 0)
        return bad("llama.cpp writes a llama model's query and key rows permuted, and this engine does not put them back");
    if (info.alignment == 0 || info.alignment > (1u << 20) || (info.alignment & (info.alignment - 1)))
        return bad("general.alignment is not a power of two up to 1 MiB");
    {
        const std::string a = std::string(info.arch) + ".";
        double v = 0;
        auto u = [&](const char* k) -> uint64_t { return meta(a + k, &v) && v >= 0 ? (uint64_t)v : 0; };
        info.block_count = u("block_count");
        info.embedding_length = u("embedding_length");
        info.feed_forward_length = u("feed_forward_length");
        info.expert_feed_forward_length = u("expert_feed_forward_length");
        info.head_count = u("attention.head_count");
        info.head_count_kv = u("attention.head_count_kv");
        info.key_length = u("attention.key_length");
        info.context_length = u("context_length");
        info.expert_count = u("expert_count");
        info.expert_used_count = u("expert_used_count");
        info.rms_eps = meta(a + "attention.layer_norm_rms_epsilon", &v) ? v : 0.0;
        info.rope_freq_base = meta(a + "rope.freq_base", &v) ? v : 0.0;
    }

    /* the tensor directory */
    struct listed {
        std::string name;
        uint32_t dims;
        uint64_t ne[3];
        uint32_t type;
        uint64_t offset;
    };
    std::vector<listed> files;
    files.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        listed t{};
        if (!r.str(&t.name)) break;
        if (t.name.size() > 255) return bad("a tensor name is longer than 255 bytes");
        t.dims = (uint32_t)r.le(4);
        if (!r.ok) break;
        if (t.dims < 1 || t.dims > 3) return bad("tensor %s has %u dimensions; 1 to 3 are read", t.name.c_str(), t.dims);
        for (uint32_t d = 0; d < t.dims; d++) t.ne[d] = r.le(8);
        t.type = (uint32_t)r.le(4);
        t.offset = r.le(8);
        if (!r.ok) break;
        for (const listed& o : files)
            if (o.name == t.name) return bad("tensor %s is listed twice", t.name.c_str());
        files.push_back(t);
    }
    if (!r.ok) return bad("its tensor directory runs past the end of the file");
    info.file_tensors = (size_t)n_tensors;
    const uint64_t at = (uint64_t)(r.p - (const uint8_t*)map);
    const uint64_t data_start = (at + info.alignment - 1) / info.alignment * info.alignment;
    if (data_start > g->size) return bad("no data section");
    const uint64_t data_size = g->size - data_start;
    const uint8_t* data = (const uint8_t*)map + data_start;
    g->data_offset = data_start;

    for (const listed& t : files) {
        std::string hf;
        bool stack = false;
        size_t layer = 0;
        const char* part = nullptr;
        if (!map_name(t.name, &hf, &stack, &layer, &part)) return bad("tensor %s is not one this engine knows where to put", t.name.c_str());
        const vitna_dtype_t dt = dtype_of_ggml(t.type);
        if (dt == VITNA_DTYPE_UNKNOWN)
            return bad("tensor %s is of ggml type %u; F32, F16, BF16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K are read", t.name.c_str(), t.type);
        if (stack != (t.dims == 3))
            return bad("tensor %s has %u dimensions, where %s", t.name.c_str(), t.dims,
                       stack ? "a stack of experts has 3" : "only a stack of experts has 3");
        const uint64_t cols = t.ne[0], rows = t.dims >= 2 ? t.ne[1] : 1, count = t.dims == 3 ? t.ne[2] : 1;
        const uint64_t rb = row_bytes_of(dt, cols);
        if (!rb || rows == 0 || count == 0 || count > 65536)
            return bad("tensor %s has rows that are not whole %s blocks, rows too wide, or no rows", t.name.c_str(), dtype_text(dt));
        if (rows > UINT64_MAX / rb || rows * rb > UINT64_MAX / count) return bad("tensor %s overflows", t.name.c_str());
        const uint64_t slice = rows * rb, bytes = slice * count;
        if (t.offset % info.alignment || t.offset > data_size || bytes > data_size - t.offset)
            return bad("tensor %s lies outside the data section, or off its alignment", t.name.c_str());
        for (uint64_t e = 0; e < count; e++) {
            vitna_hip_gguf_tensor_t d{};
            const std::string n = stack ? "model.layers." + std::to_string(layer) + ".mlp.experts." + std::to_string(e) + "." + part + ".weight" : hf;
            snprintf(d.name, sizeof(d.name), "%s", n.c_str());
            d.dtype = dt;
            if (t.dims == 1) {
                d.ndim = 1;
                d.shape[0] = (size_t)cols;
            } else {
                d.ndim = 2;
                d.shape[0] = (size_t)rows;
                d.shape[1] = (size_t)cols;
            }
            d.offset_begin = t.offset + e * slice;
            d.offset_end = d.offset_begin + slice;
            d.data = data + d.offset_begin;
            g->tensors.push_back(d);
        }
    }
    if (info_out) *info_out = info;
    return g;
}

extern "C" size_t vitna_hip_gguf_count(const vitna_hip_gguf_t* g) { return g ? g->tensors.size() : 0; }

extern "C" bool vitna_hip_gguf_tensor(const vitna_hip_gguf_t* g, size_t i, vitna_hip_gguf_tensor_t* out) {
    if (!g || !out || i >= g->tensors.size()) return false;
    *out = g->tensors[i];
    return true;
}

extern "C" uint64_t vitna_hip_gguf_data_offset(const vitna_hip_gguf_t* g) { return g ? g->data_offset : 0; }

extern "C" void vitna_hip_gguf_close(vitna_hip_gguf_t* g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    delete g;
}

namespace {

/* The first way the file's metadata and the config describe different models, else null (engine/src/model.c:160-175:
   a value the file leaves out is not compared). */
const char* disagreement(const vitna_llama_config_t* c, const vitna_hip_gguf_info_t* g) {
    const uint64_t ffn = g->expert_feed_forward_length ? g->expert_feed_forward_length : g->feed_forward_length;
    if (g->block_count && g->block_count != c->n_layers) return "the number of layers";
    if (g->embedding_length && g->embedding_length != c->hidden) return "the hidden size";
    if (ffn && ffn != c->intermediate) return "the MLP's width";
    if (g->head_count && g->head_count != c->n_heads) return "the number of attention heads";
    if (g->head_count_kv && g->head_count_kv != c->n_kv_heads) return "the number of key-value heads";
    if (g->key_length && g->key_length != c->head_dim) return "the head size";
    if (g->expert_count != c->n_experts) return "the number of experts";
    if (g->expert_used_count != c->n_experts_used) return "the experts a token goes through";
    if (g->rms_eps != 0.0 && (float)g->rms_eps != c->rms_eps) return "the RMSNorm epsilon";
    if (g->rope_freq_base != 0.0 && (float)g->rope_freq_base != c->rope_theta) return "the rotary base";
    return nullptr;
}

bool plain(vitna_dtype_t t) { return t == VITNA_DTYPE_F32 || t == VITNA_DTYPE_F16 || t == VITNA_DTYPE_BF16; }

/* name bound into *out as a rows x cols matrix (cols 0: a vector of rows), checked as engine/src/model.c:259-283. */
bool bind(const vitna_hip_gguf* g, vitna_matrix_t* out, const std::string& name, size_t rows, size_t cols, char* err, size_t len) {
    const vitna_hip_gguf_tensor_t* t = g->find(name);
    if (!t) return say(err, len, "the checkpoint has no tensor %s", name.c_str());
    const bool shape_ok = cols == 0 ? (t->ndim == 1 && t->shape[0] == rows) : (t->ndim == 2 && t->shape[0] == rows && t->shape[1] == cols);
    if (!shape_ok) return say(err, len, "tensor %s has an unexpected shape", name.c_str());
    if (cols == 0 && !plain(t->dtype))
        return say(err, len, "tensor %s is %s; a norm's weights must be F32, BF16 or F16", name.c_str(), dtype_text(t->dtype));
    if (!plain(t->dtype) && !row_bytes_of(t->dtype, cols))
        return say(err, len, "tensor %s is %s; F32, BF16, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K or Q6_K is needed", name.c_str(),
                   dtype_text(t->dtype));
    out->data = t->data;
    out->dtype = t->dtype;
    out->rows = rows;
    out->cols = cols ? cols : 1;
    return true;
}

/* A norm's n weights widened to a float32 copy (engine/src/model.c:285-294). */
float* norm_copy(const vitna_hip_gguf* g, const std::string& name, size_t n, char* err, size_t len) {
    vitna_matrix_t w;
    if (!bind(g, &w, name, n, 0, err, len)) return nullptr;
    float* f = (float*)malloc(n * sizeof(float));
    if (!f) { say(err, len, "out of memory"); return nullptr; }
    const uint8_t* b = (const uint8_t*)w.data;
    for (size_t i = 0; i < n; i++) {
        if (w.dtype == VITNA_DTYPE_F32) {
            memcpy(&f[i], b + 4 * i, 4);
        } else if (w.dtype == VITNA_DTYPE_F16) {
            f[i] = half_value((uint16_t)(b[2 * i] | b[2 * i + 1] << 8));
        } else {
            const uint32_t bits = (uint32_t)(b[2 * i] | b[2 * i + 1] << 8) << 16;
            memcpy(&f[i], &bits, 4);
        }
    }
    return f;
}

}  // namespace

extern "C" void vitna_hip_gguf_llama_free(vitna_llama_t* m) {
    if (!m) return;
    if (m->layers) {
        for (size_t l = 0; l < m->cfg.n_layers; l++) {
            free(m->layers[l].attn_norm);
            free(m->layers[l].mlp_norm);
            free(m->layers[l].q_norm);
            free(m->layers[l].k_norm);
            free(m->layers[l].experts);
        }
        free(m->layers);
    }
    free(m->router_logits); free(m->expert_out); free(m->final_norm); free(m->inv_freq); free(m->past);
    free(m->k_cache); free(m->v_cache);
    free(m->x); free(m->xn); free(m->q); free(m->k); free(m->v); free(m->att);
    free(m->proj); free(m->gate); free(m->up); free(m->scores); free(m->cos_t); free(m->sin_t);
    memset(m, 0, sizeof(*m));
}

extern "C" bool vitna_hip_gguf_llama(vitna_hip_gguf_t* g, const vitna_llama_config_t* cfg, size_t ctx, size_t seqs, vitna_llama_t* m,
                                     char* err, size_t err_len) {
    if (!g || !cfg || !m) return say(err, err_len, "missing arguments");
    memset(m, 0, sizeof(*m));
    m->gpu_kv_layers = -1;
    m->cfg = *cfg;
    const vitna_llama_config_t* c = &m->cfg;
    if (const char* d = disagreement(c, &g->info)) return say(err, err_len, "the GGUF file and the config disagree on %s", d);
    const size_t q_dim = c->n_heads * c->head_dim, kv_dim = c->n_kv_heads * c->head_dim;
    bool ok = bind(g, &m->embed, "model.embed_tokens.weight", c->vocab, c->hidden, err, err_len);
    if (ok) {
        if (g->find("lm_head.weight")) ok = bind(g, &m->lm_head, "lm_head.weight", c->vocab, c->hidden, err, err_len);
        else if (c->tied_embeddings) m->lm_head = m->embed;
        else ok = say(err, err_len, "no lm_head.weight, and the config does not tie embeddings");
    }
    if (ok) ok = (m->final_norm = norm_copy(g, "model.norm.weight", c->hidden, err, err_len)) != nullptr;
    if (ok) ok = (m->layers = (vitna_llama_layer_t*)calloc(c->n_layers, sizeof(vitna_llama_layer_t))) != nullptr || say(err, err_len, "out of memory");
    for (size_t l = 0; ok && l < c->n_layers; l++) {
        vitna_llama_layer_t* L = &m->layers[l];
        const std::string p = "model.layers." + std::to_string(l) + ".";
        ok = bind(g, &L->q, p + "self_attn.q_proj.weight", q_dim, c->hidden, err, err_len) &&
             bind(g, &L->k, p + "self_attn.k_proj.weight", kv_dim, c->hidden, err, err_len) &&
             bind(g, &L->v, p + "self_attn.v_proj.weight", kv_dim, c->hidden, err, err_len) &&
             bind(g, &L->o, p + "self_attn.o_proj.weight", c->hidden, q_dim, err, err_len);
        if (ok && c->n_experts) {
            ok = bind(g, &L->router, p + "mlp.gate.weight", c->n_experts, c->hidden, err, err_len);
            if (ok) ok = (L->experts = (vitna_expert_t*)calloc(c->n_experts, sizeof(vitna_expert_t))) != nullptr || say(err, err_len, "out of memory");
            for (size_t e = 0; ok && e < c->n_experts; e++) {
                const std::string x = p + "mlp.experts." + std::to_string(e) + ".";
                ok = bind(g, &L->experts[e].gate, x + "gate_proj.weight", c->intermediate, c->hidden, err, err_len) &&
                     bind(g, &L->experts[e].up, x + "up_proj.weight", c->intermediate, c->hidden, err, err_len) &&
                     bind(g, &L->experts[e].down, x + "down_proj.weight", c->hidden, c->intermediate, err, err_len);
            }
        } else if (ok) {
            ok = bind(g, &L->gate, p + "mlp.gate_proj.weight", c->intermediate, c->hidden, err, err_len) &&
                 bind(g, &L->up, p + "mlp.up_proj.weight", c->intermediate, c->hidden, err, err_len) &&
                 bind(g, &L->down, p + "mlp.down_proj.weight", c->hidden, c->intermediate, err, err_len);
        }
        if (ok) ok = (L->attn_norm = norm_copy(g, p + "input_layernorm.weight", c->hidden, err, err_len)) != nullptr;
        if (ok) ok = (L->mlp_norm = norm_copy(g, p + "post_attention_layernorm.weight", c->hidden, err, err_len)) != nullptr;
        if (ok && c->qk_norm) {
            ok = (L->q_norm = norm_copy(g, p + "self_attn.q_norm.weight", c->qk_norm_per_head ? c->head_dim : q_dim, err, err_len)) != nullptr &&
                 (L->k_norm = norm_copy(g, p + "self_attn.k_norm.weight", c->qk_norm_per_head ? c->head_dim : kv_dim, err, err_len)) != nullptr;
        }
    }
    if (ok) {
        m->ctx = ctx ? ctx : (c->max_positions < 4096 ? c->max_positions : 4096);
        if (m->ctx > c->max_positions) m->ctx = c->max_positions;
        m->seqs = seqs ? seqs : 1;
        const size_t cache = m->seqs * c->n_layers * m->ctx * kv_dim, half = c->head_dim / 2;
        auto f = [](size_t n) { return (float*)malloc((n ? n : 1) * sizeof(float)); };
        m->past = (size_t*)calloc(m->seqs, sizeof(size_t));
        m->k_cache = f(cache); m->v_cache = f(cache); m->inv_freq = f(half);
        m->x = f(c->hidden); m->xn = f(c->hidden); m->q = f(q_dim); m->k = f(kv_dim); m->v = f(kv_dim); m->att = f(q_dim);
        m->proj = f(c->hidden); m->gate = f(c->intermediate); m->up = f(c->intermediate); m->scores = f(m->ctx);
        m->cos_t = f(half); m->sin_t = f(half);
        if (c->n_experts) { m->router_logits = f(c->n_experts); m->expert_out = f(c->hidden); }
        ok = m->past && m->k_cache && m->v_cache && m->inv_freq && m->x && m->xn && m->q && m->k && m->v && m->att && m->proj &&
             m->gate && m->up && m->scores && m->cos_t && m->sin_t && (!c->n_experts || (m->router_logits && m->expert_out));
        if (!ok) {
            say(err, err_len, "out of memory for the key-value cache and scratch buffers");
        } else {
            /* 1 / theta ** (2j / head_dim) in float32, as transformers computes it (engine/src/model.c:398-402) */
            for (size_t j = 0; j < half; j++) m->inv_freq[j] = 1.0f / powf(c->rope_theta, (float)(2 * j) / (float)c->head_dim);
        }
    }
    if (!ok) vitna_hip_gguf_llama_free(m);
    return ok;
}
