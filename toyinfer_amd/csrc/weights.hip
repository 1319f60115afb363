// Checkpoint loading for the model harness: config.json and safetensors
// shards (src/config.cpp:10-40, src/qwen.cpp:431-518).  Host code; the only
// device work is the upload.
//
// The reference concatenates the data sections of three fixed shard files
// and finds tensors through an offset table generated for one model.  Here
// the safetensors headers are read directly: each needed tensor is located
// by name, checked (BF16, the shape the configuration implies, bytes inside
// the file), and placed at a 256-byte aligned offset of one device
// allocation, in file order so that each shard is read front to back.  The
// upload goes through two pinned staging buffers, so reading the next chunk
// overlaps the copy of the previous one.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "../../include/toyinfer_attn.h"
#include "../../include/toyinfer_qwen3.h"
#include "json.hpp"

namespace {

namespace fs = std::filesystem;

constexpr size_t kStageBytes = 64ull << 20;
constexpr uint64_t kMaxHeader = 100ull << 20;  // safetensors' own header limit

bool read_text(const fs::path& p, std::string& out) {
    std::ifstream f(p, std::ios::binary);
    if (!f) return false;
    out.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
    return !f.bad();
}

bool get_u32(const tijson::Value& root, const char* key, uint32_t& out) {
    const tijson::Value* v = root.get(key);
    uint64_t x;
    if (!v || !v->as_u64(x) || x > 0xffffffffull) return false;
    out = (uint32_t)x;
    return true;
}

bool get_f32(const tijson::Value& root, const char* key, float& out) {
    const tijson::Value* v = root.get(key);
    if (!v || v->kind != tijson::Value::Number) return false;
    out = (float)v->num;
    return true;
}

// An optional token id: absent or null gives 0; a list gives its first entry.
uint32_t token_id(const tijson::Value& root, const char* key) {
    const tijson::Value* v = root.get(key);
    if (v && v->kind == tijson::Value::Array && !v->arr.empty()) v = &v->arr[0];
    uint64_t x;
    return v && v->as_u64(x) && x <= 0xffffffffull ? (uint32_t)x : 0u;
}

struct TensorInfo {
    uint32_t shard = 0;
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t file_off = 0, bytes = 0;
    bool in_file = false;
};

struct Item {
    const void** slot;  // where the device address goes
    uint32_t shard;
    uint64_t file_off, bytes;
    size_t dst;
};

struct Plan {
    std::vector<fs::path> shards;
    std::vector<Item> items;
    size_t bytes = 0;
};

int list_shards(const fs::path& dir, std::vector<fs::path>& out) {
    std::error_code ec;
    const fs::path index = dir / "model.safetensors.index.json";
    if (fs::exists(index, ec)) {
        std::string text;
        tijson::Value root;
        if (!read_text(index, text) || !tijson::parse(text, root)) return TOYINFER_ERR_IO;
        const tijson::Value* map = root.get("weight_map");
        if (!map || map->kind != tijson::Value::Object) return TOYINFER_ERR_IO;
        std::vector<std::string> names;
        for (const auto& kv : map->obj) {
            if (kv.second.kind != tijson::Value::String) return TOYINFER_ERR_IO;
            names.push_back(kv.second.str);
        }
        std::sort(names.begin(), names.end());
        names.erase(std::unique(names.begin(), names.end()), names.end());
        for (const std::string& n : names) {
            if (n.find('/') != std::string::npos || n == ".." || !fs::is_regular_file(dir / n, ec))
                return TOYINFER_ERR_IO;
            out.push_back(dir / n);
        }
    } else {
        for (const auto& e : fs::directory_iterator(dir, ec))
            if (e.is_regular_file(ec) && e.path().extension() == ".safetensors")
                out.push_back(e.path());
        if (ec) return TOYINFER_ERR_IO;
        std::sort(out.begin(), out.end());
    }
    return out.empty() ? TOYINFER_ERR_IO : TOYINFER_OK;
}

// One shard's header: u64 length N, N bytes of JSON, then the data section.
int read_header(const fs::path& p, uint32_t shard, std::map<std::string, TensorInfo>& out) {
    std::ifstream f(p, std::ios::binary);
    if (!f) return TOYINFER_ERR_IO;
    f.seekg(0, std::ios::end);
    const uint64_t size = (uint64_t)f.tellg();
    f.seekg(0);
    unsigned char len8[8];
    if (size < 8 || !f.read(reinterpret_cast<char*>(len8), 8)) return TOYINFER_ERR_IO;
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = n << 8 | len8[i];
    if (n > kMaxHeader || n > size - 8) return TOYINFER_ERR_IO;
    std::string text(n, '\0');
    if (!f.read(&text[0], (std::streamsize)n)) return TOYINFER_ERR_IO;
    tijson::Value root;
    if (!tijson::parse(text, root) || root.kind != tijson::Value::Object) return TOYINFER_ERR_IO;
    const uint64_t data = 8 + n, data_bytes = size - data;
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const tijson::Value& t = kv.second;
        const tijson::Value *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
        if (!dt || dt->kind != tijson::Value::String || !sh || sh->kind != tijson::Value::Array ||
            !off || off->kind != tijson::Value::Array || off->arr.size() != 2)
            return TOYINFER_ERR_IO;
        TensorInfo ti;
        ti.shard = shard;
        ti.dtype = dt->str;
        for (const tijson::Value& d : sh->arr) {
            uint64_t x;
            if (!d.as_u64(x)) return TOYINFER_ERR_IO;
            ti.shape.push_back(x);
        }
        uint64_t b, e;
        if (!off->arr[0].as_u64(b) || !off->arr[1].as_u64(e)) return TOYINFER_ERR_IO;
        ti.in_file = b <= e && e <= data_bytes;
        ti.file_off = data + b;
        ti.bytes = e - b;
        out[kv.first] = std::move(ti);
    }
    return TOYINFER_OK;
}

int make_plan(const char* model_dir, const toyinfer_qwen3_config* c, int tie,
              toyinfer_qwen3_weights* w, Plan& plan) {
    if (!model_dir || !c || c->num_layers == 0 || c->hidden_size == 0 || c->num_q_heads == 0 ||
        c->num_kv_heads == 0 || c->head_dim == 0 || c->intermediate_size == 0 ||
        c->vocab_size == 0)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    const fs::path dir(model_dir);
    int st = list_shards(dir, plan.shards);
    if (st != TOYINFER_OK) return st;
    std::map<std::string, TensorInfo> tensors;
    for (uint32_t i = 0; i < plan.shards.size(); ++i)
        if ((st = read_header(plan.shards[i], i, tensors)) != TOYINFER_OK) return st;

    const uint64_t H = c->hidden_size, F = c->intermediate_size, V = c->vocab_size,
                   D = c->head_dim, QD = (uint64_t)c->num_q_heads * D,
                   KV = (uint64_t)c->num_kv_heads * D;
    auto need = [&](const std::string& name, std::vector<uint64_t> shape,
                    const void** slot) -> int {
        const auto it = tensors.find(name);
        if (it == tensors.end()) return TOYINFER_ERR_IO;
        const TensorInfo& t = it->second;
        if (t.dtype != "BF16") return TOYINFER_ERR_UNSUPPORTED;
        uint64_t elems = 1;
        for (uint64_t d : shape) elems *= d;
        if (t.shape != shape || !t.in_file || t.bytes != 2 * elems) return TOYINFER_ERR_IO;
        plan.items.push_back({slot, t.shard, t.file_off, t.bytes, 0});
        return TOYINFER_OK;
    };
    if ((st = need("model.embed_tokens.weight", {V, H}, &w->embed_tokens)) != TOYINFER_OK ||
        (st = need("model.norm.weight", {H}, &w->final_norm)) != TOYINFER_OK)
        return st;
    if (!tie && tensors.count("lm_head.weight") &&
        (st = need("lm_head.weight", {V, H}, &w->lm_head)) != TOYINFER_OK)
        return st;
    for (uint32_t l = 0; l < c->num_layers; ++l) {
        toyinfer_qwen3_layer& L = w->layers[l];
        const std::string p = "model.layers." + std::to_string(l) + ".";
        const struct {
            const char* name;
            std::vector<uint64_t> shape;
            const void** slot;
        } t[11] = {{"input_layernorm", {H}, &L.input_layernorm},
                   {"self_attn.q_proj", {QD, H}, &L.q_proj},
                   {"self_attn.k_proj", {KV, H}, &L.k_proj},
                   {"self_attn.v_proj", {KV, H}, &L.v_proj},
                   {"self_attn.q_norm", {D}, &L.q_norm},
                   {"self_attn.k_norm", {D}, &L.k_norm},
                   {"self_attn.o_proj", {H, QD}, &L.o_proj},
                   {"post_attention_layernorm", {H}, &L.post_attention_layernorm},
                   {"mlp.gate_proj", {F, H}, &L.gate_proj},
                   {"mlp.up_proj", {F, H}, &L.up_proj},
                   {"mlp.down_proj", {H, F}, &L.down_proj}};
        for (const auto& x : t)
            if ((st = need(p + x.name + ".weight", x.shape, x.slot)) != TOYINFER_OK) return st;
    }
    // File order, then 256-byte aligned destinations.
    std::sort(plan.items.begin(), plan.items.end(), [](const Item& a, const Item& b) {
        return a.shard != b.shard ? a.shard < b.shard : a.file_off < b.file_off;
    });
    size_t off = 0;
    for (Item& it : plan.items) {
        it.dst = off;
        off = (off + it.bytes + 255) / 256 * 256;
    }
    plan.bytes = off;
    return TOYINFER_OK;
}

struct Staging {
    char* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    ~Staging() {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) (void)hipEventDestroy(ev[i]);
            if (buf[i]) (void)hipHostFree(buf[i]);
        }
    }
};

int upload(const Plan& plan, char* dev, hipStream_t st) {
    uint64_t largest = 0;
    for (const Item& it : plan.items) largest = std::max(largest, it.bytes);
    const size_t stage = (size_t)std::min<uint64_t>(kStageBytes, largest);
    Staging s;
    for (int i = 0; i < 2; ++i)
        if (hipHostMalloc(reinterpret_cast<void**>(&s.buf[i]), stage, hipHostMallocDefault) !=
                hipSuccess ||
            hipEventCreateWithFlags(&s.ev[i], hipEventDisableTiming) != hipSuccess)
            return TOYINFER_ERR_HIP;
    std::vector<std::ifstream> files;
    for (const fs::path& p : plan.shards) {
        files.emplace_back(p, std::ios::binary);
        if (!files.back()) return TOYINFER_ERR_IO;
    }
    int cur = 0;
    bool used[2] = {false, false};
    for (const Item& it : plan.items) {
        std::ifstream& f = files[it.shard];
        f.clear();
        f.seekg((std::streamoff)it.file_off);
        for (uint64_t done = 0; done < it.bytes;) {
            const size_t n = (size_t)std::min<uint64_t>(stage, it.bytes - done);
            if (used[cur] && hipEventSynchronize(s.ev[cur]) != hipSuccess) return TOYINFER_ERR_HIP;
            if (!f.read(s.buf[cur], (std::streamsize)n)) return TOYINFER_ERR_IO;
            if (hipMemcpyAsync(dev + it.dst + done, s.buf[cur], n, hipMemcpyHostToDevice, st) !=
                    hipSuccess ||
                hipEventRecord(s.ev[cur], st) != hipSuccess)
                return TOYINFER_ERR_HIP;
            used[cur] = true;
            cur ^= 1;
            done += n;
        }
    }
    return hipStreamSynchronize(st) == hipSuccess ? TOYINFER_OK : TOYINFER_ERR_HIP;
}

}  // namespace

extern "C" {

int toyinfer_qwen3_read_config(const char* model_dir, uint32_t max_seq_len,
                               uint32_t max_prefill_tokens, toyinfer_qwen3_config* cfg,
                               toyinfer_qwen3_model_info* info) {
    if (!model_dir || !cfg) return TOYINFER_ERR_INVALID_ARGUMENT;
    std::string text;
    tijson::Value root;
    if (!read_text(fs::path(model_dir) / "config.json", text) || !tijson::parse(text, root) ||
        root.kind != tijson::Value::Object)
        return TOYINFER_ERR_IO;
    toyinfer_qwen3_config c{};
    uint32_t max_pos = 0;
    if (!get_u32(root, "num_hidden_layers", c.num_layers) ||
        !get_u32(root, "hidden_size", c.hidden_size) ||
        !get_u32(root, "num_attention_heads", c.num_q_heads) ||
        !get_u32(root, "num_key_value_heads", c.num_kv_heads) ||
        !get_u32(root, "intermediate_size", c.intermediate_size) ||
        !get_u32(root, "vocab_size", c.vocab_size) ||
        !get_f32(root, "rms_norm_eps", c.rms_norm_eps) ||
        !get_f32(root, "rope_theta", c.rope_theta) ||
        !get_u32(root, "max_position_embeddings", max_pos))
        return TOYINFER_ERR_IO;
    if (!get_u32(root, "head_dim", c.head_dim)) {  // absent: hidden / heads, the usual default
        if (c.num_q_heads == 0) return TOYINFER_ERR_IO;
        c.head_dim = c.hidden_size / c.num_q_heads;
    }
    c.max_seq_len = max_seq_len ? max_seq_len : max_pos;
    c.max_prefill_tokens = max_prefill_tokens;
    *cfg = c;
    if (info) {
        info->bos_token_id = token_id(root, "bos_token_id");
        info->eos_token_id = token_id(root, "eos_token_id");
        info->max_position_embeddings = max_pos;
        const tijson::Value* t = root.get("tie_word_embeddings");
        info->tie_word_embeddings = t && t->kind == tijson::Value::Bool && t->b;
    }
    return TOYINFER_OK;
}

int toyinfer_qwen3_check_weights(const char* model_dir, const toyinfer_qwen3_config* cfg,
                                 int tie_word_embeddings, size_t* device_bytes) {
    if (!device_bytes || !cfg) return TOYINFER_ERR_INVALID_ARGUMENT;
    std::vector<toyinfer_qwen3_layer> layers(cfg->num_layers);
    toyinfer_qwen3_weights w{};
    w.layers = layers.data();
    Plan plan;
    const int st = make_plan(model_dir, cfg, tie_word_embeddings, &w, plan);
    if (st == TOYINFER_OK) *device_bytes = plan.bytes;
    return st;
}

int toyinfer_qwen3_load_weights(const char* model_dir, const toyinfer_qwen3_config* cfg,
                                int tie_word_embeddings, void* stream,
                                toyinfer_qwen3_weights* out) {
    if (!out || !cfg) return TOYINFER_ERR_INVALID_ARGUMENT;
    memset(out, 0, sizeof(*out));
    toyinfer_qwen3_weights w{};
    w.num_layers = cfg->num_layers;
    w.layers = new (std::nothrow) toyinfer_qwen3_layer[cfg->num_layers ? cfg->num_layers : 1]();
    if (!w.layers) return TOYINFER_ERR_IO;
    Plan plan;
    int st = make_plan(model_dir, cfg, tie_word_embeddings, &w, plan);
    char* dev = nullptr;
    if (st == TOYINFER_OK && hipMalloc(reinterpret_cast<void**>(&dev), plan.bytes) != hipSuccess)
        st = TOYINFER_ERR_HIP;
    if (st == TOYINFER_OK) st = upload(plan, dev, reinterpret_cast<hipStream_t>(stream));
    if (st != TOYINFER_OK) {
        if (dev) (void)hipFree(dev);
        delete[] w.layers;
        return st;
    }
    // The slots held null; now device addresses.
    for (const Item& it : plan.items) *it.slot = dev + it.dst;
    if (!w.lm_head) w.lm_head = w.embed_tokens;
    w.device = dev;
    w.device_bytes = plan.bytes;
    *out = w;
    return TOYINFER_OK;
}

void toyinfer_qwen3_free_weights(toyinfer_qwen3_weights* w) {
    if (!w) return;
    if (w->device) (void)hipFree(w->device);
    delete[] w->layers;
    memset(w, 0, sizeof(*w));
}

}  // extern "C"
