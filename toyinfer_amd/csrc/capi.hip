// C ABI of the attention path (declared in include/toyinfer_attn.h).
//
// Every entry point checks its arguments on the host and returns a status
// before any HIP call, so argument errors are testable without a GPU.  The
// entry points only enqueue kernels: no allocation, no memset node, no
// synchronisation, which keeps them legal inside stream capture.
#include <stdint.h>

#include <mutex>

#include "../../include/toyinfer_attn.h"
#include "kernels.hpp"

using namespace tiattn;

namespace {

thread_local int g_last_hip_error = 0;

int from_hip(hipError_t e) {
    if (e == hipSuccess) return TOYINFER_OK;
    g_last_hip_error = (int)e;
    return TOYINFER_ERR_HIP;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Shared shape checks.  head_dim outside {64, 128} is "unsupported" rather
// than "invalid": the reference instantiates exactly these two
// (src/prefill.cu:433-452, src/transformer.cpp:26-38).
int check_heads(uint32_t hq, uint32_t hkv, uint32_t d) {
    if (hq == 0 || hkv == 0 || hq % hkv != 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (hq > 65535u) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (d != 64 && d != 128) return TOYINFER_ERR_UNSUPPORTED;
    return TOYINFER_OK;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }


// Prefill addresses one KV head's rows with 32-bit byte offsets.
bool kv_fits_32bit(uint32_t s, uint32_t hkv, uint32_t d) {
    return (uint64_t)s * hkv * d * 2 < 0xffffffffull;
}

// Where the reference-contract decode keeps its split partials: in score
// rows when they are long enough (mode B), else in O_buffer/O rows with a
// single split (mode A).  Either way each head's partials live only in that
// head's rows, which the finaliser reads before it overwrites them.
void compat_partials(uint32_t hq, uint32_t hkv, uint32_t d, uint32_t sizing_len, uint32_t msl,
                     float* score, float* o_buffer, void* o, uint32_t* splits,
                     DecodePartials* part) {
    uint32_t s = decode_default_splits(1, hq, hkv, d, sizing_len);
    uint32_t cap = msl / (d + 2);
    if (cap > decode_max_splits()) cap = decode_max_splits();
    if (s >= 2 && cap >= 2) {
        if (s > cap) s = cap;
        *splits = s;
        part->ml = score;
        part->ml_head = msl;
        part->o = score + 2 * (size_t)s;
        part->o_head = msl;
        part->o_split = d;
        return;
    }
    *splits = 1;
    part->ml = reinterpret_cast<float*>(o);  // 8 bytes at the head of O row h (D*2 bytes)
    part->ml_head = d / 2;
    part->o = o_buffer;
    part->o_head = d;
    part->o_split = d;
}

// Split-K workspace of toyinfer_decode_attention_bf16_noalloc: a file-scope
// device array, one copy per GPU, held until the process ends.  Host code
// never uses its name as an address: the per-device address comes from
// hipGetSymbolAddress, taken once per device (with that device current) on
// the entry point's first call there.  Every call on a GPU shares that
// GPU's copy, so calls that overlap on one GPU race; nothing in it needs to
// start at zero (each call writes every partial it later reads).
constexpr size_t kDecodeScratchBytes = TOYINFER_DECODE_SCRATCH_BYTES;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kScratchDevices];

int decode_scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return from_hip(e);
    if (dev < 0 || dev >= kScratchDevices) return TOYINFER_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return from_hip(e);
        if (!p) return TOYINFER_ERR_HIP;
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return TOYINFER_OK;
}

}  // namespace

extern "C" {

const char* toyinfer_status_string(int status) {
    switch (status) {
        case TOYINFER_OK: return "ok";
        case TOYINFER_ERR_INVALID_ARGUMENT: return "invalid argument";
        case TOYINFER_ERR_UNSUPPORTED: return "unsupported configuration";
        case TOYINFER_ERR_WORKSPACE: return "workspace too small";
        case TOYINFER_ERR_HIP: return "HIP error";
        case TOYINFER_ERR_IO: return "model file missing or malformed";
        default: return "unknown status";
    }
}

int toyinfer_last_hip_error(void) { return g_last_hip_error; }

uint32_t toyinfer_abi_version(void) { return TOYINFER_ABI_VERSION; }

// ------------------------------------------------------------------ prefill

int toyinfer_flash_attention_v1_bf16(const void* Qs, const void* Ks, const void* Vs, void* Os,
                                     uint32_t num_q_heads, uint32_t num_kv_heads,
                                     uint32_t heads_dim, uint32_t seq_len, void* stream) {
    return toyinfer_flash_attention_algo_bf16(Qs, Ks, Vs, Os, num_q_heads, num_kv_heads,
                                              heads_dim, seq_len, 0, stream);
}

int toyinfer_flash_attention_algo_bf16(const void* Qs, const void* Ks, const void* Vs, void* Os,
                                       uint32_t num_q_heads, uint32_t num_kv_heads,
                                       uint32_t heads_dim, uint32_t seq_len, int algo,
                                       void* stream) {
    if (int st = check_heads(num_q_heads, num_kv_heads, heads_dim)) return st;
    if (algo < 0 || algo > 4) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!kv_fits_32bit(seq_len, num_kv_heads, heads_dim)) return TOYINFER_ERR_UNSUPPORTED;
    if (seq_len == 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!Qs || !Ks || !Vs || !Os) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!aligned(Qs, 16) || !aligned(Ks, 16) || !aligned(Vs, 16) || !aligned(Os, 16))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if ((uint64_t)((seq_len + 127) / 128) * num_q_heads > 0x7fffffffull)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    PrefillProblem p{};
    p.q = static_cast<const uint16_t*>(Qs);
    p.k = static_cast<const uint16_t*>(Ks);
    p.v = static_cast<const uint16_t*>(Vs);
    p.o = static_cast<uint16_t*>(Os);
    p.s = seq_len;
    p.hq = num_q_heads;
    p.hkv = num_kv_heads;
    p.d = heads_dim;
    p.fused_q = false;
    p.variant = algo;
    return from_hip(launch_prefill(p, as_stream(stream)));
}

int toyinfer_prefill_qknorm_rope_attention_bf16(
    const void* Q_raw, const void* K_raw, const void* Vs, void* Os, void* K_out,
    const void* q_gamma, const void* k_gamma, const float* rope_cos_sin, float rms_norm_eps,
    uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t heads_dim, uint32_t seq_len,
    void* stream) {
    if (int st = check_heads(num_q_heads, num_kv_heads, heads_dim)) return st;
    if (seq_len == 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!kv_fits_32bit(seq_len, num_kv_heads, heads_dim)) return TOYINFER_ERR_UNSUPPORTED;
    if (!Q_raw || !K_raw || !Vs || !Os || !K_out || !q_gamma || !k_gamma || !rope_cos_sin)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!aligned(Q_raw, 16) || !aligned(Vs, 16) || !aligned(Os, 16) || !aligned(K_out, 16) ||
        !aligned(q_gamma, 16) || !aligned(K_raw, 16) || !aligned(k_gamma, 16) ||
        !aligned(rope_cos_sin, 16))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if ((uint64_t)((seq_len + 127) / 128) * num_q_heads > 0x7fffffffull)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    hipStream_t st = as_stream(stream);
    hipError_t e = launch_row_norm_rope(static_cast<const uint16_t*>(K_raw),
                                        static_cast<uint16_t*>(K_out),
                                        static_cast<const uint16_t*>(k_gamma), nullptr,
                                        rope_cos_sin, rms_norm_eps, seq_len, num_kv_heads,
                                        heads_dim, kRowNorm | kRowRope, st);
    if (e != hipSuccess) return from_hip(e);
    PrefillProblem p{};
    p.q = static_cast<const uint16_t*>(Q_raw);
    p.k = static_cast<const uint16_t*>(K_out);
    p.v = static_cast<const uint16_t*>(Vs);
    p.o = static_cast<uint16_t*>(Os);
    p.s = seq_len;
    p.hq = num_q_heads;
    p.hkv = num_kv_heads;
    p.d = heads_dim;
    p.fused_q = true;
    p.q_gamma = static_cast<const uint16_t*>(q_gamma);
    p.rope = rope_cos_sin;
    p.eps = rms_norm_eps;
    return from_hip(launch_prefill(p, st));
}

// ------------------------------------------------------------------- decode

static int decode_common_checks(const void* Q, const void* Ks, const void* Vs, float* score,
                                float* O_buffer, void* O, uint32_t hq, uint32_t hkv, uint32_t d,
                                uint32_t msl) {
    if (int st = check_heads(hq, hkv, d)) return st;
    if (msl == 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!Q || !Ks || !Vs || !score || !O_buffer || !O) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!aligned(Q, 16) || !aligned(Ks, 16) || !aligned(Vs, 16) || !aligned(O, 8) ||
        !aligned(score, 4) || !aligned(O_buffer, 4))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return TOYINFER_OK;
}

static int decode_compat(const void* Q, const void* Ks, const void* Vs, float* score,
                         float* O_buffer, void* O, uint32_t hq, uint32_t hkv, uint32_t d,
                         int len_mode, const uint32_t* pos_d, uint32_t pos, uint32_t msl,
                         void* stream) {
    DecodeProblem p{};
    p.q = static_cast<const uint16_t*>(Q);
    p.k = static_cast<const uint16_t*>(Ks);
    p.v = static_cast<const uint16_t*>(Vs);
    p.kv_stride = 0;
    p.batch = 1;
    p.hq = hq;
    p.hkv = hkv;
    p.d = d;
    p.len_mode = len_mode;
    p.len_dev = pos_d;
    p.len_host = pos + 1;
    p.len_cap = msl;
    DecodePartials part{};
    const uint32_t sizing = len_mode == kLenHost ? pos + 1 : msl;
    compat_partials(hq, hkv, d, sizing, msl, score, O_buffer, O, &p.splits, &part);
    hipStream_t st = as_stream(stream);
    hipError_t e = p.splits >= 2 ? launch_decode_split_compat(p, part, st)
                                 : launch_decode_split(p, part, st);
    if (e != hipSuccess) return from_hip(e);
    return from_hip(launch_decode_finalize_compat(p, part, score, msl, O_buffer,
                                                  static_cast<uint16_t*>(O), st));
}

int toyinfer_attention_bf16(const void* Q, const void* Ks, const void* Vs, float* score,
                            float* O_buffer, void* O, uint32_t num_q_heads,
                            uint32_t num_kv_heads, uint32_t heads_dim, uint32_t pos,
                            uint32_t max_seq_len, void* stream) {
    if (int st = decode_common_checks(Q, Ks, Vs, score, O_buffer, O, num_q_heads, num_kv_heads,
                                      heads_dim, max_seq_len))
        return st;
    if (pos >= max_seq_len) return TOYINFER_ERR_INVALID_ARGUMENT;
    return decode_compat(Q, Ks, Vs, score, O_buffer, O, num_q_heads, num_kv_heads, heads_dim,
                         kLenHost, nullptr, pos, max_seq_len, stream);
}

int toyinfer_attention_bf16_graph(const void* Q, const void* Ks, const void* Vs, float* score,
                                  float* O_buffer, void* O, uint32_t num_q_heads,
                                  uint32_t num_kv_heads, uint32_t heads_dim,
                                  const uint32_t* pos_d, uint32_t max_seq_len, void* stream) {
    if (int st = decode_common_checks(Q, Ks, Vs, score, O_buffer, O, num_q_heads, num_kv_heads,
                                      heads_dim, max_seq_len))
        return st;
    if (!pos_d || !aligned(pos_d, 4)) return TOYINFER_ERR_INVALID_ARGUMENT;
    return decode_compat(Q, Ks, Vs, score, O_buffer, O, num_q_heads, num_kv_heads, heads_dim,
                         kLenDevicePos, pos_d, 0, max_seq_len, stream);
}

int toyinfer_attention_bf16_graph_lean(const void* Q, const void* Ks, const void* Vs,
                                       float* score, float* O_buffer, void* O,
                                       uint32_t num_q_heads, uint32_t num_kv_heads,
                                       uint32_t heads_dim, const uint32_t* pos_d,
                                       uint32_t max_seq_len, void* stream) {
    if (int st = decode_common_checks(Q, Ks, Vs, score, O_buffer, O, num_q_heads, num_kv_heads,
                                      heads_dim, max_seq_len))
        return st;
    if (!pos_d || !aligned(pos_d, 4)) return TOYINFER_ERR_INVALID_ARGUMENT;
    DecodeProblem p{};
    p.q = static_cast<const uint16_t*>(Q);
    p.k = static_cast<const uint16_t*>(Ks);
    p.v = static_cast<const uint16_t*>(Vs);
    p.batch = 1;
    p.hq = num_q_heads;
    p.hkv = num_kv_heads;
    p.d = heads_dim;
    p.len_mode = kLenDevicePos;
    p.len_dev = pos_d;
    p.len_cap = max_seq_len;
    DecodePartials part{};
    compat_partials(num_q_heads, num_kv_heads, heads_dim, max_seq_len, max_seq_len, score,
                    O_buffer, O, &p.splits, &part);
    hipStream_t st = as_stream(stream);
    hipError_t e = launch_decode_split(p, part, st);
    if (e != hipSuccess) return from_hip(e);
    // Partials in score rows (or O_buffer/O rows) are 4-byte aligned only.
    return from_hip(launch_decode_combine(p, part, static_cast<uint16_t*>(O), st, O_buffer,
                                          false));
}

uint32_t toyinfer_decode_default_splits(uint32_t batch, uint32_t num_q_heads,
                                        uint32_t num_kv_heads, uint32_t heads_dim,
                                        uint32_t seq_len) {
    if (batch == 0 || num_kv_heads == 0 || num_q_heads % num_kv_heads != 0 || seq_len == 0)
        return 1;
    return decode_default_splits(batch, num_q_heads, num_kv_heads, heads_dim, seq_len);
}

size_t toyinfer_decode_workspace_bytes(uint32_t batch, uint32_t num_q_heads, uint32_t heads_dim,
                                       uint32_t num_splits) {
    const size_t heads = (size_t)batch * num_q_heads;
    return align_up(heads * num_splits * 2 * sizeof(float), 256) +
           heads * num_splits * heads_dim * sizeof(float);
}

// Host checks of the batched decode; on success *splits holds the split
// count the call uses.
static int decode_batched_checks(const void* q, const void* k_cache, const void* v_cache,
                                 void* o, uint32_t batch, uint32_t num_q_heads,
                                 uint32_t num_kv_heads, uint32_t heads_dim,
                                 const uint32_t* seq_lens_d, uint32_t seq_len,
                                 uint64_t kv_batch_stride, uint32_t num_splits,
                                 uint32_t* splits) {
    if (int st = check_heads(num_q_heads, num_kv_heads, heads_dim)) return st;
    if (batch == 0 || batch > 65535u || seq_len == 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!q || !k_cache || !v_cache || !o) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(o, 2) ||
        (seq_lens_d && !aligned(seq_lens_d, 4)))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if (batch > 1 && kv_batch_stride < (uint64_t)seq_len * num_kv_heads * heads_dim)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if (kv_batch_stride % 8 != 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    *splits = num_splits
                  ? num_splits
                  : decode_default_splits(batch, num_q_heads, num_kv_heads, heads_dim, seq_len);
    if (*splits > decode_max_splits()) return TOYINFER_ERR_INVALID_ARGUMENT;
    return TOYINFER_OK;
}

static int decode_batched_launch(const void* q, const void* k_cache, const void* v_cache,
                                 void* o, uint32_t batch, uint32_t num_q_heads,
                                 uint32_t num_kv_heads, uint32_t heads_dim,
                                 const uint32_t* seq_lens_d, uint32_t seq_len,
                                 uint64_t kv_batch_stride, uint32_t splits, void* workspace,
                                 void* stream) {
    DecodeProblem p{};
    p.q = static_cast<const uint16_t*>(q);
    p.k = static_cast<const uint16_t*>(k_cache);
    p.v = static_cast<const uint16_t*>(v_cache);
    p.kv_stride = (int64_t)kv_batch_stride;
    p.batch = batch;
    p.hq = num_q_heads;
    p.hkv = num_kv_heads;
    p.d = heads_dim;
    p.len_mode = seq_lens_d ? kLenDevice : kLenHost;
    p.len_dev = seq_lens_d;
    p.len_host = seq_len;
    p.len_cap = seq_len;
    p.splits = splits;
    const DecodePartials part =
        decode_partials_in(workspace, (size_t)batch * num_q_heads, splits, heads_dim);
    hipStream_t st = as_stream(stream);
    hipError_t e = launch_decode_split(p, part, st);
    if (e != hipSuccess) return from_hip(e);
    return from_hip(launch_decode_combine(p, part, static_cast<uint16_t*>(o), st));
}

int toyinfer_decode_attention_bf16(const void* q, const void* k_cache, const void* v_cache,
                                   void* o, uint32_t batch, uint32_t num_q_heads,
                                   uint32_t num_kv_heads, uint32_t heads_dim,
                                   const uint32_t* seq_lens_d, uint32_t seq_len,
                                   uint64_t kv_batch_stride, uint32_t num_splits,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    uint32_t splits = 0;
    if (int st = decode_batched_checks(q, k_cache, v_cache, o, batch, num_q_heads, num_kv_heads,
                                       heads_dim, seq_lens_d, seq_len, kv_batch_stride,
                                       num_splits, &splits))
        return st;
    if (!workspace || !aligned(workspace, 256)) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (workspace_bytes < toyinfer_decode_workspace_bytes(batch, num_q_heads, heads_dim, splits))
        return TOYINFER_ERR_WORKSPACE;
    return decode_batched_launch(q, k_cache, v_cache, o, batch, num_q_heads, num_kv_heads,
                                 heads_dim, seq_lens_d, seq_len, kv_batch_stride, splits,
                                 workspace, stream);
}

int toyinfer_decode_attention_bf16_noalloc(const void* q, const void* k_cache,
                                           const void* v_cache, void* o, uint32_t batch,
                                           uint32_t num_q_heads, uint32_t num_kv_heads,
                                           uint32_t heads_dim, const uint32_t* seq_lens_d,
                                           uint32_t seq_len, uint64_t kv_batch_stride,
                                           uint32_t num_splits, void* stream) {
    uint32_t splits = 0;
    if (int st = decode_batched_checks(q, k_cache, v_cache, o, batch, num_q_heads, num_kv_heads,
                                       heads_dim, seq_lens_d, seq_len, kv_batch_stride,
                                       num_splits, &splits))
        return st;
    if (toyinfer_decode_workspace_bytes(batch, num_q_heads, heads_dim, splits) >
        kDecodeScratchBytes)
        return TOYINFER_ERR_WORKSPACE;
    void* ws = nullptr;
    if (int st = decode_scratch_address(&ws)) return st;
    return decode_batched_launch(q, k_cache, v_cache, o, batch, num_q_heads, num_kv_heads,
                                 heads_dim, seq_lens_d, seq_len, kv_batch_stride, splits, ws,
                                 stream);
}

// ------------------------------------------------------ prologue operators

int toyinfer_precompute_freq_f32(float* inv_freq, int head_dim, float theta, void* stream) {
    if (!inv_freq || head_dim < 2 || head_dim % 2 != 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_precompute_freq(inv_freq, head_dim, theta, as_stream(stream)));
}

int toyinfer_rope_cos_sin_f32(float* table, const float* inv_freq, uint32_t num_positions,
                              uint32_t head_dim, void* stream) {
    if (!table || !inv_freq || num_positions == 0 || head_dim < 2 || head_dim % 2 != 0)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!aligned(table, 8) || !aligned(inv_freq, 4)) return TOYINFER_ERR_INVALID_ARGUMENT;
    if ((uint64_t)num_positions * (head_dim / 2) > 0xffffffffull * 128ull)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_rope_table(table, inv_freq, num_positions, head_dim, as_stream(stream)));
}

static int row_op(const void* input, const void* weight, void* output, const float* inv_freq,
                  float eps, uint32_t num_tokens, uint32_t nums_head, uint32_t head_dim, int mode,
                  void* stream) {
    if (head_dim != 64 && head_dim != 128) return TOYINFER_ERR_UNSUPPORTED;
    if (num_tokens == 0 || nums_head == 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    if ((uint64_t)num_tokens * nums_head > 0xffffffffull) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!input || !output) return TOYINFER_ERR_INVALID_ARGUMENT;
    if ((mode & kRowNorm) && !weight) return TOYINFER_ERR_INVALID_ARGUMENT;
    if ((mode & kRowRope) && !inv_freq) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!aligned(input, 16) || !aligned(output, 16) || (weight && !aligned(weight, 16)) ||
        (inv_freq && !aligned(inv_freq, 4)))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_row_norm_rope(static_cast<const uint16_t*>(input),
                                         static_cast<uint16_t*>(output),
                                         static_cast<const uint16_t*>(weight), inv_freq, nullptr,
                                         eps, num_tokens, nums_head, head_dim, mode,
                                         as_stream(stream)));
}

int toyinfer_multi_rmsnorm_bf16(const void* input, const void* weight, void* output,
                                float rms_norm_eps, uint32_t nums_head, uint32_t head_dim,
                                void* stream) {
    return row_op(input, weight, output, nullptr, rms_norm_eps, 1, nums_head, head_dim, kRowNorm,
                  stream);
}

int toyinfer_batch_multi_rmsnorm_bf16(const void* input, const void* weight, void* output,
                                      float rms_norm_eps, uint32_t num_tokens,
                                      uint32_t nums_head, uint32_t head_dim, void* stream) {
    return row_op(input, weight, output, nullptr, rms_norm_eps, num_tokens, nums_head, head_dim,
                  kRowNorm, stream);
}

int toyinfer_batch_rope_bf16(void* qk, const float* inv_freq, uint32_t num_tokens,
                             uint32_t nums_head, uint32_t head_dim, void* stream) {
    return row_op(qk, nullptr, qk, inv_freq, 0.0f, num_tokens, nums_head, head_dim, kRowRope,
                  stream);
}

int toyinfer_qk_norm_rope_bf16(const void* input, const void* weight, void* output,
                               const float* inv_freq, float rms_norm_eps, uint32_t num_tokens,
                               uint32_t nums_head, uint32_t head_dim, void* stream) {
    return row_op(input, weight, output, inv_freq, rms_norm_eps, num_tokens, nums_head, head_dim,
                  kRowNorm | kRowRope, stream);
}

// ----------------------------------------------- decode-step pre-pass ops

static int token_rows(const TokenRowsArgs& a, uint32_t head_dim, void* stream) {
    if (head_dim != 64 && head_dim != 128) return TOYINFER_ERR_UNSUPPORTED;
    return from_hip(launch_token_rows(a, head_dim, as_stream(stream)));
}

static bool rows_ok(const void* p) { return p && aligned(p, 16); }

int toyinfer_rope_bf16(void* qk, const float* inv_freq, uint32_t pos, uint32_t nums_head,
                       uint32_t head_dim, void* stream) {
    if (nums_head == 0 || !rows_ok(qk) || !inv_freq || !aligned(inv_freq, 4))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    TokenRowsArgs a;
    a.q = static_cast<const uint16_t*>(qk);
    a.q_out = static_cast<uint16_t*>(qk);
    a.inv_freq = inv_freq;
    a.pos_host = pos;
    a.pos_cap = 0xffffffffu;
    a.hq = nums_head;
    a.q_mode = kRowRope;
    return token_rows(a, head_dim, stream);
}

int toyinfer_rope_bf16_graph(void* qk, const float* inv_freq, const uint32_t* pos_d,
                             uint32_t nums_head, uint32_t head_dim, void* stream) {
    if (nums_head == 0 || !rows_ok(qk) || !inv_freq || !aligned(inv_freq, 4) || !pos_d ||
        !aligned(pos_d, 4))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    TokenRowsArgs a;
    a.q = static_cast<const uint16_t*>(qk);
    a.q_out = static_cast<uint16_t*>(qk);
    a.inv_freq = inv_freq;
    a.pos_d = pos_d;
    a.pos_cap = 0xffffffffu;
    a.hq = nums_head;
    a.q_mode = kRowRope;
    return token_rows(a, head_dim, stream);
}

int toyinfer_write_kv_cache_bf16(const void* src, void* cache, const uint32_t* pos_d,
                                 uint32_t kv_dim, void* stream) {
    if (!src || !cache || !pos_d || kv_dim == 0 || kv_dim % 2 != 0 || !aligned(src, 4) ||
        !aligned(cache, 4) || !aligned(pos_d, 4))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_kv_row_copy(static_cast<const uint16_t*>(src),
                                       static_cast<uint16_t*>(cache), pos_d, kv_dim,
                                       as_stream(stream)));
}

int toyinfer_decode_qkv_prologue_bf16(const void* q, const void* k, const void* v,
                                      const void* q_norm_weight, const void* k_norm_weight,
                                      const float* inv_freq, const uint32_t* pos_d,
                                      uint32_t max_seq_len, float rms_norm_eps, void* q_out,
                                      void* k_cache, void* v_cache, uint32_t num_q_heads,
                                      uint32_t num_kv_heads, uint32_t head_dim, void* stream) {
    if (num_q_heads == 0 || num_kv_heads == 0 || max_seq_len == 0)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!rows_ok(q) || !rows_ok(k) || !rows_ok(v) || !rows_ok(q_norm_weight) ||
        !rows_ok(k_norm_weight) || !rows_ok(q_out) || !rows_ok(k_cache) || !rows_ok(v_cache) ||
        !inv_freq || !aligned(inv_freq, 4) || !pos_d || !aligned(pos_d, 4))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    TokenRowsArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.q_out = static_cast<uint16_t*>(q_out);
    a.q_weight = static_cast<const uint16_t*>(q_norm_weight);
    a.k = static_cast<const uint16_t*>(k);
    a.k_cache = static_cast<uint16_t*>(k_cache);
    a.k_weight = static_cast<const uint16_t*>(k_norm_weight);
    a.v = static_cast<const uint16_t*>(v);
    a.v_cache = static_cast<uint16_t*>(v_cache);
    a.inv_freq = inv_freq;
    a.pos_d = pos_d;
    a.pos_cap = max_seq_len;
    a.eps = rms_norm_eps;
    a.hq = num_q_heads;
    a.hkv = num_kv_heads;
    a.q_mode = kRowNorm | kRowRope;
    a.k_mode = kRowNorm | kRowRope;
    return token_rows(a, head_dim, stream);
}

static int proj_args(const void* W, const void* x, const void* y, size_t y_align,
                     uint32_t tokens, uint32_t M, uint32_t N) {
    if (!W || !x || !y || tokens == 0 || M == 0 || N == 0 || N > kProjMaxN)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!aligned(W, 2) || !aligned(x, 2) || !aligned(y, y_align)) return TOYINFER_ERR_INVALID_ARGUMENT;
    if ((uint64_t)tokens * M > 0xffffffffull * 64) return TOYINFER_ERR_INVALID_ARGUMENT;
    return TOYINFER_OK;
}

int toyinfer_gemv_proj_bf16(const void* W, const void* hidden_states, void* y, uint32_t M,
                            uint32_t N, void* stream) {
    const int st = proj_args(W, hidden_states, y, 2, 1, M, N);
    if (st != TOYINFER_OK) return st;
    return from_hip(launch_gemv_bf16(static_cast<const uint16_t*>(W),
                                     static_cast<const uint16_t*>(hidden_states),
                                     static_cast<uint16_t*>(y), M, N, as_stream(stream)));
}

int toyinfer_gemv_proj_bf162float(const void* W, const void* hidden_states, float* y,
                                  uint32_t M, uint32_t N, void* stream) {
    const int st = proj_args(W, hidden_states, y, 4, 1, M, N);
    if (st != TOYINFER_OK) return st;
    return from_hip(launch_gemv_f32(static_cast<const uint16_t*>(W),
                                    static_cast<const uint16_t*>(hidden_states), y, M, N,
                                    as_stream(stream)));
}

int toyinfer_batch_gemv_proj_bf16(const void* W, const void* hidden_states, void* y,
                                  uint32_t num_tokens, uint32_t M, uint32_t N, void* stream) {
    const int st = proj_args(W, hidden_states, y, 2, num_tokens, M, N);
    if (st != TOYINFER_OK) return st;
    if (num_tokens > 65535u * 4 && !proj_uses_gemm(num_tokens, N, W, hidden_states))
        return TOYINFER_ERR_UNSUPPORTED;
    return from_hip(launch_batch_proj_bf16(static_cast<const uint16_t*>(W),
                                           static_cast<const uint16_t*>(hidden_states),
                                           static_cast<uint16_t*>(y), num_tokens, M, N,
                                           as_stream(stream)));
}

int toyinfer_gemm_segments_bf16(const void* hidden_states, uint32_t num_tokens, uint32_t N,
                                uint32_t num_segments, const void* const* W, void* const* y,
                                const uint32_t* rows, int residual, void* stream) {
    if (!W || !y || !rows || num_segments == 0 || num_segments > 3 || N > kProjMaxN)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    GemmArgs g;
    g.x = static_cast<const uint16_t*>(hidden_states);
    g.T = num_tokens;
    g.N = N;
    g.nseg = (int)num_segments;
    g.residual = residual != 0;
    for (uint32_t s = 0; s < num_segments; ++s) {
        const int st = proj_args(W[s], hidden_states, y[s], 2, num_tokens, rows[s], N);
        if (st != TOYINFER_OK) return st;
        if (!proj_uses_gemm(num_tokens, N, W[s], hidden_states)) return TOYINFER_ERR_UNSUPPORTED;
        g.w[s] = static_cast<const uint16_t*>(W[s]);
        g.y[s] = static_cast<uint16_t*>(y[s]);
        g.rows[s] = rows[s];
    }
    return from_hip(launch_gemm(g, as_stream(stream)));
}

int toyinfer_gemm_swiglu_bf16(const void* hidden_states, uint32_t num_tokens, uint32_t N,
                              const void* W_gate, const void* W_up, uint32_t M, void* out,
                              void* stream) {
    if (N > kProjMaxN) return TOYINFER_ERR_INVALID_ARGUMENT;
    for (const void* w : {W_gate, W_up}) {
        const int st = proj_args(w, hidden_states, out, 2, num_tokens, M, N);
        if (st != TOYINFER_OK) return st;
        if (!proj_uses_gemm(num_tokens, N, w, hidden_states)) return TOYINFER_ERR_UNSUPPORTED;
    }
    GemmArgs g;
    g.x = static_cast<const uint16_t*>(hidden_states);
    g.T = num_tokens;
    g.N = N;
    g.nseg = 2;
    g.w[0] = static_cast<const uint16_t*>(W_gate);
    g.w[1] = static_cast<const uint16_t*>(W_up);
    g.y[0] = static_cast<uint16_t*>(out);
    g.rows[0] = M;
    g.rows[1] = M;
    g.swiglu = true;
    return from_hip(launch_gemm(g, as_stream(stream)));
}

static bool bf16_ok(const void* p) { return p && aligned(p, 4); }

int toyinfer_rmsnorm_bf16(const void* input, const void* weight, void* output, float* sum,
                          float rms_norm_eps, uint32_t size, void* stream) {
    return toyinfer_batch_rmsnorm_bf16(input, weight, output, sum, rms_norm_eps, 1, size, stream);
}

int toyinfer_batch_rmsnorm_bf16(const void* input, const void* weight, void* output, float* sum,
                                float rms_norm_eps, uint32_t num_tokens, uint32_t size,
                                void* stream) {
    if (!bf16_ok(input) || !bf16_ok(weight) || !bf16_ok(output) || (sum && !aligned(sum, 4)) ||
        num_tokens == 0 || size == 0 || size % 2 != 0)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_rmsnorm_rows(static_cast<const uint16_t*>(input),
                                        static_cast<const uint16_t*>(weight),
                                        static_cast<uint16_t*>(output), sum, rms_norm_eps,
                                        num_tokens, size, as_stream(stream)));
}

int toyinfer_residual_add_bf16(const void* residual, void* hidden_state, uint32_t size,
                               void* stream) {
    return toyinfer_batch_residual_add_bf16(residual, hidden_state, 1, size, stream);
}

int toyinfer_batch_residual_add_bf16(const void* residual, void* hidden_state,
                                     uint32_t num_tokens, uint32_t size, void* stream) {
    const size_t n = (size_t)num_tokens * size;
    if (!bf16_ok(residual) || !bf16_ok(hidden_state) || n == 0 || n % 2 != 0)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_residual_add(static_cast<const uint16_t*>(residual),
                                        static_cast<uint16_t*>(hidden_state), n,
                                        as_stream(stream)));
}

int toyinfer_swiglu_bf16x2(const void* gate, const void* up, void* intermedia, uint32_t size,
                           void* stream) {
    return toyinfer_batch_swiglu_bf16x2(gate, up, intermedia, 1, size, stream);
}

int toyinfer_batch_swiglu_bf16x2(const void* gate, const void* up, void* intermedia,
                                 uint32_t num_tokens, uint32_t size, void* stream) {
    const size_t n = (size_t)num_tokens * size;
    if (!bf16_ok(gate) || !bf16_ok(up) || !bf16_ok(intermedia) || n == 0 || n % 2 != 0)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_swiglu(static_cast<const uint16_t*>(gate),
                                  static_cast<const uint16_t*>(up),
                                  static_cast<uint16_t*>(intermedia), n, as_stream(stream)));
}

int toyinfer_gather_embedding_bf16(const void* embedding_table, const uint32_t* token_ids,
                                   void* hidden_states, uint32_t num_tokens,
                                   uint32_t hidden_size, uint32_t vocab_size, void* stream) {
    if (!bf16_ok(embedding_table) || !token_ids || !aligned(token_ids, 4) ||
        !bf16_ok(hidden_states) || num_tokens == 0 || num_tokens > 65535u || hidden_size == 0 ||
        hidden_size % 2 != 0 || vocab_size == 0 || 2ull * hidden_size > 0xffffffffull)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_gather_rows(static_cast<const uint16_t*>(embedding_table), token_ids,
                                       static_cast<uint16_t*>(hidden_states), num_tokens,
                                       hidden_size, vocab_size, as_stream(stream)));
}

int toyinfer_argmax_f32(const float* logits, uint32_t n, uint32_t* out_index, void* stream) {
    if (!logits || !aligned(logits, 4) || !out_index || !aligned(out_index, 4) || n == 0)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return from_hip(launch_argmax(logits, n, out_index, nullptr, 1, as_stream(stream)));
}

size_t toyinfer_sample_workspace_bytes(void) { return sample_workspace_bytes(); }

int toyinfer_sample_topk_topp_f32(const float* logits, uint32_t vocab, float temperature,
                                  uint32_t top_k, float top_p, const float* coin,
                                  uint32_t* out_token, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    if (!logits || !aligned(logits, 4) || !out_token || !aligned(out_token, 4) || !coin ||
        !aligned(coin, 4) || !workspace || !aligned(workspace, 256))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    SampleArgs a;
    const int st = sample_config(vocab, temperature, top_k, top_p, a);
    if (st != TOYINFER_OK) return st;
    if (workspace_bytes < sample_workspace_bytes()) return TOYINFER_ERR_WORKSPACE;
    a.logits = logits;
    a.coin = coin;
    a.out = out_token;
    a.workspace = workspace;
    return from_hip(launch_sample(a, as_stream(stream)));
}

}  // extern "C"
