// Minimal Qwen3 forward (include/toyinfer_qwen3.h): the prefill layer loop
// and the greedy decode body around the attention path, with the decode body
// captured once in a hipGraph and replayed.
//
// Reference: src/transformer.cpp:320-470 (prefill), :483-628 (decode body,
// three-stream fork/join), :630-681 (graph capture / replay).  Differences,
// all keeping the reference's rounding points:
//  * one stream: the q/k/v projections the reference forks over three streams
//    are one grid over the three weight segments, and gate/up are one grid
//    whose epilogue applies SwiGLU;
//  * prefill: q_norm/k_norm + RoPE are fused into the attention call, which
//    writes the normalised, rotated K straight into the layer's cache rows;
//    the V projection writes straight into the cache rows (no D2D copies);
//    the residual stream stays in `hidden` (no residual copy);
//  * decode: the RMSNorms are applied while each fused projection stages its
//    input, the residual adds are projection epilogues, the six
//    pre-attention launches are one (decode_qkv_prologue), attention is the
//    split-K kernel with the length read on the device, and the body ends
//    with a device pick (argmax, or top-k/top-p sampling) that appends the
//    next token and advances the position, so consecutive graph replays need
//    no host work;
//  * no memset nodes (the reference's rmsnorm clears its sum with one).
#include <hip/hip_runtime.h>

#include <new>
#include <vector>

#include "../../include/toyinfer_attn.h"
#include "../../include/toyinfer_qwen3.h"
#include "kernels.hpp"

using namespace tiattn;

struct toyinfer_qwen3 {
    toyinfer_qwen3_config cfg{};
    const void* embed = nullptr;
    const void* final_norm = nullptr;
    const void* lm_head = nullptr;
    std::vector<toyinfer_qwen3_layer> layers;

    char* mem = nullptr;
    uint32_t* tokens = nullptr;
    uint32_t* pos = nullptr;
    uint32_t* seq_len = nullptr;
    void* sample_ws = nullptr;  // sampler / argmax workspace, zero between launches
    SampleArgs sample;          // the pick after the lm-head (greedy by default)
    float* inv_freq = nullptr;
    float* rope = nullptr;
    float* rope_cur = nullptr;  // the decode position's row of `rope`, [D/2] (cos, sin)
    float* logits = nullptr;
    uint16_t* k_cache = nullptr;
    uint16_t* v_cache = nullptr;
    // prefill activations, [max_prefill_tokens][...]
    uint16_t *p_hidden, *p_xn, *p_q, *p_k, *p_o, *p_tmp, *p_gate, *p_up, *p_inter;
    // decode activations, one token
    uint16_t *d_hidden, *d_xn, *d_q, *d_k, *d_v, *d_o, *d_tmp, *d_gate, *d_up, *d_inter;
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    uint32_t splits = 0;

    hipStream_t s[1] = {nullptr};
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

#define TRY(x)                                   \
    do {                                         \
        const int st_ = (x);                     \
        if (st_ != TOYINFER_OK) return st_;      \
    } while (0)
#define TRYH(x)                                                   \
    do {                                                          \
        if ((x) != hipSuccess) return TOYINFER_ERR_HIP;           \
    } while (0)

size_t up256(size_t x) { return (x + 255) / 256 * 256; }

// Offsets of every state buffer in the one allocation (dry run when m is null).
size_t carve(const toyinfer_qwen3_config& c, uint32_t splits, toyinfer_qwen3* m) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = up256(off + bytes);
        return o;
    };
    const size_t kv = (size_t)c.num_kv_heads * c.head_dim, qd = (size_t)c.num_q_heads * c.head_dim;
    const size_t P = c.max_prefill_tokens, H = c.hidden_size, F = c.intermediate_size;
    const size_t o_tokens = take(4ull * c.max_seq_len);
    const size_t o_pos = take(4), o_len = take(4), o_sws = take(sample_workspace_bytes());
    const size_t o_inv = take(4ull * c.head_dim / 2);
    const size_t o_rope = take(4ull * c.max_seq_len * c.head_dim);
    const size_t o_rope_cur = take(4ull * c.head_dim);
    const size_t o_logits = take(4ull * c.vocab_size);
    const size_t o_kc = take(2ull * c.num_layers * c.max_seq_len * kv);
    const size_t o_vc = take(2ull * c.num_layers * c.max_seq_len * kv);
    size_t o_p[9], o_d[10];
    const size_t p_sizes[9] = {P * H, P * H, P * qd, P * kv, P * qd, P * H, P * F, P * F, P * F};
    for (int i = 0; i < 9; ++i) o_p[i] = take(2 * p_sizes[i]);
    const size_t d_sizes[10] = {H, H, qd, kv, kv, qd, H, F, F, F};
    for (int i = 0; i < 10; ++i) o_d[i] = take(2 * d_sizes[i]);
    const size_t ws = toyinfer_decode_workspace_bytes(1, c.num_q_heads, c.head_dim, splits);
    const size_t o_ws = take(ws);
    if (m) {
        char* b = m->mem;
        m->tokens = reinterpret_cast<uint32_t*>(b + o_tokens);
        m->pos = reinterpret_cast<uint32_t*>(b + o_pos);
        m->seq_len = reinterpret_cast<uint32_t*>(b + o_len);
        m->sample_ws = b + o_sws;
        m->inv_freq = reinterpret_cast<float*>(b + o_inv);
        m->rope = reinterpret_cast<float*>(b + o_rope);
        m->rope_cur = reinterpret_cast<float*>(b + o_rope_cur);
        m->logits = reinterpret_cast<float*>(b + o_logits);
        m->k_cache = reinterpret_cast<uint16_t*>(b + o_kc);
        m->v_cache = reinterpret_cast<uint16_t*>(b + o_vc);
        uint16_t** pp[9] = {&m->p_hidden, &m->p_xn, &m->p_q, &m->p_k, &m->p_o,
                            &m->p_tmp, &m->p_gate, &m->p_up, &m->p_inter};
        for (int i = 0; i < 9; ++i) *pp[i] = reinterpret_cast<uint16_t*>(b + o_p[i]);
        uint16_t** dp[10] = {&m->d_hidden, &m->d_xn, &m->d_q, &m->d_k, &m->d_v,
                             &m->d_o, &m->d_tmp, &m->d_gate, &m->d_up, &m->d_inter};
        for (int i = 0; i < 10; ++i) *dp[i] = reinterpret_cast<uint16_t*>(b + o_d[i]);
        m->attn_ws = b + o_ws;
        m->attn_ws_bytes = ws;
    }
    return off;
}

bool a16(const void* p) { return p && ((uintptr_t)p & 15) == 0; }

int check_config(const toyinfer_qwen3_config* c) {
    if (!c) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (c->head_dim != 64 && c->head_dim != 128) return TOYINFER_ERR_UNSUPPORTED;
    if (c->num_layers == 0 || c->num_q_heads == 0 || c->num_kv_heads == 0 ||
        c->num_q_heads % c->num_kv_heads != 0 || c->num_q_heads > 64 ||
        c->hidden_size == 0 || c->hidden_size % 64 != 0 || c->intermediate_size == 0 ||
        c->intermediate_size % 64 != 0 || c->vocab_size == 0 || c->max_seq_len < 2 ||
        c->max_prefill_tokens == 0 || c->max_prefill_tokens >= c->max_seq_len ||
        c->max_prefill_tokens > 65535u || c->hidden_size > kDecodeGemvMaxN ||
        c->intermediate_size > kDecodeGemvMaxN ||
        c->num_q_heads * c->head_dim > kDecodeGemvMaxN || !(c->rms_norm_eps > 0.0f) ||
        !(c->rope_theta > 0.0f))
        return TOYINFER_ERR_INVALID_ARGUMENT;
    return TOYINFER_OK;
}

// The token pick after the lm-head: tokens[*pos + 1] and *pos += 1.
hipError_t launch_pick(toyinfer_qwen3* m) {
    SampleArgs a = m->sample;
    a.logits = m->logits;
    a.out = m->tokens;
    a.pos = m->pos;
    a.out_cap = m->cfg.max_seq_len;
    a.workspace = m->sample_ws;
    return launch_sample(a, m->s[0]);
}

// One decode step for the token at tokens[*pos]; ends with tokens[*pos + 1]
// and *pos += 1.  Six launches per layer, one stream, kernel launches only
// (capturable):
//   RMSNorm + q/k/v projections (one grid over the three weight segments,
//     where the reference forks them over three streams, :513-533);
//   split-K attention with the q/k norm + RoPE and the cache-row writes
//     folded in (the reference's separate norm, RoPE and cache-write
//     kernels); the split combine;
//   o projection + residual add; RMSNorm + gate/up + SwiGLU;
//   down projection + residual add;
// then the final norm, the lm-head and the token pick.
int decode_body(toyinfer_qwen3* m) {
    const toyinfer_qwen3_config& c = m->cfg;
    const uint32_t H = c.hidden_size, F = c.intermediate_size, V = c.vocab_size;
    const uint32_t hq = c.num_q_heads, hkv = c.num_kv_heads, d = c.head_dim;
    const uint32_t qd = hq * d, kv = hkv * d, msl = c.max_seq_len;
    const float eps = c.rms_norm_eps;
    hipStream_t st = m->s[0];
    void* s0 = st;
    auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
    TRYH(launch_decode_step_setup(u16(m->embed), m->tokens, m->pos, m->d_hidden, m->seq_len, H, V,
                                  msl, st, m->rope, m->rope_cur, d));
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const toyinfer_qwen3_layer& L = m->layers[l];
        uint16_t* kc = m->k_cache + (size_t)l * msl * kv;
        uint16_t* vc = m->v_cache + (size_t)l * msl * kv;
        DecodeGemvArgs qkv;
        qkv.x = m->d_hidden;
        qkv.norm_w = u16(L.input_layernorm);
        qkv.eps = eps;
        qkv.n = H;
        qkv.nseg = 3;
        qkv.w[0] = u16(L.q_proj);
        qkv.w[1] = u16(L.k_proj);
        qkv.w[2] = u16(L.v_proj);
        qkv.y[0] = m->d_q;
        qkv.y[1] = m->d_k;
        qkv.y[2] = m->d_v;
        qkv.rows[0] = qd;
        qkv.rows[1] = kv;
        qkv.rows[2] = kv;
        TRYH(launch_decode_gemv(qkv, st));
        DecodeProblem ap{};
        ap.q = m->d_q;
        ap.k = kc;
        ap.v = vc;
        ap.batch = 1;
        ap.hq = hq;
        ap.hkv = hkv;
        ap.d = d;
        ap.len_mode = kLenDevice;
        ap.len_dev = m->seq_len;
        ap.len_cap = msl;
        ap.splits = m->splits;
        ap.slice_rows = (uint64_t)m->splits * 128 >= msl ? 128 : 0;
        DecodePrologue pro;
        pro.q_w = u16(L.q_norm);
        pro.k_raw = m->d_k;
        pro.k_w = u16(L.k_norm);
        pro.v_raw = m->d_v;
        pro.rope = reinterpret_cast<const float2*>(m->rope_cur);
        pro.k_cache = kc;
        pro.v_cache = vc;
        pro.eps = eps;
        const DecodePartials part = decode_partials_in(m->attn_ws, hq, m->splits, d);
        TRYH(launch_decode_split_prologue(ap, part, pro, st));
        TRYH(launch_decode_combine(ap, part, m->d_o, st));
        DecodeGemvArgs o;
        o.x = m->d_o;
        o.n = qd;
        o.w[0] = u16(L.o_proj);
        o.y[0] = m->d_hidden;
        o.rows[0] = H;
        o.epi = kDgResidual;
        TRYH(launch_decode_gemv(o, st));
        DecodeGemvArgs gu;
        gu.x = m->d_hidden;
        gu.norm_w = u16(L.post_attention_layernorm);
        gu.eps = eps;
        gu.n = H;
        gu.w[0] = u16(L.gate_proj);
        gu.w[1] = u16(L.up_proj);
        gu.y[0] = m->d_inter;
        gu.rows[0] = F;
        gu.epi = kDgSwiglu;
        TRYH(launch_decode_gemv(gu, st));
        DecodeGemvArgs dn;
        dn.x = m->d_inter;
        dn.n = F;
        dn.w[0] = u16(L.down_proj);
        dn.y[0] = m->d_hidden;
        dn.rows[0] = H;
        dn.epi = kDgResidual;
        TRYH(launch_decode_gemv(dn, st));
    }
    // The lm-head streams the largest matrix: the plain GEMV (more waves in
    // flight) after a separate norm beats the fused form here.
    TRY(toyinfer_rmsnorm_bf16(m->d_hidden, m->final_norm, m->d_xn, nullptr, eps, H, s0));
    TRY(toyinfer_gemv_proj_bf162float(m->lm_head, m->d_xn, m->logits, V, H, s0));
    TRYH(launch_pick(m));
    return TOYINFER_OK;
}

void release(toyinfer_qwen3* m) {
    if (!m) return;
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    if (m->s[0]) (void)hipStreamDestroy(m->s[0]);
    if (m->mem) (void)hipFree(m->mem);
    delete m;
}

}  // namespace

extern "C" {

size_t toyinfer_qwen3_state_bytes(const toyinfer_qwen3_config* cfg) {
    if (check_config(cfg) != TOYINFER_OK) return 0;
    const uint32_t splits = toyinfer_decode_default_splits(1, cfg->num_q_heads, cfg->num_kv_heads,
                                                           cfg->head_dim, cfg->max_seq_len);
    return carve(*cfg, splits, nullptr);
}

int toyinfer_qwen3_create(const toyinfer_qwen3_config* cfg, const void* embed_tokens,
                          const void* final_norm, const void* lm_head,
                          const toyinfer_qwen3_layer* layers, toyinfer_qwen3** out) {
    if (!out) return TOYINFER_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    TRY(check_config(cfg));
    if (!a16(embed_tokens) || !a16(final_norm) || !a16(lm_head) || !layers)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    for (uint32_t l = 0; l < cfg->num_layers; ++l) {
        const toyinfer_qwen3_layer& L = layers[l];
        const void* w[11] = {L.input_layernorm, L.q_proj,  L.k_proj, L.v_proj,
                             L.q_norm,          L.k_norm,  L.o_proj, L.post_attention_layernorm,
                             L.gate_proj,       L.up_proj, L.down_proj};
        for (const void* p : w)
            if (!a16(p)) return TOYINFER_ERR_INVALID_ARGUMENT;
    }
    toyinfer_qwen3* m = new (std::nothrow) toyinfer_qwen3();
    if (!m) return TOYINFER_ERR_HIP;
    m->cfg = *cfg;
    m->embed = embed_tokens;
    m->final_norm = final_norm;
    m->lm_head = lm_head;
    m->layers.assign(layers, layers + cfg->num_layers);
    (void)sample_config(cfg->vocab_size, 0.0f, 1, 1.0f, m->sample);
    m->splits = toyinfer_decode_default_splits(1, cfg->num_q_heads, cfg->num_kv_heads,
                                               cfg->head_dim, cfg->max_seq_len);
    const size_t bytes = carve(*cfg, m->splits, nullptr);
    const bool ok = hipMalloc(&m->mem, bytes) == hipSuccess &&
                    hipStreamCreateWithFlags(&m->s[0], hipStreamNonBlocking) == hipSuccess;
    if (!ok) {
        release(m);
        return TOYINFER_ERR_HIP;
    }
    carve(*cfg, m->splits, m);
    int st = toyinfer_precompute_freq_f32(m->inv_freq, (int)cfg->head_dim, cfg->rope_theta, m->s[0]);
    if (st == TOYINFER_OK)
        st = toyinfer_rope_cos_sin_f32(m->rope, m->inv_freq, cfg->max_seq_len, cfg->head_dim,
                                       m->s[0]);
    uint32_t* sw = static_cast<uint32_t*>(m->sample_ws);
    uint32_t* zeros[5] = {m->pos, sw, sw + 1, sw + 2, sw + 3};
    for (uint32_t* z : zeros)
        if (st == TOYINFER_OK && launch_set_u32(z, 0, m->s[0]) != hipSuccess) st = TOYINFER_ERR_HIP;
    if (st == TOYINFER_OK && hipStreamSynchronize(m->s[0]) != hipSuccess) st = TOYINFER_ERR_HIP;
    if (st != TOYINFER_OK) {
        release(m);
        return st;
    }
    *out = m;
    return TOYINFER_OK;
}

void toyinfer_qwen3_destroy(toyinfer_qwen3* m) {
    if (!m) return;
    if (m->s[0]) (void)hipStreamSynchronize(m->s[0]);
    release(m);
}

int toyinfer_qwen3_prefill(toyinfer_qwen3* m, const uint32_t* token_ids_d, uint32_t num_tokens) {
    if (!m || !token_ids_d || ((uintptr_t)token_ids_d & 3) || num_tokens == 0 ||
        num_tokens > m->cfg.max_prefill_tokens)
        return TOYINFER_ERR_INVALID_ARGUMENT;
    const toyinfer_qwen3_config& c = m->cfg;
    const uint32_t T = num_tokens, H = c.hidden_size, F = c.intermediate_size, V = c.vocab_size;
    const uint32_t hq = c.num_q_heads, hkv = c.num_kv_heads, d = c.head_dim;
    const uint32_t qd = hq * d, kv = hkv * d, msl = c.max_seq_len;
    const float eps = c.rms_norm_eps;
    void* s0 = m->s[0];
    TRYH(hipMemcpyAsync(m->tokens, token_ids_d, 4ull * T, hipMemcpyDeviceToDevice, m->s[0]));
    TRY(toyinfer_gather_embedding_bf16(m->embed, m->tokens, m->p_hidden, T, H, V, s0));
    hipStream_t st = m->s[0];
    auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
    // Projections of more than a few tokens run as stacked-segment GEMMs
    // (q/k/v in one launch, gate/up in one) with the residual adds in the
    // o and down epilogues; short prompts take the separate GEMV calls.
    const bool gemm = proj_uses_gemm(T, H, m->layers[0].q_proj, m->p_xn) &&
                      proj_uses_gemm(T, qd, m->layers[0].o_proj, m->p_o) &&
                      proj_uses_gemm(T, F, m->layers[0].down_proj, m->p_inter);
    PrefillProblem attn{};
    attn.q = m->p_q;
    attn.o = m->p_o;
    attn.s = T;
    attn.hq = hq;
    attn.hkv = hkv;
    attn.d = d;
    const bool split_attn = prefill_uses_split(attn);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const toyinfer_qwen3_layer& L = m->layers[l];
        uint16_t* kc = m->k_cache + (size_t)l * msl * kv;
        uint16_t* vc = m->v_cache + (size_t)l * msl * kv;
        TRY(toyinfer_batch_rmsnorm_bf16(m->p_hidden, L.input_layernorm, m->p_xn, nullptr, eps, T,
                                        H, s0));
        if (gemm) {
            GemmArgs g;
            g.x = m->p_xn;
            g.T = T;
            g.N = H;
            g.nseg = 3;
            g.w[0] = u16(L.q_proj);
            g.w[1] = u16(L.k_proj);
            g.w[2] = u16(L.v_proj);
            g.y[0] = m->p_q;
            g.y[1] = m->p_k;
            g.y[2] = vc;
            g.rows[0] = qd;
            g.rows[1] = kv;
            g.rows[2] = kv;
            TRYH(launch_gemm(g, st));
        } else {
            TRY(toyinfer_batch_gemv_proj_bf16(L.q_proj, m->p_xn, m->p_q, T, qd, H, s0));
            TRY(toyinfer_batch_gemv_proj_bf16(L.k_proj, m->p_xn, m->p_k, T, kv, H, s0));
            TRY(toyinfer_batch_gemv_proj_bf16(L.v_proj, m->p_xn, vc, T, kv, H, s0));
        }
        if (split_attn) {
            // Q normalised and rotated in place, K into the cache rows, one
            // launch; then the split kernel on the prepared Q (its fused-Q
            // form cannot keep the next item's Q in flight).
            TRYH(launch_qk_norm_rope_rows(m->p_q, m->p_q, u16(L.q_norm), m->p_k, kc,
                                          u16(L.k_norm), m->rope, eps, T, hq, hkv, d, st));
            PrefillProblem pp = attn;
            pp.k = kc;
            pp.v = vc;
            TRYH(launch_prefill(pp, st));
        } else {
            TRY(toyinfer_prefill_qknorm_rope_attention_bf16(m->p_q, m->p_k, vc, m->p_o, kc,
                                                            L.q_norm, L.k_norm, m->rope, eps, hq,
                                                            hkv, d, T, s0));
        }
        if (gemm) {
            GemmArgs g;
            g.x = m->p_o;
            g.T = T;
            g.N = qd;
            g.w[0] = u16(L.o_proj);
            g.y[0] = m->p_hidden;
            g.rows[0] = H;
            g.residual = true;
            TRYH(launch_gemm(g, st));
        } else {
            TRY(toyinfer_batch_gemv_proj_bf16(L.o_proj, m->p_o, m->p_tmp, T, H, qd, s0));
            TRY(toyinfer_batch_residual_add_bf16(m->p_tmp, m->p_hidden, T, H, s0));
        }
        TRY(toyinfer_batch_rmsnorm_bf16(m->p_hidden, L.post_attention_layernorm, m->p_xn, nullptr,
                                        eps, T, H, s0));
        if (gemm) {
            GemmArgs g;
            g.x = m->p_xn;
            g.T = T;
            g.N = H;
            g.nseg = 2;
            g.w[0] = u16(L.gate_proj);
            g.w[1] = u16(L.up_proj);
            g.y[0] = m->p_inter;  // SwiGLU in the epilogue
            g.rows[0] = F;
            g.rows[1] = F;
            g.swiglu = true;
            TRYH(launch_gemm(g, st));
        } else {
            TRY(toyinfer_batch_gemv_proj_bf16(L.gate_proj, m->p_xn, m->p_gate, T, F, H, s0));
            TRY(toyinfer_batch_gemv_proj_bf16(L.up_proj, m->p_xn, m->p_up, T, F, H, s0));
            TRY(toyinfer_batch_swiglu_bf16x2(m->p_gate, m->p_up, m->p_inter, T, F, s0));
        }
        if (gemm) {
            GemmArgs g;
            g.x = m->p_inter;
            g.T = T;
            g.N = F;
            g.w[0] = u16(L.down_proj);
            g.y[0] = m->p_hidden;
            g.rows[0] = H;
            g.residual = true;
            TRYH(launch_gemm(g, st));
        } else {
            TRY(toyinfer_batch_gemv_proj_bf16(L.down_proj, m->p_inter, m->p_tmp, T, H, F, s0));
            TRY(toyinfer_batch_residual_add_bf16(m->p_tmp, m->p_hidden, T, H, s0));
        }
    }
    // Final norm of the last token, the lm-head, then the greedy pick.
    TRY(toyinfer_rmsnorm_bf16(m->p_hidden + (size_t)(T - 1) * H, m->final_norm, m->d_xn, nullptr,
                              eps, H, s0));
    TRY(toyinfer_gemv_proj_bf162float(m->lm_head, m->d_xn, m->logits, V, H, s0));
    TRYH(launch_set_u32(m->pos, T - 1, st));
    TRYH(launch_pick(m));
    return TOYINFER_OK;
}

int toyinfer_qwen3_decode(toyinfer_qwen3* m, uint32_t steps, int use_graph) {
    if (!m || steps >= m->cfg.max_seq_len) return TOYINFER_ERR_INVALID_ARGUMENT;
    if (!use_graph) {
        for (uint32_t i = 0; i < steps; ++i) TRY(decode_body(m));
        return TOYINFER_OK;
    }
    if (!m->exec) {
        TRYH(hipStreamBeginCapture(m->s[0], hipStreamCaptureModeRelaxed));
        const int st = decode_body(m);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(m->s[0], &g);
        if (st != TOYINFER_OK || e != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return st != TOYINFER_OK ? st : TOYINFER_ERR_HIP;
        }
        if (hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0) != hipSuccess) {
            (void)hipGraphDestroy(g);
            m->exec = nullptr;
            return TOYINFER_ERR_HIP;
        }
        m->graph = g;
    }
    for (uint32_t i = 0; i < steps; ++i) TRYH(hipGraphLaunch(m->exec, m->s[0]));
    return TOYINFER_OK;
}

int toyinfer_qwen3_set_sampling(toyinfer_qwen3* m, float temperature, uint32_t top_k, float top_p,
                                uint64_t seed) {
    if (!m) return TOYINFER_ERR_INVALID_ARGUMENT;
    SampleArgs a;
    TRY(sample_config(m->cfg.vocab_size, temperature, top_k, top_p, a));
    a.seed = seed;
    m->sample = a;
    // The captured step holds the old parameters: capture again on next use.
    if (m->exec) {
        TRYH(hipStreamSynchronize(m->s[0]));
        (void)hipGraphExecDestroy(m->exec);
        m->exec = nullptr;
    }
    if (m->graph) {
        (void)hipGraphDestroy(m->graph);
        m->graph = nullptr;
    }
    return TOYINFER_OK;
}

int toyinfer_qwen3_synchronize(toyinfer_qwen3* m) {
    if (!m) return TOYINFER_ERR_INVALID_ARGUMENT;
    return hipStreamSynchronize(m->s[0]) == hipSuccess ? TOYINFER_OK : TOYINFER_ERR_HIP;
}

const float* toyinfer_qwen3_logits(const toyinfer_qwen3* m) { return m ? m->logits : nullptr; }
const uint32_t* toyinfer_qwen3_tokens(const toyinfer_qwen3* m) { return m ? m->tokens : nullptr; }
const uint32_t* toyinfer_qwen3_position(const toyinfer_qwen3* m) { return m ? m->pos : nullptr; }
void* toyinfer_qwen3_stream(const toyinfer_qwen3* m) { return m ? m->s[0] : nullptr; }

}  // extern "C"
