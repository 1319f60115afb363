/* Minimal Qwen3 forward on one MI355X for the end-to-end configuration:
 * prefill of a prompt, then decode steps (greedy or sampled) whose body (all layers, the
 * lm-head, the token pick and the position advance) can be captured once in a
 * hipGraph and replayed, reading the position and the current token on the
 * device.  This re-creates the part of the reference's Transformer that the
 * attention path sits in (src/transformer.cpp:320-681): the prefill layer
 * loop (:320-470), the decode body (:483-628, whose three-stream fork/join
 * becomes fused launches here) and the graph capture/replay (:630-681).  Weights are the
 * caller's device buffers, laid out as the reference's loader produces them
 * (projections [out][in] row-major bf16, norms [dim] bf16, tied or separate
 * lm-head [vocab][hidden]).
 *
 * The model object owns its state (KV cache [layers][max_seq_len][Hkv*D],
 * activations, rotary table, token list) in one device allocation made at
 * create time, one stream (default priority) and the graph; no call after
 * create allocates.  hidden_size, intermediate_size and Hq*D are multiples
 * of 64 and at most 16384. */
#ifndef TOYINFER_QWEN3_H_
#define TOYINFER_QWEN3_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct toyinfer_qwen3_config {
    uint32_t num_layers;
    uint32_t hidden_size;
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;           /* 64 or 128 */
    uint32_t intermediate_size;
    uint32_t vocab_size;
    uint32_t max_seq_len;        /* KV-cache rows and the token list length */
    uint32_t max_prefill_tokens; /* sizes the prefill activations */
    float rms_norm_eps;
    float rope_theta;
} toyinfer_qwen3_config;

typedef struct toyinfer_qwen3_layer {
    const void* input_layernorm;          /* [hidden] */
    const void* q_proj;                   /* [Hq*D][hidden] */
    const void* k_proj;                   /* [Hkv*D][hidden] */
    const void* v_proj;                   /* [Hkv*D][hidden] */
    const void* q_norm;                   /* [D] */
    const void* k_norm;                   /* [D] */
    const void* o_proj;                   /* [hidden][Hq*D] */
    const void* post_attention_layernorm; /* [hidden] */
    const void* gate_proj;                /* [inter][hidden] */
    const void* up_proj;                  /* [inter][hidden] */
    const void* down_proj;                /* [hidden][inter] */
} toyinfer_qwen3_layer;

typedef struct toyinfer_qwen3 toyinfer_qwen3;

/* ------------------------------------------------ checkpoint files (host)
 * The reference reads config.json into LLMConfig (src/config.cpp:10-40) and
 * copies the data sections of model-0000i-of-00003.safetensors into one
 * device allocation, finding each tensor through an offset table that
 * export.py generates for Qwen3-4B (src/qwen.cpp:17-416, 431-518).  Here the
 * loader reads the safetensors headers themselves, so any layer count and
 * any shard split works: the shards are the files named by
 * model.safetensors.index.json when present, else every *.safetensors in
 * the directory (sorted by name, as export.py:254-300 orders them). */

typedef struct toyinfer_qwen3_model_info {
    uint32_t bos_token_id;
    uint32_t eos_token_id;
    uint32_t max_position_embeddings;
    int32_t tie_word_embeddings; /* 1 when config.json says so (lm_head = embed_tokens) */
} toyinfer_qwen3_model_info;

/* Fills cfg from model_dir/config.json (num_hidden_layers, hidden_size,
 * num_attention_heads, num_key_value_heads, head_dim, intermediate_size,
 * vocab_size, rms_norm_eps, rope_theta) with the caller's max_seq_len (0:
 * max_position_embeddings) and max_prefill_tokens; info (may be NULL) gets
 * the remaining fields.  TOYINFER_ERR_IO for a missing file, malformed JSON
 * or a missing or non-numeric field. */
int toyinfer_qwen3_read_config(const char* model_dir, uint32_t max_seq_len,
                               uint32_t max_prefill_tokens, toyinfer_qwen3_config* cfg,
                               toyinfer_qwen3_model_info* info);

/* Weights on the device: every tensor the model reads, each at a 256-byte
 * aligned offset of one allocation. */
typedef struct toyinfer_qwen3_weights {
    void* device;
    size_t device_bytes;
    const void* embed_tokens;
    const void* final_norm;
    const void* lm_head; /* lm_head.weight, or embed_tokens when tied or absent */
    toyinfer_qwen3_layer* layers; /* num_layers entries (host memory, owned) */
    uint32_t num_layers;
} toyinfer_qwen3_weights;

/* Host-only check of the checkpoint against cfg: every tensor present
 * (model.embed_tokens.weight, model.norm.weight, optional lm_head.weight,
 * and per layer model.layers.L.{input_layernorm, post_attention_layernorm,
 * self_attn.{q,k,v,o}_proj, self_attn.{q,k}_norm, mlp.{gate,up,down}_proj}
 * .weight), of dtype BF16, with the shape cfg implies and its bytes inside
 * its file.  *device_bytes receives what the load allocates.  No HIP call. */
int toyinfer_qwen3_check_weights(const char* model_dir, const toyinfer_qwen3_config* cfg,
                                 int tie_word_embeddings, size_t* device_bytes);

/* The check above, then one device allocation and the tensors streamed into
 * it through two pinned staging buffers (up to 64 MiB each) on `stream`
 * (waited for before returning).  On failure nothing stays allocated. */
int toyinfer_qwen3_load_weights(const char* model_dir, const toyinfer_qwen3_config* cfg,
                                int tie_word_embeddings, void* stream,
                                toyinfer_qwen3_weights* out);
void toyinfer_qwen3_free_weights(toyinfer_qwen3_weights* w);

/* Device bytes create() allocates for this configuration. */
size_t toyinfer_qwen3_state_bytes(const toyinfer_qwen3_config* cfg);

/* Checks the configuration and pointers, allocates the state, builds the
 * inverse frequencies and rotary table.  `layers` (num_layers entries) is
 * copied.  Returns a status of include/toyinfer_attn.h. */
int toyinfer_qwen3_create(const toyinfer_qwen3_config* cfg, const void* embed_tokens,
                          const void* final_norm, const void* lm_head,
                          const toyinfer_qwen3_layer* layers, toyinfer_qwen3** out);
void toyinfer_qwen3_destroy(toyinfer_qwen3* m);

/* Runs the prompt token_ids_d[0..num_tokens) (device memory) through every
 * layer (KV cache rows 0..num_tokens-1 written), the final norm and the
 * lm-head on the last token, and the pick that toyinfer_qwen3_set_sampling
 * selects (greedy by default): afterwards the logits, tokens[num_tokens] and
 * the device position (= num_tokens) are set.  Enqueued on the model's
 * stream; returns without waiting.  The ids are copied on the model's stream
 * with no ordering against the caller's streams: token_ids_d must stay valid
 * and unmodified until the model's stream has passed this call (for example
 * until toyinfer_qwen3_synchronize returns). */
int toyinfer_qwen3_prefill(toyinfer_qwen3* m, const uint32_t* token_ids_d, uint32_t num_tokens);

/* `steps` decode steps from the device position: each runs the token at
 * tokens[pos] through the layers (KV row pos), writes the pick that
 * toyinfer_qwen3_set_sampling selects (greedy by default) to tokens[pos + 1]
 * and advances pos.  With use_graph the step body is captured on first use and
 * replayed (one graph launch per step); without it the same kernels are
 * launched directly.  pos + steps must stay below max_seq_len. */
int toyinfer_qwen3_decode(toyinfer_qwen3* m, uint32_t steps, int use_graph);

/* The pick after the lm-head in prefill and decode, as the reference's
 * sampler options (--temperature, --top_k, --top_p; src/options.cpp:32-34,
 * src/sampler.cpp:18-67; see toyinfer_sample_topk_topp_f32): greedy (the
 * default after create) when |temperature| < 1e-3 or top_k == 1.  Each draw's
 * uniform number is a SplitMix64 hash of (seed, device position), so graph
 * replays sample without host work and a seed reproduces a generation.  A
 * captured decode graph is dropped and captured again on the next decode. */
int toyinfer_qwen3_set_sampling(toyinfer_qwen3* m, float temperature, uint32_t top_k,
                                float top_p, uint64_t seed);

/* Waits for the model's stream. */
int toyinfer_qwen3_synchronize(toyinfer_qwen3* m);

/* Device views of the state: logits [vocab] fp32 of the last forward, the
 * token list [max_seq_len] (prompt, then generated), the position. */
const float* toyinfer_qwen3_logits(const toyinfer_qwen3* m);
const uint32_t* toyinfer_qwen3_tokens(const toyinfer_qwen3* m);
const uint32_t* toyinfer_qwen3_position(const toyinfer_qwen3* m);
/* The hipStream_t the model enqueues on. */
void* toyinfer_qwen3_stream(const toyinfer_qwen3* m);

#ifdef __cplusplus
}
#endif

#endif /* TOYINFER_QWEN3_H_ */
