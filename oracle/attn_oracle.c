/*
 * CPU oracle for the ToyInfer causal-GQA attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker, never the thing
 * measured or shipped: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product path
 * (toyinfer_amd/) never links, imports or calls anything in oracle/.
 *
 * It restates, in plain C, the host references that the reference's own
 * tests use as ground truth (all citations are into the reference tree):
 *
 *   bf16 rounding ........ tests/test_helpers.h:50-52 (__float2bfloat16, RNE)
 *   flash case generator . tests/flash_attention_test_common.h:25-85
 *   causal-focus case .... tests/test_flash_attention_v1_bf16.cu:11-45
 *   flash reference ...... tests/flash_attention_test_common.h:87-136
 *   decode case generator  tests/attention_test_common.h:40-85
 *   decode qk scores ..... tests/attention_test_common.h:87-109
 *   decode softmax ....... tests/attention_test_common.h:111-130
 *   decode apply ......... tests/attention_test_common.h:132-151
 *   decode compositions .. tests/attention_test_common.h:153-178
 *   QK-RMSNorm ........... tests/multi_rmsnorm_test_common.h:23-76
 *   RoPE ................. tests/rope_test_common.h:23-65 (single position)
 *                          src/prefill.cu:185-208 (batched: angle = token*f)
 *   inverse frequencies .. tests/precompute_freq_test_common.h:16-26
 *   projections .......... tests/gemv_test_common.h:24-65 (GEMV case and
 *                          reference sum), tests/test_batch_gemv_proj_bf16.cu:20-66
 *                          (batched case and reference)
 *   row RMSNorm, residual  tests/rmsnorm_test_common.h, tests/add_test_common.h,
 *   add, SwiGLU, argmax .. tests/swiglu_test_common.h, the batch tests, and
 *                          src/sampler.cpp:71-82
 *   top-k/top-p sampling . src/sampler.cpp:18-67 (the draw u is an input)
 *
 * Arithmetic follows the reference's host code operation by operation
 * (float vs double, accumulation order, where bf16 rounding happens).
 * The library is compiled with -ffp-contract=off so that no product+sum is
 * fused into an FMA that the reference's host code would not have fused.
 *
 * Pinning (what checks this restatement, see tests/test_oracle.py):
 *   - golden fixtures made by an independent implementation (torch fp64 /
 *     bf16 on the CPU, tests/golden/make_golden.py);
 *   - closed forms: causal row 0 == V row 0; constant K gives the causal
 *     prefix mean of V; RoPE at position 0 is the identity; inv_freq[0] == 1;
 *     RMSNorm of a constant row is gamma * sign;
 *   - invariants: softmax rows sum to 1, GQA == MHA with repeated KV heads,
 *     adding a constant to every score leaves the output unchanged, the
 *     decode output is invariant under a permutation of the cached rows;
 *   - brute force in numpy float64 on tiny inputs;
 *   - bf16 rounding against torch's float32->bfloat16 conversion on every
 *     special value class (ties, NaN, inf, subnormals).
 * Every function below is covered by at least one of these checks.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bf16 */

/* IEEE float32 -> bfloat16, round to nearest even, NaN kept quiet.
 * Same contract as __float2bfloat16 used by tests/test_helpers.h:50-52. */
uint16_t or_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {          /* NaN: keep sign, quiet */
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float or_round_to_bf16(float f) { return or_bf16_to_f32(or_f32_to_bf16(f)); }

void or_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16(in[i]);
}

void or_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_bf16_to_f32(in[i]);
}

/* ------------------------------------------------------ case generators */

/* tests/flash_attention_test_common.h:25-85.  Layouts: q [S][Hq][D],
 * k/v [S][Hkv][D], float (before bf16 rounding). */
void or_make_flash_case(uint32_t hq, uint32_t hkv, uint32_t d_head,
                        uint32_t seq, float q_phase, float kv_phase,
                        float q_scale, float k_scale, float v_scale, float* q,
                        float* k, float* v) {
    const uint32_t q_dim = hq * d_head, kv_dim = hkv * d_head;
    for (uint32_t t = 0; t < seq; ++t)
        for (uint32_t h = 0; h < hq; ++h)
            for (uint32_t d = 0; d < d_head; ++d) {
                const uint32_t idx = t * q_dim + h * d_head + d;
                const float t_term = (float)((int)(t % 3) - 1);
                q[idx] = q_scale *
                         (0.19f * sinf((float)((t + 1) * (d + 1)) * q_phase) +
                          0.13f * cosf((float)((h + 1) * (d + 2)) * q_phase * 0.7f) -
                          0.018f * (float)((t + h + d) % 5) + 0.011f * t_term);
            }
    for (uint32_t t = 0; t < seq; ++t)
        for (uint32_t kv = 0; kv < hkv; ++kv)
            for (uint32_t d = 0; d < d_head; ++d) {
                const uint32_t idx = t * kv_dim + kv * d_head + d;
                const float alt = (float)((int)((t + d) % 4) - 2);
                k[idx] = k_scale *
                         (0.17f * cosf((float)((t + 1) * (d + 1)) * kv_phase) +
                          0.09f * sinf((float)((kv + 1) * (d + 3)) * kv_phase * 1.1f) +
                          0.012f * (float)((t + kv * 2 + d) % 7) + 0.008f * alt);
                v[idx] = v_scale *
                         (0.15f * sinf((float)((t + 2) * (d + 1)) * kv_phase * 1.3f) -
                          0.12f * cosf((float)((kv + 2) * (d + 1)) * kv_phase * 0.8f) +
                          0.01f * (float)((t * 3 + kv * 5 + d) % 11) -
                          0.014f * (float)(t % 2));
            }
}

/* tests/test_flash_attention_v1_bf16.cu:11-45: Hq=2, Hkv=1, D=64, S=6. */
void or_make_causal_focus_case(float* q, float* k, float* v) {
    const uint32_t hq = 2, d_head = 64, seq = 6;
    const uint32_t q_dim = hq * d_head, kv_dim = d_head;
    for (uint32_t t = 0; t < seq; ++t) {
        for (uint32_t h = 0; h < hq; ++h)
            for (uint32_t d = 0; d < d_head; ++d)
                q[t * q_dim + h * d_head + d] = 0.25f + 0.004f * (float)d +
                                                0.015f * (float)h +
                                                0.01f * (float)(t % 2);
        for (uint32_t d = 0; d < d_head; ++d) {
            k[t * kv_dim + d] = 0.22f * (float)(t + 1) + 0.003f * (float)((d % 13) + 1);
            v[t * kv_dim + d] = 0.5f * (float)(t + 1) - 0.025f * (float)(d % 5) +
                                0.01f * (float)(d % 3);
        }
    }
}

/* tests/attention_test_common.h:40-85.  q [Hq][D]; k/v [MSL][Hkv][D]. */
void or_make_attention_case(uint32_t hq, uint32_t hkv, uint32_t d_head,
                            uint32_t max_seq_len, float q_phase, float kv_phase,
                            float* q, float* k, float* v) {
    for (uint32_t h = 0; h < hq; ++h)
        for (uint32_t d = 0; d < d_head; ++d) {
            const uint32_t idx = h * d_head + d;
            q[idx] = 0.18f * sinf((float)(idx + 1) * q_phase) -
                     0.11f * cosf((float)((h + 1) * (d + 1)) * q_phase * 0.6f) +
                     0.01f * (float)((h + d) % 5);
        }
    for (uint32_t t = 0; t < max_seq_len; ++t)
        for (uint32_t kv = 0; kv < hkv; ++kv)
            for (uint32_t d = 0; d < d_head; ++d) {
                const uint32_t idx = t * hkv * d_head + kv * d_head + d;
                k[idx] = 0.16f * cosf((float)((t + 1) * (d + 1)) * kv_phase) +
                         0.09f * sinf((float)((kv + 2) * (d + 3)) * kv_phase * 0.7f) -
                         0.008f * (float)((t + kv + d) % 7);
                v[idx] = 0.14f * sinf((float)((t + 3) * (d + 1)) * kv_phase * 1.3f) -
                         0.12f * cosf((float)((kv + 1) * (d + 2)) * kv_phase * 0.9f) +
                         0.006f * (float)((t * 5 + kv * 3 + d) % 11);
            }
}

/* tests/multi_rmsnorm_test_common.h:23-54 (input of `buffer_size`, gamma [D]). */
void or_make_rmsnorm_case(uint32_t num_heads, uint32_t d_head,
                          uint32_t buffer_size, float input_phase,
                          float weight_phase, float* input, float* weight) {
    const uint32_t size = num_heads * d_head;
    for (uint32_t h = 0; h < num_heads; ++h)
        for (uint32_t i = 0; i < d_head; ++i) {
            const uint32_t idx = h * d_head + i;
            input[idx] = 0.31f * sinf((float)(idx + 1) * input_phase) -
                         0.24f * cosf((float)((h + 1) * (i + 3)) * input_phase * 0.7f) +
                         0.01f * (float)((h + i) % 5);
        }
    for (uint32_t i = size; i < buffer_size; ++i)
        input[i] = -0.5f + 0.07f * (float)(i - size);
    for (uint32_t i = 0; i < d_head; ++i)
        weight[i] = 0.68f + 0.14f * sinf((float)(i + 5) * weight_phase) -
                    0.05f * (float)(i % 3);
}

/* tests/test_batch_multi_rmsnorm_bf16.cu:19-51 (input [B][H][D], gamma [D]). */
void or_make_batch_rmsnorm_case(uint32_t batch, uint32_t num_heads,
                                uint32_t d_head, float input_phase,
                                float weight_phase, float* input,
                                float* weight) {
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t h = 0; h < num_heads; ++h) {
            const uint32_t off = (b * num_heads + h) * d_head;
            for (uint32_t i = 0; i < d_head; ++i) {
                const uint32_t idx = off + i;
                input[idx] = 0.31f * sinf((float)(idx + 1) * input_phase) -
                             0.24f * cosf((float)((h + 1) * (i + 3)) * input_phase * 0.7f) +
                             0.01f * (float)((b + h + i) % 5);
            }
        }
    for (uint32_t i = 0; i < d_head; ++i)
        weight[i] = 0.68f + 0.14f * sinf((float)(i + 5) * weight_phase) -
                    0.05f * (float)(i % 3);
}

/* tests/rope_test_common.h:23-49 (qk of `buffer_size`, inv_freq [D/2]). */
void or_make_rope_case(uint32_t num_heads, uint32_t d_head, uint32_t buffer_size,
                       float qk_phase, float freq_scale, float* qk,
                       float* inv_freq) {
    const uint32_t size = num_heads * d_head;
    for (uint32_t i = 0; i < size; ++i)
        qk[i] = 0.34f * sinf((float)(i + 1) * qk_phase) -
                0.21f * cosf((float)(i + 5) * qk_phase * 0.7f) +
                0.012f * (float)(i % 4);
    for (uint32_t i = size; i < buffer_size; ++i)
        qk[i] = -1.0f + 0.08f * (float)(i - size);
    for (uint32_t i = 0; i < d_head / 2; ++i)
        inv_freq[i] = freq_scale * (float)(i + 1);
}

/* ------------------------------------------------------- flash (prefill) */

/* tests/flash_attention_test_common.h:87-136, for one (query row, q-head):
 * double dot * (1/sqrt(D)), double max and sum of exp, weight cast to float,
 * expected[d] += (float)w * v accumulated in float in key order. */
static void flash_row(const float* qf, const float* kf, const float* vf,
                      float* out, double* scores, uint32_t hq, uint32_t hkv,
                      uint32_t d_head, uint32_t q_pos, uint32_t q_head) {
    const uint32_t q_dim = hq * d_head, kv_dim = hkv * d_head;
    const uint32_t q_per_kv = hq / hkv;
    const double scale = 1.0 / sqrt((double)d_head);
    const uint32_t q_off = q_pos * q_dim + q_head * d_head;
    const uint32_t kv_head = q_head / q_per_kv;
    double row_max = -INFINITY;
    for (uint32_t kv = 0; kv <= q_pos; ++kv) {
        const uint32_t kv_off = kv * kv_dim + kv_head * d_head;
        double dot = 0.0;
        for (uint32_t d = 0; d < d_head; ++d)
            dot += (double)qf[q_off + d] * (double)kf[kv_off + d];
        scores[kv] = dot * scale;
        if (scores[kv] > row_max) row_max = scores[kv];
    }
    double row_sum = 0.0;
    for (uint32_t kv = 0; kv <= q_pos; ++kv) row_sum += exp(scores[kv] - row_max);
    for (uint32_t d = 0; d < d_head; ++d) out[q_off + d] = 0.0f;
    for (uint32_t kv = 0; kv <= q_pos; ++kv) {
        const double w = exp(scores[kv] - row_max) / row_sum;
        const float wf = (float)w;
        const uint32_t kv_off = kv * kv_dim + kv_head * d_head;
        for (uint32_t d = 0; d < d_head; ++d) out[q_off + d] += wf * vf[kv_off + d];
    }
}

/* Causal GQA prefill reference on float inputs (already bf16-quantised by
 * the caller).  out: float [S][Hq][D], the value before the final bf16
 * conversion (tests/flash_attention_test_common.h:138-144 rounds it).
 * rows: optional list of query positions (NULL: all S rows); rows not
 * listed are left untouched.  nthreads <= 0: all OpenMP threads. */
void or_flash_reference_f32(const float* qf, const float* kf, const float* vf,
                            float* out, uint32_t hq, uint32_t hkv,
                            uint32_t d_head, uint32_t seq, const uint32_t* rows,
                            uint32_t n_rows, int nthreads) {
    const uint32_t nr = rows ? n_rows : seq;
    const int64_t work = (int64_t)nr * hq;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
    {
        double* scores = (double*)malloc(sizeof(double) * (seq ? seq : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (int64_t w = 0; w < work; ++w) {
            const uint32_t r = (uint32_t)(w / hq), h = (uint32_t)(w % hq);
            const uint32_t q_pos = rows ? rows[r] : r;
            flash_row(qf, kf, vf, out, scores, hq, hkv, d_head, q_pos, h);
        }
        free(scores);
    }
    (void)nthreads;
}

/* Same, on bf16 bit patterns (the form the GPU receives). */
void or_flash_reference_bf16(const uint16_t* q, const uint16_t* k,
                             const uint16_t* v, float* out, uint32_t hq,
                             uint32_t hkv, uint32_t d_head, uint32_t seq,
                             const uint32_t* rows, uint32_t n_rows,
                             int nthreads) {
    const int64_t nq = (int64_t)seq * hq * d_head, nk = (int64_t)seq * hkv * d_head;
    float* qf = (float*)malloc(sizeof(float) * (nq ? nq : 1));
    float* kf = (float*)malloc(sizeof(float) * (nk ? nk : 1));
    float* vf = (float*)malloc(sizeof(float) * (nk ? nk : 1));
    or_bf16_to_f32_array(q, qf, nq);
    or_bf16_to_f32_array(k, kf, nk);
    or_bf16_to_f32_array(v, vf, nk);
    or_flash_reference_f32(qf, kf, vf, out, hq, hkv, d_head, seq, rows, n_rows,
                           nthreads);
    free(qf);
    free(kf);
    free(vf);
}

/* -------------------------------------------------------------- decode */

/* tests/attention_test_common.h:87-109: score[h*MSL+t] += dot * scale for
 * t <= pos (float dot, float scale = 1/sqrtf(D)).  Modifies score. */
void or_decode_qk_scores(const float* qf, const float* kf, float* score,
                         uint32_t hq, uint32_t hkv, uint32_t d_head,
                         uint32_t pos, uint32_t max_seq_len) {
    const uint32_t q_per_kv = hq / hkv;
    const float scale = 1.0f / sqrtf((float)d_head);
    for (uint32_t t = 0; t <= pos; ++t)
        for (uint32_t h = 0; h < hq; ++h) {
            const uint32_t kvh = h / q_per_kv;
            const uint32_t kv_off = t * hkv * d_head + kvh * d_head;
            float dot = 0.0f;
            for (uint32_t d = 0; d < d_head; ++d) dot += qf[h * d_head + d] * kf[kv_off + d];
            score[h * max_seq_len + t] += dot * scale;
        }
}

/* tests/attention_test_common.h:111-130: in-place softmax of score[h][0..pos]
 * in float (expf), entries past pos untouched. */
void or_decode_softmax(float* score, uint32_t hq, uint32_t pos,
                       uint32_t max_seq_len) {
    for (uint32_t h = 0; h < hq; ++h) {
        float* row = score + (size_t)h * max_seq_len;
        float mx = -INFINITY;
        for (uint32_t i = 0; i <= pos; ++i) mx = row[i] > mx ? row[i] : mx;
        float sum = 0.0f;
        for (uint32_t i = 0; i <= pos; ++i) sum += expf(row[i] - mx);
        for (uint32_t i = 0; i <= pos; ++i) row[i] = expf(row[i] - mx) / sum;
    }
}

/* tests/attention_test_common.h:132-151: o[h][d] += p[h][t] * v[t][kvh][d]
 * in float, t ascending. */
void or_decode_apply(const float* score, const float* vf, float* o, uint32_t hq,
                     uint32_t hkv, uint32_t d_head, uint32_t pos,
                     uint32_t max_seq_len) {
    const uint32_t q_per_kv = hq / hkv;
    for (uint32_t h = 0; h < hq; ++h) {
        const uint32_t kvh = h / q_per_kv;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float w = score[h * max_seq_len + t];
            const uint32_t kv_off = t * hkv * d_head + kvh * d_head;
            for (uint32_t d = 0; d < d_head; ++d) o[h * d_head + d] += w * vf[kv_off + d];
        }
    }
}

/* tests/attention_test_common.h:153-178 composed, as tests/test_attention_bf16.cu
 * uses it: score_out [Hq][MSL] = probabilities (zeros past pos),
 * o_buffer_out [Hq][D] float, o_out [Hq][D] bf16 bits = RNE(o_buffer). */
void or_decode_attention_f32(const float* qf, const float* kf, const float* vf,
                             float* score_out, float* o_buffer_out,
                             uint16_t* o_out, uint32_t hq, uint32_t hkv,
                             uint32_t d_head, uint32_t pos,
                             uint32_t max_seq_len) {
    memset(score_out, 0, sizeof(float) * (size_t)hq * max_seq_len);
    or_decode_qk_scores(qf, kf, score_out, hq, hkv, d_head, pos, max_seq_len);
    or_decode_softmax(score_out, hq, pos, max_seq_len);
    memset(o_buffer_out, 0, sizeof(float) * (size_t)hq * d_head);
    or_decode_apply(score_out, vf, o_buffer_out, hq, hkv, d_head, pos, max_seq_len);
    if (o_out) or_f32_to_bf16_array(o_buffer_out, o_out, (int64_t)hq * d_head);
}

/* Batched decode on bf16 bit patterns: B independent sequences, sequence b
 * at q + b*Hq*D, k/v + b*kv_batch_stride (elements), length lens[b]
 * (pos = lens[b]-1).  o_buffer_out [B][Hq][D] float.  The score scratch is
 * [Hq][max_len] per thread.  Parallel over sequences and heads. */
void or_decode_batched_bf16(const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, float* o_buffer_out,
                            uint32_t batch, uint32_t hq, uint32_t hkv,
                            uint32_t d_head, const uint32_t* lens,
                            int64_t kv_batch_stride, int nthreads) {
    const uint32_t q_per_kv = hq / hkv;
    const float scale = 1.0f / sqrtf((float)d_head);
    const int64_t work = (int64_t)batch * hq;
    uint32_t max_len = 1;
    for (uint32_t b = 0; b < batch; ++b) max_len = lens[b] > max_len ? lens[b] : max_len;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
    {
        float* row = (float*)malloc(sizeof(float) * max_len);
        float* qf = (float*)malloc(sizeof(float) * d_head);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t w = 0; w < work; ++w) {
            const uint32_t b = (uint32_t)(w / hq), h = (uint32_t)(w % hq);
            const uint32_t kvh = h / q_per_kv;
            const uint32_t len = lens[b];
            const uint16_t* qb = q + ((size_t)b * hq + h) * d_head;
            const uint16_t* kb = k + (size_t)b * kv_batch_stride;
            const uint16_t* vb = v + (size_t)b * kv_batch_stride;
            for (uint32_t d = 0; d < d_head; ++d) qf[d] = or_bf16_to_f32(qb[d]);
            /* qk scores (attention_test_common.h:94-106) */
            for (uint32_t t = 0; t < len; ++t) {
                const uint16_t* kr = kb + ((size_t)t * hkv + kvh) * d_head;
                float dot = 0.0f;
                for (uint32_t d = 0; d < d_head; ++d) dot += qf[d] * or_bf16_to_f32(kr[d]);
                row[t] = 0.0f + dot * scale;
            }
            /* softmax (attention_test_common.h:114-128) */
            float mx = -INFINITY;
            for (uint32_t t = 0; t < len; ++t) mx = row[t] > mx ? row[t] : mx;
            float sum = 0.0f;
            for (uint32_t t = 0; t < len; ++t) sum += expf(row[t] - mx);
            for (uint32_t t = 0; t < len; ++t) row[t] = expf(row[t] - mx) / sum;
            /* apply (attention_test_common.h:137-149) */
            float* ob = o_buffer_out + ((size_t)b * hq + h) * d_head;
            for (uint32_t d = 0; d < d_head; ++d) ob[d] = 0.0f;
            for (uint32_t t = 0; t < len; ++t) {
                const uint16_t* vr = vb + ((size_t)t * hkv + kvh) * d_head;
                const float w8 = row[t];
                for (uint32_t d = 0; d < d_head; ++d) ob[d] += w8 * or_bf16_to_f32(vr[d]);
            }
        }
        free(row);
        free(qf);
    }
    (void)nthreads;
}

/* ---------------------------------------------- QK-norm, RoPE, inv_freq */

/* tests/multi_rmsnorm_test_common.h:56-76: per head, float sum of squares in
 * order, inv = 1/sqrtf(sum/D + eps), out = bf16(x * inv * w).  out is float
 * holding bf16 values; rows = num_rows heads of D (num_tokens * heads). */
void or_multi_rmsnorm(const float* x, const float* w, float* out,
                      uint32_t num_rows, uint32_t d_head, float eps) {
    for (uint32_t r = 0; r < num_rows; ++r) {
        const float* xr = x + (size_t)r * d_head;
        float sum = 0.0f;
        for (uint32_t i = 0; i < d_head; ++i) sum += xr[i] * xr[i];
        const float inv = 1.0f / sqrtf(sum / (float)d_head + eps);
        for (uint32_t i = 0; i < d_head; ++i)
            out[(size_t)r * d_head + i] = or_round_to_bf16(xr[i] * inv * w[i]);
    }
}

/* tests/rope_test_common.h:48-65 for one position, batched as
 * src/prefill.cu:185-208 does: token t of `num_tokens` rotates with angle
 * (float)(pos0 + t) * inv_freq[i] (pos0 = 0 for the batched prefill), pairs
 * (i, i + D/2), float cosf/sinf, each output rounded to bf16.  In place. */
void or_rope(float* qk, const float* inv_freq, uint32_t num_tokens,
             uint32_t num_heads, uint32_t d_head, uint32_t pos0) {
    const uint32_t half = d_head / 2;
    for (uint32_t t = 0; t < num_tokens; ++t) {
        const float pos = (float)(pos0 + t);
        for (uint32_t h = 0; h < num_heads; ++h) {
            float* row = qk + ((size_t)t * num_heads + h) * d_head;
            for (uint32_t i = 0; i < half; ++i) {
                const float re = row[i], im = row[i + half];
                const float c = cosf(pos * inv_freq[i]);
                const float s = sinf(pos * inv_freq[i]);
                row[i] = or_round_to_bf16(c * re - s * im);
                row[i + half] = or_round_to_bf16(c * im + s * re);
            }
        }
    }
}

/* tests/precompute_freq_test_common.h:16-26:
 * inv_freq[i] = 1 / powf(theta, (2.0f*i)/D), i < D/2. */
void or_inv_freq(float* inv_freq, int d_head, float theta) {
    for (int i = 0; i < d_head / 2; ++i)
        inv_freq[i] = 1.0f / powf(theta, (2.0f * (float)i) / (float)d_head);
}

/* Qwen3 pre-attention prologue as src/transformer.cpp:380-391 runs it on
 * prefill: per-head RMSNorm -> bf16 -> RoPE(position = token) -> bf16.
 * x: float [T][H][D] (bf16 values), in place. */
void or_qk_norm_rope(float* x, const float* gamma, const float* inv_freq,
                     uint32_t num_tokens, uint32_t num_heads, uint32_t d_head,
                     float eps) {
    or_multi_rmsnorm(x, gamma, x, num_tokens * num_heads, d_head, eps);
    or_rope(x, inv_freq, num_tokens, num_heads, d_head, 0);
}

/* ------------------------------------------------------------ projections */

/* tests/gemv_test_common.h:24-50: x [N], w [M][N]. */
void or_make_gemv_case(uint32_t M, uint32_t N, float x_phase, float w_phase, float* x, float* w) {
    for (uint32_t i = 0; i < N; ++i)
        x[i] = 0.45f * sinf((float)(i + 1) * x_phase) -
               0.18f * cosf((float)(i + 3) * (x_phase * 0.7f)) + 0.01f * (float)(i % 5);
    for (uint32_t r = 0; r < M; ++r)
        for (uint32_t c = 0; c < N; ++c)
            w[(size_t)r * N + c] = 0.35f * cosf((float)((r + 1) * (c + 1)) * w_phase) +
                                   0.22f * sinf((float)(r + c + 3) * (w_phase * 0.6f)) -
                                   0.015f * (float)((r * 7 + c * 3) % 9);
}

/* tests/test_batch_gemv_proj_bf16.cu:20-50: w [M][N], hidden [B][N]. */
void or_make_batch_gemv_case(uint32_t batch, uint32_t M, uint32_t N, float hidden_phase,
                             float w_phase, float* hidden, float* w) {
    for (uint32_t r = 0; r < M; ++r)
        for (uint32_t c = 0; c < N; ++c)
            w[(size_t)r * N + c] = 0.33f * cosf((float)((r + 1) * (c + 1)) * w_phase) +
                                   0.21f * sinf((float)((r + 2) * (c + 3)) * (w_phase * 0.5f)) -
                                   0.012f * (float)((r * 5 + c * 7) % 11);
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t c = 0; c < N; ++c) {
            const uint32_t idx = b * N + c;
            hidden[idx] = 0.47f * sinf((float)(idx + 1) * hidden_phase) -
                          0.18f * cosf((float)(idx + c + 3) * (hidden_phase * 0.9f)) +
                          0.02f * (float)((b + c) % 6);
        }
}

/* tests/gemv_test_common.h:52-65 and tests/test_batch_gemv_proj_bf16.cu:52-66:
 * y[t][r] = sum over c in order of w[r][c] * x[t][c], float accumulation
 * (the caller rounds to bf16 where the projection outputs bf16).  Tokens are
 * independent; `nthreads` > 0 spreads them and the rows over OpenMP threads.
 *
 * With 16 or more tokens the same sums run 16 tokens wide: each vector lane
 * holds one token's running sum and performs exactly the scalar sequence
 * (sum = 0; sum = sum + rounded(w * x) for c in order; -ffp-contract=off
 * keeps the product and the sum separately rounded), so the results are
 * bit-identical to the scalar loop; tests/test_oracle.py checks that. */
typedef float or_v8f __attribute__((vector_size(32)));

enum { OR_GT = 64, OR_GR = 64 }; /* token and row tile of one task */

static void gemv_tile(const float* w, const float* xt, float* y, uint32_t t0, uint32_t nt,
                      uint32_t r0, uint32_t nr, uint32_t M, uint32_t N) {
    /* xt: the tile's tokens transposed, [N][OR_GT], zero past nt. */
    for (uint32_t rb = 0; rb < nr; rb += 4) {
        const float* wr[4];
        for (int i = 0; i < 4; ++i) wr[i] = w + (size_t)(r0 + (rb + i < nr ? rb + i : nr - 1)) * N;
        for (uint32_t tb = 0; tb < nt; tb += 16) {
            or_v8f acc[4][2];
            for (int i = 0; i < 4; ++i) acc[i][0] = acc[i][1] = (or_v8f){0, 0, 0, 0, 0, 0, 0, 0};
            const float* xc = xt + tb;
            for (uint32_t c = 0; c < N; ++c, xc += OR_GT) {
                or_v8f x0, x1;
                memcpy(&x0, xc, 32);
                memcpy(&x1, xc + 8, 32);
                for (int i = 0; i < 4; ++i) {
                    const float wv = wr[i][c];
                    acc[i][0] = acc[i][0] + wv * x0;
                    acc[i][1] = acc[i][1] + wv * x1;
                }
            }
            for (int i = 0; i < 4 && rb + i < nr; ++i)
                for (int j = 0; j < 16 && tb + j < nt; ++j)
                    y[(size_t)(t0 + tb + j) * M + r0 + rb + i] = acc[i][j >> 3][j & 7];
        }
    }
}

void or_gemv(const float* w, const float* x, float* y, uint32_t tokens, uint32_t M, uint32_t N,
             int nthreads) {
    if (tokens < 16) {
        const int64_t total = (int64_t)tokens * M;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1) if (nthreads > 1)
        for (int64_t i = 0; i < total; ++i) {
            const uint32_t t = (uint32_t)(i / M), r = (uint32_t)(i % M);
            const float* wr = w + (size_t)r * N;
            const float* xr = x + (size_t)t * N;
            float sum = 0.0f;
            for (uint32_t c = 0; c < N; ++c) sum += wr[c] * xr[c];
            y[i] = sum;
        }
        return;
    }
    const uint32_t ntb = (tokens + OR_GT - 1) / OR_GT, nrb = (M + OR_GR - 1) / OR_GR;
    float* xt = (float*)malloc((size_t)ntb * N * OR_GT * sizeof(float));
    if (!xt) abort();
    for (uint32_t b = 0; b < ntb; ++b)
        for (uint32_t c = 0; c < N; ++c)
            for (uint32_t j = 0; j < OR_GT; ++j) {
                const uint32_t t = b * OR_GT + j;
                xt[((size_t)b * N + c) * OR_GT + j] = t < tokens ? x[(size_t)t * N + c] : 0.0f;
            }
    const int64_t tasks = (int64_t)ntb * nrb;
#pragma omp parallel for schedule(dynamic) num_threads(nthreads > 0 ? nthreads : 1) if (nthreads > 1)
    for (int64_t k = 0; k < tasks; ++k) {
        const uint32_t b = (uint32_t)(k / nrb), rb = (uint32_t)(k % nrb);
        const uint32_t t0 = b * OR_GT, r0 = rb * OR_GR;
        const uint32_t nt = tokens - t0 < OR_GT ? tokens - t0 : OR_GT;
        const uint32_t nr = M - r0 < OR_GR ? M - r0 : OR_GR;
        gemv_tile(w, xt + (size_t)b * N * OR_GT, y, t0, nt, r0, nr, M, N);
    }
    free(xt);
}

/* ------------------------------------------------- rest of a decoder layer */
/* Full-row RMSNorm is or_multi_rmsnorm with one "head" of `size` values per
 * row: tests/rmsnorm_test_common.h:44-66 and
 * tests/test_batch_rmsnorm_bf16.cu:52-71 perform the same operations (float
 * sum of squares in order, 1/sqrt(sum/size + eps), x*inv*w rounded). */

/* tests/rmsnorm_test_common.h:24-42 (input, weight over buffer_size). */
void or_make_rmsnorm_row_case(uint32_t size, uint32_t buffer_size, float input_phase,
                              float weight_phase, float* input, float* weight) {
    for (uint32_t i = 0; i < size; ++i) {
        input[i] = 0.48f * sinf((float)(i + 1) * input_phase) -
                   0.22f * cosf((float)(i + 3) * input_phase * 0.7f) + 0.013f * (float)(i % 7);
        weight[i] = 0.72f + 0.18f * sinf((float)(i + 5) * weight_phase) -
                    0.04f * (float)((i * 3) % 5);
    }
    for (uint32_t i = size; i < buffer_size; ++i) {
        input[i] = -0.75f + 0.05f * (float)(i - size);
        weight[i] = 0.95f - 0.03f * (float)(i - size);
    }
}

/* tests/test_batch_rmsnorm_bf16.cu:20-46: input [batch][size], weight [size]. */
void or_make_batch_row_rmsnorm_case(uint32_t batch, uint32_t size, float input_phase,
                                    float weight_phase, float* input, float* weight) {
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t i = 0; i < size; ++i) {
            const uint32_t idx = b * size + i;
            input[idx] = 0.43f * sinf((float)(idx + 1) * input_phase) -
                         0.27f * cosf((float)(i + 2) * input_phase * 0.4f) +
                         0.02f * (float)((b + i) % 7);
        }
    for (uint32_t i = 0; i < size; ++i)
        weight[i] = 0.72f + 0.18f * sinf((float)(i + 5) * weight_phase) -
                    0.04f * (float)((i * 3) % 5);
}

/* tests/swiglu_test_common.h:22-43 (gate, up over buffer_size). */
void or_make_swiglu_case(uint32_t size, uint32_t buffer_size, float gate_phase, float up_phase,
                         float* gate, float* up) {
    for (uint32_t i = 0; i < size; ++i) {
        gate[i] = 0.9f * sinf((float)(i + 1) * gate_phase) -
                  0.7f * cosf((float)(i + 3) * gate_phase * 0.5f);
        up[i] = 0.42f * cosf((float)(i + 5) * up_phase) -
                0.31f * sinf((float)(i + 1) * up_phase * 0.8f) - 0.02f * (float)(i % 6);
    }
    for (uint32_t i = size; i < buffer_size; ++i) {
        gate[i] = -1.2f + 0.07f * (float)(i - size);
        up[i] = 0.95f - 0.05f * (float)(i - size);
    }
}

/* tests/add_test_common.h:25-51 (residual, hidden over buffer_size). */
void or_make_add_case(uint32_t size, uint32_t buffer_size, float residual_phase,
                      float hidden_phase, float tail_bias, float* residual, float* hidden) {
    for (uint32_t i = 0; i < size; ++i) {
        residual[i] = 0.23f * sinf((float)(i + 1) * residual_phase) -
                      0.08f * cosf((float)(i + 5) * residual_phase * 0.7f) +
                      0.01f * (float)(i % 5);
        hidden[i] = -0.27f * cosf((float)(i + 3) * hidden_phase) +
                    0.19f * sinf((float)(i + 1) * hidden_phase * 0.6f) -
                    0.012f * (float)((i * 7) % 9);
    }
    for (uint32_t i = size; i < buffer_size; ++i) {
        residual[i] = tail_bias + 0.03f * (float)(i - size);
        hidden[i] = -tail_bias - 0.02f * (float)(i - size);
    }
}

/* tests/add_test_common.h:53-59: out = round_bf16(hidden + residual). */
void or_residual_add(const float* hidden, const float* residual, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_round_to_bf16(hidden[i] + residual[i]);
}

/* tests/swiglu_test_common.h:45-53 with tests/test_helpers.h:177-179:
 * out = round_bf16(up * (gate * (1 / (1 + exp(-gate))))), float exp. */
void or_swiglu(const float* gate, const float* up, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float sig = 1.0f / (1.0f + expf(-gate[i]));
        out[i] = or_round_to_bf16(up[i] * (gate[i] * sig));
    }
}

/* src/sampler.cpp:71-82: first index whose value exceeds every earlier one,
 * starting from -FLT_MAX; UINT32_MAX if none. */
uint32_t or_argmax(const float* logits, uint32_t n) {
    float best = -3.402823466e38f;
    uint32_t idx = 0xffffffffu;
    for (uint32_t i = 0; i < n; ++i)
        if (logits[i] > best) {
            best = logits[i];
            idx = i;
        }
    return idx;
}


/* ------------------------------------------------------------ sampling */

typedef struct {
    float x;
    uint32_t i;
} or_scored;

/* Larger value first; equal values by smaller index. */
static int or_scored_cmp(const void* a, const void* b) {
    const or_scored* p = (const or_scored*)a;
    const or_scored* q = (const or_scored*)b;
    if (p->x != q->x) return p->x > q->x ? -1 : 1;
    return p->i < q->i ? -1 : (p->i > q->i);
}

/* src/sampler.cpp:18-67 with the uniform draw u in [0, 1) given (the
 * reference takes it from a time-seeded mt19937, :58-60):
 *   greedy (or_argmax) when |T - 0| < 1e-3 or top_k == 1 (:20-22);
 *   x_i = logit_i / T (:24-27); the top k = min(top_k, n) of x (:29-32; a
 *   full sort here, larger first, equal values by index, where the reference
 *   quick-selects and keeps its own order among ties);
 *   p_i = expf((x_i - max) / T), summed in that order, divided by the sum
 *   (:33-44); sorted descending (:45-49, already so);
 *   kept = 1 + the first index whose running sum exceeds top_p (:50-57), or
 *   all k when none does (the reference then reads one entry past its top k);
 *   coin = u * the kept sum; the first kept index whose running sum exceeds
 *   the coin, else the last kept one (:58-67).
 * Optional outputs: order[k] (token ids, sorted), probs[k], kept. */
uint32_t or_sample_topk_topp(const float* logits, uint32_t n, float temperature, uint32_t top_k,
                             float top_p, float u, uint32_t* order, float* probs,
                             uint32_t* kept_out) {
    if (fabsf(temperature - 0.0f) < 1e-3f || top_k == 1) {
        if (kept_out) *kept_out = 1;
        return or_argmax(logits, n);
    }
    const uint32_t k = top_k < n ? top_k : n;
    or_scored* t = (or_scored*)malloc(sizeof(or_scored) * n);
    float* p = (float*)malloc(sizeof(float) * k);
    for (uint32_t i = 0; i < n; ++i) {
        t[i].x = logits[i] / temperature;
        t[i].i = i;
    }
    qsort(t, n, sizeof(or_scored), or_scored_cmp);
    const float max_x = t[0].x;
    float sum = 0.0f;
    for (uint32_t i = 0; i < k; ++i) {
        p[i] = expf((t[i].x - max_x) / temperature);
        sum += p[i];
    }
    for (uint32_t i = 0; i < k; ++i) p[i] /= sum;
    float acc = 0.0f;
    uint32_t j = 0;
    for (; j < k; ++j) {
        acc += p[j];
        if (acc > top_p) break;
    }
    const uint32_t kept = j < k ? j + 1 : k;
    const float coin = u * acc;
    uint32_t pick = t[kept - 1].i;
    float run = 0.0f;
    for (uint32_t i = 0; i < kept; ++i) {
        run += p[i];
        if (run > coin) {
            pick = t[i].i;
            break;
        }
    }
    if (order)
        for (uint32_t i = 0; i < k; ++i) order[i] = t[i].i;
    if (probs) memcpy(probs, p, sizeof(float) * k);
    if (kept_out) *kept_out = kept;
    free(t);
    free(p);
    return pick;
}

/* The draw the model harness uses for position pos: the SplitMix64 output
 * function (Steele, Lea, Flood 2014) of seed + (pos + 1) * 0x9E3779B97F4A7C15,
 * top 24 bits scaled to [0, 1). */
float or_sample_coin(uint64_t seed, uint32_t pos) {
    uint64_t z = seed + (uint64_t)(pos + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(uint32_t)(z >> 40) * 0x1p-24f;
}
