// Drop-in check of include/kernel_warpper.h: the reference's own call
// patterns (template instantiations, the prefill head_dim dispatch of
// src/transformer.cpp:20-39, the decode wrapper contract of
// tests/test_attention_bf16.cu:28-75 with dirty output buffers, and the graph
// replay with a pinned host position of tests/test_cuda_graph_pos.cu:118-200)
// compiled as ordinary C++ against the HIP library, with every result checked
// against the CPU oracle (oracle/liboracle.so, test infrastructure).
//
// Bar: bf16 outputs within max-abs 2e-2 and mean-abs 2e-3 of the oracle;
// decode score/O_buffer with the reference tests' nearly_equal tolerances
// (score 5e-3, O_buffer 5e-2).  Prints one line per case; exit status 0 iff
// every case passes.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "kernel_warpper.h"

extern "C" {
uint16_t or_f32_to_bf16(float f);
float or_bf16_to_f32(uint16_t h);
void or_make_flash_case(uint32_t hq, uint32_t hkv, uint32_t d_head, uint32_t seq, float q_phase,
                        float kv_phase, float q_scale, float k_scale, float v_scale, float* q,
                        float* k, float* v);
void or_make_causal_focus_case(float* q, float* k, float* v);
void or_make_attention_case(uint32_t hq, uint32_t hkv, uint32_t d_head, uint32_t max_seq_len,
                            float q_phase, float kv_phase, float* q, float* k, float* v);
void or_flash_reference_f32(const float* qf, const float* kf, const float* vf, float* out,
                            uint32_t hq, uint32_t hkv, uint32_t d_head, uint32_t seq,
                            const uint32_t* rows, uint32_t n_rows, int nthreads);
void or_decode_attention_f32(const float* qf, const float* kf, const float* vf, float* score_out,
                             float* o_buffer_out, uint16_t* o_out, uint32_t hq, uint32_t hkv,
                             uint32_t d_head, uint32_t pos, uint32_t max_seq_len);
void or_inv_freq(float* inv_freq, int d_head, float theta);
void or_qk_norm_rope(float* x, const float* gamma, const float* inv_freq, uint32_t num_tokens,
                     uint32_t num_heads, uint32_t d_head, float eps);
void or_multi_rmsnorm(const float* x, const float* w, float* out, uint32_t num_rows,
                      uint32_t d_head, float eps);
void or_rope(float* qk, const float* inv_freq, uint32_t num_tokens, uint32_t num_heads,
             uint32_t d_head, uint32_t pos0);
void or_make_gemv_case(uint32_t M, uint32_t N, float x_phase, float w_phase, float* x, float* w);
void or_gemv(const float* w, const float* x, float* y, uint32_t tokens, uint32_t M, uint32_t N,
             int nthreads);
}

namespace {

using toyinfer::bf16;

int g_failures = 0;

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "HIP error %s: %s\n", what, hipGetErrorString(e));
        std::exit(2);
    }
}

template <typename T>
struct Dev {
    T* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { hip_ok(hipMalloc(&p, sizeof(T) * (n ? n : 1)), "malloc"); }
    ~Dev() { (void)hipFree(p); }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
    void put(const std::vector<T>& h) {
        hip_ok(hipMemcpy(p, h.data(), sizeof(T) * n, hipMemcpyHostToDevice), "h2d");
    }
    std::vector<T> get() const {
        std::vector<T> h(n);
        hip_ok(hipMemcpy(h.data(), p, sizeof(T) * n, hipMemcpyDeviceToHost), "d2h");
        return h;
    }
};

// bf16 <-> float through the oracle's IEEE round-to-nearest-even.
std::vector<uint16_t> to_bits(const std::vector<float>& x) {
    std::vector<uint16_t> b(x.size());
    for (size_t i = 0; i < x.size(); ++i) b[i] = or_f32_to_bf16(x[i]);
    return b;
}
std::vector<float> from_bits(const std::vector<uint16_t>& b) {
    std::vector<float> x(b.size());
    for (size_t i = 0; i < b.size(); ++i) x[i] = or_bf16_to_f32(b[i]);
    return x;
}
std::vector<float> round_bf16(const std::vector<float>& x) { return from_bits(to_bits(x)); }

std::vector<uint16_t> get_bits(const Dev<bf16>& d) {
    std::vector<bf16> h = d.get();
    std::vector<uint16_t> b(h.size());
    std::memcpy(b.data(), h.data(), h.size() * 2);
    return b;
}
void put_bits(Dev<bf16>& d, const std::vector<uint16_t>& b) {
    std::vector<bf16> h(b.size());
    std::memcpy(h.data(), b.data(), b.size() * 2);
    d.put(h);
}

void report(bool ok, const std::string& label, const std::string& detail) {
    std::printf("[%s] %s %s\n", ok ? "PASS" : "FAIL", label.c_str(), detail.c_str());
    std::fflush(stdout);
    if (!ok) ++g_failures;
}

// max-abs 2e-2, mean-abs 2e-3 on bf16 outputs.
void check_bar(const std::vector<float>& got, const std::vector<float>& exp,
               const std::string& label) {
    double mx = 0, sum = 0;
    bool finite = got.size() == exp.size();
    for (size_t i = 0; finite && i < got.size(); ++i) {
        if (!std::isfinite(got[i])) finite = false;
        const double d = std::fabs((double)got[i] - exp[i]);
        mx = d > mx ? d : mx;
        sum += d;
    }
    const double mean = got.empty() ? 0 : sum / got.size();
    char buf[96];
    std::snprintf(buf, sizeof buf, "max-abs %.3g mean-abs %.3g", mx, mean);
    report(finite && mx <= 2e-2 && mean <= 2e-3, label, buf);
}

// tests/test_helpers.h nearly_equal: |a-b| <= atol + rtol*|b|.
void check_close(const std::vector<float>& got, const std::vector<float>& exp, float atol,
                 float rtol, const std::string& label) {
    size_t bad = got.size() == exp.size() ? got.size() : 0;
    for (size_t i = 0; i < got.size() && bad == got.size(); ++i)
        if (!(std::fabs(got[i] - exp[i]) <= atol + rtol * std::fabs(exp[i]))) bad = i;
    report(bad == got.size(), label,
           bad == got.size() ? "" : "first mismatch at " + std::to_string(bad));
}

// ---------------------------------------------------------------- prefill

// The dispatch of src/transformer.cpp:20-39 written against the drop-in header.
void launch_prefill(const bf16* q, const bf16* k, const bf16* v, bf16* o, uint32_t hq, uint32_t hkv,
                    uint32_t head_dim, uint32_t tokens) {
    if (head_dim == 64) {
        toyinfer::flash_attention_v1_bf16<32, 4, 64>(q, k, v, o, hq, hkv, head_dim, tokens);
        return;
    }
    if (head_dim == 128) {
        toyinfer::flash_attention_v1_bf16<32, 4, 128>(q, k, v, o, hq, hkv, head_dim, tokens);
        return;
    }
    std::fprintf(stderr, "unsupported head_dim\n");
    std::exit(2);
}

// Every instantiation the reference builds (src/prefill.cu:433-452).
void launch_instantiation(int which, const bf16* q, const bf16* k, const bf16* v, bf16* o,
                          uint32_t hq, uint32_t hkv, uint32_t d, uint32_t s) {
    switch (which) {
        case 0: toyinfer::flash_attention_v1_bf16<32, 2, 64>(q, k, v, o, hq, hkv, d, s); break;
        case 1: toyinfer::flash_attention_v1_bf16<32, 4, 64>(q, k, v, o, hq, hkv, d, s); break;
        case 2: toyinfer::flash_attention_v1_bf16<32, 4, 128>(q, k, v, o, hq, hkv, d, s); break;
        default: toyinfer::flash_attention_v1_bf16<64, 4, 128>(q, k, v, o, hq, hkv, d, s); break;
    }
}

void prefill_case(const std::string& label, uint32_t hq, uint32_t hkv, uint32_t d, uint32_t s,
                  std::vector<float> q, std::vector<float> k, std::vector<float> v) {
    const auto qb = to_bits(q), kb = to_bits(k), vb = to_bits(v);
    const auto qf = from_bits(qb), kf = from_bits(kb), vf = from_bits(vb);
    std::vector<float> ref(qb.size());
    or_flash_reference_f32(qf.data(), kf.data(), vf.data(), ref.data(), hq, hkv, d, s, nullptr, 0, 0);
    const auto exp = round_bf16(ref);
    Dev<bf16> dq(qb.size()), dk(kb.size()), dv(vb.size()), dout(qb.size());
    put_bits(dq, qb);
    put_bits(dk, kb);
    put_bits(dv, vb);
    launch_prefill(dq.p, dk.p, dv.p, dout.p, hq, hkv, d, s);
    hip_ok(hipDeviceSynchronize(), "sync");
    check_bar(from_bits(get_bits(dout)), exp, "prefill " + label + " (transformer dispatch)");
    for (int which = d == 64 ? 0 : 2; which < (d == 64 ? 2 : 4); ++which) {
        put_bits(dout, std::vector<uint16_t>(qb.size(), 0x7fc0));  // NaN: every row must be written
        launch_instantiation(which, dq.p, dk.p, dv.p, dout.p, hq, hkv, d, s);
        hip_ok(hipDeviceSynchronize(), "sync");
        check_bar(from_bits(get_bits(dout)), exp,
                  "prefill " + label + " instantiation " + std::to_string(which));
    }
}

void prefill_cases() {
    struct C {
        const char* label;
        uint32_t hq, hkv, d, s;
        float qp, kvp, qs, ks, vs;
    };
    // tests/test_flash_attention_v1_bf16.cu:113-131
    const C cases[] = {{"seq1_gqa", 2, 1, 64, 1, 0.07f, 0.03f, 1, 1, 1},
                       {"exact_kv_tile", 4, 4, 64, 32, 0.05f, 0.021f, 1, 1, 1},
                       {"gqa_tail_tiles", 8, 2, 128, 37, 0.033f, 0.017f, 1, 1, 1},
                       {"multi_kv_tile", 6, 3, 128, 65, 0.028f, 0.019f, 1, 1, 1},
                       {"large_magnitude", 4, 2, 64, 19, 0.061f, 0.027f, 12, 10, 1.7f}};
    for (const C& c : cases) {
        std::vector<float> q((size_t)c.s * c.hq * c.d), k((size_t)c.s * c.hkv * c.d), v(k.size());
        or_make_flash_case(c.hq, c.hkv, c.d, c.s, c.qp, c.kvp, c.qs, c.ks, c.vs, q.data(), k.data(),
                           v.data());
        prefill_case(c.label, c.hq, c.hkv, c.d, c.s, q, k, v);
    }
    std::vector<float> q(6 * 2 * 64), k(6 * 64), v(6 * 64);
    or_make_causal_focus_case(q.data(), k.data(), v.data());
    prefill_case("causal_focus", 2, 1, 64, 6, q, k, v);
}

// ----------------------------------------------------------------- decode

struct DecodeCase {
    const char* label;
    uint32_t hq, hkv, d, pos, msl;
    float qp, kvp;
};

struct DecodeData {
    std::vector<uint16_t> q, k, v;
    std::vector<float> score, obuf, o;
};

DecodeData decode_data(const DecodeCase& c, uint32_t pos) {
    std::vector<float> q((size_t)c.hq * c.d), k((size_t)c.msl * c.hkv * c.d), v(k.size());
    or_make_attention_case(c.hq, c.hkv, c.d, c.msl, c.qp, c.kvp, q.data(), k.data(), v.data());
    DecodeData r{to_bits(q), to_bits(k), to_bits(v), {}, {}, {}};
    const auto qf = from_bits(r.q), kf = from_bits(r.k), vf = from_bits(r.v);
    r.score.resize((size_t)c.hq * c.msl);
    r.obuf.resize((size_t)c.hq * c.d);
    std::vector<uint16_t> ob(r.obuf.size());
    or_decode_attention_f32(qf.data(), kf.data(), vf.data(), r.score.data(), r.obuf.data(), ob.data(),
                            c.hq, c.hkv, c.d, pos, c.msl);
    r.o = from_bits(ob);
    return r;
}

void check_decode(const std::string& label, const DecodeData& r, const Dev<float>& score,
                  const Dev<float>& obuf, const Dev<bf16>& o) {
    check_close(score.get(), r.score, 5e-3f, 5e-3f, label + " score");
    check_close(obuf.get(), r.obuf, 5e-2f, 5e-2f, label + " o_buffer");
    check_bar(from_bits(get_bits(o)), r.o, label + " output");
}

void decode_cases() {
    // tests/test_attention_bf16.cu:84-91
    const DecodeCase cases[] = {{"pos0_gqa", 2, 1, 64, 0, 5, 0.07f, 0.03f},
                                {"full_kv", 4, 4, 64, 6, 7, 0.05f, 0.025f},
                                {"tiled_seq", 8, 2, 128, 37, 40, 0.03f, 0.017f},
                                {"qwen3_8b_long", 32, 8, 128, 3000, 3072, 0.011f, 0.007f}};
    for (const DecodeCase& c : cases) {
        const DecodeData r = decode_data(c, c.pos);
        Dev<bf16> q(r.q.size()), k(r.k.size()), v(r.v.size()), o((size_t)c.hq * c.d);
        Dev<float> score((size_t)c.hq * c.msl), obuf((size_t)c.hq * c.d);
        put_bits(q, r.q);
        put_bits(k, r.k);
        put_bits(v, r.v);
        score.put(std::vector<float>(score.n, 7.0f));  // dirty, as the reference test leaves them
        obuf.put(std::vector<float>(obuf.n, -3.0f));
        put_bits(o, std::vector<uint16_t>(o.n, 0x4040));
        toyinfer::attention_bf16<256, 32>(q.p, k.p, v.p, score.p, obuf.p, o.p, c.hq, c.hkv, c.d,
                                          c.pos, c.msl);
        hip_ok(hipDeviceSynchronize(), "sync");
        check_decode(std::string("decode ") + c.label + " attention_bf16", r, score, obuf, o);
    }

    // Graph replay: capture an H2D copy of a pinned host position and the
    // graph wrapper once, then replay with the host position changed.
    const DecodeCase c = {"graph_replay", 8, 2, 128, 0, 40, 0.03f, 0.017f};
    const DecodeData r0 = decode_data(c, 0);
    Dev<bf16> q(r0.q.size()), k(r0.k.size()), v(r0.v.size()), o((size_t)c.hq * c.d);
    Dev<float> score((size_t)c.hq * c.msl), obuf((size_t)c.hq * c.d);
    put_bits(q, r0.q);
    put_bits(k, r0.k);
    put_bits(v, r0.v);
    score.put(std::vector<float>(score.n, 7.0f));
    uint32_t* pos_h = nullptr;
    Dev<uint32_t> pos_d(1);
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hip_ok(hipHostMalloc(reinterpret_cast<void**>(&pos_h), sizeof(uint32_t), hipHostMallocDefault),
           "host malloc");
    hip_ok(hipStreamCreate(&stream), "stream");
    *pos_h = 0;
    hip_ok(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal), "begin capture");
    hip_ok(hipMemcpyAsync(pos_d.p, pos_h, sizeof(uint32_t), hipMemcpyHostToDevice, stream), "pos");
    toyinfer::attention_bf16_graph<256, 32>(q.p, k.p, v.p, score.p, obuf.p, o.p, c.hq, c.hkv, c.d,
                                            pos_d.p, c.msl, stream);
    hip_ok(hipStreamEndCapture(stream, &graph), "end capture");
    hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate");
    for (uint32_t pos : {0u, 37u, 3u, 39u, 37u}) {
        *pos_h = pos;
        hip_ok(hipGraphLaunch(exec, stream), "launch");
        hip_ok(hipStreamSynchronize(stream), "sync");
        check_decode("decode graph replay pos " + std::to_string(pos), decode_data(c, pos), score,
                     obuf, o);
    }
    hip_ok(hipGraphExecDestroy(exec), "exec destroy");
    hip_ok(hipGraphDestroy(graph), "graph destroy");
    hip_ok(hipStreamDestroy(stream), "stream destroy");
    hip_ok(hipHostFree(pos_h), "host free");
}

// ------------------------------------------------ QK-norm, RoPE, inv_freq

void prologue_cases() {
    const uint32_t t = 70, hq = 8, hkv = 2, d = 128;
    const float theta = 1e6f, eps = 1e-6f;
    Dev<float> inv(d / 2);
    toyinfer::precompute_freq_f32(inv.p, d, theta);
    hip_ok(hipDeviceSynchronize(), "sync");
    std::vector<float> inv_ref(d / 2);
    or_inv_freq(inv_ref.data(), d, theta);
    check_close(inv.get(), inv_ref, 1e-6f, 1e-5f, "precompute_freq_f32");

    // Prefill prologue as src/transformer.cpp:380-391 sequences it, in place.
    std::vector<float> x((size_t)t * hq * d), gamma(d);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.37f * (float)i) * 1.7f + 0.05f;
    for (uint32_t i = 0; i < d; ++i) gamma[i] = 0.9f + 0.2f * (float)((i * 37) % 101) / 100.0f;
    const auto xb = to_bits(x), gb = to_bits(gamma);
    std::vector<float> ref = from_bits(xb);
    or_qk_norm_rope(ref.data(), from_bits(gb).data(), inv_ref.data(), t, hq, d, eps);
    Dev<bf16> dx(xb.size()), dg(d), dy(xb.size());
    put_bits(dx, xb);
    put_bits(dg, gb);
    toyinfer::batch_multi_rmsnorm_bf16(dx.p, dg.p, dx.p, eps, t, hq, d);
    toyinfer::batch_rope_bf16(dx.p, inv.p, t, hq, d);
    hip_ok(hipDeviceSynchronize(), "sync");
    check_bar(from_bits(get_bits(dx)), ref, "batch_multi_rmsnorm_bf16 + batch_rope_bf16 in place");
    put_bits(dx, xb);
    toyinfer::qk_norm_rope_bf16(dx.p, dg.p, dy.p, inv.p, eps, t, hq, d);
    hip_ok(hipDeviceSynchronize(), "sync");
    check_bar(from_bits(get_bits(dy)), ref, "qk_norm_rope_bf16");

    // Fused prologue + attention against norm -> rope -> attention on the CPU.
    std::vector<float> k((size_t)t * hkv * d), v(k.size());
    for (size_t i = 0; i < k.size(); ++i) {
        k[i] = std::cos(0.23f * (float)i) * 1.3f;
        v[i] = std::sin(0.11f * (float)i + 0.5f);
    }
    const auto kb = to_bits(k), vb = to_bits(v);
    std::vector<float> kref = from_bits(kb);
    or_qk_norm_rope(kref.data(), from_bits(gb).data(), inv_ref.data(), t, hkv, d, eps);
    std::vector<float> oref(x.size());
    const auto vf = from_bits(vb);
    or_flash_reference_f32(ref.data(), kref.data(), vf.data(), oref.data(), hq, hkv, d, t, nullptr,
                           0, 0);
    Dev<float> table((size_t)t * d);
    toyinfer::rope_cos_sin_f32(table.p, inv.p, t, d);
    Dev<bf16> dk(kb.size()), dv(vb.size()), dko(kb.size()), dout(xb.size());
    put_bits(dx, xb);
    put_bits(dk, kb);
    put_bits(dv, vb);
    toyinfer::prefill_qknorm_rope_attention_bf16(dx.p, dk.p, dv.p, dout.p, dko.p, dg.p, dg.p, table.p,
                                                 eps, hq, hkv, d, t);
    hip_ok(hipDeviceSynchronize(), "sync");
    check_bar(from_bits(get_bits(dko)), kref, "prefill_qknorm_rope_attention_bf16 K_out");
    check_bar(from_bits(get_bits(dout)), round_bf16(oref), "prefill_qknorm_rope_attention_bf16 O");
}

// ------------------------------------------------------ decode-step pre-pass

void decode_step_cases() {
    const uint32_t hq = 32, hkv = 8, d = 128, msl = 24, pos = 11;
    const float eps = 1e-6f;
    Dev<float> inv(d / 2);
    toyinfer::precompute_freq_f32(inv.p, d, 1e6f);
    hip_ok(hipDeviceSynchronize(), "sync");
    const std::vector<float> inv_h = inv.get();
    std::vector<float> q((size_t)hq * d), k((size_t)hkv * d), v(k.size()), gq(d), gk(d);
    for (size_t i = 0; i < q.size(); ++i) q[i] = std::sin(0.29f * (float)i) * 1.5f;
    for (size_t i = 0; i < k.size(); ++i) {
        k[i] = std::cos(0.17f * (float)i) * 1.2f;
        v[i] = std::sin(0.05f * (float)i + 1.0f);
    }
    for (uint32_t i = 0; i < d; ++i) {
        gq[i] = 0.9f + 0.2f * (float)((i * 13) % 97) / 96.0f;
        gk[i] = 1.1f - 0.2f * (float)((i * 7) % 89) / 88.0f;
    }
    const auto qb = to_bits(q), kb = to_bits(k), vb = to_bits(v), gqb = to_bits(gq), gkb = to_bits(gk);
    // Expected: per-head RMSNorm -> bf16 -> RoPE at pos -> bf16.
    std::vector<float> qe(q.size()), ke(k.size());
    or_multi_rmsnorm(from_bits(qb).data(), from_bits(gqb).data(), qe.data(), hq, d, eps);
    or_multi_rmsnorm(from_bits(kb).data(), from_bits(gkb).data(), ke.data(), hkv, d, eps);
    or_rope(qe.data(), inv_h.data(), 1, hq, d, pos);
    or_rope(ke.data(), inv_h.data(), 1, hkv, d, pos);

    Dev<uint32_t> pos_d(1);
    pos_d.put({pos});
    Dev<bf16> dq(qb.size()), dk(kb.size()), dv(vb.size()), dgq(d), dgk(d);
    Dev<bf16> kc((size_t)msl * hkv * d), vc((size_t)msl * hkv * d);
    put_bits(dgq, gqb);
    put_bits(dgk, gkb);
    auto check_step = [&](const std::string& label, const std::vector<uint16_t>& q_got) {
        const auto kcb = get_bits(kc), vcb = get_bits(vc);
        const size_t row = (size_t)pos * hkv * d;
        check_close(from_bits(q_got), qe, 2e-2f, 2e-2f, label + " q");
        check_close(from_bits(std::vector<uint16_t>(kcb.begin() + row, kcb.begin() + row + kb.size())),
                    ke, 2e-2f, 2e-2f, label + " k cache row");
        report(std::equal(vb.begin(), vb.end(), vcb.begin() + row), label + " v cache row", "");
    };

    // The reference's decode step, src/transformer.cpp:535-552, on one stream.
    hipStream_t stream;
    hip_ok(hipStreamCreate(&stream), "stream");
    put_bits(dq, qb);
    put_bits(dk, kb);
    put_bits(dv, vb);
    toyinfer::multi_rmsnorm_bf16(dq.p, dgq.p, dq.p, eps, hq, d, stream);
    toyinfer::multi_rmsnorm_bf16(dk.p, dgk.p, dk.p, eps, hkv, d, stream);
    toyinfer::rope_bf16_graph(dq.p, inv.p, pos_d.p, hq, d, stream);
    toyinfer::rope_bf16_graph(dk.p, inv.p, pos_d.p, hkv, d, stream);
    toyinfer::write_kv_cache_bf16<256>(dk.p, kc.p, pos_d.p, hkv * d, stream);
    toyinfer::write_kv_cache_bf16<256>(dv.p, vc.p, pos_d.p, hkv * d, stream);
    hip_ok(hipStreamSynchronize(stream), "sync");
    check_step("decode step (six reference ops)", get_bits(dq));

    // The same step fused into one launch.
    put_bits(dq, qb);
    put_bits(dk, kb);
    hip_ok(hipMemset(kc.p, 0, kc.n * 2), "memset");
    hip_ok(hipMemset(vc.p, 0, vc.n * 2), "memset");
    toyinfer::decode_qkv_prologue_bf16(dq.p, dk.p, dv.p, dgq.p, dgk.p, inv.p, pos_d.p, msl, eps,
                                       dq.p, kc.p, vc.p, hq, hkv, d, stream);
    hip_ok(hipStreamSynchronize(stream), "sync");
    check_step("decode_qkv_prologue_bf16", get_bits(dq));
    hip_ok(hipStreamDestroy(stream), "stream destroy");
}

// The projections as src/transformer.cpp calls them: gemv_proj_bf16<256> for
// the decode q/k/v projections (:521-533), gemv_proj_bf162float<256> for the
// lm-head (:630), batch_gemv_proj_bf16<256> for prefill (:370-378), against
// the oracle's float sums at the reference tests' bar (8e-2 / 5e-2).
void projection_cases() {
    hipStream_t stream;
    hip_ok(hipStreamCreate(&stream), "stream");
    struct Shape {
        uint32_t tokens, M, N;
    };
    for (const Shape sh : {Shape{1, 1024, 4096}, Shape{1, 300, 514}, Shape{3, 96, 256},
                           Shape{37, 200, 256}, Shape{300, 1000, 1024}}) {
        std::vector<float> x1, w((size_t)sh.M * sh.N), x((size_t)sh.tokens * sh.N);
        x1.resize(sh.N);
        or_make_gemv_case(sh.M, sh.N, 0.05f, 0.004f, x1.data(), w.data());
        for (uint32_t t = 0; t < sh.tokens; ++t)
            for (uint32_t c = 0; c < sh.N; ++c)
                x[(size_t)t * sh.N + c] = x1[c] * (1.0f - 0.01f * (float)t) + 0.001f * (float)(t % 5);
        const auto wb = to_bits(w), xb = to_bits(x);
        std::vector<float> exp((size_t)sh.tokens * sh.M);
        or_gemv(from_bits(wb).data(), from_bits(xb).data(), exp.data(), sh.tokens, sh.M, sh.N, 8);
        Dev<bf16> dw(wb.size()), dx(xb.size()), dy(exp.size());
        put_bits(dw, wb);
        put_bits(dx, xb);
        const std::string shape = std::to_string(sh.tokens) + "x" + std::to_string(sh.M) + "x" +
                                  std::to_string(sh.N);
        if (sh.tokens == 1) {
            toyinfer::gemv_proj_bf16<256>(dw.p, dx.p, dy.p, sh.M, sh.N, stream);
            Dev<float> df(sh.M);
            toyinfer::gemv_proj_bf162float<256>(dw.p, dx.p, df.p, sh.M, sh.N, stream);
            hip_ok(hipStreamSynchronize(stream), "sync");
            check_close(df.get(), exp, 5e-2f, 5e-2f, "gemv_proj_bf162float " + shape);
            check_close(from_bits(get_bits(dy)), round_bf16(exp), 8e-2f, 8e-2f,
                        "gemv_proj_bf16 " + shape);
        } else {
            toyinfer::batch_gemv_proj_bf16<256>(dw.p, dx.p, dy.p, sh.tokens, sh.M, sh.N, stream);
            hip_ok(hipStreamSynchronize(stream), "sync");
            check_close(from_bits(get_bits(dy)), round_bf16(exp), 8e-2f, 8e-2f,
                        "batch_gemv_proj_bf16 " + shape);
        }
    }
    hip_ok(hipStreamDestroy(stream), "stream destroy");
}

// The decoder-layer ops as src/transformer.cpp calls them around attention
// (:500-628 decode, :355-470 prefill), against the oracle at the reference
// tests' 2e-2 bar; the rmsnorm sum against the float sum of squares.
void layer_op_cases() {
    hipStream_t stream;
    hip_ok(hipStreamCreate(&stream), "stream");
    const uint32_t T = 3, H = 1024, F = 3072, V = 64;
    std::vector<float> h((size_t)T * H), w(H), g((size_t)T * F), u((size_t)T * F), e((size_t)V * H);
    for (size_t i = 0; i < h.size(); ++i) h[i] = std::sin(0.013f * (float)i) * 1.3f;
    for (uint32_t i = 0; i < H; ++i) w[i] = 0.8f + 0.4f * (float)((i * 7) % 13) / 12.0f;
    for (size_t i = 0; i < g.size(); ++i) {
        g[i] = std::cos(0.007f * (float)i) * 2.5f;
        u[i] = std::sin(0.011f * (float)i + 0.3f);
    }
    for (size_t i = 0; i < e.size(); ++i) e[i] = std::cos(0.003f * (float)i);
    const auto hb = to_bits(h), wb = to_bits(w), gb = to_bits(g), ub = to_bits(u), eb = to_bits(e);
    Dev<bf16> dh(hb.size()), dw(wb.size()), dy(hb.size()), dg(gb.size()), du(ub.size()),
        di(gb.size()), de(eb.size()), dx((size_t)T * H);
    Dev<float> dsum(T);
    put_bits(dh, hb);
    put_bits(dw, wb);
    put_bits(dg, gb);
    put_bits(du, ub);
    put_bits(de, eb);
    toyinfer::batch_rmsnorm_bf16<256>(dh.p, dw.p, dy.p, dsum.p, 1e-6f, T, H, stream);
    toyinfer::batch_swiglu_bf16x2<256>(dg.p, du.p, di.p, T, F, stream);
    hip_ok(hipStreamSynchronize(stream), "sync");
    std::vector<float> exp(hb.size());
    or_multi_rmsnorm(from_bits(hb).data(), from_bits(wb).data(), exp.data(), T, H, 1e-6f);
    check_close(from_bits(get_bits(dy)), exp, 2e-2f, 2e-2f, "batch_rmsnorm_bf16");
    const auto sums = dsum.get();
    const auto hf = from_bits(hb);
    bool sum_ok = true;
    for (uint32_t t = 0; t < T; ++t) {
        double ss = 0;
        for (uint32_t i = 0; i < H; ++i) ss += (double)hf[(size_t)t * H + i] * hf[(size_t)t * H + i];
        sum_ok = sum_ok && std::fabs(sums[t] - ss) <= 5e-2 + 5e-3 * ss;
    }
    report(sum_ok, "batch_rmsnorm_bf16 sum", "");
    std::vector<float> sw(gb.size());
    const auto gf = from_bits(gb), uf = from_bits(ub);
    for (size_t i = 0; i < sw.size(); ++i)
        sw[i] = or_bf16_to_f32(or_f32_to_bf16(uf[i] * (gf[i] * (1.0f / (1.0f + std::exp(-gf[i]))))));
    check_close(from_bits(get_bits(di)), sw, 2e-2f, 2e-2f, "batch_swiglu_bf16x2");
    // residual add (in place) and the single-row forms
    toyinfer::residual_add_bf16<256>(dy.p, dh.p, H, stream);
    toyinfer::rmsnorm_bf16<256>(dh.p, dw.p, dx.p, dsum.p, 1e-6f, H, stream);
    toyinfer::swiglu_bf16x2<256>(dg.p, du.p, di.p, F, stream);
    Dev<uint32_t> ids(T);
    ids.put({5, 63, 0});
    toyinfer::gather_embedding_bf16<256>(de.p, ids.p, dy.p, T, H, stream);
    hip_ok(hipStreamSynchronize(stream), "sync");
    const auto yb = get_bits(dy);
    bool gather_ok = true;
    const uint32_t want[3] = {5, 63, 0};
    for (uint32_t t = 0; t < T; ++t)
        gather_ok = gather_ok && std::equal(eb.begin() + (size_t)want[t] * H,
                                            eb.begin() + (size_t)(want[t] + 1) * H,
                                            yb.begin() + (size_t)t * H);
    report(gather_ok, "gather_embedding_bf16", "rows copied bit for bit");
    hip_ok(hipStreamDestroy(stream), "stream destroy");
}

}  // namespace

int main() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        std::fprintf(stderr, "no HIP device\n");
        return 2;
    }
    prefill_cases();
    decode_cases();
    prologue_cases();
    decode_step_cases();
    projection_cases();
    layer_op_cases();
    std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "ALL PASS", g_failures);
    return g_failures ? 1 : 0;
}
