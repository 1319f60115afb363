/*
 * Seeded synthetic bf16 inputs, host side (C, OpenMP).
 *
 * Bit-for-bit the generator specified in toyinfer_amd/synth.py: SplitMix64
 * words, Box-Muller with ln and sin/cos built from +, -, *, / only, float64
 * -> float32 -> bf16, both roundings to nearest even.  Every operation is
 * written in the same order as the numpy specification and the file is
 * compiled with -ffp-contract=off, so no product and sum are fused.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const uint64_t kGamma = 0x9E3779B97F4A7C15ull;
static const double kLn2 = 0.6931471805599453;
static const double kHalfPi = 1.5707963267948966;
static const double kTwo53 = 1.0 / 9007199254740992.0; /* 2^-53 */

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t word(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGamma); }

static double fact(int k) {
    double out = 1.0;
    for (int i = 2; i <= k; ++i) out *= (double)i;
    return out;
}

static double g_inv_fact[18];
static double g_inv_odd[13];
static int g_init = 0;

static void init_tables(void) {
    if (g_init) return;
    for (int k = 0; k <= 17; ++k) g_inv_fact[k] = 1.0 / fact(k);
    for (int k = 0; k <= 12; ++k) g_inv_odd[k] = 1.0 / (double)(2 * k + 1);
    g_init = 1;
}

static inline double ln_exact_ops(double u) {
    int e;
    double m = frexp(u, &e);
    if (m < 0.7071067811865476) {
        m = m * 2.0;
        e = e - 1;
    }
    const double z = (m - 1.0) / (m + 1.0);
    const double z2 = z * z;
    double acc = 1.0 / 25.0;
    for (int k = 11; k >= 0; --k) acc = acc * z2 + g_inv_odd[k];
    return (double)e * kLn2 + 2.0 * z * acc;
}

static inline void sincos_2pi(double u, double* sn, double* cs) {
    const double t = u * 4.0;
    const double quad = floor(t);
    const double f = t - quad;
    const int flip = f > 0.5;
    const double y = flip ? 1.0 - f : f;
    const double x = y * kHalfPi;
    const double x2 = x * x;
    double s = g_inv_fact[17];
    for (int k = 15; k >= 1; k -= 2) s = s * (-x2) + g_inv_fact[k];
    s = s * x;
    double c = g_inv_fact[16];
    for (int k = 14; k >= 0; k -= 2) c = c * (-x2) + g_inv_fact[k];
    if (flip) {
        const double tmp = s;
        s = c;
        c = tmp;
    }
    switch (((int64_t)quad) & 3) {
        case 0: *sn = s; *cs = c; break;
        case 1: *sn = c; *cs = -s; break;
        case 2: *sn = -s; *cs = -c; break;
        default: *sn = -c; *cs = s; break;
    }
}

static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* n normals of stream `key` as bf16 bits. */
void ti_synth_normal_bf16(uint64_t key, int64_t n, uint16_t* out) {
    init_tables();
    const int64_t npairs = (n + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < npairs; ++j) {
        const uint64_t w1 = word(key, 2 * (uint64_t)j), w2 = word(key, 2 * (uint64_t)j + 1);
        const double u1 = ((double)(w1 >> 11) + 1.0) * kTwo53;
        const double u2 = (double)(w2 >> 11) * kTwo53;
        const double r = sqrt(-2.0 * ln_exact_ops(u1));
        double sn, cs;
        sincos_2pi(u2, &sn, &cs);
        out[2 * j] = f32_to_bf16((float)(r * cs));
        if (2 * j + 1 < n) out[2 * j + 1] = f32_to_bf16((float)(r * sn));
    }
}

/* n uniforms lo + (hi - lo) * u, u in [0, 1), as bf16 bits. */
void ti_synth_uniform_bf16(uint64_t key, int64_t n, double lo, double hi, uint16_t* out) {
    const double span = hi - lo;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const double u = (double)(word(key, (uint64_t)i) >> 11) * kTwo53;
        out[i] = f32_to_bf16((float)(lo + span * u));
    }
}

static inline float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* bf16(float(in[i]) * scale): one float32 product, rounded to nearest even. */
void ti_synth_scale_bf16(const uint16_t* in, int64_t n, float scale, uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(bf16_to_f32(in[i]) * scale);
}
