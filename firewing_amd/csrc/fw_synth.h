/*
 * Seeded synthetic workload for the sparse-MoE block: a counter-based integer
 * hash maps (seed, layer, tensor, element) to a 16-bit uniform, which indexes a
 * 65,536-entry bf16 inverse-normal table. The same bits come out on the host
 * and on the GPU, so the CPU can regenerate any expert slice without holding
 * the 155 GB resident 48-layer bank.
 *
 * This header is plain C99 so that both the HIP library (host and device code)
 * and the C oracle include the one definition of the workload. It defines the
 * inputs only; nothing here computes a result that is checked.
 *
 * The Zipf-shaped router popularity is realised inside the router's own
 * arithmetic (the reference router has no bias term, src/router.rs:220-240):
 * the input carries a constant feature x[H-1] = 1.0 and router row e holds
 * W[e][H-1] = bias(rank_l(e)), where rank_l is a seeded per-layer permutation.
 */
#ifndef FW_SYNTH_H
#define FW_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define FW_SYNTH_HD __host__ __device__ static inline
#else
#define FW_SYNTH_HD static inline
#endif

enum fw_synth_tensor {
    FW_SYNTH_ROUTER = 1,
    FW_SYNTH_GATE_UP = 2,
    FW_SYNTH_DOWN = 3,
    FW_SYNTH_SHARED_GATE = 4,
    FW_SYNTH_SHARED_UP = 5,
    FW_SYNTH_SHARED_DOWN = 6,
    FW_SYNTH_SHARED_EXPERT_GATE = 7,
    FW_SYNTH_HIDDEN = 8,
    FW_SYNTH_PERMUTATION = 9,
    FW_SYNTH_LM_HEAD = 10
};

/* Weight standard deviation for every synthetic weight tensor. */
#define FW_SYNTH_WEIGHT_SIGMA 0.02
/* Zipf exponent of expert popularity and the bias slope that realises it
 * (calibrated by tests/golden/zipf_calibration.py for H=2048, E=512, K=10;
 * the realised exponent is checked by tests/test_workload.py). */
#define FW_SYNTH_ZIPF_S 1.1
#define FW_SYNTH_ZIPF_BIAS_SLOPE 0.45

/* MurmurHash3's 64-bit finaliser: a bijective avalanche mix. */
FW_SYNTH_HD uint64_t fw_mix64(uint64_t z) {
    z ^= z >> 33;
    z *= 0xff51afd7ed558ccdULL;
    z ^= z >> 33;
    z *= 0xc4ceb9fe1a85ec53ULL;
    z ^= z >> 33;
    return z;
}

/* Stream key of one tensor of one layer. */
FW_SYNTH_HD uint64_t fw_synth_stream(uint64_t seed, uint32_t layer, uint32_t tensor) {
    uint64_t id = (((uint64_t)layer << 8) | (uint64_t)tensor) + 1ULL;
    return fw_mix64(seed ^ fw_mix64(id * 0x9E3779B97F4A7C15ULL));
}

/* 16-bit uniform for element `index` of a stream; one hash feeds four
 * consecutive elements. */
FW_SYNTH_HD uint32_t fw_synth_u16(uint64_t stream, uint64_t index) {
    uint64_t h = fw_mix64(stream + (index >> 2));
    return (uint32_t)(h >> (16u * (uint32_t)(index & 3u))) & 0xffffu;
}

/* bf16 round-to-nearest-even of an f32 bit pattern (same rule the reference
 * uses for every boundary, src/expert.rs:315-318). */
FW_SYNTH_HD uint16_t fw_synth_round_bf16(uint32_t bits) {
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

/* Host-only helpers (plain static functions: never called from device code). */
#include <math.h>
#include <string.h>

/* Acklam's rational approximation of the standard normal quantile, refined by
 * one Halley step on erfc: |error| < 1e-15 over (0, 1). */
static inline double fw_synth_normal_quantile(double p) {
    static const double a[6] = {-3.969683028665376e+01, 2.209460984245205e+02,
                                -2.759285104469687e+02, 1.383577518672690e+02,
                                -3.066479806614716e+01, 2.506628277459239e+00};
    static const double b[5] = {-5.447609879822406e+01, 1.615858368580409e+02,
                                -1.556989798598866e+02, 6.680131188771972e+01,
                                -1.328068155288572e+01};
    static const double c[6] = {-7.784894002430293e-03, -3.223964580411365e-01,
                                -2.400758277161838e+00, -2.549732539343734e+00,
                                4.374664141464968e+00, 2.938163982698783e+00};
    static const double d[4] = {7.784695709041462e-03, 3.224671290700398e-01,
                                2.445134137142996e+00, 3.754408661907416e+00};
    const double plow = 0.02425, phigh = 1.0 - 0.02425;
    double x;
    if (p < plow) {
        double q = sqrt(-2.0 * log(p));
        x = (((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) /
            ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1.0);
    } else if (p <= phigh) {
        double q = p - 0.5;
        double r = q * q;
        x = (((((a[0] * r + a[1]) * r + a[2]) * r + a[3]) * r + a[4]) * r + a[5]) * q /
            (((((b[0] * r + b[1]) * r + b[2]) * r + b[3]) * r + b[4]) * r + 1.0);
    } else {
        double q = sqrt(-2.0 * log(1.0 - p));
        x = -(((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) /
            ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1.0);
    }
    double e = 0.5 * erfc(-x / sqrt(2.0)) - p;
    double u = e * sqrt(2.0 * 3.14159265358979323846) * exp(x * x / 2.0);
    return x - u / (1.0 + x * u / 2.0);
}

/* table[u] = bf16(sigma * Phi^-1((u + 0.5) / 65536)), rounded f64 -> f32 -> bf16. */
static inline void fw_synth_normal_table(double sigma, uint16_t* table) {
    for (uint32_t u = 0; u < 65536u; ++u) {
        double z = fw_synth_normal_quantile(((double)u + 0.5) / 65536.0);
        float v = (float)(sigma * z);
        uint32_t bits;
        memcpy(&bits, &v, sizeof bits);
        table[u] = fw_synth_round_bf16(bits);
    }
}

/* 64-bit FNV-1a over little-endian bf16 words: a drift check for the tables. */
static inline uint64_t fw_synth_fnv1a(const uint16_t* values, size_t count) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (size_t i = 0; i < count; ++i) {
        h = (h ^ (values[i] & 0xffu)) * 0x100000001b3ULL;
        h = (h ^ (values[i] >> 8)) * 0x100000001b3ULL;
    }
    return h;
}

/* Per-layer popularity ranking: expert_of_rank[r] is the expert with
 * popularity rank r (0 = most popular); seeded Fisher-Yates. */
static inline void fw_synth_layer_ranking(uint64_t seed, uint32_t layer, uint32_t experts,
                                          uint32_t* expert_of_rank) {
    uint64_t stream = fw_synth_stream(seed, layer, FW_SYNTH_PERMUTATION);
    for (uint32_t i = 0; i < experts; ++i) expert_of_rank[i] = i;
    for (uint32_t i = experts; i-- > 1;) {
        uint32_t j = (uint32_t)(fw_mix64(stream + i) % (uint64_t)(i + 1));
        uint32_t t = expert_of_rank[i];
        expert_of_rank[i] = expert_of_rank[j];
        expert_of_rank[j] = t;
    }
}

/* Router bias column for one layer: bias[e] = bf16(-slope * ln(rank(e) + 1)). */
static inline void fw_synth_router_bias(uint64_t seed, uint32_t layer, uint32_t experts,
                                        double slope, uint32_t* scratch_rank,
                                        uint16_t* bias) {
    fw_synth_layer_ranking(seed, layer, experts, scratch_rank);
    for (uint32_t r = 0; r < experts; ++r) {
        float v = (float)(-slope * log((double)r + 1.0));
        uint32_t bits;
        memcpy(&bits, &v, sizeof bits);
        bias[scratch_rank[r]] = fw_synth_round_bf16(bits);
    }
}

/* T seeded hidden vectors of width H: bf16(N(0,1)) through the unit table,
 * RMS-normalised once in f64 and rounded to bf16; with bias_feature the last
 * element is set to 1.0 (the constant router-bias feature). */
static inline void fw_synth_hidden(uint64_t seed, uint32_t first_token, uint32_t tokens,
                                   uint32_t hidden, int bias_feature,
                                   const uint16_t* unit_table, uint16_t* out) {
    for (uint32_t t = 0; t < tokens; ++t) {
        uint64_t stream = fw_synth_stream(seed, first_token + t, FW_SYNTH_HIDDEN);
        uint16_t* row = out + (size_t)t * hidden;
        double ss = 0.0;
        for (uint32_t h = 0; h < hidden; ++h) {
            row[h] = unit_table[fw_synth_u16(stream, h)];
            uint32_t bits = (uint32_t)row[h] << 16;
            float f;
            memcpy(&f, &bits, sizeof f);
            ss += (double)f * (double)f;
        }
        double inv = 1.0 / sqrt(ss / (double)hidden);
        for (uint32_t h = 0; h < hidden; ++h) {
            uint32_t bits = (uint32_t)row[h] << 16;
            float f;
            memcpy(&f, &bits, sizeof f);
            float v = (float)((double)f * inv);
            memcpy(&bits, &v, sizeof bits);
            row[h] = fw_synth_round_bf16(bits);
        }
        if (bias_feature) row[hidden - 1] = 0x3f80u;
    }
}

/* One synthetic weight element: table[u16(stream, index)]. */
FW_SYNTH_HD uint16_t fw_synth_weight(const uint16_t* table, uint64_t stream, uint64_t index) {
    return table[fw_synth_u16(stream, index)];
}

#endif /* FW_SYNTH_H */
