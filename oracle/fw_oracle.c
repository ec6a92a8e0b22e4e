/*
 * CPU oracle for the sparse-MoE block hot path. TEST INFRASTRUCTURE ONLY (the
 * checker for tests, the smoke check and bench.py's CPU baseline); nothing in
 * the product links or calls it.
 *
 * Every function restates the reference crate's Rust arithmetic operation by
 * operation; the citation above each names the lines it follows. Build with
 * -O2 -ffp-contract=off and without fast-math (oracle/Makefile) so that no
 * multiply-add is contracted and every f32 operation rounds where Rust's does.
 *
 * Parity pins (tests/test_oracle_*.py): the reference's own known-answer tests
 * (src/expert.rs:1227-1293, src/router.rs:416-433, src/decoder_layer.rs:682-689,
 * src/metal_moe.rs:661-680, tests/test_generate_*_fixture.py), the router
 * fixture's committed input hashes and selected logits/scores
 * (fixtures/router/qwen3_8_flash_next_real.json), the reference's top-k shim
 * built from its own source (oracle/_ref), and brute-force/closed-form checks.
 */
#include "fw_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../firewing_amd/csrc/fw_synth.h"

/* src/expert.rs:315-318 (also src/router.rs:126-129): round to nearest even by
 * integer addition, wrapping, with no NaN/Inf special case. */
uint16_t fwo_to_bf16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    return (uint16_t)((uint32_t)(bits + (0x7fffu + ((bits >> 16) & 1u))) >> 16);
}

/* src/expert.rs:320-322. */
float fwo_from_bf16(uint16_t value) {
    uint32_t bits = (uint32_t)value << 16;
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

/* Rust f32::exp lowers to the platform expf; on Linux that is glibc's. */
float fwo_expf(float x) { return expf(x); }

void fwo_expf_array(const float* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(in[i]);
}

/* src/expert.rs:514-552 pytorch_bf16_vector_dot: 8 registers x 4 lanes of f32
 * accumulators over 32-value blocks (multiply, then add; no FMA), the register
 * tree 4/2/1, then (a0+a1)+(a2+a3); an 8-wide tail and a scalar tail.
 * Accumulator [register][lane] is acc[4 * register + lane], i.e. column j of
 * each block feeds acc[j]; the flat form lets the compiler use vector lanes,
 * each of which performs the same f32 multiply and add. */
float fwo_dot_tree32(const uint16_t* left, const uint16_t* right, size_t n) {
    float acc[32];
    for (int j = 0; j < 32; ++j) acc[j] = 0.0f;
    size_t complete_blocks = n / 32 * 32;
    for (size_t block = 0; block < complete_blocks; block += 32) {
        for (int j = 0; j < 32; ++j) {
            uint32_t lb = (uint32_t)left[block + j] << 16;
            uint32_t rb = (uint32_t)right[block + j] << 16;
            float lf, rf;
            memcpy(&lf, &lb, sizeof lf);
            memcpy(&rf, &rb, sizeof rf);
            float product = lf * rf;
            acc[j] = acc[j] + product;
        }
    }
    static const int offsets[3] = {4, 2, 1};
    for (int o = 0; o < 3; ++o) {
        int offset = offsets[o];
        for (int reg = 0; reg < offset; ++reg) {
            for (int lane = 0; lane < 4; ++lane) {
                acc[4 * reg + lane] = acc[4 * reg + lane] + acc[4 * (offset + reg) + lane];
            }
        }
    }
    float reduced = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    size_t complete_vectors = n / 8 * 8;
    float tail[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t block = complete_blocks; block < complete_vectors; block += 8) {
        for (int lane = 0; lane < 4; ++lane) {
            float p0 = fwo_from_bf16(left[block + lane]) * fwo_from_bf16(right[block + lane]);
            tail[lane] = tail[lane] + p0;
            float p1 =
                fwo_from_bf16(left[block + 4 + lane]) * fwo_from_bf16(right[block + 4 + lane]);
            tail[lane] = tail[lane] + p1;
        }
    }
    /* Always executed, so a -0.0 sum leaves as +0.0. */
    reduced = reduced + ((tail[0] + tail[1]) + (tail[2] + tail[3]));
    for (size_t index = complete_vectors; index < n; ++index) {
        float product = fwo_from_bf16(left[index]) * fwo_from_bf16(right[index]);
        reduced = reduced + product;
    }
    return reduced;
}

/* src/router.rs:228-240: one sequential f32 fold from 0.0, sum + w * x. */
float fwo_dot_fold(const uint16_t* weight, const uint16_t* input, size_t n) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float product = fwo_from_bf16(weight[i]) * fwo_from_bf16(input[i]);
        sum = sum + product;
    }
    return sum;
}

/* src/expert.rs:554-560 linear_bf16: out[r] = bf16(tree32(W[r,:], x)). */
void fwo_linear_bf16(const uint16_t* weight, const uint16_t* input, size_t rows, size_t columns,
                     uint16_t* out) {
    for (size_t r = 0; r < rows; ++r) {
        out[r] = fwo_to_bf16(fwo_dot_tree32(weight + r * columns, input, columns));
    }
}

/* src/router.rs:228-240 logits: bf16(fold(W[r,:], x)). */
void fwo_linear_fold_bf16(const uint16_t* weight, const uint16_t* input, size_t rows,
                          size_t columns, uint16_t* out) {
    for (size_t r = 0; r < rows; ++r) {
        out[r] = fwo_to_bf16(fwo_dot_fold(weight + r * columns, input, columns));
    }
}

/* src/expert.rs:562-571 swiglu_bf16: silu = bf16(g / (1 + exp(-g))),
 * out = bf16(silu * up). */
void fwo_swiglu_bf16(const uint16_t* gate, const uint16_t* up, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; ++i) {
        float g = fwo_from_bf16(gate[i]);
        float denominator = 1.0f + expf(-g);
        float silu = fwo_from_bf16(fwo_to_bf16(g / denominator));
        out[i] = fwo_to_bf16(silu * fwo_from_bf16(up[i]));
    }
}

/* src/expert.rs:573-576 sigmoid_bf16. */
uint16_t fwo_sigmoid_bf16(uint16_t value) {
    float v = fwo_from_bf16(value);
    float denominator = 1.0f + expf(-v);
    return fwo_to_bf16(1.0f / denominator);
}

/* src/expert.rs:578-580 add_bf16. */
uint16_t fwo_add_bf16(uint16_t left, uint16_t right) {
    return fwo_to_bf16(fwo_from_bf16(left) + fwo_from_bf16(right));
}

/* Workload glue, not part of the reference's block: the pre-norm of a decoder
 * layer, h = bf16(r * 1/sqrt(mean(r^2) + 1e-6)) with mean(r^2) taken through
 * the reference's own dot (pytorch_bf16_vector_dot(r, r), src/expert.rs:514)
 * divided by H; h[H-1] = 1.0 when the router-bias feature is on. */
void fwo_rms_norm_bf16(const uint16_t* r, size_t n, int bias_feature, uint16_t* h) {
    float ss = fwo_dot_tree32(r, r, n);
    float ms = ss / (float)n;
    float inv = 1.0f / sqrtf(ms + 1e-6f);
    for (size_t i = 0; i < n; ++i) h[i] = fwo_to_bf16(fwo_from_bf16(r[i]) * inv);
    if (bias_feature) h[n - 1] = 0x3f80u;
}

/* src/metal_moe.rs:385-392 build_silu_lut: LUT[b] = bf16(silu(from_bf16(b))). */
void fwo_build_silu_lut(uint16_t* lut) {
    for (uint32_t bits = 0; bits < 65536u; ++bits) {
        float g = fwo_from_bf16((uint16_t)bits);
        float denominator = 1.0f + expf(-g);
        lut[bits] = fwo_to_bf16(g / denominator);
    }
}

/* src/hyper_connection.rs:211-283 pytorch_inner_square_sum: the sum of
 * squares in PyTorch's aarch64 contiguous f32 reduction order. The vector
 * part (n / 4 vectors of 4 lanes, in groups of 4 vectors: `cascade` groups)
 * runs 16 independent (register, lane) accumulators; group g feeds register r
 * lane l with element 16g + 4r + l. Each accumulator's terms are summed in a
 * cascade of LEVELS = 4 levels: level 0 sums `step` = 2^power consecutive
 * groups, then is added into level 1 and cleared; level 1 is added into level 2
 * only after `step` level-0 runs (index a multiple of step^2), and so on
 * (power = max(4, ceil(log2(cascade)) / 4)). Groups past the last full run go
 * straight into level 0; the levels are then folded into level 0 in order,
 * vectors past the groups go into register 0, registers 1..3 are folded into
 * register 0, and the result is the square sum of the scalar tail (n % 4
 * elements, from 0) plus lanes 0..3 in order. Every multiply and add is a
 * separately rounded f32 operation. */
float fwo_inner_square_sum(const float* v, size_t n) {
    enum { LANES = 4, REGS = 4, LEVELS = 4 };
    const size_t vectors = n / LANES;
    const size_t cascade = vectors / REGS;
    size_t ceil_log2 = 0;
    if (cascade > 1) {
        size_t x = cascade - 1;
        while (x) {
            ++ceil_log2;
            x >>= 1;
        }
    }
    const size_t power = ceil_log2 / LEVELS > 4 ? ceil_log2 / LEVELS : 4;
    const size_t step = (size_t)1 << power;
    const size_t mask = step - 1;
    float acc[LEVELS][REGS][LANES];
    memset(acc, 0, sizeof acc);
    size_t g = 0;
    while (g + step <= cascade) {
        for (size_t k = 0; k < step; ++k, ++g) {
            for (size_t r = 0; r < REGS; ++r) {
                for (size_t l = 0; l < LANES; ++l) {
                    float x = v[(g * REGS + r) * LANES + l];
                    float sq = x * x;
                    acc[0][r][l] = acc[0][r][l] + sq;
                }
            }
        }
        for (size_t lv = 1; lv < LEVELS; ++lv) {
            for (size_t r = 0; r < REGS; ++r) {
                for (size_t l = 0; l < LANES; ++l) {
                    acc[lv][r][l] = acc[lv][r][l] + acc[lv - 1][r][l];
                    acc[lv - 1][r][l] = 0.0f;
                }
            }
            if (g & (mask << (lv * power))) break;
        }
    }
    for (; g < cascade; ++g) {
        for (size_t r = 0; r < REGS; ++r) {
            for (size_t l = 0; l < LANES; ++l) {
                float x = v[(g * REGS + r) * LANES + l];
                float sq = x * x;
                acc[0][r][l] = acc[0][r][l] + sq;
            }
        }
    }
    for (size_t lv = 1; lv < LEVELS; ++lv)
        for (size_t r = 0; r < REGS; ++r)
            for (size_t l = 0; l < LANES; ++l) acc[0][r][l] = acc[0][r][l] + acc[lv][r][l];
    for (size_t vec = cascade * REGS; vec < vectors; ++vec) {
        for (size_t l = 0; l < LANES; ++l) {
            float x = v[vec * LANES + l];
            float sq = x * x;
            acc[0][0][l] = acc[0][0][l] + sq;
        }
    }
    for (size_t r = 1; r < REGS; ++r)
        for (size_t l = 0; l < LANES; ++l) acc[0][0][l] = acc[0][0][l] + acc[0][r][l];
    float result = 0.0f;
    for (size_t i = vectors * LANES; i < n; ++i) {
        float sq = v[i] * v[i];
        result = result + sq;
    }
    for (size_t l = 0; l < LANES; ++l) result = result + acc[0][0][l];
    return result;
}

/* src/hyper_connection.rs:285-303 grouped_rms: each of `streams` groups of
 * `width` values normalised on its own, out = bf16((v * inv) * (1 + w)) with
 * inv = 1 / sqrt(square_sum / width + eps), each step rounded to f32. */
void fwo_grouped_rms(const uint16_t* input, const uint16_t* weight, size_t streams, size_t width,
                     float epsilon, uint16_t* out) {
    float* f = (float*)malloc(width * sizeof(float));
    for (size_t s = 0; s < streams; ++s) {
        const uint16_t* in = input + s * width;
        for (size_t i = 0; i < width; ++i) f[i] = fwo_from_bf16(in[i]);
        float mean = fwo_inner_square_sum(f, width) / (float)width;
        float root = sqrtf(mean + epsilon);
        float inverse = 1.0f / root;
        for (size_t i = 0; i < width; ++i) {
            float scaled = f[i] * inverse;
            float gain = 1.0f + fwo_from_bf16(weight[s * width + i]);
            out[s * width + i] = fwo_to_bf16(scaled * gain);
        }
    }
    free(f);
}

/* src/hyper_connection.rs:305-307 four_stream_mean: a left fold from 0 over
 * the streams, then divided by their count. */
static float stream_mean(const float* values, size_t streams) {
    float sum = 0.0f;
    for (size_t s = 0; s < streams; ++s) sum = sum + values[s];
    return sum / (float)streams;
}

float fwo_stream_mean(const float* values, size_t streams) { return stream_mean(values, streams); }

/* src/hyper_connection.rs:309-317 silu_bf16 (the same formula as the expert's
 * SiLU, src/expert.rs:565-569). */
static uint16_t silu_of(uint16_t bits) {
    float g = fwo_from_bf16(bits);
    float denominator = 1.0f + expf(-g);
    return fwo_to_bf16(g / denominator);
}

/* src/hyper_connection.rs:412-490 run_hyper_connection for one token: the
 * hyper-connection of `streams` streams of `width` (input [S*W]) with weights
 * hc_norm [S*W], mix_down [R, S*W], mix_up [S*W, R], inject [S, S*W]
 * (R = lowrank). inject may be NULL (src/hyper_connection.rs:359-410
 * run_final_mixer: the same without the injection outputs). */
int fwo_hyper_connection(const uint16_t* input, const uint16_t* hc_norm, const uint16_t* mix_down_w,
                         const uint16_t* mix_up_w, const uint16_t* inject_w, size_t streams, size_t width,
                         size_t lowrank, fwo_hyper_outputs* o) {
    const size_t SW = streams * width;
    if (streams == 0 || width == 0 || lowrank == 0 || streams > 64) return 0;
    fwo_grouped_rms(input, hc_norm, streams, width, 1.0e-6f, o->hyper_input_normed);
    fwo_linear_bf16(mix_down_w, o->hyper_input_normed, lowrank, SW, o->mix_down);
    for (size_t i = 0; i < lowrank; ++i) {
        o->mix_down_scaled[i] = fwo_to_bf16(fwo_from_bf16(o->mix_down[i]) / (float)streams);
        o->mix_down_silu[i] = silu_of(o->mix_down_scaled[i]);
    }
    fwo_linear_bf16(mix_up_w, o->mix_down_silu, SW, lowrank, o->mix_up);
    for (size_t i = 0; i < SW; ++i) {
        o->input_mix[i] = fwo_sigmoid_bf16(o->mix_up[i]);
        o->products[i] = fwo_to_bf16(fwo_from_bf16(o->input_mix[i]) * fwo_from_bf16(o->hyper_input_normed[i]));
    }
    float column[64];
    for (size_t c = 0; c < width; ++c) {
        for (size_t s = 0; s < streams; ++s) column[s] = fwo_from_bf16(o->products[s * width + c]);
        o->mixed[c] = fwo_to_bf16(stream_mean(column, streams));
    }
    if (inject_w != NULL) {
        fwo_linear_bf16(inject_w, o->hyper_input_normed, streams, SW, o->inject);
        for (size_t s = 0; s < streams; ++s) {
            o->inject_scaled[s] = fwo_to_bf16(fwo_from_bf16(o->inject[s]) / (float)streams);
            o->inject_sigmoid[s] = fwo_sigmoid_bf16(o->inject_scaled[s]);
            o->injection_weights[s] = fwo_to_bf16(2.0f * fwo_from_bf16(o->inject_sigmoid[s]));
        }
    }
    return 1;
}

/* src/decoder_layer.rs:587-607: the block output injected into every stream,
 * products[s][h] = bf16(moe[h] * weight[s]), and added to the residual
 * streams, out[s][h] = add_bf16(post_attention[s][h], products[s][h]). */
void fwo_inject_residual(const uint16_t* post_attention, const uint16_t* moe_output,
                         const uint16_t* injection_weights, size_t streams, size_t width, uint16_t* products,
                         uint16_t* layer_output) {
    for (size_t s = 0; s < streams; ++s) {
        float w = fwo_from_bf16(injection_weights[s]);
        for (size_t h = 0; h < width; ++h) {
            uint16_t p = fwo_to_bf16(fwo_from_bf16(moe_output[h]) * w);
            if (products) products[s * width + h] = p;
            layer_output[s * width + h] = fwo_add_bf16(post_attention[s * width + h], p);
        }
    }
}

/* src/expert.rs:341-360 make_hidden (identical in src/router.rs:142-161):
 * ((i*m + a) rem_euclid M - c) / d on every sparse_stride-th index, else 0. */
int fwo_make_hidden(size_t size, int64_t multiplier, int64_t add, int64_t modulus,
                    int64_t center, int64_t divisor, size_t sparse_stride, uint16_t* out) {
    if (modulus <= 0 || divisor <= 0 || sparse_stride == 0) return 0;
    for (size_t index = 0; index < size; ++index) {
        __int128 affine = (__int128)(int64_t)index * multiplier + add;
        if (affine > INT64_MAX || affine < INT64_MIN) return 0;
        int64_t a = (int64_t)affine;
        int64_t rem = a % modulus;
        if (rem < 0) rem += modulus;
        int64_t raw = rem - center;
        float value = 0.0f;
        if (index % sparse_stride == 0) value = (float)raw / (float)divisor;
        out[index] = fwo_to_bf16(value);
    }
    return 1;
}

/* f32::total_cmp key of a bf16 logit, as an unsigned 16-bit rank. */
static uint32_t total_order_key(uint16_t bits) {
    return (bits & 0x8000u) ? ((~(uint32_t)bits) & 0xffffu) : ((uint32_t)bits | 0x8000u);
}

/* src/router.rs:241-247: stable order by logit descending under total_cmp, then
 * index ascending; truncated to k. Selection of k maxima (O(k*count)) produces
 * the same prefix as the full sort. */
int fwo_topk_total_order(const uint16_t* logits, size_t count, size_t k, int32_t* ids) {
    if (logits == NULL || ids == NULL || k == 0 || k > count) return 0;
    uint8_t* taken = (uint8_t*)calloc(count, 1);
    if (taken == NULL) return 0;
    for (size_t r = 0; r < k; ++r) {
        size_t best = count;
        uint32_t best_key = 0;
        for (size_t e = 0; e < count; ++e) {
            if (taken[e]) continue;
            uint32_t key = total_order_key(logits[e]);
            if (best == count || key > best_key) {
                best = e;
                best_key = key;
            }
        }
        taken[best] = 1;
        ids[r] = (int32_t)best;
    }
    free(taken);
    return 1;
}

/* src/router.rs:248-262 and src/decoder_layer.rs:290-306: max (f32::max fold from
 * -inf), exp(v - max) for every logit, sequential f32 sum in index order,
 * p = e / sum, selected_sum in rank order, score = bf16(p / selected_sum). */
int fwo_route_scores(const uint16_t* logits, size_t experts, const int32_t* ids, size_t k,
                     uint16_t* scores) {
    float* probabilities = (float*)malloc(experts * sizeof(float));
    if (probabilities == NULL) return 0;
    float maximum = -INFINITY;
    for (size_t e = 0; e < experts; ++e) maximum = fmaxf(maximum, fwo_from_bf16(logits[e]));
    float denominator = -0.0f;
    for (size_t e = 0; e < experts; ++e) {
        probabilities[e] = expf(fwo_from_bf16(logits[e]) - maximum);
        denominator = denominator + probabilities[e];
    }
    for (size_t e = 0; e < experts; ++e) probabilities[e] = probabilities[e] / denominator;
    float selected_sum = -0.0f;
    for (size_t r = 0; r < k; ++r) selected_sum = selected_sum + probabilities[ids[r]];
    for (size_t r = 0; r < k; ++r) scores[r] = fwo_to_bf16(probabilities[ids[r]] / selected_sum);
    free(probabilities);
    return 1;
}

/* src/router.rs:220-265 route (order FOLD) and src/decoder_layer.rs:278-307 over
 * linear_bf16 logits (order TREE32, src/decoder_layer.rs:411-413/460). The
 * in-model route rejects NaN logits (src/decoder_layer.rs:279-281). */
int fwo_route(const uint16_t* weight, const uint16_t* hidden, size_t experts, size_t width,
              size_t top_k, int order, int32_t* ids, uint16_t* logits, uint16_t* scores) {
    if (top_k == 0 || top_k > experts) return 0;
    uint16_t* l = logits;
    uint16_t* owned = NULL;
    if (l == NULL) {
        owned = (uint16_t*)malloc(experts * sizeof(uint16_t));
        if (owned == NULL) return 0;
        l = owned;
    }
    if (order == FWO_ORDER_FOLD) {
        fwo_linear_fold_bf16(weight, hidden, experts, width, l);
    } else {
        fwo_linear_bf16(weight, hidden, experts, width, l);
    }
    int ok = 1;
    if (order == FWO_ORDER_TREE32) {
        for (size_t e = 0; e < experts; ++e) {
            if (isnan(fwo_from_bf16(l[e]))) ok = 0;
        }
    }
    if (ok) ok = fwo_topk_total_order(l, experts, top_k, ids);
    if (ok) ok = fwo_route_scores(l, experts, ids, top_k, scores);
    free(owned);
    return ok;
}

/* src/decoder_layer.rs:309-322: the same set, and equal logits rank by rank. */
int fwo_equivalent_topk_order(const int32_t* expected, const int32_t* actual, size_t k,
                              const uint16_t* logits) {
    for (size_t i = 0; i < k; ++i) {
        if (logits[expected[i]] != logits[actual[i]]) return 0;
        int found = 0;
        for (size_t j = 0; j < k; ++j) found |= (expected[i] == actual[j]);
        if (!found) return 0;
    }
    return 1;
}

/* src/expert.rs:717-751: gate_up = linear(W_gu, x, 2I, H); gate = rows [0, I),
 * up = rows [I, 2I); swiglu; down = linear(W_d, swiglu, H, I);
 * weighted = bf16(down * route_weight). Captures may be NULL. */
void fwo_expert_bf16(const uint16_t* gate_up_weight, const uint16_t* down_weight,
                     const uint16_t* hidden, size_t hidden_size, size_t intermediate,
                     uint16_t route_weight, uint16_t* gate_up, uint16_t* swiglu, uint16_t* down,
                     uint16_t* weighted) {
    uint16_t* gu = (uint16_t*)malloc(2 * intermediate * sizeof(uint16_t));
    uint16_t* act = (uint16_t*)malloc(intermediate * sizeof(uint16_t));
    uint16_t* dn = (uint16_t*)malloc(hidden_size * sizeof(uint16_t));
    fwo_linear_bf16(gate_up_weight, hidden, 2 * intermediate, hidden_size, gu);
    fwo_swiglu_bf16(gu, gu + intermediate, intermediate, act);
    fwo_linear_bf16(down_weight, act, hidden_size, intermediate, dn);
    float w = fwo_from_bf16(route_weight);
    if (weighted != NULL) {
        for (size_t h = 0; h < hidden_size; ++h) weighted[h] = fwo_to_bf16(fwo_from_bf16(dn[h]) * w);
    }
    if (gate_up != NULL) memcpy(gate_up, gu, 2 * intermediate * sizeof(uint16_t));
    if (swiglu != NULL) memcpy(swiglu, act, intermediate * sizeof(uint16_t));
    if (down != NULL) memcpy(down, dn, hidden_size * sizeof(uint16_t));
    free(gu);
    free(act);
    free(dn);
}

/* src/expert.rs:906-956: mixture = bf16(0); for each expert in the given
 * (ascending-id execution) order: mixture[h] = bf16(mixture[h] + weighted[h]). */
int fwo_mixture_bf16(const uint16_t* const* gate_up_weights, const uint16_t* const* down_weights,
                     const uint16_t* hidden, size_t hidden_size, size_t intermediate,
                     const int32_t* experts, const uint16_t* route_weights, size_t count,
                     uint16_t* mixture) {
    (void)experts;
    uint16_t* weighted = (uint16_t*)malloc(hidden_size * sizeof(uint16_t));
    if (weighted == NULL) return 0;
    for (size_t h = 0; h < hidden_size; ++h) mixture[h] = fwo_to_bf16(0.0f);
    for (size_t i = 0; i < count; ++i) {
        fwo_expert_bf16(gate_up_weights[i], down_weights[i], hidden, hidden_size, intermediate,
                        route_weights[i], NULL, NULL, NULL, weighted);
        for (size_t h = 0; h < hidden_size; ++h) {
            mixture[h] = fwo_to_bf16(fwo_from_bf16(mixture[h]) + fwo_from_bf16(weighted[h]));
        }
    }
    free(weighted);
    return 1;
}

/* One token through the block, experts given by per-id pointers (only the
 * selected ones are dereferenced). src/decoder_layer.rs:460-586 with the route
 * of src/router.rs:220-265 (FOLD) or src/decoder_layer.rs:278-307 (TREE32), and
 * the shared expert of src/expert.rs:1138-1153. */
static int block_core(const fwo_shape* s, const uint16_t* router, const uint16_t* const* gate_up,
                      const uint16_t* const* down, const uint16_t* shared_gate,
                      const uint16_t* shared_up, const uint16_t* shared_down,
                      const uint16_t* shared_expert_gate, const uint16_t* hidden, int order,
                      const int32_t* known_ids, const uint16_t* known_logits, uint16_t* out,
                      fwo_block_captures* cap) {
    size_t H = s->hidden, I = s->intermediate, E = s->experts, K = s->top_k;
    size_t Is = s->shared_intermediate;
    int ok = 1;
    uint16_t* logits = (uint16_t*)malloc(E * sizeof(uint16_t));
    int32_t* ids = (int32_t*)malloc(K * sizeof(int32_t));
    uint16_t* scores = (uint16_t*)malloc(K * sizeof(uint16_t));
    uint16_t* routed = (uint16_t*)malloc(H * sizeof(uint16_t));
    uint16_t* sg = (uint16_t*)malloc(Is * sizeof(uint16_t));
    uint16_t* su = (uint16_t*)malloc(Is * sizeof(uint16_t));
    uint16_t* ss = (uint16_t*)malloc(Is * sizeof(uint16_t));
    uint16_t* sd = (uint16_t*)malloc(H * sizeof(uint16_t));
    uint16_t* weighted = (uint16_t*)malloc(H * sizeof(uint16_t));
    if (!logits || !ids || !scores || !routed || !sg || !su || !ss || !sd || !weighted) {
        ok = 0;
        goto done;
    }
    if (known_logits != NULL) {
        memcpy(logits, known_logits, E * sizeof(uint16_t));
    } else if (order == FWO_ORDER_FOLD) {
        fwo_linear_fold_bf16(router, hidden, E, H, logits);
    } else {
        fwo_linear_bf16(router, hidden, E, H, logits);
        for (size_t e = 0; e < E; ++e) {
            if (isnan(fwo_from_bf16(logits[e]))) ok = 0;
        }
        if (!ok) goto done;
    }
    if (known_ids != NULL) {
        memcpy(ids, known_ids, K * sizeof(int32_t));
    } else if (!fwo_topk_total_order(logits, E, K, ids)) {
        ok = 0;
        goto done;
    }
    if (!fwo_route_scores(logits, E, ids, K, scores)) {
        ok = 0;
        goto done;
    }
    /* Execution order: ascending expert id (src/decoder_layer.rs:422-424). */
    size_t order_idx[64];
    for (size_t r = 0; r < K; ++r) order_idx[r] = r;
    for (size_t a = 1; a < K; ++a) {
        for (size_t b = a; b > 0 && ids[order_idx[b - 1]] > ids[order_idx[b]]; --b) {
            size_t t = order_idx[b];
            order_idx[b] = order_idx[b - 1];
            order_idx[b - 1] = t;
        }
    }
    for (size_t h = 0; h < H; ++h) routed[h] = fwo_to_bf16(0.0f);
    for (size_t n = 0; n < K; ++n) {
        size_t r = order_idx[n];
        int32_t e = ids[r];
        fwo_expert_bf16(gate_up[e], down[e], hidden, H, I, scores[r], NULL, NULL, NULL, weighted);
        for (size_t h = 0; h < H; ++h) routed[h] = fwo_add_bf16(routed[h], weighted[h]);
        if (cap != NULL && cap->weighted_down) memcpy(cap->weighted_down + n * H, weighted, H * sizeof(uint16_t));
    }
    fwo_linear_bf16(shared_gate, hidden, Is, H, sg);
    fwo_linear_bf16(shared_up, hidden, Is, H, su);
    fwo_swiglu_bf16(sg, su, Is, ss);
    fwo_linear_bf16(shared_down, ss, H, Is, sd);
    uint16_t gate_logit;
    fwo_linear_bf16(shared_expert_gate, hidden, 1, H, &gate_logit);
    uint16_t gate_sigmoid = fwo_sigmoid_bf16(gate_logit);
    float sigmoid = fwo_from_bf16(gate_sigmoid);
    for (size_t h = 0; h < H; ++h) {
        uint16_t gated = fwo_to_bf16(sigmoid * fwo_from_bf16(sd[h]));
        out[h] = fwo_add_bf16(routed[h], gated);
        if (cap != NULL && cap->gated_shared) cap->gated_shared[h] = gated;
    }
    if (cap != NULL) {
        if (cap->logits) memcpy(cap->logits, logits, E * sizeof(uint16_t));
        if (cap->ids) memcpy(cap->ids, ids, K * sizeof(int32_t));
        if (cap->scores) memcpy(cap->scores, scores, K * sizeof(uint16_t));
        if (cap->routed_mixture) memcpy(cap->routed_mixture, routed, H * sizeof(uint16_t));
        if (cap->shared_down) memcpy(cap->shared_down, sd, H * sizeof(uint16_t));
        if (cap->shared_gate_sigmoid) cap->shared_gate_sigmoid[0] = gate_sigmoid;
        if (cap->shared_gate) memcpy(cap->shared_gate, sg, Is * sizeof(uint16_t));
        if (cap->shared_up) memcpy(cap->shared_up, su, Is * sizeof(uint16_t));
        if (cap->shared_swiglu) memcpy(cap->shared_swiglu, ss, Is * sizeof(uint16_t));
        if (cap->shared_gate_logit) cap->shared_gate_logit[0] = gate_logit;
    }
done:
    free(logits);
    free(ids);
    free(scores);
    free(routed);
    free(sg);
    free(su);
    free(ss);
    free(sd);
    free(weighted);
    return ok;
}

int fwo_sparse_moe_block(const fwo_shape* shape, const fwo_layer* layer, const uint16_t* hidden,
                         int order, uint16_t* out, fwo_block_captures* captures) {
    size_t E = shape->experts, H = shape->hidden, I = shape->intermediate;
    if (shape->top_k == 0 || shape->top_k > E || shape->top_k > 64) return 0;
    const uint16_t** gu = (const uint16_t**)malloc(E * sizeof(uint16_t*));
    const uint16_t** dn = (const uint16_t**)malloc(E * sizeof(uint16_t*));
    if (!gu || !dn) {
        free(gu);
        free(dn);
        return 0;
    }
    for (size_t e = 0; e < E; ++e) {
        gu[e] = layer->gate_up + e * 2 * I * H;
        dn[e] = layer->down + e * H * I;
    }
    int ok = block_core(shape, layer->router, gu, dn, layer->shared_gate, layer->shared_up,
                        layer->shared_down, layer->shared_expert_gate, hidden, order, NULL, NULL,
                        out, captures);
    free(gu);
    free(dn);
    return ok;
}

/* ---- synthetic workload regeneration (inputs only) ---- */

static uint16_t g_unit_table[65536];
static uint16_t g_weight_table[65536];
static int g_tables_ready = 0;

static void ensure_tables(void) {
    if (g_tables_ready) return;
    fw_synth_normal_table(1.0, g_unit_table);
    fw_synth_normal_table(FW_SYNTH_WEIGHT_SIGMA, g_weight_table);
    g_tables_ready = 1;
}

void fwo_synth_tables(uint16_t* unit_table, uint16_t* weight_table) {
    ensure_tables();
    if (unit_table) memcpy(unit_table, g_unit_table, sizeof g_unit_table);
    if (weight_table) memcpy(weight_table, g_weight_table, sizeof g_weight_table);
}

void fwo_synth_hidden(uint64_t seed, uint32_t first_token, uint32_t tokens, uint32_t hidden,
                      int bias_feature, uint16_t* out) {
    ensure_tables();
    fw_synth_hidden(seed, first_token, tokens, hidden, bias_feature, g_unit_table, out);
}

void fwo_synth_tensor(uint64_t seed, uint32_t layer, uint32_t tensor, uint64_t first,
                      uint64_t count, uint16_t* out) {
    ensure_tables();
    uint64_t stream = fw_synth_stream(seed, layer, tensor);
    for (uint64_t i = 0; i < count; ++i) out[i] = fw_synth_weight(g_weight_table, stream, first + i);
}

void fwo_synth_router_bias(uint64_t seed, uint32_t layer, uint32_t experts, uint16_t* bias) {
    uint32_t* rank = (uint32_t*)malloc(experts * sizeof(uint32_t));
    fw_synth_router_bias(seed, layer, experts, FW_SYNTH_ZIPF_BIAS_SLOPE, rank, bias);
    free(rank);
}

typedef struct {
    uint16_t* router;
    uint16_t* shared_gate;
    uint16_t* shared_up;
    uint16_t* shared_down;
    uint16_t* shared_expert_gate;
    uint16_t** gate_up;
    uint16_t** down;
    size_t experts;
} synth_layer;

static void synth_layer_free(synth_layer* L) {
    free(L->router);
    free(L->shared_gate);
    free(L->shared_up);
    free(L->shared_down);
    free(L->shared_expert_gate);
    if (L->gate_up) {
        for (size_t e = 0; e < L->experts; ++e) free(L->gate_up[e]);
    }
    if (L->down) {
        for (size_t e = 0; e < L->experts; ++e) free(L->down[e]);
    }
    free(L->gate_up);
    free(L->down);
    memset(L, 0, sizeof *L);
}

static int synth_layer_dense(const fwo_shape* s, const fwo_synth_config* c, uint32_t layer,
                             synth_layer* L) {
    size_t H = s->hidden, E = s->experts, Is = s->shared_intermediate;
    memset(L, 0, sizeof *L);
    L->experts = E;
    L->router = (uint16_t*)malloc(E * H * sizeof(uint16_t));
    L->shared_gate = (uint16_t*)malloc(Is * H * sizeof(uint16_t));
    L->shared_up = (uint16_t*)malloc(Is * H * sizeof(uint16_t));
    L->shared_down = (uint16_t*)malloc(H * Is * sizeof(uint16_t));
    L->shared_expert_gate = (uint16_t*)malloc(H * sizeof(uint16_t));
    L->gate_up = (uint16_t**)calloc(E, sizeof(uint16_t*));
    L->down = (uint16_t**)calloc(E, sizeof(uint16_t*));
    if (!L->router || !L->shared_gate || !L->shared_up || !L->shared_down ||
        !L->shared_expert_gate || !L->gate_up || !L->down)
        return 0;
    fwo_synth_tensor(c->seed, layer, FW_SYNTH_ROUTER, 0, E * H, L->router);
    if (c->bias_feature) {
        uint16_t* bias = (uint16_t*)malloc(E * sizeof(uint16_t));
        if (!bias) return 0;
        fwo_synth_router_bias(c->seed, layer, (uint32_t)E, bias);
        for (size_t e = 0; e < E; ++e) L->router[e * H + H - 1] = bias[e];
        free(bias);
    }
    fwo_synth_tensor(c->seed, layer, FW_SYNTH_SHARED_GATE, 0, Is * H, L->shared_gate);
    fwo_synth_tensor(c->seed, layer, FW_SYNTH_SHARED_UP, 0, Is * H, L->shared_up);
    fwo_synth_tensor(c->seed, layer, FW_SYNTH_SHARED_DOWN, 0, H * Is, L->shared_down);
    fwo_synth_tensor(c->seed, layer, FW_SYNTH_SHARED_EXPERT_GATE, 0, H, L->shared_expert_gate);
    return 1;
}

static int synth_layer_expert(const fwo_shape* s, const fwo_synth_config* c, uint32_t layer,
                              synth_layer* L, int32_t e) {
    size_t H = s->hidden, I = s->intermediate;
    if (L->gate_up[e] != NULL) return 1;
    L->gate_up[e] = (uint16_t*)malloc(2 * I * H * sizeof(uint16_t));
    L->down[e] = (uint16_t*)malloc(H * I * sizeof(uint16_t));
    if (!L->gate_up[e] || !L->down[e]) return 0;
    fwo_synth_tensor(c->seed, layer, FW_SYNTH_GATE_UP, (uint64_t)e * 2 * I * H, 2 * I * H,
                     L->gate_up[e]);
    fwo_synth_tensor(c->seed, layer, FW_SYNTH_DOWN, (uint64_t)e * H * I, H * I, L->down[e]);
    return 1;
}

/* Router logits, ids and scores of T tokens at one synthetic layer. */
int fwo_synth_route(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                    const uint16_t* hidden, size_t tokens, int32_t* ids, uint16_t* scores,
                    uint16_t* logits) {
    synth_layer L;
    if (!synth_layer_dense(shape, config, layer, &L)) {
        synth_layer_free(&L);
        return 0;
    }
    size_t H = shape->hidden, E = shape->experts, K = shape->top_k;
    int ok = 1;
    int threads = config->threads > 0 ? config->threads : 1;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1) reduction(&& : ok)
    for (long t = 0; t < (long)tokens; ++t) {
        uint16_t* l = logits ? logits + (size_t)t * E : NULL;
        ok = ok && fwo_route(L.router, hidden + (size_t)t * H, E, H, K, config->order,
                             ids + (size_t)t * K, l, scores + (size_t)t * K);
    }
    synth_layer_free(&L);
    return ok;
}

static int synth_block(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                       const uint16_t* hidden, size_t tokens, uint16_t* out, int32_t* ids,
                       uint16_t* scores, uint16_t* logits, fwo_block_captures* caps) {
    size_t H = shape->hidden, E = shape->experts, K = shape->top_k;
    if (K == 0 || K > 64 || K > E) return 0;
    synth_layer L;
    if (!synth_layer_dense(shape, config, layer, &L)) {
        synth_layer_free(&L);
        return 0;
    }
    int ok = 1;
    int32_t* sel = (int32_t*)malloc(tokens * K * sizeof(int32_t));
    uint16_t* sc = (uint16_t*)malloc(tokens * K * sizeof(uint16_t));
    uint16_t* lg = (uint16_t*)malloc(tokens * E * sizeof(uint16_t));
    if (!sel || !sc || !lg) ok = 0;
    int threads = config->threads > 0 ? config->threads : 1;
    if (ok) {
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1) reduction(&& : ok)
        for (long t = 0; t < (long)tokens; ++t) {
            ok = ok && fwo_route(L.router, hidden + (size_t)t * H, E, H, K, config->order,
                                 sel + (size_t)t * K, lg + (size_t)t * E, sc + (size_t)t * K);
        }
    }
    for (size_t t = 0; ok && t < tokens; ++t) {
        for (size_t r = 0; ok && r < K; ++r) ok = synth_layer_expert(shape, config, layer, &L, sel[t * K + r]);
    }
    if (ok) {
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1) reduction(&& : ok)
        for (long t = 0; t < (long)tokens; ++t) {
            ok = ok && block_core(shape, L.router, (const uint16_t* const*)L.gate_up,
                                  (const uint16_t* const*)L.down, L.shared_gate, L.shared_up,
                                  L.shared_down, L.shared_expert_gate, hidden + (size_t)t * H,
                                  config->order, sel + (size_t)t * K, lg + (size_t)t * E,
                                  out + (size_t)t * H, caps ? caps + t : NULL);
        }
    }
    if (ok) {
        if (ids) memcpy(ids, sel, tokens * K * sizeof(int32_t));
        if (scores) memcpy(scores, sc, tokens * K * sizeof(uint16_t));
        if (logits) memcpy(logits, lg, tokens * E * sizeof(uint16_t));
    }
    free(sel);
    free(sc);
    free(lg);
    synth_layer_free(&L);
    return ok;
}

int fwo_synth_block(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                    const uint16_t* hidden, size_t tokens, uint16_t* out, int32_t* ids,
                    uint16_t* scores, uint16_t* logits) {
    return synth_block(shape, config, layer, hidden, tokens, out, ids, scores, logits, NULL);
}

int fwo_synth_block_captured(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                             const uint16_t* hidden, size_t tokens, uint16_t* out,
                             fwo_block_captures* captures) {
    return synth_block(shape, config, layer, hidden, tokens, out, NULL, NULL, NULL, captures);
}

/* Chained decode step over `layers` synthetic layers. Workload glue, not in the
 * reference: a pre-norm residual stream, h_l = rms_norm(r_l) (fwo_rms_norm_bf16),
 * r_{l+1}[i] = add_bf16(r_l[i], block_l(h_l)[i]) (the residual add of
 * src/decoder_layer.rs:601-606 with unit injection). r_0 = hidden. */
int fwo_synth_step(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layers,
                   const uint16_t* hidden, size_t tokens, uint16_t* residual_out,
                   uint16_t* block_out, int32_t* ids, uint16_t* scores) {
    size_t H = shape->hidden, K = shape->top_k;
    uint16_t* x = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    uint16_t* o = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    if (!x || !o) {
        free(x);
        free(o);
        return 0;
    }
    uint16_t* hn = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    memcpy(x, hidden, tokens * H * sizeof(uint16_t));
    int ok = hn != NULL;
    for (uint32_t l = 0; ok && l < layers; ++l) {
        for (size_t t = 0; t < tokens; ++t) fwo_rms_norm_bf16(x + t * H, H, config->bias_feature, hn + t * H);
        ok = fwo_synth_block(shape, config, l, hn, tokens, o, ids ? ids + (size_t)l * tokens * K : NULL,
                             scores ? scores + (size_t)l * tokens * K : NULL, NULL);
        if (!ok) break;
        if (block_out) memcpy(block_out + (size_t)l * tokens * H, o, tokens * H * sizeof(uint16_t));
        for (size_t t = 0; t < tokens; ++t) {
            for (size_t h = 0; h < H; ++h) x[t * H + h] = fwo_add_bf16(x[t * H + h], o[t * H + h]);
        }
    }
    free(hn);
    if (ok && residual_out) memcpy(residual_out, x, tokens * H * sizeof(uint16_t));
    free(x);
    free(o);
    return ok;
}

static double now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* The chained step of fwo_synth_step on one thread, timing only the block
 * arithmetic (router, top-k, scores, experts, mixture, shared expert,
 * combine, residual add). Regenerating each layer's synthetic weights is
 * outside the timed region: the reference reads resident weights. */
int fwo_synth_step_timed(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layers,
                         const uint16_t* hidden, size_t tokens, uint16_t* residual_out,
                         double* compute_seconds) {
    size_t H = shape->hidden, E = shape->experts, K = shape->top_k;
    if (K == 0 || K > 64 || K > E) return 0;
    uint16_t* x = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    uint16_t* o = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    int32_t* sel = (int32_t*)malloc(tokens * K * sizeof(int32_t));
    uint16_t* sc = (uint16_t*)malloc(tokens * K * sizeof(uint16_t));
    uint16_t* lg = (uint16_t*)malloc(tokens * E * sizeof(uint16_t));
    uint16_t* hn = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    int ok = x && o && sel && sc && lg && hn;
    double timed = 0.0;
    if (ok) memcpy(x, hidden, tokens * H * sizeof(uint16_t));
    for (uint32_t l = 0; ok && l < layers; ++l) {
        synth_layer L;
        ok = synth_layer_dense(shape, config, l, &L);
        double t0 = now_seconds();
        for (size_t t = 0; t < tokens; ++t) fwo_rms_norm_bf16(x + t * H, H, config->bias_feature, hn + t * H);
        for (size_t t = 0; ok && t < tokens; ++t) {
            ok = fwo_route(L.router, hn + t * H, E, H, K, config->order, sel + t * K, lg + t * E,
                           sc + t * K);
        }
        timed += now_seconds() - t0;
        for (size_t t = 0; ok && t < tokens; ++t) {
            for (size_t r = 0; ok && r < K; ++r) ok = synth_layer_expert(shape, config, l, &L, sel[t * K + r]);
        }
        t0 = now_seconds();
        for (size_t t = 0; ok && t < tokens; ++t) {
            ok = block_core(shape, L.router, (const uint16_t* const*)L.gate_up,
                            (const uint16_t* const*)L.down, L.shared_gate, L.shared_up,
                            L.shared_down, L.shared_expert_gate, hn + t * H, config->order,
                            sel + t * K, lg + t * E, o + t * H, NULL);
        }
        for (size_t t = 0; ok && t < tokens; ++t) {
            for (size_t h = 0; h < H; ++h) x[t * H + h] = fwo_add_bf16(x[t * H + h], o[t * H + h]);
        }
        timed += now_seconds() - t0;
        synth_layer_free(&L);
    }
    if (ok && residual_out) memcpy(residual_out, x, tokens * H * sizeof(uint16_t));
    if (compute_seconds) *compute_seconds = timed;
    free(x);
    free(o);
    free(sel);
    free(sc);
    free(lg);
    free(hn);
    return ok;
}

/* ---- CPU baseline timing (the benchmark's reported CPU leg) ------------------ */

/* rows of linear_bf16 (src/expert.rs:554-560) split over threads; each row's
 * dot is the same sequential tree32 dot. */
static void linear_rows_mt(const uint16_t* w, const uint16_t* x, size_t rows, size_t cols, uint16_t* out,
                           int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (long r = 0; r < (long)rows; ++r) out[r] = fwo_to_bf16(fwo_dot_tree32(w + (size_t)r * cols, x, cols));
}

/* block_core for one token with the matrix rows split over threads (router
 * rows, each expert's gate_up and down rows, the mixture over hidden
 * elements): every output is computed by the same operations in the same
 * order as block_core (TREE32 logits). */
static int block_rows_mt(const fwo_shape* s, const synth_layer* L, const uint16_t* hidden, uint16_t* out,
                         int threads) {
    size_t H = s->hidden, I = s->intermediate, E = s->experts, K = s->top_k, Is = s->shared_intermediate;
    uint16_t* logits = (uint16_t*)malloc(E * sizeof(uint16_t));
    uint16_t* scores = (uint16_t*)malloc(K * sizeof(uint16_t));
    uint16_t* gu = (uint16_t*)malloc(2 * (I > Is ? I : Is) * sizeof(uint16_t));
    uint16_t* act = (uint16_t*)malloc((I > Is ? I : Is) * sizeof(uint16_t));
    uint16_t* dn = (uint16_t*)malloc(K * H * sizeof(uint16_t));
    uint16_t* sd = (uint16_t*)malloc(H * sizeof(uint16_t));
    int32_t ids[64];
    int ok = logits && scores && gu && act && dn && sd;
    if (ok) {
        linear_rows_mt(L->router, hidden, E, H, logits, threads);
        for (size_t e = 0; e < E; ++e) {
            if (isnan(fwo_from_bf16(logits[e]))) ok = 0;
        }
        ok = ok && fwo_topk_total_order(logits, E, K, ids);
        ok = ok && fwo_route_scores(logits, E, ids, K, scores);
    }
    size_t order_idx[64];
    for (size_t r = 0; r < K; ++r) order_idx[r] = r;
    for (size_t a = 1; a < K; ++a)
        for (size_t b = a; b > 0 && ids[order_idx[b - 1]] > ids[order_idx[b]]; --b) {
            size_t t = order_idx[b];
            order_idx[b] = order_idx[b - 1];
            order_idx[b - 1] = t;
        }
    for (size_t n = 0; ok && n < K; ++n) {
        size_t r = order_idx[n];
        linear_rows_mt(L->gate_up[ids[r]], hidden, 2 * I, H, gu, threads);
        fwo_swiglu_bf16(gu, gu + I, I, act);
        linear_rows_mt(L->down[ids[r]], act, H, I, dn + n * H, threads);
        float w = fwo_from_bf16(scores[r]);
        for (size_t h = 0; h < H; ++h) dn[n * H + h] = fwo_to_bf16(fwo_from_bf16(dn[n * H + h]) * w);
    }
    if (ok) {
        linear_rows_mt(L->shared_gate, hidden, Is, H, gu, threads);
        linear_rows_mt(L->shared_up, hidden, Is, H, gu + Is, threads);
        fwo_swiglu_bf16(gu, gu + Is, Is, act);
        linear_rows_mt(L->shared_down, act, H, Is, sd, threads);
        uint16_t gate_logit;
        fwo_linear_bf16(L->shared_expert_gate, hidden, 1, H, &gate_logit);
        float sigmoid = fwo_from_bf16(fwo_sigmoid_bf16(gate_logit));
#pragma omp parallel for num_threads(threads) schedule(static)
        for (long h = 0; h < (long)H; ++h) {
            uint16_t mix = fwo_to_bf16(0.0f);
            for (size_t n = 0; n < K; ++n) mix = fwo_add_bf16(mix, dn[n * H + h]);
            out[h] = fwo_add_bf16(mix, fwo_to_bf16(sigmoid * fwo_from_bf16(sd[h])));
        }
    }
    free(logits);
    free(scores);
    free(gu);
    free(act);
    free(dn);
    free(sd);
    return ok;
}

/* Times the block of one synthetic layer on `tokens` inputs: the layer's
 * dense weights and the experts the tokens select are generated first
 * (untimed); then `warmups` untimed and `runs` timed evaluations of the whole
 * block for every token (pre-norm when `prenorm`, route, experts, mixture,
 * shared expert, combine), seconds per run into samples[runs]; the last
 * run's outputs into out [tokens][H] (NULL to skip). threads > 1: the tokens
 * in parallel when there are at least as many as threads, else each matrix's
 * rows (TREE32 logits only). */
int fwo_bench_block(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                    const uint16_t* hidden, size_t tokens, int prenorm, int warmups, int runs,
                    double* samples, uint16_t* out) {
    size_t H = shape->hidden, E = shape->experts, K = shape->top_k;
    if (K == 0 || K > 64 || K > E || tokens == 0) return 0;
    int threads = config->threads > 0 ? config->threads : 1;
    synth_layer L;
    if (!synth_layer_dense(shape, config, layer, &L)) {
        synth_layer_free(&L);
        return 0;
    }
    uint16_t* hn = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    int32_t* sel = (int32_t*)malloc(tokens * K * sizeof(int32_t));
    uint16_t* sc = (uint16_t*)malloc(tokens * K * sizeof(uint16_t));
    uint16_t* lg = (uint16_t*)malloc(tokens * E * sizeof(uint16_t));
    uint16_t* o = (uint16_t*)malloc(tokens * H * sizeof(uint16_t));
    int ok = hn && sel && sc && lg && o;
    for (size_t t = 0; ok && t < tokens; ++t) {
        if (prenorm)
            fwo_rms_norm_bf16(hidden + t * H, H, config->bias_feature, hn + t * H);
        else
            memcpy(hn + t * H, hidden + t * H, H * sizeof(uint16_t));
        ok = fwo_route(L.router, hn + t * H, E, H, K, config->order, sel + t * K, lg + t * E, sc + t * K);
        for (size_t r = 0; ok && r < K; ++r) ok = synth_layer_expert(shape, config, layer, &L, sel[t * K + r]);
    }
    const int by_rows = threads > 1 && (long)tokens < threads && config->order == FWO_ORDER_TREE32;
    for (int run = 0; ok && run < warmups + runs; ++run) {
        double t0 = now_seconds();
        if (by_rows) {
            for (size_t t = 0; ok && t < tokens; ++t) {
                if (prenorm) fwo_rms_norm_bf16(hidden + t * H, H, config->bias_feature, hn + t * H);
                ok = block_rows_mt(shape, &L, hn + t * H, o + t * H, threads);
            }
        } else {
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1) reduction(&& : ok)
            for (long t = 0; t < (long)tokens; ++t) {
                if (prenorm) fwo_rms_norm_bf16(hidden + (size_t)t * H, H, config->bias_feature, hn + (size_t)t * H);
                ok = ok && block_core(shape, L.router, (const uint16_t* const*)L.gate_up,
                                      (const uint16_t* const*)L.down, L.shared_gate, L.shared_up, L.shared_down,
                                      L.shared_expert_gate, hn + (size_t)t * H, config->order, NULL, NULL,
                                      o + (size_t)t * H, NULL);
            }
        }
        double dt = now_seconds() - t0;
        if (run >= warmups && samples) samples[run - warmups] = dt;
    }
    if (ok && out) memcpy(out, o, tokens * H * sizeof(uint16_t));
    free(hn);
    free(sel);
    free(sc);
    free(lg);
    free(o);
    synth_layer_free(&L);
    return ok;
}
