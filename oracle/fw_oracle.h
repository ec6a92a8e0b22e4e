/*
 * CPU oracle for the sparse-MoE block hot path. TEST INFRASTRUCTURE ONLY: it is
 * the checker that the HIP library is compared against (tests, the smoke check
 * and bench.py's CPU-baseline leg); no product code calls it.
 *
 * A plain-C restatement of the reference crate's scalar Rust arithmetic
 * (src/expert.rs, src/router.rs, src/decoder_layer.rs, src/metal_moe.rs), built
 * with -O2 -ffp-contract=off and no fast-math so every f32 operation rounds
 * exactly where the Rust does. Transcendentals call glibc expf, which is what
 * Rust's f32::exp lowers to on Linux.
 *
 * Tie rule of top-k: total order on the bf16 logit (f32::total_cmp), value
 * descending then expert index ascending (src/router.rs:241-247), used for both
 * logit orders. The in-model path's libc++ nth_element tie order
 * (native/topk_shim.cpp:30-38, pinned only on macOS) is not reproducible here.
 *
 * bf16 values are uint16_t bit patterns; matrices are row-major.
 */
#ifndef FW_ORACLE_H
#define FW_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { FWO_ORDER_TREE32 = 0, FWO_ORDER_FOLD = 1 };

uint16_t fwo_to_bf16(float value);
float fwo_from_bf16(uint16_t value);
float fwo_expf(float x);
void fwo_expf_array(const float* in, float* out, size_t n);

float fwo_dot_tree32(const uint16_t* left, const uint16_t* right, size_t n);
float fwo_dot_fold(const uint16_t* weight, const uint16_t* input, size_t n);
void fwo_linear_bf16(const uint16_t* weight, const uint16_t* input, size_t rows, size_t columns,
                     uint16_t* out);
void fwo_linear_fold_bf16(const uint16_t* weight, const uint16_t* input, size_t rows,
                          size_t columns, uint16_t* out);
void fwo_swiglu_bf16(const uint16_t* gate, const uint16_t* up, size_t n, uint16_t* out);
uint16_t fwo_sigmoid_bf16(uint16_t value);
uint16_t fwo_add_bf16(uint16_t left, uint16_t right);
void fwo_build_silu_lut(uint16_t* lut);
void fwo_rms_norm_bf16(const uint16_t* r, size_t n, int bias_feature, uint16_t* h);
/* Hyper-connection (src/hyper_connection.rs) and the block's injection into
 * the residual streams (src/decoder_layer.rs:587-607). */
float fwo_inner_square_sum(const float* values, size_t n);
void fwo_grouped_rms(const uint16_t* input, const uint16_t* weight, size_t streams, size_t width,
                     float epsilon, uint16_t* out);
float fwo_stream_mean(const float* values, size_t streams);
typedef struct {
    uint16_t* hyper_input_normed; /* [S*W] */
    uint16_t* mix_down;           /* [R] */
    uint16_t* mix_down_scaled;    /* [R] */
    uint16_t* mix_down_silu;      /* [R] */
    uint16_t* mix_up;             /* [S*W] */
    uint16_t* input_mix;          /* [S*W] */
    uint16_t* products;           /* [S*W] */
    uint16_t* mixed;              /* [W] */
    uint16_t* inject;             /* [S] */
    uint16_t* inject_scaled;      /* [S] */
    uint16_t* inject_sigmoid;     /* [S] */
    uint16_t* injection_weights;  /* [S] */
} fwo_hyper_outputs;
int fwo_hyper_connection(const uint16_t* input, const uint16_t* hc_norm, const uint16_t* mix_down_w,
                         const uint16_t* mix_up_w, const uint16_t* inject_w, size_t streams, size_t width,
                         size_t lowrank, fwo_hyper_outputs* outputs);
void fwo_inject_residual(const uint16_t* post_attention, const uint16_t* moe_output,
                         const uint16_t* injection_weights, size_t streams, size_t width, uint16_t* products,
                         uint16_t* layer_output);
int fwo_make_hidden(size_t size, int64_t multiplier, int64_t add, int64_t modulus,
                    int64_t center, int64_t divisor, size_t sparse_stride, uint16_t* out);

int fwo_topk_total_order(const uint16_t* logits, size_t count, size_t k, int32_t* ids);
int fwo_route_scores(const uint16_t* logits, size_t experts, const int32_t* ids, size_t k,
                     uint16_t* scores);
int fwo_route(const uint16_t* weight, const uint16_t* hidden, size_t experts, size_t width,
              size_t top_k, int order, int32_t* ids, uint16_t* logits, uint16_t* scores);
int fwo_equivalent_topk_order(const int32_t* expected, const int32_t* actual, size_t k,
                              const uint16_t* logits);

void fwo_expert_bf16(const uint16_t* gate_up_weight, const uint16_t* down_weight,
                     const uint16_t* hidden, size_t hidden_size, size_t intermediate,
                     uint16_t route_weight, uint16_t* gate_up, uint16_t* swiglu, uint16_t* down,
                     uint16_t* weighted);
int fwo_mixture_bf16(const uint16_t* const* gate_up_weights, const uint16_t* const* down_weights,
                     const uint16_t* hidden, size_t hidden_size, size_t intermediate,
                     const int32_t* experts, const uint16_t* route_weights, size_t count,
                     uint16_t* mixture);

typedef struct {
    size_t hidden;
    size_t intermediate;
    size_t experts;
    size_t top_k;
    size_t shared_intermediate;
} fwo_shape;

typedef struct {
    const uint16_t* router;             /* [E, H] */
    const uint16_t* gate_up;            /* [E, 2I, H] */
    const uint16_t* down;               /* [E, H, I] */
    const uint16_t* shared_gate;        /* [Is, H] */
    const uint16_t* shared_up;          /* [Is, H] */
    const uint16_t* shared_down;        /* [H, Is] */
    const uint16_t* shared_expert_gate; /* [1, H] */
} fwo_layer;

typedef struct {
    uint16_t* logits;         /* [E] or NULL */
    int32_t* ids;             /* [K] rank order or NULL */
    uint16_t* scores;         /* [K] rank order or NULL */
    uint16_t* routed_mixture; /* [H] or NULL */
    uint16_t* shared_down;    /* [H] or NULL */
    uint16_t* shared_gate_sigmoid; /* [1] or NULL */
    uint16_t* shared_gate;    /* [Is] or NULL */
    uint16_t* shared_up;      /* [Is] or NULL */
    uint16_t* shared_swiglu;  /* [Is] or NULL */
    uint16_t* shared_gate_logit; /* [1] or NULL */
    uint16_t* gated_shared;   /* [H] or NULL */
    uint16_t* weighted_down;  /* [K, H] in execution (ascending id) order, or NULL */
} fwo_block_captures;

int fwo_sparse_moe_block(const fwo_shape* shape, const fwo_layer* layer, const uint16_t* hidden,
                         int order, uint16_t* out, fwo_block_captures* captures);

/* Synthetic workload (firewing_amd/csrc/fw_synth.h), regenerated on the CPU. */
void fwo_synth_tables(uint16_t* unit_table, uint16_t* weight_table);
void fwo_synth_hidden(uint64_t seed, uint32_t first_token, uint32_t tokens, uint32_t hidden,
                      int bias_feature, uint16_t* out);
void fwo_synth_tensor(uint64_t seed, uint32_t layer, uint32_t tensor, uint64_t first,
                      uint64_t count, uint16_t* out);
void fwo_synth_router_bias(uint64_t seed, uint32_t layer, uint32_t experts, uint16_t* bias);

typedef struct {
    uint64_t seed;
    int bias_feature;
    int order;
    int threads;
} fwo_synth_config;

int fwo_synth_block(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                    const uint16_t* hidden, size_t tokens, uint16_t* out, int32_t* ids,
                    uint16_t* scores, uint16_t* logits);
/* fwo_synth_block with every capture of the block, one captures record per
 * token (src/expert.rs:1154-1199, src/decoder_layer.rs:528-586 names). */
int fwo_synth_block_captured(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                             const uint16_t* hidden, size_t tokens, uint16_t* out,
                             fwo_block_captures* captures);
int fwo_synth_step(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layers,
                   const uint16_t* hidden, size_t tokens, uint16_t* residual_out,
                   uint16_t* block_out, int32_t* ids, uint16_t* scores);
int fwo_synth_step_timed(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layers,
                         const uint16_t* hidden, size_t tokens, uint16_t* residual_out,
                         double* compute_seconds);
int fwo_synth_route(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                    const uint16_t* hidden, size_t tokens, int32_t* ids, uint16_t* scores,
                    uint16_t* logits);
int fwo_bench_block(const fwo_shape* shape, const fwo_synth_config* config, uint32_t layer,
                    const uint16_t* hidden, size_t tokens, int prenorm, int warmups, int runs,
                    double* samples, uint16_t* out);

#ifdef __cplusplus
}
#endif

#endif /* FW_ORACLE_H */
