/*
 * firewing_hip_moe: MI355X (gfx950) sparse-MoE block hot path behind a C ABI.
 *
 * Conventions follow the reference crate's existing FFI,
 * `firewing_torch_topk_bf16` (src/decoder_layer.rs:19-26,
 * native/topk_shim.cpp:18-44): `firewing_` prefix, `bool` status, raw pointers
 * plus `size_t` counts, caller-owned outputs, bf16 as `uint16_t` bit patterns
 * (little-endian), matrices row-major in the reference's layouts:
 *   router [E, H], gate_up [E, 2I, H] (gate rows [0, I), up rows [I, 2I)),
 *   down [E, H, I], shared gate/up [Is, H], shared down [H, Is],
 *   shared_expert_gate [1, H]                     (src/expert.rs:362-512).
 * On `false`, firewing_hip_last_error() returns a thread-local message that the
 * Rust side turns into its `Err(String)`. No C++ exception crosses the ABI.
 *
 * Host-pointer entry points are synchronous, like the Metal command buffers
 * they replace (`wait_until_completed`, src/metal_moe.rs:351-358). `_dev`
 * entry points take device pointers and an optional stream (`hipStream_t`
 * passed as void*, NULL = the context's stream) and are asynchronous; their
 * errors surface at the next firewing_hip_synchronize().
 *
 * Arithmetic: every routed/shared expert and router output is bit-identical to
 * the reference's scalar CPU path (src/expert.rs:514-580, src/router.rs:220-265).
 * Top-k ties are broken by the total order of src/router.rs:241-247 (value
 * descending, expert index ascending) in both logit orders.
 */
#ifndef FIREWING_HIP_MOE_H
#define FIREWING_HIP_MOE_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Router logit order. TREE32: linear_bf16 logits, as the in-model block
 * computes them (src/decoder_layer.rs:411, src/expert.rs:554-560).
 * FOLD: one forward f32 fold per expert, as the standalone router
 * (src/router.rs:228-240). */
enum firewing_hip_logit_order {
    FIREWING_HIP_LOGITS_TREE32 = 0,
    FIREWING_HIP_LOGITS_FOLD = 1
};

/* Block shape. The reference's real model: H=2560, I=640, E=512, K=10,
 * Is=640, L=48 (src/metal_moe.rs:15-18, src/decoder_layer.rs:15,40-42). */
typedef struct firewing_hip_shape {
    size_t hidden;              /* H; multiple of 32 */
    size_t intermediate;        /* I; multiple of 32 */
    size_t experts;             /* E; <= 1024 */
    size_t top_k;               /* K; <= 32 */
    size_t shared_intermediate; /* Is; multiple of 32 */
    size_t layers;              /* L resident layers */
} firewing_hip_shape;

/* Optional per-call captures of the block, named as the reference's verifiers
 * name them (src/expert.rs:1154-1199 verify_sparse_moe_fixture,
 * src/decoder_layer.rs:460-586 require_capture). Every field may be NULL.
 * The fused decode kernel keeps the first five fields' values itself (except
 * routed_mixture); routed_mixture and the fields after shared_gate_sigmoid are
 * recomputed after the block by the standalone exact kernels on the same
 * resident weights and the same selection, a slower path taken only when one
 * of them is asked for. */
typedef struct firewing_hip_block_captures {
    uint16_t* router_logits;       /* [T, E] */
    size_t* selected_experts;      /* [T, K] rank order */
    uint16_t* selected_scores;     /* [T, K] rank order */
    uint16_t* routed_mixture;      /* [T, H] */
    uint16_t* shared_gate_sigmoid; /* [T] */
    uint16_t* shared_gate;         /* [T, Is] */
    uint16_t* shared_up;           /* [T, Is] */
    uint16_t* shared_swiglu;       /* [T, Is] */
    uint16_t* shared_down;         /* [T, H] */
    uint16_t* shared_gate_logit;   /* [T] */
    uint16_t* gated_shared;        /* [T, H]: bf16(shared_down * sigmoid) */
    uint16_t* weighted_down;       /* [T, K, H]: bf16(down * score) per selected expert, in
                                      execution (ascending id) order (src/decoder_layer.rs:532-579) */
} firewing_hip_block_captures;

typedef struct firewing_hip_context firewing_hip_context;

/* Thread-local message of the last failed call on this thread. */
const char* firewing_hip_last_error(void);

/* ---- stateless numeric entry points (host pointers, synchronous) -------- */

/* src/expert.rs:554-560 linear_bf16: out[r] = bf16(tree32 dot of W[r,:], x).
 * Also the Metal `firewing_bf16_gemv_exact` (kernels/bf16_gemv.metal:19-46,
 * src/metal_bf16.rs:101-147). */
bool firewing_hip_linear_bf16(const uint16_t* weight, const uint16_t* input, size_t rows,
                              size_t columns, uint16_t* out);

/* src/expert.rs:562-571 swiglu_bf16; kernels/bf16_gemv.metal:55-65. */
bool firewing_hip_swiglu_bf16(const uint16_t* gate, const uint16_t* up, size_t count,
                              uint16_t* out);

/* src/expert.rs:573-576 sigmoid_bf16, elementwise. */
bool firewing_hip_sigmoid_bf16(const uint16_t* input, size_t count, uint16_t* out);

/* Top-k of bf16 values: the GPU counterpart of `firewing_torch_topk_bf16`
 * (native/topk_shim.cpp:18-44) with the total-order tie rule. false for NULL,
 * k == 0, k > count, count > 1024 or k > 32. */
bool firewing_hip_topk_bf16(const uint16_t* values, size_t count, size_t k, size_t* indices);

/* src/router.rs:220-265 route (order FOLD) and src/decoder_layer.rs:278-307
 * (order TREE32) for T tokens: weight [E, H], hidden [T, H] -> ids [T, K]
 * (rank order), scores [T, K] bf16, logits [T, E] bf16 (NULL to skip). TREE32
 * rejects NaN logits (src/decoder_layer.rs:279-281). */
bool firewing_hip_route_bf16(const uint16_t* weight, const uint16_t* hidden, size_t tokens,
                             size_t experts, size_t width, size_t top_k, int order,
                             size_t* ids, uint16_t* scores, uint16_t* logits);

/* No counterpart in the reference: firewing_hip_route_bf16 for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc). Same arithmetic and arguments, but device pointers
 * (weight [E, H] 4-byte aligned, hidden [T, H], ids [T, K] int32 rank order,
 * scores [T, K], logits [T, E] or NULL) and an asynchronous launch on `stream`
 * (NULL: the null stream). No allocation: the logits, when `logits` is NULL,
 * live in a fixed 1 MiB scratch area of the library on each GPU, so then
 * tokens * experts <= 524288 (larger requests fail). A token whose TREE32
 * logits hold a NaN is rejected with all its ids set to -1. Calls that overlap
 * on one GPU share that scratch and race; order them on one stream. */
bool firewing_hip_route_bf16_noalloc(const uint16_t* weight, const uint16_t* hidden, size_t tokens,
                                     size_t experts, size_t width, size_t top_k, int order,
                                     int32_t* ids, uint16_t* scores, uint16_t* logits, void* stream);

/* One routed expert, src/expert.rs:717-751 (gate_up -> SwiGLU -> down ->
 * route weighting); replaces src/metal_bf16.rs:192-212 execute_expert.
 * gate_up_weight [2I, H], down_weight [H, I], hidden [H]; every capture may be
 * NULL: gate_up [2I], swiglu [I], down [H], weighted [H]. */
bool firewing_hip_expert_bf16(const uint16_t* gate_up_weight, const uint16_t* down_weight,
                              const uint16_t* hidden, size_t hidden_size,
                              size_t intermediate, uint16_t route_weight,
                              uint16_t* gate_up, uint16_t* swiglu, uint16_t* down,
                              uint16_t* weighted);

/* ---- resident context (replaces metal_moe::Runtime, src/metal_moe.rs:79-447) */

/* Allocates resident banks for `shape->layers` layers in HBM (~3.23 GB per
 * layer at H=2048, I=512, E=512), a stream and scratch. */
bool firewing_hip_create(const firewing_hip_shape* shape, firewing_hip_context** out);
void firewing_hip_destroy(firewing_hip_context* ctx);

/* Device name, as ExactResidentTop10Runner::device_name (src/metal_moe.rs:444-446). */
const char* firewing_hip_device_name(const firewing_hip_context* ctx);

/* Copy one layer's weights (host pointers, reference layouts) into HBM:
 * the install step of src/metal_moe.rs:164-207 for every expert of the layer. */
bool firewing_hip_install_layer(firewing_hip_context* ctx, size_t layer, const uint16_t* router,
                                const uint16_t* gate_up, const uint16_t* down,
                                const uint16_t* shared_gate, const uint16_t* shared_up,
                                const uint16_t* shared_down, const uint16_t* shared_expert_gate);

/* Where one of a layer's tensors lies in a safetensors checkpoint. */
typedef struct firewing_hip_tensor_span {
    uint64_t offset; /* absolute byte offset of the payload in its file */
    uint64_t bytes;  /* payload bytes */
    uint32_t shard;  /* ordinal of its file among the layer's files, in first-use order */
} firewing_hip_tensor_span;

/* Host only (no GPU needed): resolve and validate the seven tensors of one MoE
 * layer in a safetensors checkpoint. `path` is a single .safetensors file or a
 * model.safetensors.index.json (its weight_map names each tensor's shard, a
 * plain file name in the index's directory: src/checkpoint_catalog.rs:124-127,
 * 405-443). The tensors, all BF16 of exactly these shapes, are
 * "<layer_prefix>.mlp.gate.weight" [E, H], ".mlp.experts.gate_up_proj"
 * [E, 2I, H], ".mlp.experts.down_proj" [E, H, I],
 * ".mlp.shared_expert.gate_proj.weight" [Is, H], ".mlp.shared_expert.up_proj.weight"
 * [Is, H], ".mlp.shared_expert.down_proj.weight" [H, Is] and
 * ".mlp.shared_expert_gate.weight" [1, H] (src/decoder_layer1.rs:189-213,
 * src/expert_acquisition.rs:371-375;
 * layer_prefix e.g. "model.language_model.layers.0"). Each shard's header is
 * checked as src/checkpoint_catalog.rs:146-245 checks it (header length in
 * (0, 16 MiB], known dtypes, payload sizes exact and inside the file, no
 * overlaps). spans[7] receive the tensors in that order; false with the
 * reason in firewing_hip_last_error() otherwise. */
bool firewing_hip_safetensors_layer_plan(const firewing_hip_shape* shape, const char* path,
                                         const char* layer_prefix, firewing_hip_tensor_span* spans);

/* Load one layer's resident banks straight from a safetensors checkpoint (the
 * plan above against the context's shape, then every payload streamed into
 * HBM through pinned staging buffers, file reads overlapping the copies).
 * Replaces the reference's per-call slice readers read_expert_slice /
 * read_tensor_2d (src/expert.rs:362-512) and the mapped catalog's
 * expert_bf16 view (src/checkpoint_catalog.rs:416-443) with one copy per layer
 * at install time. Synchronous; nothing is copied if any tensor fails the plan. */
bool firewing_hip_load_layer_safetensors(firewing_hip_context* ctx, size_t layer, const char* path,
                                         const char* layer_prefix);

/* Fill layers [first, first+count) on the device with the seeded synthetic
 * weights (firewing_amd/csrc/fw_synth.h); bias_feature writes the Zipf router
 * bias into router column H-1. */
bool firewing_hip_generate_layers(firewing_hip_context* ctx, size_t first, size_t count,
                                  uint64_t seed, bool bias_feature);

/* Read back `count` elements from element `first` of one resident tensor
 * (tensor ids as fw_synth.h: 1 router, 2 gate_up, 3 down, 4 shared_gate,
 * 5 shared_up, 6 shared_down, 7 shared_expert_gate), for verification. */
bool firewing_hip_read_tensor(firewing_hip_context* ctx, size_t layer, int tensor,
                              size_t first, size_t count, uint16_t* out);

/* Route T tokens against a resident layer's router (as firewing_hip_route_bf16). */
bool firewing_hip_route(firewing_hip_context* ctx, size_t layer, const uint16_t* hidden,
                        size_t tokens, int order, size_t* ids, uint16_t* scores,
                        uint16_t* logits);

/* The ordered top-k mixture on a resident layer for one hidden vector, given
 * the experts in execution (ascending id) order and their bf16 route weights:
 * src/expert.rs:906-956; replaces execute_one_transaction + capture_mixture
 * (src/metal_moe.rs:310-383). */
bool firewing_hip_mixture_bf16(firewing_hip_context* ctx, size_t layer, const uint16_t* hidden,
                               const size_t* experts, const uint16_t* route_weights,
                               size_t count, uint16_t* mixture);

/* One sparse-MoE block for T <= 4 tokens (decode and MTP verify): router,
 * top-k, routed experts, ordered mixture, shared expert and gate, combine
 * (src/decoder_layer.rs:460-586; src/expert.rs:1109-1153). */
bool firewing_hip_sparse_moe_block(firewing_hip_context* ctx, size_t layer,
                                   const uint16_t* hidden, size_t tokens, int order,
                                   uint16_t* out, firewing_hip_block_captures* captures);

/* Device-pointer variant; hidden [T, H] (4-byte aligned), out [T, H] in HBM. */
bool firewing_hip_sparse_moe_block_dev(firewing_hip_context* ctx, size_t layer,
                                       const uint16_t* hidden, size_t tokens, int order,
                                       uint16_t* out, void* stream);

/* One sparse-MoE block for many tokens (prefill, T in [1, 65536]) on a
 * resident layer: the same block as firewing_hip_sparse_moe_block
 * (src/decoder_layer.rs:460-586 with the in-model TREE32 logits; the reference
 * runs it token by token), arranged for MFMA: exact router logits, top-k and
 * scores (bit-exact: src/decoder_layer.rs:278-322), (token, expert) pairs
 * grouped by expert, grouped bf16 GEMMs for gate/up (+ SwiGLU) and down
 * (+ route weight), the shared expert as one more group, and the
 * ascending-id bf16 combine (src/expert.rs:906-956). The expert GEMMs
 * accumulate in the matrix units' order, so block outputs match the reference
 * within a bf16 tolerance rather than bit for bit. Host buffers, synchronous;
 * captures: router_logits, selected_experts, selected_scores, routed_mixture
 * (the MFMA path's, within the same tolerance) and shared_gate_sigmoid; the
 * other fields must be NULL. */
bool firewing_hip_prefill_block(firewing_hip_context* ctx, size_t layer, const uint16_t* hidden,
                                size_t tokens, uint16_t* out, firewing_hip_block_captures* captures);

/* Device-pointer variant: hidden [T, H] and out [T, H] in HBM (16-byte
 * aligned); ids [T, K] (int32, rank order) and scores [T, K] may be NULL. */
bool firewing_hip_prefill_block_dev(firewing_hip_context* ctx, size_t layer, const uint16_t* hidden,
                                    size_t tokens, uint16_t* out, int32_t* ids, uint16_t* scores,
                                    void* stream);

/* No counterpart in the reference: a measurement aid. The block of
 * firewing_hip_prefill_block_dev, queued on `stream` with HIP events between
 * its phases and waited for; phase_us[0..5] (phases == 6) receive the
 * microseconds of the router logits, the selection (top-k and scores), the
 * grouping of (token, expert) pairs, the gate/up GEMM, the down GEMM and the
 * ordered combine. */
bool firewing_hip_prefill_block_profile(firewing_hip_context* ctx, size_t layer, const uint16_t* hidden,
                                        size_t tokens, uint16_t* out, void* stream, double* phase_us,
                                        size_t phases);

/* All resident layers for T <= 4 tokens in one persistent launch: the
 * 48-layer decode step the overlap benches emulate with 48 execute_exact()
 * calls (src/overlap_bound.rs:732-734). Layers are chained by a pre-norm
 * residual stream, r_0 = hidden, h_l = rms_norm(r_l) (h_l[H-1] = 1.0 when
 * bias_feature), r_{l+1} = add_bf16(r_l, block_l(h_l)), where rms_norm is
 * bf16(r / sqrt(dot(r, r) / H + 1e-6)) with the reference's dot order; this
 * glue stands in for the rest of the decoder layer, which is not built here.
 * Device pointers (hidden and residual 4-byte aligned): hidden [T, H] in,
 * residual r_L [T, H] out; block_out
 * [L, T, H], ids [L, T, K] (int32) and scores [L, T, K] may be NULL. */
bool firewing_hip_moe_step_dev(firewing_hip_context* ctx, const uint16_t* hidden, size_t tokens,
                               int order, bool bias_feature, uint16_t* residual,
                               uint16_t* block_out, int32_t* ids, uint16_t* scores,
                               void* stream);

/* Host-pointer variant of the step (synchronous). */
bool firewing_hip_moe_step(firewing_hip_context* ctx, const uint16_t* hidden, size_t tokens,
                           int order, bool bias_feature, uint16_t* residual,
                           uint16_t* block_out, int32_t* ids, uint16_t* scores);

/* Waits for the context's stream and reports any device-side failure
 * (a persistent-kernel dependency wait that timed out). */
bool firewing_hip_synchronize(firewing_hip_context* ctx);

/* Time limit of each dependency wait inside the persistent kernel, in seconds
 * (0 < seconds <= 600; default 10, or FIREWING_WAIT_TIMEOUT_S at create). A
 * wait that exceeds it ends the launch with the timeout error; the next launch
 * starts clean. No counterpart in the reference (the Metal path waits on
 * command-buffer completion, src/metal_moe.rs:351-358). */
bool firewing_hip_set_wait_timeout(firewing_hip_context* ctx, double seconds);

/* ---- hyper-connection around the block (src/hyper_connection.rs) ------- */

/* Every output of run_hyper_connection (src/hyper_connection.rs:333-346,
 * 412-490) for T tokens of S streams of width W with low rank R; each field
 * may be NULL. */
typedef struct firewing_hip_hyper_outputs {
    uint16_t* hyper_input_normed; /* [T, S*W] grouped_rms(input, hc_norm) */
    uint16_t* mix_down;           /* [T, R] */
    uint16_t* mix_down_scaled;    /* [T, R] bf16(mix_down / S) */
    uint16_t* mix_down_silu;      /* [T, R] */
    uint16_t* mix_up;             /* [T, S*W] */
    uint16_t* input_mix;          /* [T, S*W] sigmoid(mix_up) */
    uint16_t* products;           /* [T, S*W] bf16(input_mix * normed) */
    uint16_t* mixed;              /* [T, W] four-stream mean: the block's input */
    uint16_t* inject;             /* [T, S] */
    uint16_t* inject_scaled;      /* [T, S] bf16(inject / S) */
    uint16_t* inject_sigmoid;     /* [T, S] */
    uint16_t* injection_weights;  /* [T, S] bf16(2 * inject_sigmoid) */
} firewing_hip_hyper_outputs;

/* run_hyper_connection (src/hyper_connection.rs:412-490) for T tokens:
 * input [T, S*W], hc_norm [S*W], mix_down_weight [R, S*W], mix_up_weight
 * [S*W, R], inject_weight [S, S*W] (NULL: run_final_mixer,
 * src/hyper_connection.rs:359-410, without the injection outputs). The
 * grouped RMS norm sums squares in PyTorch's aarch64 cascade
 * (src/hyper_connection.rs:211-303); the projections are linear_bf16.
 * S <= 64, S*W and R even and <= 16384. Host pointers, synchronous. */
bool firewing_hip_hyper_connection_bf16(const uint16_t* input, size_t tokens, const uint16_t* hc_norm,
                                        const uint16_t* mix_down_weight, const uint16_t* mix_up_weight,
                                        const uint16_t* inject_weight, size_t streams, size_t width,
                                        size_t lowrank, firewing_hip_hyper_outputs* outputs);

/* The block output injected into the residual streams
 * (src/decoder_layer.rs:587-607): products[t][s][h] = bf16(moe[t][h] *
 * weights[t][s]) (products may be NULL), layer_output[t][s][h] =
 * add_bf16(post_attention[t][s][h], products[t][s][h]). */
bool firewing_hip_inject_residual_bf16(const uint16_t* post_attention, const uint16_t* moe_output,
                                       const uint16_t* injection_weights, size_t tokens, size_t streams,
                                       size_t width, uint16_t* products, uint16_t* layer_output);

/* Install one layer's mlp hyper-connection on the context (width = H; the
 * same streams and lowrank for every layer): hc_norm [S*H], mix_down [R, S*H],
 * mix_up [S*H, R], inject [S, S*H] (the reference's
 * mlp_hyper_connection.{hc_norm, input_mix_weight_down, input_mix_weight_up,
 * block_inject_weight}, src/decoder_layer.rs:191-216). */
bool firewing_hip_install_hyper_connection(firewing_hip_context* ctx, size_t layer, size_t streams,
                                           size_t lowrank, const uint16_t* hc_norm,
                                           const uint16_t* mix_down_weight, const uint16_t* mix_up_weight,
                                           const uint16_t* inject_weight);

/* The same from a safetensors checkpoint ("<layer_prefix>.mlp_hyper_connection.
 * {hc_norm, input_mix_weight_down, input_mix_weight_up, block_inject_weight}.weight",
 * BF16, src/decoder_layer1.rs:168-185), validated as
 * firewing_hip_safetensors_layer_plan validates. */
bool firewing_hip_load_hyper_connection_safetensors(firewing_hip_context* ctx, size_t layer, size_t streams,
                                                    size_t lowrank, const char* path,
                                                    const char* layer_prefix);

/* Captures of the in-model MoE sublayer (src/decoder_layer.rs:451-607). */
typedef struct firewing_hip_sublayer_captures {
    firewing_hip_hyper_outputs hyper;   /* mixed = mlp_input, injection_weights = mlp_injection_weights */
    firewing_hip_block_captures block;  /* of the block on mlp_input */
    uint16_t* moe_output;               /* [T, H] */
    uint16_t* mlp_injection_products;   /* [T, S*H] */
} firewing_hip_sublayer_captures;

/* The in-model MoE sublayer for T <= 4 tokens (src/decoder_layer.rs:451-607):
 * the layer's mlp hyper-connection on the S residual streams post_attention
 * [T, S*H], the sparse-MoE block on its mixed input (logit order `order`),
 * and the block output injected into the streams: layer_output [T, S*H].
 * Host pointers, synchronous; captures may be NULL. */
bool firewing_hip_moe_sublayer(firewing_hip_context* ctx, size_t layer, const uint16_t* post_attention,
                               size_t tokens, int order, uint16_t* layer_output,
                               firewing_hip_sublayer_captures* captures);

/* Device-pointer variant (4-byte aligned), queued on `stream`. */
bool firewing_hip_moe_sublayer_dev(firewing_hip_context* ctx, size_t layer, const uint16_t* post_attention,
                                   size_t tokens, int order, uint16_t* layer_output, void* stream);

/* ---- LM head (src/text_output.rs:204-317) ----------------------------- */

/* Install the LM head [vocab][H] (host pointer) on the context, replacing any
 * earlier head; the head of the reference model is 248,320 x 2560. */
bool firewing_hip_install_lm_head(firewing_hip_context* ctx, const uint16_t* weight, size_t vocab);

/* The seeded synthetic head (bf16(N(0, 0.02)), firewing_amd/csrc/fw_synth.h
 * tensor 10), generated on the device. No counterpart in the reference. */
bool firewing_hip_generate_lm_head(firewing_hip_context* ctx, size_t vocab, uint64_t seed);

/* The head from a safetensors checkpoint: tensor `tensor` (e.g. "lm_head.weight"),
 * BF16 [vocab, H], validated as firewing_hip_safetensors_layer_plan validates. */
bool firewing_hip_load_lm_head_safetensors(firewing_hip_context* ctx, const char* path, const char* tensor,
                                           size_t vocab);

/* logits = linear_bf16(lm_head, hidden) for T <= 4 tokens (hidden [T, H], the
 * final mixer's mixed output) and their top-k, k <= 64: ids [T, k] and values
 * [T, k] in rank order (src/text_output.rs:273-287; the ranking of
 * pytorch_topk_bf16, src/decoder_layer.rs:28-39, with ties broken by the lower
 * index; ceil(vocab / 4096) * k <= 8192). logits [T, vocab] may be NULL.
 * Host pointers, synchronous. */
bool firewing_hip_lm_head(firewing_hip_context* ctx, const uint16_t* hidden, size_t tokens, size_t k,
                          uint16_t* logits, size_t* ids, uint16_t* values);

/* Device-pointer variant (hidden 4-byte aligned; ids int32), queued on
 * `stream`; logits may be NULL. */
bool firewing_hip_lm_head_dev(firewing_hip_context* ctx, const uint16_t* hidden, size_t tokens, size_t k,
                              uint16_t* logits, int32_t* ids, uint16_t* values, void* stream);

/* No counterpart in the reference: how a step of `tokens` (<= 4) tokens runs
 * on this context: the number of independent one-token chains it interleaves
 * by layer (= tokens where the fused one-token path applies at the context's
 * shape: the chains' serial steps overlap), or 1 for the multi-token kernel
 * (each union expert's rows read once for all its tokens). Results are the
 * same either way. 0 for a null context. */
size_t firewing_hip_token_chains(const firewing_hip_context* ctx, size_t tokens);

/* ---- compressed expert container (src/compressed_overlap.rs) ----
 *
 * The container holds one independent zstd frame (RFC 8878; the reference
 * decodes with the zstd crate 0.13.3 = libzstd 1.5.7) per expert: the
 * expert's source bytes, gate_up [2I, H] then down [H, I] (bf16, 6*I*H bytes;
 * tools/build_sequential_shuffle_container.py), BF16 byte-shuffled (every low
 * byte, then every high byte). The reference reads a frame, decompresses it
 * into a buffer, checks the decoded size against EXPERT_BYTES, undoes the
 * shuffle and copies it into the install buffer
 * (src/compressed_overlap.rs:1426-1560 run_executable_trial,
 * src/compressed_overlap.rs:1385-1395 unshuffle_bf16). Here the frames are
 * decoded on the GPU straight into their destinations with the shuffle
 * undone on the way.
 *
 * Supported: frames of at most 2^27 - 1 decoded bytes with or without a
 * content-size field, raw / RLE / compressed blocks, every literal and
 * sequence table mode. Not supported (the frame fails): dictionaries,
 * skippable frames, bytes after the frame, more than content/1024 + 64
 * blocks. A content checksum is skipped, not verified (the container's
 * frames carry none). */
typedef struct firewing_hip_zstd_decoder firewing_hip_zstd_decoder;

/* One frame of a decode call. Decoded bytes [0, split) go to dst and
 * [split, content_bytes) to dst_tail (device pointers; dst_tail may be NULL
 * when split == content_bytes). With the BF16 unshuffle the bytes are those
 * after the shuffle is undone. */
typedef struct firewing_hip_zstd_frame {
    uint64_t src_offset;    /* the frame's first byte in the call's source buffer */
    uint64_t src_bytes;     /* its compressed size: exactly one frame */
    uint64_t content_bytes; /* the decoded size the caller expects (the reference's EXPERT_BYTES check) */
    void* dst;
    void* dst_tail;
    uint64_t split;
} firewing_hip_zstd_frame;

/* Per-frame status codes (firewing_hip_zstd_decode's status array). */
enum firewing_hip_zstd_status {
    FIREWING_HIP_ZSTD_OK = 0,
    FIREWING_HIP_ZSTD_BAD_MAGIC = 1,
    FIREWING_HIP_ZSTD_BAD_FRAME_HEADER = 2,
    FIREWING_HIP_ZSTD_TRUNCATED = 3,
    FIREWING_HIP_ZSTD_BAD_BLOCK = 4,
    FIREWING_HIP_ZSTD_TOO_MANY_BLOCKS = 5,
    FIREWING_HIP_ZSTD_BAD_LITERALS = 6,
    FIREWING_HIP_ZSTD_BAD_HUFFMAN = 7,
    FIREWING_HIP_ZSTD_BAD_FSE = 8,
    FIREWING_HIP_ZSTD_BAD_SEQUENCES = 9,
    FIREWING_HIP_ZSTD_BAD_OFFSET = 10,
    FIREWING_HIP_ZSTD_CONTENT_SIZE = 11,
    FIREWING_HIP_ZSTD_SCRATCH = 12,
    FIREWING_HIP_ZSTD_TRAILING = 13
};

/* A decoder on GPU `device` with scratch for `max_frames` frames in flight of
 * at most `max_content_bytes` decoded bytes each (about 4 bytes of scratch
 * per decoded byte: 9.8 MB experts take ~40 MB a frame). Calls with more
 * frames run in chunks of max_frames. Decoders are independent of
 * contexts: one can decode on its own stream while a context's step runs on
 * another. NULL on failure (see firewing_hip_last_error). No counterpart in
 * the reference, whose workers each own a zstd::bulk::Decompressor
 * (src/compressed_overlap.rs:1494-1505). */
firewing_hip_zstd_decoder* firewing_hip_zstd_create(int device, size_t max_frames, size_t max_content_bytes);
void firewing_hip_zstd_destroy(firewing_hip_zstd_decoder* dec);

/* Decode `n` frames whose bytes are in host memory `src` [src_bytes] (staged
 * through pinned memory) into device destinations; synchronous. status [n]
 * (may be NULL) receives each frame's firewing_hip_zstd_status. Returns false
 * if any frame failed (the message names the first) or on a usage error.
 * Replaces decompress_to_buffer + the decoded-size check + unshuffle_bf16
 * (src/compressed_overlap.rs:1541-1553) for a batch of frames. */
bool firewing_hip_zstd_decode(firewing_hip_zstd_decoder* dec, const uint8_t* src, size_t src_bytes,
                              const firewing_hip_zstd_frame* frames, size_t n, bool bf16_unshuffle,
                              uint32_t* status);

/* Device-source variant: `src` is a device buffer; queued on `stream` (NULL =
 * the null stream) after the decoder's previous call, asynchronous. Per-frame
 * statuses are read with firewing_hip_zstd_status. The decoder reads no byte
 * outside the frames. */
bool firewing_hip_zstd_decode_dev(firewing_hip_zstd_decoder* dec, const uint8_t* src, size_t src_bytes,
                                  const firewing_hip_zstd_frame* frames, size_t n, bool bf16_unshuffle,
                                  void* stream);

/* Wait for the decoder's last call and copy its per-frame statuses (status
 * [n], n = that call's frame count; may be NULL). False if any frame failed. */
bool firewing_hip_zstd_status(firewing_hip_zstd_decoder* dec, uint32_t* status, size_t n);

/* Install `n` experts of `layer` from their container frames: frame i (host
 * bytes src[offsets[i], offsets[i] + sizes[i])) decodes, unshuffled, into
 * expert experts[i]'s resident gate_up and down rows. Synchronous, ordered
 * with the context's other work. The install step of the overlap benches
 * (src/compressed_overlap.rs:1547-1553 unshuffle_bf16 + install copy) into
 * the banks a step reads (ExactResidentTop10Runner, src/metal_moe.rs:404-470). */
bool firewing_hip_install_experts_zstd(firewing_hip_context* ctx, firewing_hip_zstd_decoder* dec, size_t layer,
                                       const uint32_t* experts, size_t n, const uint8_t* src, size_t src_bytes,
                                       const uint64_t* offsets, const uint64_t* sizes);

/* Seeded synthetic hidden vectors of the benchmark workload (host memory):
 * bf16(N(0,1)) RMS-normalised, x[H-1] = 1.0 when bias_feature (the constant
 * feature that carries the Zipf router bias). No counterpart in the reference,
 * whose inputs come from make_hidden (src/expert.rs:341-360). */
void firewing_hip_synth_hidden(uint64_t seed, uint32_t first_token, uint32_t tokens,
                               uint32_t hidden, bool bias_feature, uint16_t* out);

/* Host-side copy of the library's expf (the glibc-equivalent table method the
 * kernels use), for verification against the platform libm. */
void firewing_hip_expf_host(const float* in, float* out, size_t count);

/* Device evaluation of the same expf, for verification (synchronous). */
bool firewing_hip_expf_device(const float* in, float* out, size_t count);

/* Plain device-to-device copy of `bytes` (a multiple of 16) with a streaming
 * kernel (k_copy_bytes), queued on `stream` (0: the default stream). A
 * measurement aid with no counterpart in the reference: the bytes it moves are
 * known exactly, so hardware traffic counters read over it calibrate the
 * decode kernel's counts. */
bool firewing_hip_copy_bytes(void* dst, const void* src, size_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FIREWING_HIP_MOE_H */
