// Persistent decode kernel: every resident layer of a T <= 4 token step in one
// launch (router -> top-k -> routed and shared SwiGLU experts -> ordered
// mixture -> combine, chained through the residual stream).
//
// The co-resident workgroups (cooperative launch) are split into two roles,
// each walking its own task list in (layer, phase) order (B tasks beyond one
// per rows workgroup run on the combine role, ahead of its C tasks):
//
//   rows     R  router rows, 16 per task (rows [0, E)), plus one task for the
//               shared_expert_gate row                  -> logits
//            S  shared gate/up pairs, 8 per task, fused SwiGLU -> shared_act
//            B  routed gate/up pairs, 8 per task of one selected expert
//               ("slot"), fused SwiGLU                 -> act
//   combine  C  4 hidden rows per task: the down rows of the shared expert and
//               of every slot, route weighting, the ascending-id bf16 mixture,
//               the gated shared output, the block output and the next
//               residual                                -> out, residual
//
// Expert selection (top-k, the union of the tokens' experts in ascending id,
// scores, the shared-gate sigmoid) is recomputed from the logits by every B
// and C workgroup that needs it: a few microseconds of LDS work instead of a
// further hop through memory.
//
// R and S of layer l wait for C of layer l-1; B and C for R; C also for B and
// S. Every wait points to an earlier phase, and within a role earlier phases
// come first, so with all workgroups resident the earliest unfinished task can
// always run. Weight loads never depend on activations, so tasks issue them
// before they wait: R and S stream their rows while the previous layer
// finishes, C its shared down rows at once and its routed down rows as soon as
// the selection is known, while B runs. Phase counters and tagged data words
// follow fw_device.h; every wait is bounded by a wall-clock limit and by a
// shared error word, so a failure ends the launch instead of hanging it. The
// last workgroup to finish zeroes the counters for the next launch.
#pragma once

#include "fw_device.h"

namespace fw {

struct DecodeLayer {
    const uint16_t* router;       // [E + 1][H]; row E is shared_expert_gate
    const uint16_t* gate_up;      // [E][2I][H]
    const uint16_t* down;         // [E][H][I]
    const uint16_t* shared_gate;  // [Is][H]
    const uint16_t* shared_up;    // [Is][H], = shared_gate + Is * H
    const uint16_t* shared_down;  // [H][Is]
};

enum DecodeCounter : int {
    kCntRouter = 0,
    kCntGateUp = 1,  // S and B tasks
    kCntC = 2,
    kCountersPerLayer = 3
};

enum DecodeTaskKind : int { kTaskRouter = 0, kTaskShared = 1, kTaskGateUp = 3, kTaskDown = 4 };

constexpr int kRouterRowsPerTask = 16;
constexpr int kPairsPerTask = 8;
constexpr int kRowsPerCTask = 4;
constexpr int kMaxTokens = 4;
constexpr int kMaxTopK = 32;
constexpr int kMaxSlots = kMaxTopK * kMaxTokens;
constexpr int kMaxHidden = 2560;
constexpr int kMaxExperts = 1024;
constexpr int kThreads = 256;
constexpr int kXWords = kMaxHidden / 2 / kThreads;  // residual words per thread and token

// Row stride of the logit words: the E router logits padded to an even count,
// then the shared_expert_gate logit and a zero.
__host__ __device__ constexpr int logit_stride(int E) { return ((E + 1) & ~1) + 2; }

struct DecodeParams {
    const DecodeLayer* layers;  // [nlayers], already offset to the first layer
    int nlayers;
    int T, H, I, E, K, Is;
    int order;         // 0 TREE32, 1 FOLD
    int prenorm;       // block input = rms_norm(residual) (chained step), else the input
    int bias_feature;  // with prenorm: block input [H-1] = 1.0
    int ls, gi;        // logit row stride (even) and shared_expert_gate index (even)
    const uint16_t* x_in;  // [chains][T][H] input of the first layer of each chain
    // tagged words (payload = two bf16, or one bf16 in the low half)
    uint64_t* xw;          // [nlayers + chains][T][H / 2] residual stream (indices < chains unused)
    uint64_t* logits;      // [nlayers][T][ls / 2]
    uint64_t* shared_act;  // [nlayers][T][Is / 2]
    uint64_t* act;         // [nlayers][S][T][I / 2]
    // plain outputs, read after the launch
    uint16_t* x_final;  // [chains][T][H] residual after the last layer of each chain, or null
    uint16_t* out;      // [nlayers][T][H] block outputs
    int32_t* ids;       // [nlayers][T][K] rank order
    uint16_t* scores;   // [nlayers][T][K]
    uint16_t* sig;      // [nlayers][T] sigmoid of the shared_expert_gate logit
    uint32_t* counters;  // [nlayers][kCountersPerLayer] counter groups, then the done group
    uint32_t* flags;     // [nlayers][kCountersPerLayer][kFlagCopies * kFlagStride] epoch of the completed phase
    int32_t* error;      // 0 ok, 1 timeout, 2 NaN router logit
    uint64_t limit_ticks;
    int n_router, n_shared, n_b, n_c, S;  // tasks per layer; slots
    int nb_rows;                          // B tasks per layer on the rows role (the rest on combine)
    int g_rows, g_comb;                   // workgroups of the rows and combine roles
    int cpairs;                           // > 0: gate/up pairs past the rows role's B tasks, carried
                                          // by wave 0 of each C task (one token); 0: B tasks on combine
    int n_gu;                             // tasks counted in the gate/up phase
    int cu_count;                         // compute units (workgroup b sits on the CU of b mod cu_count)
    int input_by_tags;                    // router tasks await their block input by its words' tags
                                          // alone (no combine phase flag)
    int rank_slots;                       // one token: slot s is the rank-s expert (B tasks run the
                                          // top-k only up to their own rank), not the s-th smallest id
    int chains;                           // independent token chains interleaved by layer: layer li
                                          // continues layer li - chains (1: consecutive layers)
    uint64_t* trace;     // profiling builds only
};

// A launch runs `chains` independent token chains interleaved by layer: layer
// li of the launch continues layer li - chains of the same chain, and the
// first `chains` layers read the caller's input (chain li at row li of x_in).
// With one chain that is the ordinary sequence of layers.
__device__ __forceinline__ bool chain_start(const DecodeParams& p, int li) { return li < p.chains; }
__device__ __forceinline__ int chain_prev(const DecodeParams& p, int li) { return li - p.chains; }
// this layer's input words ([T][H / 2]) when chain_start
__device__ __forceinline__ const uint32_t* chain_input(const DecodeParams& p, int li) {
    return reinterpret_cast<const uint32_t*>(p.x_in) + (size_t)li * p.T * p.H / 2;
}

// Task timing (wall clock) for profiling builds only (slots: trace_slot).
#ifdef FW_DECODE_TRACE
constexpr int kTraceWords = 18;  // start, dependency met, end, wg << 8 | kind, 12 stage marks, 2 cycle counts
#define FW_TRACE_STAMP(var)                  \
    const uint64_t var = wall_clock64();     \
    const uint64_t var##_cycles = clock64(); \
    (void)var##_cycles
#define FW_TRACE_MARK(slot_, k)                                                    \
    do {                                                                           \
        if (threadIdx.x == 0 && p.trace != nullptr && (slot_) >= 0)                \
            p.trace[(size_t)(slot_) * kTraceWords + 4 + (k)] = wall_clock64();     \
    } while (0)
#define FW_TRACE_MARK_IF(cond_, slot_, k)                                          \
    do {                                                                           \
        if ((cond_) && p.trace != nullptr && (slot_) >= 0)                         \
            p.trace[(size_t)(slot_) * kTraceWords + 4 + (k)] = wall_clock64();     \
    } while (0)
#define FW_TRACE_VALUE(slot_, k, v)                                                \
    do {                                                                           \
        if (threadIdx.x == 0 && p.trace != nullptr && (slot_) >= 0)                \
            p.trace[(size_t)(slot_) * kTraceWords + 4 + (k)] = (uint64_t)(v);      \
    } while (0)
#define FW_TRACE_WRITE(slot_, kind, a, b, c)                                       \
    do {                                                                           \
        if (threadIdx.x == 0 && p.trace != nullptr && (slot_) >= 0) {              \
            uint64_t* tr = p.trace + (size_t)(slot_) * kTraceWords;                \
            tr[0] = (a);                                                           \
            tr[1] = (b);                                                           \
            tr[2] = (c);                                                           \
            tr[3] = ((uint64_t)blockIdx.x << 8) | (uint64_t)(kind);                \
            tr[16] = a##_cycles;                                                   \
            tr[17] = c##_cycles;                                                   \
        }                                                                          \
    } while (0)
#else
#define FW_TRACE_STAMP(var)
#define FW_TRACE_MARK(slot_, k)
#define FW_TRACE_MARK_IF(cond_, slot_, k)
#define FW_TRACE_VALUE(slot_, k, v)
#define FW_TRACE_WRITE(slot_, kind, a, b, c)
#endif

// 2^(i/32) as f64 bits (the expf table); one copy per translation unit.
static __device__ __constant__ uint64_t c_exp2_table[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

constexpr int kBatchMatrices = 16;  // C task: matrices per register batch (4 per wave)

// Words of the LDS area that holds the block input (rows role) or the staged
// activation vectors (combine role): the block input of NT tokens, and the
// vectors of a whole batch for NT tokens where that fits 32 KiB.
// One token with MBI <= 16 (the fused C task) also holds, above the block
// input and the exponentials, the four gate/up rows of its pairs, and later
// the tagged words of twelve activation vectors.
constexpr int kDirectVectors = 12;
constexpr int kBRowsAt = kMaxHidden + kMaxExperts;  // words
// words between the four gate/up rows: 64 bytes past a row, so the four lane
// groups reading the same line offset of their rows hit different LDS banks
constexpr int kBRowStride = kMaxHidden / 2 + 16;
constexpr int kFusedWords = kBRowsAt + 4 * kBRowStride > kDirectVectors * 16 * 16 * 2 ? kBRowsAt + 4 * kBRowStride
                                                                                       : kDirectVectors * 16 * 16 * 2;
__host__ __device__ constexpr int stage_words(int NT, int MBI) {
    return (NT == 1 && MBI <= 20) ? kFusedWords
           : NT * kMaxHidden > (kBatchMatrices * NT * MBI * 16 < 8192 ? kBatchMatrices * NT * MBI * 16 : 8192)
               ? NT * kMaxHidden
               : (kBatchMatrices * NT * MBI * 16 < 8192 ? kBatchMatrices * NT * MBI * 16 : 8192);
}
// Matrices staged at once (a multiple of 4, so whole waves' matrices): as many
// of a batch as the area holds for NT tokens each.
__host__ __device__ constexpr int stage_matrices(int NT, int MBI) {
    return stage_words(NT, MBI) / (NT * MBI * 16) >= 16 ? 16 : (stage_words(NT, MBI) / (NT * MBI * 16) >= 8 ? 8 : 4);
}

template <int NT, int MBI>
struct DecodeShared {
    // rows: block input as f32; combine: exponentials, then staged
    // activation vectors
    alignas(16) float xs[stage_words(NT, MBI)];
    uint16_t lg[NT * logit_stride(kMaxExperts)];  // logits of the selected layer
    uint64_t exp2tab[32];
    uint16_t res[(kMaxTopK * NT + 1) * NT * kRowsPerCTask];  // down-row dots [matrix][token][row]
    int32_t ids[NT * kMaxTopK];                               // rank order per token
    int32_t sorted[kMaxTopK * NT];                            // union, ascending id
    uint32_t slot_tokens[kMaxTopK * NT];
    int32_t tslot[NT * kMaxTopK];     // [t][k]: slot of the token's k-th expert in ascending id
    int32_t pos[NT * kMaxTopK];       // [t][r]: ascending-id position of the token's rank-r expert
    int32_t rank_at[kMaxTopK];        // one token: rank of the expert at ascending-id position k
    uint16_t tweight[NT * kMaxTopK];  // [t][k]: its bf16 score
    uint16_t sig[NT];
    float inv[NT];
    int32_t vbase[kBatchMatrices];               // staged batch: first vector of its matrix i
    uint32_t vsrc[kBatchMatrices * NT];          // staged vector v: word offset of its source
    uint8_t vshared[kBatchMatrices * NT];        // staged vector v: from shared_act
    int32_t nvec;
    int32_t nunion;
    int32_t flag;
    int32_t rows_landed;  // one-token C task: its sequence number once the lead wave's gate/up rows are in
    int32_t red[kThreads / 64];  // workgroup reductions (one word per wave)
    uint32_t rin[kRowsPerCTask];  // C task: the residual words it updates
    int32_t trace_stale;  // profiling builds: stale words of the last block-input read
};

// The workgroups on one CU (blocks b, b + cu_count, ...) place their waves on
// the SIMDs identically, so a wave doing a workgroup's serial work (top-k,
// scores, the norm, the mixture) would share one SIMD with the same wave of the
// other workgroups there. That work goes to the wave whose index is rotated by
// the workgroup's slot on its CU; rel_wave is a wave's index relative to it.
__device__ __forceinline__ int rel_wave(const DecodeParams& p) {
    const int lead = (int)(blockIdx.x / (unsigned)p.cu_count) & 3;
    return (wave_id() - lead) & 3;
}

__device__ __forceinline__ uint32_t* phase_counters(const DecodeParams& p, int li, int phase) {
    return p.counters + ((size_t)li * kCountersPerLayer + phase) * kCounterGroupWords;
}
__device__ __forceinline__ uint32_t* phase_flags(const DecodeParams& p, int li, int phase) {
    return p.flags + ((size_t)li * kCountersPerLayer + phase) * kFlagCopies * kFlagStride;
}

// ---- block input ---------------------------------------------------------------------

// The residual of layer li ([T][H] bf16) into LDS as f32: the caller's input
// for the first layer of the launch, else the tagged residual words.
template <int NT, class SH>
__device__ __forceinline__ bool load_input(const DecodeParams& p, int li, uint32_t epoch, SH& sh) {
    const int pairs = p.T * p.H / 2;
    float* xs = sh.xs;
    bool ok = true;
    if (chain_start(p, li)) {
        const auto* x2 = as_global(chain_input(p, li));
        uint32_t v[NT * kXWords];
#pragma unroll
        for (int k = 0; k < NT * kXWords; ++k) {
            const int i = (int)threadIdx.x + k * kThreads;
            v[k] = x2[i < pairs ? i : pairs - 1];
        }
#pragma unroll
        for (int k = 0; k < NT * kXWords; ++k) {
            const int i = (int)threadIdx.x + k * kThreads;
            if (i < pairs) *reinterpret_cast<float2*>(xs + 2 * i) = make_float2(bf16_lo(v[k]), bf16_hi(v[k]));
        }
    } else {
        // this thread's words: tid, tid + 256, ... below pairs
        const int n = (pairs - (int)threadIdx.x + kThreads - 1) / kThreads;
        uint64_t v[NT * kXWords];
        int stale = 0;
        ok = load_tagged<NT * kXWords, kThreads>(v, p.xw + (size_t)li * pairs + threadIdx.x, n, epoch, p.error,
                                                 p.limit_ticks, &stale);
#ifdef FW_DECODE_TRACE
        stale = wg_count(sh.red, stale);
        if (threadIdx.x == 0) sh.trace_stale = stale;
#endif
        (void)stale;
#pragma unroll
        for (int k = 0; k < NT * kXWords; ++k) {
            const int i = (int)threadIdx.x + k * kThreads;
            const uint32_t w = (uint32_t)v[k];
            if (k < n) *reinterpret_cast<float2*>(xs + 2 * i) = make_float2(bf16_lo(w), bf16_hi(w));
        }
    }
    return wg_all(sh.red, ok) != 0;
}

// In the chained step the block input is the pre-norm of the residual
// (workload glue, not the reference's block): h = bf16(r * 1/sqrt(mean(r^2) +
// 1e-6)), mean(r^2) through the reference's dot order (32 chains, tree, +0.0)
// divided by H; h[H-1] = 1.0 with the bias feature. Wave t normalises token t,
// in place in LDS.
template <int NT, class SH>
__device__ __forceinline__ void normalise_input(const DecodeParams& p, SH& sh, int slot = -1) {
    (void)slot;
    if (!p.prenorm) return;
    const int T = p.T, n = p.H;
    float* xs = sh.xs;
    const int w = rel_wave(p), lane = lane_id();
    // Lane L < 32 of token t's wave sums chain j = bit-reverse of L (five
    // bits): the tree's partners (j, j + 16), (j, j + 8), (j, j + 4) are then
    // lanes L ^ 1, L ^ 2, L ^ 4 of one row (DPP), and its last four values
    // lanes 0, 16, 8, 24.
    const int j = (int)(__builtin_bitreverse32((uint32_t)lane) >> 27);
    auto finish = [&](float c, int t) {
        c = add_rn(c, dpp_f32<kDppQuadXor1>(c));  // a1[j] = c[j] + c[j+16]
        c = add_rn(c, dpp_f32<kDppQuadXor2>(c));  // a2[j] = a1[j] + a1[j+8]
        c = add_rn(c, dpp_f32<kDppRowRead4>(c));   // a3[j] = a2[j] + a2[j+4]
        const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c), 0));
        const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c), 16));
        const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c), 8));
        const float a3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c), 24));
        const float ss = add_rn(add_rn(add_rn(a0, a1), add_rn(a2, a3)), 0.0f);
        if (lane == 0) sh.inv[t] = 1.0f / sqrtf(add_rn(ss / (float)n, 1e-6f));
    };
    if (w < T) {
        const float* r = xs + w * n;
        float c = 0.0f;
        if (lane < 32) {
            // blocks in order; LDS reads batched ahead of the adds
            int b = 0;
            for (; b + 16 <= n / 32; b += 16) {
                float e[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) e[i] = r[32 * (b + i) + j];
#pragma unroll
                for (int i = 0; i < 16; ++i) c = add_rn(c, mul_rn(e[i], e[i]));
            }
            for (; b < n / 32; ++b) {
                float e = r[32 * b + j];
                c = add_rn(c, mul_rn(e, e));
            }
        }
        finish(c, w);
        FW_TRACE_MARK_IF(w == 0 && lane == 0, slot, 5);
    }
    wg_sync();
    FW_TRACE_MARK(slot, 6);
    for (int t = 0; t < T; ++t) {
        const float inv = sh.inv[t];
        float* r = xs + t * n;
        for (int i = threadIdx.x; i < n; i += kThreads) {
            float hv = from_bf16(to_bf16(mul_rn(r[i], inv)));
            if (p.bias_feature && i == n - 1) hv = 1.0f;
            r[i] = hv;
        }
    }
    wg_sync();
    FW_TRACE_MARK(slot, 7);
}

// ---- expert selection ------------------------------------------------------------------

// The layer's logits into LDS (after the router tasks): tagged words, T rows
// of ls bf16.
template <int NT, class SH>
__device__ __forceinline__ bool load_logits(const DecodeParams& p, int li, uint32_t epoch, SH& sh) {
    constexpr int kWords = (NT * logit_stride(kMaxExperts) / 2 + kThreads - 1) / kThreads;
    const int words = p.T * p.ls / 2;
    const int n = (words - (int)threadIdx.x + kThreads - 1) / kThreads;
    uint64_t v[kWords];
    bool ok = load_tagged<kWords, kThreads>(v, p.logits + (size_t)li * words + threadIdx.x, n, epoch, p.error,
                                            p.limit_ticks);
    uint32_t* lg2 = reinterpret_cast<uint32_t*>(sh.lg);
#pragma unroll
    for (int k = 0; k < kWords; ++k) {
        if (k < n) lg2[threadIdx.x + k * kThreads] = (uint32_t)v[k];
    }
    return wg_all(sh.red, ok) != 0;
}

// Top-k of every token (src/router.rs:241-247 total order) and the union of
// the selections in ascending expert id, the execution order of
// src/decoder_layer.rs:422-424: sorted[slot], slot_tokens[slot] (token mask),
// tslot[t][k] (slot of the token's k-th expert in ascending id), nunion.
// Requires the logits in LDS. TK: logits per lane in the top-k (E <= 64 * TK).
template <int NT, int TK, class SH>
__device__ __forceinline__ void select_experts(const DecodeParams& p, SH& sh, int slot_trace = -1) {
    (void)slot_trace;
    const int T = p.T, E = p.E, K = p.K, S = p.S, LS = p.ls;
    const int lane = lane_id(), w = rel_wave(p);
    if (w < T) {
        wave_topk<TK>(sh.lg + w * LS, E, K, sh.ids + w * kMaxTopK);
    }
    FW_TRACE_MARK(slot_trace, 4);
    wg_sync();
    FW_TRACE_MARK(slot_trace, 5);
    // The union, by wave 0 in registers: lane l holds entries l and l + 64 of
    // the T * K selections (entry i = token i / K, rank i % K); every loop
    // runs over the entries in order with the entry's values read from its
    // lane. One token selects distinct experts: its slots are the ranks of its
    // ids.
    if (w == 0 && (NT == 1 || T == 1)) {
        const int id = lane < K ? sh.ids[lane] : 0x7fffffff;
        int rank = 0;
        for (int j = 0; j < K; ++j) rank += (__builtin_amdgcn_readlane(id, j) < id) ? 1 : 0;
        if (lane < K) {
            sh.sorted[rank] = id;
            sh.slot_tokens[rank] = 1u;
            sh.tslot[rank] = rank;
            sh.pos[lane] = rank;
            sh.rank_at[rank] = lane;
        }
        for (int s2 = K + lane; s2 < S; s2 += kWave) sh.slot_tokens[s2] = 0u;
        if (lane == 0) sh.nunion = K;
    } else if (NT > 1 && w == 0) {
        const int n_sel = T * K;
        int id[2], tok[2], slot[2] = {0, 0}, rank_in_token[2] = {0, 0};
        bool first[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e = lane + kWave * h;
            tok[h] = e / K;
            id[h] = e < n_sel ? sh.ids[tok[h] * kMaxTopK + (e - tok[h] * K)] : 0x7fffffff;
            first[h] = e < n_sel;
        }
        // first occurrence: no earlier entry selects the same expert
        for (int j = 0; j < n_sel; ++j) {
            const int idj = j < kWave ? __builtin_amdgcn_readlane(id[0], j) : __builtin_amdgcn_readlane(id[1], j - kWave);
#pragma unroll
            for (int h = 0; h < 2; ++h) first[h] = first[h] && !(j < lane + kWave * h && idj == id[h]);
        }
        const uint64_t f0 = __ballot(first[0]), f1 = __ballot(first[1]);
        // slot = distinct experts with a smaller id; position among the token's own ids
        for (int t = 0, j = 0; t < T; ++t) {
            for (int r = 0; r < K; ++r, ++j) {
                const int idj =
                    j < kWave ? __builtin_amdgcn_readlane(id[0], j) : __builtin_amdgcn_readlane(id[1], j - kWave);
                const bool fj = ((j < kWave ? f0 >> j : f1 >> (j - kWave)) & 1ull) != 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    slot[h] += (fj && idj < id[h]) ? 1 : 0;
                    rank_in_token[h] += (t == tok[h] && idj < id[h]) ? 1 : 0;
                }
            }
        }
        // tokens of each slot
        uint32_t mask[2] = {0u, 0u};
        for (int t = 0, j = 0; t < T; ++t) {
            for (int r = 0; r < K; ++r, ++j) {
                const int sj = j < kWave ? __builtin_amdgcn_readlane(slot[0], j) : __builtin_amdgcn_readlane(slot[1], j - kWave);
#pragma unroll
                for (int h = 0; h < 2; ++h) mask[h] |= (sj == slot[h]) ? (1u << t) : 0u;
            }
        }
        const int nunion = __popcll(f0) + __popcll(f1);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (lane + kWave * h < n_sel) {
                if (first[h]) {
                    sh.sorted[slot[h]] = id[h];
                    sh.slot_tokens[slot[h]] = mask[h];
                }
                sh.tslot[tok[h] * K + rank_in_token[h]] = slot[h];
                sh.pos[lane + kWave * h] = rank_in_token[h];
            }
        }
        for (int s2 = nunion + lane; s2 < S; s2 += kWave) sh.slot_tokens[s2] = 0u;
        if (lane == 0) sh.nunion = nunion;
    }
    FW_TRACE_MARK(slot_trace, 6);
    wg_sync();
}

// Scores of the selected experts (token t on the wave first_wave + t relative
// to the lead wave; without `barrier` the caller synchronises before the
// results are read): src/router.rs:248-262 /
// src/decoder_layer.rs:290-306 (max, exp(v - max), one sequential f32 sum in
// index order, renormalised over the selection), as tweight[t][k] in the
// token's ascending-id order, and the shared-gate sigmoid. With host_outputs
// also the rank-order ids and scores and the sigmoid for the caller.
template <int NT, class SH>
__device__ __forceinline__ void score_experts(const DecodeParams& p, int li, SH& sh, bool host_outputs,
                                              int exp_offset = 0, int first_wave = 0, bool barrier = true) {
    const int T = p.T, E = p.E, K = p.K, LS = p.ls;
    const int lane = lane_id(), w = (rel_wave(p) - first_wave) & 3;
    if (w < T) {
        const uint16_t* lt = sh.lg + w * LS;
        float* ew = sh.xs + exp_offset + w * E;
        float mx = -__builtin_inff();
        for (int e = lane; e < E; e += kWave) mx = fmaxf(mx, from_bf16(lt[e]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
        for (int e = lane; e < E; e += kWave) ew[e] = expf_glibc(add_rn(from_bf16(lt[e]), -mx), sh.exp2tab);
        // the exponentials are this wave's own: order its LDS writes before
        // lane 0 reads them (no wait on the wave's memory loads)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // one sequential sum in index order (lane 0, reading four values at a
        // time when the token's row is 16-byte aligned)
        float den = -0.0f;
        if (lane == 0) {
            int e = 0;
            if (((E | (w * E)) & 3) == 0) {
                const float4* e4 = reinterpret_cast<const float4*>(ew);
                for (; e + 32 <= E; e += 32) {
                    float4 v[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = e4[e / 4 + i];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        den = add_rn(den, v[i].x);
                        den = add_rn(den, v[i].y);
                        den = add_rn(den, v[i].z);
                        den = add_rn(den, v[i].w);
                    }
                }
            }
            for (; e < E; ++e) den = add_rn(den, ew[e]);
        }
        den = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, den)));
        // lane r: the rank-r expert's probability; their sum in rank order
        const int32_t* ids = sh.ids + w * kMaxTopK;
        const float pr = lane < K ? ew[ids[lane]] / den : 0.0f;
        float sel = -0.0f;
        for (int r = 0; r < K; ++r)
            sel = add_rn(sel, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr), r)));
        if (lane < K) {
            const uint16_t score = to_bf16(pr / sel);
            sh.tweight[w * K + sh.pos[w * K + lane]] = score;
            if (host_outputs) {
                p.ids[((size_t)li * T + w) * K + lane] = ids[lane];
                p.scores[((size_t)li * T + w) * K + lane] = score;
            }
        }
        if (lane == 0) {
            const uint16_t sg = sigmoid_bf16(lt[p.gi], sh.exp2tab);
            sh.sig[w] = sg;
            if (host_outputs) p.sig[(size_t)li * T + w] = sg;
        }
    }
    if (barrier) wg_sync();
}

// ---- tasks ----------------------------------------------------------------------------
//
// A wave covers 4 rows (16 lanes each). R task: 16 router rows; the last R
// task of a layer is the shared_expert_gate row alone. S and B tasks: 8
// gate/up pairs, wave w taking pairs 2w and 2w+1 with its lane groups 0, 1 on
// the gate rows and 2, 3 on the up rows, so SwiGLU joins lane l and l + 32.
// R and S issue their weight loads before waiting for the previous layer; B
// stages and normalises the input once the previous layer is done, waits for
// the router, selects, then issues its expert's rows.

// What this workgroup's LDS holds: the layer whose raw input / normalised
// input / selection / scores are there (-1: none).
struct LdsState {
    int loaded = -1, staged = -1, selected = -1, scored = -1;  // scored: route weights and sigmoid
};

// Trace slot of a task: layer * (R + S + B + C tasks) + its index in that
// order.
__device__ __forceinline__ int trace_slot(const DecodeParams& p, int li, int index) {
    return li * (p.n_router + p.n_shared + p.n_b + p.n_c) + index;
}

// Block input of layer li in LDS, normalised.
template <int NT, class SH>
__device__ __forceinline__ bool stage_layer_input(const DecodeParams& p, uint32_t epoch, SH& sh,
                                                  LdsState& st, int li, int slot = -1) {
    (void)slot;
    if (st.staged == li) return true;
    if (st.loaded != li) {
        if (!load_input<NT>(p, li, epoch, sh)) return false;
        st.loaded = li;
        FW_TRACE_MARK(slot, 2);
        FW_TRACE_VALUE(slot, 4, sh.trace_stale);
    }
    normalise_input<NT>(p, sh, slot);
    st.staged = li;
    return true;
}

// Selection of layer li in LDS (waits for its router tasks).
template <int NT, int TK, class SH>
__device__ __forceinline__ bool select_layer(const DecodeParams& p, uint32_t epoch, SH& sh, LdsState& st,
                                             int li, int slot) {
    if (st.selected == li) return true;
    if (!wait_phase(phase_flags(p, li, kCntRouter), epoch, p.error, p.limit_ticks, &sh.flag)) return false;
    FW_TRACE_MARK(slot, 2);
    if (!load_logits<NT>(p, li, epoch, sh)) return false;
    FW_TRACE_MARK(slot, 3);
    select_experts<NT, TK>(p, sh, slot);
    st.selected = li;
    return true;
}

// One token with rank-ordered slots: the expert of rank r (of layer li) into
// sh.ids[r], from a top-k that stops after r + 1 rounds. Leaves no complete
// selection in LDS.
template <int TK, class SH>
__device__ __forceinline__ bool select_rank(const DecodeParams& p, uint32_t epoch, SH& sh, LdsState& st, int li,
                                            int r, int slot) {
    if (!wait_phase(phase_flags(p, li, kCntRouter), epoch, p.error, p.limit_ticks, &sh.flag)) return false;
    FW_TRACE_MARK(slot, 2);
    if (!load_logits<1>(p, li, epoch, sh)) return false;
    FW_TRACE_MARK(slot, 3);
    if (rel_wave(p) == 0) wave_topk<TK>(sh.lg, p.E, r + 1, sh.ids);
    FW_TRACE_MARK(slot, 4);
    wg_sync();
    st.selected = -1;
    return true;
}

// R task j of layer li: 16 router rows, or the shared_expert_gate row.
template <int NT, int MBH, class SH>
__device__ __forceinline__ bool router_task(const DecodeParams& p, uint32_t epoch, SH& sh, LdsState& st,
                                            int li, int j) {
    FW_TRACE_STAMP(t0);
    const int slot = trace_slot(p, li, j);
    (void)slot;
    const int lane = lane_id(), w = wave_id(), g = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int T = p.T, H = p.H, E = p.E;
    const DecodeLayer& L = p.layers[li];
    const bool gate_task = j == p.n_router - 1;
    const int row0 = gate_task ? E : j * kRouterRowsPerTask;
    const int rows = gate_task ? 1 : min(kRouterRowsPerTask, E - row0);
    const int rin = w * kRowsPerWave + g;
    const bool wave_active = w * kRowsPerWave < rows;
    const bool valid = rin < rows;
    const bool fold = p.order == 1 && !gate_task;
    const int out_index = row0 + (valid ? rin : 0);
    const uint16_t* wrow = L.router + (size_t)out_index * H;
    LineShare<MBH> rs;
    if (wave_active && !fold)
        line_issue(rs, L.router + (size_t)row0 * H, (uint32_t)(valid ? rin : 0) * (uint32_t)H * 2u, q);
    // one-token steps: the residual words' tags alone say when the block
    // input is complete (a flag hop less on the layer's critical path)
    if (!chain_start(p, li) && !p.input_by_tags &&
        !wait_phase(phase_flags(p, chain_prev(p, li), kCntC), epoch, p.error, p.limit_ticks, &sh.flag))
        return false;
    FW_TRACE_STAMP(t1);
    if (!stage_layer_input<NT>(p, epoch, sh, st, li, slot)) return false;
    FW_TRACE_MARK(slot, 0);
    uint64_t* lw = p.logits + (size_t)li * T * (p.ls / 2);
    if (fold) {
        // src/router.rs:228-240: one lane folds one row; lanes 0 and 2 store
        // the pairs of rows (r, r + 1).
        const int r = j * kRouterRowsPerTask + w * kRowsPerWave + lane;
        const bool mine = lane < kRowsPerWave && r < E;
        for (int tt = 0; tt < T; ++tt) {
            uint32_t bits = mine ? to_bf16(fold_row(L.router + (size_t)r * H, sh.xs + tt * H, H)) : 0u;
            uint32_t next = (uint32_t)__shfl_down((int)bits, 1, kWave);
            if (mine && (lane & 1) == 0) coherent_store64(lw + (tt * p.ls + r) / 2, tagged(bits | (next << 16), epoch));
        }
    } else if (wave_active) {
        float acc[NT][2];
        FW_TRACE_MARK(slot, 8);
        line_chains<NT, MBH>(rs, H / 32, sh.xs, H, q, acc);
        FW_TRACE_MARK(slot, 9);
        // groups 0 and 2 store the pairs (row, row + 1); the gate logit goes to
        // its own slot with a zero beside it
        const int at = gate_task ? p.gi : out_index;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            float d = tree32_reduce_lines(acc[tt][0], acc[tt][1]);
            if (q == 0) d = tree32_finish(d, wrow, sh.xs + tt * H, H);
            const uint32_t bits = to_bf16(d);
            uint32_t next = (uint32_t)__shfl((int)bits, (lane + kLanesPerRow) & 63, kWave);
            if (gate_task) next = 0u;
            if (tt < T && q == 0 && (g & 1) == 0 && valid)
                coherent_store64(lw + (tt * p.ls + at) / 2, tagged(bits | (next << 16), epoch));
        }
    }
    FW_TRACE_MARK(slot, 1);
    publish(phase_counters(p, li, kCntRouter), p.n_router, j, phase_flags(p, li, kCntRouter), epoch);
    FW_TRACE_STAMP(t2);
    FW_TRACE_WRITE(slot, kTaskRouter, t0, t1, t2);
    return true;
}

// S task (shared = true, index js < n_shared) or B task (index js < n_b) of
// layer li: 8 gate/up pairs with fused SwiGLU.
template <int NT, int MBH, int TK, class SH>
__device__ __forceinline__ bool pairs_task(const DecodeParams& p, uint32_t epoch, SH& sh, LdsState& st,
                                           int li, int js, bool shared) {
    FW_TRACE_STAMP(t0);
    const int slot = trace_slot(p, li, p.n_router + (shared ? js : p.n_shared + js));
    (void)slot;
    const int lane = lane_id(), w = wave_id(), g = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int T = p.T, H = p.H, I = p.I, Is = p.Is;
    const DecodeLayer& L = p.layers[li];
    const uint16_t* wbase;  // the task's first gate row; up rows follow `up` rows later
    uint64_t* act_out;
    int act_stride, pair0, up;  // words per token
    bool work = true;
    uint32_t mask = (1u << T) - 1u;
    if (shared) {
        pair0 = js * kPairsPerTask;
        act_out = p.shared_act + (size_t)li * T * (Is / 2);
        act_stride = Is / 2;
        wbase = L.shared_gate;  // shared_up follows it
        up = Is;
    } else {
        const int per_slot = I / kPairsPerTask;
        const int s = js / per_slot;
        if (st.staged != li) {
            // the block input is ready with the previous layer: stage it while
            // the router runs
            if (!chain_start(p, li) &&
                !wait_phase(phase_flags(p, chain_prev(p, li), kCntC), epoch, p.error, p.limit_ticks, &sh.flag))
                return false;
            if (!stage_layer_input<NT>(p, epoch, sh, st, li)) return false;
        }
        int e;
        if (p.rank_slots) {
            if (!select_rank<TK>(p, epoch, sh, st, li, s, slot)) return false;
            FW_TRACE_MARK(slot, 0);
            e = uniform(sh.ids[s]);
            mask = 1u;
        } else {
            if (!select_layer<NT, TK>(p, epoch, sh, st, li, slot)) return false;
            FW_TRACE_MARK(slot, 0);
            work = s < uniform(sh.nunion);
            e = work ? uniform(sh.sorted[s]) : 0;
            mask = work ? (uint32_t)uniform((int)sh.slot_tokens[s]) : 0u;
        }
        wbase = L.gate_up + (size_t)e * 2 * I * H;
        up = I;
        pair0 = (js - s * per_slot) * kPairsPerTask;
        act_out = p.act + ((size_t)li * p.S + s) * (size_t)T * (I / 2);
        act_stride = I / 2;
    }
    const int out_index = pair0 + 2 * w + (g & 1);
    const uint32_t row_rel = (uint32_t)((g < 2 ? 0 : up) + (g & 1));  // rows past the wave's first gate row
    const uint16_t* wave_row = wbase + (size_t)(pair0 + 2 * w) * H;
    const uint16_t* wrow = wave_row + (size_t)row_rel * H;
    LineShare<MBH> rs;
    if (work) line_issue(rs, wave_row, row_rel * (uint32_t)H * 2u, q);
    if (shared && !chain_start(p, li) &&
        !wait_phase(phase_flags(p, chain_prev(p, li), kCntC), epoch, p.error, p.limit_ticks, &sh.flag))
        return false;
    FW_TRACE_STAMP(t1);
    if (work) {
        if (shared) {
            if (!stage_layer_input<NT>(p, epoch, sh, st, li)) return false;
            FW_TRACE_MARK(slot, 0);
        }
        // three or four tokens: only the tokens in the mask (every token for
        // the shared expert), compacted in token order; one or two tokens:
        // every token, stored where the mask has it (registers for a second
        // code path would spill). Each token's arithmetic is the same.
        auto dots = [&](auto count) {
            constexpr int NA = decltype(count)::value;
            int tok[NA], xoff[NA];
            uint32_t m = mask;
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                tok[i] = NA == NT ? i : __builtin_ctz(m);
                xoff[i] = tok[i] * H;
                m &= m - 1u;
            }
            float acc[NA][2];
            line_chains_at<NA, MBH>(rs, H / 32, sh.xs, xoff, q, acc);
            // gate (groups 0, 1) meets up (groups 2, 3): lane l takes lane l + 32;
            // group 0 stores the pair (pair, pair + 1) with group 1's result
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                const int tt = tok[i];
                float d = tree32_reduce_lines(acc[i][0], acc[i][1]);
                if (q == 0) d = tree32_finish(d, wrow, sh.xs + tt * H, H);
                const uint32_t bits = to_bf16(d);
                const uint32_t up = (uint32_t)__shfl((int)bits, (lane + 32) & 63, kWave);
                const uint32_t a = swiglu_bf16(bits, up, sh.exp2tab);
                const uint32_t b = (uint32_t)__shfl((int)a, (lane + kLanesPerRow) & 63, kWave);
                if (g == 0 && q == 0 && (mask & (1u << tt)))
                    coherent_store64(act_out + (size_t)tt * act_stride + out_index / 2, tagged(a | (b << 16), epoch));
            }
        };
        if constexpr (NT <= 2) {
            dots(std::integral_constant<int, NT>{});
        } else {
            // a union expert always has a token (its mask is never empty)
            const int na = __builtin_popcount(mask & ((1u << NT) - 1u));
            if (na > 0) with_count<1, NT>(na, dots);
        }
        FW_TRACE_MARK(slot, 1);
    }
    if (p.cpairs > 0) {
        // one-token fused C tasks read the activations by their tags alone
        wg_sync();
    } else {
        publish(phase_counters(p, li, kCntGateUp), p.n_gu, shared ? js : p.n_shared + js,
                phase_flags(p, li, kCntGateUp), epoch);
    }
    FW_TRACE_STAMP(t2);
    FW_TRACE_WRITE(slot, shared ? kTaskShared : kTaskGateUp, t0, t1, t2);
    return true;
}

// Stages into LDS the activation vectors of matrices [mb, me] of layer li (m
// = 0 shared, 1 + s slot s): one vector per token in the matrix's mask, the
// batch's i-th matrix from vector sh.vbase[i], vector v at sh.xs + v * stride
// words (stride = max(I, Is) / 2 <= MBI * 16). Returns false on timeout or
// error.
template <int NT, int MBI, class SH>
__device__ __forceinline__ bool stage_acts(const DecodeParams& p, int li, uint32_t epoch, SH& sh, int mb, int me,
                                           int slot = -1) {
    (void)slot;
    constexpr int kChunks = (MBI * 16 + kThreads - 1) / kThreads;  // words of one vector per thread
    constexpr int kRound = 12 / kChunks;                           // vectors per round
    const int T = p.T, I = p.I, Is = p.Is;
    const int stride = max(I, Is) / 2;
    const int tid = threadIdx.x;
    if (T == 1) {
        // one token: vector i is matrix mb + i (every mask holds the token)
        if (tid <= me - mb) {
            const int m = mb + tid;
            sh.vbase[tid] = tid;
            sh.vshared[tid] = m == 0;
            sh.vsrc[tid] = m == 0 ? (uint32_t)((size_t)li * (Is / 2)) : (uint32_t)(((size_t)li * p.S + m - 1) * (I / 2));
        }
        if (tid == 0) sh.nvec = me - mb + 1;
    } else if (tid == 0) {
        int n = 0;
        for (int m = mb; m <= me; ++m) {
            sh.vbase[m - mb] = n;
            const uint32_t mask = m == 0 ? (1u << T) - 1u : sh.slot_tokens[m - 1];
            for (int t = 0; t < T; ++t) {
                if (mask & (1u << t)) {
                    sh.vshared[n] = m == 0;
                    sh.vsrc[n] = m == 0 ? (uint32_t)(((size_t)li * T + t) * (Is / 2))
                                        : (uint32_t)((((size_t)li * p.S + m - 1) * T + t) * (I / 2));
                    ++n;
                }
            }
        }
        sh.nvec = n;
    }
    wg_sync();
    if (mb == 0) FW_TRACE_MARK(slot, 7);
    const int nvec = uniform(sh.nvec);
    uint32_t* dst = reinterpret_cast<uint32_t*>(sh.xs);
    bool ok = true;
    for (int v0 = 0; v0 < nvec; v0 += kRound) {
        uint64_t x[kRound][kChunks];
#pragma unroll
        for (int r = 0; r < kRound; ++r) {
            if (v0 + r < nvec) {
                // one token: the source follows from the matrix index in scalar registers
                const int m1 = mb + v0 + r;
                const bool vs = T == 1 ? m1 == 0 : uniform(sh.vshared[v0 + r]) != 0;
                const uint64_t* src =
                    T == 1 ? (m1 == 0 ? p.shared_act + (size_t)li * (Is / 2) : p.act + ((size_t)li * p.S + m1 - 1) * (I / 2))
                           : (vs ? p.shared_act : p.act) + (uint32_t)uniform((int)sh.vsrc[v0 + r]);
                const int len = vs ? Is / 2 : I / 2;
#pragma unroll
                for (int c = 0; c < kChunks; ++c) {
                    const int wd = tid + c * kThreads;
                    if (wd < len)
                        x[r][c] = __hip_atomic_load(as_global(src + wd), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        }
        // words not yet carrying the epoch (stale cached lines, stores in
        // flight) are read again past the caches, all of them per pass
        if (v0 == 0 && mb == 0) FW_TRACE_MARK(slot, 8);
        uint64_t start = 0;
        for (int pass = 0;; ++pass) {
            bool all = true;
#ifdef FW_DECODE_TRACE
            if (pass == 0) {
                int stale = 0;
                for (int r = 0; r < kRound; ++r)
                    for (int c = 0; c < kChunks; ++c)
                        stale += (v0 + r < nvec && tid + c * kThreads < I / 2 && !has_tag(x[r][c], epoch)) ? 1 : 0;
                const int total = wg_count(sh.red, stale);
                if (tid == 0 && p.trace != nullptr && slot >= 0) p.trace[(size_t)slot * kTraceWords + 4 + 6] = total;
            }
#endif
#pragma unroll
            for (int r = 0; r < kRound; ++r) {
                if (v0 + r < nvec) {
#pragma unroll
                    for (int c = 0; c < kChunks; ++c) {
                        const int wd = tid + c * kThreads;
                        const bool vs = sh.vshared[v0 + r] != 0;
                        if (wd < (vs ? Is / 2 : I / 2) && !has_tag(x[r][c], epoch)) {
                            all = false;
                            x[r][c] = coherent_load64((vs ? p.shared_act : p.act) + sh.vsrc[v0 + r] + wd);
                        }
                    }
                }
            }
            if (all) break;
            if (pass == 0) start = wall_clock64();
            // the shared error word on every 8th pass
            if (((pass & 7) == 7 && coherent_load(p.error) != 0) || wall_clock64() - start > p.limit_ticks) {
                int32_t expected = 0;
                __hip_atomic_compare_exchange_strong(p.error, &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                ok = false;
                break;
            }
        }
#pragma unroll
        for (int r = 0; r < kRound; ++r) {
            if (v0 + r < nvec) {
                const int len = (T == 1 ? mb + v0 + r == 0 : sh.vshared[v0 + r] != 0) ? Is / 2 : I / 2;
#pragma unroll
                for (int c = 0; c < kChunks; ++c) {
                    const int wd = tid + c * kThreads;
                    if (wd < len) dst[(v0 + r) * stride + wd] = (uint32_t)x[r][c];
                }
            }
        }
    }
    return wg_all(sh.red, ok) != 0;
}

// The sweep of down_row_lds (STRIDE: words between activation pairs, 2 for
// tagged words).
template <int MAXB, int STRIDE = 1>
__device__ __forceinline__ uint32_t down_row_sweep(const LineShare<MAXB>& r, int nb, const uint32_t* a0, int q) {
    // the activation pairs of eight blocks at a time (one LDS wait each), then
    // their chain steps
    constexpr int kStep = 8;
    float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
    for (int u0 = 0; u0 < MAXB; u0 += kStep) {
        uint32_t a[kStep];
#pragma unroll
        for (int i = 0; i < kStep; ++i) {
            if (u0 + i < MAXB && u0 + i < nb) a[i] = a0[STRIDE * 16 * (u0 + i)];
        }
#pragma unroll
        for (int i = 0; i < kStep; i += 2) {
            const int v = (u0 + i) / 2;
            if (v < (MAXB + 1) / 2) {
                uint32_t first, second;
                line_pairs(r.w[v], q, first, second);
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int u = u0 + i + half;
                    if (u < MAXB && u < nb) {
                        const uint32_t wv = half ? second : first;
                        c0 = add_rn(c0, mul_rn(bf16_lo(wv), bf16_lo(a[i + half])));
                        c1 = add_rn(c1, mul_rn(bf16_hi(wv), bf16_hi(a[i + half])));
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    return to_bf16(add_rn(tree32_reduce_lines(c0, c1), 0.0f));
}

// One down row against an activation vector staged in LDS (av: its first
// word): the chains of src/expert.rs:514-552 over K = nblocks * 32 (so the
// tail sum is +0.0). This lane's chain pair of block b is activation pair
// 16 b + line_column(q) / 2.
template <int MAXB, int STRIDE = 1>
__device__ __forceinline__ uint32_t down_row_lds(const LineShare<MAXB>& r, int nblocks, const uint32_t* av, int q) {
    const uint32_t* a0 = av + STRIDE * (line_column(q) / 2);
    return down_row_sweep<MAXB, STRIDE>(r, opaque(nblocks), a0, q);
}

// One token, matrices 0..U (U < kDirectVectors): the tagged words of every
// activation vector of the task go straight from global memory into LDS
// (sixteen bytes per lane, no registers held while they travel), vector m at
// word m * stride (stride = max(I, Is) / 2, a multiple of 128); then words
// without the epoch are read again past the caches until they carry it.
template <int MBI, class SH>
__device__ __forceinline__ bool stage_acts_direct(const DecodeParams& p, int li, uint32_t epoch, SH& sh, int U,
                                                  int slot = -1) {
    (void)slot;
    const int I = p.I, Is = p.Is;
    const int stride = max(I, Is) / 2;
    uint64_t* raw = reinterpret_cast<uint64_t*>(sh.xs);
    const int w = wave_id(), lane = lane_id();
    auto source = [&](int m) -> const uint64_t* {
        return m == 0 ? p.shared_act + (size_t)li * (Is / 2) : p.act + ((size_t)li * p.S + m - 1) * (I / 2);
    };
    if ((I | Is) % 256 == 0) {
        // whole 1 KB parts (64 lanes x 16 bytes); the staging is on the
        // layer's critical path, so this loop is kept apart from the general one
        // part c = m * parts + h of the vectors' parts, walked by the waves in
        // turn with (m, h) stepped by subtraction (no division on the path)
        const int parts = stride / 128;
        int m = 0, h = w;
        while (h >= parts) {
            h -= parts;
            ++m;
        }
        for (; m <= U;) {
            if (h * 128 < (m == 0 ? Is / 2 : I / 2)) {
                __builtin_amdgcn_global_load_lds(
                    reinterpret_cast<const void*>(source(m) + h * 128 + 2 * lane),
                    (__attribute__((address_space(3))) void*)(raw + (size_t)m * stride + h * 128), 16, 0, 0);
            }
            h += kThreads / kWave;
            while (h >= parts) {
                h -= parts;
                ++m;
            }
        }
    } else {
        // a partial last part: lanes past the vector's end stay idle
        const int parts = (stride + 127) / 128;
        for (int c = w; c < (U + 1) * parts; c += kThreads / kWave) {
            const int m = c / parts, h = c - m * parts;
            if (h * 128 + 2 * lane < (m == 0 ? Is / 2 : I / 2)) {
                __builtin_amdgcn_global_load_lds(
                    reinterpret_cast<const void*>(source(m) + h * 128 + 2 * lane),
                    (__attribute__((address_space(3))) void*)(raw + (size_t)m * stride + h * 128), 16, 0, 0);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    // profiling: when each wave's loads have all landed
    FW_TRACE_MARK_IF(lane == 0 && w == 0, slot, 7);
    FW_TRACE_MARK_IF(lane == 0 && w == 1, slot, 8);
    FW_TRACE_MARK_IF(lane == 0 && w == 2, slot, 9);
    FW_TRACE_MARK_IF(lane == 0 && w == 3, slot, 3);
    wg_sync();
    // Thread t's words of vector m are words t and t + 256 (a vector is at
    // most 320 words). Words without the epoch are read again past the caches,
    // every stale word of the thread (per 256-word half) in one pass, until all
    // carry it.
    bool ok = true;
    const int tid = threadIdx.x;
    constexpr int kHalves = (MBI * 16 + kThreads - 1) / kThreads;
#pragma unroll
    for (int half = 0; half < kHalves; ++half) {
        if (kHalves > 1 && !ok) break;
        const int wd = kHalves == 1 ? tid : tid + half * kThreads;
        uint32_t stale = 0;
#pragma unroll
        for (int m = 0; m < kDirectVectors; ++m) {
            if (m <= U && wd < (m == 0 ? Is / 2 : I / 2) && !has_tag(raw[(size_t)m * stride + wd], epoch))
                stale |= 1u << m;
        }
        if (stale != 0) {
            const uint64_t start = wall_clock64();
            uint32_t polls = 0;
            while (stale != 0) {
                uint64_t v[kDirectVectors];
#pragma unroll
                for (int m = 0; m < kDirectVectors; ++m)
                    if (stale & (1u << m)) v[m] = coherent_load64(source(m) + wd);
#pragma unroll
                for (int m = 0; m < kDirectVectors; ++m) {
                    if ((stale & (1u << m)) && has_tag(v[m], epoch)) {
                        raw[(size_t)m * stride + wd] = v[m];
                        stale &= ~(1u << m);
                    }
                }
                if (stale == 0) break;
                // a pause between polls: 512 workgroups re-reading past the
                // caches while the layer's rows still stream slow the stream
                // (1,331 µs per step against 1,342 without it)
                __builtin_amdgcn_s_sleep(1);
                if (((++polls & 7) == 0 && coherent_load(p.error) != 0) || wall_clock64() - start > p.limit_ticks) {
                    int32_t expected = 0;
                    __hip_atomic_compare_exchange_strong(p.error, &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                    ok = false;
                    break;
                }
            }
        }
    }
    return wg_all(sh.red, ok) != 0;
}

// C task j of layer li: hidden rows 4j .. 4j + 3. Matrix m of the task: m = 0
// is the shared expert's down projection, m = 1 + s the down projection of
// slot s. Wave w covers the 4 rows (16 lanes each) of matrices w, w + 4,
// w + 8, w + 12 in its first batch, then the next 16 matrices, and so on.
template <int NT, int MBI, int TK, class SH>
__device__ __forceinline__ bool combine_task(const DecodeParams& p, uint32_t epoch, SH& sh, LdsState& st,
                                             int li, int j) {
    FW_TRACE_STAMP(t0);
    const int slot = trace_slot(p, li, p.n_router + p.n_shared + p.n_b + j);
    (void)slot;
    const int lane = lane_id(), w = wave_id(), g = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int T = p.T, H = p.H, I = p.I, Is = p.Is, K = p.K;
    const uint32_t all_tokens = (1u << T) - 1u;
    const DecodeLayer& L = p.layers[li];
    const int r0 = j * kRowsPerCTask;
    const int row = r0 + g;
    LineShare<MBI> rs0, rs1, rs2, rs3;
    // the shared expert's rows need no selection: issue them first
    if (w == 0) line_issue(rs0, L.shared_down + (size_t)r0 * Is, (uint32_t)(g * Is * 2), q);
    if (!select_layer<NT, TK>(p, epoch, sh, st, li, slot)) return false;
    FW_TRACE_MARK(slot, 2);
    const int U = uniform(sh.nunion);
#define FW_ISSUE_DOWN(RS, M)                                                                  \
    do {                                                                                      \
        const int m_ = (M);                                                                   \
        if (m_ >= 1 && m_ <= U) {                                                             \
            const uint16_t* wm_ = L.down + (size_t)uniform(sh.sorted[m_ - 1]) * (size_t)H * I; \
            line_issue(RS, wm_ + (size_t)r0 * I, (uint32_t)(g * I * 2), q);                    \
        } else if (m_ == 0) {                                                                 \
            line_issue(RS, L.shared_down + (size_t)r0 * Is, (uint32_t)(g * Is * 2), q); \
        }                                                                                     \
    } while (0)
#define FW_DOWN_DOT(RS, M)                                                                                \
    do {                                                                                                  \
        const int m_ = (M);                                                                               \
        if (m_ <= U) {                                                                                    \
            const int kd_ = m_ == 0 ? Is : I;                                                             \
            const uint32_t mask_ = m_ == 0 ? all_tokens : (uint32_t)uniform((int)sh.slot_tokens[m_ - 1]); \
            int v_ = uniform(sh.vbase[m_ - ms]);                                                          \
            _Pragma("unroll") for (int t_ = 0; t_ < NT; ++t_) {                                           \
                if (mask_ & (1u << t_)) {                                                                 \
                    const uint32_t bits_ = down_row_lds<MBI>(RS, kd_ / 32, act_lds + v_ * act_stride, q);  \
                    if (q == 0) sh.res[(m_ * NT + t_) * kRowsPerCTask + g] = bits_;                       \
                    ++v_;                                                                                 \
                }                                                                                         \
            }                                                                                             \
        }                                                                                                 \
    } while (0)
    if (w != 0) FW_ISSUE_DOWN(rs0, w);
    FW_ISSUE_DOWN(rs1, w + 4);
    FW_ISSUE_DOWN(rs2, w + 8);
    FW_ISSUE_DOWN(rs3, w + 12);
    // Route weights and the shared-gate sigmoid while the gate/up phase runs
    // (the exponentials overwrite the staged block input); task 0 also
    // reports the layer's ids, scores and sigmoid and rejects a NaN logit
    // (src/decoder_layer.rs:279-281).
    const int tid = threadIdx.x;
    if (j == 0 && p.order == 0) {
        int nan = 0;
        for (int e = tid; e < T * p.ls; e += kThreads) nan |= (e % p.ls < p.E) && ((sh.lg[e] & 0x7fffu) > 0x7f80u);
        if (wg_any(sh.red, nan) && tid == 0) atomicCAS(p.error, 0, 2);
    }
    if (st.scored != li || j == 0) {
        score_experts<NT>(p, li, sh, j == 0);
        st.loaded = st.staged = -1;
        st.scored = li;
    }
    FW_TRACE_MARK(slot, 5);
    // The residual words this task updates (ready since the router ran): one
    // lane of the lead wave per token and row.
    const int rt = rel_wave(p) * kWave + lane;
    const bool mixer = rt < T * kRowsPerCTask;
    const int mt = rt / kRowsPerCTask;
    const int mg = rt % kRowsPerCTask;
    const size_t at = ((size_t)mt * H + r0 + (mg & ~1)) / 2;
    bool ok = true;
    uint32_t rin = 0;
    if (mixer) {
        if (chain_start(p, li)) {
            rin = chain_input(p, li)[at];
        } else {
            uint64_t v[1];
            ok = load_tagged<1, 1>(v, p.xw + (size_t)li * T * H / 2 + at, 1, epoch, p.error, p.limit_ticks);
            rin = (uint32_t)v[0];
        }
    }
    FW_TRACE_MARK(slot, 3);
    if (!wait_phase(phase_flags(p, li, kCntGateUp), epoch, p.error, p.limit_ticks, &sh.flag)) return false;
    FW_TRACE_STAMP(t1);
    // Batches of 16 matrices (4 per wave): the batch's activation vectors
    // are staged in LDS once for all waves, then each wave runs its rows.
    const uint32_t* act_lds = reinterpret_cast<const uint32_t*>(sh.xs);
    const int act_stride = max(I, Is) / 2;
    st.loaded = st.staged = -1;
    constexpr int SB = stage_matrices(NT, MBI);
    for (int mb = 0; mb <= U; mb += kBatchMatrices) {
        if (mb > 0) {
            FW_ISSUE_DOWN(rs0, mb + w);
            FW_ISSUE_DOWN(rs1, mb + w + 4);
            FW_ISSUE_DOWN(rs2, mb + w + 8);
            FW_ISSUE_DOWN(rs3, mb + w + 12);
        }
        // matrices [ms, ms + SB) of the batch: register slots i with 4i in that range
        for (int sb = 0; sb < kBatchMatrices && mb + sb <= U; sb += SB) {
            const int ms = mb + sb;
            if (!stage_acts<NT, MBI>(p, li, epoch, sh, ms, min(U, ms + SB - 1), slot)) return false;
            FW_TRACE_MARK(slot, 4);
            if (sb <= 0 && 0 < sb + SB) FW_DOWN_DOT(rs0, mb + w);
            if (sb <= 4 && 4 < sb + SB) FW_DOWN_DOT(rs1, mb + w + 4);
            if (sb <= 8 && 8 < sb + SB) FW_DOWN_DOT(rs2, mb + w + 8);
            if (sb <= 12 && 12 < sb + SB) FW_DOWN_DOT(rs3, mb + w + 12);
            // the next staging overwrites these vectors
            wg_sync();
        }
    }
#undef FW_DOWN_DOT
#undef FW_ISSUE_DOWN
    FW_TRACE_MARK(slot, 0);
    if (!wg_all(sh.red, ok)) return false;
    if (mixer) {
        const int tt = mt, gg = mg;
        // src/decoder_layer.rs:528-545: weighted = bf16(down * score), summed in
        // ascending expert order from bf16 zero, rounding after each add (the
        // operands of eight steps are read ahead of the chain).
        uint32_t mix = to_bf16(0.0f);
        for (int k0 = 0; k0 < K; k0 += 8) {
            uint32_t d[8], wt[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (k0 + i < K) {
                    d[i] = sh.res[((1 + sh.tslot[tt * K + k0 + i]) * NT + tt) * kRowsPerCTask + gg];
                    wt[i] = sh.tweight[tt * K + k0 + i];
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (k0 + i < K) mix = add_bf16(mix, to_bf16(mul_rn(from_bf16(d[i]), from_bf16(wt[i]))));
            }
        }
        // src/decoder_layer.rs:563-575: gated = bf16(shared_down * sigmoid).
        const uint32_t sd = sh.res[(0 * NT + tt) * kRowsPerCTask + gg];
        const uint32_t gated = to_bf16(mul_rn(from_bf16(sd), from_bf16(sh.sig[tt])));
        const uint32_t o = add_bf16(mix, gated);
        const uint32_t xn = add_bf16((rin >> (16 * (gg & 1))) & 0xffffu, o);
        // rows 2i and 2i + 1 share a word: the even thread stores both
        const uint32_t o_odd = (uint32_t)__shfl_xor((int)o, 1, kWave);
        const uint32_t x_odd = (uint32_t)__shfl_xor((int)xn, 1, kWave);
        if ((gg & 1) == 0) {
            const uint32_t o2 = o | (o_odd << 16), x2 = xn | (x_odd << 16);
            reinterpret_cast<uint32_t*>(p.out + (size_t)li * T * H)[at] = o2;
            coherent_store64(p.xw + (size_t)(li + p.chains) * T * H / 2 + at, tagged(x2, epoch));
            if (li + p.chains >= p.nlayers && p.x_final != nullptr)
                reinterpret_cast<uint32_t*>(p.x_final)[(size_t)(li + p.chains - p.nlayers) * T * H / 2 + at] = x2;
        }
    }
    if (!wg_all(sh.red, ok)) return false;
    FW_TRACE_MARK(slot, 1);
    publish(phase_counters(p, li, kCntC), p.n_c, j, phase_flags(p, li, kCntC), epoch);
    FW_TRACE_STAMP(t2);
    FW_TRACE_WRITE(slot, kTaskDown, t0, t1, t2);
    return true;
}

// Whether a variant carries the fused C task (one token; three down-row slots
// per wave of down rows up to 640 columns).
__host__ __device__ constexpr bool fused_combine(int NT, int MBH, int MBI) {
    (void)MBH;
    return NT == 1 && MBI <= 20;
}

// C task j of layer li for one token when the gate/up pairs past the rows
// role's B tasks ride on the C tasks (p.cpairs = 2 pairs per task): the lead
// wave computes pairs nb_rows * 8 + 2j and + 1 like a B task, from rows it
// copies straight into LDS (gate rows for lane groups 0 and 2, up rows for 1
// and 3); every wave holds down rows of three matrices (matrix m: the shared
// expert for m = 0, slot m - 1 else; on wave m % 4, register slot m / 4). All
// rows are requested as soon as the selection is known, so no C task waits
// behind a B task of its workgroup.
template <int NT, int MBH, int MBI, int TK, bool PAIRS, class SH>
__device__ __forceinline__ bool combine_task_fused(const DecodeParams& p, uint32_t epoch, SH& sh, LdsState& st,
                                                   int li, int j) {
    static_assert(fused_combine(NT, MBH, MBI), "one token");
    static_assert(stage_words(NT, MBI) >= kBRowsAt + 4 * kBRowStride, "gate/up rows above the exponentials");
    static_assert(stage_words(NT, MBI) >= kDirectVectors * MBI * 16 * 2, "tagged words of the staged vectors");
    static_assert(MBI * 16 <= 2 * kThreads, "at most two staged words per thread and vector");
    FW_TRACE_STAMP(t0);
    const int slot = trace_slot(p, li, p.n_router + p.n_shared + p.n_b + j);
    (void)slot;
    // w: index relative to the lead wave
    const int lane = lane_id(), w = rel_wave(p), g = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int H = p.H, I = p.I, Is = p.Is, K = p.K;
    const DecodeLayer& L = p.layers[li];
    const int r0 = j * kRowsPerCTask;
    LineShare<MBI> c[3];
    // the shared expert's rows need no selection: issue them first
    if (w == 0) line_issue(c[0], L.shared_down + (size_t)r0 * Is, (uint32_t)(g * Is * 2), q);
    // this task's gate/up pairs need the block input (ready with the previous layer)
    if (!chain_start(p, li) &&
        !wait_phase(phase_flags(p, chain_prev(p, li), kCntC), epoch, p.error, p.limit_ticks, &sh.flag))
        return false;
    // the residual words this task updates (one lane of the lead wave per
    // row), taken from the block input before it is normalised in place
    const int rt = w * kWave + lane;
    const bool mixer = rt < kRowsPerCTask;
    const size_t at = ((size_t)r0 + (rt & ~1)) / 2;
    // without pairs of its own (PAIRS false, p.cpairs == 0: the rows role
    // runs every B task) the task needs only its residual words, not the
    // block input
    constexpr bool own_pairs = PAIRS;
    if (own_pairs && st.staged != li) {
        if (st.loaded != li) {
            if (!load_input<NT>(p, li, epoch, sh)) return false;
            st.loaded = li;
        }
        // (the values are bf16 widened exactly; normalise_input overwrites
        // them only after a workgroup barrier)
        if (mixer)
            sh.rin[rt] = (__float_as_uint(sh.xs[2 * at]) >> 16) | (__float_as_uint(sh.xs[2 * at + 1]) & 0xffff0000u);
        normalise_input<NT>(p, sh);
        st.staged = li;
    } else if (mixer) {
        uint32_t v0;
        if (chain_start(p, li)) {
            v0 = chain_input(p, li)[at];
        } else {
            uint64_t v[1];
            if (!load_tagged<1, 1>(v, p.xw + (size_t)li * H / 2 + at, 1, epoch, p.error, p.limit_ticks)) return false;
            v0 = (uint32_t)v[0];
        }
        sh.rin[rt] = v0;
    }
    if (!select_layer<NT, TK>(p, epoch, sh, st, li, slot)) return false;
    FW_TRACE_MARK(slot, 2);
    const int U = uniform(sh.nunion);
    const int fp0 = p.nb_rows * kPairsPerTask + j * p.cpairs;  // flattened (slot, pair) index
    const int bs = fp0 / I;                                      // both pairs are in this slot
    const int pr = fp0 - bs * I + (g >> 1);
    // row r (= lane group) of the pairs: gate of pair r / 2 for even r, up for odd
    auto brel = [&](int r) { return ((r & 1) ? I : 0) + (r >> 1); };
    // slot s: the rank-s expert (rank-ordered slots), else the s-th smallest id
    auto slot_expert = [&](int s) { return uniform(p.rank_slots ? sh.ids[s] : sh.sorted[s]); };
    const uint16_t* bbase = L.gate_up + ((size_t)slot_expert(bs) * 2 * I + (fp0 - bs * I)) * H;
    // the four rows of H bf16, H / 2 + 16 words apart (see kBRowStride)
    uint64_t* brows = reinterpret_cast<uint64_t*>(sh.xs + kBRowsAt);
    const int bstride = (H / 2 + 16) / 2;  // 8-byte words
    if (w == 0 && own_pairs) {
        // 1 KB per wave instruction (16 bytes per lane)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            for (int c0 = 0; c0 < H / 512; ++c0) {
                __builtin_amdgcn_global_load_lds(
                    reinterpret_cast<const void*>(bbase + (size_t)brel(r) * H + c0 * 512 + 8 * lane),
                    (__attribute__((address_space(3))) void*)(brows + r * bstride + c0 * 128), 16, 0, 0);
            }
        }
    }
    // Down rows: requested once the lead wave's gate/up rows have landed, so
    // that during the layer's burst the gate/up rows (needed first, by every
    // B task) go ahead of the down rows (needed only after the gate/up phase).
    auto issue_down = [&]() {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int m = w + 4 * k;
            if (m >= 1 && m <= U) {
                const uint16_t* wm = L.down + (size_t)slot_expert(m - 1) * (size_t)H * I;
                line_issue(c[k], wm + (size_t)r0 * I, (uint32_t)(g * I * 2), q);
            }
        }
    };
    // route weights and the shared-gate sigmoid (exponentials above the block
    // input); task 0 also reports the layer's ids, scores and sigmoid and
    // rejects a NaN logit (src/decoder_layer.rs:279-281)
    const int tid = threadIdx.x;
    if (j == 0 && p.order == 0) {
        int nan = 0;
        for (int e = tid; e < p.ls; e += kThreads) nan |= (e < p.E) && ((sh.lg[e] & 0x7fffu) > 0x7f80u);
        if (wg_any(sh.red, nan) && tid == 0) atomicCAS(p.error, 0, 2);
    }
    // wave 1 scores while the lead wave runs the pairs (the barrier before
    // the staging orders both before anything reads the scores or overwrites
    // the exponentials)
    score_experts<NT>(p, li, sh, j == 0, kMaxHidden, 1, false);
    FW_TRACE_MARK_IF(w == 1 && lane == 0, slot, 6);
    st.scored = li;
    const int seq = li * p.n_c + j;  // this task's mark in sh.rows_landed
    if (w != 0) {
        // the down rows go out once the lead wave's gate/up rows are in (the
        // gate/up rows, needed first, go ahead of them in the layer's burst)
        while (__hip_atomic_load(&sh.rows_landed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != seq)
            __builtin_amdgcn_s_sleep(1);
        issue_down();
    }
    // lead wave: as soon as its rows are in LDS (its own loads: no barrier),
    // the two pairs' dots and SwiGLU (src/expert.rs:514-571); lane 0 stores
    // the word of both activations
    if (w == 0 && !own_pairs) {
        if (lane == 0) __hip_atomic_store(&sh.rows_landed, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        issue_down();
    } else if (w == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        FW_TRACE_MARK_IF(lane == 0, slot, 10);
        if (lane == 0) __hip_atomic_store(&sh.rows_landed, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        float acc[1][2];
        line_chains_lds<MBH, 2>(brows + g * bstride, H / 32, sh.xs, q, acc);
        float d = tree32_reduce_lines(acc[0][0], acc[0][1]);
        if (q == 0) d = tree32_finish(d, bbase + (size_t)brel(g) * H, sh.xs, H);
        const uint32_t bits = to_bf16(d);
        const uint32_t up = (uint32_t)__shfl((int)bits, (lane + kLanesPerRow) & 63, kWave);
        const uint32_t a = swiglu_bf16(bits, up, sh.exp2tab);
        const uint32_t a1 = (uint32_t)__shfl((int)a, (lane + 2 * kLanesPerRow) & 63, kWave);
        if (lane == 0)
            coherent_store64(p.act + (size_t)(li * p.S + bs) * (I / 2) + pr / 2, tagged(a | (a1 << 16), epoch));
        FW_TRACE_MARK_IF(lane == 0, slot, 11);
        issue_down();
    }
    bool ok = true;
    // No wait for the gate/up phase: the staging below reads every activation
    // word until it carries this launch's epoch (a word is complete when its
    // tag is), so the down rows start as soon as the task's own words are in.
    // The staging overwrites the block input and the gate/up rows: the lead
    // wave's pairs must be done first.
    wg_sync();
    FW_TRACE_STAMP(t1);
    // every activation vector of the task at once (matrices 0..U <= 11)
    st.loaded = st.staged = -1;
    if (!stage_acts_direct<MBI>(p, li, epoch, sh, U, slot)) return false;
    FW_TRACE_MARK(slot, 4);
    // payloads: the low halves of the tagged words
    const uint32_t* act_lds = reinterpret_cast<const uint32_t*>(sh.xs);
    const int act_stride = 2 * (max(I, Is) / 2);
    // Each down-row dot leaves its weighted value: src/decoder_layer.rs:528-545
    // weighted = bf16(down * score) for slot m - 1 (one token: the slots are
    // its experts in ascending id, the order of its weights), and
    // src/decoder_layer.rs:563-575 gated = bf16(shared_down * sigmoid) for m = 0.
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int m = w + 4 * k;
        if (m <= U) {
            const uint32_t bits = down_row_lds<MBI, 2>(c[k], (m == 0 ? Is : I) / 32, act_lds + m * act_stride, q);
            if (q == 0) {
                // the slot's route weight (tweight is by ascending-id position)
                const uint32_t scale =
                    m == 0 ? sh.sig[0] : sh.tweight[p.rank_slots ? sh.pos[m - 1] : m - 1];
                sh.res[m * kRowsPerCTask + g] = to_bf16(mul_rn(from_bf16(bits), from_bf16(scale)));
            }
        }
    }
    FW_TRACE_MARK(slot, 0);
    if (!wg_all(sh.red, ok)) return false;
    if (mixer) {
        const int gg = rt;
        // the weighted values summed in ascending expert order from bf16 zero,
        // rounding after each add, then the gated shared output
        uint32_t mix = to_bf16(0.0f);
        for (int k0 = 0; k0 < K; k0 += 8) {
            uint32_t d[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                // the matrix of the expert at ascending-id position k0 + i
                if (k0 + i < K) d[i] = sh.res[(1 + (p.rank_slots ? sh.rank_at[k0 + i] : k0 + i)) * kRowsPerCTask + gg];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (k0 + i < K) mix = add_bf16(mix, d[i]);
            }
        }
        const uint32_t o = add_bf16(mix, sh.res[gg]);
        const uint32_t xn = add_bf16((sh.rin[gg] >> (16 * (gg & 1))) & 0xffffu, o);
        const uint32_t o_odd = (uint32_t)__shfl_xor((int)o, 1, kWave);
        const uint32_t x_odd = (uint32_t)__shfl_xor((int)xn, 1, kWave);
        if ((gg & 1) == 0) {
            const uint32_t o2 = o | (o_odd << 16), x2 = xn | (x_odd << 16);
            reinterpret_cast<uint32_t*>(p.out + (size_t)li * H)[at] = o2;
            coherent_store64(p.xw + (size_t)(li + p.chains) * H / 2 + at, tagged(x2, epoch));
            if (li + p.chains >= p.nlayers && p.x_final != nullptr)
                reinterpret_cast<uint32_t*>(p.x_final)[(size_t)(li + p.chains - p.nlayers) * H / 2 + at] = x2;
        }
    }
    if (!wg_all(sh.red, ok)) return false;
    FW_TRACE_MARK(slot, 1);
    publish(phase_counters(p, li, kCntC), p.n_c, j, phase_flags(p, li, kCntC), epoch);
    FW_TRACE_STAMP(t2);
    FW_TRACE_WRITE(slot, kTaskDown, t0, t1, t2);
    return true;
}

// ---- roles -----------------------------------------------------------------------------
//
// Per layer the rows role runs the R, S and the first nb_rows B tasks; the
// combine role runs the remaining B tasks, then the C tasks. Both
// walk their list in (layer, phase) order, task t on workgroup t mod (role
// size).

template <int NT, int MBH, int TK, class SH>
__device__ __forceinline__ void rows_role(const DecodeParams* __restrict__ P, uint32_t epoch, SH& sh,
                                          int rank) {
    const DecodeParams& p = *P;
    const int per = p.n_router + p.n_shared + p.nb_rows;
    const int total = p.nlayers * per;
    LdsState st;
    for (int t = rank; t < total; t += p.g_rows) {
        const int li = t / per;
        const int j = t - li * per;
        bool ok;
        if (j < p.n_router) {
            ok = router_task<NT, MBH>(p, epoch, sh, st, li, j);
        } else if (j < p.n_router + p.n_shared) {
            ok = pairs_task<NT, MBH, TK>(p, epoch, sh, st, li, j - p.n_router, true);
        } else {
            ok = pairs_task<NT, MBH, TK>(p, epoch, sh, st, li, j - p.n_router - p.n_shared, false);
        }
        if (!ok) return;
    }
}

template <int NT, int MBH, int MBI, int TK, class SH>
__device__ __forceinline__ void combine_role(const DecodeParams* __restrict__ P, uint32_t epoch, SH& sh,
                                             int rank) {
    const DecodeParams& p = *P;
    const int nb_comb = p.cpairs > 0 ? 0 : p.n_b - p.nb_rows;
    const int per = nb_comb + p.n_c;
    const int total = p.nlayers * per;
    LdsState st;
    for (int t = rank; t < total; t += p.g_comb) {
        const int li = t / per;
        const int j = t - li * per;
        bool ok;
        if constexpr (fused_combine(NT, MBH, MBI)) {
            // the host runs one-token steps it cannot fuse on the two-token kernel
            // (two instantiations: a runtime flag inside would cost the
            // common path its scheduling)
            ok = p.cpairs > 0 ? combine_task_fused<NT, MBH, MBI, TK, true>(p, epoch, sh, st, li, j)
                              : combine_task_fused<NT, MBH, MBI, TK, false>(p, epoch, sh, st, li, j);
        } else if (j < nb_comb) {
            ok = pairs_task<NT, MBH, TK>(p, epoch, sh, st, li, p.nb_rows + j, false);
        } else {
            ok = combine_task<NT, MBI, TK>(p, epoch, sh, st, li, j - nb_comb);
        }
        if (!ok) return;
    }
}

// NT tokens; MBH, MBI: 32-column blocks held per hidden row / down row; TK:
// logits per lane in the top-k.
template <int NT, int MBH, int MBI, int TK>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(NT <= 2 ? 4 : 2)))
k_moe_decode(const DecodeParams* __restrict__ P, uint32_t epoch) {
    __shared__ DecodeShared<NT, MBI> sh;
    if (threadIdx.x < 32) sh.exp2tab[threadIdx.x] = c_exp2_table[threadIdx.x];
    if (threadIdx.x == 0) sh.rows_landed = -1;
    wg_sync();
    const int b = (int)blockIdx.x;
    const int G = (int)gridDim.x;
    if (b < P->g_rows) {
        rows_role<NT, MBH, TK>(P, epoch, sh, b);
    } else if (b < P->g_rows + P->g_comb) {
        combine_role<NT, MBH, MBI, TK>(P, epoch, sh, b - P->g_rows);
    }
    // Completed counters zero themselves. After a failure some are left
    // partly counted: the last workgroup out then zeroes them all.
    wg_sync();
    if (threadIdx.x == 0) {
        uint32_t* done = P->counters + (size_t)P->nlayers * kCountersPerLayer * kCounterGroupWords;
        if (count_task(done, G, b) && coherent_load(P->error) != 0) {
            for (int i = 0; i < P->nlayers * kCountersPerLayer * kCounterGroupWords; i += kCounterStride)
                __hip_atomic_store(P->counters + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Every variant the host dispatches on; instantiated in fw_decode_kernels.hip
// (one translation unit per token count, compiled in parallel).
#define FW_DECODE_VARIANTS_FOR(X, NT) \
    X(NT, 64, 16, 8)                  \
    X(NT, 64, 32, 8)                  \
    X(NT, 80, 16, 8)                  \
    X(NT, 80, 32, 8)                  \
    X(NT, 64, 16, 16)                 \
    X(NT, 64, 32, 16)                 \
    X(NT, 80, 16, 16)                 \
    X(NT, 80, 32, 16)
// One-token variants whose fused C task holds down rows of up to 640 columns
// (the reference model's I = Is = 640).
#define FW_DECODE_VARIANTS_ONE_TOKEN(X) \
    X(1, 64, 20, 8)                     \
    X(1, 80, 20, 8)                     \
    X(1, 64, 20, 16)                    \
    X(1, 80, 20, 16)
#define FW_DECODE_VARIANTS(X)     \
    FW_DECODE_VARIANTS_FOR(X, 1)  \
    FW_DECODE_VARIANTS_FOR(X, 2)  \
    FW_DECODE_VARIANTS_FOR(X, 3)  \
    FW_DECODE_VARIANTS_FOR(X, 4)

}  // namespace fw
