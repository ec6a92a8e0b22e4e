// Persistent decode kernel: every resident layer of a T <= 4 token step in one
// launch (router -> top-k -> routed and shared SwiGLU experts -> ordered
// mixture -> combine, chained through the residual stream).
//
// The co-resident workgroups (cooperative launch) are split into three roles,
// each walking its own task list in (layer, phase) order:
//
//   rows     R  router rows, 16 per task (rows [0, E)), plus one task for the
//               shared_expert_gate row                -> logits[t][0..E]
//            S  shared gate/up pairs, 8 per task, fused SwiGLU -> shared_act
//            B  routed gate/up pairs, 8 per task per slot, fused SwiGLU -> act
//   combine  C  4 hidden rows per task: the down rows of every selected
//               expert ("slot") and of the shared expert, route weighting, the
//               ascending-id bf16 mixture, the gated shared output, the block
//               output and the next residual
//   top-k    K  one workgroup: ids, the union of selected experts, scores and
//               the shared-gate sigmoid of every layer
//
// R and S of layer l wait for C of layer l-1; K waits for R; B for K's ids; C
// for B, S and K's scores. Every wait points to an earlier phase, and within
// a role earlier phases come first, so with all workgroups resident the
// earliest unfinished task can always run. Weight loads never depend on
// activations, so tasks issue them before they wait: R and S stream their rows
// while the previous layer finishes, C its down rows while B runs. Waits are
// counters in HBM (fw_device.h), each bounded by a wall-clock limit and by a
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
    const uint16_t* shared_up;    // [Is][H]
    const uint16_t* shared_down;  // [H][Is]
};

enum DecodeCounter : int {
    kCntRouter = 0,
    kCntShared = 1,
    kCntIds = 2,
    kCntScores = 3,
    kCntB = 4,
    kCntC = 5,
    kCountersPerLayer = 8
};

enum DecodeTaskKind : int { kTaskRouter = 0, kTaskShared = 1, kTaskTopk = 2, kTaskGateUp = 3, kTaskDown = 4 };

constexpr int kRouterRowsPerTask = 16;
constexpr int kPairsPerTask = 8;
constexpr int kRowsPerCTask = 4;
constexpr int kMaxTokens = 4;
constexpr int kMaxTopK = 32;
constexpr int kMaxSlots = kMaxTopK * kMaxTokens;
constexpr int kMaxHidden = 2560;
constexpr int kMaxExperts = 1024;
constexpr int kThreads = 256;
constexpr int kXRegs = kMaxHidden / 2 / kThreads;  // bf16 pairs of x per thread and token

struct DecodeParams {
    const DecodeLayer* layers;  // [nlayers], already offset to the first layer
    int nlayers;
    int T, H, I, E, K, Is;
    int order;         // 0 TREE32, 1 FOLD
    int prenorm;       // block input = rms_norm(residual) (chained step), else the input
    int bias_feature;  // with prenorm: block input [H-1] = 1.0
    // per-layer buffers (index 0 = first layer of the launch)
    const uint16_t* x_in;     // [T][H] input of the first layer
    uint16_t* x;              // [nlayers + 1][T][H] residual stream (x[0] unused)
    uint16_t* x_final;        // [T][H] residual after the last layer, or null
    uint16_t* h;              // [nlayers][T][H] normalised block input (chained step)
    uint16_t* out;            // [nlayers][T][H]
    uint16_t* logits;         // [nlayers][T][ls]: router rows [0, E), shared_expert_gate at gi
    int ls, gi;               // logit row stride (even) and shared_expert_gate index (even)
    int32_t* ids;             // [nlayers][T][K]
    uint16_t* scores;         // [nlayers][T][K]
    int32_t* slot_expert;     // [nlayers][S]
    uint32_t* slot_tokens;    // [nlayers][S]
    int32_t* union_count;     // [nlayers]
    int32_t* token_slots;     // [nlayers][T][K] slots in ascending expert id
    uint32_t* token_weights;  // [nlayers][T][K] bf16 score of that slot (low half)
    uint32_t* sig;            // [nlayers][T] bf16 sigmoid of the shared gate logit (low half)
    uint16_t* shared_act;     // [nlayers][T][Is]
    uint16_t* act;            // [nlayers][S][T][I]
    uint32_t* counters;       // [nlayers][kCountersPerLayer] then 1 done counter
    int32_t* error;           // 0 ok, 1 timeout, 2 NaN router logit
    uint64_t limit_ticks;
    int n_router, n_shared, n_b, n_c, S;
    int n_rows;               // R + S + B tasks per layer
    int g_rows, g_comb;       // workgroups of the rows and combine roles; one more runs top-k
    uint64_t* trace;          // profiling builds only
};

// Task timing (wall clock) for profiling builds only. Trace slot of a task:
// layer * (n_rows + 1 + n_c) + [R, S, B | K | C] index.
#ifdef FW_DECODE_TRACE
constexpr int kTraceWords = 8;  // start, dependency met, end, wg << 8 | kind, 4 stage marks
#define FW_TRACE_STAMP(var) const uint64_t var = wall_clock64()
#define FW_TRACE_MARK(slot_, k)                                                    \
    do {                                                                           \
        if (threadIdx.x == 0 && p.trace != nullptr)                                \
            p.trace[(size_t)(slot_) * kTraceWords + 4 + (k)] = wall_clock64();     \
    } while (0)
#define FW_TRACE_WRITE(slot_, kind, a, b, c)                                       \
    do {                                                                           \
        if (threadIdx.x == 0 && p.trace != nullptr) {                              \
            uint64_t* tr = p.trace + (size_t)(slot_) * kTraceWords;                \
            tr[0] = (a);                                                           \
            tr[1] = (b);                                                           \
            tr[2] = (c);                                                           \
            tr[3] = ((uint64_t)blockIdx.x << 8) | (uint64_t)(kind);                \
        }                                                                          \
    } while (0)
#else
#define FW_TRACE_STAMP(var)
#define FW_TRACE_MARK(slot_, k)
#define FW_TRACE_WRITE(slot_, kind, a, b, c)
#endif

__device__ __constant__ uint64_t c_exp2_table[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

template <int NT>
struct DecodeShared {
    float xs[NT * kMaxHidden];  // rows: block input as f32; top-k: logits then exponentials
    uint64_t exp2tab[32];
    uint16_t res[(kMaxSlots + 1) * kMaxTokens * kRowsPerCTask];
    int32_t ids[kMaxTokens * kMaxTopK];
    int32_t sorted[kMaxSlots];
    int32_t slot_of[kMaxTokens * kMaxTopK];
    int32_t first[kMaxTokens * kMaxTopK];
    int32_t tslot[kMaxTokens * kMaxTopK];
    uint16_t tweight[kMaxTokens * kMaxTopK];
    uint16_t sig[kMaxTokens];
    float inv[kMaxTokens];
    int32_t nunion;
    int32_t flag;
};

// Residual-stream input of layer li of the launch.
__device__ __forceinline__ const uint16_t* layer_input(const DecodeParams& p, int li) {
    return li == 0 ? p.x_in : p.x + (size_t)li * p.T * p.H;
}

// Block input of layer li into LDS as f32, [T][H]. In the chained step the
// block input is the pre-norm of the residual (workload glue, not the
// reference's block): h = bf16(r * 1/sqrt(mean(r^2) + 1e-6)), mean(r^2)
// through the reference's dot order (32 chains, tree, +0.0) divided by H;
// h[H-1] = 1.0 with the bias feature. Wave t normalises token t. With
// from_h the normalised input is read from p.h (written by the layer's first
// router task) instead of being recomputed.
template <int NT>
__device__ __forceinline__ void stage_input(const DecodeParams& p, int li, bool from_h, DecodeShared<NT>& sh) {
    const int T = p.T, n = p.H;
    const bool norm = p.prenorm && !from_h;
    const uint16_t* src = from_h ? p.h + (size_t)li * T * n : layer_input(p, li);
    const uint32_t* x2 = reinterpret_cast<const uint32_t*>(src);
    float* xs = sh.xs;
    const int pairs = T * n / 2;
    uint32_t v[NT * kXRegs];
#pragma unroll
    for (int k = 0; k < NT * kXRegs; ++k) {
        const int i = (int)threadIdx.x + k * kThreads;
        v[k] = coherent_load(x2 + (i < pairs ? i : pairs - 1));
    }
#pragma unroll
    for (int k = 0; k < NT * kXRegs; ++k) {
        const int i = (int)threadIdx.x + k * kThreads;
        if (i < pairs) *reinterpret_cast<float2*>(xs + 2 * i) = make_float2(bf16_lo(v[k]), bf16_hi(v[k]));
    }
    __syncthreads();
    if (!norm) return;
    const int w = wave_id(), lane = lane_id();
    if (w < T) {
        const float* r = xs + w * n;
        float c = 0.0f;
        if (lane < 32) {
            for (int b = 0; b < n / 32; ++b) {
                float e = r[32 * b + lane];
                c = add_rn(c, mul_rn(e, e));
            }
        }
        c = add_rn(c, __shfl_down(c, 16, kWave));  // a'[j] = c[j] + c[j+16]
        c = add_rn(c, __shfl_down(c, 8, kWave));   // a''[j] = a'[j] + a'[j+8]
        c = add_rn(c, __shfl_down(c, 4, kWave));   // a3[j] = a''[j] + a''[j+4]
        float pair = add_rn(c, __shfl_down(c, 1, kWave));  // (a0+a1) in lane 0, (a2+a3) in lane 2
        float ss = add_rn(add_rn(pair, __shfl_down(pair, 2, kWave)), 0.0f);
        if (lane == 0) sh.inv[w] = 1.0f / sqrtf(add_rn(ss / (float)n, 1e-6f));
    }
    __syncthreads();
    for (int i = threadIdx.x; i < T * n; i += kThreads) {
        float hv = from_bf16(to_bf16(mul_rn(xs[i], sh.inv[i / n])));
        if (p.bias_feature && i % n == n - 1) hv = 1.0f;
        xs[i] = hv;
    }
    __syncthreads();
}

// ---- rows role: R, S and B tasks ------------------------------------------------------
//
// A wave covers 4 rows (16 lanes each). R task: 16 router rows; the last R
// task of a layer is the shared_expert_gate row alone. S and B tasks: 8
// gate/up pairs, wave w taking pairs 2w and 2w+1 with its lane groups 0, 1 on
// the gate rows and 2, 3 on the up rows, so SwiGLU joins lane l and l + 32.
// Each task has one point where its weight loads are issued: before its
// dependency wait for R and S, right after it for B (whose expert comes from
// the top-k).

template <int NT, int MBH>
__device__ __forceinline__ void rows_role(const DecodeParams* __restrict__ P, DecodeShared<NT>& sh, int rank) {
    const DecodeParams& p = *P;
    const int lane = lane_id(), w = wave_id(), g = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int T = p.T, H = p.H, I = p.I, E = p.E, Is = p.Is;
    const int nbh = H / 32;
    const int per_slot = I / kPairsPerTask;
    const int total = p.nlayers * p.n_rows;
    for (int t = rank; t < total; t += p.g_rows) {
        FW_TRACE_STAMP(t0);
        const int li = t / p.n_rows;
        const int j = t - li * p.n_rows;
        const int slot_trace = li * (p.n_rows + 1 + p.n_c) + j;
        (void)slot_trace;
        const DecodeLayer& L = p.layers[li];
        uint32_t* cnt = p.counters + (size_t)li * kCountersPerLayer;
        const int kind = j < p.n_router ? kTaskRouter : (j < p.n_router + p.n_shared ? kTaskShared : kTaskGateUp);
        // rows of this lane group
        const uint16_t* wrow;
        int out_index;
        bool valid = true, wave_active = true, fold = false, work = true;
        uint32_t mask = (1u << T) - 1u;
        uint16_t* act_out = nullptr;
        int act_stride = 0;
        if (kind == kTaskRouter) {
            const bool gate_task = j == p.n_router - 1;
            const int row0 = gate_task ? E : j * kRouterRowsPerTask;
            const int rows = gate_task ? 1 : min(kRouterRowsPerTask, E - row0);
            const int rin = w * kRowsPerWave + g;
            wave_active = w * kRowsPerWave < rows;
            valid = rin < rows;
            fold = p.order == 1 && !gate_task;
            out_index = row0 + (valid ? rin : 0);
            wrow = L.router + (size_t)out_index * H;
        } else {
            int pair0;
            if (kind == kTaskShared) {
                pair0 = (j - p.n_router) * kPairsPerTask;
                act_out = p.shared_act + (size_t)li * T * Is;
                act_stride = Is;
                wrow = g < 2 ? L.shared_gate : L.shared_up;
            } else {
                const int jb = j - p.n_router - p.n_shared;
                const int s = jb / per_slot;
                if (!wait_at_least(cnt + kCntIds, 1u, p.error, p.limit_ticks, &sh.flag)) return;
                const int e = uniform(coherent_load(p.slot_expert + (size_t)li * p.S + s));
                work = e >= 0;
                mask = work ? (uint32_t)uniform((int)coherent_load(p.slot_tokens + (size_t)li * p.S + s)) : 0u;
                const uint16_t* gate_w = L.gate_up + (size_t)(work ? e : 0) * 2 * I * H;
                pair0 = (jb - s * per_slot) * kPairsPerTask;
                act_out = p.act + ((size_t)li * p.S + s) * (size_t)T * I;
                act_stride = I;
                wrow = g < 2 ? gate_w : gate_w + (size_t)I * H;
            }
            out_index = pair0 + 2 * w + (g & 1);
            wrow += (size_t)out_index * H;
        }
        RowShare<MBH> rs;
        if (work && wave_active && !fold) row_issue(rs, reinterpret_cast<const uint32_t*>(wrow), nbh, q);
        if (kind != kTaskGateUp && li > 0 &&
            !wait_at_least(p.counters + (size_t)(li - 1) * kCountersPerLayer + kCntC, (uint32_t)p.n_c, p.error,
                           p.limit_ticks, &sh.flag))
            return;
        FW_TRACE_STAMP(t1);
        if (work) {
            stage_input<NT>(p, li, kind == kTaskGateUp && p.prenorm, sh);
            FW_TRACE_MARK(slot_trace, 0);
            if (kind == kTaskRouter && j == 0 && p.prenorm) {
                // the layer's normalised input, for its B tasks
                uint32_t* h2 = reinterpret_cast<uint32_t*>(p.h + (size_t)li * T * H);
                for (int i = threadIdx.x; i < T * H / 2; i += kThreads)
                    coherent_store(h2 + i, to_bf16(sh.xs[2 * i]) | (to_bf16(sh.xs[2 * i + 1]) << 16));
            }
            if (fold) {
                // src/router.rs:228-240: one lane folds one row; lanes 0 and 2
                // store the pairs of rows (r, r + 1).
                uint32_t* logits = reinterpret_cast<uint32_t*>(p.logits + (size_t)li * T * p.ls);
                const int r = j * kRouterRowsPerTask + w * kRowsPerWave + lane;
                const bool mine = lane < kRowsPerWave && r < E;
                for (int tt = 0; tt < T; ++tt) {
                    uint32_t bits = mine ? to_bf16(fold_row(L.router + (size_t)r * H, sh.xs + tt * H, H)) : 0u;
                    uint32_t next = (uint32_t)__shfl_down((int)bits, 1, kWave);
                    if (mine && (lane & 1) == 0) coherent_store(logits + (tt * p.ls + r) / 2, bits | (next << 16));
                }
            } else if (wave_active) {
                float acc[NT][2];
                row_chains<NT, MBH>(rs, nbh, sh.xs, H, q, acc);
                uint32_t bits[NT];
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
                    float d = tree32_reduce(acc[tt][0], acc[tt][1]);
                    if (q == 0) d = tree32_finish(d, wrow, sh.xs + tt * H, H);
                    bits[tt] = to_bf16(d);
                }
                if (kind == kTaskRouter) {
                    // groups 0 and 2 store the pairs (row, row + 1); the gate
                    // logit goes to its own slot with a zero beside it
                    uint32_t* logits = reinterpret_cast<uint32_t*>(p.logits + (size_t)li * T * p.ls);
                    const bool gate_task = j == p.n_router - 1;
                    const int at = gate_task ? p.gi : out_index;
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
                        uint32_t next = (uint32_t)__shfl((int)bits[tt], (lane + kLanesPerRow) & 63, kWave);
                        if (gate_task) next = 0u;
                        if (q == 0 && (g & 1) == 0 && valid) coherent_store(logits + (tt * p.ls + at) / 2, bits[tt] | (next << 16));
                    }
                } else {
                    // gate (groups 0, 1) meets up (groups 2, 3): lane l takes lane l + 32;
                    // group 0 stores the pair (pair, pair + 1) with group 1's result
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
                        uint32_t up = (uint32_t)__shfl((int)bits[tt], (lane + 32) & 63, kWave);
                        uint32_t a = swiglu_bf16(bits[tt], up, sh.exp2tab);
                        uint32_t b = (uint32_t)__shfl((int)a, (lane + kLanesPerRow) & 63, kWave);
                        if (g == 0 && q == 0 && (mask & (1u << tt)))
                            coherent_store(reinterpret_cast<uint32_t*>(act_out + (size_t)tt * act_stride + out_index), a | (b << 16));
                    }
                }
            }
            FW_TRACE_MARK(slot_trace, 1);
        }
        publish(cnt + (kind == kTaskRouter ? kCntRouter : (kind == kTaskShared ? kCntShared : kCntB)));
        FW_TRACE_STAMP(t2);
        FW_TRACE_WRITE(slot_trace, kind, t0, t1, t2);
    }
}

// ---- combine role: C tasks -----------------------------------------------------------

template <int NT, int MBI>
__device__ __forceinline__ void combine_role(const DecodeParams* __restrict__ P, DecodeShared<NT>& sh, int rank) {
    const DecodeParams& p = *P;
    const int lane = lane_id(), w = wave_id(), g = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int T = p.T, H = p.H, I = p.I, Is = p.Is, K = p.K;
    const uint32_t all_tokens = (1u << T) - 1u;
    const int total = p.nlayers * p.n_c;
    for (int t = rank; t < total; t += p.g_comb) {
        FW_TRACE_STAMP(t0);
        const int li = t / p.n_c;
        const int j = t - li * p.n_c;
        const int slot_trace = li * (p.n_rows + 1 + p.n_c) + p.n_rows + 1 + j;
        (void)slot_trace;
        const DecodeLayer& L = p.layers[li];
        uint32_t* cnt = p.counters + (size_t)li * kCountersPerLayer;
        if (!wait_at_least(cnt + kCntIds, 1u, p.error, p.limit_ticks, &sh.flag)) return;
        const int r0 = j * kRowsPerCTask;
        const int U = uniform(coherent_load(p.union_count + li));
        const int32_t* slot_expert = p.slot_expert + (size_t)li * p.S;
        const uint32_t* slot_tokens = p.slot_tokens + (size_t)li * p.S;
        const int row = r0 + g;
        // Down rows of up to 4 matrices per wave and batch (slots m0, m0+4, ...;
        // the shared expert is matrix U). The first batch is issued before
        // waiting for the gate/up phase.
        RowShare<MBI> rs0, rs1, rs2, rs3;
#define FW_ISSUE_DOWN(RS, M)                                                                     \
    do {                                                                                         \
        const int m_ = (M);                                                                      \
        if (m_ <= U) {                                                                           \
            const bool shared_ = m_ == U;                                                        \
            const int kd_ = shared_ ? Is : I;                                                    \
            const uint16_t* wm_ =                                                                \
                shared_ ? L.shared_down : L.down + (size_t)uniform(coherent_load(slot_expert + m_)) * (size_t)H * I; \
            row_issue(RS, reinterpret_cast<const uint32_t*>(wm_ + (size_t)row * kd_), kd_ / 32, q); \
        }                                                                                        \
    } while (0)
#define FW_ISSUE_BATCH(M0)             \
    do {                               \
        FW_ISSUE_DOWN(rs0, (M0));      \
        FW_ISSUE_DOWN(rs1, (M0) + 4);  \
        FW_ISSUE_DOWN(rs2, (M0) + 8);  \
        FW_ISSUE_DOWN(rs3, (M0) + 12); \
    } while (0)
#define FW_DOWN_DOT(RS, M)                                                                       \
    do {                                                                                         \
        const int m_ = (M);                                                                      \
        if (m_ <= U) {                                                                           \
            const bool shared_ = m_ == U;                                                        \
            const int kd_ = shared_ ? Is : I;                                                    \
            const uint32_t mask_ = shared_ ? all_tokens : (uint32_t)uniform((int)coherent_load(slot_tokens + m_)); \
            const uint16_t* actv_ = shared_ ? p.shared_act + (size_t)li * T * Is                 \
                                            : p.act + ((size_t)li * p.S + m_) * (size_t)T * I;   \
            float acc_[NT][2];                                                                   \
            row_chains_gx<NT, MBI>(RS, kd_ / 32, actv_, kd_, q, mask_, acc_);                    \
            _Pragma("unroll") for (int t_ = 0; t_ < NT; ++t_) {                                  \
                /* K % 32 == 0 here: the tail sum is +0.0 */                                     \
                float d_ = add_rn(tree32_reduce(acc_[t_][0], acc_[t_][1]), 0.0f);                \
                if (q == 0 && (mask_ & (1u << t_)))                                              \
                    sh.res[(m_ * kMaxTokens + t_) * kRowsPerCTask + g] = to_bf16(d_);            \
            }                                                                                    \
        }                                                                                        \
    } while (0)
        FW_ISSUE_BATCH(w);
        if (!(wait_at_least(cnt + kCntB, (uint32_t)p.n_b, p.error, p.limit_ticks, &sh.flag) &&
              wait_at_least(cnt + kCntShared, (uint32_t)p.n_shared, p.error, p.limit_ticks, &sh.flag) &&
              wait_at_least(cnt + kCntScores, 1u, p.error, p.limit_ticks, &sh.flag)))
            return;
        FW_TRACE_STAMP(t1);
        // Per-token slot order, weights and shared gate into LDS (one round trip).
        const int tid = threadIdx.x;
        if (tid < T * K) {
            sh.tslot[tid] = coherent_load(p.token_slots + (size_t)li * T * K + tid);
            sh.tweight[tid] = (uint16_t)coherent_load(p.token_weights + (size_t)li * T * K + tid);
        }
        if (tid < T) sh.sig[tid] = (uint16_t)coherent_load(p.sig + (size_t)li * T + tid);
        for (int m0 = w; m0 <= U; m0 += 16) {
            if (m0 != w) FW_ISSUE_BATCH(m0);
            FW_DOWN_DOT(rs0, m0);
            FW_DOWN_DOT(rs1, m0 + 4);
            FW_DOWN_DOT(rs2, m0 + 8);
            FW_DOWN_DOT(rs3, m0 + 12);
        }
#undef FW_DOWN_DOT
#undef FW_ISSUE_BATCH
#undef FW_ISSUE_DOWN
        FW_TRACE_MARK(slot_trace, 0);
        __syncthreads();
        if (tid < T * kRowsPerCTask / 2) {
            // one thread per token and pair of hidden rows
            const int tt = tid / (kRowsPerCTask / 2);
            const int g0 = 2 * (tid % (kRowsPerCTask / 2));
            const size_t at = ((size_t)tt * H + r0 + g0) / 2;
            const uint32_t rin = coherent_load(reinterpret_cast<const uint32_t*>(layer_input(p, li)) + at);
            uint32_t o2 = 0, x2 = 0;
            for (int half = 0; half < 2; ++half) {
                const int gg = g0 + half;
                // src/decoder_layer.rs:528-545: weighted = bf16(down * score), summed
                // in ascending expert order from bf16 zero, rounding after each add.
                uint32_t mix = to_bf16(0.0f);
                for (int k = 0; k < K; ++k) {
                    uint32_t d = sh.res[(sh.tslot[tt * K + k] * kMaxTokens + tt) * kRowsPerCTask + gg];
                    uint32_t weighted = to_bf16(mul_rn(from_bf16(d), from_bf16(sh.tweight[tt * K + k])));
                    mix = add_bf16(mix, weighted);
                }
                // src/decoder_layer.rs:563-575: gated = bf16(shared_down * sigmoid).
                uint32_t sd = sh.res[(U * kMaxTokens + tt) * kRowsPerCTask + gg];
                uint32_t gated = to_bf16(mul_rn(from_bf16(sd), from_bf16(sh.sig[tt])));
                uint32_t o = add_bf16(mix, gated);
                uint32_t xn = add_bf16((rin >> (16 * half)) & 0xffffu, o);
                o2 |= o << (16 * half);
                x2 |= xn << (16 * half);
            }
            reinterpret_cast<uint32_t*>(p.out + (size_t)li * T * H)[at] = o2;
            coherent_store(reinterpret_cast<uint32_t*>(p.x + (size_t)(li + 1) * T * H) + at, x2);
            if (li + 1 == p.nlayers && p.x_final != nullptr) reinterpret_cast<uint32_t*>(p.x_final)[at] = x2;
        }
        FW_TRACE_MARK(slot_trace, 1);
        publish(cnt + kCntC);
        FW_TRACE_STAMP(t2);
        FW_TRACE_WRITE(slot_trace, kTaskDown, t0, t1, t2);
    }
}

// ---- top-k role: one workgroup, every layer ------------------------------------------

template <int NT>
__device__ __forceinline__ void topk_role(const DecodeParams* __restrict__ P, DecodeShared<NT>& sh) {
    const DecodeParams& p = *P;
    const int lane = lane_id(), w = wave_id(), tid = threadIdx.x;
    const int T = p.T, E = p.E, K = p.K, S = p.S;
    const int LS = p.ls;
    uint16_t* lg = reinterpret_cast<uint16_t*>(sh.xs);  // [T][LS]
    float* ex = sh.xs + T * LS / 2;                     // [T][E]
    for (int li = 0; li < p.nlayers; ++li) {
        FW_TRACE_STAMP(t0);
        const int slot_trace = li * (p.n_rows + 1 + p.n_c) + p.n_rows;
        (void)slot_trace;
        uint32_t* cnt = p.counters + (size_t)li * kCountersPerLayer;
        if (!wait_at_least(cnt + kCntRouter, (uint32_t)p.n_router, p.error, p.limit_ticks, &sh.flag)) return;
        FW_TRACE_STAMP(t1);
        const uint32_t* logits = reinterpret_cast<const uint32_t*>(p.logits + (size_t)li * T * LS);
        for (int i = tid; i < T * LS / 2; i += kThreads) reinterpret_cast<uint32_t*>(lg)[i] = coherent_load(logits + i);
        __syncthreads();
        if (w < T) {
            const uint16_t* lt = lg + w * LS;
            if (p.order == 0) {
                // src/decoder_layer.rs:279-281: NaN logits are rejected.
                int nan = 0;
                for (int e = lane; e < E; e += kWave) nan |= ((lt[e] & 0x7fffu) > 0x7f80u);
                if (__any(nan) && lane == 0) atomicCAS(p.error, 0, 2);
            }
            if (E <= 512) {
                wave_topk<8>(lt, E, K, sh.ids + w * kMaxTopK);
            } else {
                wave_topk<16>(lt, E, K, sh.ids + w * kMaxTopK);
            }
        }
        __syncthreads();
        FW_TRACE_MARK(slot_trace, 0);
        // Union of the selections in ascending expert id (the execution order,
        // src/decoder_layer.rs:422-424): entry i = (token i / K, rank i % K).
        const int n_sel = T * K;
        int my_id = -1;
        if (tid < n_sel) {
            my_id = sh.ids[(tid / K) * kMaxTopK + tid % K];
            int first = 1;
            for (int i = 0; i < tid; ++i) first &= (sh.ids[(i / K) * kMaxTopK + i % K] != my_id);
            sh.first[tid] = first;
        }
        __syncthreads();
        if (tid < n_sel) {
            int slot = 0;
            for (int i = 0; i < n_sel; ++i)
                slot += (sh.first[i] && sh.ids[(i / K) * kMaxTopK + i % K] < my_id) ? 1 : 0;
            sh.slot_of[tid] = slot;
            if (sh.first[tid]) sh.sorted[slot] = my_id;
            // position of this expert among the token's own ids, ascending
            const int tt = tid / K;
            int k = 0;
            for (int r = 0; r < K; ++r) k += (sh.ids[tt * kMaxTopK + r] < my_id) ? 1 : 0;
            sh.tslot[tt * K + k] = slot;
        }
        if (tid == 0) {
            int n = 0;
            for (int i = 0; i < n_sel; ++i) n += sh.first[i];
            sh.nunion = n;
        }
        __syncthreads();
        const int n = sh.nunion;
        if (tid < n_sel) {
            p.ids[(size_t)li * T * K + tid] = my_id;
            coherent_store(p.token_slots + (size_t)li * T * K + tid, sh.tslot[tid]);
        }
        if (tid < S) {
            uint32_t mask = 0;
            if (tid < n) {
                for (int i = 0; i < n_sel; ++i) mask |= (sh.slot_of[i] == tid) ? (1u << (i / K)) : 0u;
            }
            coherent_store(p.slot_expert + (size_t)li * S + tid, tid < n ? sh.sorted[tid] : -1);
            coherent_store(p.slot_tokens + (size_t)li * S + tid, mask);
        }
        if (tid == 0) coherent_store(p.union_count + li, n);
        FW_TRACE_MARK(slot_trace, 1);
        publish(cnt + kCntIds);
        FW_TRACE_MARK(slot_trace, 2);
        // Scores: src/router.rs:248-262 / src/decoder_layer.rs:290-306.
        if (w < T) {
            const uint16_t* lt = lg + w * LS;
            float* ew = ex + w * E;
            float mx = -__builtin_inff();
            for (int e = lane; e < E; e += kWave) mx = fmaxf(mx, from_bf16(lt[e]));
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
            for (int e = lane; e < E; e += kWave) ew[e] = expf_glibc(add_rn(from_bf16(lt[e]), -mx), sh.exp2tab);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            if (lane == 0) {
                // one sequential f32 sum in index order, 32 values read per batch
                float den = -0.0f;
                int e = 0;
                for (; e + 32 <= E; e += 32) {
                    float v[32];
#pragma unroll
                    for (int i = 0; i < 32; ++i) v[i] = ew[e + i];
#pragma unroll
                    for (int i = 0; i < 32; ++i) den = add_rn(den, v[i]);
                }
                for (; e < E; ++e) den = add_rn(den, ew[e]);
                const int32_t* tid_ids = sh.ids + w * kMaxTopK;
                float sel = -0.0f;
                for (int r = 0; r < K; ++r) sel = add_rn(sel, ew[tid_ids[r]] / den);
                for (int r = 0; r < K; ++r) {
                    uint16_t score = to_bf16((ew[tid_ids[r]] / den) / sel);
                    p.scores[(size_t)li * T * K + (size_t)w * K + r] = score;
                    // this expert's place in the token's ascending-id order
                    int k = 0;
                    for (int r2 = 0; r2 < K; ++r2) k += (tid_ids[r2] < tid_ids[r]) ? 1 : 0;
                    coherent_store(p.token_weights + (size_t)li * T * K + (size_t)w * K + k, score);
                }
                coherent_store(p.sig + (size_t)li * T + w, sigmoid_bf16(lt[p.gi], sh.exp2tab));
            }
        }
        FW_TRACE_MARK(slot_trace, 3);
        publish(cnt + kCntScores);
        FW_TRACE_STAMP(t2);
        FW_TRACE_WRITE(slot_trace, kTaskTopk, t0, t1, t2);
    }
}

template <int NT, int MBH, int MBI>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
k_moe_decode(const DecodeParams* __restrict__ P) {
    __shared__ DecodeShared<NT> sh;
    if (threadIdx.x < 32) sh.exp2tab[threadIdx.x] = c_exp2_table[threadIdx.x];
    __syncthreads();
    const int b = (int)blockIdx.x;
    const int G = (int)gridDim.x;
    if (b < P->g_rows) {
        rows_role<NT, MBH>(P, sh, b);
    } else if (b < P->g_rows + P->g_comb) {
        combine_role<NT, MBI>(P, sh, b - P->g_rows);
    } else {
        topk_role<NT>(P, sh);
    }
    // The last workgroup out zeroes every counter for the next launch.
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        uint32_t* done = P->counters + (size_t)P->nlayers * kCountersPerLayer;
        uint32_t prev = __hip_atomic_fetch_add(done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == (uint32_t)G - 1u) {
            for (int i = 0; i < P->nlayers * kCountersPerLayer; ++i) {
                __hip_atomic_store(P->counters + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(done, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace fw
