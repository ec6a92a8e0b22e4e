// Persistent decode kernel: every resident layer of a T <= 4 token step in one
// launch (router -> top-k -> routed and shared SwiGLU experts -> ordered
// mixture -> combine, chained through the residual stream).
//
// Work is a fixed list of tasks per layer, dealt round-robin to co-resident
// workgroups (cooperative launch) that take theirs in increasing order:
//
//   R  router rows, 16 per task (rows [0, E)), plus one task for the
//      shared_expert_gate row                    -> logits[t][0..E]
//   S  shared gate/up pairs, 8 per task, fused SwiGLU -> shared_act[t][Is]
//   K  one top-k task: ids, the union of selected experts ("slots"), scores,
//      and the shared-gate sigmoid
//   B  routed gate/up pairs, 8 per task per slot, fused SwiGLU -> act[s][t][I]
//   C  4 hidden rows per task: the down rows of every slot and of the shared
//      expert, then route weighting, the ascending-id bf16 mixture, the gated
//      shared output, the block output and the next residual
//
// A task waits only for tasks earlier in the list (R and S of layer l on C of
// layer l-1; K on R; B on K; C on B, S and K), so with every workgroup
// resident the earliest unfinished task can always run. Waits are counters in
// HBM bumped with agent-scope release after a fence; each wait is bounded by a
// wall-clock limit and by a shared error word, so a failure ends the launch
// instead of hanging it. The last workgroup to finish zeroes the counters for
// the next launch.
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

constexpr int kRouterRowsPerTask = 16;
constexpr int kPairsPerTask = 8;
constexpr int kRowsPerCTask = 4;
constexpr int kMaxTokens = 4;
constexpr int kMaxTopK = 32;
constexpr int kMaxSlots = kMaxTopK * kMaxTokens;
constexpr int kMaxHidden = 2560;
constexpr int kMaxExperts = 1024;

struct DecodeParams {
    const DecodeLayer* layers;  // [nlayers], already offset to the first layer
    int nlayers;
    int T, H, I, E, K, Is;
    int order;         // 0 TREE32, 1 FOLD
    int bias_feature;  // reset x[H-1] = 1.0 in the residual
    // per-layer buffers (index 0 = first layer of the launch)
    const uint16_t* x_in;     // [T][H] input of the first layer
    uint16_t* x;              // [nlayers + 1][T][H] residual stream (x[0] unused)
    uint16_t* x_final;        // [T][H] residual after the last layer, or null
    uint16_t* out;            // [nlayers][T][H]
    uint16_t* logits;         // [nlayers][T][E + 1]
    int32_t* ids;             // [nlayers][T][K]
    uint16_t* scores;         // [nlayers][T][K]
    int32_t* slot_expert;     // [nlayers][S]
    uint32_t* slot_tokens;    // [nlayers][S]
    int32_t* union_count;     // [nlayers]
    int32_t* token_slots;     // [nlayers][T][K] slots in ascending expert id
    uint16_t* token_weights;  // [nlayers][T][K] bf16 score of that slot
    uint16_t* sig;            // [nlayers][T]
    uint16_t* shared_act;     // [nlayers][T][Is]
    uint16_t* act;            // [nlayers][S][T][I]
    uint32_t* counters;       // [nlayers][kCountersPerLayer] then 1 done counter
    int32_t* error;           // 0 ok, 1 timeout, 2 NaN router logit
    uint64_t limit_ticks;
    int n_router, n_shared, n_b, n_c, per_layer, S;
};

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
    float xs[NT * kMaxHidden];  // x as f32, or the top-k exponentials
    uint16_t res[(kMaxSlots + 1) * kMaxTokens * kRowsPerCTask];
    int32_t ids[kMaxTokens * kMaxTopK];
    int32_t sorted[kMaxSlots];
    int32_t flag;
};

// Residual-stream input of layer li of the launch.
__device__ __forceinline__ const uint16_t* layer_input(const DecodeParams& p, int li) {
    return li == 0 ? p.x_in : p.x + (size_t)li * p.T * p.H;
}

// Load T bf16 vectors of width n (global, row stride n) into LDS as f32.
__device__ __forceinline__ void load_x_f32(float* xs, const uint16_t* x, int T, int n) {
    const uint32_t* x2 = reinterpret_cast<const uint32_t*>(x);
    int pairs = T * n / 2;
    for (int i = threadIdx.x; i < pairs; i += blockDim.x) {
        uint32_t p = x2[i];
        xs[2 * i] = bf16_lo(p);
        xs[2 * i + 1] = bf16_hi(p);
    }
    __syncthreads();
}

// Four rows (one per 16-lane group) of a K-column matrix against the LDS
// vectors: lane q == 0 of each group returns the tree32 dot per token.
template <int NT>
__device__ __forceinline__ void rows_tree32(const uint16_t* w, int row, int nrows_valid, int K,
                                            const float* xs, int xstride, uint32_t token_mask,
                                            float (&dot)[NT]) {
    const int lane = lane_id();
    const int g = lane / kLanesPerRow;
    const int q = lane % kLanesPerRow;
    float acc[NT][2];
    const int r = row + g;
    const bool valid = g < nrows_valid;
    const uint32_t* wrow =
        reinterpret_cast<const uint32_t*>(w + (size_t)(valid ? r : row) * (size_t)K);
    tree32_sweep<NT, 8>(wrow, K / 32, xs, xstride, q, valid ? token_mask : 0u, acc);
#pragma unroll
    for (int t = 0; t < NT; ++t) dot[t] = tree32_reduce(acc[t][0], acc[t][1]);
}

// R task: 16 router rows (or the shared-expert-gate row) for all tokens.
template <int NT>
__device__ void task_router(const DecodeParams& p, const DecodeLayer& L, int li, int task,
                            DecodeShared<NT>& sh) {
    const int T = p.T, H = p.H, E = p.E;
    load_x_f32(sh.xs, layer_input(p, li), T, H);
    const bool gate_row = task == p.n_router - 1;
    const int row0 = gate_row ? E : task * kRouterRowsPerTask;
    const int rows = gate_row ? 1 : min(kRouterRowsPerTask, E - row0);
    uint16_t* logits = p.logits + (size_t)li * T * (E + 1);
    const int w = wave_id();
    const int lane = lane_id();
    if (!gate_row && p.order == 1) {
        // src/router.rs:228-240: one lane folds one row.
        if (lane < kRowsPerWave) {
            int r = row0 + w * kRowsPerWave + lane;
            if (r < row0 + rows) {
                for (int t = 0; t < T; ++t) {
                    float s = fold_row(L.router + (size_t)r * H, sh.xs + t * H, H);
                    logits[(size_t)t * (E + 1) + r] = to_bf16(s);
                }
            }
        }
        return;
    }
    const int wrow0 = row0 + w * kRowsPerWave;
    const int valid = rows - w * kRowsPerWave;
    if (valid <= 0) return;
    float dot[NT];
    rows_tree32<NT>(L.router, wrow0, valid, H, sh.xs, H, (1u << T) - 1u, dot);
    const int g = lane / kLanesPerRow;
    if ((lane % kLanesPerRow) == 0 && g < valid) {
        const uint16_t* wr = L.router + (size_t)(wrow0 + g) * H;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t < T) {
                float v = tree32_finish(dot[t], wr, sh.xs + t * H, H);
                logits[(size_t)t * (E + 1) + wrow0 + g] = to_bf16(v);
            }
        }
    }
}

// Gate and up rows of 8 pairs -> SwiGLU, for a routed expert (B) or the
// shared expert (S). gate_w/up_w point at row 0 of the gate and up blocks.
template <int NT>
__device__ void task_pairs(const uint16_t* gate_w, const uint16_t* up_w, int pair0, int npairs,
                           int K, const float* xs, uint32_t token_mask, uint16_t* act_out,
                           size_t act_token_stride) {
    const int w = wave_id();
    const int lane = lane_id();
    const int g = lane / kLanesPerRow;
    const int q = lane % kLanesPerRow;
    // wave w covers pairs pair0 + 2w and pair0 + 2w + 1:
    // groups 0,1 = gate rows, groups 2,3 = up rows of those pairs.
    const int pw = pair0 + 2 * w;
    const int valid_pairs = min(2, pair0 + npairs - pw);
    if (valid_pairs <= 0) return;
    const int pr = pw + (g & 1);
    const bool valid = (g & 1) < valid_pairs;
    const uint16_t* base = (g < 2) ? gate_w : up_w;
    const uint32_t* wrow =
        reinterpret_cast<const uint32_t*>(base + (size_t)(valid ? pr : pw) * (size_t)K);
    float acc[NT][2];
    tree32_sweep<NT, 8>(wrow, K / 32, xs, K, q, valid ? token_mask : 0u, acc);
    float dot[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        dot[t] = tree32_reduce(acc[t][0], acc[t][1]);
        if (q == 0) {
            const uint16_t* wr = base + (size_t)(valid ? pr : pw) * (size_t)K;
            dot[t] = tree32_finish(dot[t], wr, xs + t * K, K);
        }
    }
    // bf16 gate (groups 0/1) meets bf16 up (groups 2/3): lane l takes lane l+32.
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        uint32_t mine = to_bf16(dot[t]);
        uint32_t up = (uint32_t)__shfl((int)mine, (lane + 32) & 63, kWave);
        if (g < 2 && q == 0 && valid && (token_mask & (1u << t))) {
            act_out[(size_t)t * act_token_stride + pr] = swiglu_bf16(mine, up, c_exp2_table);
        }
    }
}

// K task: top-k per token (wave t), the slot union, scores and the shared gate.
template <int NT>
__device__ void task_topk(const DecodeParams& p, int li, DecodeShared<NT>& sh, uint32_t* counters) {
    const int T = p.T, E = p.E, K = p.K, S = p.S;
    const int w = wave_id();
    const int lane = lane_id();
    const uint16_t* logits = p.logits + (size_t)li * T * (E + 1);
    int32_t* ids = p.ids + (size_t)li * T * K;
    if (w < T) {
        const uint16_t* lt = logits + (size_t)w * (E + 1);
        if (p.order == 0) {
            // src/decoder_layer.rs:279-281: NaN logits are rejected.
            int nan = 0;
            for (int e = lane; e < E; e += kWave) nan |= ((lt[e] & 0x7fffu) > 0x7f80u);
            if (__any(nan)) {
                if (lane == 0) atomicCAS(p.error, 0, 2);
            }
        }
        wave_topk<kMaxExperts / kWave>(lt, E, K, sh.ids + w * kMaxTopK);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        // Union of the selections, ascending expert id (the execution order,
        // src/decoder_layer.rs:422-424), and each token's slots in that order.
        int32_t* slot_expert = p.slot_expert + (size_t)li * S;
        uint32_t* slot_tokens = p.slot_tokens + (size_t)li * S;
        int32_t* token_slots = p.token_slots + (size_t)li * T * K;
        int32_t* sorted = sh.sorted;
        int n = 0;
        for (int t = 0; t < T; ++t) {
            for (int r = 0; r < K; ++r) {
                int32_t e = sh.ids[t * kMaxTopK + r];
                ids[t * K + r] = e;
                int pos = n;
                bool dup = false;
                for (int i = 0; i < n; ++i) dup |= (sorted[i] == e);
                if (dup) continue;
                while (pos > 0 && sorted[pos - 1] > e) {
                    sorted[pos] = sorted[pos - 1];
                    --pos;
                }
                sorted[pos] = e;
                ++n;
            }
        }
        for (int s = 0; s < S; ++s) {
            slot_expert[s] = s < n ? sorted[s] : -1;
            slot_tokens[s] = 0u;
        }
        for (int t = 0; t < T; ++t) {
            int k = 0;
            for (int s = 0; s < n; ++s) {
                for (int r = 0; r < K; ++r) {
                    if (sh.ids[t * kMaxTopK + r] == sorted[s]) {
                        token_slots[t * K + k++] = s;
                        slot_tokens[s] |= 1u << t;
                    }
                }
            }
        }
        p.union_count[li] = n;
    }
    publish(counters + kCntIds);
    // Scores: src/router.rs:248-262 / src/decoder_layer.rs:290-306.
    if (w < T) {
        const uint16_t* lt = logits + (size_t)w * (E + 1);
        float* ex = sh.xs + w * kMaxExperts;
        float mx = -__builtin_inff();
        for (int e = lane; e < E; e += kWave) mx = fmaxf(mx, from_bf16(lt[e]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
        for (int e = lane; e < E; e += kWave) ex[e] = expf_glibc(add_rn(from_bf16(lt[e]), -mx), c_exp2_table);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (lane == 0) {
            float den = -0.0f;
            for (int e = 0; e < E; ++e) den = add_rn(den, ex[e]);
            const int32_t* tid = sh.ids + w * kMaxTopK;
            float sel = -0.0f;
            for (int r = 0; r < K; ++r) sel = add_rn(sel, ex[tid[r]] / den);
            uint16_t* sc = p.scores + (size_t)li * T * K + (size_t)w * K;
            for (int r = 0; r < K; ++r) sc[r] = to_bf16((ex[tid[r]] / den) / sel);
            // weights per slot in the token's ascending-id order
            const int32_t* ts = p.token_slots + (size_t)li * T * K + (size_t)w * K;
            const int32_t* slot_expert = p.slot_expert + (size_t)li * S;
            uint16_t* tw = p.token_weights + (size_t)li * T * K + (size_t)w * K;
            for (int k = 0; k < K; ++k) {
                int32_t e = slot_expert[ts[k]];
                for (int r = 0; r < K; ++r) {
                    if (tid[r] == e) tw[k] = sc[r];
                }
            }
            p.sig[(size_t)li * T + w] = sigmoid_bf16(lt[E], c_exp2_table);
        }
    }
    publish(counters + kCntScores);
}

// C task: rows [r0, r0+4) of every slot's down projection and the shared
// down projection, then the combine.
template <int NT>
__device__ void task_combine(const DecodeParams& p, const DecodeLayer& L, int li, int task,
                             DecodeShared<NT>& sh) {
    const int T = p.T, H = p.H, I = p.I, Is = p.Is, K = p.K, S = p.S;
    const int r0 = task * kRowsPerCTask;
    const int U = p.union_count[li];
    const int w = wave_id();
    const int lane = lane_id();
    const int g = lane / kLanesPerRow;
    const int q = lane % kLanesPerRow;
    const int32_t* slot_expert = p.slot_expert + (size_t)li * S;
    const uint32_t* slot_tokens = p.slot_tokens + (size_t)li * S;
    for (int m = w; m <= U; m += 4) {
        const bool shared = (m == U);
        const int Kd = shared ? Is : I;
        const uint16_t* wmat =
            shared ? L.shared_down : L.down + (size_t)slot_expert[m] * (size_t)H * (size_t)I;
        const uint32_t mask = shared ? ((1u << T) - 1u) : slot_tokens[m];
        const uint16_t* actv = shared ? p.shared_act + (size_t)li * T * Is
                                      : p.act + ((size_t)li * S + m) * (size_t)T * I;
        // activations come from global (L2) as bf16 pairs
        float acc[NT][2];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = 0.0f;
        const int r = r0 + g;
        const uint32_t* wrow = reinterpret_cast<const uint32_t*>(wmat + (size_t)r * Kd);
        const int nb = Kd / 32;
        for (int b = 0; b < nb; b += 8) {
            uint32_t wv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) wv[u] = (b + u < nb) ? __builtin_nontemporal_load(wrow + (b + u) * 16 + q) : 0u;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (!(mask & (1u << t))) continue;
                const uint32_t* a2 = reinterpret_cast<const uint32_t*>(actv + (size_t)t * Kd);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (b + u < nb) {
                        uint32_t av = a2[(b + u) * 16 + q];
                        acc[t][0] = add_rn(acc[t][0], mul_rn(bf16_lo(wv[u]), bf16_lo(av)));
                        acc[t][1] = add_rn(acc[t][1], mul_rn(bf16_hi(wv[u]), bf16_hi(av)));
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float d = tree32_reduce(acc[t][0], acc[t][1]);
            if (q == 0 && (mask & (1u << t))) {
                // K % 32 == 0 here: the tail sum is +0.0.
                d = add_rn(d, 0.0f);
                sh.res[(m * kMaxTokens + t) * kRowsPerCTask + g] = to_bf16(d);
            }
        }
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < T * kRowsPerCTask) {
        const int t = tid / kRowsPerCTask;
        const int gg = tid % kRowsPerCTask;
        const int row = r0 + gg;
        const int32_t* ts = p.token_slots + (size_t)li * T * K + (size_t)t * K;
        const uint16_t* tw = p.token_weights + (size_t)li * T * K + (size_t)t * K;
        // src/decoder_layer.rs:528-545: weighted = bf16(down * score), summed in
        // ascending expert order from bf16 zero, rounding after each add.
        uint32_t mix = to_bf16(0.0f);
        for (int k = 0; k < K; ++k) {
            uint32_t d = sh.res[(ts[k] * kMaxTokens + t) * kRowsPerCTask + gg];
            uint32_t weighted = to_bf16(mul_rn(from_bf16(d), from_bf16(tw[k])));
            mix = add_bf16(mix, weighted);
        }
        // src/decoder_layer.rs:563-575: gated = bf16(shared_down * sigmoid).
        uint32_t sd = sh.res[(U * kMaxTokens + t) * kRowsPerCTask + gg];
        uint32_t sg = p.sig[(size_t)li * T + t];
        uint32_t gated = to_bf16(mul_rn(from_bf16(sd), from_bf16(sg)));
        uint16_t o = add_bf16(mix, gated);
        p.out[((size_t)li * T + t) * H + row] = o;
        uint16_t xin = layer_input(p, li)[(size_t)t * H + row];
        uint16_t xn = add_bf16(xin, o);
        if (p.bias_feature && row == H - 1) xn = 0x3f80u;
        p.x[((size_t)(li + 1) * T + t) * H + row] = xn;
        if (li + 1 == p.nlayers && p.x_final != nullptr) p.x_final[(size_t)t * H + row] = xn;
    }
}

template <int NT>
__global__ void __launch_bounds__(256) k_moe_decode(DecodeParams p) {
    __shared__ DecodeShared<NT> sh;
    const int total = p.nlayers * p.per_layer;
    const int G = (int)gridDim.x;
    for (int task = (int)blockIdx.x; task < total; task += G) {
        // Workgroup-uniform stop check (one reader, broadcast through LDS).
        if (threadIdx.x == 0)
            sh.flag = __hip_atomic_load(p.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const bool stop = sh.flag != 0;
        __syncthreads();
        if (stop) break;
        const int li = task / p.per_layer;
        int j = task - li * p.per_layer;
        const DecodeLayer& L = p.layers[li];
        uint32_t* cnt = p.counters + (size_t)li * kCountersPerLayer;
        if (j < p.n_router + p.n_shared) {
            if (li > 0 &&
                !wait_at_least(p.counters + (size_t)(li - 1) * kCountersPerLayer + kCntC,
                               (uint32_t)p.n_c, p.error, p.limit_ticks, &sh.flag))
                break;
            if (j < p.n_router) {
                task_router<NT>(p, L, li, j, sh);
                publish(cnt + kCntRouter);
            } else {
                j -= p.n_router;
                load_x_f32(sh.xs, layer_input(p, li), p.T, p.H);
                task_pairs<NT>(L.shared_gate, L.shared_up, j * kPairsPerTask,
                               min(kPairsPerTask, p.Is - j * kPairsPerTask), p.H, sh.xs,
                               (1u << p.T) - 1u, p.shared_act + (size_t)li * p.T * p.Is,
                               (size_t)p.Is);
                publish(cnt + kCntShared);
            }
            continue;
        }
        j -= p.n_router + p.n_shared;
        if (j == 0) {
            if (!wait_at_least(cnt + kCntRouter, (uint32_t)p.n_router, p.error, p.limit_ticks,
                               &sh.flag))
                break;
            task_topk<NT>(p, li, sh, cnt);
            continue;
        }
        j -= 1;
        if (j < p.n_b) {
            if (!wait_at_least(cnt + kCntIds, 1u, p.error, p.limit_ticks, &sh.flag)) break;
            const int per_slot = p.I / kPairsPerTask;
            const int s = j / per_slot;
            const int pb = j - s * per_slot;
            const int32_t e = p.slot_expert[(size_t)li * p.S + s];
            if (e >= 0) {
                const uint32_t mask = p.slot_tokens[(size_t)li * p.S + s];
                load_x_f32(sh.xs, layer_input(p, li), p.T, p.H);
                const uint16_t* gu = L.gate_up + (size_t)e * 2 * p.I * p.H;
                task_pairs<NT>(gu, gu + (size_t)p.I * p.H, pb * kPairsPerTask, kPairsPerTask,
                               p.H, sh.xs, mask,
                               p.act + ((size_t)li * p.S + s) * (size_t)p.T * p.I, (size_t)p.I);
            }
            publish(cnt + kCntB);
            continue;
        }
        j -= p.n_b;
        if (!wait_at_least(cnt + kCntB, (uint32_t)p.n_b, p.error, p.limit_ticks, &sh.flag)) break;
        if (!wait_at_least(cnt + kCntShared, (uint32_t)p.n_shared, p.error, p.limit_ticks, &sh.flag))
            break;
        if (!wait_at_least(cnt + kCntScores, 1u, p.error, p.limit_ticks, &sh.flag)) break;
        task_combine<NT>(p, L, li, j, sh);
        publish(cnt + kCntC);
    }
    // The last workgroup out zeroes every counter for the next launch.
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        uint32_t* done = p.counters + (size_t)p.nlayers * kCountersPerLayer;
        uint32_t prev = __hip_atomic_fetch_add(done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == (uint32_t)G - 1u) {
            for (int i = 0; i < p.nlayers * kCountersPerLayer; ++i) {
                __hip_atomic_store(p.counters + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(done, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace fw
