// Device building blocks of the sparse-MoE path on gfx950 (wave64).
//
// Exact-order GEMV. src/expert.rs:514-552 sums a row as 32 independent f32
// chains (chain j takes columns j, j+32, j+64, ...), then a fixed tree. Here 16
// lanes share a row: lane q owns chains 2q and 2q+1, i.e. one packed bf16 pair
// (a 32-bit load) per 32-column block, so 16 lanes read one 64-byte block per
// step and a wave covers 4 rows. After the sweep the tree is evaluated across
// the 16 lanes: +16 is lane q+8, +8 is lane q+4, +4 is lane q+2, and
// (a0+a1)+(a2+a3) joins lanes 0 and 1. Multiplies and adds stay separate
// (-ffp-contract=off), so every chain rounds exactly where the CPU's does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fw_numerics.h"

namespace fw {

constexpr int kWave = 64;
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerWave = kWave / kLanesPerRow;  // 4

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }
__device__ __forceinline__ int wave_id() { return (int)(threadIdx.x / kWave); }

// Tree of the 32 chains after the sweep: returns (a0+a1)+(a2+a3) in lane
// q == 0 of every 16-lane row group (other lanes hold partials).
__device__ __forceinline__ float tree32_reduce(float c0, float c1) {
    // a'[j] = c[j] + c[j+16]   (chains 2q+c and 2q+16+c live in lanes q, q+8)
    c0 = add_rn(c0, __shfl_down(c0, 8, kLanesPerRow));
    c1 = add_rn(c1, __shfl_down(c1, 8, kLanesPerRow));
    // a''[j] = a'[j] + a'[j+8]
    c0 = add_rn(c0, __shfl_down(c0, 4, kLanesPerRow));
    c1 = add_rn(c1, __shfl_down(c1, 4, kLanesPerRow));
    // a'''[j] = a''[j] + a''[j+4]
    c0 = add_rn(c0, __shfl_down(c0, 2, kLanesPerRow));
    c1 = add_rn(c1, __shfl_down(c1, 2, kLanesPerRow));
    // lane 0 holds a0, a1; lane 1 holds a2, a3: (a0 + a1) + (a2 + a3)
    float pair = add_rn(c0, c1);
    float other = __shfl_down(pair, 1, kLanesPerRow);
    return add_rn(pair, other);
}

// src/expert.rs:541-550, by one lane after the tree: the 8-wide tail sum is
// always added (+((0+0)+(0+0)) when K % 32 == 0, which turns -0.0 into +0.0),
// then the scalar tail.
__device__ __forceinline__ float tree32_finish(float reduced, const uint16_t* __restrict__ w,
                                               const float* __restrict__ x, int K) {
    int complete_blocks = K / 32 * 32;
    int complete_vectors = K / 8 * 8;
    float tail[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = complete_blocks; b < complete_vectors; b += 8) {
        for (int l = 0; l < 4; ++l) {
            tail[l] = add_rn(tail[l], mul_rn(from_bf16(w[b + l]), x[b + l]));
            tail[l] = add_rn(tail[l], mul_rn(from_bf16(w[b + 4 + l]), x[b + 4 + l]));
        }
    }
    float r = add_rn(reduced, add_rn(add_rn(tail[0], tail[1]), add_rn(tail[2], tail[3])));
    for (int i = complete_vectors; i < K; ++i) r = add_rn(r, mul_rn(from_bf16(w[i]), x[i]));
    return r;
}

// Chains of one row for NT tokens. `wrow` points at the row (bf16 pairs as
// u32), `xs` at NT f32 vectors of stride `xstride` (LDS or registers' source),
// q is the lane's position in its row group. Only complete 32-blocks.
template <int NT, int UNROLL>
__device__ __forceinline__ void tree32_sweep(const uint32_t* __restrict__ wrow, int nblocks,
                                             const float* __restrict__ xs, int xstride, int q,
                                             uint32_t token_mask, float (&acc)[NT][2]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = 0.0f;
    int b = 0;
    for (; b + UNROLL <= nblocks; b += UNROLL) {
        uint32_t w[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) w[u] = __builtin_nontemporal_load(wrow + (b + u) * 16 + q);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            float w0 = bf16_lo(w[u]);
            float w1 = bf16_hi(w[u]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (!(token_mask & (1u << t))) continue;
                float2 xv = *reinterpret_cast<const float2*>(xs + t * xstride + (b + u) * 32 + 2 * q);
                acc[t][0] = add_rn(acc[t][0], mul_rn(w0, xv.x));
                acc[t][1] = add_rn(acc[t][1], mul_rn(w1, xv.y));
            }
        }
    }
    for (; b < nblocks; ++b) {
        uint32_t w = __builtin_nontemporal_load(wrow + b * 16 + q);
        float w0 = bf16_lo(w);
        float w1 = bf16_hi(w);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (!(token_mask & (1u << t))) continue;
            float2 xv = *reinterpret_cast<const float2*>(xs + t * xstride + b * 32 + 2 * q);
            acc[t][0] = add_rn(acc[t][0], mul_rn(w0, xv.x));
            acc[t][1] = add_rn(acc[t][1], mul_rn(w1, xv.y));
        }
    }
}

// src/router.rs:228-240 forward fold of one row by one lane: sum = sum + w*x.
__device__ __forceinline__ float fold_row(const uint16_t* __restrict__ w,
                                          const float* __restrict__ x, int K) {
    float sum = 0.0f;
    const uint4* w4 = reinterpret_cast<const uint4*>(w);
    int k = 0;
    if ((reinterpret_cast<uintptr_t>(w) & 15u) == 0) {
        for (; k + 8 <= K; k += 8) {
            uint4 v = w4[k / 8];
            uint32_t p[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sum = add_rn(sum, mul_rn(bf16_lo(p[i]), x[k + 2 * i]));
                sum = add_rn(sum, mul_rn(bf16_hi(p[i]), x[k + 2 * i + 1]));
            }
        }
    }
    for (; k < K; ++k) sum = add_rn(sum, mul_rn(from_bf16(w[k]), x[k]));
    return sum;
}

// Wave-wide maximum of a 32-bit unsigned key, broadcast to all lanes.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint32_t o = __shfl_xor(v, off, kWave);
        v = v > o ? v : o;
    }
    return v;
}

// One wave selects the top k of `count` bf16 logits under the total order
// (value descending, then index ascending; src/router.rs:241-247). Writes ids
// in rank order to ids[0..k) (all lanes write the same value; lane 0 is enough).
// count <= 64 * MAXPER, k <= count.
template <int MAXPER>
__device__ __forceinline__ void wave_topk(const uint16_t* __restrict__ logits, int count, int k,
                                          int32_t* __restrict__ ids) {
    const int lane = lane_id();
    uint32_t keys[MAXPER];
#pragma unroll
    for (int m = 0; m < MAXPER; ++m) {
        int e = lane + kWave * m;
        keys[m] = e < count ? topk_key(logits[e], (uint32_t)e) : 0u;  // 0 is below every key
    }
    for (int r = 0; r < k; ++r) {
        uint32_t best = 0;
#pragma unroll
        for (int m = 0; m < MAXPER; ++m) best = keys[m] > best ? keys[m] : best;
        best = wave_max_u32(best);
#pragma unroll
        for (int m = 0; m < MAXPER; ++m) {
            if (keys[m] == best) keys[m] = 0u;  // keys are unique per expert
        }
        if (lane == 0) ids[r] = (int32_t)topk_key_expert(best);
    }
}

// ---- inter-workgroup synchronisation for the persistent kernel ----------------------

__device__ __forceinline__ uint32_t load_acquire(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void add_release(uint32_t* p, uint32_t v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// Publish: every wave's stores complete and are made visible at agent scope
// before thread 0 bumps the counter.
__device__ __forceinline__ void publish(uint32_t* counter) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) add_release(counter, 1u);
}

// Thread 0 spins until *counter >= target, bounded by a wall-clock limit and
// by the shared error word; the verdict is broadcast to the workgroup.
// Returns false if the kernel must stop.
__device__ __forceinline__ bool wait_at_least(const uint32_t* counter, uint32_t target,
                                              int32_t* error, uint64_t limit_ticks,
                                              int32_t* lds_flag) {
    if (threadIdx.x == 0) {
        int32_t ok = 1;
        if (load_acquire(counter) < target) {
            uint64_t start = wall_clock64();
            while (load_acquire(counter) < target) {
                if (__hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                    ok = 0;
                    break;
                }
                if (wall_clock64() - start > limit_ticks) {
                    int32_t expected = 0;
                    __hip_atomic_compare_exchange_strong(error, &expected, 1, __ATOMIC_RELAXED,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        *lds_flag = ok;
    }
    __syncthreads();
    int32_t ok = *lds_flag;
    __threadfence();
    __syncthreads();
    return ok != 0;
}

}  // namespace fw
