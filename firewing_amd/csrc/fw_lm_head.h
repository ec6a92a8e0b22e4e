// LM head: logits = linear_bf16(lm_head [V][H], x) in the reference's exact
// order (src/text_output.rs:273-287, src/expert.rs:514-560) and their top-k in
// the total order (value descending, index ascending). HBM-bound: the head is
// 1.27 GB at V = 248,320, H = 2560, read once per step.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "fw_device.h"
#include "fw_numerics.h"

namespace fw {

// logits[t][r] for NT tokens (x [NT][H] staged in LDS as f32, NT * H floats of
// dynamic LDS). A wave takes groups of four rows (one per 16-lane group, the
// full-line lane layout of the decode kernel) over a grid-strided list, and
// issues the next group's loads before the current group's chains, so two row
// groups per wave are in flight. w must extend kLineSharePad bytes past the
// last row start.
template <int NT, int MBH>
__global__ void __launch_bounds__(256, 2) k_lm_head(const uint16_t* __restrict__ w, const uint16_t* __restrict__ x,
                                                    int V, int H, uint16_t* __restrict__ logits) {
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < NT * H; i += blockDim.x) xs[i] = from_bf16(x[i]);
    __syncthreads();
    const int lane = lane_id(), g = lane / kLanesPerRow, q = lane % kLanesPerRow;
    const int groups = (V + kRowsPerWave - 1) / kRowsPerWave;
    const int stride = (int)gridDim.x * (int)(blockDim.x / kWave);
    int grp = (int)blockIdx.x * (int)(blockDim.x / kWave) + wave_id();
    const uint32_t row_bytes = (uint32_t)g * (uint32_t)H * 2u;
    auto issue = [&](LineShare<MBH>& rs, int gi) {
        // rows past V read the group's first row again (their results are not stored)
        const bool valid = gi * kRowsPerWave + g < V;
        line_issue(rs, w + (size_t)gi * kRowsPerWave * H, valid ? row_bytes : 0u, q);
    };
    auto finish = [&](const LineShare<MBH>& rs, int gi) {
        float acc[NT][2];
        line_chains<NT, MBH>(rs, H / 32, xs, H, q, acc);
        const int row = gi * kRowsPerWave + g;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float d = tree32_reduce_lines(acc[t][0], acc[t][1]);
            if (q == 0 && row < V) {
                d = tree32_finish(d, w + (size_t)row * H, xs + t * H, H);
                logits[(size_t)t * V + row] = to_bf16(d);
            }
        }
    };
    LineShare<MBH> a, b;
    if (grp < groups) issue(a, grp);
    while (grp < groups) {
        if (grp + stride < groups) issue(b, grp + stride);
        finish(a, grp);
        grp += stride;
        if (grp >= groups) break;
        if (grp + stride < groups) issue(a, grp + stride);
        finish(b, grp);
        grp += stride;
    }
}

// Selection key of (logit, index): larger key = larger logit, then the smaller
// index (total_order_key16 ranks -0.0 below +0.0 and NaNs outermost).
__device__ __forceinline__ uint64_t lm_key(uint32_t bf16_bits, uint32_t index) {
    return ((uint64_t)total_order_key16(bf16_bits) << 32) | (uint64_t)(0xffffffffu - index);
}

constexpr int kTopkChunk = 4096;         // logits per workgroup of the first pass
constexpr int kTopkPerThread = kTopkChunk / 256;

// Largest key over the workgroup (256 threads); every thread gets it.
__device__ __forceinline__ uint64_t wg_max_key(uint64_t v, uint64_t* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = (uint64_t)__shfl_xor((long long)v, off, kWave);
        v = o > v ? o : v;
    }
    const int w = (int)threadIdx.x / kWave;
    __syncthreads();
    if (lane_id() == 0) red[w] = v;
    __syncthreads();
    uint64_t m = red[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) m = red[i] > m ? red[i] : m;
    return m;
}

// First pass: workgroup c takes logits [c * kTopkChunk, ...) of token t
// (blockIdx.y) and writes its k largest keys, in order, to
// cand[t][c][0..k) (0 past the chunk's logits).
__global__ void __launch_bounds__(256) k_lm_topk_chunks(const uint16_t* __restrict__ logits, int V, int k,
                                                         uint64_t* __restrict__ cand) {
    __shared__ uint64_t red[4];
    const int t = (int)blockIdx.y, c = (int)blockIdx.x;
    const int chunks = (int)gridDim.x;
    uint64_t keys[kTopkPerThread];
#pragma unroll
    for (int i = 0; i < kTopkPerThread; ++i) {
        const int idx = c * kTopkChunk + i * 256 + (int)threadIdx.x;
        keys[i] = idx < V ? lm_key(logits[(size_t)t * V + idx], (uint32_t)idx) : 0ull;
    }
    uint64_t* out = cand + ((size_t)t * chunks + c) * k;
    for (int r = 0; r < k; ++r) {
        uint64_t best = 0;
#pragma unroll
        for (int i = 0; i < kTopkPerThread; ++i) best = keys[i] > best ? keys[i] : best;
        const uint64_t m = wg_max_key(best, red);
        // keys are distinct (they carry the index): exactly one thread holds m
#pragma unroll
        for (int i = 0; i < kTopkPerThread; ++i)
            if (keys[i] == m) keys[i] = 0;
        if (threadIdx.x == 0) out[r] = m;
    }
}

// Second pass, one workgroup per token: the k largest of its n chunk
// candidates, as ids and bf16 values in rank order (round r takes the largest
// key below round r - 1's: the keys are distinct).
__global__ void __launch_bounds__(256) k_lm_topk_merge(const uint64_t* __restrict__ cand, int n, int k,
                                                        int32_t* __restrict__ ids, uint16_t* __restrict__ values) {
    __shared__ uint64_t red[4];
    const int t = (int)blockIdx.x;
    const uint64_t* c = cand + (size_t)t * n;
    uint64_t prev = ~0ull;
    for (int r = 0; r < k; ++r) {
        uint64_t best = 0;
        for (int i = (int)threadIdx.x; i < n; i += 256) {
            const uint64_t v = c[i];
            best = (v < prev && v > best) ? v : best;
        }
        const uint64_t m = wg_max_key(best, red);
        if (threadIdx.x == 0) {
            const uint32_t idx = 0xffffffffu - (uint32_t)m;
            const uint32_t key16 = (uint32_t)(m >> 32);
            // the inverse of total_order_key16
            const uint32_t bits = (key16 & 0x8000u) ? (key16 & 0x7fffu) : ((~key16) & 0xffffu);
            ids[(size_t)t * k + r] = (int32_t)idx;
            values[(size_t)t * k + r] = (uint16_t)bits;
        }
        prev = m;
    }
}

}  // namespace fw
