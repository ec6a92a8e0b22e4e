// LM head: logits = linear_bf16(lm_head [V][H], x) in the reference's exact
// order (src/text_output.rs:273-287, src/expert.rs:514-560) and their top-k in
// the total order (value descending, index ascending; keys as fw_numerics.h
// topk_key). HBM-bound: the head is
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

constexpr int kTopkChunk = 4096;  // logits per workgroup of the first pass (1,024 per wave)

// The k largest of the 32-bit keys a wave holds (MAXPER per lane, distinct,
// 0 = none), in descending order to out[0..k) (lane 0 writes): each lane sorts
// its keys, then every round the wave maximum of the lane heads is taken and
// its lane pops it (the selection of wave_topk).
template <int MAXPER>
__device__ __forceinline__ void wave_top_keys(uint32_t (&keys)[MAXPER], int k, uint32_t* out) {
#pragma unroll
    for (int pass = 0; pass < MAXPER; ++pass) {
#pragma unroll
        for (int m = pass & 1; m + 1 < MAXPER; m += 2) {
            const uint32_t a = keys[m], b = keys[m + 1];
            keys[m] = a > b ? a : b;
            keys[m + 1] = a > b ? b : a;
        }
    }
    for (int r = 0; r < k; ++r) {
        const uint32_t best = wave_max_u32(keys[0]);
        if (keys[0] == best) {
#pragma unroll
            for (int m = 0; m + 1 < MAXPER; ++m) keys[m] = keys[m + 1];
            keys[MAXPER - 1] = 0u;
        }
        if (lane_id() == 0) out[r] = best;
    }
}

// First pass: workgroup c takes logits [c * kTopkChunk, ...) of token t
// (blockIdx.y). Keys are topk_key(logit, index within the chunk): larger key =
// larger logit, then the lower index. Each wave the k largest of its 1,024,
// then wave 0 the k largest of the four lists, written in descending order as
// their bf16 order keys (key16[t][c][r]) and chunk positions (pos[t][c][r]).
__global__ void __launch_bounds__(256) k_lm_topk_chunks(const uint16_t* __restrict__ logits, int V, int k,
                                                         uint16_t* __restrict__ key16, uint16_t* __restrict__ pos) {
    __shared__ uint32_t lists[4 * 64];
    __shared__ uint32_t best[64];
    const int t = (int)blockIdx.y, c = (int)blockIdx.x;
    const int chunks = (int)gridDim.x;
    const int w = (int)threadIdx.x / kWave, lane = lane_id();
    uint32_t keys[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int local = w * 1024 + i * kWave + lane;
        const int idx = c * kTopkChunk + local;
        keys[i] = idx < V ? topk_key(logits[(size_t)t * V + idx], (uint32_t)local) : 0u;
    }
    wave_top_keys<16>(keys, k, lists + w * 64);
    wg_sync();
    if (w == 0) {
        uint32_t m[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) m[i] = lane < k ? lists[i * 64 + lane] : 0u;
        wave_top_keys<4>(m, k, best);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < k) {
            // a chunk with fewer than k logits pads its list with position 0xffff
            const size_t at = ((size_t)t * chunks + c) * k + lane;
            key16[at] = (uint16_t)(best[lane] >> 16);
            pos[at] = best[lane] != 0u ? (uint16_t)topk_key_expert(best[lane]) : (uint16_t)0xffffu;
        }
    }
}

// Second pass, one workgroup per token: the k largest of the n = chunks * k
// candidates. Candidate p (= c * k + r) gets the key key16 << 16 | (0xffff - p):
// among equal values a lower p is a lower chunk, or the same chunk and a lower
// rank, so a lower vocabulary index. Writes ids (c * kTopkChunk + position)
// and bf16 values in rank order. kPerLane candidates a lane: n <= 256 *
// kPerLane (the launch takes the smallest of 8, 16, 32 that holds n; the
// lanes' sorts cost kPerLane^2 / 2 compare-exchanges).
template <int kPerLane>
__global__ void __launch_bounds__(256) k_lm_topk_merge(const uint16_t* __restrict__ key16,
                                                        const uint16_t* __restrict__ pos, int n, int k,
                                                        int32_t* __restrict__ ids, uint16_t* __restrict__ values) {
    __shared__ uint32_t lists[4 * 64];
    __shared__ uint32_t best[64];
    const int t = (int)blockIdx.x;
    const int w = (int)threadIdx.x / kWave, lane = lane_id();
    const uint16_t* kk = key16 + (size_t)t * n;
    uint32_t keys[kPerLane];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int p = (w * kPerLane + i) * kWave + lane;
        const bool real = p < n && pos[(size_t)t * n + p] != 0xffffu;
        keys[i] = real ? ((uint32_t)kk[p] << 16) | (0xffffu - (uint32_t)p) : 0u;
    }
    wave_top_keys<kPerLane>(keys, k, lists + w * 64);
    wg_sync();
    if (w == 0) {
        uint32_t m[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) m[i] = lane < k ? lists[i * 64 + lane] : 0u;
        wave_top_keys<4>(m, k, best);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < k) {
            const uint32_t key = best[lane];
            const int p = (int)topk_key_expert(key);
            const uint32_t k16 = key >> 16;
            // the inverse of total_order_key16
            const uint32_t bits = (k16 & 0x8000u) ? (k16 & 0x7fffu) : ((~k16) & 0xffffu);
            ids[(size_t)t * k + lane] = (p / k) * kTopkChunk + (int)pos[(size_t)t * n + p];
            values[(size_t)t * k + lane] = (uint16_t)bits;
        }
    }
}

}  // namespace fw
