// Hyper-connection kernels around the sparse-MoE block: the grouped RMS norm
// with PyTorch's aarch64 square-sum cascade, the low-rank input mix, the
// injection weights (src/hyper_connection.rs:211-490), and the block output's
// injection into the residual streams (src/decoder_layer.rs:587-607). The two
// projections in between run on the exact-order GEMV (k_linear_tree32).
// Shapes: T tokens of S streams of W values; R = low rank. Uses c_exp2_table
// (fw_decode.h) for exp.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "fw_numerics.h"

namespace fw {

// hyper_input_normed = grouped_rms(x, hc_norm, eps 1e-6): grid (S, T), 256
// threads, W floats of dynamic LDS. The square sum runs in the order of
// src/hyper_connection.rs:211-283: 16 chains (register r, lane l) each take
// every 16th element from 4r + l, summed in cascades of `step` groups, then
// folded (levels, vectors past the chains into register 0, registers, scalar
// tail, lanes) by one thread each stage.
__global__ void __launch_bounds__(256) k_hc_norm(const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm,
                                                 int S, int W, uint16_t* __restrict__ out) {
    extern __shared__ float v[];
    __shared__ float chain[16];
    __shared__ float lanes[4];
    __shared__ float inv_s;
    const int s = blockIdx.x, t = blockIdx.y;
    const size_t base = ((size_t)t * S + s) * W;
    for (int i = threadIdx.x; i < W; i += blockDim.x) v[i] = from_bf16(x[base + i]);
    __syncthreads();
    const int vectors = W / 4, cascade = vectors / 4;
    const int ceil_log2 = cascade > 1 ? 32 - __clz(cascade - 1) : 0;
    const int power = max(4, ceil_log2 / 4);
    const int step = 1 << power, mask = step - 1;
    if (threadIdx.x < 16) {
        const int c = threadIdx.x;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        int g = 0;
        while (g + step <= cascade) {
            for (int k = 0; k < step; ++k, ++g) {
                const float e = v[16 * g + c];
                a0 = add_rn(a0, mul_rn(e, e));
            }
            a1 = add_rn(a1, a0);
            a0 = 0.0f;
            if (g & (mask << power)) continue;
            a2 = add_rn(a2, a1);
            a1 = 0.0f;
            if (g & (mask << (2 * power))) continue;
            a3 = add_rn(a3, a2);
            a2 = 0.0f;
        }
        for (; g < cascade; ++g) {
            const float e = v[16 * g + c];
            a0 = add_rn(a0, mul_rn(e, e));
        }
        chain[c] = add_rn(add_rn(add_rn(a0, a1), a2), a3);
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        const int l = threadIdx.x;
        float acc = chain[l];  // register 0
        for (int vec = cascade * 4; vec < vectors; ++vec) {
            const float e = v[vec * 4 + l];
            acc = add_rn(acc, mul_rn(e, e));
        }
        for (int r = 1; r < 4; ++r) acc = add_rn(acc, chain[4 * r + l]);
        lanes[l] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (int i = vectors * 4; i < W; ++i) sum = add_rn(sum, mul_rn(v[i], v[i]));
        for (int l = 0; l < 4; ++l) sum = add_rn(sum, lanes[l]);
        const float mean = sum / (float)W;
        inv_s = 1.0f / sqrtf(add_rn(mean, 1.0e-6f));
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = threadIdx.x; i < W; i += blockDim.x) {
        const float scaled = mul_rn(v[i], inv);
        const float gain = add_rn(1.0f, from_bf16(norm[(size_t)s * W + i]));
        out[base + i] = to_bf16(mul_rn(scaled, gain));
    }
}

// mix_down_scaled = bf16(mix_down / S), mix_down_silu = silu(scaled): n = T * R.
__global__ void k_hc_scale_silu(const uint16_t* __restrict__ mix_down, int n, int S,
                                uint16_t* __restrict__ scaled, uint16_t* __restrict__ silu) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint16_t sc = to_bf16(from_bf16(mix_down[i]) / (float)S);
    scaled[i] = sc;
    silu[i] = silu_bf16(sc, c_exp2_table);
}

// input_mix = sigmoid(mix_up), products = bf16(input_mix * normed) and
// mixed[c] = bf16(((0 + p_0c) + ... + p_(S-1)c) / S): grid (ceil(W/256), T),
// one thread per column. Workgroup (0, t) also finishes the injection
// weights: bf16(2 * sigmoid(bf16(inject / S))) (inject may be null).
__global__ void __launch_bounds__(256) k_hc_mix(const uint16_t* __restrict__ mix_up,
                                                const uint16_t* __restrict__ normed,
                                                const uint16_t* __restrict__ inject, int S, int W,
                                                uint16_t* __restrict__ input_mix,
                                                uint16_t* __restrict__ products, uint16_t* __restrict__ mixed,
                                                uint16_t* __restrict__ inject_scaled,
                                                uint16_t* __restrict__ inject_sigmoid,
                                                uint16_t* __restrict__ injection_weights) {
    const int t = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c < W) {
        float sum = 0.0f;
        for (int s = 0; s < S; ++s) {
            const size_t i = ((size_t)t * S + s) * W + c;
            const uint16_t im = sigmoid_bf16(mix_up[i], c_exp2_table);
            const uint16_t p = to_bf16(mul_rn(from_bf16(im), from_bf16(normed[i])));
            input_mix[i] = im;
            products[i] = p;
            sum = add_rn(sum, from_bf16(p));
        }
        mixed[(size_t)t * W + c] = to_bf16(sum / (float)S);
    }
    if (inject && blockIdx.x == 0 && threadIdx.x < (unsigned)S) {
        const size_t i = (size_t)t * S + threadIdx.x;
        const uint16_t sc = to_bf16(from_bf16(inject[i]) / (float)S);
        const uint16_t sg = sigmoid_bf16(sc, c_exp2_table);
        inject_scaled[i] = sc;
        inject_sigmoid[i] = sg;
        injection_weights[i] = to_bf16(mul_rn(2.0f, from_bf16(sg)));
    }
}

// products[t][s][h] = bf16(moe[t][h] * weight[t][s]) (may be null),
// out[t][s][h] = add_bf16(post[t][s][h], product): grid (ceil(S*W/256), T).
__global__ void k_inject_residual(const uint16_t* __restrict__ post, const uint16_t* __restrict__ moe,
                                  const uint16_t* __restrict__ weights, int S, int W,
                                  uint16_t* __restrict__ products, uint16_t* __restrict__ out) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= S * W) return;
    const int s = i / W, h = i - s * W;
    const size_t at = (size_t)t * S * W + i;
    const uint16_t p = to_bf16(mul_rn(from_bf16(moe[(size_t)t * W + h]), from_bf16(weights[(size_t)t * S + s])));
    if (products) products[at] = p;
    out[at] = add_bf16(post[at], p);
}

}  // namespace fw
