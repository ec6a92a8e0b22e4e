// Device building blocks of the sparse-MoE path on gfx950 (wave64).
//
// Exact-order GEMV. src/expert.rs:514-552 sums a row as 32 independent f32
// chains (chain j takes columns j, j+32, j+64, ...), then a fixed tree. Here 16
// lanes share a row: lane q owns chains 2q and 2q+1, i.e. one packed bf16 pair
// (a 32-bit load) per 32-column block, so 16 lanes read one 64-byte block per
// step and a wave covers 4 rows. A lane issues the loads of its whole row
// share before the first multiply (a row of 2048 columns is 64 loads, 16 KB in
// flight per wave), so a wave pays one memory round trip per row set instead
// of one per block. After the sweep the tree is evaluated across the 16 lanes
// of the row with DPP row shifts: +16 is lane q+8, +8 is lane q+4, +4 is lane
// q+2, and (a0+a1)+(a2+a3) joins lanes 0 and 1. Multiplies and adds stay
// separate (-ffp-contract=off), so every chain rounds exactly where the CPU's
// does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fw_numerics.h"

namespace fw {

constexpr int kWave = 64;
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerWave = kWave / kLanesPerRow;  // 4

// Lane and wave indices, opaque to loop-invariant code motion: what a task
// derives from them is recomputed in the task instead of being hoisted out of
// the persistent task loop and held in registers for its whole length.
__device__ __forceinline__ int lane_id() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t & (kWave - 1);
}
// The workgroup thread index, opaque in the same way.
__device__ __forceinline__ int thread_id() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int wave_id() {
    int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    asm volatile("" : "+s"(w));
    return w;
}

// DPP controls (GFX9 encoding).
constexpr int kDppRowShl1 = 0x101, kDppRowShl2 = 0x102, kDppRowShl4 = 0x104, kDppRowShl8 = 0x108;
constexpr int kDppRowMirror = 0x140, kDppRowHalfMirror = 0x141;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E;  // quad_perm [1,0,3,2], [2,3,0,1]
// row_ror:n moves values n lanes up the 16-lane row: lane i reads lane
// (i - n) mod 16. Reading lane (i + 4) mod 16 is therefore row_ror:12.
constexpr int kDppRowRead4 = 0x12C;                      // lane (i + 4) mod 16 of the row

// v from lane (i + n) of the same 16-lane row (0 past the row's end).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}

// Tree of the 32 chains after the sweep: returns (a0+a1)+(a2+a3) in lane
// q == 0 of every 16-lane row group (other lanes hold partials).
__device__ __forceinline__ float tree32_reduce(float c0, float c1) {
    // a'[j] = c[j] + c[j+16]   (chains 2q+c and 2q+16+c live in lanes q, q+8)
    c0 = add_rn(c0, dpp_f32<kDppRowShl8>(c0));
    c1 = add_rn(c1, dpp_f32<kDppRowShl8>(c1));
    // a''[j] = a'[j] + a'[j+8]
    c0 = add_rn(c0, dpp_f32<kDppRowShl4>(c0));
    c1 = add_rn(c1, dpp_f32<kDppRowShl4>(c1));
    // a'''[j] = a''[j] + a''[j+4]
    c0 = add_rn(c0, dpp_f32<kDppRowShl2>(c0));
    c1 = add_rn(c1, dpp_f32<kDppRowShl2>(c1));
    // lane 0 holds a0, a1; lane 1 holds a2, a3: (a0 + a1) + (a2 + a3)
    float pair = add_rn(c0, c1);
    return add_rn(pair, dpp_f32<kDppRowShl1>(pair));
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

// Global-memory view of a pointer (loads through it are global, not flat,
// instructions: they do not wait on LDS traffic).
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* as_global(const T* p) {
    return (const __attribute__((address_space(1))) T*)(p);
}

// Agent-scope relaxed atomic 32-bit accesses: data exchanged between
// workgroups of one launch (see the synchronisation notes below).
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* as_global_rw(T* p) {
    return (__attribute__((address_space(1))) T*)(p);
}
__device__ __forceinline__ uint32_t coherent_load(const uint32_t* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t coherent_load(const int32_t* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store(uint32_t* p, uint32_t v) {
    __hip_atomic_store(as_global_rw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store(int32_t* p, int32_t v) {
    __hip_atomic_store(as_global_rw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t coherent_load64(const uint64_t* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(as_global_rw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged words: a 32-bit payload and the launch's epoch in one 64-bit store,
// so a reader that sees the epoch also sees the payload. Words from earlier
// launches carry older epochs.
__device__ __forceinline__ uint64_t tagged(uint32_t payload, uint32_t epoch) {
    return ((uint64_t)epoch << 32) | payload;
}
__device__ __forceinline__ bool has_tag(uint64_t word, uint32_t epoch) { return (uint32_t)(word >> 32) == epoch; }

// Wave-uniform value as a scalar (lets the compiler branch on it without
// exec masks).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// The same scalar, opaque to loop-invariant code motion: values derived from
// it are computed where they are used instead of being hoisted out of the
// task loop and held in registers for its whole length.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+s"(v));
    return v;
}

// A lane's share of one row: the packed bf16 pair of every 32-column block.
template <int MAXB>
struct RowShare {
    uint32_t w[MAXB];
};

// Issue the loads of a row share: nblocks <= MAXB complete 32-column blocks.
// Every slot is loaded (slots past nblocks repeat the last block), so the
// loads carry no branches; the chain sweeps skip the repeats.
template <int MAXB>
__device__ __forceinline__ void row_issue(RowShare<MAXB>& r, const uint32_t* wrow, int nblocks, int q) {
    const auto* g = as_global(wrow) + q;
    const int last = opaque(nblocks - 1);
#pragma unroll
    for (int u = 0; u < MAXB; ++u) {
        const int b = u < last ? u : last;
        r.w[u] = __builtin_nontemporal_load(g + b * 16);
    }
}

// Chains of one row for NT tokens against f32 vectors in LDS (stride xstride),
// accumulated onto acc (the caller zeroes it once per row). Every token is
// computed; the caller discards what it does not need. nblocks is uniform.
// Scheduling barriers every 8 blocks keep the LDS operand reads next to their
// use (hoisting all of them would need two registers per block and token).
template <int NT, int MAXB>
__device__ __forceinline__ void row_chains_acc(const RowShare<MAXB>& r, int nblocks,
                                               const float* __restrict__ xs, int xstride, int q,
                                               float (&acc)[NT][2]) {
    nblocks = opaque(nblocks);
#pragma unroll
    for (int u0 = 0; u0 < MAXB; u0 += 8) {
#pragma unroll
        for (int u = u0; u < u0 + 8 && u < MAXB; ++u) {
            if (u < nblocks) {
                float w0 = bf16_lo(r.w[u]);
                float w1 = bf16_hi(r.w[u]);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    float2 xv = *reinterpret_cast<const float2*>(xs + t * xstride + u * 32 + 2 * q);
                    acc[t][0] = add_rn(acc[t][0], mul_rn(w0, xv.x));
                    acc[t][1] = add_rn(acc[t][1], mul_rn(w1, xv.y));
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int NT, int MAXB>
__device__ __forceinline__ void row_chains(const RowShare<MAXB>& r, int nblocks,
                                           const float* __restrict__ xs, int xstride, int q,
                                           float (&acc)[NT][2]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = 0.0f;
    row_chains_acc<NT, MAXB>(r, nblocks, xs, xstride, q, acc);
}

// Chains of one row for NT tokens against bf16 vectors that other workgroups
// wrote in this launch (packed pairs, token stride xstride elements, read with
// coherent loads). token_mask is wave-uniform:
// tokens outside it are not loaded. A token's loads are all issued before its
// first multiply: one memory round trip per token.
template <int NT, int MAXB>
__device__ __forceinline__ void row_chains_gx(const RowShare<MAXB>& r, int nblocks,
                                              const uint16_t* x, int xstride, int q,
                                              uint32_t token_mask, float (&acc)[NT][2]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (!(token_mask & (1u << t))) continue;
        const uint32_t* x2 = reinterpret_cast<const uint32_t*>(x + (size_t)t * xstride) + q;
        uint32_t xv[MAXB];
        nblocks = opaque(nblocks);
        const int last = nblocks - 1;
#pragma unroll
        for (int u = 0; u < MAXB; ++u) {
            const int b = u < last ? u : last;
            xv[u] = coherent_load(x2 + b * 16);
        }
#pragma unroll
        for (int u = 0; u < MAXB; ++u) {
            if (u < nblocks) {
                acc[t][0] = add_rn(acc[t][0], mul_rn(bf16_lo(r.w[u]), bf16_lo(xv[u])));
                acc[t][1] = add_rn(acc[t][1], mul_rn(bf16_hi(r.w[u]), bf16_hi(xv[u])));
            }
        }
    }
}

// ---- full-line row shares ------------------------------------------------------------
//
// The same chains, loaded a whole 128-byte line (two 32-column blocks) per
// 16-lane group and instruction: lane q reads bytes 8q..8q+7 of the line, i.e.
// columns 4(q%8)..4(q%8)+3 of block 2v + q/8. Whole-line requests stream
// about a fifth faster than the half-line pattern above. Before the sweep a
// DPP rotate by 8 lanes trades halves so that lane q owns chains
// j = 4(q%8) + 2(q/8) and j + 1 of both blocks of every line:
//   lane c < 8:   block 2v from its own low dword, block 2v+1 from lane c+8's low dword
//   lane c + 8:   block 2v from lane c's high dword, block 2v+1 from its own high dword
// The tree then pairs chain j with j+16 in lane +4, j+8 in lane +2, j+4 in
// lane +1, and (a0+a1) in lane 0 with (a2+a3) in lane 8.

constexpr int kDppRowRor8 = 0x128;

template <int MAXB>
struct LineShare {
    uint64_t w[(MAXB + 1) / 2];
};

// A pointer that is the same in every lane, as a scalar pair.
__device__ __forceinline__ const char* uniform_ptr(const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}

// Issue the loads of a row's line share: all (MAXB + 1) / 2 lines from the
// row start, whatever the row's length (the sweeps skip blocks past the row),
// so the allocation must extend kLineSharePad bytes past any row start. The
// row is given as a base shared by the wave plus this lane's byte offset to
// its row (below 4 GiB): every load then addresses the scalar base, one 32-bit
// offset register and an immediate.
constexpr int kLineSharePad = 80 * 64;  // the widest variant's line share
template <int MAXB>
__device__ __forceinline__ void line_issue(LineShare<MAXB>& r, const uint16_t* base, uint32_t row_bytes, int q) {
    static_assert((MAXB + 1) / 2 * 128 <= kLineSharePad, "allocation padding");
    const auto* b = as_global(uniform_ptr(base));
    const uint32_t off = row_bytes + 8u * (uint32_t)q;
#pragma unroll
    for (int v = 0; v < (MAXB + 1) / 2; ++v)
        r.w[v] = __builtin_nontemporal_load(
            reinterpret_cast<const __attribute__((address_space(1))) uint64_t*>(b + off + 128 * v));
}

// The two blocks of line v as this lane's chain pairs (first: block 2v,
// second: block 2v+1). Executed by the whole wave.
__device__ __forceinline__ void line_pairs(uint64_t word, int q, uint32_t& first, uint32_t& second) {
    const uint32_t x = (uint32_t)word, y = (uint32_t)(word >> 32);
    const uint32_t tx = dpp_u32<kDppRowRor8>(x), ty = dpp_u32<kDppRowRor8>(y);
    const bool upper = q >= 8;
    first = upper ? ty : x;
    second = upper ? y : tx;
}

// Column offset of this lane's chain pair within a block.
__device__ __forceinline__ int line_column(int q) { return 4 * (q & 7) + 2 * (q >> 3); }

// The pipelined sweep of line_chains (NT <= 2), G lines per group.
template <int NT, int MAXB, int G>
__device__ __forceinline__ void line_sweep(const LineShare<MAXB>& r, int nblocks, const float* __restrict__ xq,
                                           const int (&xoff)[NT], int q, float (&acc)[NT][2]) {
    constexpr int NL = (MAXB + 1) / 2;  // lines
    float2 xv[2][NT][2 * G];
#pragma unroll
    for (int i = 0; i < G && i < NL; ++i) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            xv[0][t][2 * i] = *reinterpret_cast<const float2*>(xq + xoff[t] + 64 * i);
            xv[0][t][2 * i + 1] = *reinterpret_cast<const float2*>(xq + xoff[t] + 64 * i + 32);
        }
    }
#pragma unroll
    for (int v0 = 0, buf = 0; v0 < NL; v0 += G, buf ^= 1) {
        if (v0 + G < NL) {
#pragma unroll
            for (int i = 0; i < G && v0 + G + i < NL; ++i) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float* xa = xq + xoff[t] + 64 * (v0 + G + i);
                    xv[buf ^ 1][t][2 * i] = *reinterpret_cast<const float2*>(xa);
                    xv[buf ^ 1][t][2 * i + 1] = *reinterpret_cast<const float2*>(xa + 32);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < G && v0 + i < NL; ++i) {
            const int v = v0 + i;
            uint32_t first, second;
            line_pairs(r.w[v], q, first, second);
            if (2 * v < nblocks) {
                const float w0 = bf16_lo(first), w1 = bf16_hi(first);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t][0] = add_rn(acc[t][0], mul_rn(w0, xv[buf][t][2 * i].x));
                    acc[t][1] = add_rn(acc[t][1], mul_rn(w1, xv[buf][t][2 * i].y));
                }
            }
            if (2 * v + 1 < nblocks) {
                const float w0 = bf16_lo(second), w1 = bf16_hi(second);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t][0] = add_rn(acc[t][0], mul_rn(w0, xv[buf][t][2 * i + 1].x));
                    acc[t][1] = add_rn(acc[t][1], mul_rn(w1, xv[buf][t][2 * i + 1].y));
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Chains of one row for NT tokens against f32 vectors in LDS (token t's at
// xs + xoff[t], uniform offsets); nblocks is uniform. The vector values of the next
// group of G lines are read from LDS while the current group is computed (G
// = 0: 4 lines for one token, 2 for two; fewer registers with a smaller G).
template <int NT, int MAXB, int G = 0>
__device__ __forceinline__ void line_chains_at(const LineShare<MAXB>& r, int nblocks, const float* __restrict__ xs,
                                               const int (&xoff)[NT], int q, float (&acc)[NT][2]) {
    constexpr int NL = (MAXB + 1) / 2;  // lines
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = 0.0f;
    nblocks = opaque(nblocks);
    const float* xq = xs + line_column(q);
    if constexpr (NT > 2) {
        // no registers to spare for a second group: read as used
#pragma unroll
        for (int v0 = 0; v0 < NL; v0 += 4) {
#pragma unroll
            for (int v = v0; v < v0 + 4 && v < NL; ++v) {
                uint32_t first, second;
                line_pairs(r.w[v], q, first, second);
                if (2 * v < nblocks) {
                    const float w0 = bf16_lo(first), w1 = bf16_hi(first);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const float2 x2 = *reinterpret_cast<const float2*>(xq + xoff[t] + 64 * v);
                        acc[t][0] = add_rn(acc[t][0], mul_rn(w0, x2.x));
                        acc[t][1] = add_rn(acc[t][1], mul_rn(w1, x2.y));
                    }
                }
                if (2 * v + 1 < nblocks) {
                    const float w0 = bf16_lo(second), w1 = bf16_hi(second);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const float2 x2 = *reinterpret_cast<const float2*>(xq + xoff[t] + 64 * v + 32);
                        acc[t][0] = add_rn(acc[t][0], mul_rn(w0, x2.x));
                        acc[t][1] = add_rn(acc[t][1], mul_rn(w1, x2.y));
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    line_sweep<NT, MAXB, G != 0 ? G : (NT == 1 ? 4 : 2)>(r, nblocks, xq, xoff, q, acc);
}

// line_chains_at with token t's vector at xs + t * xstride.
template <int NT, int MAXB, int G = 0>
__device__ __forceinline__ void line_chains(const LineShare<MAXB>& r, int nblocks, const float* __restrict__ xs,
                                            int xstride, int q, float (&acc)[NT][2]) {
    int xoff[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xoff[t] = t * xstride;
    line_chains_at<NT, MAXB, G>(r, nblocks, xs, xoff, q, acc);
}

// f(std::integral_constant<int, n>) for a uniform n in [LO, HI] (n > HI runs HI).
template <int LO, int HI, class F>
__device__ __forceinline__ void with_count(int n, F&& f) {
    if constexpr (LO < HI) {
        if (n == LO) {
            f(std::integral_constant<int, LO>{});
            return;
        }
        with_count<LO + 1, HI>(n, f);
    } else {
        f(std::integral_constant<int, HI>{});
    }
}

// line_chains for one token with the row's line words in LDS (wrow: the row's
// first word; line v is words 16 v .. 16 v + 15, this lane's is 16 v + q):
// the weights and vector values of the next G lines are read while the
// current group is computed.
template <int MAXB, int G>
__device__ __forceinline__ void line_chains_lds(const uint64_t* wrow, int nblocks, const float* __restrict__ xs, int q,
                                                float (&acc)[1][2]) {
    constexpr int NL = (MAXB + 1) / 2;
    acc[0][0] = acc[0][1] = 0.0f;
    nblocks = opaque(nblocks);
    const uint64_t* wq = wrow + q;
    const float* xq = xs + line_column(q);
    uint64_t wv[2][G];
    float2 xv[2][2 * G];
#pragma unroll
    for (int i = 0; i < G && i < NL; ++i) {
        wv[0][i] = wq[16 * i];
        xv[0][2 * i] = *reinterpret_cast<const float2*>(xq + 64 * i);
        xv[0][2 * i + 1] = *reinterpret_cast<const float2*>(xq + 64 * i + 32);
    }
#pragma unroll
    for (int v0 = 0, buf = 0; v0 < NL; v0 += G, buf ^= 1) {
        if (v0 + G < NL) {
#pragma unroll
            for (int i = 0; i < G && v0 + G + i < NL; ++i) {
                wv[buf ^ 1][i] = wq[16 * (v0 + G + i)];
                xv[buf ^ 1][2 * i] = *reinterpret_cast<const float2*>(xq + 64 * (v0 + G + i));
                xv[buf ^ 1][2 * i + 1] = *reinterpret_cast<const float2*>(xq + 64 * (v0 + G + i) + 32);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < G && v0 + i < NL; ++i) {
            const int v = v0 + i;
            uint32_t first, second;
            line_pairs(wv[buf][i], q, first, second);
            if (2 * v < nblocks) {
                acc[0][0] = add_rn(acc[0][0], mul_rn(bf16_lo(first), xv[buf][2 * i].x));
                acc[0][1] = add_rn(acc[0][1], mul_rn(bf16_hi(first), xv[buf][2 * i].y));
            }
            if (2 * v + 1 < nblocks) {
                acc[0][0] = add_rn(acc[0][0], mul_rn(bf16_lo(second), xv[buf][2 * i + 1].x));
                acc[0][1] = add_rn(acc[0][1], mul_rn(bf16_hi(second), xv[buf][2 * i + 1].y));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Tree of the 32 chains in the full-line lane order: (a0+a1)+(a2+a3) in lane
// q == 0 of every 16-lane group.
__device__ __forceinline__ float tree32_reduce_lines(float c0, float c1) {
    c0 = add_rn(c0, dpp_f32<kDppRowShl4>(c0));  // a1[j] = c[j] + c[j+16]
    c1 = add_rn(c1, dpp_f32<kDppRowShl4>(c1));
    c0 = add_rn(c0, dpp_f32<kDppRowShl2>(c0));  // a2[j] = a1[j] + a1[j+8]
    c1 = add_rn(c1, dpp_f32<kDppRowShl2>(c1));
    c0 = add_rn(c0, dpp_f32<kDppRowShl1>(c0));  // a3[j] = a2[j] + a2[j+4]
    c1 = add_rn(c1, dpp_f32<kDppRowShl1>(c1));
    // lane 0 holds a3[0], a3[1]; lane 8 holds a3[2], a3[3]
    float pair = add_rn(c0, c1);
    return add_rn(pair, dpp_f32<kDppRowShl8>(pair));
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

// Wave-wide maximum of a 32-bit unsigned key, as a wave-uniform value: quad
// swaps, half-row and row mirrors, then row broadcasts 15 and 31.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    uint32_t o;
    o = dpp_u32<kDppQuadXor1>(v);
    v = v > o ? v : o;
    o = dpp_u32<kDppQuadXor2>(v);
    v = v > o ? v : o;
    o = dpp_u32<kDppRowHalfMirror>(v);
    v = v > o ? v : o;
    o = dpp_u32<kDppRowMirror>(v);
    v = v > o ? v : o;
    o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, kDppRowBcast15, 0xa, 0xf, false);
    v = v > o ? v : o;
    o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, kDppRowBcast31, 0xc, 0xf, false);
    v = v > o ? v : o;
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// One wave selects the top k of `count` bf16 logits under the total order
// (value descending, then index ascending; src/router.rs:241-247). Each lane
// sorts its MAXPER keys; every round the wave maximum of the lane heads is
// selected and its lane pops it. Writes ids in rank order (lane 0).
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
    // descending odd-even transposition sort of the lane's keys
#pragma unroll
    for (int pass = 0; pass < MAXPER; ++pass) {
#pragma unroll
        for (int m = pass & 1; m + 1 < MAXPER; m += 2) {
            uint32_t a = keys[m], b = keys[m + 1];
            keys[m] = a > b ? a : b;
            keys[m + 1] = a > b ? b : a;
        }
    }
    for (int r = 0; r < k; ++r) {
        uint32_t best = wave_max_u32(keys[0]);
        if (keys[0] == best) {  // keys are unique per expert: exactly one lane
#pragma unroll
            for (int m = 0; m + 1 < MAXPER; ++m) keys[m] = keys[m + 1];
            keys[MAXPER - 1] = 0u;
        }
        if (lane == 0) ids[r] = (int32_t)topk_key_expert(best);
    }
}

// ---- workgroup barriers ----------------------------------------------------------
//
// Barrier for LDS exchange between the waves of a workgroup: the wave's LDS
// (and scalar memory) operations complete, then s_barrier. Unlike
// __syncthreads, whose workgroup-scope fence also waits for every global load
// and store the wave has in flight, it lets prefetched weight rows keep
// streaming across it. The waves of a workgroup exchange data only through
// LDS (between workgroups, tagged words carry their own validity).
__device__ __forceinline__ void wg_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Number of the workgroup's threads with a nonzero predicate (red: four LDS
// words), and the all / any forms; every thread calls them.
__device__ __forceinline__ int wg_count(int32_t* red, int pred) {
    const int c = (int)__popcll(__ballot(pred != 0));
    if (lane_id() == 0) red[wave_id()] = c;
    wg_sync();
    const int total = red[0] + red[1] + red[2] + red[3];
    wg_sync();
    return total;
}
__device__ __forceinline__ bool wg_all(int32_t* red, bool pred) { return wg_count(red, !pred) == 0; }
__device__ __forceinline__ bool wg_any(int32_t* red, bool pred) { return wg_count(red, pred) != 0; }

// ---- inter-workgroup synchronisation for the persistent kernel ----------------------
//
// The per-XCD L2 caches are not coherent with each other, and no cache is
// written back or invalidated here (such a fence is one L2-wide operation, and
// hundreds of workgroups issuing them at once on one XCD serialise behind each
// other). Instead:
//
// * Data one workgroup writes for another (logits, activations, the residual
//   stream) travels as tagged 64-bit words, payload and launch epoch in one
//   agent-scope store that writes through to the coherence point. Readers
//   load through the caches first, so the hundreds of workgroups that read
//   the same small vector mostly hit their XCD's L2 instead of queueing on
//   the few memory channels that hold it, and re-read with agent-scope loads
//   (past the caches) only the words whose tag is not the current epoch.
// * Each phase of each layer has a counter group that every task of the
//   phase increments once, right after issuing its stores (no wait for their
//   acknowledgement: readers check the tags). Atomics on one word are
//   serialised at the coherence point (about 12 ns each: a thousand
//   simultaneous arrivals on one counter take 12 us), so task j of a phase of
//   more than kDirectCount tasks increments sub-counter j mod kSubCounters,
//   and the task completing a sub-counter increments the group's top counter
//   (smaller phases count on the top counter directly). The task completing the top counter
//   writes the epoch into kFlagCopies flag words; a waiter polls the copy for
//   its workgroup, so no single word is polled by more than a few dozen
//   workgroups. The completing task of each counter zeroes it for the next
//   launch (nothing else touches it in this launch).

constexpr int kFlagCopies = 64;
constexpr int kFlagStride = 64;  // words between copies (256 bytes: different memory channels)
constexpr int kSubCounters = 32;
constexpr int kCounterStride = 64;  // words between counters of a group
constexpr int kCounterGroupWords = (1 + kSubCounters) * kCounterStride;  // top, then the sub-counters
constexpr int kDirectCount = 64;  // phases of at most this many tasks count on the top counter only

// Task j of a phase of n tasks counts itself in `group`; returns true in the
// task that completes the phase (thread 0 only).
__device__ __forceinline__ bool count_task(uint32_t* group, int n, int j) {
    auto* top = as_global_rw(group);
    if (n <= kDirectCount) {
        // few tasks: one level (one round trip)
        if (__hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u != (uint32_t)n)
            return false;
        __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
    const int sub = j % kSubCounters;
    const uint32_t sub_target = (uint32_t)((n - sub + kSubCounters - 1) / kSubCounters);
    const uint32_t top_target = (uint32_t)(n < kSubCounters ? n : kSubCounters);
    auto* sc = as_global_rw(group + (1 + sub) * kCounterStride);
    if (__hip_atomic_fetch_add(sc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u != sub_target) return false;
    __hip_atomic_store(sc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u != top_target) return false;
    __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// Announce finished task j of a phase of n tasks from one wave that made all of
// the task's stores (its lane 0 counts; no barrier).
__device__ __forceinline__ void publish_wave(uint32_t* group, int n, int j, uint32_t* flags, uint32_t epoch) {
    if (lane_id() == 0 && count_task(group, n, j)) {
        for (int i = 0; i < kFlagCopies; ++i) coherent_store(flags + i * kFlagStride, epoch);
    }
}

// Announce finished task j of a phase of n tasks. Every wave has issued its
// tagged stores (program order up to the barrier).
__device__ __forceinline__ void publish(uint32_t* group, int n, int j, uint32_t* flags, uint32_t epoch) {
    wg_sync();
    if (threadIdx.x == 0 && count_task(group, n, j)) {
        for (int i = 0; i < kFlagCopies; ++i) coherent_store(flags + i * kFlagStride, epoch);
    }
}

// The pause between two polls of a wait (s_sleep units of 64 clocks, about
// 0.2 µs): thousands of waves polling past the caches slow the weight stream
// they wait on. Measured on the 48-layer decode step (five interleaved runs
// each): 1,331.6 µs per step at 2, 1,322.7 at 8, 1,322.0 at 16, 1,345.1 at 32.
constexpr int kPollSleep = 8;

// Thread 0 polls this workgroup's copy of a phase flag until it holds the
// epoch, bounded by a wall-clock limit and by the shared error word; the
// verdict is broadcast to the workgroup. Returns false if the kernel must stop.
__device__ __forceinline__ bool wait_phase(const uint32_t* flags, uint32_t epoch, int32_t* error,
                                           uint64_t limit_ticks, int32_t* lds_flag) {
    if (threadIdx.x == 0) {
        const uint32_t* f = flags + (blockIdx.x % kFlagCopies) * kFlagStride;
        int32_t ok = 1;
        if (coherent_load(f) != epoch) {
            uint64_t start = wall_clock64();
            // the shared error word (one address every workgroup reads) on
            // every 8th poll
            for (uint32_t poll = 0; coherent_load(f) != epoch; ++poll) {
                if ((poll & 7) == 7 && coherent_load(error) != 0) {
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
                __builtin_amdgcn_s_sleep(kPollSleep);
            }
        }
        *lds_flag = ok;
    }
    wg_sync();
    int32_t ok = *lds_flag;
    wg_sync();
    return ok != 0;
}

// Tagged words v[k] = base[k * STRIDE] for k < n (slots k >= n are left
// alone). The first read goes through the caches; words that do not carry
// `epoch` (a stale cached line, or a store still in flight) are read again past
// the caches until they do, bounded by the wall-clock limit and the shared
// error word. Per lane; false on timeout or error. With `stale`, the number
// of words the first read found without the epoch.
template <int N, int STRIDE>
__device__ __forceinline__ bool load_tagged(uint64_t (&v)[N], const uint64_t* base, int n, uint32_t epoch,
                                            int32_t* error, uint64_t limit_ticks, int* stale = nullptr) {
    const auto* g = as_global(base);
#pragma unroll
    for (int k = 0; k < N; ++k) {
        if (k < n) v[k] = __hip_atomic_load(g + k * STRIDE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok = ok && (k >= n || has_tag(v[k], epoch));
    if (stale != nullptr) {
        int c = 0;
#pragma unroll
        for (int k = 0; k < N; ++k) c += (k < n && !has_tag(v[k], epoch)) ? 1 : 0;
        *stale = c;
    }
    if (ok) return true;
    const uint64_t start = wall_clock64();
    for (uint32_t poll = 0;; ++poll) {
#pragma unroll
        for (int k = 0; k < N; ++k) {
            if (k < n && !has_tag(v[k], epoch))
                v[k] = __hip_atomic_load(g + k * STRIDE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        ok = true;
#pragma unroll
        for (int k = 0; k < N; ++k) ok = ok && (k >= n || has_tag(v[k], epoch));
        if (ok) return true;
        // the shared error word (one address every workgroup reads) on every
        // 8th poll
        if ((poll & 7) == 7 && coherent_load(error) != 0) return false;
        if (wall_clock64() - start > limit_ticks) {
            int32_t expected = 0;
            __hip_atomic_compare_exchange_strong(error, &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(kPollSleep);
    }
}

}  // namespace fw
