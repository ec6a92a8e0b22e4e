// Many-token (prefill) sparse-MoE block: the same block as the decode kernel
// (src/decoder_layer.rs:460-586) for T > 4 tokens, arranged as
//
//   router    exact logits for every (token, router row): k_pf_router_mx on
//             the matrix units, k_pf_router for tiles it flags
//   select    top-k, scores (k_select), shared-gate sigmoid
//   group     (token, expert) pairs grouped by expert, the shared expert as
//             one more group holding every token: k_pf_count, k_pf_scan,
//             k_pf_scatter
//   experts   grouped bf16 GEMMs on MFMA: gate/up with SwiGLU in the
//             epilogue, then down with the route weight (or the shared-gate
//             sigmoid) in the epilogue: k_pf_gemm
//   combine   per token, the weighted expert rows summed in ascending expert
//             id from bf16 zero, then the gated shared row: k_pf_combine
//
// The router keeps the reference's exact dot order (expert ids and scores are
// bit-exact); the expert GEMMs accumulate in the MFMA units' order, so their
// outputs match the reference within a bf16 tolerance, not bit for bit.
#pragma once

#include "fw_device.h"
#include "fw_numerics.h"

namespace fw {

// ---- router -----------------------------------------------------------------------------

constexpr int kPfRouterTokens = 32;  // tokens per block
constexpr int kPfRouterRows = 16;    // router rows per block
constexpr int kPfRouterChunk = 512;  // columns staged per step
constexpr int kPfRouterPad = 32;     // LDS row padding (u16): the two halves of a wave hit other banks

// logits[t][r] = bf16(tree32(W[r,:], x[t,:])) for router rows r < E and
// gate[t] for row E (the shared_expert_gate row), src/expert.rs:514-560 order:
// 32 chains over the 32-column blocks, each summed in block order (multiply,
// then add, each rounded), then the tree (c + c+16, + c+8, + c+4), (a0 + a1) +
// (a2 + a3), + 0.0. Eight groups of 32 lanes per block; group g takes tokens
// 8 (g & 3) .. and rows 8 (g >> 2) .. of the block's tile, lane l of a group
// chain bitrev5(l), so the tree's partners are DPP neighbours.
//
// With `redo` set, a block runs only if the matrix-unit router below flagged
// its tile (redo[token tile * redo_rows + row tile], tiles of kPfMxTokens
// tokens and kPfMxRows rows); it then rewrites that tile's logits.
__global__ void __launch_bounds__(256) k_pf_router(const uint16_t* __restrict__ x, int T, int H,
                                                   const uint16_t* __restrict__ w, int E,
                                                   uint16_t* __restrict__ logits, uint16_t* __restrict__ gate,
                                                   const int32_t* __restrict__ redo, int redo_rows) {
    static_assert(kPfRouterTokens == 32 && kPfRouterRows == 16, "redo tile mapping assumes 32 x 16 blocks");
    if (redo && redo[(int)blockIdx.x * redo_rows + (int)blockIdx.y / 2] == 0) return;
    __shared__ __attribute__((aligned(16))) uint16_t xs[kPfRouterTokens][kPfRouterChunk + kPfRouterPad];
    __shared__ __attribute__((aligned(16))) uint16_t ws[kPfRouterRows][kPfRouterChunk + kPfRouterPad];
    const int tid = (int)threadIdx.x, grp = tid >> 5, lane32 = tid & 31;
    const int ch = (int)(__builtin_bitreverse32((uint32_t)lane32) >> 27);
    const int t0 = (int)blockIdx.x * kPfRouterTokens, r0 = (int)blockIdx.y * kPfRouterRows;
    const int rows = E + 1;
    const int tg = (grp & 3) * 8, rg = (grp >> 2) * 8;
    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i][e] = 0.0f;
    for (int k0 = 0; k0 < H; k0 += kPfRouterChunk) {
        const int kc = min(kPfRouterChunk, H - k0);
        const int pieces = kc / 8;  // 16-byte pieces per row
        for (int id = tid; id < kPfRouterTokens * pieces; id += 256) {
            const int r = id / pieces, pc = id - r * pieces;
            const int t = min(t0 + r, T - 1);
            *reinterpret_cast<uint4*>(&xs[r][pc * 8]) =
                *reinterpret_cast<const uint4*>(x + (size_t)t * H + k0 + pc * 8);
        }
        for (int id = tid; id < kPfRouterRows * pieces; id += 256) {
            const int r = id / pieces, pc = id - r * pieces;
            const int wr = min(r0 + r, rows - 1);
            *reinterpret_cast<uint4*>(&ws[r][pc * 8]) =
                *reinterpret_cast<const uint4*>(w + (size_t)wr * H + k0 + pc * 8);
        }
        __syncthreads();
        for (int p = 0; p < kc / 32; ++p) {
            float xv[8], wv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = from_bf16(xs[tg + i][32 * p + ch]);
#pragma unroll
            for (int e = 0; e < 8; ++e) wv[e] = from_bf16(ws[rg + e][32 * p + ch]);
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[i][e] = add_rn(acc[i][e], mul_rn(wv[e], xv[i]));
        }
        __syncthreads();
    }
    const int base = tid & 32;  // first lane of this group in the wave
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float c = acc[i][e];
            c = add_rn(c, dpp_f32<kDppQuadXor1>(c));  // chain j + (j + 16)
            c = add_rn(c, dpp_f32<kDppQuadXor2>(c));  // + (j + 8)
            c = add_rn(c, dpp_f32<kDppRowRead4>(c));   // + (j + 4)
            const float a1 = __shfl(c, base + 16, kWave);
            const float a2 = __shfl(c, base + 8, kWave);
            const float a3 = __shfl(c, base + 24, kWave);
            const float d = add_rn(add_rn(add_rn(c, a1), add_rn(a2, a3)), 0.0f);
            const int t = t0 + tg + i, r = r0 + rg + e;
            if (lane32 == 0 && t < T && r < rows) {
                if (r < E)
                    logits[(size_t)t * E + r] = to_bf16(d);
                else
                    gate[t] = to_bf16(d);
            }
        }
    }
}

// ---- router on the matrix units ----------------------------------------------------------
//
// The same logits from v_mfma_f32_16x16x1_4b_f32 (four 16 x 16 blocks, K = 1):
// each MFMA step is d = c + a * b for one (chain, token, row), and a product of
// two bf16 values is exact in f32, so the step equals the reference's multiply
// then add with their two roundings (src/expert.rs:514-552) — provided no
// product or partial sum is denormal (the matrix units flush those to zero) and
// nothing overflows. A workgroup takes 32 tokens x 32 rows in eight waves:
// wave v takes the 16 x 16 output tile q = v & 3 (tokens 16 (q & 1), rows
// 16 (q >> 1)) and the chains 16 h .. 16 h + 15, h = v >> 2. Chain 16 h + 4 b + s
// is block b of accumulator set s, so lane l (block l / 16) feeds its 4 sets
// from one 8-byte LDS read of columns 32 p + 16 h + 4 (l / 16) .. + 3, and the
// chains of output (token 4 (l / 16) + r, row l % 16) sit in lane l, register
// 4 b + r of the sets. The tree's first level (chain c + chain c + 16) pairs
// the two halves: the h = 1 wave hands its 64 values over through LDS, and the
// h = 0 wave finishes the tree in registers. 64 accumulator registers per wave
// leave room for four waves per SIMD.
//
// Guard: a tile whose staged x or W holds a nonzero |v| < 2^-55 or |v| >= 2^57
// (Inf and NaN included) is flagged in redo[] and recomputed by k_pf_router.
// Otherwise every nonzero product lies in [2^-110, 2^114): products and partial
// sums are multiples of 2^-125, hence zero or normal, and a chain of H / 32
// terms stays below 2^114 * H / 32 (finite for H < 2^18).
constexpr int kPfMxTokens = 32;
constexpr int kPfMxRows = 32;
constexpr int kPfMxThreads = 512;
constexpr int kPfMxChunk = 256;              // columns per LDS stage
constexpr int kPfMxStride = kPfMxChunk + 8;  // u16 per LDS row: 528 B, rows 4 banks apart
constexpr int kPfMxStageRows = kPfMxTokens + kPfMxRows;
constexpr int kPfMxPieces = kPfMxStageRows * kPfMxChunk / 8 / kPfMxThreads;  // 16-byte pieces per thread
constexpr size_t kPfMxLds = 2 * (size_t)kPfMxStageRows * kPfMxStride * sizeof(uint16_t);  // 67,584 B
constexpr uint16_t kPfMxSmall = 0x2400;  // |bf16| bits of 2^-55
constexpr uint16_t kPfMxLarge = 0x5C00;  // |bf16| bits of 2^57
static_assert(4 * 64 * 64 * sizeof(float) <= kPfMxLds, "hand-over area fits in the stages");

typedef float fw_v16f __attribute__((ext_vector_type(16)));
typedef uint16_t fw_u16x2 __attribute__((ext_vector_type(2)));

// Running range of the magnitudes of eight staged bf16 values: lo = min(|v| - 1)
// (zero wraps to 0xFFFF and never counts as small), hi = max |v|, per u16 half.
__device__ __forceinline__ void mx_range(const uint4& v, fw_u16x2& lo, fw_u16x2& hi) {
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const fw_u16x2 a = __builtin_bit_cast(fw_u16x2, words[q] & 0x7FFF7FFFu);
        lo = __builtin_elementwise_min(lo, a - (fw_u16x2)(1));
        hi = __builtin_elementwise_max(hi, a);
    }
}

// Grid: 8 * ceil(tiles / 8) blocks of kPfMxThreads threads, tiles =
// ceil(T / 32) token tiles x redo_rows = ceil((E + 1) / 32) row tiles;
// kPfMxLds bytes of dynamic LDS. Block b works on tile (b % 8) * ceil(tiles / 8)
// + b / 8: each XCD takes a contiguous range of token tiles with all their row
// tiles, so a token tile's rows are read from HBM once and shared in that
// XCD's L2.
__global__ void __launch_bounds__(kPfMxThreads, 4) k_pf_router_mx(const uint16_t* __restrict__ x, int T, int H,
                                                                  const uint16_t* __restrict__ w, int E,
                                                                  uint16_t* __restrict__ logits,
                                                                  uint16_t* __restrict__ gate,
                                                                  int32_t* __restrict__ redo, int redo_rows) {
    extern __shared__ __attribute__((aligned(16))) uint8_t mx_lds[];
    uint16_t(*stage)[kPfMxStageRows][kPfMxStride] = reinterpret_cast<uint16_t(*)[kPfMxStageRows][kPfMxStride]>(mx_lds);
    const int total = (T + kPfMxTokens - 1) / kPfMxTokens * redo_rows;
    const int per = (total + 7) / 8;
    const int seq = (int)blockIdx.x / 8;
    const int tile = ((int)blockIdx.x % 8) * per + seq;
    if (seq >= per || tile >= total) return;
    const int t0 = tile / redo_rows * kPfMxTokens, r0 = tile % redo_rows * kPfMxRows;
    const int rows = E + 1;
    const int tid = (int)threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int blk = lane >> 4, idx = lane & 15;
    const int quad = wv & 3, half = wv >> 2;
    const int ti = 16 * (quad & 1), rj = 16 * (quad >> 1);
    const int col = 16 * half + 4 * blk;  // first column of this lane's chains in a 32-column block

    // staging: 64 rows (32 token rows, then 32 weight rows) of 32 pieces of 16 B
    const uint16_t* src[kPfMxPieces];
    int dst[kPfMxPieces];
#pragma unroll
    for (int q = 0; q < kPfMxPieces; ++q) {
        const int id = tid + kPfMxThreads * q, row = id >> 5, pc = id & 31;
        dst[q] = row * kPfMxStride + 8 * pc;
        src[q] = row < kPfMxTokens ? x + (size_t)min(t0 + row, T - 1) * H + 8 * pc
                                   : w + (size_t)min(r0 + row - kPfMxTokens, rows - 1) * H + 8 * pc;
    }
    fw_u16x2 lo = (fw_u16x2)(0xFFFF), hi = (fw_u16x2)(0);
    uint4 pre[kPfMxPieces];
#pragma unroll
    for (int q = 0; q < kPfMxPieces; ++q) pre[q] = *reinterpret_cast<const uint4*>(src[q]);
#pragma unroll
    for (int q = 0; q < kPfMxPieces; ++q) {
        mx_range(pre[q], lo, hi);
        *reinterpret_cast<uint4*>(&stage[0][0][0] + dst[q]) = pre[q];
    }
    __syncthreads();

    fw_v16f acc[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[s] = (fw_v16f)(0.0f);
    const int chunks = H / kPfMxChunk;
    constexpr int kSteps = kPfMxChunk / 32;
    for (int c = 0; c < chunks; ++c) {
        const int buf = c & 1;
        const bool more = c + 1 < chunks;
        if (more) {
#pragma unroll
            for (int q = 0; q < kPfMxPieces; ++q)
                pre[q] = *reinterpret_cast<const uint4*>(src[q] + (size_t)(c + 1) * kPfMxChunk);
        }
        // operands of step p + 1 are read while step p's MFMAs run; the next
        // stage is checked and stored mid-chunk (its buffer was last read
        // before the previous barrier)
        const uint16_t* xrow = &stage[buf][ti + idx][col];
        const uint16_t* wrow = &stage[buf][kPfMxTokens + rj + idx][col];
        uint2 xa[2], wb[2];
        xa[0] = *reinterpret_cast<const uint2*>(xrow);
        wb[0] = *reinterpret_cast<const uint2*>(wrow);
#pragma unroll
        for (int p = 0; p < kSteps; ++p) {
            if (p + 1 < kSteps) {
                xa[(p + 1) & 1] = *reinterpret_cast<const uint2*>(xrow + 32 * (p + 1));
                wb[(p + 1) & 1] = *reinterpret_cast<const uint2*>(wrow + 32 * (p + 1));
            }
            const uint32_t xw[2] = {xa[p & 1].x, xa[p & 1].y};
            const uint32_t ww[2] = {wb[p & 1].x, wb[p & 1].y};
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                acc[2 * q] = __builtin_amdgcn_mfma_f32_16x16x1f32(__uint_as_float(xw[q] << 16),
                                                                  __uint_as_float(ww[q] << 16), acc[2 * q], 0, 0, 0);
                acc[2 * q + 1] = __builtin_amdgcn_mfma_f32_16x16x1f32(__uint_as_float(xw[q] & 0xFFFF0000u),
                                                                      __uint_as_float(ww[q] & 0xFFFF0000u),
                                                                      acc[2 * q + 1], 0, 0, 0);
            }
            if (p == kSteps - 3 && more) {
#pragma unroll
                for (int q = 0; q < kPfMxPieces; ++q) {
                    mx_range(pre[q], lo, hi);
                    *reinterpret_cast<uint4*>(&stage[buf ^ 1][0][0] + dst[q]) = pre[q];
                }
            }
        }
        __syncthreads();
    }

    const bool risky = min((int)lo.x, (int)lo.y) < kPfMxSmall - 1 || max((int)hi.x, (int)hi.y) >= kPfMxLarge;
    const int flagged = __syncthreads_or(risky ? 1 : 0);
    if (tid == 0) redo[tile] = flagged ? 1 : 0;
    if (flagged) return;

    // hand-over: value k = 16 s + 4 b + r of the h = 1 wave of tile q at
    // xch[q][k][lane] (the stages are free after the last barrier)
    float* xch = reinterpret_cast<float*>(mx_lds) + quad * 64 * 64 + lane;
    if (half == 1) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int k = 0; k < 16; ++k) xch[(16 * s + k) * 64] = acc[s][k];
    }
    __syncthreads();
    if (half == 1) return;
    // tree per output: (c + c+16) + (c+8) + (c+4) for the four low chains, then
    // ((y0 + y1) + (y2 + y3)) + 0.0; chain 4 b + s is acc[s][4 b + r] here and
    // chain 16 + 4 b + s the partner's value 16 s + 4 b + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float u[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const int s = c & 3, b = c >> 2;
            u[c] = add_rn(acc[s][4 * b + r], xch[(16 * s + 4 * b + r) * 64]);
        }
        float v8[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) v8[c] = add_rn(u[c], u[c + 8]);
        float y[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) y[c] = add_rn(v8[c], v8[c + 4]);
        const float d = add_rn(add_rn(add_rn(y[0], y[1]), add_rn(y[2], y[3])), 0.0f);
        const int t = t0 + ti + 4 * blk + r, row = r0 + rj + idx;
        if (t < T && row < rows) {
            if (row < E)
                logits[(size_t)t * E + row] = to_bf16(d);
            else
                gate[t] = to_bf16(d);
        }
    }
}

// ---- grouping --------------------------------------------------------------------------

// Pair groups: g < E the routed expert g, g = E the shared expert (every token).
struct PfGroups {
    int32_t* counts;        // [E + 1]
    int32_t* cursor;        // [E + 1]
    int32_t* offsets;       // [E + 2] first pair of group g
    int32_t* tile_group;    // [max tiles] group of m-tile i
    int32_t* tile_row0;     // [max tiles] first pair of m-tile i
    int32_t* tiles;         // [1] m-tiles in use
    int32_t* pair_token;    // [P] token of pair p
    uint16_t* pair_scale;   // [P] route weight (score) or shared-gate sigmoid
    int32_t* pair_of;       // [T][K] pair of the token's k-th expert in ascending id
};

constexpr int kPfTileM = 128;  // pairs per GEMM tile

__global__ void k_pf_zero(int32_t* __restrict__ a, int32_t* __restrict__ b, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) a[i] = b[i] = 0;
}

// Selections per expert. Each block takes kPfChunk pairs, counts them in an
// LDS histogram and adds its nonzero bins to the global counts (popular
// experts would otherwise serialise thousands of atomics on one address).
// Ids outside [0, E) occur only when the top-k rejected a NaN logit and left
// them unwritten; such a launch reports the error and its results are void,
// but every access stays in bounds.
constexpr int kPfChunk = 4096;

__global__ void __launch_bounds__(256) k_pf_count(const int32_t* __restrict__ ids, int n, int E,
                                                  int32_t* __restrict__ counts) {
    __shared__ int32_t hist[kMaxExperts];
    for (int e = (int)threadIdx.x; e < E; e += 256) hist[e] = 0;
    __syncthreads();
    const int i0 = (int)blockIdx.x * kPfChunk, i1 = min(n, i0 + kPfChunk);
    for (int i = i0 + (int)threadIdx.x; i < i1; i += 256) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
    }
    __syncthreads();
    for (int e = (int)threadIdx.x; e < E; e += 256)
        if (hist[e] != 0) atomicAdd(&counts[e], hist[e]);
}

// One block of 1024 threads: exclusive scans of the group sizes (pairs and
// m-tiles) and the m-tile table. counts[E] (the shared group) is T.
__global__ void __launch_bounds__(1024) k_pf_scan(PfGroups g, int E, int T) {
    __shared__ int32_t sp[1024], st[1024];
    const int tid = (int)threadIdx.x, G = E + 1;
    const int per = (G + 1023) / 1024;  // groups per thread (G <= 1025)
    int np[2] = {0, 0}, nt[2] = {0, 0}, sump = 0, sumt = 0;
    for (int u = 0; u < per; ++u) {
        const int gi = tid * per + u;
        const int n = gi < E ? g.counts[gi] : (gi == E ? T : 0);
        np[u] = n;
        nt[u] = (n + kPfTileM - 1) / kPfTileM;
        sump += np[u];
        sumt += nt[u];
    }
    sp[tid] = sump;
    st[tid] = sumt;
    __syncthreads();
    // Hillis-Steele inclusive scan
    for (int off = 1; off < 1024; off <<= 1) {
        const int a = tid >= off ? sp[tid - off] : 0, b = tid >= off ? st[tid - off] : 0;
        __syncthreads();
        sp[tid] += a;
        st[tid] += b;
        __syncthreads();
    }
    int p0 = sp[tid] - sump, m0 = st[tid] - sumt;
    for (int u = 0; u < per; ++u) {
        const int gi = tid * per + u;
        if (gi < G) {
            g.offsets[gi] = p0;
            for (int m = 0; m < nt[u]; ++m) {
                g.tile_group[m0 + m] = gi;
                g.tile_row0[m0 + m] = p0 + m * kPfTileM;
            }
        }
        p0 += np[u];
        m0 += nt[u];
    }
    if (tid == 1023) {
        g.offsets[G] = sp[1023];
        g.tiles[0] = st[1023];
    }
}

// Pair p of group e for every (token, rank) selection, and the shared group's
// pair for every token. A block takes kPfChunk selections: it ranks them per
// expert in LDS, reserves one range per expert in the group with a single
// global atomic, and places each selection at its range + rank. The order of
// pairs inside a group follows the atomics; no result depends on it.
__global__ void __launch_bounds__(256) k_pf_scatter(PfGroups g, const int32_t* __restrict__ ids,
                                                    const uint16_t* __restrict__ scores,
                                                    const uint16_t* __restrict__ gate_logit, int T, int K, int E) {
    __shared__ int32_t hist[kMaxExperts];
    const int n = T * K;
    const int chunks = (n + kPfChunk - 1) / kPfChunk;
    if ((int)blockIdx.x >= chunks) {
        // the shared group: token t is pair offsets[E] + t
        const int t = ((int)blockIdx.x - chunks) * 256 + (int)threadIdx.x;
        if (t < T) {
            const int slot = g.offsets[E] + t;
            g.pair_token[slot] = t;
            // src/decoder_layer.rs:563-575: sigmoid of the shared_expert_gate logit
            g.pair_scale[slot] = sigmoid_bf16(gate_logit[t], c_exp2_table);
        }
        return;
    }
    for (int e = (int)threadIdx.x; e < E; e += 256) hist[e] = 0;
    __syncthreads();
    const int i0 = (int)blockIdx.x * kPfChunk, i1 = min(n, i0 + kPfChunk);
    constexpr int kPer = kPfChunk / 256;
    int rank[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = i0 + (int)threadIdx.x + 256 * u;
        const int e = i < i1 ? ids[i] : -1;
        rank[u] = (e >= 0 && e < E) ? atomicAdd(&hist[e], 1) : -1;
    }
    __syncthreads();
    // reserve this block's range in each expert's group
    for (int e = (int)threadIdx.x; e < E; e += 256)
        if (hist[e] != 0) hist[e] = g.offsets[e] + atomicAdd(&g.cursor[e], hist[e]);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        if (rank[u] < 0) continue;
        const int i = i0 + (int)threadIdx.x + 256 * u;
        const int t = i / K, e = ids[i];
        const int slot = hist[e] + rank[u];
        g.pair_token[slot] = t;
        g.pair_scale[slot] = scores[i];
        // the expert's position among the token's experts in ascending id
        int asc = 0;
        for (int j = 0; j < K; ++j) asc += ids[t * K + j] < e ? 1 : 0;
        if (asc < K) g.pair_of[t * K + asc] = slot;
    }
}

// ---- grouped GEMM on MFMA ------------------------------------------------------------
//
// C[p][n] = sum_k A[p][k] W_g[n][k] for the pairs p of each group g (A rows:
// the pair's token row of X for gate/up, the pair's activation row for down).
// Block tile 128 pairs x 256 weight rows, eight waves of 64 x 64, each 2 x 2
// v_mfma_f32_32x32x16_bf16 tiles. Both operands are k-contiguous rows; they
// travel global -> LDS directly (16 bytes per lane) in stages of 32 k, a ring
// of three stages (loads two stages ahead of the MFMAs) in 72 KB, so two
// workgroups share a CU (four waves per SIMD). In a stage each 64-byte row
// holds its four 16-byte chunks permuted by the row (chunk ^ pf_swz(row)), so
// the operand reads (32 rows, one chunk) spread over the LDS banks.
//
// kPfGateUp: the tile's weight rows are 128 gate rows and the matching 128 up
// rows; the epilogue rounds both to bf16 and writes SwiGLU (src/expert.rs:
// 562-571, the SiLU from its 65,536-entry table) to act[p][n]. kPfDown: the epilogue writes bf16(bf16(C) * scale[p])
// (route weighting src/decoder_layer.rs:528-545, shared gating 563-575).

enum PfGemmMode : int { kPfGateUp = 0, kPfDown = 1 };

struct PfGemm {
    const uint16_t* a;          // gate/up: X [T][H]; down: act [P][lda]
    int lda;
    const uint16_t* w_routed;   // gate_up [E][2I][H] or down [E][H][I]
    const uint16_t* w_shared;   // shared_gate (+ shared_up) [2Is][H] or shared_down [H][Is]
    int I, Is;                  // intermediate sizes of routed / shared groups
    int H;
    int E;
    uint16_t* out;              // gate/up: act [P][ldo]; down: weighted rows [P][H]
    int ldo;
    int n_tiles;                // weight-row tiles per pair tile
    const uint16_t* silu;       // gate/up: the SiLU table (k_pf_silu_lut)
};

// silu[b] = silu_bf16(b) for all 65,536 bf16 patterns: the lookup form of
// src/metal_moe.rs:385-392, equal to the computed SiLU on every input.
__global__ void k_pf_silu_lut(uint16_t* __restrict__ silu) {
    const int b = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (b < 65536) silu[b] = silu_bf16((uint32_t)b, c_exp2_table);
}

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPfTileN = 256;                            // weight rows per tile
constexpr int kPfTileK = 32;                             // k per stage (64-byte rows)
constexpr int kPfGemmThreads = 512;
constexpr int kPfABytes = kPfTileM * kPfTileK * 2;       // 8 KB
constexpr int kPfWBytes = kPfTileN * kPfTileK * 2;       // 16 KB
constexpr int kPfActCols = kPfTileN / 2;                 // gate/up: activation columns per tile

// 16-byte chunk c of row r sits at chunk c ^ pf_swz(r) of the row's 64 bytes:
// the 16 rows that one 16-byte read per lane touches (and any 8 of them in
// order) then fall on distinct bank groups.
__device__ __forceinline__ int pf_swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

constexpr int kPfStages = 3;                              // stages in the LDS ring
constexpr int kPfStageLds = kPfStages * (kPfABytes + kPfWBytes);  // 72 KB: two workgroups per CU
constexpr int kPfOutStride = 72;  // u16 per row of a wave's output tile in LDS (64 + 8: banks)
static_assert(8 * 64 * kPfOutStride * 2 <= kPfStageLds, "output tiles fit in the stages");

// Consecutive workgroups go to the eight XCDs in turn, each XCD with its own
// L2: workgroup b runs on XCD b % 8. The tiles in use are ordered pair-tile
// major (all weight tiles of pair tile 0, then of 1, ...; pair tiles are
// sorted by group) and XCD x takes the x-th eighth of that order: the weight
// tiles of one pair tile run side by side on one XCD and share its pair rows
// in L2, and so do the pair tiles of one expert, which share its weights.
// (Grid: m_grid * n_tiles blocks, m_grid >= the tiles in use, a multiple of 8.)
constexpr int kPfXcds = 8;

template <int MODE>
__global__ void __launch_bounds__(kPfGemmThreads, 4) k_pf_gemm(PfGemm q, PfGroups g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_lds[];  // [2 stages][A | W]
    const int total = g.tiles[0] * q.n_tiles;
    const int per = (total + kPfXcds - 1) / kPfXcds;
    const int seq = (int)blockIdx.x / kPfXcds;
    const int order = ((int)blockIdx.x % kPfXcds) * per + seq;
    if (seq >= per || order >= total) return;
    const int mt = order / q.n_tiles, nt = order - mt * q.n_tiles;
    const int grp = g.tile_group[mt], row0 = g.tile_row0[mt];
    const int rows = min(kPfTileM, g.offsets[grp + 1] - row0);
    const bool shared = grp == q.E;
    const int Ig = shared ? q.Is : q.I;
    // K and the weight rows of this tile
    int K;
    const uint16_t* wbase;
    if constexpr (MODE == kPfGateUp) {
        if (nt * kPfActCols >= Ig) return;
        K = q.H;
        wbase = shared ? q.w_shared : q.w_routed + (size_t)grp * 2 * q.I * q.H;
    } else {
        if (nt * kPfTileN >= q.H) return;
        K = Ig;
        wbase = shared ? q.w_shared : q.w_routed + (size_t)grp * q.H * q.I;
    }
    const int tid = (int)threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // down: the pair weights of the tile's rows, for the epilogue (ordered
    // before it by the loop's barriers)
    float* scales = reinterpret_cast<float*>(pf_lds + kPfStageLds);
    if (MODE == kPfDown && tid < kPfTileM) scales[tid] = from_bf16(g.pair_scale[row0 + min(tid, rows - 1)]);
    // this thread's loads per stage: 1 pair-row and 2 weight-row instructions
    // of the wave, 16 rows each (one 1 KB LDS block per instruction, lane l at
    // byte 16 l): rows 16 wv + lane / 4 and 16 (2 wv + i) + lane / 4
    const uint16_t* arow[1];
    int achunk[1];
#pragma unroll
    for (int i = 0; i < 1; ++i) {
        const int r = 16 * wv + (lane >> 2);
        const int pr = row0 + min(r, rows - 1);  // rows past the group's end repeat its last
        if constexpr (MODE == kPfGateUp)
            arow[i] = q.a + (size_t)g.pair_token[pr] * q.lda;
        else
            arow[i] = q.a + (size_t)pr * q.lda;
        achunk[i] = (lane & 3) ^ pf_swz(r);
    }
    const uint16_t* wrow[2];
    int wchunk[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 16 * (2 * wv + i) + (lane >> 2);
        int wr;
        if constexpr (MODE == kPfGateUp)  // gate rows, then the up rows
            wr = r < kPfActCols ? nt * kPfActCols + r : Ig + nt * kPfActCols + (r - kPfActCols);
        else
            wr = nt * kPfTileN + r;
        wrow[i] = wbase + (size_t)wr * K;
        wchunk[i] = (lane & 3) ^ pf_swz(r);
    }
    auto stage = [&](int s) { return pf_lds + s * (kPfABytes + kPfWBytes); };
    auto issue = [&](int s, int k0) {
        uint8_t* base = stage(s);
#pragma unroll
        for (int i = 0; i < 1; ++i)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(arow[i] + k0 + 8 * achunk[i]),
                                             (__attribute__((address_space(3))) void*)(base + (wv + i) * 1024),
                                             16, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(wrow[i] + k0 + 8 * wchunk[i]),
                                             (__attribute__((address_space(3))) void*)(base + kPfABytes + (2 * wv + i) * 1024),
                                             16, 0, 0);
    };
    // A tile of at most 64 pairs spreads its 64 x 256 outputs over all eight
    // waves (32 x 64 each, one MFMA row); loads and barriers are unchanged.
    const bool half = rows <= kPfTileM / 2;
    const int wm = wv & 1, wn = wv >> 1;
    const int rbase = half ? 32 * wm : 64 * wm;  // first tile row of this wave
    pf_f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[mi][ni][e] = 0.0f;
    // operand rows of this lane: pair rows rbase + 32 mi + lane % 32; weight
    // rows (gate/up) 32 wn + lane % 32 and 128 + 32 wn + lane % 32, (down)
    // 64 wn + 32 ni + lane % 32
    int ar[2], br[2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) ar[mi] = rbase + 32 * mi + (lane & 31);
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
        br[ni] = MODE == kPfGateUp ? kPfActCols * ni + 32 * wn + (lane & 31) : 64 * wn + 32 * ni + (lane & 31);
    const int khalf = lane >> 5;
    const int nk = K / kPfTileK;
    // three stages: loads run two stages ahead of the MFMAs
    issue(0, 0);
    if (nk > 1) issue(1, kPfTileK);
    for (int kb = 0; kb < nk; ++kb) {
        // stage kb has landed (only stage kb + 1's three loads per lane may
        // still be in flight), and every wave is done with stage kb - 1,
        // whose buffer the issue below refills (an LDS-only barrier:
        // __syncthreads would also wait for the loads in flight)
        if (kb + 1 < nk)
            asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        wg_sync();
        if (kb + 2 < nk) issue((kb + 2) % kPfStages, (kb + 2) * kPfTileK);
        const uint8_t* at = stage(kb % kPfStages);
        const uint8_t* bt = at + kPfABytes;
        // raised wave priority while this wave feeds the matrix pipe
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kk = 0; kk < kPfTileK / 16; ++kk) {
            const int c = 2 * kk + khalf;
            pf_bf16x8 af[2], bf[2];
            af[0] = *reinterpret_cast<const pf_bf16x8*>(at + ar[0] * 64 + ((c ^ pf_swz(ar[0])) << 4));
            if (!half) af[1] = *reinterpret_cast<const pf_bf16x8*>(at + ar[1] * 64 + ((c ^ pf_swz(ar[1])) << 4));
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                bf[ni] = *reinterpret_cast<const pf_bf16x8*>(bt + br[ni] * 64 + ((c ^ pf_swz(br[ni])) << 4));
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                acc[0][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0], bf[ni], acc[0][ni], 0, 0, 0);
            if (!half) {
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[1][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1], bf[ni], acc[1][ni], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
    }
    // Epilogue: element e of lane l is C[i][j], i = 8 (e / 4) + 4 (l / 32) +
    // e % 4, j = l % 32. Each wave writes its results into its own LDS tile
    // (the stages are free once every wave is past the loop), then stores
    // them as 16-byte row pieces.
    wg_sync();
    const int j = lane & 31;
    uint16_t* ot = reinterpret_cast<uint16_t*>(pf_lds) + wv * 64 * kPfOutStride;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
        if (mi == 1 && half) break;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = 32 * mi + 8 * (e >> 2) + 4 * khalf + (e & 3);  // row in the wave's tile
            if constexpr (MODE == kPfGateUp) {
                // swiglu_bf16 with the SiLU read from its table
                const uint32_t gb = to_bf16(acc[mi][0][e]), ub = to_bf16(acc[mi][1][e]);
                ot[r * kPfOutStride + j] = to_bf16(mul_rn(from_bf16(q.silu[gb]), from_bf16(ub)));
            } else {
                const float scale = scales[rbase + r];
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    const uint32_t y = to_bf16(acc[mi][ni][e]);
                    ot[r * kPfOutStride + 32 * ni + j] = to_bf16(mul_rn(from_bf16(y), scale));
                }
            }
        }
    }
    // (the wave reads back what its other lanes wrote)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr int kPieces = MODE == kPfGateUp ? 4 : 8;  // 16-byte pieces per row of the wave's tile
    const int wave_rows = half ? 32 : 64;
#pragma unroll
    for (int u = 0; u < kPieces; ++u) {
        const int c = lane + kWave * u, r = c / kPieces, pc = c - r * kPieces;
        if (r >= wave_rows || rbase + r >= rows) continue;
        const int pr = row0 + rbase + r;
        const int col = MODE == kPfGateUp ? nt * kPfActCols + 32 * wn + 8 * pc : nt * kPfTileN + 64 * wn + 8 * pc;
        *reinterpret_cast<uint4*>(q.out + (size_t)pr * q.ldo + col) =
            *reinterpret_cast<const uint4*>(ot + r * kPfOutStride + 8 * pc);
    }
}

constexpr size_t kPfGemmLds = kPfStageLds + kPfTileM * 4;  // 72 KB of stages + the pair scales

// ---- combine ---------------------------------------------------------------------------

// out[t][h] = add_bf16(mix, gated): mix = 0; for the token's experts in
// ascending id, mix = bf16(mix + weighted) (src/expert.rs:953-955,
// src/decoder_layer.rs:475-546), gated = the shared group's row
// (src/decoder_layer.rs:576-586). Eight columns per thread.
__global__ void __launch_bounds__(256) k_pf_combine(const uint16_t* __restrict__ weighted, PfGroups g, int T, int K,
                                                    int H, int E, uint16_t* __restrict__ out,
                                                    uint16_t* __restrict__ mixture) {
    const int t = (int)blockIdx.x;
    const int shared_pair = g.offsets[E] + t;
    const int last = g.offsets[E + 1] - 1;  // (pair indices clamped: see k_pf_count)
    for (int h0 = 8 * (int)threadIdx.x; h0 < H; h0 += 8 * (int)blockDim.x) {
        uint32_t mix[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) mix[u] = to_bf16(0.0f);
        for (int k = 0; k < K; ++k) {
            const int pr = min(max(g.pair_of[t * K + k], 0), last);
            const uint4 v = *reinterpret_cast<const uint4*>(weighted + (size_t)pr * H + h0);
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                mix[2 * u] = add_bf16(mix[2 * u], w4[u] & 0xffffu);
                mix[2 * u + 1] = add_bf16(mix[2 * u + 1], w4[u] >> 16);
            }
        }
        const uint4 s = *reinterpret_cast<const uint4*>(weighted + (size_t)shared_pair * H + h0);
        const uint32_t s4[4] = {s.x, s.y, s.z, s.w};
        uint32_t o4[4], m4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t lo = add_bf16(mix[2 * u], s4[u] & 0xffffu);
            const uint32_t hi = add_bf16(mix[2 * u + 1], s4[u] >> 16);
            o4[u] = lo | (hi << 16);
            m4[u] = mix[2 * u] | (mix[2 * u + 1] << 16);
        }
        *reinterpret_cast<uint4*>(out + (size_t)t * H + h0) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
        if (mixture != nullptr)
            *reinterpret_cast<uint4*>(mixture + (size_t)t * H + h0) = make_uint4(m4[0], m4[1], m4[2], m4[3]);
    }
}

}  // namespace fw
