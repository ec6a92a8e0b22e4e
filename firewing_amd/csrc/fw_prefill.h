// Many-token (prefill) sparse-MoE block: the same block as the decode kernel
// (src/decoder_layer.rs:460-586) for T > 4 tokens, arranged as
//
//   router    exact logits for every (token, router row): k_pf_router
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
__global__ void __launch_bounds__(256) k_pf_router(const uint16_t* __restrict__ x, int T, int H,
                                                   const uint16_t* __restrict__ w, int E,
                                                   uint16_t* __restrict__ logits, uint16_t* __restrict__ gate) {
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

__global__ void k_pf_zero(int32_t* __restrict__ a, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) a[i] = 0;
}

// (ids outside [0, E) occur only when the top-k rejected a NaN logit and left
// them unwritten; such a launch reports the error and its results are void,
// but every access stays in bounds)
__global__ void k_pf_count(const int32_t* __restrict__ ids, int n, int E, int32_t* __restrict__ counts) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&counts[e], 1);
    }
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
// pair for every token. The order of pairs inside a group follows the
// atomics; no result depends on it.
__global__ void k_pf_scatter(PfGroups g, const int32_t* __restrict__ ids, const uint16_t* __restrict__ scores,
                             const uint16_t* __restrict__ gate_logit, int T, int K, int E) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < T * K) {
        const int t = i / K, k = i - t * K;
        const int e = ids[i];
        if (e < 0 || e >= E) return;
        const int slot = g.offsets[e] + atomicAdd(&g.cursor[e], 1);
        g.pair_token[slot] = t;
        g.pair_scale[slot] = scores[i];
        // the expert's position among the token's experts in ascending id
        int asc = 0;
        for (int j = 0; j < K; ++j) asc += ids[t * K + j] < e ? 1 : 0;
        if (asc < K) g.pair_of[t * K + asc] = slot;
        (void)k;
    } else if (i < T * K + T) {
        const int t = i - T * K;
        const int slot = g.offsets[E] + t;
        g.pair_token[slot] = t;
        // src/decoder_layer.rs:563-575: sigmoid of the shared_expert_gate logit
        g.pair_scale[slot] = sigmoid_bf16(gate_logit[t], c_exp2_table);
    }
}

// ---- grouped GEMM on MFMA ------------------------------------------------------------
//
// C[p][n] = sum_k A[p][k] W_g[n][k] for the pairs p of each group g (A rows:
// the pair's token row of X for gate/up, the pair's activation row for down).
// Block tile 128 pairs x 128 weight rows x 64 k, four waves of 64 x 64, each
// 2 x 2 v_mfma_f32_32x32x16_bf16 tiles. Both operands are k-contiguous rows;
// they travel global -> LDS directly (16 bytes per lane), double-buffered,
// each 128-byte row chunk stored with its eight 16-byte slots permuted by the
// row (slot ^ swz(row)) so that the operand reads (32 rows, one slot) spread
// over the LDS banks.
//
// kPfGateUp: the tile's weight rows are 64 gate rows and the matching 64 up
// rows; the epilogue rounds both to bf16 and writes SwiGLU (src/expert.rs:
// 562-571) to act[p][n]. kPfDown: the epilogue writes bf16(bf16(C) * scale[p])
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
    int n_tiles;                // weight-row tiles per m-tile in the grid
};

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPfTileN = 128;
constexpr int kPfTileK = 64;
constexpr int kPfTileBytes = kPfTileM * kPfTileK * 2;  // 16 KB per operand tile

__device__ __forceinline__ int pf_swz(int row) { return ((row >> 1) ^ (row << 2)) & 7; }

template <int MODE>
__global__ void __launch_bounds__(256) k_pf_gemm(PfGemm q, PfGroups g) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kPfTileBytes];  // [buffer][A, W]
    const int mt = (int)blockIdx.x / q.n_tiles, nt = (int)blockIdx.x - mt * q.n_tiles;
    if (mt >= g.tiles[0]) return;
    const int grp = g.tile_group[mt], row0 = g.tile_row0[mt];
    const int rows = min(kPfTileM, g.offsets[grp + 1] - row0);
    const bool shared = grp == q.E;
    const int Ig = shared ? q.Is : q.I;
    // K and the weight rows of this tile
    int K;
    const uint16_t* wbase;
    if constexpr (MODE == kPfGateUp) {
        if (nt * 64 >= Ig) return;
        K = q.H;
        wbase = shared ? q.w_shared : q.w_routed + (size_t)grp * 2 * q.I * q.H;
    } else {
        if (nt * kPfTileN >= q.H) return;
        K = Ig;
        wbase = shared ? q.w_shared : q.w_routed + (size_t)grp * q.H * q.I;
    }
    const int tid = (int)threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // rows this thread's loads cover: wave wv, instruction i -> rows 8 (4 wv + i) + lane / 8
    const uint16_t* arow[4];
    const uint16_t* wrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * (4 * wv + i) + (lane >> 3);
        const int pr = row0 + min(r, rows - 1);
        if constexpr (MODE == kPfGateUp)
            arow[i] = q.a + (size_t)g.pair_token[pr] * q.lda;
        else
            arow[i] = q.a + (size_t)pr * q.lda;
        int wr;
        if constexpr (MODE == kPfGateUp)
            wr = r < 64 ? nt * 64 + r : Ig + nt * 64 + (r - 64);  // gate rows, then the up rows
        else
            wr = nt * kPfTileN + r;
        wrow[i] = wbase + (size_t)wr * K;
    }
    const int slot = lane & 7;
    auto load_tile = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 8 * (4 * wv + i) + (lane >> 3);
            const int c = slot ^ pf_swz(r);  // the 16-byte chunk this lane's slot holds
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(arow[i] + k0 + 8 * c),
                                             (__attribute__((address_space(3))) void*)(&lds[buf][0][(4 * wv + i) * 1024]),
                                             16, 0, 0);
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(wrow[i] + k0 + 8 * c),
                                             (__attribute__((address_space(3))) void*)(&lds[buf][1][(4 * wv + i) * 1024]),
                                             16, 0, 0);
        }
    };
    const int wm = wv & 1, wn = wv >> 1;
    pf_f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[mi][ni][e] = 0.0f;
    // operand rows of this lane: A rows wm*64 + 32 mi + lane % 32; weight rows
    // (gate/up) 32 wn + lane % 32 and 64 + 32 wn + lane % 32, (down) 64 wn + 32 ni + lane % 32
    int ar[2], br[2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) ar[mi] = wm * 64 + 32 * mi + (lane & 31);
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
        br[ni] = MODE == kPfGateUp ? 64 * ni + 32 * wn + (lane & 31) : 64 * wn + 32 * ni + (lane & 31);
    const int khalf = lane >> 5;
    const int nk = K / kPfTileK;
    load_tile(0, 0);
    for (int kb = 0; kb < nk; ++kb) {
        const int buf = kb & 1;
        // this tile's loads (the only ones in flight) have landed in every wave
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (kb + 1 < nk) load_tile(buf ^ 1, (kb + 1) * kPfTileK);
        const uint8_t* at = lds[buf][0];
        const uint8_t* bt = lds[buf][1];
#pragma unroll
        for (int kk = 0; kk < kPfTileK / 16; ++kk) {
            const int c = 2 * kk + khalf;
            pf_bf16x8 af[2], bf[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
                af[mi] = *reinterpret_cast<const pf_bf16x8*>(at + ar[mi] * 128 + ((c ^ pf_swz(ar[mi])) << 4));
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                bf[ni] = *reinterpret_cast<const pf_bf16x8*>(bt + br[ni] * 128 + ((c ^ pf_swz(br[ni])) << 4));
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bf[ni], acc[mi][ni], 0, 0, 0);
        }
        // the next iteration's loads overwrite the other buffer only after
        // this barrier-protected read phase of every wave
        __syncthreads();
    }
    // epilogue: element e of lane l is C[i][j], i = 8 (e / 4) + 4 (l / 32) + e % 4, j = l % 32
    const int j = lane & 31;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int i = 8 * (e >> 2) + 4 * khalf + (e & 3);
            const int r = wm * 64 + 32 * mi + i;
            if (r >= rows) continue;
            const int pr = row0 + r;
            if constexpr (MODE == kPfGateUp) {
                const uint32_t gb = to_bf16(acc[mi][0][e]), ub = to_bf16(acc[mi][1][e]);
                q.out[(size_t)pr * q.ldo + nt * 64 + 32 * wn + j] = swiglu_bf16(gb, ub, c_exp2_table);
            } else {
                const float scale = from_bf16(g.pair_scale[pr]);
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    const uint32_t y = to_bf16(acc[mi][ni][e]);
                    q.out[(size_t)pr * q.ldo + nt * kPfTileN + 64 * wn + 32 * ni + j] =
                        to_bf16(mul_rn(from_bf16(y), scale));
                }
            }
        }
    }
}

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
