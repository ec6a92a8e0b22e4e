// GPU decoding of independent zstd frames (the compressed expert container of
// src/compressed_overlap.rs): the kernels that run fw_zstd.h's passes and the
// Decoder that queues them. A call decodes its frames in chunks of the
// decoder's frame capacity; per chunk:
//   k_zs_reset      clears the chunk's work-list counters (a kernel, not a
//                   memset, so a captured graph replays it correctly);
//   k_zs_index      one thread per frame: headers, block list, work lists;
//   k_zs_literals   one wave per Huffman literal section;
//   k_zs_sequences  one wave per block with sequences;
//   k_zs_execute    one 512-thread workgroup per frame, blocks in order, each
//                   block's output built in LDS (a block regenerates at most
//                   128 KB) and then written to the frame's output scratch;
//   k_zs_finish     output scratch -> destination, undoing the BF16 byte
//                   shuffle and splitting at `split`.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdexcept>

#include "fw_zstd.h"
#include "fw_zstd_host.h"

namespace fw::zs {

namespace {

struct DevFrame {
    const uint8_t* src;
    uint64_t size;
    uint64_t content;
    uint8_t* dst;
    uint8_t* dst_tail;
    uint64_t split;
    uint32_t unshuffle;
    uint32_t status;
    uint32_t err_block;
    uint32_t nblocks;
};

struct Work {
    uint32_t frame;  // within the chunk
    uint32_t block;
};

struct Launch {
    DevFrame* frames;  // the chunk's first frame
    uint32_t count;
    Block* blocks;  // [count][max_blocks]
    uint32_t max_blocks;
    uint8_t* lit;  // [count][lit_cap]
    uint64_t lit_cap;
    uint64_t* seq;  // [count][seq_cap]
    uint64_t seq_cap;
    uint8_t* out;  // [count][out_cap]
    uint64_t out_cap;
    Work* huf_work;  // [count * max_blocks]
    Work* seq_work;
    uint32_t* counters;  // [0] Huffman work, [1] sequence work
};

constexpr int kExecThreads = 512;
constexpr int kChunk = 1024;  // sequences per execute round set (2 per thread)

__global__ void k_zs_reset(uint32_t* counters) {
    if (threadIdx.x < 2) counters[threadIdx.x] = 0;
}

__global__ void __launch_bounds__(64) k_zs_index(Launch L) {
    const uint32_t f = blockIdx.x * 64 + threadIdx.x;
    if (f >= L.count) return;
    DevFrame& F = L.frames[f];
    Block* bl = L.blocks + (size_t)f * L.max_blocks;
    FrameInfo info;
    uint32_t st = F.content > L.out_cap ? (uint32_t)kErrContentSize
                                        : index_frame(F.src, F.size, F.content, bl, L.max_blocks, L.lit_cap,
                                                      L.seq_cap, info);
    F.status = st;
    F.err_block = info.err_block;
    F.nblocks = st == kOk ? info.nblocks : 0;
    if (st != kOk) return;
    uint32_t nh = 0, ns = 0;
    for (uint32_t b = 0; b < info.nblocks; ++b) {
        Block& B = bl[b];
        B.rep_end[0] = rep_entry(0);
        B.rep_end[1] = rep_entry(1);
        B.rep_end[2] = rep_entry(2);
        if (B.type != 2) continue;
        nh += B.lit_type == 2;
        if (B.nseq) {
            ++ns;
        } else {
            B.regen = B.lit_size;
            B.sum_ll = 0;
        }
    }
    uint32_t hb = nh ? atomicAdd(&L.counters[0], nh) : 0, sb = ns ? atomicAdd(&L.counters[1], ns) : 0;
    for (uint32_t b = 0; b < info.nblocks; ++b) {
        const Block& B = bl[b];
        if (B.type != 2) continue;
        if (B.lit_type == 2) L.huf_work[hb++] = Work{f, b};
        if (B.nseq) L.seq_work[sb++] = Work{f, b};
    }
}

// One wave per Huffman literal section: lane 0 builds the decoding table in
// LDS, lanes 0..streams-1 decode one stream each into the literal scratch.
__global__ void __launch_bounds__(64) k_zs_literals(Launch L) {
    __shared__ uint16_t dt[1 << kMaxHufBits];
    __shared__ uint8_t wt[256];
    __shared__ FseEntry ft[64];
    __shared__ int16_t norm[256];
    __shared__ uint16_t next[256];
    __shared__ int s_log;
    const int lane = (int)threadIdx.x;
    const uint32_t total = L.counters[0];
    for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        const Work wk = L.huf_work[w];
        const DevFrame& F = L.frames[wk.frame];
        Block& B = L.blocks[(size_t)wk.frame * L.max_blocks + wk.block];
        if (lane == 0) {
            int log = 0;
            const int nsym = huf_weights(F.src + B.huf_desc, (uint32_t)(F.size - B.huf_desc), wt, &log, ft, norm,
                                         next);
            if (nsym) {
                uint32_t start[kMaxHufBits + 2];
                huf_rank_starts(wt, nsym, start);
                for (int s = 0; s < nsym; ++s) {
                    const int wgt = wt[s];
                    if (!wgt) continue;
                    const uint32_t len = (1u << wgt) >> 1;
                    const uint16_t e = huf_entry(s, wgt, log);
                    for (uint32_t i = 0; i < len; ++i) dt[start[wgt] + i] = e;
                    start[wgt] += len;
                }
            }
            s_log = nsym ? log : -1;
        }
        __syncthreads();
        const int log = s_log;
        if (log < 0) {
            if (lane == 0) B.status = kErrHuffman;
        } else if (lane < (int)B.nstreams) {
            const uint32_t seg = B.nstreams == 1 ? B.lit_size : (B.lit_size + 3) / 4;
            const uint32_t cnt = lane == 3 ? B.lit_size - 3 * seg : seg;
            uint8_t* o = L.lit + (size_t)wk.frame * L.lit_cap + B.lit_out + (size_t)lane * seg;
            const bool ok = huf_stream(F.src + B.stream_off[lane], B.stream_size[lane], dt, log, cnt,
                                       [&](uint32_t i, uint8_t v) { o[i] = v; });
            if (!ok) B.status = kErrHuffman;
        }
        __syncthreads();
    }
}

// One wave per block with sequences: lane 0 builds the LL/OF/ML tables in LDS
// and decodes the block's sequences.
__global__ void __launch_bounds__(64) k_zs_sequences(Launch L) {
    __shared__ FseEntry tab[3][512];
    __shared__ int16_t norm[64];
    __shared__ uint16_t next[64];
    const uint32_t total = L.counters[1];
    for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        if (threadIdx.x == 0) {
            const Work wk = L.seq_work[w];
            const DevFrame& F = L.frames[wk.frame];
            Block& B = L.blocks[(size_t)wk.frame * L.max_blocks + wk.block];
            SeqTables T;
            uint32_t st = kOk;
            for (int k = 0; k < 3 && st == kOk; ++k) {
                const int lg = table_for(F.src, B.src + B.size, B.table[k], k, tab[k], norm, next);
                if (lg < 0) st = kErrFse;
                T.t[k] = tab[k];
                T.log[k] = lg;
            }
            uint64_t sll = 0, sml = 0;
            if (st == kOk)
                st = decode_sequences(F.src, B, T, L.seq + (size_t)wk.frame * L.seq_cap + B.seq_out, &sll, &sml,
                                      B.rep_end);
            if (st == kOk && B.lit_size + sml > kBlockMax) st = kErrBlock;
            B.sum_ll = sll;
            B.regen = B.lit_size + sml;
            if (st != kOk) B.status = st;
        }
    }
}

// ---- execute ----------------------------------------------------------------

struct ExecLds {
    uint8_t obuf[kBlockMax];   // the block's output
    uint32_t lit[kChunk + 1];  // literal index where sequence i's literals start (block-relative)
    uint32_t mst[kChunk];      // output position of sequence i's match (block-relative)
    uint32_t ml[kChunk];
    uint32_t off[kChunk];
    uint32_t rpre[kChunk];     // this round's ready match bytes before sequence i
    uint32_t pend[kChunk / 32];
    uint32_t ready[kChunk / 32];
    uint64_t scan[kExecThreads / 64];
    uint32_t flag;
    uint32_t err;
};

// exclusive prefix over the workgroup of a 64-bit value; *total = the sum
__device__ uint64_t wg_scan(uint64_t v, uint64_t* tmp, uint64_t* total) {
    const int lane = (int)threadIdx.x & 63, w = (int)threadIdx.x >> 6;
    uint64_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t lo = __shfl_up((uint32_t)x, d), hi = __shfl_up((uint32_t)(x >> 32), d);
        if (lane >= d) x += ((uint64_t)hi << 32) | lo;
    }
    if (lane == 63) tmp[w] = x;
    __syncthreads();
    uint64_t before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < kExecThreads / 64; ++i) {
        const uint64_t t = tmp[i];
        before += i < w ? t : 0;
        all += t;
    }
    *total = all;
    __syncthreads();
    return before + x - v;
}

// last i in [0, n) with a[i] <= x (a ascending, a[0] <= x)
__device__ __forceinline__ int last_le(const uint32_t* a, int n, uint32_t x) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a[mid] <= x)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Bytes [b, e) of src, 4-byte aligned words loaded whole and the partial ends
// byte by byte (no byte outside [b, e) is read): f(index, byte).
template <typename F>
__device__ __forceinline__ void for_bytes(const uint8_t* src, uint64_t b, uint64_t e, F f) {
    uint64_t i = b;
    const uintptr_t base = (uintptr_t)src;
    while (i < e && ((base + i) & 3)) {
        f(i, src[i]);
        ++i;
    }
    for (; i + 4 <= e; i += 4) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(src + i);
        f(i, (uint8_t)v);
        f(i + 1, (uint8_t)(v >> 8));
        f(i + 2, (uint8_t)(v >> 16));
        f(i + 3, (uint8_t)(v >> 24));
    }
    for (; i < e; ++i) f(i, src[i]);
}

// Literal bytes [j0, j1) of the block (block-relative literal indices) into
// obuf: with `cnt` sequences, literal j of sequence i lands at
// mst[i] - (lit[i + 1] - j); with cnt == 0 (the trailing literals) at
// tail_pos + (j - j0). Each thread takes 16-byte windows of the literal index.
__device__ void copy_literals(ExecLds& S, const Block& B, const uint8_t* litp, uint32_t j0, uint32_t j1, int cnt,
                              uint32_t tail_pos) {
    if (j1 <= j0) return;
    const uint32_t w0 = j0 & ~15u;
    const uint32_t nwin = ((j1 + 15) & ~15u) - w0;
    for (uint32_t a = w0 + 16 * threadIdx.x; a < w0 + nwin; a += 16 * kExecThreads) {
        const uint32_t b = a > j0 ? a : j0, e = a + 16 < j1 ? a + 16 : j1;
        if (b >= e) continue;
        int i = cnt ? last_le(S.lit, cnt, b) : 0;
        auto put = [&](uint64_t j, uint8_t v) {
            if (cnt) {
                while (j >= S.lit[i + 1]) ++i;
                S.obuf[S.mst[i] - (S.lit[i + 1] - (uint32_t)j)] = v;
            } else {
                S.obuf[tail_pos + ((uint32_t)j - j0)] = v;
            }
        };
        if (B.lit_type == 2) {
            for_bytes(litp, b, e, put);
        } else if (B.lit_type == 0) {
            for_bytes(litp, b, e, put);
        } else {
            const uint8_t v = litp[0];
            for (uint32_t j = b; j < e; ++j) put(j, v);
        }
    }
}

// a pending sequence in [lo, hi) of the chunk?
__device__ __forceinline__ bool any_pending(const uint32_t* pend, int lo, int hi) {
    while (lo < hi) {
        const int w = lo >> 5, b = lo & 31;
        const int n = min(32 - b, hi - lo);
        const uint32_t m = (n == 32 ? 0xffffffffu : ((1u << n) - 1)) << b;
        if (pend[w] & m) return true;
        lo += n;
    }
    return false;
}

__device__ void exec_block(ExecLds& S, const DevFrame& F, const Launch& L, uint32_t f, const Block& B,
                           uint8_t* fout) {
    const int t = (int)threadIdx.x;
    const uint64_t base = B.out;
    const uint8_t* litp = B.lit_type == 2 ? L.lit + (size_t)f * L.lit_cap + B.lit_out : F.src + B.lit_src;
    const uint64_t* sq = L.seq + (size_t)f * L.seq_cap + B.seq_out;
    const uint32_t rs[3] = {B.rep_start[0], B.rep_start[1], B.rep_start[2]};
    uint32_t pos = 0, lp = 0;
    for (uint32_t c0 = 0; c0 < B.nseq; c0 += kChunk) {
        const int cnt = (int)min<uint32_t>(kChunk, B.nseq - c0);
        uint32_t ll[2], ml[2], off[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int i = 2 * t + q;
            if (i < cnt) {
                const uint64_t s = sq[c0 + i];
                ll[q] = seq_ll(s);
                ml[q] = seq_ml(s);
                const uint64_t o = rep_resolve(seq_rep(s), rs);
                off[q] = o < (1ull << 31) ? (uint32_t)o : 0;
            } else {
                ll[q] = ml[q] = off[q] = 0;
            }
        }
        const uint64_t mine = ((uint64_t)(ll[0] + ll[1]) << 32) | (ll[0] + ml[0] + ll[1] + ml[1]);
        uint64_t tot;
        const uint64_t pre = wg_scan(mine, S.scan, &tot);
        const uint32_t lit_pre = lp + (uint32_t)(pre >> 32), out_pre = pos + (uint32_t)pre;
        uint32_t li = lit_pre, oi = out_pre;
        if (t < kChunk / 32) S.pend[t] = 0;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int i = 2 * t + q;
            if (i < cnt) {
                S.lit[i] = li;
                S.mst[i] = oi + ll[q];
                S.ml[i] = ml[q];
                S.off[i] = off[q];
                if (ml[q]) {
                    if (off[q] == 0 || (uint64_t)off[q] > base + oi + ll[q]) atomicOr(&S.err, 1u);
                    atomicOr(&S.pend[i >> 5], 1u << (i & 31));
                }
            }
            li += ll[q];
            oi += ll[q] + ml[q];
        }
        if (t == 0) S.lit[cnt] = lp + (uint32_t)(tot >> 32);
        __syncthreads();
        if (S.err) return;
        copy_literals(S, B, litp, lp, lp + (uint32_t)(tot >> 32), cnt, 0);
        __syncthreads();
        // matches in dependency rounds: a match runs once no pending earlier
        // match writes any byte of its source
        for (;;) {
            bool rdy[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int i = 2 * t + q;
                rdy[q] = false;
                if (i < cnt && (S.pend[i >> 5] >> (i & 31) & 1)) {
                    const int64_t src = (int64_t)S.mst[i] - S.off[i];
                    const int64_t e = min<int64_t>(src + S.ml[i], S.mst[i]);
                    bool clash = false;
                    if (e > 0 && i > 0) {
                        const uint32_t s0 = src > 0 ? (uint32_t)src : 0;
                        // first sequence whose match ends past s0, first whose match starts at or past e
                        int lo = 0, hi = i;
                        while (lo < hi) {
                            const int mid = (lo + hi) >> 1;
                            if (S.mst[mid] + S.ml[mid] > s0)
                                hi = mid;
                            else
                                lo = mid + 1;
                        }
                        int lo2 = lo, hi2 = i;
                        while (lo2 < hi2) {
                            const int mid = (lo2 + hi2) >> 1;
                            if (S.mst[mid] >= (uint32_t)e)
                                hi2 = mid;
                            else
                                lo2 = mid + 1;
                        }
                        clash = any_pending(S.pend, lo, lo2);
                    }
                    rdy[q] = !clash;
                }
            }
            const uint64_t mlen = (rdy[0] ? ml[0] : 0) + (rdy[1] ? ml[1] : 0);
            uint64_t rtot;
            const uint32_t rpre = (uint32_t)wg_scan(mlen, S.scan, &rtot);
            if (2 * t < cnt) S.rpre[2 * t] = rpre;
            if (2 * t + 1 < cnt) S.rpre[2 * t + 1] = rpre + (rdy[0] ? ml[0] : 0);
            if (t < kChunk / 32) S.ready[t] = 0;
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 2; ++q)
                if (rdy[q]) atomicOr(&S.ready[(2 * t + q) >> 5], 1u << ((2 * t + q) & 31));
            __syncthreads();
            const uint32_t R = (uint32_t)rtot;
            for (uint32_t b = t; b < R; b += kExecThreads) {
                int i = last_le(S.rpre, cnt, b);
                while (i > 0 && !(S.ready[i >> 5] >> (i & 31) & 1)) --i;  // zero-length entries share a prefix
                const uint32_t k = b - S.rpre[i], o = S.off[i], m = S.mst[i];
                const uint32_t kk = o < S.ml[i] ? k % o : k;
                const int64_t si = (int64_t)m - o + kk;
                S.obuf[m + k] = si >= 0 ? S.obuf[si] : fout[(int64_t)base + si];
            }
            __syncthreads();
            if (t < kChunk / 32) S.pend[t] &= ~S.ready[t];
            if (t == 0) S.flag = 0;
            __syncthreads();
            if (t < kChunk / 32 && S.pend[t]) atomicOr(&S.flag, 1u);
            __syncthreads();
            if (!S.flag) break;
        }
        pos += (uint32_t)tot;
        lp += (uint32_t)(tot >> 32);
    }
    // literals after the last sequence
    copy_literals(S, B, litp, lp, B.lit_size, 0, pos);
    __syncthreads();
}

// obuf[0, n) -> dst[0, n): aligned words stored whole, the ends byte by byte
__device__ void store_block(const uint8_t* obuf, uint8_t* dst, uint32_t n) {
    const uint32_t head = (uint32_t)((4 - ((uintptr_t)dst & 3)) & 3);
    const uint32_t h = head < n ? head : n;
    const int t = (int)threadIdx.x;
    if (t < (int)h) dst[t] = obuf[t];
    const uint32_t words = (n - h) / 4;
    for (uint32_t w = t; w < words; w += kExecThreads) {
        const uint32_t i = h + 4 * w;
        const uint32_t v = (uint32_t)obuf[i] | ((uint32_t)obuf[i + 1] << 8) | ((uint32_t)obuf[i + 2] << 16) |
                           ((uint32_t)obuf[i + 3] << 24);
        *reinterpret_cast<uint32_t*>(dst + i) = v;
    }
    const uint32_t rest = h + 4 * words;
    if (t < (int)(n - rest)) dst[rest + t] = obuf[rest + t];
}

__global__ void __launch_bounds__(kExecThreads) k_zs_execute(Launch L) {
    extern __shared__ __attribute__((aligned(16))) uint8_t zs_lds[];
    ExecLds& S = *reinterpret_cast<ExecLds*>(zs_lds);
    const uint32_t f = blockIdx.x;
    DevFrame& F = L.frames[f];
    if (F.status != kOk) return;
    Block* bl = L.blocks + (size_t)f * L.max_blocks;
    uint8_t* fout = L.out + (size_t)f * L.out_cap;
    const int t = (int)threadIdx.x;
    if (t == 0) {
        // blocks' failures, output positions and starting repeat-offset histories
        uint32_t st = kOk, eb = 0;
        uint32_t cur[3] = {1, 4, 8};
        uint64_t out = 0;
        for (uint32_t b = 0; b < F.nblocks && st == kOk; ++b) {
            Block& B = bl[b];
            if (B.status != kOk) {
                st = B.status;
                eb = b;
                break;
            }
            B.out = out;
            out += B.regen;
            uint32_t nx[3];
            for (int k = 0; k < 3; ++k) {
                B.rep_start[k] = cur[k];
                const uint64_t v = rep_resolve(B.rep_end[k], cur);
                nx[k] = v < (1ull << 31) ? (uint32_t)v : 0;
            }
            for (int k = 0; k < 3; ++k) cur[k] = nx[k];
        }
        if (st == kOk && out != F.content) st = kErrContentSize;
        S.err = 0;
        S.flag = st;
        if (st != kOk) {
            F.status = st;
            F.err_block = eb;
        }
    }
    __syncthreads();
    if (S.flag != kOk) return;
    for (uint32_t b = 0; b < F.nblocks; ++b) {
        const Block& B = bl[b];
        const uint32_t n = (uint32_t)B.regen;
        if (B.type == 0) {
            // raw: through LDS so the stores are whole words
            for (uint64_t a = (B.src & ~3ull) + 4 * t; a < (uint64_t)B.src + n; a += 4 * kExecThreads) {
                const uint64_t lo = a > B.src ? a : B.src, hi = a + 4 < (uint64_t)B.src + n ? a + 4 : B.src + n;
                for_bytes(F.src, lo, hi, [&](uint64_t i, uint8_t v) { S.obuf[i - B.src] = v; });
            }
            __syncthreads();
        } else if (B.type == 1) {
            const uint8_t v = F.src[B.src];
            for (uint32_t i = t; i < n; i += kExecThreads) S.obuf[i] = v;
            __syncthreads();
        } else {
            exec_block(S, F, L, f, B, fout);
            if (S.err) {
                if (t == 0) {
                    F.status = kErrOffset;
                    F.err_block = b;
                }
                return;
            }
        }
        store_block(S.obuf, fout + B.out, n);
        __syncthreads();
    }
}

// Output scratch -> destination. With the unshuffle, element e of the expert
// is (low byte scr[e], high byte scr[half + e]); decoded bytes [0, split) go to
// dst and the rest to dst_tail. grid: (pieces, frames), 4096 bytes a piece.
__global__ void __launch_bounds__(256) k_zs_finish(Launch L) {
    const DevFrame& F = L.frames[blockIdx.y];
    if (F.status != kOk) return;
    const uint8_t* scr = L.out + (size_t)blockIdx.y * L.out_cap;
    const uint64_t n = F.content;
    const uint64_t half = F.unshuffle ? n / 2 : 0;
    const bool tail_ok8 = F.dst_tail == nullptr || (uintptr_t)F.dst_tail % 8 == 0;
    const bool tail_ok16 = F.dst_tail == nullptr || (uintptr_t)F.dst_tail % 16 == 0;
    const bool fast = F.unshuffle ? (half % 4 == 0 && F.split % 8 == 0 && (uintptr_t)F.dst % 8 == 0 && tail_ok8)
                                  : (n % 16 == 0 && F.split % 16 == 0 && (uintptr_t)F.dst % 16 == 0 && tail_ok16);
    for (uint64_t piece = blockIdx.x; piece * 4096 < n; piece += gridDim.x) {
        const uint64_t p0 = piece * 4096;  // output bytes [p0, p0 + 4096)
        if (fast && F.unshuffle) {
            // 4 elements (8 output bytes) at a time: 4 low and 4 high bytes
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const uint64_t e = p0 / 2 + 4 * (threadIdx.x + 256 * r);
                if (e < half) {
                    const uint32_t lo = *reinterpret_cast<const uint32_t*>(scr + e);
                    const uint32_t hi = *reinterpret_cast<const uint32_t*>(scr + half + e);
                    uint64_t v = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        v |= (uint64_t)(((lo >> (8 * i)) & 0xff) | (((hi >> (8 * i)) & 0xff) << 8)) << (16 * i);
                    const uint64_t u = 2 * e;
                    uint8_t* d = u < F.split ? F.dst + u : F.dst_tail + (u - F.split);
                    *reinterpret_cast<uint64_t*>(d) = v;
                }
            }
        } else if (fast) {
            const uint64_t u = p0 + 16 * threadIdx.x;
            if (u < n) {
                const uint4 v = *reinterpret_cast<const uint4*>(scr + u);
                uint8_t* d = u < F.split ? F.dst + u : F.dst_tail + (u - F.split);
                *reinterpret_cast<uint4*>(d) = v;
            }
        } else {
            for (uint64_t u = p0 + threadIdx.x; u < p0 + 4096 && u < n; u += 256) {
                const uint64_t q = half ? ((u & 1) ? half + u / 2 : u / 2) : u;
                uint8_t* d = u < F.split ? F.dst + u : F.dst_tail + (u - F.split);
                *d = scr[q];
            }
        }
    }
}

void hcheck(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename T>
T* dev_alloc(size_t bytes) {
    void* p = nullptr;
    hcheck(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
    return static_cast<T*>(p);
}

}  // namespace

Decoder::Decoder(int device, size_t max_frames, uint64_t max_content) : device_(device) {
    if (max_frames == 0 || max_frames > 65535) throw std::runtime_error("zstd decoder: max_frames must be in [1, 65535]");
    if (max_content == 0 || max_content > kMaxContent)
        throw std::runtime_error("zstd decoder: max_content must be in [1, 2^27 - 1]");
    hcheck(hipSetDevice(device), "hipSetDevice");
    max_frames_ = max_frames;
    max_content_ = max_content;
    max_blocks_ = (uint32_t)(max_content / 1024 + 64);
    out_cap_ = (max_content + 15) & ~15ull;
    lit_cap_ = out_cap_ + 16ull * max_blocks_;
    seq_cap_ = max_content / 3 + 1;
    try {
        blocks_ = dev_alloc<void>(max_frames * (size_t)max_blocks_ * sizeof(Block));
        lit_ = dev_alloc<uint8_t>(max_frames * lit_cap_);
        seq_ = dev_alloc<uint64_t>(max_frames * seq_cap_ * sizeof(uint64_t));
        out_ = dev_alloc<uint8_t>(max_frames * out_cap_);
        work_ = dev_alloc<void>(2 * max_frames * (size_t)max_blocks_ * sizeof(Work));
        counters_ = dev_alloc<uint32_t>(2 * sizeof(uint32_t));
        hcheck(hipEventCreateWithFlags(&last_, hipEventDisableTiming), "hipEventCreate");
        hcheck(hipEventCreateWithFlags(&copied_, hipEventDisableTiming), "hipEventCreate");
        hcheck(hipFuncSetAttribute((const void*)k_zs_execute, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)sizeof(ExecLds)),
               "hipFuncSetAttribute");
        int cus = 0;
        hcheck(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
        grid_ = std::max(1, cus) * 16;
    } catch (...) {
        this->~Decoder();
        throw;
    }
}

Decoder::~Decoder() {
    if (last_) (void)hipEventSynchronize(last_);
    for (void* p : {blocks_, (void*)lit_, (void*)seq_, (void*)out_, work_, (void*)counters_, frames_, (void*)src_})
        if (p) (void)hipFree(p);
    if (pinned_) (void)hipHostFree(pinned_);
    if (frames_host_) (void)hipHostFree(frames_host_);
    if (last_) (void)hipEventDestroy(last_);
    if (copied_) (void)hipEventDestroy(copied_);
    frames_host_ = nullptr;
    copied_ = nullptr;
    blocks_ = work_ = frames_ = nullptr;
    lit_ = out_ = src_ = pinned_ = nullptr;
    seq_ = nullptr;
    counters_ = nullptr;
    last_ = nullptr;
}

uint8_t* Decoder::pinned(size_t bytes) {
    if (bytes > pinned_bytes_) {
        if (last_) hcheck(hipEventSynchronize(last_), "hipEventSynchronize");
        if (pinned_) (void)hipHostFree(pinned_);
        pinned_ = nullptr;
        pinned_bytes_ = 0;
        hcheck(hipHostMalloc((void**)&pinned_, bytes, hipHostMallocDefault), "hipHostMalloc");
        pinned_bytes_ = bytes;
    }
    return pinned_;
}

uint8_t* Decoder::device_source(size_t bytes) {
    if (bytes > src_bytes_) {
        if (last_) hcheck(hipEventSynchronize(last_), "hipEventSynchronize");
        if (src_) (void)hipFree(src_);
        src_ = nullptr;
        src_bytes_ = 0;
        src_ = dev_alloc<uint8_t>(bytes);
        src_bytes_ = bytes;
    }
    return src_;
}

bool Decoder::queue(const std::vector<FrameJob>& jobs, hipStream_t s, std::string* why) {
    const size_t n = jobs.size();
    for (size_t i = 0; i < n; ++i) {
        const FrameJob& j = jobs[i];
        auto bad = [&](const char* m) {
            *why = "zstd frame " + std::to_string(i) + ": " + m;
            return false;
        };
        if (!j.src && j.size) return bad("null source");
        if (j.size > 0xffffffffull) return bad("compressed frame larger than 4 GiB");
        if (j.content > max_content_) return bad("content larger than the decoder's max_content");
        if (j.split > j.content) return bad("split past the content");
        if (j.split && !j.dst) return bad("null dst");
        if (j.split < j.content && !j.dst_tail) return bad("null dst_tail for the bytes past split");
        if (j.unshuffle && (j.content & 1)) return bad("unshuffle needs an even content size");
    }
    hcheck(hipSetDevice(device_), "hipSetDevice");
    hcheck(hipStreamWaitEvent(s, last_, 0), "hipStreamWaitEvent");
    if (n > frames_cap_) {
        hcheck(hipEventSynchronize(last_), "hipEventSynchronize");
        if (frames_) (void)hipFree(frames_);
        if (frames_host_) (void)hipHostFree(frames_host_);
        frames_ = frames_host_ = nullptr;
        frames_cap_ = 0;
        frames_ = dev_alloc<void>(n * sizeof(DevFrame));
        hcheck(hipHostMalloc(&frames_host_, n * sizeof(DevFrame), hipHostMallocDefault), "hipHostMalloc");
        frames_cap_ = n;
    }
    // the frame records go up from pinned memory; the previous call's copy
    // must have left it first
    hcheck(hipEventSynchronize(copied_), "hipEventSynchronize");
    DevFrame* host = static_cast<DevFrame*>(frames_host_);
    for (size_t i = 0; i < n; ++i) {
        const FrameJob& j = jobs[i];
        host[i] = DevFrame{j.src, j.size, j.content, j.dst, j.dst_tail, j.split, j.unshuffle ? 1u : 0u, 0, 0, 0};
    }
    frames_n_ = n;
    if (n) {
        hcheck(hipMemcpyAsync(frames_, host, n * sizeof(DevFrame), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
        hcheck(hipEventRecord(copied_, s), "hipEventRecord");
    }
    for (size_t c0 = 0; c0 < n; c0 += max_frames_) {
        const uint32_t count = (uint32_t)std::min(max_frames_, n - c0);
        Launch L{};
        L.frames = static_cast<DevFrame*>(frames_) + c0;
        L.count = count;
        L.blocks = static_cast<Block*>(blocks_);
        L.max_blocks = max_blocks_;
        L.lit = lit_;
        L.lit_cap = lit_cap_;
        L.seq = seq_;
        L.seq_cap = seq_cap_;
        L.out = out_;
        L.out_cap = out_cap_;
        L.huf_work = static_cast<Work*>(work_);
        L.seq_work = static_cast<Work*>(work_) + max_frames_ * (size_t)max_blocks_;
        L.counters = counters_;
        hipLaunchKernelGGL(k_zs_reset, dim3(1), dim3(64), 0, s, counters_);
        hipLaunchKernelGGL(k_zs_index, dim3((count + 63) / 64), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_literals, dim3(grid_), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_sequences, dim3(grid_), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_execute, dim3(count), dim3(kExecThreads), sizeof(ExecLds), s, L);
        const uint32_t pieces = (uint32_t)std::min<uint64_t>((max_content_ + 4095) / 4096, 2048);
        hipLaunchKernelGGL(k_zs_finish, dim3(pieces, count), dim3(256), 0, s, L);
        hcheck(hipGetLastError(), "zstd kernel launch");
    }
    hcheck(hipEventRecord(last_, s), "hipEventRecord");
    return true;
}

void Decoder::statuses(std::vector<uint32_t>* status, std::vector<uint32_t>* block) {
    hcheck(hipSetDevice(device_), "hipSetDevice");
    hcheck(hipEventSynchronize(last_), "hipEventSynchronize");
    std::vector<DevFrame> host(frames_n_);
    if (frames_n_)
        hcheck(hipMemcpy(host.data(), frames_, frames_n_ * sizeof(DevFrame), hipMemcpyDeviceToHost), "hipMemcpy");
    status->resize(frames_n_);
    block->resize(frames_n_);
    for (size_t i = 0; i < frames_n_; ++i) {
        (*status)[i] = host[i].status;
        (*block)[i] = host[i].err_block;
    }
}

}  // namespace fw::zs
