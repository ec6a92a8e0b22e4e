// GPU decoding of independent zstd frames (the compressed expert container of
// src/compressed_overlap.rs): the kernels that run fw_zstd.h's passes and the
// Decoder that queues them. A call decodes its frames in chunks of the
// decoder's frame capacity; per chunk:
//   k_zs_reset      clears the chunk's work-list counters (a kernel, not a
//                   memset, so a captured graph replays it correctly);
//   k_zs_walk       one thread per frame: frame and block headers;
//   k_zs_parse      one thread per compressed block: its section headers;
//   k_zs_link       one thread per frame: inherited tables, scratch offsets,
//                   the work lists;
//   k_zs_literals   one workgroup per Huffman literal section, a wave per
//                   stream, every lane decoding a segment of it;
//   k_zs_sequences  eight blocks with sequences per wave, a lane each;
//   k_zs_layout     one thread per frame: block output positions and starting
//                   repeat-offset histories;
//   k_zs_raw        one workgroup per raw or RLE block: its bytes in place;
//   k_zs_execute    one 512-thread workgroup per frame, its compressed blocks
//                   in order, each block's output built in LDS (a block
//                   regenerates at most 128 KB) and then written to the
//                   frame's output scratch;
//   k_zs_finish     output scratch -> destination, undoing the BF16 byte
//                   shuffle and splitting at `split`.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <type_traits>

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
    Work* huf_work;  // [count * max_blocks] each
    Work* seq_work;
    Work* raw_work;      // raw and RLE blocks
    Work* parse_work;    // compressed blocks to parse
    uint32_t* counters;  // [0] Huffman work, [1] sequence work, [2] raw/RLE work, [3] parse work
};

constexpr int kExecThreads = 512;
constexpr int kChunk = 1024;  // sequences per execute round set (2 per thread)
constexpr int kFar = 7168;    // LDS bytes for a chunk's sources in earlier blocks
constexpr uint32_t kShort = 64;  // matches up to this long are copied by their own thread

__global__ void k_zs_reset(uint32_t* counters) {
    if (threadIdx.x < 4) counters[threadIdx.x] = 0;
}

// A byte of global memory (a global, not flat, load).
__device__ __forceinline__ uint8_t load_byte(const uint8_t* a) {
    return *(const __attribute__((address_space(1))) uint8_t*)(a);
}

// The 4 bytes at q (any alignment) as a little-endian word: two aligned words
// when those lie inside [ok_lo, ok_hi), else byte by byte.
__device__ __forceinline__ uint32_t load4(const uint8_t* q, const uint8_t* ok_lo, const uint8_t* ok_hi) {
    const uint8_t* a = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(q) & ~uintptr_t(3));
    const int sh = 8 * (int)(q - a);
    if (a >= ok_lo && a + 8 <= ok_hi) {
        const uint64_t x = (uint64_t)load_word(a) | ((uint64_t)load_word(a + 4) << 32);
        return (uint32_t)(x >> sh);
    }
    return (uint32_t)load_byte(q) | ((uint32_t)load_byte(q + 1) << 8) | ((uint32_t)load_byte(q + 2) << 16) |
           ((uint32_t)load_byte(q + 3) << 24);
}

// One thread per frame: the frame header and the block headers; the
// compressed blocks go to the parse work list.
__global__ void __launch_bounds__(64) k_zs_walk(Launch L) {
    const uint32_t f = blockIdx.x * 64 + threadIdx.x;
    if (f >= L.count) return;
    DevFrame& F = L.frames[f];
    Block* bl = L.blocks + (size_t)f * L.max_blocks;
    FrameInfo info;
    const uint32_t st = F.content > L.out_cap ? (uint32_t)kErrContentSize
                                              : walk_frame(F.src, F.size, F.content, bl, L.max_blocks, info);
    F.status = st;
    F.err_block = st == kOk ? 0 : info.err_block;
    F.nblocks = st == kOk ? info.nblocks : 0;
    if (st != kOk) return;
    uint32_t nc = 0;
    for (uint32_t b = 0; b < info.nblocks; ++b) nc += bl[b].type == 2;
    uint32_t pb = nc ? atomicAdd(&L.counters[3], nc) : 0;
    for (uint32_t b = 0; b < info.nblocks; ++b)
        if (bl[b].type == 2) L.parse_work[pb++] = Work{f, b};
}

// One thread per compressed block: its literal and sequence section headers.
__global__ void __launch_bounds__(64) k_zs_parse(Launch L) {
    const uint32_t total = L.counters[3];
    for (uint32_t w = blockIdx.x * 64 + threadIdx.x; w < total; w += gridDim.x * 64) {
        const Work wk = L.parse_work[w];
        const DevFrame& F = L.frames[wk.frame];
        Block& B = L.blocks[(size_t)wk.frame * L.max_blocks + wk.block];
        const uint32_t st = parse_block(F.src, B.src, B.size, B);
        if (st != kOk) B.status = st;
    }
}

// One thread per frame: the blocks linked in order (inherited tables,
// scratch offsets), then the work lists of the decode passes.
__global__ void __launch_bounds__(64) k_zs_link(Launch L) {
    const uint32_t f = blockIdx.x * 64 + threadIdx.x;
    if (f >= L.count) return;
    DevFrame& F = L.frames[f];
    if (F.status != kOk) return;
    Block* bl = L.blocks + (size_t)f * L.max_blocks;
    FrameInfo info;
    const uint32_t st = link_frame(bl, F.nblocks, L.lit_cap, L.seq_cap, info);
    if (st != kOk) {
        F.status = st;
        F.err_block = info.err_block;
        F.nblocks = 0;
        return;
    }
    uint32_t nh = 0, ns = 0, nr = 0;
    for (uint32_t b = 0; b < F.nblocks; ++b) {
        Block& B = bl[b];
        B.rep_end[0] = rep_entry(0);
        B.rep_end[1] = rep_entry(1);
        B.rep_end[2] = rep_entry(2);
        if (B.type != 2) {
            nr += B.regen > 0;
            continue;
        }
        nh += B.lit_type == 2;
        if (B.nseq) {
            ++ns;
        } else {
            B.regen = B.lit_size;
            B.sum_ll = 0;
        }
    }
    uint32_t hb = nh ? atomicAdd(&L.counters[0], nh) : 0, sb = ns ? atomicAdd(&L.counters[1], ns) : 0;
    uint32_t rb = nr ? atomicAdd(&L.counters[2], nr) : 0;
    for (uint32_t b = 0; b < F.nblocks; ++b) {
        const Block& B = bl[b];
        if (B.type != 2) {
            if (B.regen) L.raw_work[rb++] = Work{f, b};
            continue;
        }
        if (B.lit_type == 2) L.huf_work[hb++] = Work{f, b};
        if (B.nseq) L.seq_work[sb++] = Work{f, b};
    }
}


constexpr uint32_t kLitStage = 32 * 1024;  // LDS copy of a block's Huffman streams (larger: read in place)

// Copy bytes [g, g + n) of the frame into LDS at lds + phase (phase = g's
// address mod 4, so words stay aligned): aligned words inside the frame
// [ok_lo, ok_hi) as words, the frame's edge words byte by byte. Returns the
// bytes' LDS address. All `threads` threads of the workgroup take part.
__device__ const uint8_t* stage_bytes(uint8_t* lds, const uint8_t* g, uint32_t n, const uint8_t* ok_lo,
                                      const uint8_t* ok_hi, int threads) {
    const uint8_t* a0 = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(g) & ~uintptr_t(3));
    const uint32_t phase = (uint32_t)(g - a0);
    const uint32_t words = (phase + n + 3) / 4;
    uint32_t* dst = reinterpret_cast<uint32_t*>(lds);
    // eight words a thread in flight, then their stores (one word at a time
    // would wait a memory latency per word)
    for (uint32_t w0 = threadIdx.x; w0 < words; w0 += 8 * (uint32_t)threads) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t w = w0 + (uint32_t)(u * threads);
            const uint8_t* a = a0 + 4 * w;
            v[u] = (w < words && a >= ok_lo && a + 4 <= ok_hi) ? load_word(a) : 0u;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t w = w0 + (uint32_t)(u * threads);
            if (w >= words) break;
            const uint8_t* a = a0 + 4 * w;
            if (!(a >= ok_lo && a + 4 <= ok_hi)) {
                // a frame edge word: its bytes inside the frame
                for (int k = 0; k < 4; ++k)
                    if (a + k >= ok_lo && a + k < ok_hi) v[u] |= (uint32_t)load_byte(a + k) << (8 * k);
            }
            dst[w] = v[u];
        }
    }
    return lds + phase;
}

// 8 bytes of an LDS buffer at q as a little-endian word without a branch:
// three aligned word reads (the buffer is padded so they stay inside it)
// joined by byte alignment.
typedef const __attribute__((address_space(3))) uint8_t* LdsBytes;
__device__ __forceinline__ uint64_t lds_word8(LdsBytes q) {
    typedef const __attribute__((address_space(3))) uint32_t* lp;
    const uint32_t sb = (uint32_t)(uintptr_t)q & 3u;
    const lp a = (lp)(q - sb);
    const uint32_t w0 = a[0], w1 = a[1], w2 = a[2];
    const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, sb), hi = __builtin_amdgcn_alignbyte(w2, w1, sb);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}

// Backward bit reader of the sequence pass: every refill reloads the word at
// the read position (no branch), leaving at least 57 bits above `lo` (or
// the stream's start). A sequence step reads at most 47 bits between
// refills, and a valid stream never reads below its start, so read() is one
// shift; a malformed stream that does gets arbitrary bits (masked to
// the count, so table states stay in range) and drives pos negative, which
// fails the end check. peek() shifts in zeros below the start (the Huffman
// readers' last codewords look past it).
struct SeqBits {
    LdsBytes p;  // stream byte 0 in the lane's window (an LDS address)
    int32_t pos, lo;
    uint64_t c;
    __device__ __forceinline__ void refill() {
        int32_t b = ((pos + 7) >> 3) - 8;
        b = b < 0 ? 0 : b;
        lo = 8 * b;
        c = lds_word8(p + b);
    }
    // nb <= 31 bits below pos, not consumed
    __device__ __forceinline__ uint32_t peek(int nb) const {
        const int32_t sh = pos - lo - nb;
        const uint32_t s1 = (uint32_t)(sh > 0 ? (sh < 63 ? sh : 63) : 0);
        const uint32_t s2 = (uint32_t)(sh < 0 ? -sh : 0) & 63u;
        return (uint32_t)((c >> s1) << s2) & ((1u << nb) - 1u);
    }
    // nb <= 31 bits below pos. After a refill pos - lo <= 64 (64 only when
    // pos is a multiple of 8, where a read of 0 bits gives 0 through the
    // mask), so the shift is (pos - lo) mod 64, what the shift unit takes.
    __device__ __forceinline__ uint32_t read(int nb) {
        pos -= nb;
        return (uint32_t)(c >> ((uint32_t)(pos - lo) & 63u)) & ((1u << nb) - 1u);
    }
};

// One stream of `count` Huffman symbols decoded by a whole wave: lane l
// starts at bit pos0 - l*S (S = pos0/64 rounded up) as if a codeword began
// there and decodes until it passes its segment's end. A prefix code
// resynchronises within a few codewords, so once lane l-1's true end is
// known, lane l redoes its segment from there only if its guess differed,
// and the fix travels up the lanes until nothing changes. Counts then give
// each lane's output offset and a last pass writes the symbols. For a
// stream read in place (too large to stage); staged streams take
// huf_stream_wave_lds.
template <class Mem>
__device__ bool huf_stream_wave(const uint8_t* s, uint32_t size, const uint8_t* ok_lo, const uint8_t* ok_hi,
                                const uint16_t* dt, int log, uint32_t count, uint8_t* out) {
    const int lane = (int)(threadIdx.x & 63);
    if (size == 0) return false;
    const uint32_t lastb = s[size - 1];
    if (lastb == 0) return false;
    const int64_t pos0 = 8 * (int64_t)(size - 1) + highbit32(lastb);
    const int64_t S = (pos0 + 63) / 64;
    int64_t stop = pos0 - (int64_t)(lane + 1) * S;
    if (stop < 0) stop = 0;
    int64_t p = pos0 - (int64_t)lane * S;
    if (p < 0) p = 0;
    BackBitsT<Mem> r;
    r.p = s;
    r.n = size;
    r.ok_lo = ok_lo;
    r.ok_hi = ok_hi;
    auto run = [&](int64_t from, uint8_t* dst, uint32_t& cnt, int64_t& end) -> bool {
        cnt = 0;
        end = from;
        if (from <= stop) return true;
        r.seek(from);
        while (r.pos > stop) {
            if (cnt >= count) return false;
            const uint16_t e = dt[r.peek(log)];
            if (dst) dst[cnt] = (uint8_t)e;
            r.skip(e >> 8);
            ++cnt;
        }
        end = r.pos;
        return true;
    };
    uint32_t c = 0;
    int64_t e = 0;
    bool ok = run(p, nullptr, c, e);
    bool synced = false;
    for (int it = 0; it <= 64; ++it) {
        const uint32_t lo = __shfl_up((uint32_t)e, 1), hi = __shfl_up((uint32_t)((uint64_t)e >> 32), 1);
        const int64_t t = lane == 0 ? pos0 : (int64_t)(((uint64_t)hi << 32) | lo);
        const bool redo = t != p;
        if (!__any(redo)) {
            synced = true;
            break;
        }
        if (redo) {
            p = t;
            ok = run(p, nullptr, c, e);
        }
    }
    // exclusive prefix of the counts
    uint32_t x = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    const uint32_t total = __shfl(x, 63);
    const uint32_t base = x - c;
    const int64_t last_end_lo = (int64_t)__shfl((uint32_t)e, 63);
    const bool good = synced && total == count && last_end_lo == 0 && !__any(!ok);
    if (!good) return false;
    uint32_t c2;
    int64_t e2;
    run(p, out + base, c2, e2);
    return true;
}

// huf_stream_wave for a stream staged in LDS. A lane's first pass from its
// guessed start remembers the first kHufRec codeword boundaries it passes; a
// lane whose guess was wrong decodes from its true start only until it lands
// on its guessed start or one of those boundaries (a prefix code
// resynchronises within a few codewords) and takes the first pass's count
// from there, else it decodes its whole segment again. Steps have no
// branch: the bit word is reloaded at every group of four codewords (4 x 12
// bits <= 57) and a lane past its segment's end stops moving. Every step
// consumes at least one bit (a valid table has no zero-length code), so
// each loop ends.
constexpr int kHufRec = 8;
__device__ bool huf_stream_wave_lds(LdsBytes s, uint32_t size, const uint16_t* dt, int log, uint32_t count,
                                    uint8_t* out) {
    const int lane = (int)(threadIdx.x & 63);
    if (size == 0) return false;
    const uint32_t lastb = s[size - 1];
    if (lastb == 0) return false;
    const int32_t pos0 = 8 * (int32_t)(size - 1) + highbit32(lastb);
    const int32_t S = (pos0 + 63) / 64;
    int32_t stop = pos0 - (lane + 1) * S;
    if (stop < 0) stop = 0;
    int32_t p = pos0 - lane * S;
    if (p < 0) p = 0;
    // the symbols from `from` down to stop (count only); q.pos ends at or below stop
    auto rest = [&](SeqBits& q, uint32_t cnt) -> uint32_t {
        while (q.pos > stop) {
            q.refill();
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool live = q.pos > stop;
                const uint32_t e = dt[q.peek(log)];
                q.pos -= live ? max((int32_t)(e >> 8), 1) : 0;
                cnt += live ? 1u : 0u;
            }
        }
        return cnt;
    };
    // first pass
    const int32_t p1 = p;
    int32_t rec[kHufRec];
    uint32_t c1;
    int32_t e1;
    {
        SeqBits q{s, p, 0, 0};
        uint32_t cnt = 0;
#pragma unroll
        for (int g = 0; g < kHufRec / 4; ++g) {
            q.refill();
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool live = q.pos > stop;
                const uint32_t e = dt[q.peek(log)];
                q.pos -= live ? max((int32_t)(e >> 8), 1) : 0;
                cnt += live ? 1u : 0u;
                rec[4 * g + u] = live ? q.pos : INT32_MAX;  // INT32_MAX: no boundary (never a position)
            }
        }
        c1 = rest(q, cnt);
        e1 = q.pos;
    }
    uint32_t c = c1;
    int32_t e = e1;
    bool synced = false;
    for (int it = 0; it <= 64; ++it) {
        const int32_t tr = __shfl_up(e, 1);
        const int32_t t = lane == 0 ? pos0 : tr;
        const bool redo = t != p;
        if (!__any(redo)) {
            synced = true;
            break;
        }
        if (redo) {
            p = t;
            // position x on the first pass's path: the symbols it has left
            auto on_path = [&](int32_t x, uint32_t* left) -> bool {
                bool hit = x == p1;
                uint32_t l = c1;
#pragma unroll
                for (int k = 0; k < kHufRec; ++k) {
                    const bool h = x == rec[k];
                    l = h ? c1 - (uint32_t)(k + 1) : l;
                    hit = hit || h;
                }
                *left = l;
                return hit;
            };
            SeqBits q{s, t, 0, 0};
            uint32_t j = 0, left = 0;
            bool found = on_path(t, &left);
#pragma unroll
            for (int g = 0; g < kHufRec / 4; ++g) {
                q.refill();
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const bool live = !found && q.pos > stop;
                    const uint32_t en = dt[q.peek(log)];
                    q.pos -= live ? max((int32_t)(en >> 8), 1) : 0;
                    j += live ? 1u : 0u;
                    uint32_t l2;
                    const bool h = live && on_path(q.pos, &l2);
                    left = h ? l2 : left;
                    found = found || h;
                }
            }
            if (found) {
                c = j + left;
                e = e1;
            } else {
                c = rest(q, j);
                e = q.pos;
            }
        }
    }
    // exclusive prefix of the counts
    uint32_t x = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    const uint32_t total = __shfl(x, 63);
    const uint32_t base = x - c;
    const int32_t last_end = __shfl(e, 63);
    if (!(synced && total == count && last_end == 0)) return false;
    // final pass: the lane's c symbols from p
    SeqBits q{s, p, 0, 0};
    uint8_t* dst = out + base;
    uint32_t cnt = 0;
    while (q.pos > stop && cnt < c) {
        q.refill();
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bool live = q.pos > stop && cnt < c;
            const uint32_t en = dt[q.peek(log)];
            if (live) dst[cnt] = (uint8_t)en;
            q.pos -= live ? max((int32_t)(en >> 8), 1) : 0;
            cnt += live ? 1u : 0u;
        }
    }
    return true;
}

// One workgroup per Huffman literal section: thread 0 builds the decoding
// table in LDS, the streams are copied into LDS when they fit, and wave k
// decodes stream k.
__global__ void __launch_bounds__(256) k_zs_literals(Launch L) {
    __shared__ uint16_t dt[1 << kMaxHufBits];
    __shared__ uint8_t wt[256];
    __shared__ FseEntry ft[64];
    __shared__ int16_t norm[256];
    __shared__ uint16_t next[256];
    __shared__ __attribute__((aligned(16))) uint8_t stage[kLitStage + 16];
    __shared__ uint8_t hdesc[128];  // the tree description (at most 128 bytes)
    __shared__ uint16_t s_carry[4];
    __shared__ uint16_t s_wcount[4][kMaxHufBits + 1];  // symbols of each weight, per wave
    __shared__ int s_log, s_nsym;
    __shared__ uint32_t s_bad;
    const int wave = (int)(threadIdx.x >> 6);
    const uint32_t total = L.counters[0];
    for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        const Work wk = L.huf_work[w];
        const DevFrame& F = L.frames[wk.frame];
        Block& B = L.blocks[(size_t)wk.frame * L.max_blocks + wk.block];
        const uint8_t* ok_lo = F.src;
        const uint8_t* ok_hi = F.src + F.size;
        const uint32_t s0 = B.stream_off[0];
        const uint32_t span = B.stream_off[B.nstreams - 1] + B.stream_size[B.nstreams - 1] - s0;
        const bool staged = span + 8 <= kLitStage;
        const uint8_t* sbase = staged ? stage_bytes(stage, F.src + s0, span, ok_lo, ok_hi, 256) : F.src + s0;
        // the description copied to LDS: thread 0's serial weight decoding
        // reads it there (an empty readable window sends every read of the
        // bit readers down their byte path, which LDS serves)
        const uint32_t dn = (uint32_t)min<uint64_t>(sizeof(hdesc), F.size - B.huf_desc);
        if (threadIdx.x < dn) hdesc[threadIdx.x] = load_byte(F.src + B.huf_desc + threadIdx.x);
        __syncthreads();
        if (threadIdx.x == 0) {
            s_bad = 0;
            int log = 0;
            const int nsym = huf_weights(hdesc, dn, wt, &log, ft, norm, next, nullptr, nullptr);
            s_log = nsym ? log : -1;
            s_nsym = nsym;
        }
        __syncthreads();
        const int log = s_log;
        if (log >= 0) {
            // The table in parallel: zeros, then each symbol's entry at its
            // range start (an entry is never 0: its bit count is >= 1), then
            // every entry takes the last range start at or before it (a
            // workgroup scan of "last nonzero" over contiguous pieces).
            const int size = 1 << log, nsym = s_nsym, t = (int)threadIdx.x, lane = t & 63;
            for (int u = t; u < size; u += 256) dt[u] = 0;
            // symbol t's range (weights ascending, symbols ascending within a
            // weight): its rank among the symbols of its weight from a ballot
            // per weight, the weight's first entry from the weights' counts
            const int mw = t < nsym ? wt[t] : 0;
            uint32_t rank = 0;
            for (int w1 = 1; w1 <= kMaxHufBits; ++w1) {
                const uint64_t m = __ballot(mw == w1);
                if (lane == 0) s_wcount[wave][w1] = (uint16_t)__popcll(m);
                if (mw == w1) rank = (uint32_t)__popcll(m & ((1ull << lane) - 1));
            }
            __syncthreads();
            if (mw) {
                uint32_t first = 0;
                for (int w1 = 1; w1 <= kMaxHufBits; ++w1) {
                    const uint32_t n = (uint32_t)s_wcount[0][w1] + s_wcount[1][w1] + s_wcount[2][w1] + s_wcount[3][w1];
                    if (w1 < mw) first += n * ((1u << w1) >> 1);
                }
                for (int w2 = 0; w2 < wave; ++w2) rank += s_wcount[w2][mw];
                dt[first + rank * ((1u << mw) >> 1)] = huf_entry(t, mw, log);
            }
            __syncthreads();
            const int per = (size + 255) / 256, u0 = min(t * per, size), u1 = min(u0 + per, size);
            uint32_t last = 0;
            for (int u = u0; u < u1; ++u)
                if (dt[u]) last = dt[u];
            uint32_t x = last;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t y = (uint32_t)__shfl_up((int)x, d);
                if (lane >= d && x == 0) x = y;
            }
            if (lane == 63) s_carry[wave] = (uint16_t)x;
            uint32_t before = (uint32_t)__shfl_up((int)x, 1);
            if (lane == 0) before = 0;
            __syncthreads();
            for (int w2 = wave - 1; w2 >= 0 && before == 0; --w2) before = s_carry[w2];
            uint32_t cur = before;
            for (int u = u0; u < u1; ++u) {
                const uint32_t e = dt[u];
                if (e)
                    cur = e;
                else
                    dt[u] = (uint16_t)cur;
            }
            __syncthreads();
        }
        if (log < 0) {
            if (threadIdx.x == 0) B.status = kErrHuffman;
        } else if (wave < (int)B.nstreams) {
            const uint32_t seg = B.nstreams == 1 ? B.lit_size : (B.lit_size + 3) / 4;
            const uint32_t cnt = wave == 3 ? B.lit_size - 3 * seg : seg;
            uint8_t* o = L.lit + (size_t)wk.frame * L.lit_cap + B.lit_out + (size_t)wave * seg;
            const uint32_t off = B.stream_off[wave] - s0;
            bool ok;
            if (staged)
                ok = huf_stream_wave_lds((LdsBytes)(sbase + off), B.stream_size[wave], dt, log, cnt, o);
            else
                ok = huf_stream_wave<GlobalMem>(sbase + off, B.stream_size[wave], ok_lo, ok_hi, dt, log, cnt, o);
            if (!ok && (threadIdx.x & 63) == 0) s_bad = 1;
        }
        __syncthreads();
        if (threadIdx.x == 0 && s_bad) B.status = kErrHuffman;
    }
}

constexpr int kSeqLanes = 8;     // blocks per wave in the sequence pass
constexpr int kSeqFlush = 32;    // sequences per lane between record flushes
constexpr int kSeqTable = 1280;  // LL [0, 512), OF [512, 768), ML [768, 1280)
// A sequence reads at most 31 + 16 + 16 extra bits and 9 + 9 + 8 state bits:
// kSeqFlush sequences consume at most 32 x 89 bits = 356 bytes.
constexpr int kSeqBack = 360;
constexpr int kSeqWin = 400;     // a lane's window of its bitstream (>= kSeqBack + 19)

// kSeqLanes blocks per wave, one lane each: the lane builds its block's
// LL/OF/ML tables in LDS and decodes its sequences. Its bitstream is read
// from a window of LDS that the whole wave refills between batches of
// kSeqFlush sequences, so a sequence step never waits on global memory; two
// refills of the bit word per sequence (offset + match-length extra bits <=
// 47, literal-length extra bits + the three state updates <= 42). The wave
// also writes the staged records out between batches.
//
// Table entries: with kWide the four-byte FseEntry (state bits and base read
// directly; 6 KB of LDS a block, three workgroups a CU), else two bytes
// (build_fse16: symbol and state counter, the bits and base recomputed per
// step; 3.2 KB a block, six workgroups a CU). The decoder takes the wide form
// when the call's blocks fit three workgroups a CU and the narrow one when
// more blocks must run at once.
template <bool kWide>
__global__ void __launch_bounds__(64) k_zs_sequences(Launch L) {
    // the table build's counts share the record staging
    using Entry = std::conditional_t<kWide, FseEntry, uint16_t>;
    __shared__ Entry tabs[kSeqLanes][kSeqTable];
    __shared__ union {
        struct {
            int16_t norm[64];
            uint16_t next[64];
        } b;
        uint64_t recs[kSeqFlush];
    } lane_lds[kSeqLanes];
    __shared__ __attribute__((aligned(16))) uint8_t win[kSeqLanes][kSeqWin + 16];
    __shared__ uint32_t llcode[36], mlcode[53];  // value | extra bits << 24
    __shared__ uint32_t s_n[kSeqLanes], s_i[kSeqLanes];
    __shared__ int32_t s_wb[kSeqLanes];
    __shared__ uint64_t* s_out[kSeqLanes];
    __shared__ const uint8_t* s_src[kSeqLanes];
    __shared__ const uint8_t* s_flo[kSeqLanes];
    __shared__ const uint8_t* s_fhi[kSeqLanes];
    __shared__ uint32_t s_active;
    const int lane = (int)threadIdx.x;
    if (lane < 36) llcode[lane] = kLLBase[lane] | ((uint32_t)kLLBits[lane] << 24);
    if (lane < 53) mlcode[lane] = kMLBase[lane] | ((uint32_t)kMLBits[lane] << 24);
    __syncthreads();
    const uint32_t total = L.counters[1];
    for (uint32_t w0 = blockIdx.x * kSeqLanes; w0 < total; w0 += gridDim.x * kSeqLanes) {
        const uint32_t w = w0 + (uint32_t)lane;
        const bool mine = lane < kSeqLanes && w < total;
        Block* Bp = nullptr;
        uint64_t* out = nullptr;
        const uint8_t* sp = nullptr;  // the bitstream in global memory
        const uint8_t* flo = nullptr;
        const uint8_t* fhi = nullptr;
        uint32_t st = kOk, nseq = 0, i = 0;
        SeqBits r{};
        int lg[3] = {0, 0, 0};
        uint32_t sll = 0, sof = 0, sml = 0, rep[3] = {0, 0, 0};
        uint64_t tll = 0, tml = 0;
        Entry* tl = tabs[lane < kSeqLanes ? lane : 0];
        if (mine) {
            const Work wk = L.seq_work[w];
            const DevFrame& F = L.frames[wk.frame];
            Bp = &L.blocks[(size_t)wk.frame * L.max_blocks + wk.block];
            const Block& B = *Bp;
            const uint8_t* f = F.src;
            out = L.seq + (size_t)wk.frame * L.seq_cap + B.seq_out;
            nseq = B.nseq;
            const uint32_t end = B.src + B.size;
            const int off3[3] = {0, 512, 768};
            for (int k = 0; k < 3 && st == kOk; ++k) {
                if constexpr (kWide)
                    lg[k] = table_for(f, end, B.table[k], k, tl + off3[k], lane_lds[lane].b.norm, lane_lds[lane].b.next);
                else
                    lg[k] = table_for16(f, end, B.table[k], k, tl + off3[k], lane_lds[lane].b.norm,
                                        lane_lds[lane].b.next);
                if (lg[k] < 0) st = kErrFse;
            }
            rep[0] = rep_entry(0);
            rep[1] = rep_entry(1);
            rep[2] = rep_entry(2);
            sp = f + B.seq_src;
            flo = f;
            fhi = f + end;
            const uint32_t lastb = B.seq_size ? load_byte(sp + B.seq_size - 1) : 0u;
            if (st == kOk && lastb == 0) st = kErrSequences;
            if (st == kOk) r.pos = 8 * (int32_t)(B.seq_size - 1) + highbit32(lastb);
        }
        bool first = true;
        for (;;) {
            // each lane's window: stream bytes [wb, wb + kSeqWin), wb word-aligned
            // in global memory, reaching kSeqBack bytes below the read position
            int32_t wb = 0;
            const bool reading = mine && st == kOk;
            if (reading) {
                int32_t lo_b = ((r.pos + 7) >> 3) - 8 - kSeqBack;
                lo_b = lo_b < 0 ? 0 : lo_b;
                wb = lo_b - (int32_t)(reinterpret_cast<uintptr_t>(sp + lo_b) & 3);
            }
            if (lane < kSeqLanes) {
                s_wb[lane] = wb;
                s_src[lane] = reading ? sp : nullptr;
                s_flo[lane] = flo;
                s_fhi[lane] = fhi;
            }
            __syncthreads();
            {
                const int ln = lane >> 3, sub = lane & 7;  // 8 threads per lane's window
                const uint8_t* src = s_src[ln];
                if (src) {
                    const uint8_t* a0 = src + s_wb[ln];
                    const uint8_t* lo = s_flo[ln];
                    const uint8_t* hi = s_fhi[ln];
                    // every word of this thread in flight, then the stores (a
                    // word at a time would wait a memory latency per word)
                    constexpr int kPer = (kSeqWin / 4 + 7) / 8;
                    uint32_t v[kPer];
#pragma unroll
                    for (int u = 0; u < kPer; ++u) {
                        const int j = sub + 8 * u;
                        const uint8_t* a = a0 + 4 * j;
                        v[u] = (j < kSeqWin / 4 && a >= lo && a + 4 <= hi) ? load_word(a) : 0u;
                    }
#pragma unroll
                    for (int u = 0; u < kPer; ++u) {
                        const int j = sub + 8 * u;
                        if (j >= kSeqWin / 4) break;
                        const uint8_t* a = a0 + 4 * j;
                        if (!(a >= lo && a + 4 <= hi)) {
                            // a frame edge word: its bytes inside the frame
                            for (int k = 0; k < 4; ++k)
                                if (a + k >= lo && a + k < hi) v[u] |= (uint32_t)load_byte(a + k) << (8 * k);
                        }
                        *reinterpret_cast<uint32_t*>(&win[ln][4 * j]) = v[u];
                    }
                }
            }
            __syncthreads();
            uint32_t k = 0;
            if (reading) {
                r.p = (LdsBytes)(win[lane]) - wb;
                r.refill();
                if (first) {
                    sll = r.read(lg[0]);
                    sof = r.read(lg[1]);
                    sml = r.read(lg[2]);
                }
                const Entry* tll_ = tl;
                const Entry* tof_ = tl + 512;
                const Entry* tml_ = tl + 768;
                // symbols are in range by construction (table_for: counts of
                // at most kMaxSym[kind] symbols, RLE symbols checked)
                // No branch in a step: the first refill goes out with the
                // table reads, a failed offset is noted and ends the lane's
                // batch, and the last sequence reads zero state bits.
                bool bad = false;
                for (; k < (uint32_t)kSeqFlush && i < nseq; ++k) {
                    r.refill();
                    uint32_t ll_sym, ll_nb, ll_base, of_sym, of_nb, of_base, ml_sym, ml_nb, ml_base;
                    if constexpr (kWide) {
                        const FseEntry ell = tll_[sll], eof = tof_[sof], eml = tml_[sml];
                        ll_sym = ell.sym, ll_nb = ell.nb, ll_base = ell.base;
                        of_sym = eof.sym, of_nb = eof.nb, of_base = eof.base;
                        ml_sym = eml.sym, ml_nb = eml.nb, ml_base = eml.base;
                    } else {
                        fse16_unpack(tll_[sll], lg[0], &ll_sym, &ll_nb, &ll_base);
                        fse16_unpack(tof_[sof], lg[1], &of_sym, &of_nb, &of_base);
                        fse16_unpack(tml_[sml], lg[2], &ml_sym, &ml_nb, &ml_base);
                    }
                    const uint32_t mc = mlcode[ml_sym], lc = llcode[ll_sym];
                    const uint32_t ov = (1u << of_sym) + r.read(of_sym);
                    const uint32_t ml = (mc & 0xffffff) + r.read(mc >> 24);
                    r.refill();
                    const uint32_t ll = (lc & 0xffffff) + r.read(lc >> 24);
                    // repeat offsets (RFC 8878 3.1.1.5) without branches: idx 0..2
                    // take history entry idx (idx from the code and ll == 0),
                    // 3 = entry 0 minus one, 4 = a new offset
                    const bool fresh = ov > 3;
                    const uint32_t idx = fresh ? 4u : ov - 1u + (ll == 0);
                    uint32_t m1;
                    const bool m1ok = rep_minus_one(rep[0], &m1);
                    // one of five by masks (a chain of selects on idx is
                    // compiled to a switch, branches in a divergent loop)
                    const uint32_t off = (rep[0] & (0u - (uint32_t)(idx == 0))) |
                                         (rep[1] & (0u - (uint32_t)(idx == 1))) |
                                         (rep[2] & (0u - (uint32_t)(idx == 2))) | (m1 & (0u - (uint32_t)(idx == 3))) |
                                         ((ov - 3) & (0u - (uint32_t)(idx == 4)));
                    bad |= (fresh && ov - 3 >= (1u << 27)) || (idx == 3 && !m1ok);
                    const uint32_t n1 = idx == 0 ? rep[1] : rep[0];
                    const uint32_t n2 = idx <= 1 ? rep[2] : rep[1];
                    rep[0] = off;
                    rep[1] = n1;
                    rep[2] = n2;
                    tll += ll;
                    tml += ml;
                    lane_lds[lane].recs[k] = seq_pack(ll, ml, off);
                    const bool more = ++i < nseq;
                    sll = ll_base + r.read(more ? (int)ll_nb : 0);
                    sml = ml_base + r.read(more ? (int)ml_nb : 0);
                    sof = of_base + r.read(more ? (int)of_nb : 0);
                }
                if (bad) st = kErrOffset;
                // the literal lengths only grow: one check per batch
                if (tll > Bp->lit_size) st = kErrSequences;
            }
            first = false;
            if (lane < kSeqLanes) {
                s_n[lane] = k;
                s_i[lane] = i;
                s_out[lane] = out;
            }
            if (lane == 0) s_active = 0;
            __syncthreads();
            if (mine && st == kOk && i < nseq) atomicOr(&s_active, 1u);
            // the staged records of every lane, written by the whole wave
            for (int q = lane; q < kSeqLanes * kSeqFlush; q += 64) {
                const int ln = q / kSeqFlush, kk = q % kSeqFlush;
                const uint32_t nl = s_n[ln];
                if ((uint32_t)kk < nl) s_out[ln][s_i[ln] - nl + kk] = lane_lds[ln].recs[kk];
            }
            __syncthreads();
            if (!s_active) break;
        }
        if (mine) {
            if (st == kOk && nseq && r.pos != 0) st = kErrSequences;  // the stream ends exactly
            if (st == kOk && Bp->lit_size + tml > kBlockMax) st = kErrBlock;
            Bp->sum_ll = tll;
            Bp->regen = Bp->lit_size + tml;
            if (st == kOk)
                for (int k = 0; k < 3; ++k) Bp->rep_end[k] = rep[k];
            else
                Bp->status = st;
        }
        __syncthreads();
    }
}

// One thread per frame: the blocks' failures, output positions and starting
// repeat-offset histories (composing the blocks' transfers in order).
__global__ void __launch_bounds__(64) k_zs_layout(Launch L) {
    const uint32_t f = blockIdx.x * 64 + threadIdx.x;
    if (f >= L.count) return;
    DevFrame& F = L.frames[f];
    if (F.status != kOk) return;
    Block* bl = L.blocks + (size_t)f * L.max_blocks;
    uint32_t st = kOk, eb = 0;
    uint32_t cur[3] = {1, 4, 8};
    uint64_t out = 0;
    for (uint32_t b = 0; b < F.nblocks; ++b) {
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
    if (st != kOk) {
        F.status = st;
        F.err_block = eb;
    }
}

// Raw and RLE blocks, one workgroup each: the block's bytes to the frame's
// output scratch, whole aligned words (4 per thread in flight) and the ends
// byte by byte.
__global__ void __launch_bounds__(256) k_zs_raw(Launch L) {
    const uint32_t total = L.counters[2];
    const int t = (int)threadIdx.x;
    for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        const Work wk = L.raw_work[w];
        const DevFrame& F = L.frames[wk.frame];
        if (F.status != kOk) continue;
        const Block& B = L.blocks[(size_t)wk.frame * L.max_blocks + wk.block];
        uint8_t* dst = L.out + (size_t)wk.frame * L.out_cap + B.out;
        const uint32_t n = (uint32_t)B.regen;
        const uint8_t* src = F.src + B.src;
        const uint8_t* ok_lo = F.src;
        const uint8_t* ok_hi = F.src + F.size;
        const bool rle = B.type == 1;
        const uint32_t rv = rle ? load_byte(src) * 0x01010101u : 0;
        const uint32_t head = std::min<uint32_t>((4 - ((uintptr_t)dst & 3)) & 3, n);
        if (t < (int)head) dst[t] = rle ? (uint8_t)rv : load_byte(src + t);
        const uint32_t words = (n - head) / 4;
        for (uint32_t w0 = t; w0 < words; w0 += 4 * 256) {
            uint32_t v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t wi = w0 + 256 * u;
                v[u] = wi < words ? (rle ? rv : load4(src + head + 4 * wi, ok_lo, ok_hi)) : 0;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t wi = w0 + 256 * u;
                if (wi < words) *reinterpret_cast<uint32_t*>(dst + head + 4 * wi) = v[u];
            }
        }
        const uint32_t rest = head + 4 * words;
        if (t < (int)(n - rest)) dst[rest + t] = rle ? (uint8_t)rv : load_byte(src + rest + t);
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
    uint32_t fpre[kChunk];     // first byte of sequence i's earlier-block source in far
    // pending matches (a bit per sequence): pq[0] for the general rounds; the
    // rounds of a chunk without shared-out matches rotate over all three
    alignas(16) uint32_t pq[3][kChunk / 32];
    uint32_t ready[kChunk / 32];
    uint64_t scan[kExecThreads / 64];
    uint32_t err;
    uint8_t far[kFar + 20];    // the chunk's match-source bytes from earlier blocks (+ room for the
                               // word reads of a short match's source)
};
static_assert(sizeof(ExecLds) <= 160 * 1024, "the execute pass's LDS fits a workgroup");

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
// tail_pos + (j - j0). Each thread takes 16-byte windows of the literal index,
// loaded whole before they are placed.
__device__ void copy_literals(ExecLds& S, const Block& B, const uint8_t* litp, const uint8_t* ok_lo,
                              const uint8_t* ok_hi, uint32_t j0, uint32_t j1, int cnt, uint32_t tail_pos) {
    if (j1 <= j0) return;
    const uint32_t w0 = j0 & ~15u;
    const uint32_t wend = (j1 + 15) & ~15u;
    for (uint32_t a = w0 + 16 * threadIdx.x; a < wend; a += 16 * kExecThreads) {
        const uint32_t b = a > j0 ? a : j0, e = a + 16 < j1 ? a + 16 : j1;
        uint32_t v[4];
        if (B.lit_type == 2) {
            // the Huffman scratch: 16-byte aligned windows inside the allocation
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = load_word(litp + a + 4 * u);
        } else if (B.lit_type == 0) {
            // raw literals in the frame: the window's bytes inside the literals
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t o = a + 4 * u;
                v[u] = (o >= b && o + 4 <= e) ? load4(litp + o, ok_lo, ok_hi) : 0;
                if (!(o >= b && o + 4 <= e))
                    for (int k = 0; k < 4; ++k)
                        if (o + k >= b && o + k < e) v[u] |= (uint32_t)load_byte(litp + o + k) << (8 * k);
            }
        } else {
            const uint32_t r = load_byte(litp) * 0x01010101u;
            v[0] = v[1] = v[2] = v[3] = r;
        }
        // the current sequence's literal end and output shift (byte j goes
        // to shift + j) in registers: stores to obuf do not force re-reads
        int i = cnt ? last_le(S.lit, cnt, b) : 0;
        uint32_t nxt = cnt ? S.lit[i + 1] : 0xffffffffu;
        uint32_t shift = cnt ? S.mst[i] - nxt : tail_pos - j0;
        for (uint32_t j = b; j < e; ++j) {
            const uint8_t x = (uint8_t)(v[(j - a) >> 2] >> (8 * ((j - a) & 3)));
            while (j >= nxt) {
                ++i;
                nxt = S.lit[i + 1];
                shift = S.mst[i] - nxt;
            }
            S.obuf[shift + j] = x;
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
    const uint8_t* ok_lo = F.src;
    const uint8_t* ok_hi = F.src + F.size;
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
        if (t < kChunk / 32) S.pq[0][t] = S.pq[1][t] = 0;
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
                    atomicOr(&S.pq[0][i >> 5], 1u << (i & 31));
                }
            }
            li += ll[q];
            oi += ll[q] + ml[q];
        }
        if (t == 0) S.lit[cnt] = lp + (uint32_t)(tot >> 32);
        __syncthreads();
        if (S.err) return;
        copy_literals(S, B, litp, ok_lo, ok_hi, lp, lp + (uint32_t)(tot >> 32), cnt, 0);
        __syncthreads();
        // the bytes of earlier blocks that this chunk's matches copy: staged
        // in LDS once (those blocks are final), unless they do not fit
        uint32_t need[2];
        int64_t srcq[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int i = 2 * t + q;
            srcq[q] = (i < cnt && ml[q]) ? (int64_t)S.mst[i] - off[q] : 0;
            // a match reads its first min(off, ml) source bytes (the rest repeat them)
            const int64_t used = srcq[q] + (int64_t)min(off[q], ml[q]);
            need[q] = srcq[q] < 0 ? (uint32_t)((used < 0 ? used : 0) - srcq[q]) : 0;
        }
        uint64_t ftot;
        const uint32_t fpre = (uint32_t)wg_scan(need[0] + need[1], S.scan, &ftot);
        const bool far_ok = ftot <= (uint64_t)kFar;
        if (2 * t < cnt) S.fpre[2 * t] = fpre;
        if (2 * t + 1 < cnt) S.fpre[2 * t + 1] = fpre + need[0];
        __syncthreads();
        if (far_ok) {
            const uint32_t F_ = (uint32_t)ftot;
            for (uint32_t b0 = t; b0 < F_; b0 += 4 * kExecThreads) {
                uint32_t at[4];
                uint8_t v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t b = b0 + u * kExecThreads;
                    at[u] = 0xffffffffu;
                    v[u] = 0;
                    if (b < F_) {
                        // the last sequence with fpre <= b owns byte b (sequences that
                        // stage nothing share their successor's prefix)
                        const int i = last_le(S.fpre, cnt, b);
                        const int64_t src = (int64_t)S.mst[i] - S.off[i];
                        at[u] = b;
                        v[u] = load_byte(fout + ((int64_t)base + src + (b - S.fpre[i])));
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (at[u] != 0xffffffffu) S.far[at[u]] = v[u];
            }
        }
        // matches in dependency rounds: a match runs once no pending earlier
        // match writes any byte of its source. The earlier matches that could
        // (those whose output meets the source) are found once per chunk.
        int clo[2], chi[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int i = 2 * t + q;
            clo[q] = chi[q] = 0;
            if (i < cnt && ml[q]) {
                const int64_t src = srcq[q];
                const int64_t e = min<int64_t>(src + S.ml[i], S.mst[i]);
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
                    clo[q] = lo;
                    chi[q] = lo2;
                }
            }
        }
        __syncthreads();  // far bytes staged
        bool left[2] = {false, false};
#pragma unroll
        for (int q = 0; q < 2; ++q) left[q] = (2 * t + q) < cnt && ml[q] > 0;
        // a match copied by its own thread (short, and its source in this
        // block or in far)
        auto copy_own = [&](int q) {
            const uint32_t m = S.mst[2 * t + q], o = off[q], n = ml[q];
            const int64_t src = srcq[q];
            const uint32_t fb = S.fpre[2 * t + q];
            if (o >= n && n <= 16 && (src >= 0 || (far_ok && src + n <= 0))) {
                // not overlapping its output, the source wholly in this
                // block or wholly staged in far (far[fb + k] = source byte
                // k): the five aligned words around it in one round trip
                // (bytes outside the source may change meanwhile; they are
                // not used)
                typedef const __attribute__((address_space(3))) uint32_t* lw;
                const uint8_t* sbase = src >= 0 ? S.obuf : S.far;
                const uint32_t s0 = src >= 0 ? (uint32_t)src : fb, sb = s0 & 3u;
                const lw wp = (lw)(sbase + (s0 - sb));
                const uint32_t w0 = wp[0], w1 = wp[1], w2 = wp[2], w3 = wp[3], w4 = wp[4];
                const uint32_t v[4] = {__builtin_amdgcn_alignbyte(w1, w0, sb), __builtin_amdgcn_alignbyte(w2, w1, sb),
                                       __builtin_amdgcn_alignbyte(w3, w2, sb), __builtin_amdgcn_alignbyte(w4, w3, sb)};
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    if ((uint32_t)k < n) S.obuf[m + k] = (uint8_t)(v[k >> 2] >> (8 * (k & 3)));
            } else {
                uint32_t k2 = 0;
                for (uint32_t k = 0; k < n; ++k) {
                    // source byte src + k2 (k2 = k mod o): in this block, or staged in far
                    const int64_t si = src + k2;
                    S.obuf[m + k] = si >= 0 ? S.obuf[si] : S.far[fb + k2];
                    if (++k2 == o) k2 = 0;
                }
            }
        };
        // long matches, and earlier-block sources that did not fit in far, are
        // shared out bytewise by the general rounds; a chunk without them runs
        // rounds of one barrier each: a round reads pq[r % 3], marks the
        // matches still to run in pq[(r + 1) % 3] and clears pq[(r + 2) % 3],
        // which nobody reads in that round
        bool shared_out = false;
#pragma unroll
        for (int q = 0; q < 2; ++q) shared_out |= left[q] && (ml[q] > kShort || (srcq[q] < 0 && !far_ok));
        const bool general = __syncthreads_or(shared_out);
        for (int r = 0; !general; ++r) {
            const uint32_t* cur = S.pq[r % 3];
            uint32_t* nxt = S.pq[(r + 1) % 3];
            uint32_t* clr = S.pq[(r + 2) % 3];
            bool rdy[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) rdy[q] = left[q] && !any_pending(cur, clo[q], chi[q]);
#pragma unroll
            for (int q = 0; q < 2; ++q)
                if (rdy[q]) copy_own(q);
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if (left[q] && !rdy[q]) atomicOr(&nxt[(2 * t + q) >> 5], 1u << ((2 * t + q) & 31));
                left[q] = left[q] && !rdy[q];
            }
            if (t < kChunk / 32) clr[t] = 0;
            __syncthreads();
            // the earliest pending match is always ready, so each round ends one
            const uint4* nv = reinterpret_cast<const uint4*>(nxt);
            uint32_t anyw = 0;
#pragma unroll
            for (int w = 0; w < kChunk / 128; ++w) {
                const uint4 x = nv[w];
                anyw |= x.x | x.y | x.z | x.w;
            }
            if (anyw == 0) break;
        }
        for (; general;) {
            bool rdy[2], coop[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                rdy[q] = left[q] && !any_pending(S.pq[0], clo[q], chi[q]);
                // long matches, and earlier-block sources that did not fit in
                // far, are shared out bytewise; the rest stay with their thread
                coop[q] = rdy[q] && (ml[q] > kShort || (srcq[q] < 0 && !far_ok));
            }
#pragma unroll
            for (int q = 0; q < 2; ++q)
                if (rdy[q] && !coop[q]) copy_own(q);
            if (__syncthreads_or(coop[0] || coop[1])) {
                const uint64_t mlen = (coop[0] ? ml[0] : 0) + (coop[1] ? ml[1] : 0);
                uint64_t rtot;
                const uint32_t rpre = (uint32_t)wg_scan(mlen, S.scan, &rtot);
                if (2 * t < cnt) S.rpre[2 * t] = rpre;
                if (2 * t + 1 < cnt) S.rpre[2 * t + 1] = rpre + (coop[0] ? ml[0] : 0);
                if (t < kChunk / 32) S.ready[t] = 0;
                __syncthreads();
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    if (coop[q]) atomicOr(&S.ready[(2 * t + q) >> 5], 1u << ((2 * t + q) & 31));
                __syncthreads();
                const uint32_t R = (uint32_t)rtot;
                for (uint32_t b0 = t; b0 < R; b0 += 4 * kExecThreads) {
                    uint32_t dpos[4];
                    uint8_t val[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const uint32_t b = b0 + u * kExecThreads;
                        dpos[u] = 0xffffffffu;
                        val[u] = 0;
                        if (b < R) {
                            int i = last_le(S.rpre, cnt, b);
                            while (i > 0 && !(S.ready[i >> 5] >> (i & 31) & 1)) --i;  // zero-length entries share a prefix
                            const uint32_t k = b - S.rpre[i], o = S.off[i], m = S.mst[i];
                            const uint32_t kk = o < S.ml[i] ? k % o : k;
                            const int64_t si = (int64_t)m - o + kk;
                            dpos[u] = m + k;
                            val[u] = si >= 0 ? S.obuf[si] : load_byte(fout + ((int64_t)base + si));
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (dpos[u] != 0xffffffffu) S.obuf[dpos[u]] = val[u];
                }
                __syncthreads();
            }
#pragma unroll
            for (int q = 0; q < 2; ++q)
                if (rdy[q]) {
                    atomicAnd(&S.pq[0][(2 * t + q) >> 5], ~(1u << ((2 * t + q) & 31)));
                    left[q] = false;
                }
            if (!__syncthreads_or(left[0] || left[1])) break;
        }
        pos += (uint32_t)tot;
        lp += (uint32_t)(tot >> 32);
    }
    // literals after the last sequence
    copy_literals(S, B, litp, ok_lo, ok_hi, lp, B.lit_size, 0, pos);
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
    const Block* bl = L.blocks + (size_t)f * L.max_blocks;
    uint8_t* fout = L.out + (size_t)f * L.out_cap;
    const int t = (int)threadIdx.x;
    if (t == 0) S.err = 0;
    __syncthreads();
    // compressed blocks in order (raw and RLE blocks are already in place)
    for (uint32_t b = 0; b < F.nblocks; ++b) {
        const Block& B = bl[b];
        if (B.type != 2) continue;
        exec_block(S, F, L, f, B, fout);
        if (S.err) {
            if (t == 0) {
                F.status = kErrOffset;
                F.err_block = b;
            }
            return;
        }
        store_block(S.obuf, fout + B.out, (uint32_t)B.regen);
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
        work_ = dev_alloc<void>(4 * max_frames * (size_t)max_blocks_ * sizeof(Work));
        counters_ = dev_alloc<uint32_t>(4 * sizeof(uint32_t));
        hcheck(hipEventCreateWithFlags(&last_, hipEventDisableTiming), "hipEventCreate");
        hcheck(hipEventCreateWithFlags(&copied_, hipEventDisableTiming), "hipEventCreate");
        hcheck(hipFuncSetAttribute((const void*)k_zs_execute, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)sizeof(ExecLds)),
               "hipFuncSetAttribute");
        int cus = 0;
        hcheck(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
        grid_ = std::max(1, cus) * 16;
        if (const char* e = std::getenv("FIREWING_ZSTD_SEQ_TABLES"))
            seq_tables_ = std::strcmp(e, "wide") == 0 ? 1 : std::strcmp(e, "narrow") == 0 ? 2 : 0;
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
        L.raw_work = static_cast<Work*>(work_) + 2 * max_frames_ * (size_t)max_blocks_;
        L.parse_work = static_cast<Work*>(work_) + 3 * max_frames_ * (size_t)max_blocks_;
        L.counters = counters_;
        hipLaunchKernelGGL(k_zs_reset, dim3(1), dim3(64), 0, s, counters_);
        hipLaunchKernelGGL(k_zs_walk, dim3((count + 63) / 64), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_parse, dim3(grid_), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_link, dim3((count + 63) / 64), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_literals, dim3(grid_), dim3(256), 0, s, L);
        // kSeqLanes blocks per workgroup; the wide tables while the call's
        // compressed blocks fit three workgroups a CU (estimated as one block
        // per kBlockMax of the largest content: a performance choice only,
        // both forms decode alike)
        const uint64_t blocks_est = (uint64_t)count * ((max_content_ + kBlockMax - 1) / kBlockMax);
        const bool wide = seq_tables_ == 1 || (seq_tables_ == 0 && blocks_est <= (uint64_t)(grid_ / 16) * 3 * kSeqLanes);
        if (wide)
            hipLaunchKernelGGL(k_zs_sequences<true>, dim3(grid_), dim3(64), 0, s, L);
        else
            hipLaunchKernelGGL(k_zs_sequences<false>, dim3(grid_), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_layout, dim3((count + 63) / 64), dim3(64), 0, s, L);
        hipLaunchKernelGGL(k_zs_raw, dim3(grid_), dim3(256), 0, s, L);
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
