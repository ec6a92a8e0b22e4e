// Host run of the zstd format core (firewing_amd/csrc/fw_zstd.h: the frame
// index, table builders, Huffman streams and sequence decoding that the GPU
// passes call) under AddressSanitizer, for tests/test_zstd_host.py.
//
//   zstd_host_check decode CASES   every case decodes to its expected bytes
//   zstd_host_check fuzz CASES N S N corrupted variants of each case (seed S)
//                                  decode or fail with a status, never touch
//                                  memory outside the frame and the buffers
//
// CASES: u32 count, then per case u64 content bytes, u64 frame bytes, the
// frame, the content. The executor here places the decoded blocks serially
// with the same rules as the GPU's layout and execute passes (repeat-offset
// histories composed per block, offsets checked against the bytes produced).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "fw_zstd.h"

using namespace fw::zs;

namespace {

struct Case {
    std::vector<uint8_t> frame, content;
};

bool read_cases(const char* path, std::vector<Case>* out) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    uint32_t n = 0;
    bool ok = std::fread(&n, 4, 1, f) == 1;
    for (uint32_t i = 0; ok && i < n; ++i) {
        uint64_t c = 0, fl = 0;
        ok = std::fread(&c, 8, 1, f) == 1 && std::fread(&fl, 8, 1, f) == 1 && c < (1ull << 30) && fl < (1ull << 30);
        if (!ok) break;
        Case k;
        k.frame.resize(fl);
        k.content.resize(c);
        ok = (fl == 0 || std::fread(k.frame.data(), 1, fl, f) == fl) && (c == 0 || std::fread(k.content.data(), 1, c, f) == c);
        out->push_back(std::move(k));
    }
    std::fclose(f);
    return ok;
}

// Decode a frame of `content` bytes into out (exactly that size); a Status.
uint32_t decode(const std::vector<uint8_t>& fr, uint64_t content, std::vector<uint8_t>* out) {
    // the frame in its own allocation, so any read past it is reported
    std::vector<uint8_t> frame(fr);
    const uint8_t* f = frame.empty() ? nullptr : frame.data();
    const uint64_t n = frame.size();
    if (n == 0) return kErrTruncated;
    const uint32_t max_blocks = (uint32_t)(content / 1024 + 64);
    const uint64_t lit_cap = ((content + 15) & ~15ull) + 16ull * max_blocks;
    const uint64_t seq_cap = content / 3 + 1;
    std::vector<Block> blocks(max_blocks);
    FrameInfo info;
    uint32_t st = index_frame(f, n, content, blocks.data(), max_blocks, lit_cap, seq_cap, info);
    if (st) return st;
    std::vector<uint8_t> lit(lit_cap + 16);
    std::vector<uint64_t> seq(seq_cap);
    for (uint32_t b = 0; b < info.nblocks; ++b) {
        Block& B = blocks[b];
        B.rep_end[0] = rep_entry(0);
        B.rep_end[1] = rep_entry(1);
        B.rep_end[2] = rep_entry(2);
        if (B.type != 2) continue;
        if (B.lit_type == 2) {
            uint8_t wt[256];
            FseEntry ft[64];
            int16_t norm[256];
            uint16_t next[256];
            int log = 0;
            const int nsym = huf_weights(f + B.huf_desc, (uint32_t)(n - B.huf_desc), wt, &log, ft, norm, next, f,
                                         f + n);
            if (!nsym) return kErrHuffman;
            uint32_t start[kMaxHufBits + 2];
            huf_rank_starts(wt, nsym, start);
            std::vector<uint16_t> dt(1 << kMaxHufBits);
            for (int s = 0; s < nsym; ++s) {
                if (!wt[s]) continue;
                const uint32_t len = (1u << wt[s]) >> 1;
                for (uint32_t i = 0; i < len; ++i) dt.at(start[wt[s]] + i) = huf_entry(s, wt[s], log);
                start[wt[s]] += len;
            }
            const uint32_t seg = B.nstreams == 1 ? B.lit_size : (B.lit_size + 3) / 4;
            for (uint32_t k = 0; k < B.nstreams; ++k) {
                const uint32_t cnt = k == 3 ? B.lit_size - 3 * seg : seg;
                uint8_t* o = lit.data() + B.lit_out + (size_t)k * seg;
                if (!huf_stream(f + B.stream_off[k], B.stream_size[k], dt.data(), log, cnt,
                                [&](uint32_t i, uint8_t v) { o[i] = v; }, f, f + n))
                    return kErrHuffman;
            }
        }
        if (B.nseq) {
            FseEntry t[512];
            SeqEntry se[3][512];
            int16_t norm[64];
            uint16_t next[64];
            SeqTables T;
            for (int k = 0; k < 3; ++k) {
                const int lg = table_for(f, B.src + B.size, B.table[k], k, t, norm, next);
                // the GPU's two-byte tables (build_fse16) fail alike and unpack
                // to the same entries
                uint16_t t16[512];
                const int lg16 = table_for16(f, B.src + B.size, B.table[k], k, t16, norm, next);
                if (lg16 != lg) {
                    std::fprintf(stderr, "table_for16 log %d, table_for %d\n", lg16, lg);
                    std::abort();
                }
                for (int u = 0; lg >= 0 && u < (1 << lg); ++u) {
                    uint32_t sym, nb, base;
                    fse16_unpack(t16[u], lg, &sym, &nb, &base);
                    if (sym != t[u].sym || nb != t[u].nb || base != t[u].base) {
                        std::fprintf(stderr, "table_for16 entry %d differs\n", u);
                        std::abort();
                    }
                }
                if (lg < 0 || !seq_entries(t, lg, k, se[k])) return kErrFse;
                T.t[k] = se[k];
                T.log[k] = lg;
            }
            uint64_t sll = 0, sml = 0;
            st = decode_sequences(f, B, T, seq.data() + B.seq_out, &sll, &sml, B.rep_end);
            if (st) return st;
            if (B.lit_size + sml > kBlockMax) return kErrBlock;
            B.regen = B.lit_size + sml;
        } else {
            B.regen = B.lit_size;
        }
    }
    // layout: output positions and starting histories
    uint32_t cur[3] = {1, 4, 8};
    uint64_t pos = 0;
    for (uint32_t b = 0; b < info.nblocks; ++b) {
        Block& B = blocks[b];
        B.out = pos;
        pos += B.regen;
        uint32_t nx[3];
        for (int k = 0; k < 3; ++k) {
            B.rep_start[k] = cur[k];
            const uint64_t v = rep_resolve(B.rep_end[k], cur);
            nx[k] = v < (1ull << 31) ? (uint32_t)v : 0;
        }
        for (int k = 0; k < 3; ++k) cur[k] = nx[k];
    }
    if (pos != content) return kErrContentSize;
    out->assign(content, 0);
    uint8_t* o = out->data();
    for (uint32_t b = 0; b < info.nblocks; ++b) {
        const Block& B = blocks[b];
        uint64_t q = B.out;
        if (B.type == 0) {
            std::memcpy(o + q, f + B.src, B.regen);
            continue;
        }
        if (B.type == 1) {
            std::memset(o + q, f[B.src], B.regen);
            continue;
        }
        auto litb = [&](uint64_t i) -> uint8_t {
            return B.lit_type == 0 ? f[B.lit_src + i] : B.lit_type == 1 ? f[B.lit_src] : lit[B.lit_out + i];
        };
        uint64_t lp = 0;
        for (uint32_t i = 0; i < B.nseq; ++i) {
            const uint64_t s = seq[B.seq_out + i];
            const uint32_t ll = seq_ll(s), ml = seq_ml(s);
            const uint64_t off = rep_resolve(seq_rep(s), B.rep_start);
            for (uint32_t j = 0; j < ll; ++j) o[q + j] = litb(lp + j);
            lp += ll;
            q += ll;
            if (off == 0 || off > q) return kErrOffset;
            for (uint32_t j = 0; j < ml; ++j) o[q + j] = o[q + j - off];
            q += ml;
        }
        for (; lp < B.lit_size; ++lp) o[q++] = litb(lp);
    }
    return kOk;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s decode|fuzz CASES [N SEED]\n", argv[0]);
        return 2;
    }
    std::vector<Case> cases;
    if (!read_cases(argv[2], &cases)) {
        std::fprintf(stderr, "cannot read %s\n", argv[2]);
        return 2;
    }
    if (!std::strcmp(argv[1], "decode")) {
        int bad = 0;
        for (size_t i = 0; i < cases.size(); ++i) {
            std::vector<uint8_t> out;
            const uint32_t st = decode(cases[i].frame, cases[i].content.size(), &out);
            const bool ok = st == 0 && out == cases[i].content;
            std::printf("case %zu %s status %u\n", i, ok ? "ok" : "FAIL", st);
            bad += !ok;
        }
        return bad ? 1 : 0;
    }
    if (!std::strcmp(argv[1], "fuzz") && argc >= 5) {
        const int n = std::atoi(argv[3]);
        std::mt19937_64 rng(std::strtoull(argv[4], nullptr, 0));
        uint64_t statuses[16] = {0};
        for (size_t i = 0; i < cases.size(); ++i) {
            for (int v = 0; v < n; ++v) {
                std::vector<uint8_t> fr = cases[i].frame;
                if (fr.empty()) continue;
                const int kind = (int)(rng() % 5);
                if (kind == 0) {  // flip a few bytes
                    for (int k = 0, m = 1 + (int)(rng() % 8); k < m; ++k) fr[rng() % fr.size()] ^= (uint8_t)(1 + rng() % 255);
                } else if (kind == 1) {  // truncate
                    fr.resize(rng() % fr.size());
                } else if (kind == 2) {  // a zeroed or 0xff run
                    const size_t a = rng() % fr.size(), len = 1 + rng() % 64;
                    const uint8_t v8 = (rng() & 1) ? 0xff : 0x00;
                    for (size_t k = a; k < fr.size() && k < a + len; ++k) fr[k] = v8;
                } else if (kind == 3) {  // a byte in the headers (first 32 bytes)
                    fr[rng() % std::min<size_t>(32, fr.size())] = (uint8_t)rng();
                } else {  // random bytes appended or a slice repeated
                    const size_t a = rng() % fr.size(), len = 1 + rng() % 32;
                    std::vector<uint8_t> slice(fr.begin() + a, fr.begin() + std::min(fr.size(), a + len));
                    fr.insert(fr.begin() + rng() % fr.size(), slice.begin(), slice.end());
                }
                std::vector<uint8_t> out;
                const uint32_t st = decode(fr, cases[i].content.size(), &out);
                statuses[st < 16 ? st : 15]++;
            }
        }
        for (int s = 0; s < 16; ++s)
            if (statuses[s]) std::printf("status %d: %llu\n", s, (unsigned long long)statuses[s]);
        return 0;
    }
    std::fprintf(stderr, "unknown mode\n");
    return 2;
}
