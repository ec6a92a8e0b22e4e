// Host side of the GPU zstd frame decoder (kernels in fw_zstd.hip): scratch
// for a bounded number of frames in flight, queued on a caller's stream.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

namespace fw::zs {

// One frame of a call: its bytes on the device, the decoded size the caller
// expects, and where the decoded bytes go (decoded bytes [0, split) to dst,
// the rest to dst_tail; with unshuffle the BF16 byte shuffle is undone first).
struct FrameJob {
    const uint8_t* src = nullptr;
    uint64_t size = 0;
    uint64_t content = 0;
    uint8_t* dst = nullptr;
    uint8_t* dst_tail = nullptr;
    uint64_t split = 0;
    bool unshuffle = false;
};

class Decoder {
   public:
    // Scratch for `max_frames` frames of at most `max_content` decoded bytes
    // each; calls with more frames run in chunks of that many. Throws
    // std::runtime_error on bad limits or a failed allocation.
    Decoder(int device, size_t max_frames, uint64_t max_content);
    ~Decoder();
    Decoder(const Decoder&) = delete;
    Decoder& operator=(const Decoder&) = delete;

    // Queue the decode of `jobs` on stream s after this decoder's previous
    // call (whatever stream that used); returns false with *why on an invalid
    // job (nothing queued). Per-frame statuses stay on the device until
    // statuses() is called.
    bool queue(const std::vector<FrameJob>& jobs, hipStream_t s, std::string* why);
    // Wait for the last call and copy its per-frame statuses (Status codes)
    // and, for failed frames, the block index where the failure was found.
    void statuses(std::vector<uint32_t>* status, std::vector<uint32_t>* block);

    // The host staging of the synchronous entry point: a pinned buffer of at
    // least `bytes` and a device buffer of the same size (kept between calls).
    uint8_t* pinned(size_t bytes);
    uint8_t* device_source(size_t bytes);

    int device() const { return device_; }
    uint64_t max_content() const { return max_content_; }
    size_t max_frames() const { return max_frames_; }
    hipEvent_t last() const { return last_; }

   private:
    int device_ = 0;
    size_t max_frames_ = 0;
    uint64_t max_content_ = 0;
    uint32_t max_blocks_ = 0;
    uint64_t lit_cap_ = 0, seq_cap_ = 0, out_cap_ = 0;
    void* blocks_ = nullptr;
    uint8_t* lit_ = nullptr;
    uint64_t* seq_ = nullptr;
    uint8_t* out_ = nullptr;
    void* work_ = nullptr;         // four work lists of max_frames * max_blocks entries
    uint32_t* counters_ = nullptr;  // the work lists' lengths
    void* frames_ = nullptr;        // device frame records of the last call
    void* frames_host_ = nullptr;   // pinned staging of the frame records
    hipEvent_t copied_ = nullptr;   // the last upload of the records has run
    size_t frames_cap_ = 0, frames_n_ = 0;
    uint8_t* pinned_ = nullptr;
    size_t pinned_bytes_ = 0;
    uint8_t* src_ = nullptr;
    size_t src_bytes_ = 0;
    hipEvent_t last_ = nullptr;
    int grid_ = 0;  // workgroups of the per-block passes
    // sequence-pass table entries: 0 chosen per call, 1 four bytes, 2 two
    // bytes (environment FIREWING_ZSTD_SEQ_TABLES = wide | narrow at creation;
    // both decode alike, the choice is for speed)
    int seq_tables_ = 0;
};

}  // namespace fw::zs
