// safetensors checkpoints for the resident banks: header parsing and
// validation, shard resolution through model.safetensors.index.json, and the
// plan of one layer's seven tensors. Host code only; the streaming copy into
// HBM is in fw_moe.hip.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace fw::st {

struct TensorInfo {
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t offset = 0;  // absolute byte offset of the payload in the file
    uint64_t bytes = 0;
};

struct Shard {
    std::string path;
    uint64_t file_bytes = 0;
    std::map<std::string, TensorInfo> tensors;
};

// Parse and validate one .safetensors file's header (the format's rules:
// little-endian u64 header length in (0, 16 MiB], a JSON object of
// name -> {dtype, shape, data_offsets} plus an optional __metadata__ object,
// every payload inside the file, of exactly dtype size x shape bytes, no two
// payloads overlapping). Throws std::runtime_error naming the file and fault.
Shard read_shard(const std::string& path);

// A checkpoint: one .safetensors file, or a model.safetensors.index.json whose
// weight_map names each tensor's shard (a plain file name in the index's
// directory). Shards are parsed when first needed.
class Checkpoint {
   public:
    explicit Checkpoint(const std::string& path);
    // the tensor, which must be BF16 of exactly `shape`; throws otherwise
    const TensorInfo& bf16(const std::string& name, const std::vector<uint64_t>& shape, std::string* file);

   private:
    const Shard& shard(const std::string& file);
    std::string dir_;
    std::string single_;                          // set for a single-file checkpoint
    std::map<std::string, std::string> weight_map_;  // tensor -> shard file name
    std::map<std::string, std::unique_ptr<Shard>> shards_;
};

struct Span {
    std::string file;
    uint64_t offset = 0;
    uint64_t bytes = 0;
};

// The seven tensors of one MoE layer under `prefix` (for example
// "model.language_model.layers.0"), in the resident-bank tensor order
// 1 router (mlp.gate.weight [E, H]), 2 gate_up (mlp.experts.gate_up_proj
// [E, 2I, H]), 3 down (mlp.experts.down_proj [E, H, I]), 4 shared gate
// (mlp.shared_expert.gate_proj.weight [Is, H]), 5 shared up
// (mlp.shared_expert.up_proj.weight [Is, H]), 6 shared down
// (mlp.shared_expert.down_proj.weight [H, Is]), 7 shared_expert_gate
// (mlp.shared_expert_gate.weight [1, H]).
std::vector<Span> layer_plan(Checkpoint& ckpt, const std::string& prefix, uint64_t hidden, uint64_t intermediate,
                             uint64_t experts, uint64_t shared_intermediate);

}  // namespace fw::st
