// SafeTensors container indexing and the MLX affine-quantized convention
// (host): exact per-tensor byte ranges of a .safetensors file, restating the
// reference's indexer (crates/dyninfer-checkpoint-safetensors/src/container.rs)
// under its default inspection limits (crates/dyninfer-checkpoint/src/limits.rs),
// and the pairing and validation of an MLX weight's three components
// (crates/dyninfer-checkpoint-safetensors/src/mlx.rs:17-261).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace dmx {

struct StTensor {
    std::string name;
    std::string dtype;            // SafeTensors dtype string ("U32", "BF16", ...)
    uint32_t elem = 0;            // bytes per element
    std::vector<uint64_t> shape;  // row-major
    uint64_t offset = 0;          // absolute byte offset of the data in the file
    uint64_t nbytes = 0;          // exact byte length
};

struct StIndex {
    const uint8_t* base = nullptr;  // the file's bytes (mapped or caller-owned)
    uint64_t len = 0;
    void* map = nullptr;            // non-null when this index mapped the file itself
    uint64_t data_base = 0;         // 8 + header length
    std::string metadata_json;      // header __metadata__ plus config.json's mapped keys, one JSON object
    // MLX quantization metadata (mlx.rs:63-64): present only as JSON numbers,
    // from __metadata__ or from config.json's quantization(_config) object
    bool has_bits = false, has_group = false, format_mlx = false;
    uint64_t bits = 0, group = 0;
    std::vector<StTensor> tensors;  // sorted by name, as the reference's entries
};

// Parses base[0, len) into idx.  Returns "" or an error message.
std::string st_index(const uint8_t* base, uint64_t len, StIndex& idx);

// Adds the keys load_hf_config_metadata (config_json.rs:10-146) maps from a
// sibling config.json that this convention reads (quantization bits and group
// size), where the header did not set them.  Malformed text is ignored, as
// the reference ignores an unreadable config.json.
void st_merge_config(StIndex& idx, const std::string& config_text);

// The MLX affine weight `weight_key` (a ".weight" tensor) with its ".scales"
// and ".biases" components, validated as decode_affine_weight (mlx.rs:152-261)
// and the convention's pairing rules (:63-136).  On success fills the three
// tensors, the logical shape [N, K] and the group size and returns "".
std::string st_mlx_weight(const StIndex& idx, const std::string& weight_key, const StTensor** packed,
                          const StTensor** scales, const StTensor** biases, uint64_t* n, uint64_t* k,
                          uint64_t* group);

const StTensor* st_find(const StIndex& idx, const std::string& name);

}  // namespace dmx
