// GGUF container indexing (host): exact per-tensor byte ranges of a GGUF file,
// restating the reference's indexer (crates/dyninfer-checkpoint-gguf/src/container.rs:179-340)
// with its default inspection limits (crates/dyninfer-checkpoint/src/limits.rs).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace dmx {

struct GgufTensor {
    std::string name;
    uint32_t type_code;
    std::vector<uint64_t> shape;  // row-major logical shape (GGUF stores it reversed)
    uint64_t offset;              // absolute byte offset of the data in the file
    uint64_t nbytes;              // exact byte length
};

struct GgufIndex {
    const uint8_t* base = nullptr;  // the file's bytes (mapped or caller-owned)
    uint64_t len = 0;
    void* map = nullptr;            // non-null when this index mapped the file itself
    uint32_t version = 0;
    uint64_t alignment = 32;
    std::string metadata_json;      // metadata as a JSON object (keys sorted)
    std::vector<GgufTensor> tensors;  // sorted by name, as the reference's entries
};

// Block geometry of a GGUF type code (types.rs:137-201): weights per block
// (1 for plain scalar types) and bytes per block; false for an unknown code.
bool gguf_type_geometry(uint32_t code, uint64_t* block, uint64_t* bytes);

// Well-formed UTF-8 (RFC 3629), the check Rust's String::from_utf8 makes.
bool valid_utf8(const uint8_t* s, uint64_t n);

// Parses base[0, len) into idx (tensors, metadata).  Returns "" or an error message.
std::string gguf_index(const uint8_t* base, uint64_t len, GgufIndex& idx);

}  // namespace dmx
