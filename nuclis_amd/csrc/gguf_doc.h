// Parsed GGUF directory shared by gguf.cpp (parser and accessors) and
// api.hip (device upload). Host only.
#pragma once
#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace nuq {

// gguf.Value with gguf.Array's fields (inference/src/formats/gguf.zig:49-57, 105-112)
struct GgufValue {
    uint32_t kind = 0, type = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string str;
    uint32_t element_type = 0;
    uint64_t count = 0, file_offset = 0;
    bool retained = false;
    std::vector<GgufValue> values;
};

struct GgufMetadata {
    std::string key;
    GgufValue value;
};

struct GgufTensor {
    std::string name;
    uint32_t rank = 0, encoding = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint64_t offset = 0, bytes = 0, elements = 0;
};

}  // namespace nuq

struct nuq_gguf {
    const uint8_t *bytes = nullptr;  // the file image (borrowed, or the mapping)
    uint64_t avail = 0;              // bytes present at `bytes`
    uint64_t file_bytes = 0;
    void *map = nullptr;  // owned mapping (nuq_gguf_open)
    uint64_t map_len = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t directory_bytes = 0, data_offset = 0;
    std::vector<nuq::GgufMetadata> metadata;
    std::vector<nuq::GgufTensor> tensors;
    std::unordered_map<std::string_view, uint64_t> tensor_index;
};
