// st_format.hpp -- host-side checkpoint formats (st_format.cpp) used by the
// device loader (loader.cpp).  Plain C++, no HIP.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "../../include/atlas_engine.h"
#include "../../include/atlas_loader.h"
#include "errors.hpp"

#define LTRY(expr)                \
    do {                          \
        const int rc_ = (expr);   \
        if (rc_) return rc_;      \
    } while (0)

// One tensor of a safetensors header (TensorDesc, lib.rs:2063-2070).
struct StTensor {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    uint64_t start = 0, end = 0;
};

// SafetensorsFile: the header's tensors and the data section.
struct atlas_st {
    std::vector<StTensor> tensors;
    const uint8_t* data = nullptr;      // the data section (after the header)
    size_t data_len = 0;
    void* map = nullptr;                // memory map of the file (open)
    size_t map_len = 0;
    std::vector<uint8_t> owned;         // copied bytes (from_bytes)
    ~atlas_st();
};

namespace atlas {

// SafetensorsFile::open over a memory map of the file.
int st_open(const char* path, std::unique_ptr<atlas_st>* out);
// The first tensor named `name`, or nullptr.
const StTensor* st_find(const atlas_st* st, const char* name);
// Bytes per element of F32 / BF16 / F16; 0 for any other dtype.
int elem_bytes(const std::string& dtype);
// A tensor's byte range, checked against the data section.
int st_range(const atlas_st* st, const StTensor& t, const uint8_t** p, size_t* n);
// The whole file as text.
bool read_text(const std::string& path, std::string* out, std::string* err);
// The shards a model.safetensors.index.json names, sorted and deduplicated.
std::vector<std::string> index_shards(const std::string& text);

}  // namespace atlas
