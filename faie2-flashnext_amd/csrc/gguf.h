// GGUF reader (memory-mapped, read-only) for fn_load: the file's key/value metadata and tensor table, and a pointer to
// each tensor's bytes inside the mapping.  The format is GGUF v2/v3 (magic "GGUF", little-endian): header, n_kv
// key/value pairs, n_tensors tensor infos (name, dims, ggml type, offset), then the data section aligned to
// general.alignment (32 by default).  The reference reads the same files through a Win32 mapping
// (engine/faie2fn.cu:120-263); this one maps with POSIX mmap.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace fn {

struct GTensor {
    uint32_t type = 0;              // ggml type id
    int nd = 0;
    uint64_t ne[4] = {1, 1, 1, 1};  // ne[0] = values per row (fastest), then rows, ...
    uint64_t offset = 0;            // inside the data section
    uint64_t nbytes = 0;
    const uint8_t *data = nullptr;  // inside the mapping
};

struct Gguf {
    std::string path;
    const uint8_t *base = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    std::map<std::string, GTensor> tensors;
    std::map<std::string, double> nums;                   // scalar numbers (ints, floats, bools)
    std::map<std::string, std::string> strs;              // scalar strings
    std::map<std::string, std::vector<int64_t>> iarrays;  // integer arrays (and float arrays, truncated: not used)

    Gguf() = default;
    Gguf(const Gguf &) = delete;
    Gguf &operator=(const Gguf &) = delete;
    ~Gguf();

    const GTensor *find(const std::string &name) const {
        auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
    double num(const std::string &key, double dflt) const {
        auto it = nums.find(key);
        return it == nums.end() ? dflt : it->second;
    }
};

// values per block and bytes per block of a ggml type (the block formats of GGUF); false for a type not known here
bool ggml_type_block(uint32_t type, int &values, int &bytes);

// map and parse a GGUF file; -1 with fn_error() set on any malformed or truncated header or tensor
int gguf_open(Gguf &g, const char *path);

}  // namespace fn
