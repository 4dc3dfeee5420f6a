// gguf.h - GGUF v2/v3 reader for jepa model files (the role ggml's gguf.h plays in the reference,
// src/jepa-gguf.cpp:100-229 / 802-810). Every length and offset is checked against the file, so a
// truncated or hostile file is an error with a message, not an out-of-bounds read.
#pragma once
#include <cstdint>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

namespace gguf {

enum vtype : uint32_t {
    U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, BOOL = 7, STR = 8, ARR = 9,
    U64 = 10, I64 = 11, F64 = 12,
};

struct value {
    uint32_t type = 0;
    int64_t  i = 0;          // integer / bool scalars (and the integer value of floats)
    double   f = 0;          // float scalars (and the float value of integers)
    std::string s;           // STR
    uint32_t arr_type = 0;   // ARR element type
    std::vector<int64_t> ai; // integer arrays
    std::vector<double>  af; // float arrays (also filled for integer arrays)
    std::vector<std::string> as; // string arrays
    std::string render() const;
};

struct tensor_info {
    std::string name;
    int     type = 0;
    int     n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;     // absolute offset in the file
    uint64_t nbytes = 0;
};

struct file {
    std::string path;
    std::vector<std::pair<std::string, value>> kv;   // in file order
    std::vector<std::pair<uint64_t, uint64_t>> kv_span;   // [begin, end) byte range of each kv pair in the file
    std::vector<tensor_info> tensors;
    uint64_t file_size = 0;
    uint64_t data_offset = 0;                        // start of the tensor data section

    const value * find(const std::string & key) const;
    const tensor_info * tensor(const std::string & name) const;
};

// Parse header, metadata and tensor infos (no tensor data). Returns false with a message.
bool open(const std::string & path, file & out, std::string & err);

}  // namespace gguf
