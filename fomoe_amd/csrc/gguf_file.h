// gguf_file.h — host-side GGUF reader behind the gpu_gguf_* entry points.
//
// The on-disk format (reference include/gguf.h:8-56, src/gguf.c:10-250):
//   u32 magic "GGUF", u32 version (2..3), i64 n_tensors, i64 n_kv,
//   n_kv x {string key, i32 type, value}, n_tensors x {string name, u32 n_dims,
//   i64 dims[n_dims], i32 ggml type, u64 offset}, then the tensor data from the
//   first multiple of general.alignment (default 32) past the header; strings
//   are u64 length + bytes. A model split as xxx-00001-of-0000N.gguf is read as
//   one: every split's tensors are appended in split order and its keys are
//   added when not yet present.
#pragma once

#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace fo {

struct GgufValue {
    int type = -1;              // gguf value type
    uint64_t u = 0;             // unsigned / bool
    int64_t i = 0;              // signed
    double f = 0.0;             // float32 / float64
    std::string s;              // string
    int arr_type = -1;          // array element type
    uint64_t arr_n = 0;
    std::vector<uint8_t> arr;   // raw elements of a scalar array
    std::vector<std::string> arr_str;
};

struct GgufTensor {
    std::string name;
    uint32_t n_dims = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    int type = -1;
    uint64_t offset = 0;        // within its split's data section
    uint64_t size = 0;          // bytes (0 for a type without a known block size)
    int split = 0;
};

struct GgufFile {
    uint32_t version = 0;
    uint64_t alignment = 32;
    std::vector<std::string> paths;         // one per split that was read
    std::vector<uint64_t> data_offset;      // absolute start of each split's data
    std::vector<uint64_t> file_size;
    std::vector<std::string> keys;
    std::vector<GgufValue> values;
    std::vector<GgufTensor> tensors;
    std::unordered_map<std::string, int64_t> key_index, tensor_index;

    // Parse `path` (and its splits). Returns false with `err` set on a file
    // that is unreadable or malformed.
    bool open(const char *path, std::string &err);
    int64_t find_key(const char *key) const;
    int64_t find_tensor(const char *name) const;
};

// Bytes of n elements of ggml type t: whole blocks only (n / block * block
// bytes, as reference src/gguf.c:53-58), 0 for a type without a known size.
uint64_t gguf_type_bytes(int t, uint64_t n);

}  // namespace fo
