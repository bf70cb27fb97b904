// gguf_file.cpp — host-side GGUF parser (format summary in gguf_file.h).
//
// Behaviour follows reference src/gguf.c: versions 2 and 3, at most 4 dims,
// strings of at most 1 MiB, general.alignment (u32) overriding the default 32,
// tensor sizes in whole blocks (gguf.c:53-58), split files found from the
// "-NNNNN-of-MMMMM" part of the file name with missing splits skipped
// (gguf.c:255-449), first occurrence winning for a repeated key or tensor
// name (gguf.c:470-475, 523-528). Beyond the reference, counts and lengths
// are bounded by the file size before anything is allocated, so a corrupt
// header fails cleanly instead of allocating or reading past the end.
#include "gguf_file.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

namespace fo {

namespace {

struct TypeBytes { int block, bytes; };

// ggml block geometry (elements per block, bytes per block) of the types a
// GGUF expert model carries; reference src/gguf.c:19-35.
TypeBytes type_geometry(int t) {
    switch (t) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 36};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
        case 30: return {1, 2};     // BF16
        case 39: return {32, 17};   // MXFP4
        default: return {0, 0};
    }
}

// Size of one scalar of a gguf value type, 0 for string / array / unknown.
int scalar_bytes(int t) {
    switch (t) {
        case 0: case 1: case 7: return 1;      // u8, i8, bool
        case 2: case 3: return 2;              // u16, i16
        case 4: case 5: case 6: return 4;      // u32, i32, f32
        case 10: case 11: case 12: return 8;   // u64, i64, f64
        default: return 0;
    }
}

constexpr uint32_t kMagic = 0x46554747u;   // "GGUF"
constexpr uint64_t kMaxString = 1u << 20;
constexpr int kMaxSplits = 16;

class Reader {
  public:
    Reader(FILE *f, uint64_t size) : f_(f), size_(size) {}
    uint64_t pos() const { return pos_; }
    uint64_t left() const { return size_ - pos_; }
    bool bytes(void *dst, uint64_t n) {
        if (n > left() || fread(dst, 1, n, f_) != n) return false;
        pos_ += n;
        return true;
    }
    template <typename T>
    bool get(T &v) { return bytes(&v, sizeof v); }
    bool str(std::string &s) {
        uint64_t n;
        if (!get(n) || n > kMaxString || n > left()) return false;
        s.resize(n);
        return n == 0 || bytes(&s[0], n);
    }

  private:
    FILE *f_;
    uint64_t size_, pos_ = 0;
};

bool read_scalar(Reader &r, int t, GgufValue &v) {
    switch (t) {
        case 0: { uint8_t x; if (!r.get(x)) return false; v.u = x; v.i = x; return true; }
        case 1: { int8_t x; if (!r.get(x)) return false; v.i = x; v.u = (uint64_t)x; return true; }
        case 2: { uint16_t x; if (!r.get(x)) return false; v.u = x; v.i = x; return true; }
        case 3: { int16_t x; if (!r.get(x)) return false; v.i = x; v.u = (uint64_t)x; return true; }
        case 4: { uint32_t x; if (!r.get(x)) return false; v.u = x; v.i = x; return true; }
        case 5: { int32_t x; if (!r.get(x)) return false; v.i = x; v.u = (uint64_t)x; return true; }
        case 6: { float x; if (!r.get(x)) return false; v.f = x; return true; }
        case 7: { int8_t x; if (!r.get(x)) return false; v.u = x != 0; v.i = x != 0; return true; }
        case 10: { uint64_t x; if (!r.get(x)) return false; v.u = x; v.i = (int64_t)x; return true; }
        case 11: { int64_t x; if (!r.get(x)) return false; v.i = x; v.u = (uint64_t)x; return true; }
        case 12: { double x; if (!r.get(x)) return false; v.f = x; return true; }
        default: return false;
    }
}

bool read_value(Reader &r, GgufValue &v) {
    int32_t t;
    if (!r.get(t)) return false;
    v.type = t;
    if (t == 8) return r.str(v.s);
    if (t != 9) return read_scalar(r, t, v);
    int32_t at;
    uint64_t n;
    if (!r.get(at) || !r.get(n)) return false;
    v.arr_type = at;
    v.arr_n = n;
    if (at == 8) {
        if (n > r.left() / 8) return false;   // every string costs >= 8 bytes
        v.arr_str.resize(n);
        for (uint64_t i = 0; i < n; i++)
            if (!r.str(v.arr_str[i])) return false;
        return true;
    }
    const int eb = scalar_bytes(at);
    if (eb == 0 || n > r.left() / eb) return false;
    v.arr.resize(n * eb);
    return n == 0 || r.bytes(v.arr.data(), n * eb);
}

// One file of the model: header, keys, tensor directory.
bool parse_one(const std::string &path, GgufFile &out, std::vector<std::string> &keys,
               std::vector<GgufValue> &values, std::vector<GgufTensor> &tensors, uint64_t &data_off,
               uint64_t &fsize, std::string &err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) { err = "gguf: cannot open " + path; return false; }
    struct stat st;
    if (fstat(fileno(f), &st) != 0) { fclose(f); err = "gguf: cannot stat " + path; return false; }
    fsize = (uint64_t)st.st_size;
    Reader r(f, fsize);
    bool ok = false;
    uint32_t magic = 0, version = 0;
    int64_t n_tensors = 0, n_kv = 0;
    uint64_t alignment = 32;
    do {
        if (!r.get(magic) || magic != kMagic) { err = "gguf: bad magic in " + path; break; }
        if (!r.get(version) || version < 2 || version > 3) { err = "gguf: unsupported version in " + path; break; }
        if (!r.get(n_tensors) || !r.get(n_kv) || n_tensors < 0 || n_kv < 0 ||
            (uint64_t)n_kv > r.left() / 12 || (uint64_t)n_tensors > r.left() / 24) {
            err = "gguf: bad tensor / key counts in " + path;
            break;
        }
        keys.resize(n_kv);
        values.resize(n_kv);
        int64_t i = 0;
        for (; i < n_kv; i++) {
            if (!r.str(keys[i]) || !read_value(r, values[i])) break;
            if (keys[i] == "general.alignment" && values[i].type == 4) alignment = values[i].u;
        }
        if (i < n_kv) { err = "gguf: malformed key/value " + std::to_string(i) + " in " + path; break; }
        if (alignment == 0 || (alignment & (alignment - 1))) { err = "gguf: bad alignment in " + path; break; }
        tensors.resize(n_tensors);
        for (i = 0; i < n_tensors; i++) {
            GgufTensor &t = tensors[i];
            if (!r.str(t.name) || !r.get(t.n_dims) || t.n_dims > 4) break;
            uint64_t ne = 1;
            bool dims_ok = true;
            for (uint32_t d = 0; d < t.n_dims; d++) {
                if (!r.get(t.dims[d]) || t.dims[d] < 0) { dims_ok = false; break; }
                ne *= (uint64_t)t.dims[d];
            }
            int32_t ty;
            if (!dims_ok || !r.get(ty) || !r.get(t.offset)) break;
            t.type = ty;
            t.size = gguf_type_bytes(ty, ne);
        }
        if (i < n_tensors) { err = "gguf: malformed tensor entry " + std::to_string(i) + " in " + path; break; }
        data_off = (r.pos() + alignment - 1) & ~(alignment - 1);
        ok = true;
    } while (0);
    fclose(f);
    if (ok && out.paths.empty()) {
        out.version = version;
        out.alignment = alignment;
    }
    return ok;
}

// Position of the "-of-" of a split name: the last one in the file's base
// name (the reference takes the first in the whole path, gguf.c:255-262, which
// a directory such as /tmp/pytest-of-user/ would capture).
size_t split_mark(const std::string &p) {
    const size_t slash = p.rfind('/');
    const size_t at = p.rfind("-of-");
    return (at == std::string::npos || (slash != std::string::npos && at < slash)) ? std::string::npos : at;
}

// xxx-00001-of-00004.gguf -> number of splits (1 when the name has no such part).
int split_count(const std::string &p) {
    const size_t at = split_mark(p);
    if (at == std::string::npos) return 1;
    const int n = atoi(p.c_str() + at + 4);
    return (n > 1 && n <= kMaxSplits) ? n : 1;
}

std::string split_name(const std::string &p, int no, int total) {
    const size_t at = split_mark(p);
    size_t b = at;
    while (b > 0 && p[b - 1] >= '0' && p[b - 1] <= '9') b--;
    size_t e = at + 4;
    while (e < p.size() && p[e] >= '0' && p[e] <= '9') e++;
    char mid[32];
    snprintf(mid, sizeof mid, "%05d-of-%05d", no, total);
    return p.substr(0, b) + mid + p.substr(e);
}

}  // namespace

uint64_t gguf_type_bytes(int t, uint64_t n) {
    const TypeBytes g = type_geometry(t);
    return g.block ? n / g.block * g.bytes : 0;
}

bool GgufFile::open(const char *path, std::string &err) {
    if (!path) { err = "gguf: null path"; return false; }
    const std::string first(path);
    const int n_splits = split_count(first);
    for (int s = 1; s <= n_splits; s++) {
        const std::string p = s == 1 ? first : split_name(first, s, n_splits);
        std::vector<std::string> k;
        std::vector<GgufValue> v;
        std::vector<GgufTensor> t;
        uint64_t doff = 0, fsz = 0;
        std::string e;
        if (!parse_one(p, *this, k, v, t, doff, fsz, e)) {
            if (s == 1) { err = e; return false; }
            continue;   // a missing or unreadable later split is skipped
        }
        const int si = (int)paths.size();
        paths.push_back(p);
        data_offset.push_back(doff);
        file_size.push_back(fsz);
        for (size_t i = 0; i < k.size(); i++) {
            if (key_index.count(k[i])) continue;
            key_index.emplace(k[i], (int64_t)keys.size());
            keys.push_back(std::move(k[i]));
            values.push_back(std::move(v[i]));
        }
        for (auto &ti : t) {
            ti.split = si;
            tensor_index.emplace(ti.name, (int64_t)tensors.size());
            tensors.push_back(std::move(ti));
        }
    }
    return true;
}

int64_t GgufFile::find_key(const char *key) const {
    if (!key) return -1;
    auto it = key_index.find(key);
    return it == key_index.end() ? -1 : it->second;
}

int64_t GgufFile::find_tensor(const char *name) const {
    if (!name) return -1;
    auto it = tensor_index.find(name);
    return it == tensor_index.end() ? -1 : it->second;
}

}  // namespace fo
