// tc_gguf.cpp -- GGUF v3 tensor reader (C-ABI in include/tc_gguf.h).
//
// The file is mapped read-only once; the header, metadata and tensor records
// are parsed from the mapping through a cursor that checks every length
// against the file size, so a truncated or corrupt file is refused instead of
// read past its end. Tensor bytes are never copied on the host: callers get a
// pointer into the mapping or a device copy.
//
// Format (GGUF v3, little-endian): magic "GGUF", u32 version, u64 tensor
// count, u64 metadata count; metadata entries (string key, u32 value type,
// value); tensor records (string name, u32 n_dims, u64 dims[n_dims], u32 GGML
// type, u64 offset); padding to the alignment; the tensor data section.
// Strings are u64 length + bytes. The reference reads the same layout in
// src/cpp/core/GGUFLoader.cpp:242-739.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "tc_gguf.h"
#include "tc_qmatmul.h"

namespace tc {
void set_error(const std::string &msg);
}

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint32_t kMaxDims = 4;          // GGML_MAX_DIMS

enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12,
};

uint32_t scalar_bytes(uint32_t t) {
    switch (t) {
        case V_U8: case V_I8: case V_BOOL: return 1;
        case V_U16: case V_I16: return 2;
        case V_U32: case V_I32: case V_F32: return 4;
        case V_U64: case V_I64: case V_F64: return 8;
        default: return 0;
    }
}

struct Record {
    std::string name;
    uint32_t type = 0, n_dims = 0;
    uint64_t dims[kMaxDims] = {1, 1, 1, 1};
    uint64_t offset = 0, bytes = 0;
};

// Bounds-checked reader over [p, p+n).
struct Cursor {
    const uint8_t *p;
    uint64_t n, pos = 0;
    bool ok = true;
    bool take(void *dst, uint64_t k) {
        if (!ok || k > n - pos) return ok = false;
        if (dst) std::memcpy(dst, p + pos, k);
        pos += k;
        return true;
    }
    template <class T>
    T get() {
        T v{};
        take(&v, sizeof v);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (!ok || len > n - pos) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p + pos), len);
        pos += len;
        return s;
    }
};

// One scalar rendered as the reference's metadata map holds it
// (std::to_string of the value; bools as "true"/"false").
std::string render(Cursor &c, uint32_t t) {
    switch (t) {
        case V_U8: return std::to_string(unsigned(c.get<uint8_t>()));
        case V_I8: return std::to_string(int(c.get<int8_t>()));
        case V_U16: return std::to_string(unsigned(c.get<uint16_t>()));
        case V_I16: return std::to_string(int(c.get<int16_t>()));
        case V_U32: return std::to_string(c.get<uint32_t>());
        case V_I32: return std::to_string(c.get<int32_t>());
        case V_F32: return std::to_string(c.get<float>());
        case V_BOOL: return c.get<uint8_t>() ? "true" : "false";
        case V_STR: return c.str();
        case V_U64: return std::to_string(c.get<uint64_t>());
        case V_I64: return std::to_string(c.get<int64_t>());
        case V_F64: return std::to_string(c.get<double>());
        default: c.ok = false; return {};
    }
}

bool ends_with(const std::string &s, const char *suf) {
    const size_t k = std::strlen(suf);
    return s.size() >= k && s.compare(s.size() - k, k, suf) == 0;
}

}  // namespace

struct tc_gguf {
    int fd = -1;
    void *map = nullptr;
    uint64_t map_len = 0;
    bool data = false;  // tensor data may be handed out (full open)
    uint32_t version = 0;
    uint64_t n_tensors = 0, n_kv = 0, data_off = 0;
    std::vector<Record> recs;
    std::unordered_map<std::string, uint64_t> index;
    std::unordered_map<std::string, std::string> meta;

    ~tc_gguf() {
        if (map) munmap(map, map_len);
        if (fd >= 0) close(fd);
    }
    const uint8_t *base() const { return static_cast<const uint8_t *>(map); }
};

namespace {

bool refuse(const std::string &m) {
    tc::set_error("gguf: " + m);
    return false;
}

// Metadata entries (GGUFLoader.cpp:287-593 for the value rendering).
bool parse_metadata(tc_gguf *g, Cursor &c) {
    for (uint64_t i = 0; i < g->n_kv; ++i) {
        const std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (!c.ok) return refuse("truncated metadata entry " + std::to_string(i));
        if (t != V_ARR) {
            std::string v = render(c, t);
            if (!c.ok) return refuse("bad value (type " + std::to_string(t) + ") for key '" + key + "'");
            g->meta[key] = std::move(v);
            continue;
        }
        const uint32_t et = c.get<uint32_t>();
        const uint64_t len = c.get<uint64_t>();
        if (!c.ok) return refuse("truncated array header for key '" + key + "'");
        if (et == V_ARR) return refuse("nested array for key '" + key + "'");
        const bool prism = key.rfind("prism.hadamard.", 0) == 0;  // captured elsewhere by the reference
        const bool joined = ends_with(key, ".rope.dimension_sections") && (et == V_U32 || et == V_I32);
        std::string first;
        for (uint64_t j = 0; j < len; ++j) {
            if (et == V_STR) {
                c.str();
            } else {
                const uint32_t b = scalar_bytes(et);
                if (b == 0) return refuse("bad array element type for key '" + key + "'");
                if (j == 0 || joined) {
                    std::string v = render(c, et);
                    first = j == 0 ? v : first + "," + v;
                } else if (len - j > (c.n - c.pos) / b) {
                    c.ok = false;
                } else {
                    c.take(nullptr, (len - j) * b);  // skip the rest at once
                    break;
                }
            }
            if (!c.ok) return refuse("truncated array for key '" + key + "'");
        }
        if (!prism && et != V_STR && len > 0) g->meta[key] = first;
    }
    return true;
}

bool parse_records(tc_gguf *g, Cursor &c) {
    // a record takes at least 28 bytes (empty name, 1 dimension)
    if (g->n_tensors > (c.n - c.pos) / 28) return refuse(std::to_string(g->n_tensors) + " tensor records cannot fit the file");
    g->recs.resize(g->n_tensors);
    for (uint64_t i = 0; i < g->n_tensors; ++i) {
        Record &r = g->recs[i];
        r.name = c.str();
        r.n_dims = c.get<uint32_t>();
        if (!c.ok) return refuse("truncated tensor record " + std::to_string(i));
        if (r.n_dims > kMaxDims)
            return refuse("tensor '" + r.name + "' has " + std::to_string(r.n_dims) + " dimensions");
        for (uint32_t d = 0; d < r.n_dims; ++d) r.dims[d] = c.get<uint64_t>();
        r.type = c.get<uint32_t>();
        r.offset = c.get<uint64_t>();
        if (!c.ok) return refuse("truncated tensor record '" + r.name + "'");
        const uint32_t bs = tc_gguf_block_size(r.type), ts = tc_gguf_type_size(r.type);
        uint64_t n = 1;
        for (uint32_t d = 0; d < r.n_dims; ++d) {
            if (r.dims[d] != 0 && n > UINT64_MAX / r.dims[d]) return refuse("tensor '" + r.name + "' is too large");
            n *= r.dims[d];
        }
        const uint64_t blocks = (n + bs - 1) / bs;
        if (ts != 0 && blocks > UINT64_MAX / ts) return refuse("tensor '" + r.name + "' is too large");
        r.bytes = blocks * ts;
        if (!g->index.emplace(r.name, i).second) return refuse("duplicate tensor name '" + r.name + "'");
    }
    return true;
}

tc_gguf *open_impl(const char *path, bool with_data) {
    if (!path) {
        refuse("null path");
        return nullptr;
    }
    tc_gguf *g = new tc_gguf;
    auto bail = [&](const std::string &m) -> tc_gguf * {
        refuse(m);
        delete g;
        return nullptr;
    };
    g->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) return bail(std::string("cannot open ") + path + ": " + std::strerror(errno));
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 24) return bail(std::string(path) + ": not a GGUF file (too short)");
    g->map_len = uint64_t(st.st_size);
    g->map = mmap(nullptr, g->map_len, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->map == MAP_FAILED) {
        g->map = nullptr;
        return bail(std::string("mmap failed: ") + std::strerror(errno));
    }
    Cursor c{g->base(), g->map_len};
    const uint32_t magic = c.get<uint32_t>();
    g->version = c.get<uint32_t>();
    g->n_tensors = c.get<uint64_t>();
    g->n_kv = c.get<uint64_t>();
    if (magic != kMagic) return bail(std::string(path) + ": bad magic");
    // The reference accepts version 3 only (GGUFLoader.cpp:251-255).
    if (g->version != 3) return bail("unsupported GGUF version " + std::to_string(g->version));
    if (!parse_metadata(g, c) || !parse_records(g, c)) {
        delete g;
        return nullptr;
    }
    // Data section alignment: general.alignment when the file sets it (GGUF
    // v3), else 32 as the reference always assumes (GGUFLoader.cpp:735-737).
    uint64_t align = 32;
    auto it = g->meta.find("general.alignment");
    if (it != g->meta.end()) {
        const uint64_t a = std::strtoull(it->second.c_str(), nullptr, 10);
        if (a == 0 || (a & (a - 1)) != 0) return bail("general.alignment " + it->second + " is not a power of two");
        align = a;
    }
    g->data_off = (c.pos + align - 1) / align * align;
    for (const Record &r : g->recs) {
        if (r.offset > g->map_len || r.bytes > g->map_len - r.offset ||
            g->data_off > g->map_len - r.offset - r.bytes)
            return bail("tensor '" + r.name + "' extends past the end of the file");
    }
    g->data = with_data;
    if (with_data) (void)madvise(g->map, g->map_len, MADV_SEQUENTIAL);
    return g;
}

}  // namespace

extern "C" {

uint32_t tc_gguf_type_size(uint32_t type) {
    switch (type) {
        case 0: return 4;    // F32
        case 1: return 2;    // F16
        case 2: return 18;   // Q4_0
        case 3: return 20;   // Q4_1
        case 6: return 22;   // Q5_0
        case 7: return 24;   // Q5_1
        case 8: return 34;   // Q8_0
        case 9: return 36;   // Q8_1
        case 10: return 84;  // Q2_K
        case 11: return 110; // Q3_K
        case 12: return 144; // Q4_K
        case 13: return 176; // Q5_K
        case 14: return 210; // Q6_K
        case 15: return 292; // Q8_K
        case 16: return 66;  // IQ2_XXS
        case 17: return 74;  // IQ2_XS
        case 18: return 98;  // IQ3_XXS
        case 19: return 50;  // IQ1_S (2 + 32 + 16; the reference's table says 34)
        case 20: return 18;  // IQ4_NL
        case 21: return 110; // IQ3_S
        case 22: return 82;  // IQ2_S
        case 23: return 136; // IQ4_XS
        case 24: return 1;   // I8
        case 25: return 2;   // I16
        case 26: return 4;   // I32
        case 30: return 2;   // BF16
        default: return 0;
    }
}

uint32_t tc_gguf_block_size(uint32_t type) {
    switch (type) {
        case 2: case 3: case 6: case 7: case 8: case 9: case 20: return 32;
        case 10: case 11: case 12: case 13: case 14: case 15: case 16: case 17: case 18: case 19: case 21: case 22:
        case 23: return 256;
        default: return 1;
    }
}

tc_gguf *tc_gguf_open(const char *path) { return open_impl(path, true); }
tc_gguf *tc_gguf_open_metadata(const char *path) { return open_impl(path, false); }
void tc_gguf_close(tc_gguf *g) { delete g; }

uint32_t tc_gguf_version(const tc_gguf *g) { return g ? g->version : 0; }
uint64_t tc_gguf_tensor_count(const tc_gguf *g) { return g ? g->n_tensors : 0; }
uint64_t tc_gguf_metadata_count(const tc_gguf *g) { return g ? g->n_kv : 0; }
uint64_t tc_gguf_data_offset(const tc_gguf *g) { return g ? g->data_off : 0; }

int64_t tc_gguf_find_tensor(const tc_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->index.find(name);
    return it == g->index.end() ? -1 : int64_t(it->second);
}

int tc_gguf_tensor_info(const tc_gguf *g, uint64_t i, const char **name, uint32_t *type, uint32_t *n_dims,
                        uint64_t *dims, uint64_t *offset, uint64_t *bytes) {
    if (!g || i >= g->recs.size()) {
        tc::set_error("gguf: no tensor record " + std::to_string(i));
        return TC_E_ARG;
    }
    const Record &r = g->recs[i];
    if (name) *name = r.name.c_str();
    if (type) *type = r.type;
    if (n_dims) *n_dims = r.n_dims;
    if (dims)
        for (uint32_t d = 0; d < kMaxDims; ++d) dims[d] = r.dims[d];
    if (offset) *offset = r.offset;
    if (bytes) *bytes = r.bytes;
    return TC_OK;
}

const void *tc_gguf_tensor_data(const tc_gguf *g, uint64_t i) {
    if (!g || !g->data || i >= g->recs.size()) return nullptr;
    return g->base() + g->data_off + g->recs[i].offset;
}

int tc_gguf_upload(const tc_gguf *g, uint64_t i, void *dst, uint64_t dst_bytes, void *stream) {
    const void *src = tc_gguf_tensor_data(g, i);
    if (!src || !dst) {
        tc::set_error("gguf: upload needs a fully opened file, a valid tensor and a destination");
        return TC_E_ARG;
    }
    const Record &r = g->recs[i];
    if (r.bytes == 0 || dst_bytes < r.bytes) {
        tc::set_error("gguf: tensor '" + r.name + "' needs " + std::to_string(r.bytes) + " bytes (type " +
                      std::to_string(r.type) + "), destination has " + std::to_string(dst_bytes));
        return TC_E_ARG;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(dst, src, r.bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        tc::set_error(std::string("gguf: upload of '") + r.name + "' failed: " + hipGetErrorString(e));
        return TC_E_LAUNCH;
    }
    return TC_OK;
}

const char *tc_gguf_meta(const tc_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : it->second.c_str();
}

}  // extern "C"
