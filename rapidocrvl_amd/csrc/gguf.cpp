// gguf.cpp — the checkpoint container of the reference (internal/gguf/
// gguf.go) read natively: header parse and validation as gguf.Open does
// (gguf.go:111-251, 253-296, 586-667), tensor bytes by positioned reads.
// Host code only; pocr_model_load_gguf (pocr_runtime.hip) uploads the
// tensors it finds here into a device model.
//
// Layout (GGUF v3 subset written by convert.go:436-520): "GGUF", u32 version
// 3, u64 tensor count, u64 metadata count; metadata as (string key, u32 type,
// value) with types u32 (4), u64 (10), string (8); tensor infos as (string
// name, u32 ndim, u64 dims[ndim] in row-major order, u32 type, u64 offset);
// data from the header end aligned to 32 bytes.  Tensor types: F32 (0),
// Q8_ROW (1000), Q4_ROW (1001), Q6_ROW (1002), the Q*_ROW payload being f32
// scales[rows] followed by the packed rows.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/pocr_hip.h"

namespace pocr {
int fail(int code, const char *fmt, ...);
}
using pocr::fail;

namespace {

constexpr uint32_t kVersion = 3, kAlign = 32;
constexpr uint32_t kF32 = 0, kQ8 = 1000, kQ4 = 1001, kQ6 = 1002;
constexpr uint32_t kMetaU32 = 4, kMetaU64 = 10, kMetaString = 8;
constexpr uint64_t kMaxHeader = 256ull << 20, kMaxString = 16ull << 20;
constexpr uint64_t kMaxTensors = 1ull << 20, kMaxKV = 1ull << 20;
constexpr uint32_t kMaxDims = 8;

struct Tensor {
    std::string name;
    std::vector<int64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};
struct Meta {
    std::string key;
    uint32_t type = 0;
    uint64_t u = 0;
    std::string s;
};

// buffered sequential header reader counting the bytes consumed
struct Reader {
    int fd;
    std::vector<uint8_t> buf;
    size_t pos = 0, len = 0;
    uint64_t n = 0;  // header bytes consumed
    bool read(void *dst, size_t k) {
        uint8_t *d = static_cast<uint8_t *>(dst);
        while (k) {
            if (pos == len) {
                const ssize_t r = ::read(fd, buf.data(), buf.size());
                if (r <= 0) return false;
                pos = 0;
                len = (size_t)r;
            }
            const size_t c = std::min(k, len - pos);
            std::memcpy(d, buf.data() + pos, c);
            pos += c;
            d += c;
            k -= c;
            n += c;
        }
        return true;
    }
    bool u32(uint32_t &v) { return read(&v, 4); }  // little-endian host
    bool u64(uint64_t &v) { return read(&v, 8); }
};

bool printable(const std::string &s) {
    for (unsigned char c : s)
        if (c < 0x20 || c == 0x7f) return false;
    return true;
}

// checkedElemCount64 (gguf.go:652-667)
bool elem_count(const std::vector<int64_t> &dims, int64_t &n) {
    if (dims.size() > kMaxDims) return false;
    n = 1;
    for (int64_t d : dims) {
        if (d < 0) return false;
        if (d != 0 && n > INT64_MAX / d) return false;
        n *= d;
    }
    return true;
}

// TensorBytes (gguf.go:586-629): 0 for an invalid type or shape
int64_t tensor_bytes(const Tensor &t) {
    if (t.type == kF32) {
        int64_t n;
        if (!elem_count(t.dims, n) || n > INT64_MAX / 4) return 0;
        return n * 4;
    }
    if (t.type != kQ8 && t.type != kQ4 && t.type != kQ6) return 0;
    if (t.dims.size() != 2) return 0;
    const int64_t rows = t.dims[0], cols = t.dims[1];
    if (rows < 0 || cols < 0) return 0;
    int64_t per_row;
    if (t.type == kQ8) {
        if (cols > INT64_MAX - 4) return 0;
        per_row = cols;
    } else if (t.type == kQ4) {
        if (cols == INT64_MAX) return 0;
        per_row = (cols + 1) / 2;
    } else {
        if (cols > (INT64_MAX - 7) / 6) return 0;
        per_row = (cols * 6 + 7) / 8;
    }
    if (rows > INT64_MAX / (4 + per_row)) return 0;
    return rows * 4 + rows * per_row;
}

}  // namespace

struct pocr_gguf {
    int fd = -1;
    uint64_t data_start = 0;
    int64_t file_size = 0;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int> index;
    std::vector<Meta> meta;
    ~pocr_gguf() {
        if (fd >= 0) ::close(fd);
    }
};

namespace {

int read_string(Reader &r, std::string &s, const char *what) {
    uint64_t n;
    if (!r.u64(n)) return fail(POCR_ERR_ARG, "gguf: truncated %s", what);
    if (n > kMaxString) return fail(POCR_ERR_ARG, "gguf: string too large: %llu bytes", (unsigned long long)n);
    s.resize(n);
    if (n && !r.read(&s[0], n)) return fail(POCR_ERR_ARG, "gguf: truncated %s", what);
    return POCR_OK;
}

int parse(pocr_gguf *g) {
    struct stat st;
    if (fstat(g->fd, &st) != 0) return fail(POCR_ERR_ARG, "gguf: stat: %s", std::strerror(errno));
    g->file_size = st.st_size;
    Reader r{g->fd, std::vector<uint8_t>(64 << 10)};
    char magic[4];
    if (!r.read(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail(POCR_ERR_ARG, "gguf: bad magic");
    uint32_t version;
    if (!r.u32(version)) return fail(POCR_ERR_ARG, "gguf: truncated header");
    if (version != kVersion) return fail(POCR_ERR_ARG, "gguf: unsupported version %u", version);
    uint64_t nt, nkv;
    if (!r.u64(nt) || !r.u64(nkv)) return fail(POCR_ERR_ARG, "gguf: truncated header");
    if (nt > kMaxTensors) return fail(POCR_ERR_ARG, "gguf: tensor count too large: %llu", (unsigned long long)nt);
    if (nkv > kMaxKV) return fail(POCR_ERR_ARG, "gguf: metadata count too large: %llu", (unsigned long long)nkv);
    std::unordered_map<std::string, int> keys;
    for (uint64_t i = 0; i < nkv; ++i) {
        if (r.n > kMaxHeader) return fail(POCR_ERR_ARG, "gguf: header too large");
        Meta m;
        if (int rc = read_string(r, m.key, "metadata key")) return rc;
        if (!r.u32(m.type)) return fail(POCR_ERR_ARG, "gguf: truncated metadata");
        if (m.type == kMetaU32) {
            uint32_t v;
            if (!r.u32(v)) return fail(POCR_ERR_ARG, "gguf: truncated metadata");
            m.u = v;
        } else if (m.type == kMetaU64) {
            if (!r.u64(m.u)) return fail(POCR_ERR_ARG, "gguf: truncated metadata");
        } else if (m.type == kMetaString) {
            if (int rc = read_string(r, m.s, "metadata value")) return rc;
        } else {
            return fail(POCR_ERR_ARG, "gguf: unsupported metadata type %u", m.type);
        }
        if (m.key.empty()) return fail(POCR_ERR_ARG, "gguf: metadata has empty key");
        if (!printable(m.key)) return fail(POCR_ERR_ARG, "gguf: metadata key contains control character");
        if (!keys.emplace(m.key, (int)i).second)
            return fail(POCR_ERR_ARG, "gguf: metadata key %s is duplicated", m.key.c_str());
        g->meta.push_back(std::move(m));
    }
    for (uint64_t i = 0; i < nt; ++i) {
        if (r.n > kMaxHeader) return fail(POCR_ERR_ARG, "gguf: header too large");
        Tensor t;
        if (int rc = read_string(r, t.name, "tensor name")) return rc;
        if (t.name.empty()) return fail(POCR_ERR_ARG, "gguf: tensor has empty name");
        if (!printable(t.name)) return fail(POCR_ERR_ARG, "gguf: tensor name contains control character");
        if (g->index.count(t.name)) return fail(POCR_ERR_ARG, "gguf: tensor %s is duplicated", t.name.c_str());
        uint32_t nd;
        if (!r.u32(nd)) return fail(POCR_ERR_ARG, "gguf: truncated tensor info");
        if (nd > kMaxDims) return fail(POCR_ERR_ARG, "gguf: tensor %s has too many dimensions: %u", t.name.c_str(), nd);
        t.dims.resize(nd);
        for (uint32_t j = 0; j < nd; ++j) {
            uint64_t d;
            if (!r.u64(d)) return fail(POCR_ERR_ARG, "gguf: truncated tensor info");
            t.dims[j] = (int64_t)d;  // values above INT64_MAX turn negative and are rejected below
        }
        if (!r.u32(t.type) || !r.u64(t.offset)) return fail(POCR_ERR_ARG, "gguf: truncated tensor info");
        g->index.emplace(t.name, (int)g->tensors.size());
        g->tensors.push_back(std::move(t));
    }
    g->data_start = (r.n + kAlign - 1) / kAlign * kAlign;
    if (g->data_start > (uint64_t)g->file_size) return fail(POCR_ERR_ARG, "gguf: header exceeds file size");
    // validateTensorMeta (gguf.go:277-296)
    for (const Tensor &t : g->tensors) {
        int64_t n;
        if (!elem_count(t.dims, n)) return fail(POCR_ERR_ARG, "gguf: tensor %s has invalid shape", t.name.c_str());
        const int64_t size = tensor_bytes(t);
        if (size <= 0) return fail(POCR_ERR_ARG, "gguf: tensor %s has invalid type or shape", t.name.c_str());
        // compared in unsigned before any addition (data_start ≤ file_size
        // above), so no sum can overflow
        if (t.offset > (uint64_t)g->file_size - g->data_start)
            return fail(POCR_ERR_ARG, "gguf: tensor %s offset exceeds file size", t.name.c_str());
        const int64_t start = (int64_t)(g->data_start + t.offset);
        if (size > g->file_size - start) return fail(POCR_ERR_ARG, "gguf: tensor %s exceeds file size", t.name.c_str());
    }
    return POCR_OK;
}

}  // namespace

extern "C" int pocr_gguf_open(const char *path, pocr_gguf **out) {
    if (!path || !out) return fail(POCR_ERR_ARG, "pocr_gguf_open: null argument");
    *out = nullptr;
    pocr_gguf *g = new pocr_gguf();
    g->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        delete g;
        return fail(POCR_ERR_ARG, "gguf: open %s: %s", path, std::strerror(errno));
    }
    const int rc = parse(g);
    if (rc != POCR_OK) {
        delete g;
        return rc;
    }
    *out = g;
    return POCR_OK;
}

extern "C" void pocr_gguf_close(pocr_gguf *g) { delete g; }

extern "C" int pocr_gguf_tensor_count(const pocr_gguf *g) {
    return g ? (int)g->tensors.size() : fail(POCR_ERR_ARG, "pocr_gguf_tensor_count: null");
}

extern "C" int pocr_gguf_find(const pocr_gguf *g, const char *name) {
    if (!g || !name) return fail(POCR_ERR_ARG, "pocr_gguf_find: null argument");
    const auto it = g->index.find(name);
    return it == g->index.end() ? fail(POCR_ERR_ARG, "gguf: missing tensor %s", name) : it->second;
}

extern "C" int pocr_gguf_tensor_info(const pocr_gguf *g, int i, const char **name, uint32_t *type, int *ndim,
                                     int64_t *dims, int64_t *bytes) {
    if (!g || i < 0 || i >= (int)g->tensors.size()) return fail(POCR_ERR_ARG, "pocr_gguf_tensor_info: bad index");
    const Tensor &t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (ndim) *ndim = (int)t.dims.size();
    if (dims)
        for (size_t j = 0; j < t.dims.size(); ++j) dims[j] = t.dims[j];
    if (bytes) *bytes = tensor_bytes(t);
    return POCR_OK;
}

extern "C" int pocr_gguf_read(const pocr_gguf *g, int i, void *dst, int64_t bytes) {
    if (!g || !dst || i < 0 || i >= (int)g->tensors.size()) return fail(POCR_ERR_ARG, "pocr_gguf_read: bad arguments");
    const Tensor &t = g->tensors[i];
    if (bytes != tensor_bytes(t))
        return fail(POCR_ERR_ARG, "gguf: tensor %s holds %lld bytes, not %lld", t.name.c_str(),
                    (long long)tensor_bytes(t), (long long)bytes);
    uint8_t *d = static_cast<uint8_t *>(dst);
    int64_t off = (int64_t)g->data_start + (int64_t)t.offset, left = bytes;
    while (left > 0) {
        const ssize_t r = ::pread(g->fd, d, (size_t)std::min<int64_t>(left, 1 << 30), off);
        if (r <= 0) return fail(POCR_ERR_ARG, "gguf: read %s: %s", t.name.c_str(), r < 0 ? std::strerror(errno) : "EOF");
        d += r;
        off += r;
        left -= r;
    }
    return POCR_OK;
}

extern "C" int pocr_gguf_meta_count(const pocr_gguf *g) {
    return g ? (int)g->meta.size() : fail(POCR_ERR_ARG, "pocr_gguf_meta_count: null");
}

extern "C" int pocr_gguf_meta(const pocr_gguf *g, int i, const char **key, uint32_t *type, uint64_t *value,
                              const char **str) {
    if (!g || i < 0 || i >= (int)g->meta.size()) return fail(POCR_ERR_ARG, "pocr_gguf_meta: bad index");
    const Meta &m = g->meta[i];
    if (key) *key = m.key.c_str();
    if (type) *type = m.type;
    if (value) *value = m.u;
    if (str) *str = m.type == kMetaString ? m.s.c_str() : nullptr;
    return POCR_OK;
}
