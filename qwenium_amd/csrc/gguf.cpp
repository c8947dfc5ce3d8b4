// gguf.cpp -- GGUF ingestion for the MoE layer: map a GGUF file, parse its
// key/value metadata and tensor inventory, hand out tensor descriptors in the
// layer's qmoe_tensor form and copy tensor bytes to device memory unchanged
// (the on-disk block layout is the layer's input layout).
//
// Behaviour restated from the reference's loader:
//   src/loader/gguf_loader.cpp:46-91    header (magic "GGUF", version <= 3, u64 tensor and KV counts),
//                                       metadata, inventory, data offset aligned to 32 bytes (:84-85)
//   src/loader/gguf_loader.cpp:245-436  KV parsing (u64-length strings, typed values, arrays skipped)
//   src/loader/gguf_loader.cpp:474-497  inventory: name, n_dims (u32), ne (u64 each), ggml type (u32),
//                                       offset (u64, relative to the data start)
//   src/loader/gguf_loader.cpp:540-590  value skipping, incl. arrays of strings
//   src/loader/gguf_loader.cpp:621-639  tensor data = data start + offset, bounds-checked
//   src/loader/gguf_loader.cpp:213      tensor bytes = type size * elements / block size
// A general.alignment key (u32), when present, replaces the 32-byte default
// (files written with the default are read identically).
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "qmoe.h"
#include "qmoe_internal.h"

namespace {

enum GgufType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kStr = 8, kArr = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint32_t kMaxVersion = 3;
constexpr uint64_t kDefaultAlign = 32;

struct KV {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned / bool value
    int64_t i = 0;    // signed value
    double f = 0.0;   // float value
    std::string s;    // string value
};

struct TensorRec {
    int32_t type = 0;
    int32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;  // relative to the data start
};

// ggml block geometry (type id -> {block elements, block bytes}) for the types a
// GGUF tensor size can be computed for; the layer itself consumes F32, Q4_0, Q8_0.
bool type_geometry(int32_t type, uint64_t* blk, uint64_t* bytes) {
    switch (type) {
        case 0: *blk = 1; *bytes = 4; return true;    // F32
        case 1: *blk = 1; *bytes = 2; return true;    // F16
        case 2: *blk = 32; *bytes = 18; return true;  // Q4_0
        case 3: *blk = 32; *bytes = 20; return true;  // Q4_1
        case 6: *blk = 32; *bytes = 22; return true;  // Q5_0
        case 7: *blk = 32; *bytes = 24; return true;  // Q5_1
        case 8: *blk = 32; *bytes = 34; return true;  // Q8_0
        case 9: *blk = 32; *bytes = 36; return true;  // Q8_1
        case 24: *blk = 1; *bytes = 1; return true;   // I8
        case 25: *blk = 1; *bytes = 2; return true;   // I16
        case 26: *blk = 1; *bytes = 4; return true;   // I32
        case 27: *blk = 1; *bytes = 8; return true;   // I64
        case 28: *blk = 1; *bytes = 8; return true;   // F64
        case 30: *blk = 1; *bytes = 2; return true;   // BF16
        default: return false;
    }
}

struct Reader {
    const uint8_t* p;
    uint64_t size;
    uint64_t off = 0;
    std::string err;
    bool ok() const { return err.empty(); }
    bool need(uint64_t n, const char* what) {
        if (!err.empty()) return false;
        if (n > size || off > size - n) {
            err = std::string("gguf: read past end of file while reading ") + what + " at offset " + std::to_string(off);
            return false;
        }
        return true;
    }
    template <typename V>
    V get(const char* what) {
        V v{};
        if (need(sizeof(V), what)) {
            std::memcpy(&v, p + off, sizeof(V));
            off += sizeof(V);
        }
        return v;
    }
    std::string str(const char* what) {
        const uint64_t n = get<uint64_t>(what);
        if (!need(n, what)) return {};
        std::string s((const char*)p + off, n);
        off += n;
        return s;
    }
    void skip(uint64_t n, const char* what) {
        if (need(n, what)) off += n;
    }
};

uint64_t scalar_bytes(uint32_t type) {
    switch (type) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

// Reads one value of `type`; arrays are skipped (only scalars are kept).
bool read_value(Reader& r, uint32_t type, KV* kv) {
    kv->type = type;
    switch (type) {
        case kU8: kv->u = r.get<uint8_t>("u8"); break;
        case kI8: kv->i = r.get<int8_t>("i8"); break;
        case kU16: kv->u = r.get<uint16_t>("u16"); break;
        case kI16: kv->i = r.get<int16_t>("i16"); break;
        case kU32: kv->u = r.get<uint32_t>("u32"); break;
        case kI32: kv->i = r.get<int32_t>("i32"); break;
        case kF32: kv->f = r.get<float>("f32"); break;
        case kBool: kv->u = r.get<uint8_t>("bool") != 0; break;
        case kU64: kv->u = r.get<uint64_t>("u64"); break;
        case kI64: kv->i = r.get<int64_t>("i64"); break;
        case kF64: kv->f = r.get<double>("f64"); break;
        case kStr: kv->s = r.str("string"); break;
        case kArr: {
            const uint32_t et = r.get<uint32_t>("array type");
            const uint64_t n = r.get<uint64_t>("array length");
            if (!r.ok()) return false;
            if (et == kStr) {
                for (uint64_t k = 0; k < n && r.ok(); ++k) r.skip(r.get<uint64_t>("array string length"), "array string");
            } else {
                const uint64_t es = scalar_bytes(et);
                if (!es) {
                    r.err = "gguf: unknown array element type " + std::to_string(et);
                    return false;
                }
                if (n > r.size / es) {
                    r.err = "gguf: read past end of file while skipping an array";
                    return false;
                }
                r.skip(n * es, "array");
            }
            break;
        }
        default:
            r.err = "gguf: unknown metadata value type " + std::to_string(type);
            return false;
    }
    return r.ok();
}

}  // namespace

struct qmoe_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t data_offset = 0;
    uint64_t alignment = kDefaultAlign;
    std::unordered_map<std::string, KV> kv;
    std::vector<std::string> names;  // inventory order
    std::unordered_map<std::string, TensorRec> tensors;
    ~qmoe_gguf() {
        if (map) munmap((void*)map, size);
        if (fd >= 0) close(fd);
    }
};

static int gguf_fail(const std::string& msg) { return qmoe::set_error(QMOE_ERR_VALUE, msg); }

// The tensor's byte size: 0 on success; 1 for a type of unknown size or rows
// that are not whole blocks; 2 when a dimension is negative or the element
// count or byte size does not fit 64 bits (a crafted inventory must not wrap
// around to a small size that passes the end-of-file check).
static int tensor_bytes(const TensorRec& t, uint64_t* out) {
    uint64_t blk = 0, bytes = 0;
    if (!type_geometry(t.type, &blk, &bytes)) return 1;
    uint64_t n = 1;
    for (int d = 0; d < 4; ++d) {
        if (t.ne[d] < 0 || __builtin_mul_overflow(n, (uint64_t)t.ne[d], &n)) return 2;
    }
    if (n % blk) return 1;
    if (__builtin_mul_overflow(n / blk, bytes, out)) return 2;
    return 0;
}

extern "C" {

int qmoe_gguf_open(const char* path, qmoe_gguf** out) {
    qmoe::clear_error();
    if (!path || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: path and out expected non-null, got null");
    *out = nullptr;
    auto g = new qmoe_gguf();
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) {
        delete g;
        return gguf_fail(std::string("gguf: failed to open file: ") + path);
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        delete g;
        return gguf_fail(std::string("gguf: failed to map file: ") + path);
    }
    g->size = (uint64_t)st.st_size;
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        delete g;
        return gguf_fail(std::string("gguf: failed to map file: ") + path);
    }
    g->map = (const uint8_t*)m;
    Reader r{g->map, g->size};
    if (!r.need(24, "header")) {
        delete g;
        return gguf_fail("gguf: file is too small for the GGUF header");
    }
    const uint32_t magic = r.get<uint32_t>("magic");
    g->version = r.get<uint32_t>("version");
    if (magic != kMagic) {
        delete g;
        return gguf_fail("gguf: invalid magic number");
    }
    if (g->version > kMaxVersion || g->version < 2) {
        const uint32_t v = g->version;
        delete g;
        return gguf_fail("gguf: unsupported GGUF version: expected 2 or 3, got " + std::to_string(v));
    }
    const uint64_t n_tensors = r.get<uint64_t>("tensor count");
    const uint64_t n_kv = r.get<uint64_t>("metadata count");
    for (uint64_t k = 0; k < n_kv && r.ok(); ++k) {
        std::string key = r.str("metadata key");
        const uint32_t type = r.get<uint32_t>("metadata type");
        KV v;
        if (!r.ok() || !read_value(r, type, &v)) break;
        g->kv[key] = std::move(v);
    }
    for (uint64_t k = 0; k < n_tensors && r.ok(); ++k) {
        std::string name = r.str("tensor name");
        TensorRec t;
        const uint32_t nd = r.get<uint32_t>("tensor n_dims");
        if (r.ok() && (nd < 1 || nd > 4)) {
            r.err = "gguf: tensor \"" + name + "\" expected 1..4 dims, got " + std::to_string(nd);
            break;
        }
        t.n_dims = (int32_t)nd;
        for (uint32_t d = 0; d < nd && r.ok(); ++d) t.ne[d] = (int64_t)r.get<uint64_t>("tensor shape");
        t.type = (int32_t)r.get<uint32_t>("tensor type");
        t.offset = r.get<uint64_t>("tensor offset");
        if (!r.ok()) break;
        g->names.push_back(name);
        g->tensors[name] = t;
    }
    if (!r.ok()) {
        const std::string e = r.err;
        delete g;
        return gguf_fail(e);
    }
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end() && al->second.type == kU32 && al->second.u > 0) g->alignment = al->second.u;
    g->data_offset = (r.off + g->alignment - 1) / g->alignment * g->alignment;
    *out = g;
    return QMOE_OK;
}

void qmoe_gguf_close(qmoe_gguf* g) { delete g; }

int qmoe_gguf_info(const qmoe_gguf* g, uint32_t* version, int64_t* n_tensors, int64_t* n_kv, uint64_t* data_offset) {
    qmoe::clear_error();
    if (!g) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: gguf expected non-null, got null");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = (int64_t)g->names.size();
    if (n_kv) *n_kv = (int64_t)g->kv.size();
    if (data_offset) *data_offset = g->data_offset;
    return QMOE_OK;
}

int qmoe_gguf_get_u32(const qmoe_gguf* g, const char* key, uint32_t* out) {
    qmoe::clear_error();
    if (!g || !key || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: gguf, key and out expected non-null, got null");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: key \"") + key + "\" expected present, got absent");
    if (it->second.type != kU32)
        return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: key \"") + key + "\" expected type UINT32, got type " +
                                              std::to_string(it->second.type));
    *out = (uint32_t)it->second.u;
    return QMOE_OK;
}

int qmoe_gguf_get_f32(const qmoe_gguf* g, const char* key, float* out) {
    qmoe::clear_error();
    if (!g || !key || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: gguf, key and out expected non-null, got null");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: key \"") + key + "\" expected present, got absent");
    if (it->second.type != kF32)
        return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: key \"") + key + "\" expected type FLOAT32, got type " +
                                              std::to_string(it->second.type));
    *out = (float)it->second.f;
    return QMOE_OK;
}

int qmoe_gguf_get_str(const qmoe_gguf* g, const char* key, const char** out) {
    qmoe::clear_error();
    if (!g || !key || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: gguf, key and out expected non-null, got null");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: key \"") + key + "\" expected present, got absent");
    if (it->second.type != kStr)
        return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: key \"") + key + "\" expected type STRING, got type " +
                                              std::to_string(it->second.type));
    *out = it->second.s.c_str();
    return QMOE_OK;
}

int qmoe_gguf_tensor_name(const qmoe_gguf* g, int64_t index, const char** out) {
    qmoe::clear_error();
    if (!g || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: gguf and out expected non-null, got null");
    if (index < 0 || index >= (int64_t)g->names.size())
        return qmoe::set_error(QMOE_ERR_VALUE, "gguf: tensor index expected in [0, " + std::to_string(g->names.size()) +
                                              "), got " + std::to_string(index));
    *out = g->names[(size_t)index].c_str();
    return QMOE_OK;
}

int qmoe_gguf_find(const qmoe_gguf* g, const char* name, qmoe_gguf_tensor* out) {
    qmoe::clear_error();
    if (!g || !name || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: gguf, name and out expected non-null, got null");
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: tensor \"") + name + "\" expected present, got absent");
    const TensorRec& t = it->second;
    uint64_t bytes = 0;
    const int tb = tensor_bytes(t, &bytes);
    if (tb == 1)
        return qmoe::set_error(QMOE_ERR_TYPE, std::string("gguf: tensor \"") + name + "\" has ggml type " + std::to_string(t.type) +
                                             " whose size is unknown here (or a row not a whole number of blocks)");
    if (tb == 2)
        return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: tensor \"") + name +
                                                  "\" expected a shape whose byte size fits 64 bits, got one that overflows");
    uint64_t start = 0;
    if (__builtin_add_overflow(g->data_offset, t.offset, &start) || start > g->size || bytes > g->size - start)
        return qmoe::set_error(QMOE_ERR_VALUE, std::string("gguf: tensor data for \"") + name + "\" would read past end of file");
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    out->file_offset = start;
    out->nbytes = bytes;
    return QMOE_OK;
}

int qmoe_gguf_read(const qmoe_gguf* g, const char* name, void* dst, uint64_t dst_bytes) {
    qmoe_gguf_tensor t;
    int rc = qmoe_gguf_find(g, name, &t);
    if (rc) return rc;
    if (!dst) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: dst expected non-null, got null");
    if (dst_bytes < t.nbytes)
        return qmoe::set_error(QMOE_ERR_CAPACITY, std::string("gguf: tensor \"") + name + "\" needs " + std::to_string(t.nbytes) +
                                                 " bytes, got a buffer of " + std::to_string(dst_bytes));
    std::memcpy(dst, g->map + t.file_offset, t.nbytes);
    return QMOE_OK;
}

int qmoe_gguf_upload(const qmoe_gguf* g, const char* name, void* dst_device, uint64_t dst_bytes, void* hip_stream) {
    qmoe_gguf_tensor t;
    int rc = qmoe_gguf_find(g, name, &t);
    if (rc) return rc;
    if (!dst_device) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: dst_device expected a device pointer, got null");
    if (dst_bytes < t.nbytes)
        return qmoe::set_error(QMOE_ERR_CAPACITY, std::string("gguf: tensor \"") + name + "\" needs " + std::to_string(t.nbytes) +
                                                 " bytes, got a buffer of " + std::to_string(dst_bytes));
    // pageable source: the copy has finished reading the mapping when the call returns
    hipError_t err = hipMemcpyAsync(dst_device, g->map + t.file_offset, t.nbytes, hipMemcpyHostToDevice,
                                    (hipStream_t)hip_stream);
    if (err == hipSuccess) err = hipStreamSynchronize((hipStream_t)hip_stream);
    return err == hipSuccess ? QMOE_OK : qmoe::hip_error(err, "gguf upload");
}

int qmoe_gguf_tensor_view(const qmoe_gguf_tensor* t, const void* device_data, qmoe_tensor* out) {
    qmoe::clear_error();
    if (!t || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: t and out expected non-null, got null");
    uint64_t blk = 0, bytes = 0;
    if (!type_geometry(t->type, &blk, &bytes))
        return qmoe::set_error(QMOE_ERR_TYPE, "gguf: ggml type " + std::to_string(t->type) + " has no known block geometry");
    if (t->ne[0] % (int64_t)blk)
        return qmoe::set_error(QMOE_ERR_SHAPE, "gguf: ne[0] expected a multiple of " + std::to_string(blk) + ", got " +
                                                   std::to_string(t->ne[0]));
    out->data = device_data;
    out->type = t->type;
    out->n_dims = t->n_dims;
    for (int d = 0; d < 4; ++d) out->ne[d] = t->ne[d];
    out->nb[0] = bytes;
    out->nb[1] = (uint64_t)(t->ne[0] / (int64_t)blk) * bytes;
    for (int d = 2; d < 4; ++d) out->nb[d] = out->nb[d - 1] * (uint64_t)t->ne[d - 1];
    return QMOE_OK;
}

}  // extern "C"
