// gguf.cpp -- GGUF (v2/v3) reader and device upload, the host side of the
// load path (GgufFile::open / read_tensor_bytes / find_tensor, gguf.cpp:
// 288-368; the engine's verbatim upload, metal_decode.mm:157-176).
//
// Layout (little-endian): "GGUF" | u32 version | u64 n_tensors | u64 n_kv |
// n_kv x (string key, u32 type, value) | n_tensors x (string name, u32 n_dims,
// u64 dims[n_dims], u32 ggml type, u64 offset) | padding to the alignment
// (metadata "general.alignment", default 32) | tensor data, each tensor at
// data_start + offset.  A string is a u64 length and its bytes; an array is
// u32 element type, u64 count and the elements.
//
// The file is mapped read-only once; every read is bounds-checked against
// its size, so a truncated or corrupt header is an error (RT_HIP_E_FORMAT),
// never an out-of-range read.  Tensor bytes are copied to the device
// straight from the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "rt_hip.h"
#include "rt_launch.hpp"

namespace {
int fail(int code, const std::string& msg) { return rt_hip::set_error(code, msg); }

// The metadata types an unsigned read accepts: u8, u16, u32, u64, i32, i64
// (GgufMetaValue::as_u64, gguf.cpp:104-112; signed ones sign-extended).
bool u64_type(uint32_t t) { return t == 0 || t == 2 || t == 4 || t == 10 || t == 5 || t == 11; }
}  // namespace

namespace {

// Bytes per block and values per block of the ggml types the path sizes
// (gguf_block_info, gguf.cpp:81-93); 0 for the rest.
void block_info(int32_t type, int64_t* bytes, int64_t* elems) {
    *bytes = 0;
    *elems = 1;
    switch (type) {
        case RT_HIP_GGUF_F32: *bytes = 4; break;
        case RT_HIP_GGUF_F16: *bytes = 2; break;
        case RT_HIP_GGUF_BF16: *bytes = 2; break;
        case RT_HIP_GGUF_Q4_0: *bytes = 18; *elems = 32; break;
        case RT_HIP_GGUF_Q8_0: *bytes = 34; *elems = 32; break;
        case RT_HIP_GGUF_Q4_K: *bytes = 144; *elems = 256; break;
        case RT_HIP_GGUF_Q5_K: *bytes = 176; *elems = 256; break;
        case RT_HIP_GGUF_Q6_K: *bytes = 210; *elems = 256; break;
        default: break;
    }
}

// Metadata value.  Arrays keep their elements (nested arrays included).
struct Meta {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned and signed integers, bool (two's complement for signed)
    double f = 0.0;   // f32 / f64
    std::string s;
    std::vector<Meta> arr;
};

class Reader {
   public:
    Reader(const uint8_t* p, uint64_t n) : p_(p), n_(n) {}
    uint64_t pos() const { return pos_; }
    bool bytes(void* dst, uint64_t n) {
        if (n > n_ - pos_) return false;
        std::memcpy(dst, p_ + pos_, n);
        pos_ += n;
        return true;
    }
    template <typename T>
    bool le(T* v) {
        uint8_t b[sizeof(T)];
        if (!bytes(b, sizeof(T))) return false;
        uint64_t x = 0;
        for (int i = static_cast<int>(sizeof(T)) - 1; i >= 0; --i) x = (x << 8) | b[i];
        *v = static_cast<T>(x);
        return true;
    }
    bool str(std::string* s) {
        uint64_t len;
        if (!le(&len) || len > n_ - pos_) return false;
        s->assign(reinterpret_cast<const char*>(p_ + pos_), len);
        pos_ += len;
        return true;
    }

   private:
    const uint8_t* p_;
    uint64_t n_;
    uint64_t pos_ = 0;
};

constexpr int kMaxArrayDepth = 4;

bool read_value(Reader& r, uint32_t type, Meta* m, int depth) {
    m->type = type;
    switch (type) {
        case 0: { uint8_t v; if (!r.le(&v)) return false; m->u = v; return true; }
        case 1: { uint8_t v; if (!r.le(&v)) return false; m->u = static_cast<uint64_t>(static_cast<int64_t>(static_cast<int8_t>(v))); return true; }
        case 2: { uint16_t v; if (!r.le(&v)) return false; m->u = v; return true; }
        case 3: { uint16_t v; if (!r.le(&v)) return false; m->u = static_cast<uint64_t>(static_cast<int64_t>(static_cast<int16_t>(v))); return true; }
        case 4: { uint32_t v; if (!r.le(&v)) return false; m->u = v; return true; }
        case 5: { uint32_t v; if (!r.le(&v)) return false; m->u = static_cast<uint64_t>(static_cast<int64_t>(static_cast<int32_t>(v))); return true; }
        case 6: { uint32_t v; if (!r.le(&v)) return false; float f; std::memcpy(&f, &v, 4); m->f = f; return true; }
        case 7: { uint8_t v; if (!r.le(&v)) return false; m->u = v != 0; return true; }
        case 8: return r.str(&m->s);
        case 9: {
            uint32_t et;
            uint64_t count;
            if (depth >= kMaxArrayDepth || !r.le(&et) || !r.le(&count)) return false;
            // Every element takes at least one byte: a count above the bytes
            // left is corrupt.
            if (count > (1ull << 40)) return false;
            m->arr.clear();
            for (uint64_t i = 0; i < count; ++i) {
                Meta e;
                if (!read_value(r, et, &e, depth + 1)) return false;
                m->arr.push_back(std::move(e));
            }
            return true;
        }
        case 10: return r.le(&m->u);
        case 11: { uint64_t v; if (!r.le(&v)) return false; m->u = v; return true; }
        case 12: { uint64_t v; if (!r.le(&v)) return false; double d; std::memcpy(&d, &v, 8); m->f = d; return true; }
        default: return false;
    }
}

}  // namespace

struct rt_hip_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t data_start = 0;
    std::map<std::string, Meta> meta;
    struct Tensor {
        std::string name;
        std::vector<int64_t> dims;
        int32_t type;
        uint64_t offset;
        int64_t n_elements;
        int64_t bytes;  // -1: a type this reader does not size
    };
    std::vector<Tensor> tensors;
};

namespace {

void close_file(rt_hip_gguf* f) {
    if (!f) return;
    if (f->map) munmap(const_cast<uint8_t*>(f->map), f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
}

int bad(rt_hip_gguf* f, const std::string& msg) {
    close_file(f);
    return fail(RT_HIP_E_FORMAT, msg);
}

}  // namespace

extern "C" {

int64_t rt_hip_gguf_type_bytes(int32_t type, int64_t n_elements) {
    int64_t b, e;
    block_info(type, &b, &e);
    if (b == 0 || n_elements < 0) return -1;
    return (n_elements + e - 1) / e * b;
}

int rt_hip_gguf_open(const char* path, rt_hip_gguf** out) {
    if (!path || !out) return fail(RT_HIP_E_ARG, "rt_hip_gguf_open: null argument");
    *out = nullptr;
    auto* f = new rt_hip_gguf();
    f->fd = open(path, O_RDONLY);
    if (f->fd < 0) return bad(f, std::string("cannot open GGUF file: ") + path);
    struct stat st;
    if (fstat(f->fd, &st) != 0) return bad(f, std::string("cannot stat GGUF file: ") + path);
    f->size = static_cast<uint64_t>(st.st_size);
    if (f->size < 4) return bad(f, std::string("not a GGUF file: ") + path);
    void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) return bad(f, std::string("cannot map GGUF file: ") + path);
    f->map = static_cast<const uint8_t*>(m);

    Reader r(f->map, f->size);
    char magic[4];
    if (!r.bytes(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0)
        return bad(f, std::string("not a GGUF file: ") + path);
    if (!r.le(&f->version)) return bad(f, "GGUF header: unexpected end of file");
    if (f->version < 2 || f->version > 3)
        return bad(f, "unsupported GGUF version " + std::to_string(f->version));
    uint64_t n_tensors, n_kv;
    if (!r.le(&n_tensors) || !r.le(&n_kv)) return bad(f, "GGUF header: unexpected end of file");
    // A key-value pair takes at least 12 bytes and a tensor info at least
    // 24: larger counts than the file can hold are corrupt.
    if (n_kv > f->size / 12 || n_tensors > f->size / 24) return bad(f, "GGUF header: counts exceed the file");
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t type;
        Meta v;
        if (!r.str(&key) || !r.le(&type) || !read_value(r, type, &v, 0))
            return bad(f, "GGUF metadata: unexpected end of file or bad value type");
        f->meta[key] = std::move(v);
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        rt_hip_gguf::Tensor t;
        uint32_t n_dims;
        if (!r.str(&t.name) || !r.le(&n_dims) || n_dims == 0 || n_dims > RT_HIP_GGUF_MAX_DIMS)
            return bad(f, "GGUF tensor info: unexpected end of file or bad rank");
        int64_t n = 1;
        for (uint32_t d = 0; d < n_dims; ++d) {
            uint64_t dim;
            if (!r.le(&dim) || dim > (1ull << 40)) return bad(f, "GGUF tensor info: bad dimension");
            if (dim != 0 && static_cast<uint64_t>(n) > (1ull << 62) / dim)
                return bad(f, "GGUF tensor info: element count overflows");
            n *= static_cast<int64_t>(dim);
            t.dims.push_back(static_cast<int64_t>(dim));
        }
        uint32_t type;
        if (!r.le(&type) || !r.le(&t.offset)) return bad(f, "GGUF tensor info: unexpected end of file");
        t.type = static_cast<int32_t>(type);
        t.n_elements = n;
        t.bytes = rt_hip_gguf_type_bytes(t.type, n);
        f->tensors.push_back(std::move(t));
    }
    uint64_t alignment = 32;
    auto it = f->meta.find("general.alignment");
    if (it != f->meta.end() && u64_type(it->second.type)) {
        alignment = it->second.u;
    }
    if (alignment == 0 || alignment > (1u << 20)) return bad(f, "GGUF: bad general.alignment");
    f->data_start = (r.pos() + alignment - 1) / alignment * alignment;
    // Every sized tensor must lie inside the file.
    for (const auto& t : f->tensors) {
        if (t.bytes < 0) continue;
        if (t.offset > f->size || f->data_start > f->size - t.offset ||
            static_cast<uint64_t>(t.bytes) > f->size - f->data_start - t.offset)
            return bad(f, "GGUF tensor " + t.name + ": data past the end of the file");
    }
    *out = f;
    return RT_HIP_OK;
}

void rt_hip_gguf_close(rt_hip_gguf* f) { close_file(f); }

int64_t rt_hip_gguf_tensor_count(const rt_hip_gguf* f) { return f ? static_cast<int64_t>(f->tensors.size()) : -1; }

int64_t rt_hip_gguf_find_tensor(const rt_hip_gguf* f, const char* name) {
    if (!f || !name) return -1;
    for (size_t i = 0; i < f->tensors.size(); ++i)
        if (f->tensors[i].name == name) return static_cast<int64_t>(i);
    return -1;
}

int rt_hip_gguf_tensor_info(const rt_hip_gguf* f, int64_t idx, rt_hip_gguf_tensor* out) {
    if (!f || !out) return fail(RT_HIP_E_ARG, "rt_hip_gguf_tensor_info: null argument");
    if (idx < 0 || idx >= static_cast<int64_t>(f->tensors.size()))
        return fail(RT_HIP_E_ARG, "rt_hip_gguf_tensor_info: index out of range");
    const auto& t = f->tensors[static_cast<size_t>(idx)];
    std::memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = static_cast<int32_t>(t.dims.size());
    for (size_t d = 0; d < t.dims.size(); ++d) out->dims[d] = t.dims[d];
    out->n_elements = t.n_elements;
    out->bytes = t.bytes;
    out->file_offset = t.bytes < 0 ? -1 : static_cast<int64_t>(f->data_start + t.offset);
    return RT_HIP_OK;
}

int rt_hip_gguf_read_tensor(const rt_hip_gguf* f, int64_t idx, void* dst, int64_t bytes) {
    rt_hip_gguf_tensor t;
    int rc = rt_hip_gguf_tensor_info(f, idx, &t);
    if (rc) return rc;
    if (!dst) return fail(RT_HIP_E_ARG, "rt_hip_gguf_read_tensor: null destination");
    if (t.bytes < 0) return fail(RT_HIP_E_UNSUPPORTED, std::string("unsupported gguf type for tensor ") + t.name);
    if (bytes != t.bytes) return fail(RT_HIP_E_ARG, std::string("rt_hip_gguf_read_tensor: tensor ") + t.name +
                                                        " has " + std::to_string(t.bytes) + " bytes");
    std::memcpy(dst, f->map + t.file_offset, static_cast<size_t>(t.bytes));
    return RT_HIP_OK;
}

int rt_hip_gguf_upload(const rt_hip_gguf* f, int64_t idx, void* device_dst, int64_t bytes, rt_hip_stream stream) {
    rt_hip_gguf_tensor t;
    int rc = rt_hip_gguf_tensor_info(f, idx, &t);
    if (rc) return rc;
    if (!device_dst) return fail(RT_HIP_E_ARG, "rt_hip_gguf_upload: null destination");
    if (t.bytes < 0) return fail(RT_HIP_E_UNSUPPORTED, std::string("unsupported gguf type for tensor ") + t.name);
    if (bytes != t.bytes)
        return fail(RT_HIP_E_ARG, std::string("rt_hip_gguf_upload: tensor ") + t.name + " has " +
                                      std::to_string(t.bytes) + " bytes");
    // From the read-only mapping (pageable memory: the copy completes before
    // the call returns, so the mapping may be closed afterwards).
    const auto s = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(device_dst, f->map + t.file_offset, static_cast<size_t>(t.bytes),
                                  hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(RT_HIP_E_HIP, std::string("rt_hip_gguf_upload: ") + hipGetErrorString(e));
    return RT_HIP_OK;
}

int rt_hip_gguf_linear_shape(const rt_hip_gguf* f, int64_t idx, int64_t* rows, int64_t* cols) {
    rt_hip_gguf_tensor t;
    int rc = rt_hip_gguf_tensor_info(f, idx, &t);
    if (rc) return rc;
    if (!rows || !cols) return fail(RT_HIP_E_ARG, "rt_hip_gguf_linear_shape: null argument");
    if (t.n_dims == 1) {
        *rows = 1;
        *cols = t.dims[0];
    } else if (t.n_dims == 2) {
        *rows = t.dims[1];
        *cols = t.dims[0];
    } else {
        return fail(RT_HIP_E_SHAPE, std::string("unexpected shape rank ") + std::to_string(t.n_dims) + " for " + t.name);
    }
    return RT_HIP_OK;
}

namespace {
static const Meta* meta_at(const rt_hip_gguf* f, const char* key, int64_t index) {
    if (!f || !key) return nullptr;
    auto it = f->meta.find(key);
    if (it == f->meta.end()) return nullptr;
    const Meta* m = &it->second;
    if (index >= 0) {
        if (m->type != 9 || index >= static_cast<int64_t>(m->arr.size())) return nullptr;
        m = &m->arr[static_cast<size_t>(index)];
    }
    return m;
}
}  // namespace

int rt_hip_gguf_meta_u64(const rt_hip_gguf* f, const char* key, int64_t index, uint64_t* out) {
    const Meta* m = meta_at(f, key, index);
    if (!m || !out) return fail(RT_HIP_E_ARG, std::string("gguf metadata: no entry ") + (key ? key : "(null)"));
    if (!u64_type(m->type))
        return fail(RT_HIP_E_UNSUPPORTED, std::string("gguf metadata: ") + key + " is not an integer");
    *out = m->u;
    return RT_HIP_OK;
}

int rt_hip_gguf_meta_f32(const rt_hip_gguf* f, const char* key, int64_t index, float* out) {
    const Meta* m = meta_at(f, key, index);
    if (!m || !out) return fail(RT_HIP_E_ARG, std::string("gguf metadata: no entry ") + (key ? key : "(null)"));
    if (m->type != 6 && m->type != 12)
        return fail(RT_HIP_E_UNSUPPORTED, std::string("gguf metadata: ") + key + " is not a float");
    *out = static_cast<float>(m->f);
    return RT_HIP_OK;
}

int rt_hip_gguf_meta_str(const rt_hip_gguf* f, const char* key, int64_t index, const char** out) {
    const Meta* m = meta_at(f, key, index);
    if (!m || !out) return fail(RT_HIP_E_ARG, std::string("gguf metadata: no entry ") + (key ? key : "(null)"));
    if (m->type != 8) return fail(RT_HIP_E_UNSUPPORTED, std::string("gguf metadata: ") + key + " is not a string");
    *out = m->s.c_str();
    return RT_HIP_OK;
}

int64_t rt_hip_gguf_meta_array_len(const rt_hip_gguf* f, const char* key) {
    const Meta* m = meta_at(f, key, -1);
    if (!m || m->type != 9) return -1;
    return static_cast<int64_t>(m->arr.size());
}

}  // extern "C"
