// GGUF reader and upload repacker (include/mvlm_gguf.h).
//
// Parses the GGUF container (header, metadata key/values, tensor infos,
// aligned data section) of a memory-mapped file with every read bounds-
// checked, the way gguf_open does (src/models/gguf_loader.cpp:163-349), and
// hands tensors to mvlm_weight_pack for the packed HBM layout.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "../../include/mvlm_gguf.h"

struct mvlm_gguf {
    void* map = nullptr;
    size_t size = 0;
    mvlm_gguf_info info{};
    struct KV {
        std::string key;
        uint32_t type = 0;
        uint64_t value = 0;        // file offset of the value
    };
    std::vector<KV> kvs;
    struct Tensor {
        uint64_t name_off = 0, name_len = 0;
        uint32_t n_dims = 0;
        uint64_t dims[4] = {1, 1, 1, 1};
        uint32_t type = 0;
        uint64_t offset = 0, bytes = 0;
    };
    std::vector<Tensor> tensors;
    const uint8_t* base() const { return static_cast<const uint8_t*>(map); }
};

namespace mvlm {
namespace {

// Block bytes / block elements of the ggml types (the public ggml
// definitions; gguf_loader.cpp:13-55 lists the same for the types it knows,
// except Q8_1, which it gives 40 bytes where ggml's block is 36).
struct TypeSize { uint32_t type; uint32_t bytes; uint32_t elems; };
constexpr TypeSize kTypes[] = {
    {0, 4, 1},      {1, 2, 1},      {2, 18, 32},    {3, 20, 32},    {6, 22, 32},   {7, 24, 32},
    {8, 34, 32},    {9, 36, 32},    {10, 84, 256},  {11, 110, 256}, {12, 144, 256}, {13, 176, 256},
    {14, 210, 256}, {15, 292, 256}, {24, 1, 1},     {25, 2, 1},     {26, 4, 1},    {27, 8, 1},
    {28, 8, 1},     {30, 2, 1},
};

const TypeSize* type_size(uint32_t type) {
    for (const TypeSize& t : kTypes)
        if (t.type == type) return &t;
    return nullptr;
}

// Bounds-checked reader over [pos, end).
struct Cursor {
    const uint8_t* base;
    uint64_t pos, end;
    bool ok = true;
    bool need(uint64_t n) {
        if (!ok || n > end - pos) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, base + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    // a GGUF string: uint64 length + bytes; returns the offset of the bytes
    uint64_t string(uint64_t* len) {
        *len = get<uint64_t>();
        const uint64_t at = pos;
        if (need(*len)) pos += *len;
        return at;
    }
};

int value_size(uint32_t type) {
    switch (type) {
        case MVLM_GGUF_UINT8: case MVLM_GGUF_INT8: case MVLM_GGUF_BOOL: return 1;
        case MVLM_GGUF_UINT16: case MVLM_GGUF_INT16: return 2;
        case MVLM_GGUF_UINT32: case MVLM_GGUF_INT32: case MVLM_GGUF_FLOAT32: return 4;
        case MVLM_GGUF_UINT64: case MVLM_GGUF_INT64: case MVLM_GGUF_FLOAT64: return 8;
        default: return 0;
    }
}

// Skips one value of `type`; false (with c.ok false or an unknown type) on error.
bool skip_value(Cursor& c, uint32_t type, int depth) {
    const int sz = value_size(type);
    if (sz) return c.need(sz) && (c.pos += sz, true);
    if (type == MVLM_GGUF_STRING) {
        uint64_t len;
        c.string(&len);
        return c.ok;
    }
    if (type == MVLM_GGUF_ARRAY && depth < 8) {
        const uint32_t et = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        if (!c.ok) return false;
        const int esz = value_size(et);
        if (esz) {
            if (n > (c.end - c.pos) / (uint64_t)esz) return c.ok = false;
            c.pos += n * esz;
            return true;
        }
        for (uint64_t i = 0; i < n; ++i)
            if (!skip_value(c, et, depth + 1)) return false;
        return true;
    }
    return false;
}

int fail(mvlm_gguf* g, int code, const char* path, const char* what) {
    if (g) {
        if (g->map) munmap(g->map, g->size);
        delete g;
    }
    return set_error(code, "mvlm_gguf_open: %s: %s", path, what);
}

const mvlm_gguf::KV* find_kv(const mvlm_gguf* g, const char* key) {
    const size_t n = std::strlen(key);
    for (const auto& kv : g->kvs)
        if (kv.key.size() == n && std::memcmp(kv.key.data(), key, n) == 0) return &kv;
    return nullptr;
}

}  // namespace
}  // namespace mvlm

using namespace mvlm;

extern "C" int mvlm_gguf_open(const char* path, mvlm_gguf** out) {
    REQUIRE(path && out, "mvlm_gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return set_error(MVLM_ERR_NOT_FOUND, "mvlm_gguf_open: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return set_error(MVLM_ERR_NOT_FOUND, "mvlm_gguf_open: cannot stat %s", path);
    }
    mvlm_gguf* g = new (std::nothrow) mvlm_gguf();
    if (!g) {
        close(fd);
        return set_error(MVLM_ERR_OUT_OF_MEMORY, "mvlm_gguf_open: out of memory");
    }
    g->size = (size_t)st.st_size;
    if (g->size < 24) {
        close(fd);
        return fail(g, MVLM_ERR_FORMAT, path, "file too small for a GGUF header");
    }
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return fail(g, MVLM_ERR_FORMAT, path, "mmap failed");
    g->map = m;

    Cursor c{g->base(), 0, g->size};
    const uint32_t magic = c.get<uint32_t>();
    if (magic != 0x46554747u) return fail(g, MVLM_ERR_FORMAT, path, "bad magic (not GGUF)");
    g->info.version = c.get<uint32_t>();
    if (g->info.version < 2 || g->info.version > 3)
        return fail(g, MVLM_ERR_FORMAT, path, "unsupported GGUF version (2 and 3 are read)");
    g->info.tensor_count = c.get<uint64_t>();
    g->info.metadata_kv_count = c.get<uint64_t>();
    g->info.file_size = g->size;
    // every key/value and tensor info takes at least 12 / 24 bytes
    if (g->info.metadata_kv_count > g->size / 12 || g->info.tensor_count > g->size / 24)
        return fail(g, MVLM_ERR_FORMAT, path, "implausible tensor or key/value count");

    g->info.alignment = 32;
    g->kvs.reserve(g->info.metadata_kv_count);
    for (uint64_t i = 0; i < g->info.metadata_kv_count; ++i) {
        mvlm_gguf::KV kv;
        uint64_t len;
        const uint64_t at = c.string(&len);
        kv.type = c.get<uint32_t>();
        if (!c.ok) return fail(g, MVLM_ERR_FORMAT, path, "truncated metadata key");
        kv.key.assign(reinterpret_cast<const char*>(g->base() + at), len);
        kv.value = c.pos;
        if (!skip_value(c, kv.type, 0)) return fail(g, MVLM_ERR_FORMAT, path, "truncated or unknown metadata value");
        if (kv.key == "general.alignment") {
            if (kv.type != MVLM_GGUF_UINT32) return fail(g, MVLM_ERR_FORMAT, path, "general.alignment is not uint32");
            uint32_t a;
            std::memcpy(&a, g->base() + kv.value, 4);
            if (a == 0 || (a & (a - 1)) != 0) return fail(g, MVLM_ERR_FORMAT, path, "general.alignment not a power of 2");
            g->info.alignment = a;
        }
        g->kvs.push_back(std::move(kv));
    }

    g->tensors.resize(g->info.tensor_count);
    for (auto& t : g->tensors) {
        t.name_off = c.string(&t.name_len);
        t.n_dims = c.get<uint32_t>();
        if (!c.ok) return fail(g, MVLM_ERR_FORMAT, path, "truncated tensor info");
        if (t.n_dims > 4) return fail(g, MVLM_ERR_FORMAT, path, "tensor with more than 4 dims");
        uint64_t elems = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            t.dims[d] = c.get<uint64_t>();
            if (t.dims[d] != 0 && elems > UINT64_MAX / t.dims[d])
                return fail(g, MVLM_ERR_FORMAT, path, "tensor element count overflows");
            elems *= t.dims[d];
        }
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) return fail(g, MVLM_ERR_FORMAT, path, "truncated tensor info");
        if (t.offset % g->info.alignment != 0) return fail(g, MVLM_ERR_FORMAT, path, "tensor offset not aligned");
        const TypeSize* ts = type_size(t.type);
        t.bytes = ts ? (elems + ts->elems - 1) / ts->elems * ts->bytes : 0;
    }
    g->info.data_offset = (c.pos + g->info.alignment - 1) / g->info.alignment * g->info.alignment;
    if (g->info.data_offset > g->size) return fail(g, MVLM_ERR_FORMAT, path, "data section starts past the end");
    for (const auto& t : g->tensors)
        if (t.offset > g->size - g->info.data_offset || t.bytes > g->size - g->info.data_offset - t.offset)
            return fail(g, MVLM_ERR_FORMAT, path, "tensor data past the end of the file");
    *out = g;
    return MVLM_OK;
}

extern "C" int mvlm_gguf_close(mvlm_gguf* g) {
    REQUIRE(g, "mvlm_gguf_close: null handle");
    if (g->map) munmap(g->map, g->size);
    delete g;
    return MVLM_OK;
}

extern "C" int mvlm_gguf_get_info(const mvlm_gguf* g, mvlm_gguf_info* out) {
    REQUIRE(g && out, "mvlm_gguf_get_info: null argument");
    *out = g->info;
    return MVLM_OK;
}

extern "C" int mvlm_gguf_tensor_info(const mvlm_gguf* g, uint64_t index, mvlm_gguf_tensor* out) {
    REQUIRE(g && out, "mvlm_gguf_tensor_info: null argument");
    REQUIRE(index < g->tensors.size(), "mvlm_gguf_tensor_info: index %llu >= %zu tensors",
            (unsigned long long)index, g->tensors.size());
    const auto& t = g->tensors[index];
    out->name = reinterpret_cast<const char*>(g->base() + t.name_off);
    out->name_len = t.name_len;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->dims[d] = t.dims[d];
    out->type = t.type;
    out->offset = t.offset;
    out->bytes = t.bytes;
    return MVLM_OK;
}

extern "C" int mvlm_gguf_find_tensor(const mvlm_gguf* g, const char* name, uint64_t* index) {
    REQUIRE(g && name && index, "mvlm_gguf_find_tensor: null argument");
    const size_t n = std::strlen(name);
    for (size_t i = 0; i < g->tensors.size(); ++i) {
        const auto& t = g->tensors[i];
        if (t.name_len == n && std::memcmp(g->base() + t.name_off, name, n) == 0) {
            *index = i;
            return MVLM_OK;
        }
    }
    return set_error(MVLM_ERR_NOT_FOUND, "mvlm_gguf_find_tensor: no tensor named %s", name);
}

extern "C" int mvlm_gguf_tensor_data(const mvlm_gguf* g, uint64_t index, const void** data) {
    REQUIRE(g && data, "mvlm_gguf_tensor_data: null argument");
    REQUIRE(index < g->tensors.size(), "mvlm_gguf_tensor_data: index out of range");
    *data = g->base() + g->info.data_offset + g->tensors[index].offset;
    return MVLM_OK;
}

extern "C" int mvlm_gguf_get_u32(const mvlm_gguf* g, const char* key, uint32_t* out) {
    REQUIRE(g && key && out, "mvlm_gguf_get_u32: null argument");
    const auto* kv = find_kv(g, key);
    if (!kv) return set_error(MVLM_ERR_NOT_FOUND, "mvlm_gguf_get_u32: no key %s", key);
    REQUIRE(kv->type == MVLM_GGUF_UINT32 || kv->type == MVLM_GGUF_INT32,
            "mvlm_gguf_get_u32: %s has value type %u", key, kv->type);
    std::memcpy(out, g->base() + kv->value, 4);
    return MVLM_OK;
}

extern "C" int mvlm_gguf_get_string(const mvlm_gguf* g, const char* key, const char** str, uint64_t* len) {
    REQUIRE(g && key && str && len, "mvlm_gguf_get_string: null argument");
    const auto* kv = find_kv(g, key);
    if (!kv) return set_error(MVLM_ERR_NOT_FOUND, "mvlm_gguf_get_string: no key %s", key);
    REQUIRE(kv->type == MVLM_GGUF_STRING, "mvlm_gguf_get_string: %s has value type %u", key, kv->type);
    Cursor c{g->base(), kv->value, g->size};
    const uint64_t at = c.string(len);
    *str = reinterpret_cast<const char*>(g->base() + at);
    return MVLM_OK;
}

extern "C" int mvlm_gguf_get_array(const mvlm_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count,
                                   const void** data) {
    REQUIRE(g && key && elem_type && count && data, "mvlm_gguf_get_array: null argument");
    const auto* kv = find_kv(g, key);
    if (!kv) return set_error(MVLM_ERR_NOT_FOUND, "mvlm_gguf_get_array: no key %s", key);
    REQUIRE(kv->type == MVLM_GGUF_ARRAY, "mvlm_gguf_get_array: %s has value type %u", key, kv->type);
    Cursor c{g->base(), kv->value, g->size};
    *elem_type = c.get<uint32_t>();
    *count = c.get<uint64_t>();
    *data = value_size(*elem_type) ? g->base() + c.pos : nullptr;
    return MVLM_OK;
}

extern "C" int mvlm_gguf_get_array_string(const mvlm_gguf* g, const char* key, uint64_t i, const char** str,
                                          uint64_t* len) {
    REQUIRE(g && key && str && len, "mvlm_gguf_get_array_string: null argument");
    const auto* kv = find_kv(g, key);
    if (!kv) return set_error(MVLM_ERR_NOT_FOUND, "mvlm_gguf_get_array_string: no key %s", key);
    REQUIRE(kv->type == MVLM_GGUF_ARRAY, "mvlm_gguf_get_array_string: %s is not an array", key);
    Cursor c{g->base(), kv->value, g->size};
    const uint32_t et = c.get<uint32_t>();
    const uint64_t n = c.get<uint64_t>();
    REQUIRE(et == MVLM_GGUF_STRING, "mvlm_gguf_get_array_string: %s holds value type %u", key, et);
    REQUIRE(i < n, "mvlm_gguf_get_array_string: index %llu >= %llu", (unsigned long long)i, (unsigned long long)n);
    for (uint64_t k = 0; k < i; ++k) skip_value(c, MVLM_GGUF_STRING, 0);   // validated at open
    const uint64_t at = c.string(len);
    *str = reinterpret_cast<const char*>(g->base() + at);
    return MVLM_OK;
}

extern "C" int mvlm_ggml_type_size(uint32_t type, uint64_t* block_bytes, uint32_t* block_elems) {
    REQUIRE(block_bytes && block_elems, "mvlm_ggml_type_size: null argument");
    const TypeSize* t = type_size(type);
    if (!t) return set_error(MVLM_ERR_NOT_FOUND, "mvlm_ggml_type_size: unknown ggml type %u", type);
    *block_bytes = t->bytes;
    *block_elems = t->elems;
    return MVLM_OK;
}

extern "C" int mvlm_weight_from_gguf(mvlm_device* dev, const mvlm_gguf* g, uint64_t index, mvlm_weight** out) {
    REQUIRE(dev && g && out, "mvlm_weight_from_gguf: null argument");
    REQUIRE(index < g->tensors.size(), "mvlm_weight_from_gguf: index out of range");
    const auto& t = g->tensors[index];
    REQUIRE(t.n_dims == 2, "mvlm_weight_from_gguf: tensor has %u dims (2 expected: ne0 = K, ne1 = N)", t.n_dims);
    REQUIRE(t.dims[0] <= (uint64_t)INT32_MAX && t.dims[1] <= (uint64_t)INT32_MAX,
            "mvlm_weight_from_gguf: dims too large");
    if (!is_dense((int)t.type) && !is_quant((int)t.type))
        return set_error(MVLM_ERR_UNSUPPORTED, "mvlm_weight_from_gguf: ggml type %u is not packed by this library "
                         "(F32, F16, BF16, Q8_0, Q4_0)", t.type);
    const void* data = g->base() + g->info.data_offset + t.offset;
    return mvlm_weight_pack(dev, data, (int)t.type, MVLM_LAYOUT_NK, (int)t.dims[1], (int)t.dims[0], out);
}
