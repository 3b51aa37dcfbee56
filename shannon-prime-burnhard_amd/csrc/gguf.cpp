// gguf.cpp — GGUF model-file reader of libspq4k (include/spq4k_gguf.h).
//
// Host code only. The file is memory-mapped read-only and parsed in place:
// header, key/value metadata and tensor infos are decoded into tables, and
// tensor data is handed out as pointers into the mapping (no copy), as the
// reference engine's loader does (LlamaWeights::load_cpu_mmap_,
// desktop/engine/src/llama_weights.cpp:441-480, on top of
// gguf_init_from_file with no_alloc, vendor/ggml/src/gguf.cpp:395-850).
//
// Validation follows gguf_init_from_file_ptr rule for rule (gguf.cpp:395-740):
// magic "GGUF"; version 2 or 3 (0, 1, > 3 and byte-swapped versions are
// rejected); tensor and key counts non-negative; keys unique, of a known
// type (arrays of arrays rejected), strings and arrays within 2^30 entries
// and within the file; "general.alignment", when present, a u32 power of two
// (the reference aborts on another type; here it is an error); tensor names
// shorter than 64 bytes and unique; at most 4 dimensions, each
// non-negative, element and byte counts representable; a ggml type whose
// block size is non-zero and divides ne[0]; tensor offsets in file order,
// each the padded end of the one before. One check is added: every tensor's
// bytes lie inside the file, since pointers into the mapping are returned
// (the reference reads no data in its no_alloc mode and checks nothing).
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "spq4k_gguf.h"

namespace {
thread_local char g_err[512];
}

// failure message of the calling thread (also set by the residency code)
namespace spq4k_gguf_detail {
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace spq4k_gguf_detail

namespace {

using spq4k_gguf_detail::fail;

constexpr uint64_t kMaxString = 1ull << 30;   // GGUF_MAX_STRING_LENGTH
constexpr uint64_t kMaxArray = 1ull << 30;    // GGUF_MAX_ARRAY_ELEMENTS
constexpr size_t kMaxName = 64;               // GGML_MAX_NAME
constexpr int kTypeCount = 42;                // GGML_TYPE_COUNT

// ggml's block size and bytes per block of each type id (ggml.c type_traits;
// removed ids have block size 0 and are rejected as the reference does)
struct TypeSize { int64_t blck; size_t size; };
constexpr TypeSize kTypes[kTypeCount] = {
    {1, 4},     {1, 2},     {32, 18},   {32, 20},   {0, 0},     {0, 0},     {32, 22},   // 0 f32 .. 6 q5_0
    {32, 24},   {32, 34},   {32, 36},   {256, 84},  {256, 110}, {256, 144}, {256, 176}, // 7 q5_1 .. 13 q5_K
    {256, 210}, {256, 292}, {256, 66},  {256, 74},  {256, 98},  {256, 50},  {32, 18},   // 14 q6_K .. 20 iq4_nl
    {256, 110}, {256, 82},  {256, 136}, {1, 1},     {1, 2},     {1, 4},     {1, 8},     // 21 iq3_s .. 27 i64
    {1, 8},     {256, 56},  {1, 2},     {0, 0},     {0, 0},     {0, 0},     {256, 54},  // 28 f64 .. 34 tq1_0
    {256, 66},  {0, 0},     {0, 0},     {0, 0},     {32, 17},   {64, 36},   {128, 18},  // 35 tq2_0 .. 41 q1_0
};

// bytes of one value of a GGUF scalar type, 0 for strings and invalid types
size_t kv_scalar_size(int32_t t) {
    switch (t) {
        case SPQ4K_GGUF_UINT8: case SPQ4K_GGUF_INT8: case SPQ4K_GGUF_BOOL: return 1;
        case SPQ4K_GGUF_UINT16: case SPQ4K_GGUF_INT16: return 2;
        case SPQ4K_GGUF_UINT32: case SPQ4K_GGUF_INT32: case SPQ4K_GGUF_FLOAT32: return 4;
        case SPQ4K_GGUF_UINT64: case SPQ4K_GGUF_INT64: case SPQ4K_GGUF_FLOAT64: return 8;
        default: return 0;
    }
}

struct Kv {
    std::string key;
    int32_t type = -1;        // SPQ4K_GGUF_* of the value, or SPQ4K_GGUF_ARRAY
    int32_t arr_type = -1;    // element type of an array
    uint64_t n = 1;           // elements (1 for a scalar)
    std::vector<uint8_t> data;        // scalar values, little-endian, bools as 0 / 1
    std::vector<std::string> strs;    // string values
};

struct Tensor {
    std::string name;
    int32_t type = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;      // within the data section
    uint64_t nbytes = 0;
};

// Bounds-checked little-endian reader over the mapping.
struct Cursor {
    const uint8_t* p;
    uint64_t remain;
    template <typename T>
    bool get(T& v) {
        if (remain < sizeof(T)) return false;
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        remain -= sizeof(T);
        return true;
    }
    bool bytes(void* dst, uint64_t n) {
        if (remain < n) return false;
        if (n) memcpy(dst, p, n);   // an empty array's buffer may be null: no copy at all
        p += n;
        remain -= n;
        return true;
    }
    bool str(std::string& s) {
        uint64_t n = 0;
        if (!get(n) || n > kMaxString || n > remain) return false;
        s.assign(reinterpret_cast<const char*>(p), (size_t)n);
        p += n;
        remain -= n;
        return true;
    }
};

}  // namespace

struct spq4k_gguf {
    int fd = -1;
    void* map = nullptr;
    size_t file_size = 0;
    uint32_t version = 0;
    size_t alignment = 32;
    size_t data_offset = 0;
    size_t data_size = 0;
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> tindex;
    std::unordered_map<std::string, int64_t> kindex;
};

namespace {

int parse(spq4k_gguf* g) {
    Cursor c{static_cast<const uint8_t*>(g->map), g->file_size};
    char magic[4];
    if (!c.bytes(magic, 4)) return fail(-EINVAL, "gguf: failed to read magic");
    if (memcmp(magic, "GGUF", 4) != 0) return fail(-EINVAL, "gguf: invalid magic");
    if (!c.get(g->version)) return fail(-EINVAL, "gguf: failed to read header");
    if (g->version == 0) return fail(-EINVAL, "gguf: bad version 0");
    if ((g->version & 0xFFFFu) == 0) return fail(-EINVAL, "gguf: version %u (byte-swapped file?)", g->version);
    if (g->version == 1) return fail(-EINVAL, "gguf: version 1 is not supported");
    if (g->version > 3) return fail(-EINVAL, "gguf: version %u is newer than 3", g->version);
    int64_t n_tensors = 0, n_kv = 0;
    if (!c.get(n_tensors) || !c.get(n_kv)) return fail(-EINVAL, "gguf: failed to read header");
    // every tensor info and key needs at least 8 bytes: counts beyond the file are malformed
    if (n_tensors < 0 || (uint64_t)n_tensors > c.remain / 8) return fail(-EINVAL, "gguf: bad tensor count %lld", (long long)n_tensors);
    if (n_kv < 0 || (uint64_t)n_kv > c.remain / 8) return fail(-EINVAL, "gguf: bad key count %lld", (long long)n_kv);

    g->kv.reserve((size_t)n_kv);
    for (int64_t i = 0; i < n_kv; ++i) {
        Kv kv;
        if (!c.str(kv.key)) return fail(-EINVAL, "gguf: failed to read key %lld", (long long)i);
        if (g->kindex.count(kv.key)) return fail(-EINVAL, "gguf: duplicate key '%s'", kv.key.c_str());
        int32_t t = -1;
        if (!c.get(t)) return fail(-EINVAL, "gguf: failed to read the type of key '%s'", kv.key.c_str());
        int32_t et = t;
        if (t == SPQ4K_GGUF_ARRAY) {
            if (!c.get(et) || !c.get(kv.n)) return fail(-EINVAL, "gguf: failed to read array '%s'", kv.key.c_str());
            if (kv.n > kMaxArray) return fail(-EINVAL, "gguf: array '%s' too long", kv.key.c_str());
        }
        if (et == SPQ4K_GGUF_STRING) {
            if (kv.n > c.remain / 8) return fail(-EINVAL, "gguf: array '%s' exceeds the file", kv.key.c_str());
            kv.strs.resize((size_t)kv.n);
            for (uint64_t j = 0; j < kv.n; ++j)
                if (!c.str(kv.strs[j])) return fail(-EINVAL, "gguf: failed to read the value of '%s'", kv.key.c_str());
        } else {
            const size_t es = kv_scalar_size(et);
            if (es == 0) return fail(-EINVAL, "gguf: key '%s' has invalid type %d", kv.key.c_str(), et);
            if (kv.n > c.remain / es) return fail(-EINVAL, "gguf: value of '%s' exceeds the file", kv.key.c_str());
            kv.data.resize((size_t)(kv.n * es));
            if (!c.bytes(kv.data.data(), kv.n * es)) return fail(-EINVAL, "gguf: failed to read '%s'", kv.key.c_str());
            if (et == SPQ4K_GGUF_BOOL)
                for (auto& b : kv.data) b = b != 0;
        }
        kv.type = t;
        kv.arr_type = t == SPQ4K_GGUF_ARRAY ? et : -1;
        g->kindex.emplace(kv.key, i);
        g->kv.push_back(std::move(kv));
    }
    auto al = g->kindex.find("general.alignment");
    if (al != g->kindex.end()) {
        const Kv& kv = g->kv[(size_t)al->second];
        if (kv.type != SPQ4K_GGUF_UINT32) return fail(-EINVAL, "gguf: general.alignment is not a u32");
        uint32_t a;
        memcpy(&a, kv.data.data(), 4);
        g->alignment = a;
    }
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1)) != 0)
        return fail(-EINVAL, "gguf: alignment %zu is not a power of 2", g->alignment);

    g->tensors.reserve((size_t)n_tensors);
    for (int64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        if (!c.str(t.name)) return fail(-EINVAL, "gguf: failed to read tensor name %lld", (long long)i);
        if (t.name.size() >= kMaxName) return fail(-EINVAL, "gguf: tensor name %lld too long", (long long)i);
        if (g->tindex.count(t.name)) return fail(-EINVAL, "gguf: duplicate tensor name '%s'", t.name.c_str());
        uint32_t n_dims = 0;
        if (!c.get(n_dims)) return fail(-EINVAL, "gguf: failed to read tensor info");
        if (n_dims > 4) return fail(-EINVAL, "gguf: tensor '%s' has %u dimensions", t.name.c_str(), n_dims);
        for (uint32_t j = 0; j < n_dims; ++j) {
            if (!c.get(t.ne[j])) return fail(-EINVAL, "gguf: failed to read tensor info");
            if (t.ne[j] < 0) return fail(-EINVAL, "gguf: tensor '%s' has a negative dimension", t.name.c_str());
        }
        // the element count is representable (the reference's test, zero dimensions included)
        const int64_t* ne = t.ne;
        if (ne[1] == 0 || ne[2] == 0 || ne[3] == 0 ? false
            : (INT64_MAX / ne[1] <= ne[0] || INT64_MAX / ne[2] <= ne[0] * ne[1] ||
               INT64_MAX / ne[3] <= ne[0] * ne[1] * ne[2]))
            return fail(-EINVAL, "gguf: tensor '%s' has too many elements", t.name.c_str());
        if (!c.get(t.type)) return fail(-EINVAL, "gguf: failed to read tensor info");
        if (t.type < 0 || t.type >= kTypeCount) return fail(-EINVAL, "gguf: tensor '%s' has invalid type %d", t.name.c_str(), t.type);
        const TypeSize ts = kTypes[t.type];
        if (ts.blck == 0 || ne[0] % ts.blck != 0)
            return fail(-EINVAL, "gguf: tensor '%s' row of %lld is not whole blocks of type %d", t.name.c_str(),
                        (long long)ne[0], t.type);
        const uint64_t nel = (uint64_t)ne[0] * (uint64_t)ne[1] * (uint64_t)ne[2] * (uint64_t)ne[3];
        if (nel / (uint64_t)ts.blck > SIZE_MAX / ts.size) return fail(-EINVAL, "gguf: tensor '%s' too large", t.name.c_str());
        t.nbytes = nel / (uint64_t)ts.blck * ts.size;
        if (!c.get(t.offset)) return fail(-EINVAL, "gguf: failed to read tensor info");
        g->tindex.emplace(t.name, i);
        g->tensors.push_back(std::move(t));
    }
    const size_t pos = g->file_size - (size_t)c.remain;
    g->data_offset = (pos + g->alignment - 1) / g->alignment * g->alignment;
    uint64_t size = 0, end = 0;
    for (const Tensor& t : g->tensors) {
        if (t.offset != size) return fail(-EINVAL, "gguf: tensor '%s' has offset %llu, expected %llu", t.name.c_str(),
                                          (unsigned long long)t.offset, (unsigned long long)size);
        const uint64_t padded = (t.nbytes + g->alignment - 1) / g->alignment * g->alignment;
        if (padded < t.nbytes || UINT64_MAX - size < padded) return fail(-EINVAL, "gguf: tensor '%s' size overflow", t.name.c_str());
        end = size + t.nbytes;
        size += padded;
    }
    g->data_size = (size_t)size;
    if (!g->tensors.empty() && (g->data_offset > g->file_size || end > g->file_size - g->data_offset))
        return fail(-EINVAL, "gguf: tensor data ends at %llu, beyond the file (%zu bytes)",
                    (unsigned long long)(g->data_offset + end), g->file_size);
    return 0;
}

bool bad(const spq4k_gguf* g, int64_t i, size_t n) { return !g || i < 0 || (uint64_t)i >= n; }

}  // namespace

extern "C" {

const char* spq4k_gguf_strerror(void) { return g_err; }

int spq4k_gguf_open(const char* path, spq4k_gguf** out) {
    if (!out) return fail(-EINVAL, "gguf: null out");
    *out = nullptr;
    if (!path) return fail(-EINVAL, "gguf: null path");
    spq4k_gguf* g = new (std::nothrow) spq4k_gguf();
    if (!g) return fail(-ENOMEM, "gguf: out of memory");
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        const int e = errno;
        delete g;
        return fail(-e, "gguf: cannot open %s: %s", path, strerror(e));
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 0) {
        const int e = errno;
        close(g->fd);
        delete g;
        return fail(-e, "gguf: cannot stat %s", path);
    }
    g->file_size = (size_t)st.st_size;
    if (g->file_size > 0) {
        g->map = mmap(nullptr, g->file_size, PROT_READ, MAP_PRIVATE, g->fd, 0);
        if (g->map == MAP_FAILED) {
            const int e = errno;
            g->map = nullptr;
            close(g->fd);
            delete g;
            return fail(-e, "gguf: cannot map %s", path);
        }
    }
    int rc = g->file_size > 0 ? parse(g) : fail(-EINVAL, "gguf: empty file");
    if (rc) {
        spq4k_gguf_close(g);
        return rc;
    }
    *out = g;
    return 0;
}

void spq4k_gguf_close(spq4k_gguf* g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->file_size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

uint32_t spq4k_gguf_version(const spq4k_gguf* g) { return g ? g->version : 0; }
size_t spq4k_gguf_alignment(const spq4k_gguf* g) { return g ? g->alignment : 0; }
size_t spq4k_gguf_data_offset(const spq4k_gguf* g) { return g ? g->data_offset : 0; }
size_t spq4k_gguf_data_size(const spq4k_gguf* g) { return g ? g->data_size : 0; }
size_t spq4k_gguf_file_size(const spq4k_gguf* g) { return g ? g->file_size : 0; }

int64_t spq4k_gguf_n_kv(const spq4k_gguf* g) { return g ? (int64_t)g->kv.size() : -1; }

int64_t spq4k_gguf_find_key(const spq4k_gguf* g, const char* key) {
    if (!g || !key) return -1;
    auto it = g->kindex.find(key);
    return it == g->kindex.end() ? -1 : it->second;
}

const char* spq4k_gguf_key(const spq4k_gguf* g, int64_t i) { return bad(g, i, g ? g->kv.size() : 0) ? nullptr : g->kv[i].key.c_str(); }

int spq4k_gguf_kv_type(const spq4k_gguf* g, int64_t i) { return bad(g, i, g ? g->kv.size() : 0) ? -EINVAL : g->kv[i].type; }

int spq4k_gguf_arr_type(const spq4k_gguf* g, int64_t i) {
    if (bad(g, i, g ? g->kv.size() : 0) || g->kv[i].type != SPQ4K_GGUF_ARRAY) return -EINVAL;
    return g->kv[i].arr_type;
}

int64_t spq4k_gguf_arr_n(const spq4k_gguf* g, int64_t i) { return bad(g, i, g ? g->kv.size() : 0) ? -EINVAL : (int64_t)g->kv[i].n; }

const void* spq4k_gguf_val_data(const spq4k_gguf* g, int64_t i) {
    if (bad(g, i, g ? g->kv.size() : 0) || !g->kv[i].strs.empty() || g->kv[i].data.empty()) return nullptr;
    return g->kv[i].data.data();
}

const char* spq4k_gguf_val_str(const spq4k_gguf* g, int64_t i, int64_t j) {
    if (bad(g, i, g ? g->kv.size() : 0) || j < 0 || (uint64_t)j >= g->kv[i].strs.size()) return nullptr;
    return g->kv[i].strs[(size_t)j].c_str();
}

int64_t spq4k_gguf_n_tensors(const spq4k_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int64_t spq4k_gguf_find_tensor(const spq4k_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->tindex.find(name);
    return it == g->tindex.end() ? -1 : it->second;
}

const char* spq4k_gguf_tensor_name(const spq4k_gguf* g, int64_t i) {
    return bad(g, i, g ? g->tensors.size() : 0) ? nullptr : g->tensors[i].name.c_str();
}

int spq4k_gguf_tensor_type(const spq4k_gguf* g, int64_t i) {
    return bad(g, i, g ? g->tensors.size() : 0) ? -EINVAL : g->tensors[i].type;
}

int spq4k_gguf_tensor_shape(const spq4k_gguf* g, int64_t i, int64_t ne[4]) {
    if (bad(g, i, g ? g->tensors.size() : 0) || !ne) return -EINVAL;
    int n = 1;
    for (int j = 0; j < 4; ++j) {
        ne[j] = g->tensors[i].ne[j];
        if (ne[j] != 1) n = j + 1;
    }
    return n;   // ggml_n_dims: dimensions up to the last one that is not 1
}

size_t spq4k_gguf_tensor_offset(const spq4k_gguf* g, int64_t i) {
    return bad(g, i, g ? g->tensors.size() : 0) ? 0 : (size_t)g->tensors[i].offset;
}

size_t spq4k_gguf_tensor_nbytes(const spq4k_gguf* g, int64_t i) {
    return bad(g, i, g ? g->tensors.size() : 0) ? 0 : (size_t)g->tensors[i].nbytes;
}

const void* spq4k_gguf_tensor_data(const spq4k_gguf* g, int64_t i) {
    if (bad(g, i, g ? g->tensors.size() : 0)) return nullptr;
    return static_cast<const uint8_t*>(g->map) + g->data_offset + g->tensors[i].offset;
}

}  // extern "C"
