// gguf.cpp -- the GGUF reader (include/gguf_mmap.h): parse a version-3 file (and its splits) from a read-only
// mapping, answer the reference's introspection calls, stage tensors into HBM, and bind weights for the matvecs.
//
// Follows the reference's src/gguf_mmap.cpp for every observable result (key/value widening rules, size formulas,
// legacy key lists, split naming) and src/inference.cpp:362-389 for bind_weight. Different by design:
//   * bounds: every read of the header, keys, arrays and tensor table is checked against the file size, and each
//     tensor's data extent against its file; a file that fails is refused at open (NULL);
//   * lookup: tensors and keys by name through hash maps (the reference scans the tables per call);
//   * residency: gguf_hbm_stage copies tensors into caller-owned device memory through a ring of pinned host
//     buffers filled by several threads, where the reference pins the host mapping for zero-copy reads.
#include "gguf_mmap.h"
#include "quant_types.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

constexpr uint32_t GGUF_V3 = 3;
constexpr size_t GGUF_DEFAULT_ALIGN = 32;
constexpr int MAX_SPLITS = 64;  // as the reference's GGUF_MAX_SPLITS
constexpr size_t NAME_MAX_CHARS = 63;  // the reference keeps tensor names in char[64]

enum : int {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7, T_STRING = 8,
    T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

size_t scalar_bytes(int t) {
    switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    }
    return 0;
}

// GGML block geometry (values per block, bytes per block) of every type id a GGUF may hold: the public format's
// table, the same entries as the reference's qt_traits (src/quant_types.cpp:586-614)
struct Geo {
    int type, blck, bytes;
};
constexpr Geo k_geo[] = {
    {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},   {8, 32, 34},
    {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {16, 256, 66}, {17, 256, 74},
    {18, 256, 98}, {19, 256, 50}, {20, 32, 18},  {21, 256, 110}, {22, 256, 82}, {23, 256, 136}, {29, 256, 56},
    {30, 1, 2},    {34, 256, 54}, {35, 256, 66}, {39, 32, 17},  {40, 64, 36},  {100, 32, 18}, {101, 32, 17},
};
const Geo *geo(int type) {
    for (const Geo &g : k_geo)
        if (g.type == type) return &g;
    return nullptr;
}

struct Tensor {
    char name[NAME_MAX_CHARS + 1];
    uint8_t n_dims;
    int64_t ne[4];  // entries past n_dims stay 0
    int type;
    uint64_t offset;  // from its file's data start
    int split;
    const void *staged;
};

struct Kv {
    std::string key;
    bool is_array = false;
    int type = 0;       // scalar: its type; array: the element type
    uint64_t raw = 0;   // scalar bits (little-endian, zero-extended)
    std::string str;    // string scalar
    bool has_str = false;
    std::vector<std::string> strs;  // string array
    std::vector<const char *> strp;  // pointers into strs (what the string-array getters hand out)
    const void *arr = nullptr;       // numeric array, in the mapping
    uint64_t arr_n = 0;
};

struct File {
    void *map = nullptr;
    size_t size = 0;
    size_t data_off = 0;
    std::string path;
    uint64_t id[4] = {0, 0, 0, 0};
    int fd_remap = -1;
};

}  // namespace

struct gguf_model {
    uint32_t version = 0;
    size_t alignment = GGUF_DEFAULT_ALIGN;
    std::vector<Tensor> tensors;
    std::vector<Kv> kvs;
    std::unordered_map<std::string, int64_t> tensor_idx, kv_idx;
    std::vector<File> files;
    // the reference returns these strings from static buffers; here they live with the model
    std::string arch_s, vocab_s, pre_s;
};

namespace {

// bounds-checked little-endian reader over [p, end)
struct Rd {
    const uint8_t *p, *end;
    bool ok = true;
    bool take(void *dst, size_t n) {
        if (!ok || (size_t)(end - p) < n) return ok = false;
        memcpy(dst, p, n);
        p += n;
        return true;
    }
    template <typename T>
    T get() {
        T v{};
        take(&v, sizeof v);
        return v;
    }
    bool str(std::string &s) {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1ull << 30) || (uint64_t)(end - p) < n) return ok = false;  // (the reference's 1 GiB cap)
        s.assign((const char *)p, (size_t)n);
        p += n;
        return true;
    }
    bool skip(uint64_t n) {
        if (!ok || (uint64_t)(end - p) < n) return ok = false;
        p += n;
        return true;
    }
};

void *map_readonly(const char *path, size_t &size, uint64_t id[4]) {
    struct stat st;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return nullptr;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return nullptr;
    }
    size = (size_t)st.st_size;
    void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return nullptr;
    id[0] = (uint64_t)st.st_dev;
    id[1] = (uint64_t)st.st_ino;
    id[2] = (uint64_t)st.st_size;
    id[3] = (uint64_t)st.st_mtim.tv_sec * 1000000000ull + (uint64_t)st.st_mtim.tv_nsec;
    return m;
}

int64_t kv_int(const Kv &k) {  // the reference's kv_as_int64
    if (k.is_array) return 0;
    switch (k.type) {
    case T_U8: return (int64_t)(uint8_t)k.raw;
    case T_I8: return (int64_t)(int8_t)k.raw;
    case T_U16: return (int64_t)(uint16_t)k.raw;
    case T_I16: return (int64_t)(int16_t)k.raw;
    case T_U32: return (int64_t)(uint32_t)k.raw;
    case T_I32: return (int64_t)(int32_t)k.raw;
    case T_U64: return (int64_t)k.raw;
    case T_I64: return (int64_t)k.raw;
    case T_BOOL: return (uint8_t)k.raw ? 1 : 0;
    }
    return 0;
}

// one file: header, keys, tensor table; tensors tagged with `split`
bool parse_file(gguf_model *m, const char *path, int split, std::vector<Kv> *kvs_out) {
    File f;
    f.path = path;
    f.map = map_readonly(path, f.size, f.id);
    if (!f.map) return false;
    const uint8_t *base = (const uint8_t *)f.map;
    Rd r{base, base + f.size};
    char magic[4];
    r.take(magic, 4);
    const uint32_t version = r.get<uint32_t>();
    const int64_t n_tensors = r.get<int64_t>(), n_kv = r.get<int64_t>();
    bool good = r.ok && memcmp(magic, "GGUF", 4) == 0 && version == GGUF_V3 && n_tensors >= 0 && n_kv >= 0 &&
                (uint64_t)n_tensors <= f.size && (uint64_t)n_kv <= f.size;
    std::vector<Kv> kvs;
    size_t alignment = GGUF_DEFAULT_ALIGN;
    for (int64_t i = 0; good && i < n_kv; ++i) {
        Kv k;
        r.str(k.key);
        const int32_t t = r.get<int32_t>();
        if (!r.ok) break;
        if (t == T_STRING) {
            k.type = T_STRING;
            k.has_str = r.str(k.str);
        } else if (t == T_ARRAY) {
            const int32_t et = r.get<int32_t>();
            const uint64_t n = r.get<uint64_t>();
            k.is_array = true;
            k.type = et;
            k.arr_n = n;
            if (et == T_STRING) {
                if (n > f.size) r.ok = false;
                for (uint64_t j = 0; r.ok && j < n; ++j) {
                    std::string s;
                    if (r.str(s)) k.strs.push_back(std::move(s));
                }
                for (const std::string &s : k.strs) k.strp.push_back(s.c_str());
            } else {
                const size_t es = scalar_bytes(et);
                if (!es || n > f.size / es) {
                    r.ok = false;
                } else {
                    k.arr = r.p;
                    r.skip(n * es);
                }
            }
        } else {
            const size_t es = scalar_bytes(t);
            k.type = t;
            if (!es) r.ok = false;
            else r.take(&k.raw, es);
            if (r.ok && k.key == "general.alignment") alignment = (size_t)(uint32_t)k.raw;  // (read as u32, as the reference)
        }
        if (r.ok) kvs.push_back(std::move(k));
    }
    good = good && r.ok && alignment > 0 && (alignment & (alignment - 1)) == 0;
    std::vector<Tensor> ts;
    for (int64_t i = 0; good && i < n_tensors; ++i) {
        Tensor t{};
        std::string name;
        r.str(name);
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd < 1 || nd > 4) {
            good = false;
            break;
        }
        const size_t nl = std::min(name.size(), NAME_MAX_CHARS);
        memcpy(t.name, name.data(), nl);
        t.name[nl] = '\0';
        t.n_dims = (uint8_t)nd;
        for (uint32_t d = 0; d < nd; ++d) t.ne[d] = r.get<int64_t>();
        t.type = r.get<int32_t>();
        t.offset = r.get<uint64_t>();
        t.split = split;
        good = r.ok;
        for (uint32_t d = 0; good && d < nd; ++d) good = t.ne[d] >= 0;
        if (good) ts.push_back(t);
    }
    if (good) {
        const size_t hdr = (size_t)(r.p - base);
        f.data_off = (hdr + alignment - 1) & ~(alignment - 1);
        good = f.data_off <= f.size;
        // each tensor's data inside its file (types without a known size are not checked)
        for (const Tensor &t : ts) {
            const Geo *g = geo(t.type);
            if (!good || !g) continue;
            __int128 n = 1;
            for (int d = 0; d < t.n_dims; ++d) n *= t.ne[d];
            const __int128 bytes = (n + g->blck - 1) / g->blck * g->bytes;
            good = (__int128)t.offset + bytes <= (__int128)(f.size - f.data_off);
        }
    }
    if (!good) {
        munmap(f.map, f.size);
        return false;
    }
    if (split == 0) {
        m->version = version;
        m->alignment = alignment;
    }
    for (Tensor &t : ts) m->tensors.push_back(t);
    m->files.push_back(std::move(f));
    *kvs_out = std::move(kvs);
    return true;
}

void free_model(gguf_model *m) {
    for (File &f : m->files) {
        if (f.map) munmap(f.map, f.size);
        if (f.fd_remap >= 0) close(f.fd_remap);
    }
    delete m;
}

int64_t find_kv(const gguf_model *m, const char *key) {
    if (!m || !key) return -1;
    const auto it = m->kv_idx.find(key);
    return it == m->kv_idx.end() ? -1 : it->second;
}

// "<general.architecture>.<suffix>" first, then the legacy keys in order
int64_t find_arch(const gguf_model *m, const char *suffix, std::initializer_list<const char *> legacy) {
    const int64_t a = find_kv(m, "general.architecture");
    if (a >= 0 && m->kvs[a].has_str && !m->kvs[a].str.empty()) {
        const int64_t i = find_kv(m, (m->kvs[a].str + "." + suffix).c_str());
        if (i >= 0) return i;
    }
    for (const char *k : legacy) {
        const int64_t i = find_kv(m, k);
        if (i >= 0) return i;
    }
    return -1;
}

const Kv *scalar_kv(const gguf_model *m, int64_t idx, const void *out) {
    if (!m || !out || idx < 0 || idx >= (int64_t)m->kvs.size() || m->kvs[idx].is_array) return nullptr;
    return &m->kvs[idx];
}

bool in_range(const gguf_model *m, int64_t idx) { return m && idx >= 0 && idx < (int64_t)m->tensors.size(); }

size_t tensor_bytes_ceil(const Tensor &t) {  // gguf_get_tensor_ptr's size: ceil(elements / block) blocks
    const Geo *g = geo(t.type);
    int64_t n = t.ne[0];
    for (int d = 1; d < t.n_dims; ++d) n *= t.ne[d];
    if (!g) return (size_t)-1;
    return (size_t)((n + g->blck - 1) / g->blck) * (size_t)g->bytes;
}

const char *str_or_empty(const gguf_model *m, int64_t idx, std::string &buf) {
    if (idx >= 0 && m->kvs[idx].has_str && !m->kvs[idx].str.empty()) {
        buf = m->kvs[idx].str.substr(0, 127);  // (the reference copies into 128-byte buffers)
        return buf.c_str();
    }
    return nullptr;
}

}  // namespace

extern "C" {

gguf_model_t *gguf_mmap_open(const char *path) {
    if (!path) return nullptr;
    gguf_model *m = new gguf_model();
    std::vector<Kv> kvs;
    if (!parse_file(m, path, 0, &kvs)) {
        free_model(m);
        return nullptr;
    }
    m->kvs = std::move(kvs);
    for (int64_t i = 0; i < (int64_t)m->kvs.size(); ++i) m->kv_idx.emplace(m->kvs[i].key, i);  // (first wins)
    // a split model: <prefix>-00001-of-<count>.gguf, then the others, each with split.no = its index
    const int64_t sc = find_kv(m, "split.count");
    const int64_t count = sc < 0 ? 1 : kv_int(m->kvs[sc]);
    if (count > 1) {
        char suffix[64];
        snprintf(suffix, sizeof suffix, "-00001-of-%05d.gguf", (int)count);
        const std::string p(path), sfx(suffix);
        if (count > MAX_SPLITS || p.size() < sfx.size() || p.compare(p.size() - sfx.size(), sfx.size(), sfx) != 0) {
            free_model(m);
            return nullptr;
        }
        for (int i = 1; i < count; ++i) {
            char part[64];
            snprintf(part, sizeof part, "-%05d-of-%05d.gguf", i + 1, (int)count);
            const std::string sub = p.substr(0, p.size() - sfx.size()) + part;
            std::vector<Kv> skv;
            bool ok = parse_file(m, sub.c_str(), i, &skv);
            if (ok) {
                int64_t no = -1;
                for (const Kv &k : skv)
                    if (k.key == "split.no") {
                        no = kv_int(k);
                        break;
                    }
                ok = no == i;
            }
            if (!ok) {
                free_model(m);
                return nullptr;
            }
        }
    }
    for (int64_t i = 0; i < (int64_t)m->tensors.size(); ++i) m->tensor_idx.emplace(m->tensors[i].name, i);
    return m;
}

void gguf_mmap_close(gguf_model_t *model) {
    if (model) free_model(model);
}

const void *gguf_get_tensor_ptr(const gguf_model_t *m, const char *name, size_t *out_bytes) {
    if (!m || !name || !out_bytes) return nullptr;
    const auto it = m->tensor_idx.find(name);
    if (it == m->tensor_idx.end()) return nullptr;
    const Tensor &t = m->tensors[it->second];
    *out_bytes = tensor_bytes_ceil(t);
    if (t.staged) return t.staged;
    const File &f = m->files[t.split];
    return (const char *)f.map + f.data_off + t.offset;
}

const void *gguf_mmap_get_tensor(const gguf_model_t *m, const char *name, size_t *out_bytes) {
    return gguf_get_tensor_ptr(m, name, out_bytes);
}

int64_t gguf_n_tensors(const gguf_model_t *m) { return m ? (int64_t)m->tensors.size() : 0; }
const char *gguf_tensor_name(const gguf_model_t *m, int64_t idx) {
    return in_range(m, idx) ? m->tensors[idx].name : "(null)";
}
int gguf_tensor_type(const gguf_model_t *m, int64_t idx) { return in_range(m, idx) ? m->tensors[idx].type : -1; }
int64_t *gguf_tensor_ne(const gguf_model_t *m, int64_t idx) {
    return in_range(m, idx) ? const_cast<int64_t *>(m->tensors[idx].ne) : nullptr;
}
uint8_t gguf_tensor_dims(const gguf_model_t *m, int64_t idx) { return in_range(m, idx) ? m->tensors[idx].n_dims : 0; }
size_t gguf_tensor_block_size(const gguf_model_t *m, int64_t idx) {
    if (!in_range(m, idx)) return (size_t)-1;
    const Geo *g = geo(m->tensors[idx].type);
    return g ? (size_t)g->blck : (size_t)-1;
}
size_t gguf_tensor_type_size(const gguf_model_t *m, int64_t idx) {
    if (!in_range(m, idx)) return (size_t)-1;
    const Geo *g = geo(m->tensors[idx].type);
    return g ? (size_t)g->bytes : (size_t)-1;
}
size_t gguf_tensor_row_size(const gguf_model_t *m, int64_t idx) {
    if (!in_range(m, idx)) return (size_t)-1;
    const Geo *g = geo(m->tensors[idx].type);
    if (!g) return (size_t)-1;
    const size_t nb = (size_t)((m->tensors[idx].ne[0] + g->blck - 1) / g->blck);
    return (nb * (size_t)g->bytes + GGUF_DEFAULT_ALIGN - 1) & ~(GGUF_DEFAULT_ALIGN - 1);
}
uint64_t gguf_tensor_offset(const gguf_model_t *m, int64_t idx) {
    return in_range(m, idx) ? m->tensors[idx].offset : UINT64_MAX;
}
size_t gguf_tensor_nbytes(const gguf_model_t *m, int64_t idx) {
    if (!in_range(m, idx)) return (size_t)-1;
    const Tensor &t = m->tensors[idx];
    const Geo *g = geo(t.type);
    if (!g) return (size_t)-1;
    int64_t n = 1;
    for (int d = 0; d < t.n_dims; ++d) n *= t.ne[d];
    return (size_t)(n / g->blck) * (size_t)g->bytes;
}
size_t gguf_tensor_nbytes_pad(const gguf_model_t *m, int64_t idx) { return gguf_tensor_nbytes(m, idx); }

int64_t gguf_n_kv(const gguf_model_t *m) { return m ? (int64_t)m->kvs.size() : 0; }
const char *gguf_kv_key(const gguf_model_t *m, int64_t idx) {
    return m && idx >= 0 && idx < (int64_t)m->kvs.size() ? m->kvs[idx].key.c_str() : "(null)";
}
int gguf_kv_type(const gguf_model_t *m, int64_t idx) {
    return m && idx >= 0 && idx < (int64_t)m->kvs.size() ? m->kvs[idx].type : -1;
}

// The scalar getters: which stored types each accepts and how it converts them (src/gguf_mmap.cpp:527-671).
#define KV_SCALAR(k) const Kv *k = scalar_kv(m, idx, out); if (!k) return -1
int32_t gguf_kv_get_u8(const gguf_model_t *m, int64_t idx, uint8_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_U8: case T_I8: *out = (uint8_t)k->raw; return 0;
    case T_BOOL: *out = (uint8_t)k->raw ? 1 : 0; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_i8(const gguf_model_t *m, int64_t idx, int8_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_U8: case T_I8: *out = (int8_t)k->raw; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_u16(const gguf_model_t *m, int64_t idx, uint16_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_U8: *out = (uint8_t)k->raw; return 0;
    case T_I8: *out = (uint16_t)(int8_t)k->raw; return 0;
    case T_U16: case T_I16: *out = (uint16_t)k->raw; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_i16(const gguf_model_t *m, int64_t idx, int16_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_I8: *out = (int8_t)k->raw; return 0;
    case T_U8: *out = (int16_t)(uint8_t)k->raw; return 0;
    case T_I16: case T_U16: *out = (int16_t)(uint16_t)k->raw; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_u32(const gguf_model_t *m, int64_t idx, uint32_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_U8: *out = (uint8_t)k->raw; return 0;
    case T_I8: *out = (uint32_t)(int8_t)k->raw; return 0;
    case T_U16: *out = (uint16_t)k->raw; return 0;
    case T_I16: *out = (uint32_t)(int16_t)k->raw; return 0;
    case T_U32: case T_I32: *out = (uint32_t)k->raw; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_i32(const gguf_model_t *m, int64_t idx, int32_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_U8: *out = (uint8_t)k->raw; return 0;
    case T_I8: *out = (int8_t)k->raw; return 0;
    case T_U16: *out = (uint16_t)k->raw; return 0;
    case T_I16: *out = (int16_t)k->raw; return 0;
    case T_U32: case T_I32: *out = (int32_t)(uint32_t)k->raw; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_f32(const gguf_model_t *m, int64_t idx, float *out) {
    KV_SCALAR(k);
    if (k->type != T_F32) return -1;
    const uint32_t b = (uint32_t)k->raw;
    memcpy(out, &b, 4);
    return 0;
}
int32_t gguf_kv_get_u64(const gguf_model_t *m, int64_t idx, uint64_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_U8: *out = (uint8_t)k->raw; return 0;
    case T_I8: *out = (uint64_t)(uint8_t)k->raw; return 0;  // (zero-extended, as the reference)
    case T_U16: *out = (uint16_t)k->raw; return 0;
    case T_I16: *out = (uint64_t)(int16_t)k->raw; return 0;
    case T_U32: *out = (uint32_t)k->raw; return 0;
    case T_I32: *out = (uint64_t)(int32_t)k->raw; return 0;
    case T_U64: *out = k->raw; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_i64(const gguf_model_t *m, int64_t idx, int64_t *out) {
    KV_SCALAR(k);
    switch (k->type) {
    case T_U8: *out = (uint8_t)k->raw; return 0;
    case T_I8: *out = (int8_t)k->raw; return 0;
    case T_U16: *out = (uint16_t)k->raw; return 0;
    case T_I16: *out = (int16_t)k->raw; return 0;
    case T_U32: *out = (int64_t)(uint32_t)k->raw; return 0;
    case T_I32: *out = (int32_t)k->raw; return 0;
    case T_U64: case T_I64: *out = (int64_t)k->raw; return 0;
    }
    return -1;
}
int32_t gguf_kv_get_f64(const gguf_model_t *m, int64_t idx, double *out) {
    KV_SCALAR(k);
    if (k->type == T_F32) {
        float f;
        const uint32_t b = (uint32_t)k->raw;
        memcpy(&f, &b, 4);
        *out = (double)f;
        return 0;
    }
    if (k->type == T_F64) {
        memcpy(out, &k->raw, 8);
        return 0;
    }
    return -1;
}
#undef KV_SCALAR

const char *gguf_kv_str_val(const gguf_model_t *m, int64_t idx) {
    if (!m || idx < 0 || idx >= (int64_t)m->kvs.size()) return nullptr;
    const Kv &k = m->kvs[idx];
    if (!k.is_array && k.type != T_STRING) return nullptr;
    return k.has_str ? k.str.c_str() : "";  // (an array gives "", as the reference)
}

size_t gguf_alignment(const gguf_model_t *m) { return m ? m->alignment : GGUF_DEFAULT_ALIGN; }
size_t gguf_data_offset(const gguf_model_t *m) { return m && !m->files.empty() ? m->files[0].data_off : 0; }
uint32_t gguf_version(const gguf_model_t *m) { return m ? m->version : 0; }

const char *gguf_arch(const gguf_model_t *m) {
    if (!m) return "(unknown)";
    gguf_model *w = const_cast<gguf_model *>(m);
    if (const char *s = str_or_empty(m, find_kv(m, "general.architecture"), w->arch_s)) return s;
    for (const char *k : {"tokenizer.ggml.model", "llmark", "backpack"}) {  // (the reference's fallbacks, in order)
        const int64_t i = find_kv(m, k);
        if (i >= 0) {
            const char *s = str_or_empty(m, i, w->arch_s);
            return s ? s : "(unknown)";
        }
    }
    return "(unknown)";
}
const char *gguf_vocab_name(const gguf_model_t *m) {
    if (!m) return "";
    const char *s = str_or_empty(m, find_kv(m, "tokenizer.ggml.model"), const_cast<gguf_model *>(m)->vocab_s);
    return s ? s : "";
}
const char *gguf_tokenizer_type(const gguf_model_t *m) { return gguf_vocab_name(m); }
const char *gguf_pre_type(const gguf_model_t *m) {
    if (!m) return "";
    int64_t i = find_kv(m, "tokenizer.ggml.pre");
    if (i < 0) i = find_kv(m, "preprocessing");
    const char *s = str_or_empty(m, i, const_cast<gguf_model *>(m)->pre_s);
    return s ? s : "";
}
int64_t gguf_vocab_size(const gguf_model_t *m) {
    for (const char *k : {"tokenizer.ggml.vocab_size", "tokenizer_vocab_size", "vocab_size"}) {
        const int64_t i = find_kv(m, k);
        if (i >= 0) return kv_int(m->kvs[i]);
    }
    return 0;
}
int64_t gguf_head_count(const gguf_model_t *m) {
    const int64_t i = find_arch(m, "attention.head_count",
                                {"attention.head_count", "qwen35.attention.head_count", "llama.attention.heads"});
    return i < 0 ? 0 : kv_int(m->kvs[i]);
}
int64_t gguf_head_count_kv(const gguf_model_t *m) {
    const int64_t i = find_arch(m, "attention.head_count_kv",
                                {"attention.head_count_kv", "qwen35.attention.head_count_kv",
                                 "llama.attention.heads_kv", "attention.kv_heads"});
    return i < 0 ? 0 : kv_int(m->kvs[i]);
}
int64_t gguf_context_length(const gguf_model_t *m) {
    const int64_t i = find_arch(m, "context_length",
                                {"general.context_length", "qwen35.context_length", "qwen2.context_length",
                                 "context_length", "llama.context_length"});
    return i < 0 ? 0 : kv_int(m->kvs[i]);
}
int64_t gguf_embedding_length(const gguf_model_t *m) {
    const int64_t i = find_arch(m, "embedding_length",
                                {"embedding_length", "qwen35.embedding_length", "qwen2.embedding_length",
                                 "llama.embedding_length", "model_dim"});
    return i < 0 ? 0 : kv_int(m->kvs[i]);
}
int64_t gguf_block_count(const gguf_model_t *m) {
    const int64_t i = find_arch(m, "block_count",
                                {"block_count", "qwen35.block_count", "qwen2.block_count", "llama.n_layer",
                                 "n_layer"});
    return i < 0 ? 0 : kv_int(m->kvs[i]);
}
int64_t gguf_arch_int(const gguf_model_t *m, const char *suffix, int64_t def) {
    if (!m || !suffix) return def;
    const int64_t i = find_arch(m, suffix, {});
    return i < 0 ? def : kv_int(m->kvs[i]);
}
float gguf_arch_float(const gguf_model_t *m, const char *suffix, float def) {
    if (!m || !suffix) return def;
    const int64_t i = find_arch(m, suffix, {});
    if (i < 0 || m->kvs[i].is_array) return def;
    const Kv &k = m->kvs[i];
    if (k.type == T_F32) {
        float f;
        const uint32_t b = (uint32_t)k.raw;
        memcpy(&f, &b, 4);
        return f;
    }
    if (k.type == T_F64) {
        double d;
        memcpy(&d, &k.raw, 8);
        return (float)d;
    }
    return (float)kv_int(k);
}

int32_t gguf_kv_get_string_array(const gguf_model_t *m, const char *key, const char ***out_strings,
                                 size_t *out_count) {
    if (!m || !key || !out_strings || !out_count) return -1;
    const int64_t i = find_kv(m, key);
    if (i < 0 || !m->kvs[i].is_array || m->kvs[i].type != T_STRING) return -1;
    *out_strings = const_cast<const char **>(m->kvs[i].strp.data());
    *out_count = m->kvs[i].strp.size();
    return 0;
}
void gguf_free_string_array(const char **strings, size_t count) {
    (void)strings;
    (void)count;
}
int32_t gguf_kv_get_array(const gguf_model_t *m, const char *key, int32_t *out_type, const void **out_data,
                          size_t *out_count) {
    if (!m || !key || !out_type || !out_data || !out_count) return -1;
    const int64_t i = find_kv(m, key);
    if (i < 0 || !m->kvs[i].is_array || m->kvs[i].type == T_STRING || !m->kvs[i].arr) return -1;
    *out_type = m->kvs[i].type;
    *out_data = m->kvs[i].arr;
    *out_count = (size_t)m->kvs[i].arr_n;
    return 0;
}
int64_t gguf_find_kv(const gguf_model_t *m, const char *key) { return find_kv(m, key); }
int32_t gguf_kv_get_added_tokens(const gguf_model_t *m, const char *key, const char ***out_strings,
                                 size_t *out_count) {
    return gguf_kv_get_string_array(m, key, out_strings, out_count);
}

const void *gguf_map_base(const gguf_model_t *m, size_t *out_size) {
    if (!m || m->files.empty()) return nullptr;
    if (out_size) *out_size = m->files[0].size;
    return m->files[0].map;
}
int gguf_n_maps(const gguf_model_t *m) { return m ? (int)m->files.size() : 0; }
const void *gguf_map_at(const gguf_model_t *m, int i, size_t *out_size) {
    if (!m || i < 0 || i >= (int)m->files.size()) return nullptr;
    if (out_size) *out_size = m->files[i].size;
    return m->files[i].map;
}
int gguf_remap(gguf_model_t *m, const void *p, size_t len) {
    const size_t page = (size_t)sysconf(_SC_PAGESIZE);
    if (!m || !p || !len || (uintptr_t)p % page || len % page) return -1;
    for (File &f : m->files) {
        const char *b = (const char *)f.map;
        if ((const char *)p < b || (const char *)p + len > b + f.size) continue;
        if (f.fd_remap < 0) {  // the file as it was at open, or nothing
            const int fd = open(f.path.c_str(), O_RDONLY);
            struct stat st;
            if (fd < 0) return -1;
            if (fstat(fd, &st) != 0 || (uint64_t)st.st_dev != f.id[0] || (uint64_t)st.st_ino != f.id[1] ||
                (uint64_t)st.st_size != f.id[2]) {
                close(fd);
                return -1;
            }
            f.fd_remap = fd;
        }
        const void *r = mmap(const_cast<void *>(p), len, PROT_READ, MAP_PRIVATE | MAP_FIXED, f.fd_remap,
                             (off_t)((const char *)p - b));
        return r == MAP_FAILED ? -1 : 0;
    }
    return -1;
}
const void *gguf_tensor_source(const gguf_model_t *m, int64_t idx) {
    if (!in_range(m, idx)) return nullptr;
    const Tensor &t = m->tensors[idx];
    const File &f = m->files[t.split];
    return (const char *)f.map + f.data_off + t.offset;
}
int gguf_tensor_split(const gguf_model_t *m, int64_t idx) { return in_range(m, idx) ? m->tensors[idx].split : -1; }
void gguf_set_tensor_staged(gguf_model_t *m, int64_t idx, const void *p) {
    if (in_range(m, idx)) m->tensors[idx].staged = p;
}
const char *gguf_file_path(const gguf_model_t *m, int i) {
    return m && i >= 0 && i < (int)m->files.size() ? m->files[i].path.c_str() : nullptr;
}
int gguf_file_identity(const gguf_model_t *m, int i, uint64_t out[4]) {
    if (!m || !out || i < 0 || i >= (int)m->files.size()) return -1;
    memcpy(out, m->files[i].id, sizeof m->files[i].id);
    return 0;
}

int gguf_type_is_self_contained(int type) {
    (void)type;
    return 1;
}

// ---------------------------------------------------------------- HBM residency
static constexpr size_t HBM_ALIGN = 256;

size_t gguf_hbm_bytes(const gguf_model_t *m, const uint8_t *keep) {
    if (!m) return (size_t)-1;
    size_t off = 0;
    for (size_t i = 0; i < m->tensors.size(); ++i) {
        if (keep && !keep[i]) continue;
        const size_t b = tensor_bytes_ceil(m->tensors[i]);
        if (b == (size_t)-1) return (size_t)-1;
        off = (off + HBM_ALIGN - 1) / HBM_ALIGN * HBM_ALIGN + b;
    }
    return off;
}

int gguf_hbm_stage(gguf_model_t *m, void *dev, size_t dev_bytes, const uint8_t *keep, hipStream_t stream) {
    const size_t need = gguf_hbm_bytes(m, keep);
    if (!m || !dev || need == (size_t)-1 || dev_bytes < need) return -1;
    // a ring of pinned chunks: host threads copy the mapping's pages into one while the DMA engine empties another
    constexpr int RING = 3;
    constexpr size_t CHUNK = (size_t)64 << 20;
    void *pin[RING] = {nullptr, nullptr, nullptr};
    hipEvent_t done[RING] = {nullptr, nullptr, nullptr};
    bool ok = true;
    for (int b = 0; b < RING && ok; ++b)
        ok = hipHostMalloc(&pin[b], CHUNK, hipHostMallocDefault) == hipSuccess &&
             hipEventCreateWithFlags(&done[b], hipEventDisableTiming) == hipSuccess;
    const unsigned hw = std::thread::hardware_concurrency();
    const int nthr = (int)std::max(1u, std::min(8u, hw ? hw : 1u));
    std::vector<size_t> at(m->tensors.size(), (size_t)-1);
    size_t off = 0;
    int slot = 0;
    bool used[RING] = {false, false, false};
    for (size_t i = 0; ok && i < m->tensors.size(); ++i) {
        if (keep && !keep[i]) continue;
        const size_t bytes = tensor_bytes_ceil(m->tensors[i]);
        off = (off + HBM_ALIGN - 1) / HBM_ALIGN * HBM_ALIGN;
        at[i] = off;
        const char *src = (const char *)gguf_tensor_source(m, (int64_t)i);
        for (size_t c = 0; ok && c < bytes; c += CHUNK) {
            const size_t n = std::min(CHUNK, bytes - c);
            if (used[slot]) ok = hipEventSynchronize(done[slot]) == hipSuccess;  // its previous copy is out
            if (!ok) break;
            char *dst = (char *)pin[slot];
            const size_t per = (n + nthr - 1) / nthr;
            std::vector<std::thread> th;
            for (int t = 1; t < nthr && (size_t)t * per < n; ++t)
                th.emplace_back([=] { memcpy(dst + t * per, src + c + t * per, std::min(per, n - t * per)); });
            memcpy(dst, src + c, std::min(per, n));
            for (std::thread &x : th) x.join();
            ok = hipMemcpyAsync((char *)dev + off + c, dst, n, hipMemcpyHostToDevice, stream) == hipSuccess &&
                 hipEventRecord(done[slot], stream) == hipSuccess;
            used[slot] = true;
            slot = (slot + 1) % RING;
        }
        off += bytes;
    }
    if (ok) ok = hipStreamSynchronize(stream) == hipSuccess;
    for (int b = 0; b < RING; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (pin[b]) (void)hipHostFree(pin[b]);
    }
    if (!ok) return -1;
    for (size_t i = 0; i < m->tensors.size(); ++i)
        if (at[i] != (size_t)-1) m->tensors[i].staged = (const char *)dev + at[i];
    return 0;
}

int gguf_bind_weight(const gguf_model_t *m, const char *name, gguf_weight *w) {
    if (!m || !name || !w) return -1;
    const auto it = m->tensor_idx.find(name);
    if (it == m->tensor_idx.end()) return 1;
    const Tensor &t = m->tensors[it->second];
    if (!qt_get_traits(t.type) || t.n_dims < 1 || t.n_dims > 3) return -1;
    const int64_t K = t.ne[0], N = (t.n_dims >= 2 ? t.ne[1] : 1) * (t.n_dims == 3 ? t.ne[2] : 1);
    const size_t rb = qt_row_size(t.type, K);
    size_t bytes = 0;
    const void *p = gguf_get_tensor_ptr(m, name, &bytes);
    if (!p || rb == 0 || N <= 0 || N > INT32_MAX || K > INT32_MAX || bytes != rb * (size_t)N) return -1;
    w->type = t.type;
    w->N = (int)N;
    w->K = (int)K;
    w->row_bytes = rb;
    w->data = p;
    return 0;
}

}  // extern "C"
