// GGUF v2/v3 reader. Format and validation rules follow the reference reader
// (src/io/trc_gguf.cpp:465-654, gguf_parse; :966-1127 conversion and loading),
// which follows ggml's gguf.cpp. The data section is memory-mapped rather
// than read into a std::vector, so loading a tensor copies its bytes once,
// straight to the device.
#include "hip_hooks.h"
#include "impl.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <limits>
#include <string>
#include <unordered_map>
#include <vector>

namespace traincpp {

struct GgufKvEntry {
    std::string key;
    GgufType    type = GgufType::U8;
    uint64_t    u = 0;       // integer payloads (bit pattern)
    double      f = 0.0;     // F32/F64 payloads
    std::string str;
    GgufType    arr_type = GgufType::U8;
    uint64_t    arr_n = 0;
    std::vector<uint64_t>    arr_words;  // scalar array payload, 8-byte aligned copy
    std::vector<std::string> arr_strs;   // string array payload
};

struct GgufFile {
    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_offset = 0;
    std::vector<GgufKvEntry> kvs;
    std::unordered_map<std::string, int64_t> key_index;
    std::vector<std::string> names;
    std::vector<GgufTensorInfo> infos;
    std::unordered_map<std::string, int64_t> tensor_index;
    // data section: a read-only mapping of the whole file
    const uint8_t* map = nullptr;
    size_t map_size = 0;
    bool has_data = false;
};

namespace {

struct Reader {
    const uint8_t* p;
    size_t size;
    size_t pos = 0;
    bool ok = true;

    bool take(void* dst, size_t n) {
        if (!ok || n > size - pos) return ok = false;
        if (n) std::memcpy(dst, p + pos, n);
        pos += n;
        return true;
    }
    template <typename T>
    bool get(T& v) { return take(&v, sizeof(T)); }
    bool str(std::string& s) {
        uint64_t n = 0;
        if (!get(n) || n > size - pos) return ok = false;
        s.assign((const char*) p + pos, (size_t) n);
        pos += (size_t) n;
        return true;
    }
    bool skip(uint64_t n) {
        if (!ok || n > size - pos) return ok = false;
        pos += (size_t) n;
        return true;
    }
};

size_t scalar_size(GgufType t) {
    switch (t) {
        case GgufType::U8: case GgufType::I8: case GgufType::BOOL: return 1;
        case GgufType::U16: case GgufType::I16: return 2;
        case GgufType::U32: case GgufType::I32: case GgufType::F32: return 4;
        case GgufType::U64: case GgufType::I64: case GgufType::F64: return 8;
        default: return 0;
    }
}

bool read_kv(Reader& r, GgufKvEntry& kv) {
    int32_t t = 0;
    if (!r.str(kv.key) || !r.get(t) || t < 0 || t > (int32_t) GgufType::F64) return false;
    kv.type = (GgufType) t;
    switch (kv.type) {
        case GgufType::STRING: return r.str(kv.str);
        case GgufType::ARRAY: {
            int32_t et = 0;
            if (!r.get(et) || et < 0 || et > (int32_t) GgufType::F64 || et == (int32_t) GgufType::ARRAY) return false;
            kv.arr_type = (GgufType) et;
            if (!r.get(kv.arr_n)) return false;
            if (kv.arr_type == GgufType::STRING) {
                // every element takes at least its 8-byte length
                if (kv.arr_n > (r.size - r.pos) / 8) return false;
                kv.arr_strs.resize((size_t) kv.arr_n);
                for (uint64_t i = 0; i < kv.arr_n; ++i) {
                    if (!r.str(kv.arr_strs[(size_t) i])) return false;
                }
                return true;
            }
            const size_t es = scalar_size(kv.arr_type);
            if (kv.arr_n > (r.size - r.pos) / es) return false;
            const size_t bytes = (size_t) kv.arr_n * es;
            kv.arr_words.resize((bytes + 7) / 8);
            return r.take(kv.arr_words.data(), bytes);
        }
        case GgufType::F32: { float v; if (!r.get(v)) return false; kv.f = v; return true; }
        case GgufType::F64: return r.get(kv.f);
        default: {
            const size_t n = scalar_size(kv.type);
            uint64_t v = 0;
            if (!r.take(&v, n)) return false;
            kv.u = v;
            return true;
        }
    }
}

size_t round_up(size_t v, size_t a) {
    return (v + a - 1) / a * a;
}

GgufFile* fail_parse(GgufFile* f, const char* why) {
    log_error("GGUF: parse failed (%s)", why);
    if (f->map) munmap((void*) f->map, f->map_size);
    delete f;
    return nullptr;
}

const GgufKvEntry* typed_kv(const GgufFile* f, const char* key, GgufType want) {
    auto it = f->key_index.find(key);
    if (it == f->key_index.end()) {
        log_error("GGUF: missing key %s", key);
        return nullptr;
    }
    const GgufKvEntry& kv = f->kvs[(size_t) it->second];
    if (kv.type != want) {
        log_error("GGUF: key %s has type %d, not %d", key, (int) kv.type, (int) want);
        return nullptr;
    }
    return &kv;
}

}  // namespace

GgufFile* gguf_open(const char* path, bool load_data) {
    TRC_CHECK(path != nullptr, "gguf_open: path is NULL");
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) {
        log_error("GGUF: cannot open %s", path);
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        log_error("GGUF: cannot stat %s", path);
        return nullptr;
    }
    GgufFile* f = new GgufFile();
    f->map_size = (size_t) st.st_size;
    void* m = mmap(nullptr, f->map_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) {
        delete f;
        log_error("GGUF: cannot map %s", path);
        return nullptr;
    }
    f->map = (const uint8_t*) m;
    Reader r{f->map, f->map_size};

    char magic[4];
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail_parse(f, "bad magic");
    if (!r.get(f->version) || f->version < 2 || f->version > 3) return fail_parse(f, "unsupported version");
    if (!r.get(n_tensors) || !r.get(n_kv)) return fail_parse(f, "truncated header");
    if (n_kv > (r.size - r.pos) / 13 || n_tensors > (r.size - r.pos) / 32) return fail_parse(f, "counts exceed file");
    for (uint64_t i = 0; i < n_kv; ++i) {
        GgufKvEntry kv;
        if (!read_kv(r, kv) || kv.key.empty()) return fail_parse(f, "bad metadata entry");
        if (!f->key_index.emplace(kv.key, (int64_t) f->kvs.size()).second) return fail_parse(f, "duplicate key");
        f->kvs.push_back(std::move(kv));
    }
    if (auto it = f->key_index.find("general.alignment"); it != f->key_index.end()) {
        const GgufKvEntry& kv = f->kvs[(size_t) it->second];
        if (kv.type != GgufType::U32 || kv.u == 0 || (kv.u & (kv.u - 1)) != 0 || kv.u > (1u << 30)) {
            return fail_parse(f, "bad general.alignment");
        }
        f->alignment = (uint32_t) kv.u;
    }
    uint64_t expect = 0;
    f->names.reserve((size_t) n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        std::string name;
        uint32_t n_dims = 0;
        if (!r.str(name) || name.empty() || name.size() >= (size_t) MAX_NAME) return fail_parse(f, "bad tensor name");
        if (!r.get(n_dims) || n_dims < 1 || n_dims > (uint32_t) MAX_DIMS) return fail_parse(f, "bad dimension count");
        GgufTensorInfo info;
        for (uint32_t d = 0; d < n_dims; ++d) {
            uint64_t ne = 0;
            if (!r.get(ne) || ne == 0 || ne > (uint64_t) std::numeric_limits<int64_t>::max()) {
                return fail_parse(f, "bad dimension");
            }
            info.ne[d] = (int64_t) ne;
        }
        int32_t type = 0;
        uint64_t off = 0;
        if (!r.get(type) || type < 0 || type >= (int32_t) TYPE_COUNT) return fail_parse(f, "bad tensor type");
        info.type = (Type) type;
        const int64_t blck = type_blck_size(info.type);
        if (blck <= 0) return fail_parse(f, "tensor type without a block layout");
        if (!r.get(off)) return fail_parse(f, "truncated tensor info");
        if (info.ne[0] % blck != 0) return fail_parse(f, "ne0 is not a whole number of blocks");
        int64_t n = 1;
        for (int d = 0; d < MAX_DIMS; ++d) {
            if (info.ne[d] > std::numeric_limits<int64_t>::max() / n) return fail_parse(f, "element count overflow");
            n *= info.ne[d];
        }
        if (off != expect) return fail_parse(f, "tensor offsets are not contiguous");
        info.offset = (size_t) off;
        info.nbytes = (size_t) (n / blck) * type_size(info.type);
        expect += round_up(info.nbytes, f->alignment);
        if (!f->tensor_index.emplace(name, (int64_t) f->names.size()).second) return fail_parse(f, "duplicate tensor");
        f->names.push_back(name);
        f->infos.push_back(info);
    }
    for (size_t i = 0; i < f->infos.size(); ++i) f->infos[i].name = f->names[i].c_str();
    f->data_offset = round_up(r.pos, f->alignment);
    if (!f->infos.empty()) {
        const GgufTensorInfo& last = f->infos.back();
        if (f->data_offset > f->map_size || last.offset + last.nbytes > f->map_size - f->data_offset) {
            return fail_parse(f, "tensor data exceeds the file");
        }
    } else if (f->data_offset > f->map_size) {
        f->data_offset = f->map_size;
    }
    f->has_data = load_data;
    return f;
}

void gguf_close(GgufFile* f) {
    if (f == nullptr) return;
    if (f->map) munmap((void*) f->map, f->map_size);
    delete f;
}

int64_t gguf_version(const GgufFile* f) { return f->version; }
size_t  gguf_alignment(const GgufFile* f) { return f->alignment; }
size_t  gguf_data_offset(const GgufFile* f) { return (size_t) f->data_offset; }
int64_t gguf_kv_count(const GgufFile* f) { return (int64_t) f->kvs.size(); }

int64_t gguf_find_key(const GgufFile* f, const char* key) {
    auto it = f->key_index.find(key);
    return it == f->key_index.end() ? -1 : it->second;
}

const char* gguf_key(const GgufFile* f, int64_t index) {
    TRC_CHECK(index >= 0 && index < (int64_t) f->kvs.size(), "gguf_key: index out of range");
    return f->kvs[(size_t) index].key.c_str();
}

GgufType gguf_kv_type(const GgufFile* f, int64_t index) {
    TRC_CHECK(index >= 0 && index < (int64_t) f->kvs.size(), "gguf_kv_type: index out of range");
    return f->kvs[(size_t) index].type;
}

bool gguf_has_key(const GgufFile* f, const char* key) { return gguf_find_key(f, key) >= 0; }

// A key that is not an array is an error the caller may probe for: it is
// logged and answered with U8 / 0, as in src/io/trc_gguf.cpp:814-834.
GgufType gguf_arr_type(const GgufFile* f, int64_t index) {
    TRC_CHECK(index >= 0 && index < (int64_t) f->kvs.size(), "gguf_arr_type: index out of range");
    const GgufKvEntry& kv = f->kvs[(size_t) index];
    if (kv.type != GgufType::ARRAY) {
        log_error("GGUF: key %s is not an array", kv.key.c_str());
        return GgufType::U8;
    }
    return kv.arr_type;
}

int64_t gguf_arr_count(const GgufFile* f, int64_t index) {
    TRC_CHECK(index >= 0 && index < (int64_t) f->kvs.size(), "gguf_arr_count: index out of range");
    const GgufKvEntry& kv = f->kvs[(size_t) index];
    if (kv.type != GgufType::ARRAY) {
        log_error("GGUF: key %s is not an array", kv.key.c_str());
        return 0;
    }
    return (int64_t) kv.arr_n;
}

uint8_t gguf_get_u8(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::U8);
    return kv ? (uint8_t) kv->u : 0;
}
int8_t gguf_get_i8(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::I8);
    return kv ? (int8_t) (uint8_t) kv->u : 0;
}
uint16_t gguf_get_u16(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::U16);
    return kv ? (uint16_t) kv->u : 0;
}
int16_t gguf_get_i16(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::I16);
    return kv ? (int16_t) (uint16_t) kv->u : 0;
}
double gguf_get_f64(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::F64);
    return kv ? kv->f : 0.0;
}

uint32_t gguf_get_u32(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::U32);
    return kv ? (uint32_t) kv->u : 0;
}
int32_t gguf_get_i32(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::I32);
    return kv ? (int32_t) (uint32_t) kv->u : 0;
}
uint64_t gguf_get_u64(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::U64);
    return kv ? kv->u : 0;
}
int64_t gguf_get_i64(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::I64);
    return kv ? (int64_t) kv->u : 0;
}
float gguf_get_f32(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::F32);
    return kv ? (float) kv->f : 0.0f;
}
bool gguf_get_bool(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::BOOL);
    return kv != nullptr && kv->u != 0;
}
const char* gguf_get_str(const GgufFile* f, const char* key) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::STRING);
    return kv ? kv->str.c_str() : nullptr;
}

namespace {

// The array under `key` if its elements are of type `elem` (else an error and nullptr).
const GgufKvEntry* typed_arr(const GgufFile* f, const char* key, GgufType elem) {
    const GgufKvEntry* kv = typed_kv(f, key, GgufType::ARRAY);
    if (kv == nullptr) return nullptr;
    if (kv->arr_type != elem) {
        log_error("GGUF: array %s holds type %d, not %d", key, (int) kv->arr_type, (int) elem);
        return nullptr;
    }
    return kv;
}

template <typename T>
const T* scalar_array(const GgufFile* f, const char* key, GgufType elem, int64_t* n) {
    const GgufKvEntry* kv = typed_arr(f, key, elem);
    if (kv == nullptr) return nullptr;  // *n untouched, as in src/io/trc_gguf.cpp:900-931
    if (n != nullptr) *n = (int64_t) kv->arr_n;
    return (const T*) kv->arr_words.data();
}

}  // namespace

const int32_t* gguf_get_arr_i32(const GgufFile* f, const char* key, int64_t* n) {
    return scalar_array<int32_t>(f, key, GgufType::I32, n);
}
const int64_t* gguf_get_arr_i64(const GgufFile* f, const char* key, int64_t* n) {
    return scalar_array<int64_t>(f, key, GgufType::I64, n);
}
const float* gguf_get_arr_f32(const GgufFile* f, const char* key, int64_t* n) {
    return scalar_array<float>(f, key, GgufType::F32, n);
}
const char* gguf_get_arr_str(const GgufFile* f, const char* key, int64_t index) {
    const GgufKvEntry* kv = typed_arr(f, key, GgufType::STRING);
    if (kv == nullptr) return nullptr;
    if (index < 0 || index >= (int64_t) kv->arr_n) {
        log_error("GGUF: index %lld out of range for %s", (long long) index, key);
        return nullptr;
    }
    return kv->arr_strs[(size_t) index].c_str();
}

int64_t gguf_tensor_count(const GgufFile* f) { return (int64_t) f->infos.size(); }

int64_t gguf_find_tensor(const GgufFile* f, const char* name) {
    auto it = f->tensor_index.find(name);
    return it == f->tensor_index.end() ? -1 : it->second;
}

const GgufTensorInfo* gguf_tensor_info(const GgufFile* f, int64_t index) {
    TRC_CHECK(index >= 0 && index < (int64_t) f->infos.size(), "gguf_tensor_info: index out of range");
    return &f->infos[(size_t) index];
}

int64_t gguf_tensor_nelements(const GgufFile* f, int64_t index) {
    const GgufTensorInfo* i = gguf_tensor_info(f, index);
    return i->ne[0] * i->ne[1] * i->ne[2] * i->ne[3];
}

const uint8_t* gguf_tensor_data(const GgufFile* f, int64_t index) {
    if (!f->has_data) return nullptr;
    return f->map + f->data_offset + gguf_tensor_info(f, index)->offset;
}

namespace {

// Looks a tensor up and checks that its data can be read.
const GgufTensorInfo* readable(const GgufFile* f, const char* name, const uint8_t** src) {
    const int64_t ti = gguf_find_tensor(f, name);
    if (ti < 0) {
        log_error("GGUF: no tensor named %s", name);
        return nullptr;
    }
    if (!f->has_data) {
        log_error("GGUF: %s was opened without data", name);
        return nullptr;
    }
    *src = gguf_tensor_data(f, ti);
    return &f->infos[(size_t) ti];
}

template <typename T, typename Conv>
void convert(const uint8_t* src, float* out, int64_t n, Conv conv) {
    for (int64_t i = 0; i < n; ++i) {
        T v;
        std::memcpy(&v, src + (size_t) i * sizeof(T), sizeof(T));
        out[i] = conv(v);
    }
}

// IEEE binary16 -> binary32 by field decode (exact; NaN payloads kept, quieted).
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else {
        bits = sign | __builtin_bit_cast(uint32_t, (float) man * 0x1p-24f);
    }
    return __builtin_bit_cast(float, bits);
}

// The legacy block formats decoded on the host, element for element as the
// reference's dequantize_q* (src/io/trc_gguf.cpp:320-417): (float) q * d, plus m
// for Q4_1/Q5_1, each * and + rounded on its own (this file is built with
// -ffp-contract=off). Used by gguf_tensor_to_f32 when no HIP device is there.
float fp16_field(const uint8_t* p) {
    uint16_t h;
    std::memcpy(&h, p, 2);
    return half_to_float(h);
}

void dequant_blocks_host(Type type, const uint8_t* src, int64_t n_blocks, float* out) {
    const size_t bs = type_size(type);
    for (int64_t i = 0; i < n_blocks; ++i) {
        const uint8_t* b = src + (size_t) i * bs;
        float* y = out + i * 32;
        switch (type) {
            case TYPE_Q4_0: {  // {d; qs[16]}
                const float d = fp16_field(b);
                for (int j = 0; j < 16; ++j) {
                    y[j] = (float) ((b[2 + j] & 0x0F) - 8) * d;
                    y[j + 16] = (float) ((b[2 + j] >> 4) - 8) * d;
                }
                break;
            }
            case TYPE_Q4_1: {  // {d; m; qs[16]}
                const float d = fp16_field(b), m = fp16_field(b + 2);
                for (int j = 0; j < 16; ++j) {
                    y[j] = (float) (b[4 + j] & 0x0F) * d + m;
                    y[j + 16] = (float) (b[4 + j] >> 4) * d + m;
                }
                break;
            }
            case TYPE_Q5_0: {  // {d; qh (LE u32); qs[16]}: bit j and j + 16 of qh are the fifth bits
                const float d = fp16_field(b);
                uint32_t qh;
                std::memcpy(&qh, b + 2, 4);
                for (int j = 0; j < 16; ++j) {
                    const int lo = (b[6 + j] & 0x0F) | (int) (((qh >> j) & 1u) << 4);
                    const int hi = (b[6 + j] >> 4) | (int) (((qh >> (j + 16)) & 1u) << 4);
                    y[j] = (float) (lo - 16) * d;
                    y[j + 16] = (float) (hi - 16) * d;
                }
                break;
            }
            case TYPE_Q5_1: {  // {d; m; qh; qs[16]}
                const float d = fp16_field(b), m = fp16_field(b + 2);
                uint32_t qh;
                std::memcpy(&qh, b + 4, 4);
                for (int j = 0; j < 16; ++j) {
                    const int lo = (b[8 + j] & 0x0F) | (int) (((qh >> j) & 1u) << 4);
                    const int hi = (b[8 + j] >> 4) | (int) (((qh >> (j + 16)) & 1u) << 4);
                    y[j] = (float) lo * d + m;
                    y[j + 16] = (float) hi * d + m;
                }
                break;
            }
            case TYPE_Q8_0: {  // {d; qs[32] int8}
                const float d = fp16_field(b);
                for (int j = 0; j < 32; ++j) y[j] = (float) (int8_t) b[2 + j] * d;
                break;
            }
            default:
                break;
        }
    }
}

}  // namespace

bool gguf_tensor_to_f32(const GgufFile* f, const char* name, float* out, int64_t n_elems) {
    TRC_CHECK(f != nullptr && name != nullptr && out != nullptr, "gguf_tensor_to_f32: NULL argument");
    const uint8_t* src = nullptr;
    const GgufTensorInfo* info = readable(f, name, &src);
    if (info == nullptr) return false;
    const int64_t n = info->ne[0] * info->ne[1] * info->ne[2] * info->ne[3];
    if (n_elems < n) {
        log_error("GGUF: output of %lld elements is smaller than %s (%lld)", (long long) n_elems, name, (long long) n);
        return false;
    }
    switch (info->type) {
        case TYPE_F32: std::memcpy(out, src, (size_t) n * 4); return true;
        case TYPE_F16: convert<uint16_t>(src, out, n, half_to_float); return true;
        case TYPE_BF16:
            convert<uint16_t>(src, out, n, [](uint16_t h) { return __builtin_bit_cast(float, (uint32_t) h << 16); });
            return true;
        case TYPE_F64: convert<double>(src, out, n, [](double v) { return (float) v; }); return true;
        case TYPE_I8: convert<int8_t>(src, out, n, [](int8_t v) { return (float) v; }); return true;
        case TYPE_I16: convert<int16_t>(src, out, n, [](int16_t v) { return (float) v; }); return true;
        case TYPE_I32: convert<int32_t>(src, out, n, [](int32_t v) { return (float) v; }); return true;
        case TYPE_I64: convert<int64_t>(src, out, n, [](int64_t v) { return (float) v; }); return true;
        case TYPE_Q4_0: case TYPE_Q4_1: case TYPE_Q5_0: case TYPE_Q5_1: case TYPE_Q8_0:
            // on the GPU when one is there (the same bits), else on the host
            if (!hip_dequant_host(info->type, src, n / 32, out)) dequant_blocks_host(info->type, src, n / 32, out);
            return true;
        default:
            log_error("GGUF: type %s of %s cannot be converted", type_name(info->type), name);
            return false;
    }
}

bool gguf_load_tensor(const GgufFile* f, const char* name, Tensor* dst) {
    TRC_CHECK(f != nullptr && name != nullptr && dst != nullptr, "gguf_load_tensor: NULL argument");
    const uint8_t* src = nullptr;
    const GgufTensorInfo* info = readable(f, name, &src);
    if (info == nullptr) return false;
    const int64_t n = info->ne[0] * info->ne[1] * info->ne[2] * info->ne[3];
    if (!tensor_is_contiguous(dst)) {
        log_error("GGUF: destination %s must be contiguous", name);
        return false;
    }
    if (tensor_nelements(dst) != n) {
        log_error("GGUF: %s has %lld elements in the file and %lld in the tensor", name, (long long) n,
                  (long long) tensor_nelements(dst));
        return false;
    }
    if (dst->type == info->type) {  // raw copy (also how quantized tensors reach the GPU)
        tensor_set(dst, src, 0, info->nbytes);
        return true;
    }
    if (dst->type != TYPE_F32) {
        log_error("GGUF: %s is %s in the file; the destination must be F32 or the same type", name,
                  type_name(info->type));
        return false;
    }
    const bool legacy_quant = info->type == TYPE_Q4_0 || info->type == TYPE_Q4_1 || info->type == TYPE_Q5_0 ||
                              info->type == TYPE_Q5_1 || info->type == TYPE_Q8_0;
    if (legacy_quant && hip_dequant_into(dst, info->type, src, n / 32)) return true;
    std::vector<float> tmp((size_t) n);
    if (!gguf_tensor_to_f32(f, name, tmp.data(), n)) return false;
    tensor_set(dst, tmp.data(), 0, tmp.size() * sizeof(float));
    return true;
}

Tensor* gguf_new_tensor(Context* ctx, const GgufFile* f, const char* name, Type type) {
    TRC_CHECK(ctx != nullptr && name != nullptr, "gguf_new_tensor: NULL argument");
    const int64_t ti = gguf_find_tensor(f, name);
    if (ti < 0) {
        log_error("GGUF: no tensor named %s", name);
        return nullptr;
    }
    if (!type_is_storable(type)) {
        log_error("GGUF: tensors of type %s cannot be created", type_name(type));
        return nullptr;
    }
    const GgufTensorInfo& info = f->infos[(size_t) ti];
    const int64_t blck = type_blck_size(type);
    if (info.ne[0] % blck != 0) {
        log_error("GGUF: ne0 of %s is not a multiple of the %s block size", name, type_name(type));
        return nullptr;
    }
    int n_dims = 1;
    for (int i = 1; i < MAX_DIMS; ++i) {
        if (info.ne[i] > 1) n_dims = i + 1;
    }
    Tensor* t = new_tensor_nd(ctx, type, n_dims, info.ne);
    tensor_set_name(t, "%s", name);
    return t;
}

bool gguf_validate(const char* path) {
    GgufFile* f = gguf_open(path, true);
    if (f == nullptr) return false;
    size_t expect = 0;
    bool ok = true;
    for (const GgufTensorInfo& i : f->infos) {
        if (i.offset != expect || f->data_offset + i.offset + i.nbytes > f->map_size) {
            log_error("GGUF: tensor %s has a bad offset or range", i.name);
            ok = false;
            break;
        }
        expect += round_up(i.nbytes, f->alignment);
    }
    gguf_close(f);
    return ok;
}

}  // namespace traincpp
