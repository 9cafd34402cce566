// safetensors.cpp — checkpoint ingest for the expert path: memory-mapped
// safetensors files (one file or a directory of shards) and the DeepSeek tensor
// naming of routed experts, shared experts and routers.
//
// Follows ModelWeights (crates/objeta-parser/src/lib.rs:88-293): the 8-byte
// little-endian header length, the JSON header of {name: {dtype, shape,
// data_offsets}} entries with "__metadata__" skipped, data addressed from
// 8 + header_len, shards taken in file-name order with later names replacing
// earlier ones, zero-copy raw access and F32/F16/BF16 -> f32 conversion. The
// DeepSeek names follow classify_tensor (crates/objeta-parser/src/deepseek.rs:
// 178-262: w1 = gate, w3 = up, w2 = down, ".scale" suffix for scales, "layers.L"
// or "mtp.L" prefixes), load_shared_expert_fp8 and find_router_tensor
// (crates/objeta-cuda/src/bin/deepseek_single_layer_moe.rs:209-330, 1034-1080).
//
// The header is parsed by a small recursive-descent JSON reader of its own; every
// tensor's byte range is checked against its file when the model is opened, so a
// later raw access never reads outside the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <dirent.h>
#include <map>
#include <string>
#include <vector>

#include "host_common.hpp"

namespace objeta {
namespace st {

struct Mapping {
    std::string path;
    const uint8_t* base = nullptr;
    size_t size = 0;
};

struct Tensor {
    int32_t dtype = 0;
    std::vector<uint64_t> shape;
    uint32_t file = 0;
    uint64_t offset = 0;  // from the start of the file
    uint64_t nbytes = 0;
    uint64_t nelem = 0;
};

// Dtype::from_str (lib.rs:56-71) and element sizes (lib.rs:44-53).
bool parse_dtype(const std::string& s, int32_t* out) {
    static const struct {
        const char* a;
        const char* b;
        int32_t v;
    } table[] = {{"F32", "FLOAT32", OBJETA_HIP_DT_F32},   {"F16", "FLOAT16", OBJETA_HIP_DT_F16},
                 {"BF16", "BFLOAT16", OBJETA_HIP_DT_BF16}, {"I64", "INT64", OBJETA_HIP_DT_I64},
                 {"I32", "INT32", OBJETA_HIP_DT_I32},     {"I8", "INT8", OBJETA_HIP_DT_I8},
                 {"U8", "UINT8", OBJETA_HIP_DT_U8},       {"F8_E8M0", nullptr, OBJETA_HIP_DT_F8_E8M0},
                 {"F8_E4M3", nullptr, OBJETA_HIP_DT_F8_E4M3}, {"BOOL", nullptr, OBJETA_HIP_DT_BOOL}};
    for (const auto& t : table)
        if (s == t.a || (t.b && s == t.b)) {
            *out = t.v;
            return true;
        }
    return false;
}

const char* dtype_name(int32_t d) {
    switch (d) {
        case OBJETA_HIP_DT_F32: return "F32";
        case OBJETA_HIP_DT_F16: return "F16";
        case OBJETA_HIP_DT_BF16: return "BF16";
        case OBJETA_HIP_DT_I64: return "I64";
        case OBJETA_HIP_DT_I32: return "I32";
        case OBJETA_HIP_DT_I8: return "I8";
        case OBJETA_HIP_DT_U8: return "U8";
        case OBJETA_HIP_DT_F8_E8M0: return "F8_E8M0";
        case OBJETA_HIP_DT_F8_E4M3: return "F8_E4M3";
        default: return "BOOL";
    }
}

// ---------------------------------------------------------------- JSON reader
// Enough JSON for a safetensors header: objects, arrays, strings with escapes
// (\uXXXX and surrogate pairs to UTF-8), numbers (unsigned integers kept exactly,
// others skipped), true / false / null.
struct Json {
    enum Type { kNull, kBool, kNum, kStr, kArr, kObj } type = kNull;
    bool is_uint = false;
    uint64_t u = 0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
};

class Reader {
  public:
    Reader(const char* p, size_t n) : p_(p), end_(p + n) {}
    bool parse(Json* out, std::string* err) {
        if (!value(out, 0)) {
            *err = err_.empty() ? "invalid JSON" : err_;
            return false;
        }
        ws();
        if (p_ != end_) {
            *err = "trailing characters after the header object";
            return false;
        }
        return true;
    }

  private:
    const char* p_;
    const char* end_;
    std::string err_;

    bool fail(const char* m) {
        if (err_.empty()) err_ = m;
        return false;
    }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = std::strlen(w);
        if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, w, n) != 0) return fail("invalid literal");
        p_ += n;
        return true;
    }
    static void utf8(std::string& s, uint32_t c) {
        if (c < 0x80) {
            s += static_cast<char>(c);
        } else if (c < 0x800) {
            s += static_cast<char>(0xC0 | (c >> 6));
            s += static_cast<char>(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += static_cast<char>(0xE0 | (c >> 12));
            s += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (c & 0x3F));
        } else {
            s += static_cast<char>(0xF0 | (c >> 18));
            s += static_cast<char>(0x80 | ((c >> 12) & 0x3F));
            s += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t* v) {
        if (end_ - p_ < 4) return fail("truncated \\u escape");
        uint32_t r = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            r <<= 4;
            if (c >= '0' && c <= '9') r |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') r |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') r |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail("invalid \\u escape");
        }
        *v = r;
        return true;
    }
    bool str(std::string* out) {
        if (p_ >= end_ || *p_ != '"') return fail("expected a string");
        ++p_;
        std::string s;
        while (true) {
            if (p_ >= end_) return fail("unterminated string");
            const unsigned char c = static_cast<unsigned char>(*p_++);
            if (c == '"') break;
            if (c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                s += static_cast<char>(c);
                continue;
            }
            if (p_ >= end_) return fail("unterminated escape");
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t v = 0;
                    if (!hex4(&v)) return false;
                    if (v >= 0xD800 && v < 0xDC00) {  // a high surrogate needs its low half
                        uint32_t lo = 0;
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
                        p_ += 2;
                        if (!hex4(&lo) || lo < 0xDC00 || lo > 0xDFFF) return fail("lone surrogate");
                        v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (v >= 0xDC00 && v < 0xE000) {
                        return fail("lone surrogate");
                    }
                    utf8(s, v);
                    break;
                }
                default: return fail("invalid escape");
            }
        }
        *out = std::move(s);
        return true;
    }
    bool num(Json* out) {
        const char* b = p_;
        bool neg = false, frac = false;
        if (p_ < end_ && *p_ == '-') {
            neg = true;
            ++p_;
        }
        uint64_t v = 0;
        bool overflow = false, digits = false;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = static_cast<uint64_t>(*p_ - '0');
            if (v > (UINT64_MAX - d) / 10) overflow = true;
            v = v * 10 + d;
            digits = true;
            ++p_;
        }
        if (!digits) return fail("invalid number");
        if (p_ < end_ && *p_ == '.') {
            frac = true;
            ++p_;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        (void)b;
        out->type = Json::kNum;
        out->is_uint = !neg && !frac && !overflow;
        out->u = v;
        return true;
    }
    bool value(Json* out, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p_ >= end_) return fail("unexpected end of header");
        const char c = *p_;
        if (c == '{') {
            ++p_;
            out->type = Json::kObj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            while (true) {
                ws();
                std::string k;
                if (!str(&k)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
                ++p_;
                Json v;
                if (!value(&v, depth + 1)) return false;
                out->obj.emplace_back(std::move(k), std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            out->type = Json::kArr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            while (true) {
                Json v;
                if (!value(&v, depth + 1)) return false;
                out->arr.push_back(std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            out->type = Json::kStr;
            return str(&out->s);
        }
        if (c == 't') {
            out->type = Json::kBool;
            return lit("true");
        }
        if (c == 'f') {
            out->type = Json::kBool;
            return lit("false");
        }
        if (c == 'n') {
            out->type = Json::kNull;
            return lit("null");
        }
        return num(out);
    }
};

bool valid_utf8(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        size_t len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (len == 0 || i + len > n) return false;
        for (size_t k = 1; k < len; ++k)
            if ((s[i + k] & 0xC0) != 0x80) return false;
        i += len;
    }
    return true;
}

}  // namespace st
}  // namespace objeta

struct objeta_hip_st_model {
    std::vector<objeta::st::Mapping> files;
    std::map<std::string, objeta::st::Tensor> index;  // ordered: keys() is sorted
};

namespace objeta {
namespace st {
namespace {

void unmap_all(objeta_hip_st_model* m) {
    for (auto& f : m->files)
        if (f.base && f.size) munmap(const_cast<uint8_t*>(f.base), f.size);
    m->files.clear();
}

// Maps one file and adds its tensors to the index (parse_header and the entry loop
// of ModelWeights::open, lib.rs:104-203).
int32_t add_file(objeta_hip_st_model* m, const std::string& path) {
    const std::string action = "open safetensors '" + path + "'";
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) OBJ_FAIL(kIo, action, std::strerror(errno));
    struct stat sb{};
    if (fstat(fd, &sb) != 0) {
        const int e = errno;
        ::close(fd);
        OBJ_FAIL(kIo, action, std::strerror(e));
    }
    const size_t size = static_cast<size_t>(sb.st_size);
    if (size < 8) {
        ::close(fd);
        OBJ_FAIL(kIo, action, "parse: file too short");
    }
    void* base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (base == MAP_FAILED) OBJ_FAIL(kIo, action, std::string("mmap: ") + std::strerror(errno));
    const uint8_t* b = static_cast<const uint8_t*>(base);
    const uint32_t file_index = static_cast<uint32_t>(m->files.size());
    m->files.push_back(Mapping{path, b, size});
    uint64_t header_len = 0;
    for (int i = 7; i >= 0; --i) header_len = (header_len << 8) | b[i];
    if (header_len > size - 8) OBJ_FAIL(kIo, action, "parse: header length exceeds file size");
    const uint8_t* h = b + 8;
    if (!valid_utf8(h, header_len)) OBJ_FAIL(kIo, action, "parse: invalid UTF-8 in header");
    Json root;
    std::string err;
    if (!Reader(reinterpret_cast<const char*>(h), header_len).parse(&root, &err))
        OBJ_FAIL(kIo, action, "parse: invalid header JSON: " + err);
    if (root.type != Json::kObj) OBJ_FAIL(kIo, action, "parse: the header is not a JSON object");
    const uint64_t data_start = 8 + header_len;
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& v = kv.second;
        const std::string bad = "parse: invalid tensor entry for '" + kv.first + "'";
        if (v.type != Json::kObj) OBJ_FAIL(kIo, action, bad);
        const Json *dt = nullptr, *shape = nullptr, *offs = nullptr;
        for (const auto& f : v.obj) {
            if (f.first == "dtype") dt = &f.second;
            else if (f.first == "shape") shape = &f.second;
            else if (f.first == "data_offsets") offs = &f.second;
        }
        if (!dt || dt->type != Json::kStr || !shape || shape->type != Json::kArr || !offs ||
            offs->type != Json::kArr || offs->arr.size() != 2 || !offs->arr[0].is_uint || !offs->arr[1].is_uint)
            OBJ_FAIL(kIo, action, bad);
        Tensor t;
        if (!parse_dtype(dt->s, &t.dtype)) OBJ_FAIL(kIo, action, "parse: Unknown dtype: " + dt->s);
        uint64_t nelem = 1;
        for (const auto& d : shape->arr) {
            if (!d.is_uint) OBJ_FAIL(kIo, action, bad);
            t.shape.push_back(d.u);
            nelem *= d.u;
        }
        const uint64_t a = offs->arr[0].u, e = offs->arr[1].u;
        if (e < a || e > size - data_start)
            OBJ_FAIL(kIo, action, "parse: tensor '" + kv.first + "' data_offsets lie outside the file");
        t.file = file_index;
        t.offset = data_start + a;
        t.nbytes = e - a;
        t.nelem = nelem;
        m->index[kv.first] = std::move(t);
    }
    return 0;
}

const Tensor* find(const objeta_hip_st_model* m, const std::string& name) {
    auto it = m->index.find(name);
    return it == m->index.end() ? nullptr : &it->second;
}

// half_to_f32 (lib.rs:299-323): subnormals as m * 2^-24, NaN as the canonical NaN.
float half_to_f32(uint16_t h) {
    const uint32_t sign = h >> 15, exp = (h >> 10) & 0x1F, man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign << 31;
        } else {
            float v = static_cast<float>(man) * 5.9604644775390625e-08f;  // 2^-24, exact
            return sign ? -v : v;
        }
    } else if (exp == 31) {
        bits = man == 0 ? ((sign << 31) | 0x7F800000u) : 0x7FC00000u;
    } else {
        bits = (sign << 31) | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Parses "<a>.<n>." for a = "layers" or "mtp": the layer of a tensor name and its
// block family (classify_tensor's layer parse and matches_block_family).
bool layer_of(const std::string& name, uint64_t* layer, bool* mtp) {
    std::vector<std::string> parts;
    size_t s = 0;
    while (true) {
        const size_t d = name.find('.', s);
        parts.push_back(name.substr(s, d == std::string::npos ? std::string::npos : d - s));
        if (d == std::string::npos) break;
        s = d + 1;
    }
    auto num_after = [&](const char* key, uint64_t* v) {
        for (size_t i = 0; i + 1 < parts.size(); ++i)
            if (parts[i] == key) {
                const std::string& q = parts[i + 1];
                if (q.empty() || q.size() > 19 || !std::all_of(q.begin(), q.end(), ::isdigit)) return false;
                *v = std::stoull(q);
                return true;
            }
        return false;
    };
    *mtp = std::find(parts.begin(), parts.end(), "mtp") != parts.end();
    return num_after("layers", layer) || num_after("mtp", layer);
}

std::string family_prefix(uint64_t layer, int32_t mtp) {
    return (mtp ? "mtp." : "layers.") + std::to_string(layer);
}

void fill_info(const Tensor& t, objeta_hip_st_info* out) {
    std::memset(out, 0, sizeof(*out));
    out->dtype = t.dtype;
    out->ndim = static_cast<uint32_t>(std::min<size_t>(t.shape.size(), 8));
    for (uint32_t i = 0; i < out->ndim; ++i) out->shape[i] = t.shape[i];
    out->nbytes = t.nbytes;
    out->nelem = t.nelem;
    out->file = t.file;
}

const void* data_of(const objeta_hip_st_model* m, const Tensor& t) { return m->files[t.file].base + t.offset; }

// The expert tensors are one byte per element (I8/U8 nibble pairs, F8_E4M3 codes,
// F8_E8M0 scales): a tensor must hold exactly as many bytes as its shape has
// elements, or the kernels would read past the end of a truncated tensor.
int32_t check_byte_count(const Tensor& t, const char* action, const char* what) {
    if (t.nbytes != t.nelem)
        OBJ_FAIL(kInvalidInput, action,
                 strf("%s: %llu bytes for %llu one-byte elements", what, (unsigned long long)t.nbytes,
                      (unsigned long long)t.nelem));
    return 0;
}

std::string shape_str(const std::vector<uint64_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

}  // namespace
}  // namespace st
}  // namespace objeta

using namespace objeta;
using namespace objeta::st;

extern "C" {

int32_t objeta_hip_st_open(const char* path, objeta_hip_st_model** out) {
    OBJ_GUARD_BEGIN
    if (!path || !out) OBJ_FAIL(kInvalidInput, "open safetensors", "NULL argument");
    *out = nullptr;
    struct stat sb{};
    if (stat(path, &sb) != 0) OBJ_FAIL(kIo, std::string("open safetensors '") + path + "'", std::strerror(errno));
    auto* m = new objeta_hip_st_model();
    int32_t rc = 0;
    if (S_ISDIR(sb.st_mode)) {
        std::vector<std::string> names;
        if (DIR* d = opendir(path)) {
            while (dirent* e = readdir(d)) {
                const std::string n = e->d_name;
                if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) names.push_back(n);
            }
            closedir(d);
        } else {
            delete m;
            OBJ_FAIL(kIo, std::string("open safetensors directory '") + path + "'", std::strerror(errno));
        }
        std::sort(names.begin(), names.end());  // shards in file-name order (lib.rs:113-121)
        for (const auto& n : names)
            if ((rc = add_file(m, std::string(path) + "/" + n))) break;
    } else {
        rc = add_file(m, path);
    }
    if (rc) {
        unmap_all(m);
        delete m;
        return rc;
    }
    *out = m;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_st_close(objeta_hip_st_model* m) {
    if (!m) return 0;
    unmap_all(m);
    delete m;
    return 0;
}

int32_t objeta_hip_st_len(const objeta_hip_st_model* m, uint64_t* n) {
    if (!m || !n) OBJ_FAIL(kInvalidInput, "safetensors len", "NULL argument");
    *n = m->index.size();
    return 0;
}

int32_t objeta_hip_st_key(const objeta_hip_st_model* m, uint64_t i, char* buf, uint64_t cap, uint64_t* len) {
    if (!m || !len) OBJ_FAIL(kInvalidInput, "safetensors key", "NULL argument");
    if (i >= m->index.size()) OBJ_FAIL(kInvalidInput, "safetensors key", "index out of range");
    auto it = m->index.begin();
    std::advance(it, static_cast<long>(i));
    *len = it->first.size();
    if (buf && cap) {
        const size_t n = std::min<size_t>(it->first.size(), cap - 1);
        std::memcpy(buf, it->first.data(), n);
        buf[n] = '\0';
    }
    return 0;
}

int32_t objeta_hip_st_info_get(const objeta_hip_st_model* m, const char* name, int32_t* found,
                               objeta_hip_st_info* out) {
    if (!m || !name || !found) OBJ_FAIL(kInvalidInput, "safetensors info", "NULL argument");
    const Tensor* t = find(m, name);
    *found = t ? 1 : 0;
    if (t && out) fill_info(*t, out);
    return 0;
}

int32_t objeta_hip_st_get_raw(const objeta_hip_st_model* m, const char* name, const void** ptr, uint64_t* nbytes) {
    if (!m || !name || !ptr) OBJ_FAIL(kInvalidInput, "safetensors get_raw", "NULL argument");
    const Tensor* t = find(m, name);
    if (!t) OBJ_FAIL(kIo, std::string("load raw tensor '") + name + "'", std::string("missing tensor: ") + name);
    *ptr = data_of(m, *t);
    if (nbytes) *nbytes = t->nbytes;
    return 0;
}

int32_t objeta_hip_st_get_f32(const objeta_hip_st_model* m, const char* name, float* out, uint64_t cap,
                              uint64_t* nelem) {
    OBJ_GUARD_BEGIN
    if (!m || !name || !nelem) OBJ_FAIL(kInvalidInput, "safetensors get_f32", "NULL argument");
    const Tensor* t = find(m, name);
    const std::string action = std::string("load f32 tensor '") + name + "'";
    if (!t) OBJ_FAIL(kIo, action, std::string("missing tensor: ") + name);
    const size_t es = t->dtype == OBJETA_HIP_DT_F32 ? 4 : 2;
    if (t->dtype != OBJETA_HIP_DT_F32 && t->dtype != OBJETA_HIP_DT_F16 && t->dtype != OBJETA_HIP_DT_BF16)
        OBJ_FAIL(kIo, action, std::string("parse: cannot convert ") + dtype_name(t->dtype) + " to f32");
    const uint64_t n = t->nbytes / es;  // the reference converts raw.len() / element size values
    *nelem = n;
    if (!out) return 0;
    if (cap < n) OBJ_FAIL(kInvalidInput, action, strf("output holds %llu of %llu values", (unsigned long long)cap,
                                                      (unsigned long long)n));
    const uint8_t* src = static_cast<const uint8_t*>(data_of(m, *t));
    if (t->dtype == OBJETA_HIP_DT_F32) {
        std::memcpy(out, src, n * 4);
    } else {
        for (uint64_t i = 0; i < n; ++i) {
            uint16_t h;
            std::memcpy(&h, src + 2 * i, 2);
            if (t->dtype == OBJETA_HIP_DT_F16) {
                out[i] = half_to_f32(h);
            } else {
                const uint32_t b = static_cast<uint32_t>(h) << 16;  // bf16_to_f32 (lib.rs:325-329)
                std::memcpy(&out[i], &b, 4);
            }
        }
    }
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_st_deepseek_expert(const objeta_hip_st_model* m, uint64_t layer, uint64_t expert, int32_t mtp,
                                      objeta_hip_host_expert* out, uint64_t* hidden, uint64_t* intermediate,
                                      uint64_t* out_dim) {
    OBJ_GUARD_BEGIN
    if (!m || !out) OBJ_FAIL(kInvalidInput, "find fp4 expert tensors", "NULL argument");
    // classify_tensor over the index: ffn/mlp tensors of this layer and family under
    // "experts.<expert>", kind from ".w1." / ".w3." / ".w2.", scale by ".scale"
    const Tensor* found[6] = {};  // gate, gate_scale, up, up_scale, down, down_scale
    for (const auto& kv : m->index) {
        const std::string& n = kv.first;
        uint64_t l = 0;
        bool is_mtp = false;
        if (!layer_of(n, &l, &is_mtp) || l != layer || is_mtp != (mtp != 0)) continue;
        if (n.find(".ffn.") == std::string::npos && n.find(".mlp.") == std::string::npos) continue;
        if (n.find("shared_expert") != std::string::npos) continue;
        const std::string tag = ".experts." + std::to_string(expert) + ".";
        const std::string tag2 = ".expert." + std::to_string(expert) + ".";
        if (n.find(tag) == std::string::npos && n.find(tag2) == std::string::npos) continue;
        const bool scale = n.size() >= 6 && n.compare(n.size() - 6, 6, ".scale") == 0;
        int slot = -1;
        if (n.find(".w1.") != std::string::npos) slot = 0;
        else if (n.find(".w3.") != std::string::npos) slot = 2;
        else if (n.find(".w2.") != std::string::npos) slot = 4;
        if (slot < 0) continue;
        found[slot + (scale ? 1 : 0)] = &kv.second;
    }
    std::string missing;
    const char* kinds[3] = {"gate", "up", "down"};
    for (int k = 0; k < 3; ++k)
        if (!found[2 * k]) missing += std::string(missing.empty() ? "" : ", ") + "\"" + kinds[k] + "\"";
    if (!missing.empty())
        OBJ_FAIL(kInvalidInput, "find fp4 expert tensors",
                 strf("layer %llu block family %s expert %llu missing tensors: [%s]", (unsigned long long)layer,
                      mtp ? "Mtp" : "Decoder", (unsigned long long)expert, missing.c_str()));
    for (int k = 0; k < 3; ++k)
        if (!found[2 * k + 1])
            OBJ_FAIL(kInvalidInput, "find fp4 scale tensor",
                     strf("%s weight of layer %llu expert %llu has no scale tensor — not FP4?", kinds[k],
                          (unsigned long long)layer, (unsigned long long)expert));
    // the split FP4 layout: packed nibbles [rows][cols/2] (I8 or U8) and E8M0 [rows][cols/32]
    uint64_t dims[3][2];
    for (int k = 0; k < 3; ++k) {
        const Tensor& w = *found[2 * k];
        const Tensor& s = *found[2 * k + 1];
        if ((w.dtype != OBJETA_HIP_DT_I8 && w.dtype != OBJETA_HIP_DT_U8) || w.shape.size() != 2)
            OBJ_FAIL(kInvalidInput, "validate fp4 expert tensor",
                     strf("%s weight: dtype %s shape %s, expected I8/U8 [rows, cols/2]", kinds[k],
                          dtype_name(w.dtype), shape_str(w.shape).c_str()));
        const uint64_t rows = w.shape[0], cols = 2 * w.shape[1];
        if ((s.dtype != OBJETA_HIP_DT_F8_E8M0 && s.dtype != OBJETA_HIP_DT_U8) || s.shape.size() != 2 ||
            s.shape[0] != rows || cols % 32 != 0 || s.shape[1] != cols / 32)
            OBJ_FAIL(kInvalidInput, "validate fp4 expert tensor",
                     strf("%s scale: dtype %s shape %s, expected F8_E8M0 [%llu, %llu]", kinds[k], dtype_name(s.dtype),
                          shape_str(s.shape).c_str(), (unsigned long long)rows, (unsigned long long)(cols / 32)));
        OBJ_TRY(check_byte_count(w, "validate fp4 expert tensor", (std::string(kinds[k]) + " weight").c_str()));
        OBJ_TRY(check_byte_count(s, "validate fp4 expert tensor", (std::string(kinds[k]) + " scale").c_str()));
        dims[k][0] = rows;
        dims[k][1] = cols;
    }
    if (dims[0][0] != dims[1][0] || dims[0][1] != dims[1][1] || dims[2][1] != dims[0][0])
        OBJ_FAIL(kInvalidInput, "validate fp4 expert tensor",
                 strf("gate [%llu, %llu], up [%llu, %llu] and down [%llu, %llu] do not form one expert",
                      (unsigned long long)dims[0][0], (unsigned long long)dims[0][1], (unsigned long long)dims[1][0],
                      (unsigned long long)dims[1][1], (unsigned long long)dims[2][0], (unsigned long long)dims[2][1]));
    out->gate = data_of(m, *found[0]);
    out->gate_len = found[0]->nbytes;
    out->gate_scale = data_of(m, *found[1]);
    out->gate_scale_len = found[1]->nbytes;
    out->up = data_of(m, *found[2]);
    out->up_len = found[2]->nbytes;
    out->up_scale = data_of(m, *found[3]);
    out->up_scale_len = found[3]->nbytes;
    out->down = data_of(m, *found[4]);
    out->down_len = found[4]->nbytes;
    out->down_scale = data_of(m, *found[5]);
    out->down_scale_len = found[5]->nbytes;
    if (hidden) *hidden = dims[0][1];
    if (intermediate) *intermediate = dims[0][0];
    if (out_dim) *out_dim = dims[2][0];
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_st_deepseek_shared_expert(const objeta_hip_st_model* m, uint64_t layer, int32_t mtp,
                                             objeta_hip_host_expert* out, uint64_t* hidden, uint64_t* intermediate,
                                             uint64_t* out_dim) {
    OBJ_GUARD_BEGIN
    if (!m || !out) OBJ_FAIL(kInvalidInput, "load shared expert", "NULL argument");
    const std::string prefix = family_prefix(layer, mtp) + ".ffn.shared_experts";
    const char* parts[6] = {".w1.weight", ".w1.scale", ".w3.weight", ".w3.scale", ".w2.weight", ".w2.scale"};
    const Tensor* t[6];
    for (int i = 0; i < 6; ++i) {
        const std::string n = prefix + parts[i];
        t[i] = find(m, n);
        if (!t[i]) OBJ_FAIL(kIo, "load '" + n + "'", "missing tensor: " + n);
    }
    // FP8 E4M3 [rows][cols] with E8M0 scales on the 128 x 128 tile grid
    uint64_t dims[3][2];
    const char* kinds[3] = {"gate", "up", "down"};
    for (int k = 0; k < 3; ++k) {
        const Tensor& w = *t[2 * k];
        const Tensor& s = *t[2 * k + 1];
        if ((w.dtype != OBJETA_HIP_DT_F8_E4M3 && w.dtype != OBJETA_HIP_DT_U8) || w.shape.size() != 2)
            OBJ_FAIL(kInvalidInput, "validate shared expert tensor",
                     strf("%s weight: dtype %s shape %s, expected F8_E4M3 [rows, cols]", kinds[k],
                          dtype_name(w.dtype), shape_str(w.shape).c_str()));
        const uint64_t rows = w.shape[0], cols = w.shape[1];
        if ((s.dtype != OBJETA_HIP_DT_F8_E8M0 && s.dtype != OBJETA_HIP_DT_U8) || s.shape.size() != 2 ||
            s.shape[0] != (rows + 127) / 128 || s.shape[1] != (cols + 127) / 128)
            OBJ_FAIL(kInvalidInput, "validate shared expert tensor",
                     strf("%s scale: dtype %s shape %s, expected F8_E8M0 [%llu, %llu]", kinds[k], dtype_name(s.dtype),
                          shape_str(s.shape).c_str(), (unsigned long long)((rows + 127) / 128),
                          (unsigned long long)((cols + 127) / 128)));
        OBJ_TRY(check_byte_count(w, "validate shared expert tensor", (std::string(kinds[k]) + " weight").c_str()));
        OBJ_TRY(check_byte_count(s, "validate shared expert tensor", (std::string(kinds[k]) + " scale").c_str()));
        dims[k][0] = rows;
        dims[k][1] = cols;
    }
    if (dims[0][0] != dims[1][0] || dims[0][1] != dims[1][1] || dims[2][1] != dims[0][0])
        OBJ_FAIL(kInvalidInput, "validate shared expert tensor", "gate, up and down shapes do not form one expert");
    const void* p[6];
    for (int i = 0; i < 6; ++i) p[i] = data_of(m, *t[i]);
    *out = objeta_hip_host_expert{p[0], t[0]->nbytes, p[2], t[2]->nbytes, p[4], t[4]->nbytes,
                                  p[1], t[1]->nbytes, p[3], t[3]->nbytes, p[5], t[5]->nbytes};
    if (hidden) *hidden = dims[0][1];
    if (intermediate) *intermediate = dims[0][0];
    if (out_dim) *out_dim = dims[2][0];
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_st_deepseek_router(const objeta_hip_st_model* m, uint64_t layer, int32_t mtp, char* name_buf,
                                      uint64_t cap, objeta_hip_st_info* info) {
    OBJ_GUARD_BEGIN
    if (!m) OBJ_FAIL(kInvalidInput, "find router tensor", "NULL argument");
    // classify_tensor's "router" entries of this layer and family (ffn/mlp tensors
    // with a "gate" or "router" part outside experts), the Hyper-Connection
    // hc_ffn_* tensors excluded, then only names ending in "gate.weight"
    std::vector<std::string> any, gate_w;
    for (const auto& kv : m->index) {
        const std::string& n = kv.first;
        uint64_t l = 0;
        bool is_mtp = false;
        if (!layer_of(n, &l, &is_mtp) || l != layer || is_mtp != (mtp != 0)) continue;
        if (n.find(".ffn.") == std::string::npos && n.find(".mlp.") == std::string::npos) continue;
        if (n.find("experts") != std::string::npos || n.find(".expert.") != std::string::npos) continue;
        if (n.find("hc_ffn_") != std::string::npos) continue;
        if (n.find(".gate.") == std::string::npos && n.find(".router.") == std::string::npos &&
            !(n.size() >= 5 && n.compare(n.size() - 5, 5, ".gate") == 0))
            continue;
        any.push_back(n);
        if (n.size() >= 11 && n.compare(n.size() - 11, 11, "gate.weight") == 0) gate_w.push_back(n);
    }
    const char* fam = mtp ? "Mtp" : "Decoder";
    if (any.empty())
        OBJ_FAIL(kInvalidInput, "find router tensor",
                 strf("no router tensor found for layer %llu and block family %s", (unsigned long long)layer, fam));
    if (gate_w.size() != 1)
        OBJ_FAIL(kInvalidInput, "find router tensor",
                 strf("%zu router tensors found for layer %llu and block family %s", gate_w.size(),
                      (unsigned long long)layer, fam));
    const Tensor& t = *find(m, gate_w[0]);
    if (t.shape.size() != 2)
        OBJ_FAIL(kInvalidInput, "validate router tensor shape",
                 "router tensor '" + gate_w[0] + "' has shape " + shape_str(t.shape) +
                     ", expected [num_experts, hidden_size]");
    if (name_buf && cap) {
        const size_t n = std::min<size_t>(gate_w[0].size(), cap - 1);
        std::memcpy(name_buf, gate_w[0].data(), n);
        name_buf[n] = '\0';
    }
    if (info) fill_info(t, info);
    return 0;
    OBJ_GUARD_END
}

}  // extern "C"
