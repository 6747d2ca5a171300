// loader.cpp -- safetensors checkpoints and HuggingFace config.json into
// device residency.
//
// Reference: SafetensorsFile, f16_to_f32, load_model_from_safetensors,
// patch_config_from_hf_json and load_model_from_dir
// (crates/atlas-model/src/lib.rs:2048-2570), over the atlas-json parser
// (crates/atlas-json/src/lib.rs:80-349).  The reference reads each file into
// host memory, widens every tensor to f32 and re-encodes bf16 on the host.
// Here a file is memory-mapped, each tensor's bytes go through two pinned
// buffers to a device staging buffer (copy of one buffer overlapping the
// transfer of the other), and the device converts them (F16 -> F32, F32 ->
// bf16 truncation, or the atlas-quant int8/int4 rules) and places the rows
// into the engine's fused layouts (atlas_model_set_tensor_dev).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <memory>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "../../include/atlas_engine.h"
#include "../../include/atlas_loader.h"
#include "common.hpp"
#include "fused.hpp"

#define LTRY(expr)                \
    do {                          \
        const int rc_ = (expr);   \
        if (rc_) return rc_;      \
    } while (0)

// ---------------------------------------------------------------------------
// JSON with atlas-json's value model: integers without '.'/'e' are Int (i64,
// falling back to Float when out of range), objects keep insertion order and
// duplicate keys, as_usize accepts a Float by truncation.
// ---------------------------------------------------------------------------
namespace {

struct Json {
    enum Type { Null, Bool, Int, Float, Str, Arr, Obj } type = Null;
    bool b = false;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const char* key) const {
        if (type != Obj) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;     // first match, as Json::get
        return nullptr;
    }
    // Json::as_i64: Float converts like Rust's `f as i64` (saturating, NaN -> 0)
    bool as_i64(int64_t* out) const {
        if (type == Int) { *out = i; return true; }
        if (type != Float) return false;
        if (f != f) *out = 0;
        else if (f >= 9223372036854775807.0) *out = INT64_MAX;
        else if (f <= -9223372036854775808.0) *out = INT64_MIN;
        else *out = (int64_t)f;
        return true;
    }
    bool as_usize(uint64_t* out) const {
        int64_t v;
        if (!as_i64(&v) || v < 0) return false;
        *out = (uint64_t)v;
        return true;
    }
    bool as_f64(double* out) const {
        if (type == Int) { *out = (double)i; return true; }
        if (type == Float) { *out = f; return true; }
        return false;
    }
    const std::string* as_str() const { return type == Str ? &s : nullptr; }
};

// Strict UTF-8 (what Rust's str::from_utf8 accepts): no overlong forms, no
// surrogates, nothing above U+10FFFF.
bool utf8_valid(const unsigned char* p, size_t n) {
    size_t k = 0;
    while (k < n) {
        const unsigned c = p[k];
        if (c < 0x80) { ++k; continue; }
        int len;
        unsigned lo = 0x80, hi = 0xBF;
        if (c >= 0xC2 && c <= 0xDF) len = 2;
        else if (c >= 0xE0 && c <= 0xEF) {
            len = 3;
            if (c == 0xE0) lo = 0xA0;
            if (c == 0xED) hi = 0x9F;
        } else if (c >= 0xF0 && c <= 0xF4) {
            len = 4;
            if (c == 0xF0) lo = 0x90;
            if (c == 0xF4) hi = 0x8F;
        } else {
            return false;
        }
        if (k + len > n) return false;
        if (p[k + 1] < lo || p[k + 1] > hi) return false;
        for (int j = 2; j < len; ++j)
            if (p[k + j] < 0x80 || p[k + j] > 0xBF) return false;
        k += len;
    }
    return true;
}

class JsonParser {
public:
    JsonParser(const char* s, size_t n) : src_((const unsigned char*)s), n_(n) {}

    // Json::parse: one value, then only whitespace
    bool parse(Json* out, std::string* err) {
        if (!value(out)) { *err = msg_; return false; }
        ws();
        if (pos_ != n_) { fail("trailing data after JSON value"); *err = msg_; return false; }
        return true;
    }

private:
    const unsigned char* src_;
    size_t n_, pos_ = 0;
    std::string msg_;

    int peek() const { return pos_ < n_ ? src_[pos_] : -1; }
    int advance() { return pos_ < n_ ? src_[pos_++] : -1; }
    bool fail(const char* what) {
        char b[160];
        snprintf(b, sizeof b, "%s at byte %zu", what, pos_);
        msg_ = b;
        return false;
    }
    void ws() {
        while (pos_ < n_ && (src_[pos_] == ' ' || src_[pos_] == '\t' || src_[pos_] == '\n' ||
                             src_[pos_] == '\r'))
            ++pos_;
    }
    bool expect(const char* lit) {
        for (const char* c = lit; *c; ++c)
            if (advance() != (unsigned char)*c) return fail("unexpected literal");
        return true;
    }
    bool value(Json* v) {
        ws();
        const int c = peek();
        if (c < 0) return fail("unexpected end of input");
        if (c == 'n') { v->type = Json::Null; return expect("null"); }
        if (c == 't') { v->type = Json::Bool; v->b = true; return expect("true"); }
        if (c == 'f') { v->type = Json::Bool; v->b = false; return expect("false"); }
        if (c == '"') { v->type = Json::Str; return string(&v->s); }
        if (c == '[') return array(v);
        if (c == '{') return object(v);
        if (c == '-' || (c >= '0' && c <= '9')) return number(v);
        return fail("unexpected byte");
    }
    bool hex4(uint32_t* out) {
        uint32_t code = 0;
        for (int k = 0; k < 4; ++k) {
            const int b = advance();
            uint32_t d;
            if (b >= '0' && b <= '9') d = b - '0';
            else if (b >= 'a' && b <= 'f') d = b - 'a' + 10;
            else if (b >= 'A' && b <= 'F') d = b - 'A' + 10;
            else return fail("invalid hex digit in \\uXXXX");
            code = (code << 4) | d;
        }
        *out = code;
        return true;
    }
    static void utf8(uint32_t cp, std::string* out) {
        if (cp < 0x80) {
            out->push_back((char)cp);
        } else if (cp < 0x800) {
            out->push_back((char)(0xC0 | (cp >> 6)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            out->push_back((char)(0xE0 | (cp >> 12)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            out->push_back((char)(0xF0 | ((cp >> 18) & 0xFF)));
            out->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    bool string(std::string* out) {
        advance();   // opening quote
        out->clear();
        while (true) {
            const int c = advance();
            if (c < 0) return fail("unterminated string");
            if (c == '"') break;
            if (c != '\\') { out->push_back((char)c); continue; }
            const int e = advance();
            switch (e) {
            case '"': out->push_back('"'); break;
            case '\\': out->push_back('\\'); break;
            case '/': out->push_back('/'); break;
            case 'n': out->push_back('\n'); break;
            case 'r': out->push_back('\r'); break;
            case 't': out->push_back('\t'); break;
            case 'b': out->push_back('\b'); break;
            case 'f': out->push_back('\f'); break;
            case 'u': {
                uint32_t cp;
                if (!hex4(&cp)) return false;
                if (cp >= 0xD800 && cp <= 0xDBFF) {
                    // a high surrogate takes the next \uXXXX as its low half
                    uint32_t low;
                    if (!expect("\\u") || !hex4(&low)) return false;
                    cp = 0x10000u + ((cp - 0xD800u) << 10) + (low - 0xDC00u);
                }
                utf8(cp, out);
                break;
            }
            default: return fail("invalid escape sequence");
            }
        }
        if (!utf8_valid((const unsigned char*)out->data(), out->size()))
            return fail("invalid UTF-8 in string");
        return true;
    }
    bool number(Json* v) {
        const size_t start = pos_;
        if (peek() == '-') ++pos_;
        if (peek() == '0') ++pos_;
        else while (peek() >= '0' && peek() <= '9') ++pos_;
        bool is_float = false;
        if (peek() == '.') {
            is_float = true;
            ++pos_;
            while (peek() >= '0' && peek() <= '9') ++pos_;
        }
        if (peek() == 'e' || peek() == 'E') {
            is_float = true;
            ++pos_;
            if (peek() == '+' || peek() == '-') ++pos_;
            while (peek() >= '0' && peek() <= '9') ++pos_;
        }
        const std::string t((const char*)src_ + start, pos_ - start);
        char* end = nullptr;
        if (!is_float) {
            errno = 0;
            const long long iv = strtoll(t.c_str(), &end, 10);
            if (!t.empty() && end == t.c_str() + t.size() && errno == 0) {
                v->type = Json::Int;
                v->i = iv;
                return true;
            }
        }
        // a float literal, or an integer beyond i64
        const bool digits = t.find_first_of("0123456789") != std::string::npos;
        const double fv = strtod(t.c_str(), &end);
        if (!digits || end != t.c_str() + t.size()) return fail("invalid number");
        v->type = Json::Float;
        v->f = fv;
        return true;
    }
    bool array(Json* v) {
        advance();
        v->type = Json::Arr;
        ws();
        if (peek() == ']') { advance(); return true; }
        while (true) {
            v->arr.emplace_back();
            if (!value(&v->arr.back())) return false;
            ws();
            const int c = advance();
            if (c == ']') return true;
            if (c != ',') return fail("expected ',' or ']'");
        }
    }
    bool object(Json* v) {
        advance();
        v->type = Json::Obj;
        ws();
        if (peek() == '}') { advance(); return true; }
        while (true) {
            ws();
            if (peek() != '"') return fail("expected '\"' for object key");
            std::string key;
            if (!string(&key)) return false;
            ws();
            if (advance() != ':') return fail("expected ':'");
            Json val;
            if (!value(&val)) return false;
            v->obj.emplace_back(std::move(key), std::move(val));
            ws();
            const int c = advance();
            if (c == '}') return true;
            if (c != ',') return fail("expected ',' or '}'");
        }
    }
};

bool read_text(const std::string& path, std::string* out, std::string* err) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) { *err = strerror(errno); return false; }
    out->clear();
    char buf[65536];
    size_t k;
    while ((k = fread(buf, 1, sizeof buf, f)) > 0) out->append(buf, k);
    const bool ok = !ferror(f);
    fclose(f);
    if (!ok) *err = "read error";
    return ok;
}

}  // namespace

// ---------------------------------------------------------------------------
// SafetensorsFile (lib.rs:2048-2241)
// ---------------------------------------------------------------------------
struct StTensor {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    uint64_t start = 0, end = 0;
};

struct atlas_st {
    std::vector<StTensor> tensors;
    const uint8_t* data = nullptr;      // the data section (after the header)
    size_t data_len = 0;
    void* map = nullptr;                // memory map of the file (open)
    size_t map_len = 0;
    std::vector<uint8_t> owned;         // copied bytes (from_bytes)
    ~atlas_st() {
        if (map) munmap(map, map_len);
    }
};

namespace {

using atlas::set_error;

// SafetensorsFile::from_bytes (lib.rs:2080-2125) over bytes that st keeps alive
int st_parse(atlas_st* st, const uint8_t* bytes, size_t n) {
    if (n < 8) {
        set_error(ATLAS_EINVAL, "safetensors: file too short");
        return ATLAS_EINVAL;
    }
    uint64_t hs = 0;
    for (int k = 7; k >= 0; --k) hs = (hs << 8) | bytes[k];      // little-endian u64
    if (hs > n - 8) {
        set_error(ATLAS_EINVAL, "safetensors: header truncated");
        return ATLAS_EINVAL;
    }
    const char* hdr = (const char*)bytes + 8;
    if (!utf8_valid((const unsigned char*)hdr, hs)) {
        set_error(ATLAS_EINVAL, "safetensors: header not UTF-8");
        return ATLAS_EINVAL;
    }
    Json root;
    std::string err;
    if (!JsonParser(hdr, hs).parse(&root, &err)) {
        set_error(ATLAS_EINVAL, "safetensors header JSON: %s", err.c_str());
        return ATLAS_EINVAL;
    }
    st->tensors.clear();
    if (root.type == Json::Obj) {
        for (const auto& kv : root.obj) {
            if (kv.first == "__metadata__") continue;
            const Json& d = kv.second;
            StTensor t;
            t.name = kv.first;
            const Json* dt = d.get("dtype");
            t.dtype = dt && dt->as_str() ? *dt->as_str() : std::string("F32");
            const Json* sh = d.get("shape");
            if (sh && sh->type == Json::Arr)
                for (const Json& x : sh->arr) {
                    uint64_t u;
                    if (x.as_usize(&u)) t.shape.push_back(u);   // filter_map(as_usize)
                }
            const Json* off = d.get("data_offsets");
            if (!off || off->type != Json::Arr) {
                set_error(ATLAS_EINVAL, "missing data_offsets for %s", kv.first.c_str());
                return ATLAS_EINVAL;
            }
            if (off->arr.size() < 2) {
                set_error(ATLAS_EINVAL, "data_offsets for %s needs two entries", kv.first.c_str());
                return ATLAS_EINVAL;
            }
            if (!off->arr[0].as_usize(&t.start)) t.start = 0;
            if (!off->arr[1].as_usize(&t.end)) t.end = 0;
            st->tensors.push_back(std::move(t));
        }
    }
    st->data = bytes + 8 + hs;
    st->data_len = n - 8 - hs;
    return ATLAS_OK;
}

int st_open(const char* path, std::unique_ptr<atlas_st>* out) {
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        set_error(ATLAS_EIO, "safetensors: %s: %s", path, strerror(errno));
        return ATLAS_EIO;
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        set_error(ATLAS_EIO, "safetensors: %s: %s", path, strerror(errno));
        close(fd);
        return ATLAS_EIO;
    }
    std::unique_ptr<atlas_st> st(new atlas_st());
    const size_t n = (size_t)sb.st_size;
    if (n > 0) {
        void* p = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            set_error(ATLAS_EIO, "safetensors: mmap %s: %s", path, strerror(errno));
            close(fd);
            return ATLAS_EIO;
        }
        (void)madvise(p, n, MADV_SEQUENTIAL);
        st->map = p;
        st->map_len = n;
    }
    close(fd);
    LTRY(st_parse(st.get(), (const uint8_t*)st->map, n));
    *out = std::move(st);
    return ATLAS_OK;
}

const StTensor* st_find(const atlas_st* st, const char* name) {
    for (const auto& t : st->tensors)
        if (t.name == name) return &t;      // first match, as the reference's find
    return nullptr;
}

int elem_bytes(const std::string& dtype) {
    if (dtype == "F32") return 4;
    if (dtype == "BF16" || dtype == "F16") return 2;
    return 0;
}

// The byte range of a tensor, checked against the data section.
int st_range(const atlas_st* st, const StTensor& t, const uint8_t** p, size_t* n) {
    if (t.start > t.end || t.end > st->data_len) {
        set_error(ATLAS_EINVAL, "tensor '%s': bytes [%llu, %llu) outside the %zu-byte data section",
                  t.name.c_str(), (unsigned long long)t.start, (unsigned long long)t.end,
                  st->data_len);
        return ATLAS_EINVAL;
    }
    *p = st->data + t.start;
    *n = (size_t)(t.end - t.start);
    return ATLAS_OK;
}

// f16_to_f32 (lib.rs:2243-2263)
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    if (ex == 0) {
        const float m = (float)mant * 5.9604644775390625e-8f;    // (mant / 1024) * 2^-14
        return sign ? -m : m;
    }
    if (ex == 31) {
        uint32_t bits = mant ? 0x7FC00000u : (sign ? 0xFF800000u : 0x7F800000u);
        float f;
        memcpy(&f, &bits, 4);
        return f;
    }
    const uint32_t bits = (sign << 31) | ((ex + 112u) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

// ---- C ABI: SafetensorsFile --------------------------------------------------

ATLAS_API int atlas_st_open(const char* path, atlas_st** out) {
    ATLAS_REQUIRE(path && out, "st_open: null argument");
    *out = nullptr;
    std::unique_ptr<atlas_st> st;
    LTRY(st_open(path, &st));
    *out = st.release();
    return ATLAS_OK;
}

ATLAS_API int atlas_st_from_bytes(const void* bytes, size_t n, atlas_st** out) {
    ATLAS_REQUIRE(out && (bytes || n == 0), "st_from_bytes: null argument");
    *out = nullptr;
    std::unique_ptr<atlas_st> st(new atlas_st());
    st->owned.assign((const uint8_t*)bytes, (const uint8_t*)bytes + n);
    LTRY(st_parse(st.get(), st->owned.data(), n));
    *out = st.release();
    return ATLAS_OK;
}

ATLAS_API void atlas_st_close(atlas_st* st) { delete st; }

ATLAS_API int atlas_st_count(const atlas_st* st) { return st ? (int)st->tensors.size() : -1; }

ATLAS_API int atlas_st_find(const atlas_st* st, const char* name) {
    if (!st || !name) return -1;
    for (size_t k = 0; k < st->tensors.size(); ++k)
        if (st->tensors[k].name == name) return (int)k;
    return -1;
}

ATLAS_API int atlas_st_desc(const atlas_st* st, int index, const char** name, const char** dtype,
                            int* ndim, const uint64_t** shape, uint64_t* offsets) {
    ATLAS_REQUIRE(st && index >= 0 && index < (int)st->tensors.size(), "st_desc: index %d", index);
    const StTensor& t = st->tensors[index];
    if (name) *name = t.name.c_str();
    if (dtype) *dtype = t.dtype.c_str();
    if (ndim) *ndim = (int)t.shape.size();
    if (shape) *shape = t.shape.data();
    if (offsets) { offsets[0] = t.start; offsets[1] = t.end; }
    return ATLAS_OK;
}

ATLAS_API int atlas_st_get_f32(const atlas_st* st, const char* name, float* out, size_t cap,
                               size_t* n_out) {
    ATLAS_REQUIRE(st && name && n_out, "st_get_f32: null argument");
    const StTensor* t = st_find(st, name);
    if (!t) {
        set_error(ATLAS_EINVAL, "tensor '%s' not found", name);
        return ATLAS_EINVAL;
    }
    const int eb = elem_bytes(t->dtype);
    if (!eb) {
        set_error(ATLAS_EUNSUPPORTED, "unsupported dtype: %s", t->dtype.c_str());
        return ATLAS_EUNSUPPORTED;
    }
    const uint8_t* p;
    size_t nb;
    LTRY(st_range(st, *t, &p, &nb));
    const size_t n = nb / eb;              // chunks_exact: a ragged tail is dropped
    *n_out = n;
    if (!out) return ATLAS_OK;             // size query
    ATLAS_REQUIRE(cap >= n, "st_get_f32: '%s' has %zu elements, buffer %zu", name, n, cap);
    for (size_t k = 0; k < n; ++k) {
        if (t->dtype == "F32") {
            memcpy(out + k, p + 4 * k, 4);
        } else {
            const uint16_t h = (uint16_t)(p[2 * k] | (p[2 * k + 1] << 8));
            if (t->dtype == "BF16") {
                const uint32_t bits = (uint32_t)h << 16;
                memcpy(out + k, &bits, 4);
            } else {
                out[k] = f16_to_f32(h);
            }
        }
    }
    return ATLAS_OK;
}

ATLAS_API int atlas_st_get_bf16(const atlas_st* st, const char* name, uint16_t* out, size_t cap,
                                size_t* n_out) {
    ATLAS_REQUIRE(st && name && n_out, "st_get_bf16: null argument");
    const StTensor* t = st_find(st, name);
    if (!t) {
        set_error(ATLAS_EINVAL, "tensor '%s' not found", name);
        return ATLAS_EINVAL;
    }
    if (t->dtype != "BF16") {
        set_error(ATLAS_EINVAL, "tensor '%s' dtype is '%s', not BF16", name, t->dtype.c_str());
        return ATLAS_EINVAL;
    }
    const uint8_t* p;
    size_t nb;
    LTRY(st_range(st, *t, &p, &nb));
    const size_t n = nb / 2;
    *n_out = n;
    if (!out) return ATLAS_OK;
    ATLAS_REQUIRE(cap >= n, "st_get_bf16: '%s' has %zu elements, buffer %zu", name, n, cap);
    memcpy(out, p, n * 2);                 // little-endian host
    return ATLAS_OK;
}

ATLAS_API float atlas_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

// ---- config.json (patch_config_from_hf_json, lib.rs:2367-2432) ---------------

ATLAS_API int atlas_config_patch_hf_json(const char* path, atlas_model_config* cfg,
                                         uint8_t* layer_types, int cap, int* n_layer_types,
                                         int64_t* eos_token_id) {
    ATLAS_REQUIRE(path && cfg && n_layer_types && eos_token_id && cap >= 0 &&
                  (layer_types || cap == 0), "config patch: null argument");
    std::string text, err;
    if (!read_text(path, &text, &err)) {
        set_error(ATLAS_EIO, "config.json read: %s: %s", path, err.c_str());
        return ATLAS_EIO;
    }
    Json j;
    if (!utf8_valid((const unsigned char*)text.data(), text.size()) ||
        !JsonParser(text.data(), text.size()).parse(&j, &err)) {
        set_error(ATLAS_EINVAL, "config.json parse: %s", err.empty() ? "not UTF-8" : err.c_str());
        return ATLAS_EINVAL;
    }
    *n_layer_types = -1;
    if (const Json* lt = j.get("layer_types"); lt && lt->type == Json::Arr) {
        // "sliding_attention" -> Sliding, anything else -> Full
        for (size_t k = 0; k < lt->arr.size() && (int)k < cap; ++k) {
            const std::string* s = lt->arr[k].as_str();
            layer_types[k] = s && *s == "sliding_attention" ? 1 : 0;
        }
        *n_layer_types = (int)lt->arr.size();
    }
    uint64_t u;
    if (const Json* sw = j.get("sliding_window"); sw && sw->as_usize(&u)) {
        ATLAS_REQUIRE(u <= 0x7FFFFFFF, "config.json: sliding_window %llu", (unsigned long long)u);
        cfg->sliding_window = (int)u;
    }
    if (const Json* rs = j.get("rope_scaling")) {
        const Json* t = rs->get("rope_type");
        if (t && t->as_str() && *t->as_str() == "yarn") {
            double v;
            const Json* x;
            cfg->yarn = 1;
            cfg->yarn_factor = (x = rs->get("factor")) && x->as_f64(&v) ? (float)v : 1.0f;
            uint64_t om = (uint64_t)cfg->max_seq;
            if ((x = rs->get("original_max_position_embeddings"))) (void)x->as_usize(&om);
            ATLAS_REQUIRE(om <= 0x7FFFFFFF, "config.json: original_max_position_embeddings");
            cfg->yarn_orig_max_pos = (int)om;
            cfg->yarn_attn_factor = (x = rs->get("attention_factor")) && x->as_f64(&v) ? (float)v : 1.0f;
            cfg->yarn_beta_fast = (x = rs->get("beta_fast")) && x->as_f64(&v) ? (float)v : 32.0f;
            cfg->yarn_beta_slow = (x = rs->get("beta_slow")) && x->as_f64(&v) ? (float)v : 1.0f;
        }
    }
    double v;
    if (const Json* x = j.get("rope_theta"); x && x->as_f64(&v)) cfg->rope_theta = (float)v;
    if (const Json* x = j.get("rms_norm_eps"); x && x->as_f64(&v)) cfg->rms_eps = (float)v;
    if (const Json* x = j.get("eos_token_id"); x && x->as_usize(&u))
        *eos_token_id = (int64_t)(uint32_t)u;          // `eos as u32`
    return ATLAS_OK;
}

// ---- model loading (load_model_from_safetensors / load_model_from_dir) --------
namespace {

struct Placement {
    const atlas_st* st;
    const StTensor* t;
    int kind, layer;
    size_t file;                   // index of st in the file list
};

// "model.layers.N." / "layers.N." with N < n_layers in canonical decimal
// (the reference tests each prefix format!("model.layers.{i}.") in turn)
bool layer_local(const std::string& name, int n_layers, int* layer, std::string* local) {
    size_t p;
    if (name.compare(0, 13, "model.layers.") == 0) p = 13;
    else if (name.compare(0, 7, "layers.") == 0) p = 7;
    else return false;
    size_t q = p;
    while (q < name.size() && name[q] >= '0' && name[q] <= '9') ++q;
    if (q == p || q >= name.size() || name[q] != '.') return false;
    if (name[p] == '0' && q - p > 1) return false;           // "01" is no "{i}"
    if (q - p > 9) return false;
    const int i = atoi(name.substr(p, q - p).c_str());
    if (i >= n_layers) return false;
    *layer = i;
    *local = name.substr(q + 1);
    return true;
}

int expected_numel(const atlas_model_config& c, int kind, size_t* n) {
    const size_t d = c.d_model, hd = c.d_model / c.n_heads, kvd = hd * c.n_kv_heads;
    switch (kind) {
    case ATLAS_T_WQ: case ATLAS_T_WO: *n = d * d; break;
    case ATLAS_T_WK: case ATLAS_T_WV: *n = kvd * d; break;
    case ATLAS_T_W_GATE: case ATLAS_T_W_UP: case ATLAS_T_W_DOWN: *n = (size_t)c.ffn_hidden * d; break;
    case ATLAS_T_ATTN_NORM: case ATLAS_T_FFN_NORM: case ATLAS_T_FINAL_NORM: *n = d; break;
    case ATLAS_T_Q_NORM: *n = (size_t)c.n_heads * hd; break;
    case ATLAS_T_K_NORM: *n = kvd; break;
    case ATLAS_T_EMBED: case ATLAS_T_LM_HEAD: *n = (size_t)c.vocab * d; break;
    default: return ATLAS_EINVAL;
    }
    return ATLAS_OK;
}

struct PinnedRing {
    static constexpr size_t kChunk = 64u << 20;
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    int next = 0;
    int init() {
        for (int k = 0; k < 2; ++k) {
            ATLAS_HIP(hipHostMalloc(&buf[k], kChunk, hipHostMallocDefault));
            ATLAS_HIP(hipEventCreateWithFlags(&ev[k], hipEventDisableTiming));
        }
        return ATLAS_OK;
    }
    ~PinnedRing() {
        for (int k = 0; k < 2; ++k) {
            if (ev[k]) {
                if (used[k]) (void)hipEventSynchronize(ev[k]);
                (void)hipEventDestroy(ev[k]);
            }
            if (buf[k]) (void)hipHostFree(buf[k]);
        }
    }
    // bytes [p, p + n) of host memory to dst on stream st: each chunk is copied
    // into a pinned buffer the previous transfer out of it has released, by
    // kThreads threads (one thread's copy out of the page cache, faults
    // included, runs at a third of the host-to-device rate)
    static constexpr int kThreads = 8;
    static void copy_mt(void* dst, const uint8_t* src, size_t len) {
        if (len < (4u << 20)) {
            memcpy(dst, src, len);
            return;
        }
        const size_t part = ((len + kThreads - 1) / kThreads + 4095) & ~(size_t)4095;
        std::thread th[kThreads];
        int nt = 0;
        for (size_t o = 0; o < len; o += part) {
            const size_t l = std::min(part, len - o);
            th[nt++] = std::thread([=] { memcpy((uint8_t*)dst + o, src + o, l); });
        }
        for (int k = 0; k < nt; ++k) th[k].join();
    }
    int upload(void* dst, const uint8_t* p, size_t n, hipStream_t st) {
        for (size_t off = 0; off < n; off += kChunk) {
            const size_t len = std::min(kChunk, n - off);
            const int k = next;
            next ^= 1;
            if (used[k]) ATLAS_HIP(hipEventSynchronize(ev[k]));
            copy_mt(buf[k], p + off, len);
            ATLAS_HIP(hipMemcpyAsync((char*)dst + off, buf[k], len, hipMemcpyHostToDevice, st));
            ATLAS_HIP(hipEventRecord(ev[k], st));
            used[k] = true;
        }
        return ATLAS_OK;
    }
};

struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) {
            (void)hipDeviceSynchronize();
            (void)hipFree(p);
        }
    }
};

// Builds and fills a model from the tensors of `files` in application order
// (file by file, each in header order; a later tensor of the same name is
// applied after an earlier one, as the reference's insertion into its map).
int load_model(const std::vector<std::unique_ptr<atlas_st>>& files, atlas_model_config cfg,
               atlas_model** out) {
    // every tensor must convert to f32 (the reference calls get_f32 on each)
    struct Src { const atlas_st* st; const StTensor* t; size_t file; };
    std::vector<Src> all;
    for (size_t fi = 0; fi < files.size(); ++fi) {
        const auto& f = files[fi];
        for (const auto& t : f->tensors) {
            if (!elem_bytes(t.dtype)) {
                set_error(ATLAS_EUNSUPPORTED, "unsupported dtype: %s (tensor '%s')", t.dtype.c_str(),
                          t.name.c_str());
                return ATLAS_EUNSUPPORTED;
            }
            const uint8_t* p;
            size_t nb;
            LTRY(st_range(f.get(), t, &p, &nb));
            all.push_back({f.get(), &t, fi});
        }
    }
    // architecture from the tensor names, before any placement
    bool has_lm_head = false, post_norm = false;
    const StTensor* embed = nullptr;
    for (const auto& a : all) {
        const std::string& nm = a.t->name;
        if (nm == "lm_head.weight") has_lm_head = true;
        if (nm.find("post_feedforward_layernorm") != std::string::npos) post_norm = true;
        if (nm == "model.embed_tokens.weight" || nm == "tok_embeddings.weight") embed = a.t;
    }
    if (embed) {
        // Embedding::from_data: vocab = len / d_model
        const size_t n = (embed->end - embed->start) / elem_bytes(embed->dtype);
        ATLAS_REQUIRE(n / cfg.d_model >= 1 && n / cfg.d_model <= 0x7FFFFFFF,
                      "embedding of %zu elements for d_model %d", n, cfg.d_model);
        cfg.vocab = (int)(n / cfg.d_model);
    }
    cfg.post_norm = post_norm ? 1 : 0;
    // placements
    std::vector<Placement> pl;
    std::vector<int> q_norm_layers(cfg.n_layers, 0), k_norm_layers(cfg.n_layers, 0);
    for (const auto& a : all) {
        const std::string& nm = a.t->name;
        auto add = [&](int kind, int layer) { pl.push_back({a.st, a.t, kind, layer, a.file}); };
        if (nm == "model.embed_tokens.weight" || nm == "tok_embeddings.weight") {
            add(ATLAS_T_EMBED, 0);
            if (!has_lm_head) add(ATLAS_T_LM_HEAD, 0);           // tied
        } else if (nm == "model.norm.weight" || nm == "norm.weight") {
            add(ATLAS_T_FINAL_NORM, 0);
        } else if (nm == "lm_head.weight") {
            add(ATLAS_T_LM_HEAD, 0);
        } else {
            int li;
            std::string loc;
            if (!layer_local(nm, cfg.n_layers, &li, &loc)) continue;
            if (loc == "self_attn.q_proj.weight") add(ATLAS_T_WQ, li);
            else if (loc == "self_attn.k_proj.weight") add(ATLAS_T_WK, li);
            else if (loc == "self_attn.v_proj.weight") add(ATLAS_T_WV, li);
            else if (loc == "self_attn.o_proj.weight") add(ATLAS_T_WO, li);
            else if (loc == "mlp.gate_proj.weight") add(ATLAS_T_W_GATE, li);
            else if (loc == "mlp.up_proj.weight") add(ATLAS_T_W_UP, li);
            else if (loc == "mlp.down_proj.weight") add(ATLAS_T_W_DOWN, li);
            else if (loc == "input_layernorm.weight") add(ATLAS_T_ATTN_NORM, li);
            else if (loc == "post_attention_layernorm.weight")
                add(post_norm ? ATLAS_T_ATTN_NORM : ATLAS_T_FFN_NORM, li);
            else if (loc == "post_feedforward_layernorm.weight") add(ATLAS_T_FFN_NORM, li);
            else if (loc == "self_attn.q_norm.weight") { add(ATLAS_T_Q_NORM, li); q_norm_layers[li] = 1; }
            else if (loc == "self_attn.k_norm.weight") { add(ATLAS_T_K_NORM, li); k_norm_layers[li] = 1; }
        }
    }
    // QK-norm is on where the file has its weights; the engine applies it to
    // every layer and both q and k, so the file must hold all of them or none
    int nq = 0, nk = 0;
    for (int li = 0; li < cfg.n_layers; ++li) { nq += q_norm_layers[li]; nk += k_norm_layers[li]; }
    ATLAS_REQUIRE((nq == 0 && nk == 0) || (nq == cfg.n_layers && nk == cfg.n_layers),
                  "QK-norm weights in %d (q) and %d (k) of %d layers: all or none supported", nq,
                  nk, cfg.n_layers);
    cfg.qk_norm = nq > 0 ? 1 : 0;
    // one placement per target: the last in application order (an earlier
    // one would be overwritten), so the reads below may go in file order
    {
        std::vector<Placement> last;
        std::vector<char> taken((size_t)(cfg.n_layers + 1) * 16, 0);
        for (size_t k = pl.size(); k-- > 0;) {
            char& t = taken[(size_t)pl[k].layer * 16 + pl[k].kind];
            if (t) continue;
            t = 1;
            last.push_back(pl[k]);
        }
        std::reverse(last.begin(), last.end());
        pl.swap(last);
    }
    // element counts against the model's shapes
    for (const auto& p : pl) {
        size_t want;
        LTRY(expected_numel(cfg, p.kind, &want));
        const size_t n = (p.t->end - p.t->start) / elem_bytes(p.t->dtype);
        ATLAS_REQUIRE(n == want, "tensor '%s' has %zu elements, the model expects %zu",
                      p.t->name.c_str(), n, want);
    }
    atlas_model* m = atlas_model_create(&cfg);
    if (!m) return atlas_last_error_code() ? atlas_last_error_code() : ATLAS_EINVAL;
    auto fail = [&](int rc) {
        atlas_model_destroy(m);
        return rc;
    };
    // tensors the file lacks keep a random init (OlmoModel::new initialises
    // every tensor before the file overwrites it)
    {
        // global kinds (embedding, lm_head, final norm) are placed at layer 0
        std::vector<char> seen((size_t)cfg.n_layers * 16, 0);
        for (const auto& p : pl) seen[(size_t)p.layer * 16 + p.kind] = 1;
        bool missing = !seen[ATLAS_T_EMBED] || !seen[ATLAS_T_LM_HEAD] || !seen[ATLAS_T_FINAL_NORM];
        for (int li = 0; li < cfg.n_layers && !missing; ++li)
            for (int k = ATLAS_T_WQ; k <= ATLAS_T_K_NORM; ++k) {
                if ((k == ATLAS_T_Q_NORM || k == ATLAS_T_K_NORM) && !cfg.qk_norm) continue;
                if (!seen[(size_t)li * 16 + k]) missing = true;
            }
        if (missing) {
            const int rc = atlas_model_init_random(m, 0x5DEECE66DULL);
            if (rc) return fail(rc);
        }
    }
    // read in file order: sequential pages of each map
    std::stable_sort(pl.begin(), pl.end(), [](const Placement& a, const Placement& b) {
        if (a.file != b.file) return a.file < b.file;
        return a.t->start < b.t->start;
    });
    size_t max_raw = 0, max_f16 = 0;
    for (const auto& p : pl) {
        const size_t nb = p.t->end - p.t->start;
        max_raw = std::max(max_raw, nb);
        if (p.t->dtype == "F16") max_f16 = std::max(max_f16, nb / 2 * 4);
    }
    hipStream_t st = (hipStream_t)atlas_model_stream(m);
    PinnedRing ring;
    DevBuf raw, wide;
    int rc = ring.init();
    if (!rc && max_raw && hipMalloc(&raw.p, max_raw) != hipSuccess) rc = ATLAS_ENOMEM;
    if (!rc && max_f16 && hipMalloc(&wide.p, max_f16) != hipSuccess) rc = ATLAS_ENOMEM;
    if (rc) {
        (void)hipGetLastError();
        if (rc == ATLAS_ENOMEM) set_error(ATLAS_ENOMEM, "loader: staging buffers");
        return fail(rc);
    }
    atlas_load_scratch* scratch = atlas_load_scratch_create();
    const StTensor* prev = nullptr;
    for (const auto& p : pl) {
        const uint8_t* src;
        size_t nb;
        rc = st_range(p.st, *p.t, &src, &nb);
        // a tied embedding is placed twice from one upload
        if (!rc && p.t != prev) rc = ring.upload(raw.p, src, nb, st);
        prev = p.t;
        if (rc) break;
        const int eb = elem_bytes(p.t->dtype);
        const size_t n = nb / eb;
        const void* dsrc = raw.p;
        int dtype = eb == 4 ? ATLAS_W_F32 : ATLAS_W_BF16;
        if (p.t->dtype == "F16") {
            rc = atlas::cvt_launch(atlas::CVT_F16_F32, raw.p, wide.p, (long)n, st);
            if (rc) break;
            dsrc = wide.p;
            dtype = ATLAS_W_F32;
        }
        rc = atlas_model_set_tensor_dev(m, p.kind, p.layer, dsrc, dtype, (int64_t)n, scratch);
        if (rc) break;
    }
    if (!rc && hipStreamSynchronize(st) != hipSuccess) {
        set_error(ATLAS_EHIP, "loader: stream synchronisation failed");
        rc = ATLAS_EHIP;
    }
    atlas_load_scratch_destroy(scratch);
    if (!rc) rc = atlas_model_reset(m);
    if (rc) return fail(rc);
    *out = m;
    return ATLAS_OK;
}

}  // namespace

ATLAS_API int atlas_model_load_safetensors(const char* path, const atlas_model_config* cfg,
                                           atlas_model** out) {
    ATLAS_REQUIRE(path && cfg && out, "load_safetensors: null argument");
    *out = nullptr;
    std::vector<std::unique_ptr<atlas_st>> files(1);
    LTRY(st_open(path, &files[0]));
    return load_model(files, *cfg, out);
}

ATLAS_API int atlas_model_load_dir(const char* dir, const atlas_model_config* cfg_in,
                                   atlas_model** out, int64_t* eos_token_id) {
    ATLAS_REQUIRE(dir && cfg_in && out && eos_token_id, "load_dir: null argument");
    *out = nullptr;
    *eos_token_id = -1;
    atlas_model_config cfg = *cfg_in;
    const std::string base(dir);
    // config.json overlay
    std::vector<uint8_t> types((size_t)std::max(cfg.n_layers, 0), 0);
    const std::string cj = base + "/config.json";
    struct stat sb;
    if (stat(cj.c_str(), &sb) == 0) {
        int n_types = -1;
        LTRY(atlas_config_patch_hf_json(cj.c_str(), &cfg, types.data(), (int)types.size(), &n_types,
                                        eos_token_id));
        if (n_types >= 0) {
            // cfg.layer_types.get(i): entries past the list are Full
            for (int k = std::max(n_types, 0); k < cfg.n_layers; ++k) types[k] = 0;
            cfg.layer_sliding = types.data();
        }
    }
    // shards: every quoted string of the index ending in ".safetensors",
    // deduplicated and sorted; model.safetensors when there is no index
    const std::string ij = base + "/model.safetensors.index.json";
    std::vector<std::string> shards;
    if (stat(ij.c_str(), &sb) == 0) {
        std::string text, err;
        if (!read_text(ij, &text, &err)) {
            set_error(ATLAS_EIO, "index.json: %s", err.c_str());
            return ATLAS_EIO;
        }
        size_t a = 0;
        while (a <= text.size()) {
            const size_t b = text.find('"', a);
            const std::string seg = text.substr(a, b == std::string::npos ? std::string::npos : b - a);
            if (seg.size() >= 12 && seg.compare(seg.size() - 12, 12, ".safetensors") == 0)
                shards.push_back(seg);
            if (b == std::string::npos) break;
            a = b + 1;
        }
        std::sort(shards.begin(), shards.end());
        shards.erase(std::unique(shards.begin(), shards.end()), shards.end());
    } else {
        shards.push_back("model.safetensors");
    }
    std::vector<std::unique_ptr<atlas_st>> files(shards.size());
    for (size_t k = 0; k < shards.size(); ++k)
        LTRY(st_open((base + "/" + shards[k]).c_str(), &files[k]));
    return load_model(files, cfg, out);
}
