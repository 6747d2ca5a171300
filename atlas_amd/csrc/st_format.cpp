// st_format.cpp -- the checkpoint formats on the host: safetensors headers,
// HuggingFace config.json and the shard index, over a JSON parser with
// atlas-json's value model.  No device code: this part also builds with a
// plain C++ compiler, which is how it is run under AddressSanitizer and
// UndefinedBehaviorSanitizer against malformed files.
//
// Reference: SafetensorsFile, f16_to_f32, patch_config_from_hf_json and the
// shard list of load_model_from_dir (crates/atlas-model/src/lib.rs:2048-2570),
// over the atlas-json parser (crates/atlas-json/src/lib.rs:80-349).
#include "st_format.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

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
    // Nesting bound: the parser recurses per array / object level, so an
    // unbounded depth would let a crafted header overflow the stack.
    static constexpr int kMaxDepth = 512;
    const unsigned char* src_;
    size_t n_, pos_ = 0;
    int depth_ = 0;
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
        if (c == '[' || c == '{') {
            if (depth_ >= kMaxDepth) return fail("nesting deeper than 512 levels");
            ++depth_;
            const bool ok = c == '[' ? array(v) : object(v);
            --depth_;
            return ok;
        }
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

}  // namespace

namespace atlas {

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

}  // namespace atlas

// ---------------------------------------------------------------------------
// SafetensorsFile (lib.rs:2048-2241)
// ---------------------------------------------------------------------------
atlas_st::~atlas_st() {
    if (map) munmap(map, map_len);
}

namespace atlas {
namespace {

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

}  // namespace

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
static float f16_to_f32(uint16_t h) {
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

// The shard list of a model.safetensors.index.json (load_model_from_dir,
// lib.rs:2437-2570): every quoted string ending in ".safetensors",
// deduplicated and sorted.
std::vector<std::string> index_shards(const std::string& text) {
    std::vector<std::string> shards;
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
    return shards;
}

}  // namespace atlas

using namespace atlas;

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

