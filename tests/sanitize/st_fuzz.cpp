// st_fuzz.cpp -- drives the host-side checkpoint parsers (st_format.cpp:
// safetensors headers and data ranges, config.json, the shard index) over a
// corpus of malformed files and a bounded, seeded mutation fuzz.  Built by
// tests/test_loader_sanitize.py with g++ -fsanitize=address,undefined and
// -fno-sanitize-recover, so any out-of-bounds access, use-after-free, leak
// or undefined behaviour aborts the run; a clean run exits 0 and prints a
// summary line.  Test infrastructure: not part of the library.
//
// Usage: st_fuzz <workdir> <iterations> <seed> [corpus files...]
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../atlas_amd/csrc/st_format.hpp"

extern "C" {
int atlas_st_open(const char* path, atlas_st** out);
int atlas_st_from_bytes(const void* bytes, size_t n, atlas_st** out);
void atlas_st_close(atlas_st* st);
int atlas_st_count(const atlas_st* st);
int atlas_st_find(const atlas_st* st, const char* name);
int atlas_st_desc(const atlas_st* st, int index, const char** name, const char** dtype, int* ndim,
                  const uint64_t** shape, uint64_t* offsets);
int atlas_st_get_f32(const atlas_st* st, const char* name, float* out, size_t cap, size_t* n_out);
int atlas_st_get_bf16(const atlas_st* st, const char* name, uint16_t* out, size_t cap,
                      size_t* n_out);
int atlas_config_patch_hf_json(const char* path, atlas_model_config* cfg, uint8_t* layer_types,
                               int cap, int* n_layer_types, int64_t* eos_token_id);
}

namespace {

uint64_t g_state = 0;
uint64_t next_u64() {   // SplitMix64
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
size_t below(size_t n) { return n ? (size_t)(next_u64() % n) : 0; }

using Bytes = std::vector<uint8_t>;

struct Stats { long parsed_ok = 0, parsed_err = 0, reads = 0, configs_ok = 0, shards = 0; };

// Every query a caller can make of a parsed file, with buffers sized from the
// file's own answers.
void exercise(atlas_st* st, Stats& s) {
    const int n = atlas_st_count(st);
    for (int i = 0; i < n; ++i) {
        const char *name = nullptr, *dtype = nullptr;
        int ndim = 0;
        const uint64_t* shape = nullptr;
        uint64_t off[2] = {0, 0};
        if (atlas_st_desc(st, i, &name, &dtype, &ndim, &shape, off) != 0) continue;
        volatile uint64_t sink = 0;
        for (int d = 0; d < ndim; ++d) sink += shape[d];
        (void)sink;
        (void)atlas_st_find(st, name);
        size_t cnt = 0;
        if (atlas_st_get_f32(st, name, nullptr, 0, &cnt) == 0 && cnt <= (64u << 20)) {
            std::vector<float> out(cnt + 1);
            if (atlas_st_get_f32(st, name, out.data(), cnt, &cnt) == 0) ++s.reads;
            if (cnt > 0) (void)atlas_st_get_f32(st, name, out.data(), cnt - 1, &cnt);  // too small
        }
        if (atlas_st_get_bf16(st, name, nullptr, 0, &cnt) == 0 && cnt <= (64u << 20)) {
            std::vector<uint16_t> out(cnt + 1);
            if (atlas_st_get_bf16(st, name, out.data(), cnt, &cnt) == 0) ++s.reads;
        }
    }
    (void)atlas_st_find(st, "");
    (void)atlas_st_desc(st, n, nullptr, nullptr, nullptr, nullptr, nullptr);   // out of range
}

bool write_file(const std::string& path, const Bytes& b) {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = b.empty() || fwrite(b.data(), 1, b.size(), f) == b.size();
    return fclose(f) == 0 && ok;
}

void run_one(const std::string& work, const Bytes& b, Stats& s, bool via_file) {
    atlas_st* st = nullptr;
    if (atlas_st_from_bytes(b.data(), b.size(), &st) == 0) {
        ++s.parsed_ok;
        exercise(st, s);
        atlas_st_close(st);
    } else {
        ++s.parsed_err;
    }
    const std::string path = work + "/case.bin";
    if (!write_file(path, b)) {
        fprintf(stderr, "cannot write %s\n", path.c_str());
        exit(2);
    }
    if (via_file) {
        st = nullptr;
        if (atlas_st_open(path.c_str(), &st) == 0) {
            exercise(st, s);
            atlas_st_close(st);
        }
    }
    // the same bytes as a config.json and as a shard index
    atlas_model_config cfg{};
    cfg.n_layers = 32;
    cfg.max_seq = 4096;
    uint8_t types[48];
    int n_types = 0;
    int64_t eos = -1;
    if (atlas_config_patch_hf_json(path.c_str(), &cfg, types, 48, &n_types, &eos) == 0) ++s.configs_ok;
    s.shards += (long)atlas::index_shards(std::string(b.begin(), b.end())).size();
}

// A safetensors file: 8-byte little-endian header length, JSON header, data.
Bytes safetensors(const std::string& header, const Bytes& data) {
    Bytes b(8);
    uint64_t n = header.size();
    for (int k = 0; k < 8; ++k) b[k] = (uint8_t)(n >> (8 * k));
    b.insert(b.end(), header.begin(), header.end());
    b.insert(b.end(), data.begin(), data.end());
    return b;
}

std::vector<Bytes> seeds() {
    std::vector<Bytes> v;
    Bytes data(64);
    for (size_t k = 0; k < data.size(); ++k) data[k] = (uint8_t)(k * 37 + 11);
    v.push_back(safetensors(
        "{\"__metadata__\":{\"format\":\"pt\"},"
        "\"w\":{\"dtype\":\"F32\",\"shape\":[2,4],\"data_offsets\":[0,32]},"
        "\"b\":{\"dtype\":\"BF16\",\"shape\":[8],\"data_offsets\":[32,48]},"
        "\"h\":{\"dtype\":\"F16\",\"shape\":[8],\"data_offsets\":[48,64]}}",
        data));
    v.push_back(safetensors("{\"x\":{\"dtype\":\"BF16\",\"shape\":[1e300,-1,2.5],"
                            "\"data_offsets\":[0,2]},\"y\":{\"data_offsets\":[0]}}",
                            Bytes(2, 0x80)));
    const std::string cfg =
        "{\"sliding_window\":4096,\"rope_theta\":500000.0,\"rms_norm_eps\":1e-6,"
        "\"eos_token_id\":100257,\"rope_scaling\":{\"rope_type\":\"yarn\",\"factor\":8.0,"
        "\"original_max_position_embeddings\":8192,\"attention_factor\":1.2079441541679836,"
        "\"beta_fast\":32,\"beta_slow\":1},\"layer_types\":[\"sliding_attention\","
        "\"full_attention\",\"sliding_attention\"],\"name\":\"\\u00e9\\ud83d\\ude00\"}";
    v.emplace_back(cfg.begin(), cfg.end());
    const std::string idx =
        "{\"weight_map\":{\"a\":\"model-00001-of-00002.safetensors\","
        "\"b\":\"model-00002-of-00002.safetensors\"}}";
    v.emplace_back(idx.begin(), idx.end());
    return v;
}

const char* kTokens[] = {"{", "}", "[", "]", "\"", ":", ",", "\\u", "\\ud800", "\\udc00",
                         "1e309", "-0", "18446744073709551616", "9223372036854775807",
                         "-9223372036854775809", "null", "true", "\xff", "\xc0\x80",
                         "\"data_offsets\":[0,99999999999]", "\"dtype\":\"F16\"",
                         "\"shape\":[]", "\"data_offsets\":[5,1]"};

Bytes mutate(Bytes b) {
    const int n_ops = 1 + (int)below(4);
    for (int op = 0; op < n_ops; ++op) {
        switch (below(8)) {
        case 0:                                   // bit flip
            if (!b.empty()) b[below(b.size())] ^= (uint8_t)(1u << below(8));
            break;
        case 1:                                   // byte set
            if (!b.empty()) b[below(b.size())] = (uint8_t)next_u64();
            break;
        case 2:                                   // truncate
            b.resize(below(b.size() + 1));
            break;
        case 3: {                                 // delete a run
            if (b.empty()) break;
            const size_t a = below(b.size()), l = 1 + below(16);
            b.erase(b.begin() + a, b.begin() + std::min(b.size(), a + l));
            break;
        }
        case 4: {                                 // insert a JSON token
            const char* t = kTokens[below(sizeof(kTokens) / sizeof(kTokens[0]))];
            b.insert(b.begin() + below(b.size() + 1), t, t + strlen(t));
            break;
        }
        case 5:                                   // header length field
            if (b.size() >= 8) {
                const uint64_t v = below(3) == 0 ? next_u64() : b.size() - 8 + below(16) - 8;
                for (int k = 0; k < 8; ++k) b[k] = (uint8_t)(v >> (8 * k));
            }
            break;
        case 6: {                                 // deep nesting
            const size_t a = below(b.size() + 1), depth = 1 + below(2000);
            const char open = below(2) ? '[' : '{';
            b.insert(b.begin() + a, depth, (uint8_t)open);
            break;
        }
        default: {                                // duplicate a slice
            if (b.empty()) break;
            const size_t a = below(b.size()), l = 1 + below(std::min<size_t>(64, b.size() - a));
            const Bytes slice(b.begin() + a, b.begin() + a + l);
            b.insert(b.begin() + below(b.size() + 1), slice.begin(), slice.end());
            break;
        }
        }
    }
    if (b.size() > (1u << 20)) b.resize(1u << 20);
    return b;
}

// A safetensors file whose header (not its length prefix) is mutated, then
// framed again with a consistent length, so the mutant reaches the tensor
// table and the data-range checks instead of failing on the prefix.
bool split_safetensors(const Bytes& b, std::string* header, Bytes* data) {
    if (b.size() < 8) return false;
    uint64_t n = 0;
    for (int k = 7; k >= 0; --k) n = (n << 8) | b[k];
    if (n > b.size() - 8) return false;
    header->assign(b.begin() + 8, b.begin() + 8 + (long)n);
    data->assign(b.begin() + 8 + (long)n, b.end());
    return true;
}

Bytes mutate_framed(const Bytes& b) {
    std::string header;
    Bytes data;
    if (!split_safetensors(b, &header, &data)) return mutate(b);
    Bytes h(header.begin(), header.end());
    h = mutate(h);
    if (below(4) == 0) data = mutate(data);
    return safetensors(std::string(h.begin(), h.end()), data);
}

// A well-formed header with random tensor entries: dtypes the reader
// accepts and others, shapes and data_offsets inside, past and across the
// data section (reversed, huge, negative, fractional), duplicate names.
std::string rand_num(uint64_t data_len) {
    char b[64];
    switch (below(6)) {
    case 0: snprintf(b, sizeof b, "%llu", (unsigned long long)below(data_len + 1)); break;
    case 1: snprintf(b, sizeof b, "%llu", (unsigned long long)(data_len + below(64))); break;
    case 2: snprintf(b, sizeof b, "%llu", (unsigned long long)next_u64()); break;
    case 3: snprintf(b, sizeof b, "-%llu", (unsigned long long)below(1000)); break;
    case 4: snprintf(b, sizeof b, "%llu.%u", (unsigned long long)below(data_len + 1),
                     (unsigned)below(10)); break;
    default: snprintf(b, sizeof b, "%lluE%u", (unsigned long long)below(10), (unsigned)below(30));
    }
    return b;
}

Bytes random_file() {
    static const char* dtypes[] = {"F32", "BF16", "F16", "I8", "U8", "F64", "", "bf16"};
    const uint64_t data_len = below(4096);
    std::string h = "{";
    const int nt = (int)below(12);
    for (int t = 0; t < nt; ++t) {
        if (t) h += ",";
        char name[32];
        snprintf(name, sizeof name, "\"t%u\"", (unsigned)below(6));
        h += name;
        h += ":{";
        bool first = true;
        auto field = [&](const std::string& f) { if (!first) h += ","; h += f; first = false; };
        if (below(5)) field(std::string("\"dtype\":\"") + dtypes[below(8)] + "\"");
        if (below(4)) {
            std::string sh = "\"shape\":[";
            const int nd = (int)below(5);
            for (int d = 0; d < nd; ++d) sh += (d ? "," : "") + rand_num(64);
            field(sh + "]");
        }
        if (below(8)) {
            std::string off = "\"data_offsets\":[";
            const int no = below(6) ? 2 : (int)below(4);
            for (int d = 0; d < no; ++d) off += (d ? "," : "") + rand_num(data_len);
            field(off + "]");
        }
        h += "}";
    }
    h += "}";
    Bytes data(data_len);
    for (auto& x : data) x = (uint8_t)next_u64();
    return safetensors(h, data);
}

Bytes read_file(const char* path) {
    Bytes b;
    FILE* f = fopen(path, "rb");
    if (!f) return b;
    uint8_t buf[65536];
    size_t k;
    while ((k = fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + k);
    fclose(f);
    return b;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 4) {
        fprintf(stderr, "usage: %s <workdir> <iterations> <seed> [corpus files...]\n", argv[0]);
        return 2;
    }
    const std::string work = argv[1];
    const long iters = atol(argv[2]);
    g_state = strtoull(argv[3], nullptr, 10);
    Stats s;
    long corpus = 0;
    for (int i = 4; i < argc; ++i, ++corpus) run_one(work, read_file(argv[i]), s, true);
    // a header nested far past the parser's bound: an error, not a crash
    {
        std::string deep(200000, '[');
        deep += std::string(200000, ']');
        run_one(work, safetensors(deep, Bytes()), s, false);
        run_one(work, Bytes(deep.begin(), deep.end()), s, false);
    }
    std::vector<Bytes> pool = seeds();
    for (const Bytes& b : pool) run_one(work, b, s, true);
    for (long it = 0; it < iters; ++it) {
        const Bytes& src = pool[below(pool.size())];
        const uint64_t mode = below(3);
        const Bytes b = mode == 0 ? random_file() : mode == 1 ? mutate_framed(src) : mutate(src);
        run_one(work, b, s, it % 64 == 0);
        if (below(16) == 0 && pool.size() < 64) pool.push_back(b);   // keep some mutants
    }
    printf("st_fuzz ok: %ld corpus files, %ld mutants; %ld parsed, %ld rejected, %ld tensor reads, "
           "%ld configs applied, %ld shard names\n",
           corpus, iters, s.parsed_ok, s.parsed_err, s.reads, s.configs_ok, s.shards);
    return 0;
}
