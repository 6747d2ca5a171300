// loader.cpp -- safetensors checkpoints and HuggingFace config.json into
// device residency (the file formats themselves: st_format.cpp).
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
#include "st_format.hpp"

using namespace atlas;

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
            if (host_malloc_pinned(&buf[k], kChunk) != hipSuccess) {
                (void)hipGetLastError();
                buf[k] = nullptr;
                set_error(ATLAS_ENOMEM, "loader: pinned staging of %zu bytes", kChunk);
                return ATLAS_ENOMEM;
            }
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
    if (!rc && max_raw && dev_malloc(&raw.p, max_raw) != hipSuccess) rc = ATLAS_ENOMEM;
    if (!rc && max_f16 && dev_malloc(&wide.p, max_f16) != hipSuccess) rc = ATLAS_ENOMEM;
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
        shards = index_shards(text);
    } else {
        shards.push_back("model.safetensors");
    }
    std::vector<std::unique_ptr<atlas_st>> files(shards.size());
    for (size_t k = 0; k < shards.size(); ++k)
        LTRY(st_open((base + "/" + shards[k]).c_str(), &files[k]));
    return load_model(files, cfg, out);
}
