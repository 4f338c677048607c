// GEMM autotuner: benchmark candidate configs on the GPU, keep the fastest,
// cache it in memory and on disk (one JSON file per problem).
//
// Follows GemmTuner (src/t0/auto_gemm.rs:28-417) and auto_gemm
// (auto_gemm.rs:445-480): same lookup order (memory, disk, benchmark), same
// file keys, same defaults (8 candidates, median of 5).  Differences that
// matter on MI355X: candidates come from the 256-CU model of auto_select,
// timings are device time between HIP events (not host time around a
// synchronous dispatch), operands hold random bf16 data (all-zero operands
// let a power-limited GPU clock higher than real data does, which skews the
// ranking), and all candidates share one set of buffers.
//
// The same tuner also serves tune_tile_ir (src/t0/cost_model.rs:757-1013):
// the tile ABI's configs (NT, f32 out, no stream-K), cached as
// tile_ir_MxNxK.json with that file's keys (cost_model.rs:1030-1097).
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>
#include <dirent.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "t0g.h"
#include "t0g_internal.h"

namespace t0g {
namespace {

// Which tuner a result belongs to: GemmTuner (gemm_*.json) or tune_tile_ir
// (tile_ir_*.json, NT with f32 output only).
enum TuneKind : uint32_t { kGemm = 0, kTileIr = 1 };

struct TuneKey {
    uint32_t m, n, k, transpose, out_dtype;
    uint32_t kind = kGemm;
    bool operator<(const TuneKey &o) const {
        return std::tie(kind, m, n, k, transpose, out_dtype) < std::tie(o.kind, o.m, o.n, o.k, o.transpose, o.out_dtype);
    }
};

struct TuneEntry {
    t0g_tune_result result;
    std::vector<std::pair<std::string, double>> all;
};

const char *const kLayoutTag[] = {"nt", "nn", "tn", "tt"};

std::string default_cache_dir() {
    const char *home = getenv("HOME");
    if (home && *home) return std::string(home) + "/.t0_autotune";
    return "/tmp/.t0_autotune";
}

int check_key(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype) {
    if (m == 0 || n == 0 || k == 0) return fail(T0G_ERR_INVALID_ARG, "tune key %ux%ux%u: sizes must be > 0", m, n, k);
    if (transpose > T0G_TT) return fail(T0G_ERR_INVALID_ARG, "bad transpose %u", transpose);
    if (out_dtype > T0G_BF16) return fail(T0G_ERR_INVALID_ARG, "bad out_dtype %u", out_dtype);
    return T0G_OK;
}

std::string config_name(const t0g_gemm_config &cfg) {
    char buf[128];
    if (t0g_config_name(&cfg, buf, sizeof buf)) return "?";
    return buf;
}

std::string tile_name(const t0g_gemm_config &cfg) {
    char buf[128];
    if (t0g_tile_config_name(&cfg, 0, buf, sizeof buf)) return "?";
    return buf;
}

std::string entry_name(const TuneKey &key, const t0g_gemm_config &cfg) {
    return key.kind == kTileIr ? tile_name(cfg) : config_name(cfg);
}

// mkdir -p
int make_dirs(const std::string &dir) {
    std::string cur;
    size_t pos = 0;
    while (pos <= dir.size()) {
        size_t next = dir.find('/', pos);
        if (next == std::string::npos) next = dir.size();
        cur = dir.substr(0, next);
        if (!cur.empty() && mkdir(cur.c_str(), 0755) != 0 && errno != EEXIST)
            return fail(T0G_ERR_INVALID_ARG, "cannot create %s: %s", cur.c_str(), strerror(errno));
        pos = next + 1;
    }
    return T0G_OK;
}

// ---- minimal JSON reading (the files are flat objects written below) --------

// Position just after `"key"` and the following ':' (whitespace allowed), or npos.
size_t value_pos(const std::string &js, const char *key) {
    const std::string needle = std::string("\"") + key + "\"";
    size_t p = 0;
    while ((p = js.find(needle, p)) != std::string::npos) {
        size_t q = p + needle.size();
        while (q < js.size() && isspace((unsigned char)js[q])) ++q;
        if (q < js.size() && js[q] == ':') {
            ++q;
            while (q < js.size() && isspace((unsigned char)js[q])) ++q;
            return q;
        }
        p = q;
    }
    return std::string::npos;
}

bool read_u32(const std::string &js, const char *key, uint32_t *v) {
    size_t p = value_pos(js, key);
    if (p == std::string::npos || p >= js.size() || !isdigit((unsigned char)js[p])) return false;
    unsigned long long x = 0;
    while (p < js.size() && isdigit((unsigned char)js[p])) {
        x = x * 10 + (uint64_t)(js[p++] - '0');
        if (x > 0xFFFFFFFFull) return false;
    }
    *v = (uint32_t)x;
    return true;
}

bool read_f64(const std::string &js, const char *key, double *v) {
    size_t p = value_pos(js, key);
    if (p == std::string::npos) return false;
    const char *s = js.c_str() + p;
    char *end = nullptr;
    double x = strtod(s, &end);
    if (end == s) return false;
    *v = x;
    return true;
}

bool read_bool(const std::string &js, const char *key, bool *v) {
    size_t p = value_pos(js, key);
    if (p == std::string::npos) return false;
    if (js.compare(p, 4, "true") == 0) {
        *v = true;
        return true;
    }
    if (js.compare(p, 5, "false") == 0) {
        *v = false;
        return true;
    }
    return false;
}

// A JSON string without escapes (the only kind written here).
bool read_plain_string(const std::string &js, size_t *p, std::string *out) {
    if (*p >= js.size() || js[*p] != '"') return false;
    size_t e = js.find('"', *p + 1);
    if (e == std::string::npos) return false;
    *out = js.substr(*p + 1, e - *p - 1);
    if (out->find('\\') != std::string::npos) return false;
    *p = e + 1;
    return true;
}

bool read_str(const std::string &js, const char *key, std::string *v) {
    size_t p = value_pos(js, key);
    return p != std::string::npos && read_plain_string(js, &p, v);
}

void skip_ws(const std::string &js, size_t *p) {
    while (*p < js.size() && isspace((unsigned char)js[*p])) ++*p;
}

// "all":[["name",tflops],...]
bool read_ranking(const std::string &js, std::vector<std::pair<std::string, double>> *all) {
    all->clear();
    size_t p = value_pos(js, "all");
    if (p == std::string::npos) return true;   // optional
    if (p >= js.size() || js[p] != '[') return false;
    ++p;
    for (;;) {
        skip_ws(js, &p);
        if (p < js.size() && js[p] == ']') return true;
        if (p >= js.size() || js[p] != '[') return false;
        ++p;
        skip_ws(js, &p);
        std::string name;
        if (!read_plain_string(js, &p, &name)) return false;
        skip_ws(js, &p);
        if (p >= js.size() || js[p] != ',') return false;
        ++p;
        skip_ws(js, &p);
        const char *s = js.c_str() + p;
        char *end = nullptr;
        double tf = strtod(s, &end);
        if (end == s) return false;
        p += (size_t)(end - s);
        skip_ws(js, &p);
        if (p >= js.size() || js[p] != ']') return false;
        ++p;
        all->emplace_back(name, tf);
        skip_ws(js, &p);
        if (p < js.size() && js[p] == ',') ++p;
    }
}

uint64_t xorshift64(uint64_t *s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return *s = x;
}

// bf16 values uniform in [-1, 1) (upper half of an f32, truncated).
void fill_random_bf16(std::vector<uint16_t> *v, uint64_t seed) {
    uint64_t s = seed ? seed : 0x9E3779B97F4A7C15ull;
    for (uint16_t &x : *v) {
        const float f = (float)(xorshift64(&s) >> 40) * (1.0f / 8388608.0f) - 1.0f;
        uint32_t bits;
        memcpy(&bits, &f, 4);
        x = (uint16_t)(bits >> 16);
    }
}

}  // namespace
}  // namespace t0g

struct t0g_tuner {
    std::mutex mu;
    std::string dir;
    uint32_t max_candidates = 8;
    uint32_t n_iters = 5;
    bool global = false;
    std::map<t0g::TuneKey, t0g::TuneEntry> cache;
};

namespace t0g {
namespace {

std::string cache_path(const t0g_tuner *t, const TuneKey &key) {
    if (key.kind == kTileIr)   // tile_ir_cache_path (cost_model.rs:1068-1070)
        return t->dir + "/tile_ir_" + std::to_string(key.m) + "x" + std::to_string(key.n) + "x" +
               std::to_string(key.k) + ".json";
    std::string p = t->dir + "/gemm_" + std::to_string(key.m) + "x" + std::to_string(key.n) + "x" +
                    std::to_string(key.k);
    if (key.transpose != T0G_NT) p += std::string("_") + kLayoutTag[key.transpose];
    if (key.out_dtype == T0G_BF16) p += "_bf16";
    return p + ".json";
}

// load_cache (auto_gemm.rs:329-362).  False on a miss: no file, unreadable,
// written for another architecture or key, or a config not valid here.
bool load_entry(const t0g_tuner *t, const TuneKey &key, TuneEntry *e) {
    FILE *f = fopen(cache_path(t, key).c_str(), "rb");
    if (!f) return false;
    std::string js;
    char buf[4096];
    size_t got;
    while ((got = fread(buf, 1, sizeof buf, f)) > 0 && js.size() < (1u << 20)) js.append(buf, got);
    fclose(f);
    std::string arch, layout, out;
    if (!read_str(js, "arch", &arch) || arch != "gfx950") return false;
    if (read_str(js, "layout", &layout) && layout != kLayoutTag[key.transpose]) return false;
    if (read_str(js, "out", &out) && out != (key.out_dtype == T0G_BF16 ? "bf16" : "f32")) return false;
    uint32_t dim;
    if (read_u32(js, "m", &dim) && dim != key.m) return false;
    if (read_u32(js, "n", &dim) && dim != key.n) return false;
    if (read_u32(js, "k", &dim) && dim != key.k) return false;
    t0g_gemm_config cfg;
    memset(&cfg, 0, sizeof cfg);
    double tflops = 0;
    if (!read_u32(js, "tile_m", &cfg.tile_m) || !read_u32(js, "tile_n", &cfg.tile_n) ||
        !read_u32(js, "tile_k", &cfg.tile_k) || !read_f64(js, "tflops", &tflops))
        return false;
    if (!read_u32(js, "wg_size", &cfg.wg_size)) {
        // load_tile_ir_cache's keys have no workgroup size: the tile implies it
        if (key.kind != kTileIr) return false;
        for (const TileDef &td : kTiles)
            if (td.bm == cfg.tile_m && td.bn == cfg.tile_n) cfg.wg_size = td.wg;
    }
    uint32_t sk = 1;
    read_u32(js, "split_k", &sk);
    cfg.split_k = sk > 1 ? sk : 0;
    if (!read_u32(js, "lds_pad", &cfg.lds_pad)) cfg.lds_pad = 0;
    if (!read_u32(js, "n_col_passes", &cfg.n_col_passes)) cfg.n_col_passes = 1;
    bool b = false;
    cfg.wgp_mode = read_bool(js, "wgp", &b) && b;
    b = true;
    cfg.swap_grid = read_bool(js, "swap", &b) ? b : true;
    cfg.use_lds = 1;
    cfg.double_buffer = 1;
    cfg.transpose = key.transpose;
    cfg.epilogue = T0G_EPI_STORE_F32;
    // results of this build are gfx950 kernels; an RDNA3 tile here is not one of its files
    if (validate(&cfg) || !native_tile(&cfg)) return false;
    if (key.kind == kTileIr && cfg.split_k == T0G_STREAM_K) return false;
    if (!read_ranking(js, &e->all)) e->all.clear();
    memset(&e->result, 0, sizeof e->result);
    e->result.best = cfg;
    e->result.best_tflops = tflops;
    e->result.m = key.m;
    e->result.n = key.n;
    e->result.k = key.k;
    e->result.transpose = key.transpose;
    e->result.out_dtype = key.out_dtype;
    e->result.from_cache = 1;
    e->result.n_all = (uint32_t)e->all.size();
    return true;
}

// save_cache (auto_gemm.rs:364-391): the reference's keys first, then ours.
// Written to a temporary file and renamed, so readers never see half a file.
int save_entry(const t0g_tuner *t, const TuneKey &key, const TuneEntry &e) {
    int rc = make_dirs(t->dir);
    if (rc) return rc;
    const t0g_gemm_config &c = e.result.best;
    std::string js;
    char buf[512];
    if (key.kind == kTileIr)   // save_tile_ir_cache's keys (cost_model.rs:1076-1093), then ours
        snprintf(buf, sizeof buf,
                 "{\"tile_m\":%u,\"tile_n\":%u,\"tile_k\":%u,\"split_k\":%u,\"wgp\":%s,\"tflops\":%.2f,"
                 "\"arch\":\"gfx950\",\"wg_size\":%u,\"layout\":\"%s\",\"out\":\"f32\",\"m\":%u,\"n\":%u,"
                 "\"k\":%u,\"all\":[",
                 c.tile_m, c.tile_n, c.tile_k, c.split_k > 1 ? c.split_k : 1, c.wgp_mode ? "true" : "false",
                 e.result.best_tflops, c.wg_size, kLayoutTag[key.transpose], key.m, key.n, key.k);
    else
        snprintf(buf, sizeof buf,
                 "{\"tile_m\":%u,\"tile_n\":%u,\"tile_k\":%u,\"wg_size\":%u,\"split_k\":%u,\"lds_pad\":%u,"
                 "\"n_col_passes\":%u,\"wgp\":%s,\"swap\":%s,\"tflops\":%.2f,\"arch\":\"gfx950\",\"layout\":\"%s\","
                 "\"out\":\"%s\",\"m\":%u,\"n\":%u,\"k\":%u,\"all\":[",
                 c.tile_m, c.tile_n, c.tile_k, c.wg_size, c.split_k > 1 ? c.split_k : 1, c.lds_pad, c.n_col_passes,
                 c.wgp_mode ? "true" : "false", c.swap_grid ? "true" : "false", e.result.best_tflops,
                 kLayoutTag[key.transpose], key.out_dtype == T0G_BF16 ? "bf16" : "f32", key.m, key.n, key.k);
    js = buf;
    for (size_t i = 0; i < e.all.size(); ++i) {
        snprintf(buf, sizeof buf, "%s[\"%s\",%.2f]", i ? "," : "", e.all[i].first.c_str(), e.all[i].second);
        js += buf;
    }
    js += "]}";
    const std::string path = cache_path(t, key);
    const std::string tmp = path + ".tmp." + std::to_string((long)getpid());
    FILE *f = fopen(tmp.c_str(), "wb");
    if (!f) return fail(T0G_ERR_INVALID_ARG, "cannot write %s: %s", tmp.c_str(), strerror(errno));
    const bool wrote = fwrite(js.data(), 1, js.size(), f) == js.size();
    if (fclose(f) != 0 || !wrote) {
        unlink(tmp.c_str());
        return fail(T0G_ERR_INVALID_ARG, "cannot write %s", tmp.c_str());
    }
    if (rename(tmp.c_str(), path.c_str()) != 0) {
        unlink(tmp.c_str());
        return fail(T0G_ERR_INVALID_ARG, "cannot rename %s: %s", tmp.c_str(), strerror(errno));
    }
    return T0G_OK;
}

// Memory, then disk.  Caller holds t->mu.
const TuneEntry *find_entry(t0g_tuner *t, const TuneKey &key) {
    auto it = t->cache.find(key);
    if (it != t->cache.end()) return &it->second;
    TuneEntry e;
    if (!load_entry(t, key, &e)) return nullptr;
    return &(t->cache[key] = std::move(e));
}

// with_stream_k = false for the tile ABI, which has no stream-K launch.
void candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, std::vector<t0g_gemm_config> *out,
                bool with_stream_k = true) {
    struct Cand {
        double t;
        int order;
        t0g_gemm_config cfg;
    };
    std::vector<Cand> all;
    int order = 0;
    for (const TileDef &tile : kTiles) {
        for (uint32_t sk = 1; sk <= kMaxSplitK; sk *= 2) {
            if (sk > 1 && k < sk * 4 * kTileK) break;   // >= 4 K tiles per split, as auto_select
            Cand c;
            c.t = model_time_us(tile, m, k, n, sk);
            c.order = order++;
            make_config(tile, sk, &c.cfg);
            c.cfg.transpose = transpose;
            all.push_back(c);
        }
    }
    if (with_stream_k) {
        // stream-K, ranked with the margin auto_select demands of it
        Cand c;
        c.t = model_time_sk_us(m, k, n) / 0.85;
        c.order = order++;
        make_config(kTiles[0], T0G_STREAM_K, &c.cfg);
        c.cfg.transpose = transpose;
        all.push_back(c);
    }
    std::stable_sort(all.begin(), all.end(), [](const Cand &a, const Cand &b) { return a.t < b.t; });
    out->clear();
    for (const Cand &c : all) out->push_back(c.cfg);
}

int tune_locked(t0g_tuner *t, t0g_device *dev, const TuneKey &key, const TuneEntry **out) {
    if (const TuneEntry *e = find_entry(t, key)) {
        *out = e;
        return T0G_OK;
    }
    std::vector<t0g_gemm_config> cands;
    candidates(key.m, key.n, key.k, key.transpose, &cands, key.kind != kTileIr);
    if (cands.size() > t->max_candidates) cands.resize(t->max_candidates);

    const size_t a_elems = (size_t)key.m * key.k, b_elems = (size_t)key.n * key.k;
    const size_t c_bytes = (size_t)key.m * key.n * (key.out_dtype == T0G_BF16 ? 2 : 4);
    uint64_t a = 0, b = 0, c = 0;
    int rc = t0g_alloc(dev, a_elems * 2, &a);
    if (!rc) rc = t0g_alloc(dev, b_elems * 2, &b);
    if (!rc) rc = t0g_alloc(dev, c_bytes, &c);
    if (!rc) {
        std::vector<uint16_t> host(std::max(a_elems, b_elems));
        fill_random_bf16(&host, 0x5EEDull + key.m * 131ull + key.n * 7ull + key.k);
        rc = t0g_memcpy_h2d(dev, a, host.data(), a_elems * 2);
        if (!rc) rc = t0g_memcpy_h2d(dev, b, host.data() + (host.size() - b_elems), b_elems * 2);
    }
    // Every candidate is timed in kRounds interleaved rounds (the middle one in
    // reverse order) and ranked by the median of all its samples: the shader clock
    // of a power-limited MI355X drifts with temperature over a tuning run, and one
    // block of samples per candidate let that drift decide near ties.  The first
    // round warms each candidate for about 10 ms (by the model's time), the clock's
    // settling time under load; later rounds for a quarter of that.
    constexpr int kRounds = 3;
    std::vector<std::vector<double>> samples(cands.size());
    std::vector<char> failed(cands.size(), 0);
    std::string last_failure;
    const double flop = 2.0 * key.m * key.n * key.k;
    bool poisoned_dev = false;
    for (int r = 0; !rc && !poisoned_dev && r < kRounds; ++r) {
        for (size_t j = 0; j < cands.size(); ++j) {
            const size_t i = (r == 1) ? cands.size() - 1 - j : j;
            if (failed[i]) continue;
            t0g_gemm_desc d;
            memset(&d, 0, sizeof d);
            d.a = a;
            d.b = b;
            d.c = c;
            d.m = key.m;
            d.n = key.n;
            d.k = key.k;
            d.transpose = key.transpose;
            d.out_dtype = key.out_dtype;
            d.config = &cands[i];
            const TileDef *tile = find_tile(cands[i].tile_m, cands[i].tile_n, cands[i].tile_k, cands[i].wg_size);
            const double model_us = cands[i].split_k == T0G_STREAM_K ? model_time_sk_us(key.m, key.k, key.n)
                                    : tile ? model_time_us(*tile, key.m, key.k, key.n, cfg_split(&cands[i]))
                                           : 100.0;
            const double warm_us = r == 0 ? 10000.0 : 2500.0;
            const uint32_t warm = (uint32_t)std::min(500.0, std::max(2.0, warm_us / std::max(model_us, 1.0)));
            std::vector<double> ms;
            int brc = time_gemm(dev, &d, warm, t->n_iters, &ms);
            if (brc) {
                last_failure = entry_name(key, cands[i]) + ": " + g_last_error;
                failed[i] = 1;
                int poisoned = 0;
                if (t0g_device_is_poisoned(dev, &poisoned) == T0G_OK && poisoned) {
                    poisoned_dev = true;
                    break;
                }
                continue;
            }
            samples[i].insert(samples[i].end(), ms.begin(), ms.end());
        }
    }
    std::vector<std::pair<t0g_gemm_config, double>> results;
    for (size_t i = 0; i < cands.size(); ++i) {
        if (failed[i] || samples[i].empty()) continue;
        std::vector<double> &ms = samples[i];
        std::sort(ms.begin(), ms.end());
        const double med = ms[ms.size() / 2];
        results.emplace_back(cands[i], med > 0 ? flop / (med * 1e-3) / 1e12 : 0.0);
    }
    const std::string setup_error = rc ? g_last_error : std::string();
    if (c) t0g_free(dev, c);
    if (b) t0g_free(dev, b);
    if (a) t0g_free(dev, a);
    if (rc) return fail(rc, "autotune setup failed: %s", setup_error.c_str());
    if (results.empty())
        return fail(T0G_ERR_HIP, "autotune: all candidates failed (last: %s)", last_failure.c_str());
    std::stable_sort(results.begin(), results.end(),
                     [](const std::pair<t0g_gemm_config, double> &x, const std::pair<t0g_gemm_config, double> &y) {
                         return x.second > y.second;
                     });
    TuneEntry e;
    memset(&e.result, 0, sizeof e.result);
    e.result.best = results[0].first;
    e.result.best_tflops = results[0].second;
    e.result.m = key.m;
    e.result.n = key.n;
    e.result.k = key.k;
    e.result.transpose = key.transpose;
    e.result.out_dtype = key.out_dtype;
    e.result.from_cache = 0;
    for (const auto &r : results) e.all.emplace_back(entry_name(key, r.first), r.second);
    e.result.n_all = (uint32_t)e.all.size();
    // A cache directory that cannot be written costs the persistence, not the result
    // (the reference only logs the failed write).
    if (save_entry(t, key, e)) fprintf(stderr, "[t0g autotune] cache write failed: %s\n", g_last_error.c_str());
    *out = &(t->cache[key] = std::move(e));
    return T0G_OK;
}

std::once_flag g_global_once;
t0g_tuner *g_global = nullptr;

}  // namespace
}  // namespace t0g

using namespace t0g;

extern "C" {

int t0g_tuner_create(const char *cache_dir, t0g_tuner **out) {
    if (!out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    t0g_tuner *t = new t0g_tuner;
    t->dir = (cache_dir && *cache_dir) ? cache_dir : default_cache_dir();
    while (t->dir.size() > 1 && t->dir.back() == '/') t->dir.pop_back();
    *out = t;
    return ok();
}

int t0g_tuner_destroy(t0g_tuner *tuner) {
    if (!tuner) return ok();
    if (tuner->global) return fail(T0G_ERR_INVALID_ARG, "the global tuner lives until the process ends");
    delete tuner;
    return ok();
}

int t0g_tuner_global(t0g_tuner **out) {
    if (!out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::call_once(g_global_once, []() {
        g_global = new t0g_tuner;
        g_global->dir = default_cache_dir();
        g_global->global = true;
    });
    *out = g_global;
    return ok();
}

int t0g_tuner_set_params(t0g_tuner *tuner, uint32_t max_candidates, uint32_t n_iters) {
    if (!tuner) return fail(T0G_ERR_INVALID_ARG, "tuner is NULL");
    if (max_candidates == 0 || n_iters == 0 || n_iters > 1000)
        return fail(T0G_ERR_INVALID_ARG, "max_candidates must be > 0 and n_iters in 1..1000");
    std::lock_guard<std::mutex> lk(tuner->mu);
    tuner->max_candidates = max_candidates;
    tuner->n_iters = n_iters;
    return ok();
}

int t0g_tuner_get_params(t0g_tuner *tuner, uint32_t *max_candidates, uint32_t *n_iters, uint32_t *n_cached) {
    if (!tuner) return fail(T0G_ERR_INVALID_ARG, "tuner is NULL");
    std::lock_guard<std::mutex> lk(tuner->mu);
    if (max_candidates) *max_candidates = tuner->max_candidates;
    if (n_iters) *n_iters = tuner->n_iters;
    if (n_cached) *n_cached = (uint32_t)tuner->cache.size();
    return ok();
}

int t0g_tuner_cache_dir(t0g_tuner *tuner, char *buf, size_t len) {
    if (!tuner || !buf || len == 0) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::lock_guard<std::mutex> lk(tuner->mu);
    if (tuner->dir.size() + 1 > len) return fail(T0G_ERR_INVALID_ARG, "buffer too small");
    memcpy(buf, tuner->dir.c_str(), tuner->dir.size() + 1);
    return ok();
}

int t0g_tune_candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t max,
                        t0g_gemm_config *out, uint32_t *count) {
    if (!count || (max && !out)) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = check_key(m, n, k, transpose, T0G_F32)) return rc;
    std::vector<t0g_gemm_config> c;
    candidates(m, n, k, transpose, &c);
    const uint32_t nc = (uint32_t)std::min<size_t>(c.size(), max);
    for (uint32_t i = 0; i < nc; ++i) out[i] = c[i];
    *count = nc;
    return ok();
}

int t0g_tuner_tune(t0g_tuner *tuner, t0g_device *dev, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                   uint32_t out_dtype, t0g_gemm_config *best) {
    if (!tuner || !dev || !best) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = check_key(m, n, k, transpose, out_dtype)) return rc;
    std::lock_guard<std::mutex> lk(tuner->mu);
    const TuneEntry *e = nullptr;
    if (int rc = tune_locked(tuner, dev, TuneKey{m, n, k, transpose, out_dtype}, &e)) return rc;
    *best = e->result.best;
    return ok();
}

int t0g_tuner_lookup(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                     t0g_tune_result *out, int *found) {
    if (!tuner || !out || !found) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = check_key(m, n, k, transpose, out_dtype)) return rc;
    std::lock_guard<std::mutex> lk(tuner->mu);
    const TuneEntry *e = find_entry(tuner, TuneKey{m, n, k, transpose, out_dtype});
    *found = e != nullptr;
    if (e) *out = e->result;
    return ok();
}

int t0g_tuner_ranking(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                      uint32_t i, char *name, size_t name_len, double *tflops) {
    if (!tuner || !name || name_len == 0 || !tflops) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = check_key(m, n, k, transpose, out_dtype)) return rc;
    std::lock_guard<std::mutex> lk(tuner->mu);
    const TuneEntry *e = find_entry(tuner, TuneKey{m, n, k, transpose, out_dtype});
    if (!e) return fail(T0G_ERR_INVALID_ARG, "no tuning result for %ux%ux%u", m, n, k);
    if (i >= e->all.size()) return fail(T0G_ERR_INVALID_ARG, "ranking index %u >= %zu", i, e->all.size());
    const std::string &s = e->all[i].first;
    if (s.size() + 1 > name_len) return fail(T0G_ERR_INVALID_ARG, "name buffer too small");
    memcpy(name, s.c_str(), s.size() + 1);
    *tflops = e->all[i].second;
    return ok();
}

int t0g_tuner_store(t0g_tuner *tuner, const t0g_tune_result *result, const char *const *names, const double *tflops,
                    uint32_t n_all) {
    if (!tuner || !result || (n_all && (!names || !tflops))) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    const TuneKey key{result->m, result->n, result->k, result->transpose, result->out_dtype};
    if (int rc = check_key(key.m, key.n, key.k, key.transpose, key.out_dtype)) return rc;
    t0g_gemm_config cfg = result->best;
    cfg.transpose = key.transpose;
    if (int rc = validate(&cfg)) return rc;
    if (!native_tile(&cfg))
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "a tuned config names a gfx950 kernel (t0g_config_is_native)");
    TuneEntry e;
    e.result = *result;
    e.result.best = cfg;
    e.result.from_cache = 0;
    for (uint32_t i = 0; i < n_all; ++i) {
        if (!names[i]) return fail(T0G_ERR_INVALID_ARG, "names[%u] is NULL", i);
        if (strchr(names[i], '"') || strchr(names[i], '\\'))
            return fail(T0G_ERR_INVALID_ARG, "names[%u] contains a quote or backslash", i);
        e.all.emplace_back(names[i], tflops[i]);
    }
    e.result.n_all = n_all;
    std::lock_guard<std::mutex> lk(tuner->mu);
    if (int rc = save_entry(tuner, key, e)) return rc;
    tuner->cache[key] = std::move(e);
    return ok();
}

int t0g_tuner_invalidate(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                         uint32_t out_dtype) {
    if (!tuner) return fail(T0G_ERR_INVALID_ARG, "tuner is NULL");
    if (int rc = check_key(m, n, k, transpose, out_dtype)) return rc;
    const TuneKey key{m, n, k, transpose, out_dtype};
    std::lock_guard<std::mutex> lk(tuner->mu);
    tuner->cache.erase(key);
    unlink(cache_path(tuner, key).c_str());
    return ok();
}

// clear (auto_gemm.rs:400-403) removes the whole directory; here only the
// files this tuner writes (gemm_*.json, tile_ir_*.json) and then the directory
// if it is empty, so a directory shared with other tools keeps their files.
int t0g_tuner_clear(t0g_tuner *tuner) {
    if (!tuner) return fail(T0G_ERR_INVALID_ARG, "tuner is NULL");
    std::lock_guard<std::mutex> lk(tuner->mu);
    tuner->cache.clear();
    if (DIR *d = opendir(tuner->dir.c_str())) {
        std::vector<std::string> victims;
        while (struct dirent *de = readdir(d)) {
            const std::string name = de->d_name;
            const bool ours = name.compare(0, 5, "gemm_") == 0 || name.compare(0, 8, "tile_ir_") == 0;
            if (ours && name.size() > 8 && name.compare(name.size() - 5, 5, ".json") == 0)
                victims.push_back(tuner->dir + "/" + name);
        }
        closedir(d);
        for (const std::string &v : victims) unlink(v.c_str());
        rmdir(tuner->dir.c_str());   // fails harmlessly when other files remain
    }
    return ok();
}

int t0g_tuner_report(t0g_tuner *tuner, char *buf, size_t len, size_t *needed) {
    if (!tuner || !needed) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::lock_guard<std::mutex> lk(tuner->mu);
    std::string s = "GEMM autotune cache (" + std::to_string(tuner->cache.size()) + " entries)\n";
    char line[256];
    for (const auto &kv : tuner->cache) {
        const TuneKey &k = kv.first;
        const t0g_tune_result &r = kv.second.result;
        snprintf(line, sizeof line, "  %s%ux%ux%u %s %s -> %s (%.1f TF) %s\n", k.kind == kTileIr ? "tile_ir " : "",
                 k.m, k.n, k.k, kLayoutTag[k.transpose], k.out_dtype == T0G_BF16 ? "bf16" : "f32",
                 entry_name(k, r.best).c_str(), r.best_tflops, r.from_cache ? "[cached]" : "[measured]");
        s += line;
    }
    *needed = s.size() + 1;
    if (buf && len) {
        const size_t n = std::min(len - 1, s.size());
        memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return ok();
}

static TuneKey tile_key(uint32_t m, uint32_t n, uint32_t k) {
    TuneKey key{m, n, k, T0G_NT, T0G_F32};
    key.kind = kTileIr;
    return key;
}

int t0g_tune_tile_ir(t0g_tuner *tuner, t0g_device *dev, uint32_t m, uint32_t n, uint32_t k, t0g_tune_result *out) {
    if (!dev || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (!tuner) {
        int rc = t0g_tuner_global(&tuner);
        if (rc) return rc;
    }
    if (int rc = check_key(m, n, k, T0G_NT, T0G_F32)) return rc;
    std::lock_guard<std::mutex> lk(tuner->mu);
    const TuneEntry *e = nullptr;
    if (int rc = tune_locked(tuner, dev, tile_key(m, n, k), &e)) return rc;
    *out = e->result;
    return ok();
}

int t0g_tile_ir_lookup(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, t0g_tune_result *out, int *found) {
    if (!tuner || !out || !found) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = check_key(m, n, k, T0G_NT, T0G_F32)) return rc;
    std::lock_guard<std::mutex> lk(tuner->mu);
    const TuneEntry *e = find_entry(tuner, tile_key(m, n, k));
    *found = e != nullptr;
    if (e) *out = e->result;
    return ok();
}

int t0g_tile_ir_ranking(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t i, char *name, size_t name_len,
                        double *tflops) {
    if (!tuner || !name || name_len == 0 || !tflops) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = check_key(m, n, k, T0G_NT, T0G_F32)) return rc;
    std::lock_guard<std::mutex> lk(tuner->mu);
    const TuneEntry *e = find_entry(tuner, tile_key(m, n, k));
    if (!e) return fail(T0G_ERR_INVALID_ARG, "no tile_ir tuning result for %ux%ux%u", m, n, k);
    if (i >= e->all.size()) return fail(T0G_ERR_INVALID_ARG, "ranking index %u >= %zu", i, e->all.size());
    const std::string &s = e->all[i].first;
    if (s.size() + 1 > name_len) return fail(T0G_ERR_INVALID_ARG, "name buffer too small");
    memcpy(name, s.c_str(), s.size() + 1);
    *tflops = e->all[i].second;
    return ok();
}

int t0g_tile_ir_store(t0g_tuner *tuner, const t0g_tune_result *result, const char *const *names, const double *tflops,
                      uint32_t n_all) {
    if (!tuner || !result || (n_all && (!names || !tflops))) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    const TuneKey key = tile_key(result->m, result->n, result->k);
    if (int rc = check_key(key.m, key.n, key.k, key.transpose, key.out_dtype)) return rc;
    t0g_gemm_config cfg = result->best;
    cfg.transpose = T0G_NT;
    if (int rc = validate(&cfg)) return rc;
    if (!native_tile(&cfg))
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "a tuned config names a gfx950 kernel (t0g_config_is_native)");
    if (cfg.split_k == T0G_STREAM_K) return fail(T0G_ERR_UNSUPPORTED_CONFIG, "the tile ABI has no stream-K launch");
    TuneEntry e;
    e.result = *result;
    e.result.best = cfg;
    e.result.transpose = T0G_NT;
    e.result.out_dtype = T0G_F32;
    e.result.from_cache = 0;
    for (uint32_t i = 0; i < n_all; ++i) {
        if (!names[i]) return fail(T0G_ERR_INVALID_ARG, "names[%u] is NULL", i);
        if (strchr(names[i], '"') || strchr(names[i], '\\'))
            return fail(T0G_ERR_INVALID_ARG, "names[%u] contains a quote or backslash", i);
        e.all.emplace_back(names[i], tflops[i]);
    }
    e.result.n_all = n_all;
    std::lock_guard<std::mutex> lk(tuner->mu);
    if (int rc = save_entry(tuner, key, e)) return rc;
    tuner->cache[key] = std::move(e);
    return ok();
}

int t0g_auto_gemm(t0g_tuner *tuner, t0g_device *dev, uint64_t a, uint64_t b, uint64_t c, uint32_t m, uint32_t n,
                  uint32_t k, double *tflops) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    if (!tuner) {
        int rc = t0g_tuner_global(&tuner);
        if (rc) return rc;
    }
    if (int rc = check_key(m, n, k, T0G_NT, T0G_F32)) return rc;
    t0g_gemm_config cfg;
    double tf = 0;
    {
        std::lock_guard<std::mutex> lk(tuner->mu);
        const TuneEntry *e = nullptr;
        if (int rc = tune_locked(tuner, dev, TuneKey{m, n, k, T0G_NT, T0G_F32}, &e)) return rc;
        cfg = e->result.best;
        tf = e->result.best_tflops;
    }
    t0g_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = a;
    d.b = b;
    d.c = c;
    d.m = m;
    d.n = n;
    d.k = k;
    d.transpose = T0G_NT;
    d.out_dtype = T0G_F32;
    d.config = &cfg;
    // The reference dispatches synchronously (GpuRuntime::dispatch).
    int rc = t0g_gemm(dev, &d);
    if (!rc) rc = t0g_wait_idle(dev);
    if (rc) return rc;
    if (tflops) *tflops = tf;
    return ok();
}

}  // extern "C"
