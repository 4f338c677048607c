// Host-only half of the C ABI: GemmConfig presets, validation, naming,
// auto_select for 256 CUs, grids, kernarg builders and the backward helpers.
// No HIP calls here, so every function in this file works without a GPU.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "t0g.h"
#include "t0g_internal.h"
#include "t0g_kernel_args.h"

namespace t0g {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return T0G_OK;
}

// MI355X tile set.  Every entry has a precompiled kernel family in
// t0g_gemm_gfx950.hsaco (gemm_gfx950.hip).  The timing fields were fitted to
// kernel times measured on one MI355X (bf16 in, bf16 out, random data, so at
// the power-limited shader clock that data draws): time per wave of
// workgroups = t0_us + (per-CU FLOP) / rate, linear in K to within a few
// percent over K = 256 .. 8192.  64x64 gains throughput from co-resident
// workgroups.  256x256 runs 4 waves, one 128x128 wave tile per SIMD (its config
// keeps wg_size 512, the unit of the reference-style thread grids; the
// stream-K kernels for NN/NT run 8 waves in ping-pong).  Grids of at
// most one workgroup per CU run the 64x64 and 128x128 deep-ring kernels, whose
// fixed cost and rate were fitted on 256-workgroup grids over K = 512 .. 8192
// (1024^2 and 2048^2 outputs); 128x128's two-workgroup rate on 4096^2 outputs.
// 128x128 deep: 4590 FLOP/ns with operands resident in the Infinity Cache, but
// its grid fetches twice the panel bytes of a 256x256 split-K grid, and inside
// the MLP step (operands streamed from HBM) 1024x4096x11008 took 100-104 us
// against 83 us alone: the rate below is the one measured in that setting.
// 256x256 (4 waves): 4096x4096xK for K = 1024 .. 8192 gives 1.375 us per 64-K
// stage per CU (6101 FLOP/ns) and 7.2 us per launch, with A and B resident in
// the 256 MiB Infinity Cache; kRate256Hbm is the rate once they are not.
const TileDef kTiles[kNumTiles] = {
    {256, 256, 512, 1, 7.2, 6101.0, 6101.0, 0.0, 0.0, "t0g_gemm_256x256_k64"},
    {128, 128, 256, 2, 4.75, 3628.0, 3628.0, 4.83, 3700.0, "t0g_gemm_128x128_k64"},
    {64, 64, 256, 4, 2.6, 931.0, 1606.0, 3.54, 2186.0, "t0g_gemm_64x64_k64"},
};

// 8192x11008x32768 (1.2 GB of operands, six rounds of 256 tiles) ran at 4952
// FLOP/ns per CU.  The stream-K kernels run at 0.81 of the data-parallel
// rate in either regime (4352x4096x8192: 267 us, 6144x11008x32768: 4327 us).
constexpr double kRate256Hbm = 4952.0;
constexpr double kInfinityCacheBytes = 256.0 * 1024 * 1024;
constexpr double kStreamKRateFactor = 0.81;

double rate256(uint32_t m, uint32_t k, uint32_t n) {
    const double operands = 2.0 * ((double)m * k + (double)k * n);
    return operands > kInfinityCacheBytes ? kRate256Hbm : kTiles[0].rate1;
}

const TileDef *find_tile(uint32_t tile_m, uint32_t tile_n, uint32_t tile_k, uint32_t wg_size) {
    if (tile_k != kTileK) return nullptr;
    for (const TileDef &t : kTiles)
        if (t.bm == tile_m && t.bn == tile_n && t.wg == wg_size) return &t;
    return nullptr;
}

void make_config(const TileDef &t, uint32_t split_k, t0g_gemm_config *out) {
    memset(out, 0, sizeof *out);
    out->tile_m = t.bm;
    out->tile_n = t.bn;
    out->tile_k = kTileK;
    out->wg_size = t.wg;
    out->split_k = split_k > 1 ? split_k : 0;
    out->lds_pad = 0;
    out->n_col_passes = 1;
    out->use_lds = 1;
    out->double_buffer = 1;
    out->swap_grid = 1;
    out->wgp_mode = 0;
    out->transpose = T0G_NT;
    out->epilogue = T0G_EPI_STORE_F32;
}

uint32_t cfg_split(const t0g_gemm_config *cfg) { return cfg->split_k > 1 ? cfg->split_k : 1; }

const TileDef *native_tile(const t0g_gemm_config *cfg) {
    if (!cfg->use_lds || !cfg->double_buffer || cfg->n_col_passes != 1) return nullptr;
    return find_tile(cfg->tile_m, cfg->tile_n, cfg->tile_k, cfg->wg_size);
}

// The reference's config space: gemm_gen takes tile_m 16..128, tile_n 32..128,
// tile_k 16/32/64, wave32 workgroups and 1-2 column passes
// (src/t0/gemm_gen.rs:88-145, 684-803); tile_ir's TileGemm adds 256-row tiles,
// tile_n in steps of 16 and tile_k 48/128 (src/t0/tile_ir.rs:85-358).  The
// RDNA3 limits on top of that (VGPR estimate, LDS per WGP) do not apply here.
static bool ref_shape(const t0g_gemm_config *cfg) {
    auto step16 = [](uint32_t v, uint32_t hi) { return v >= 16 && v <= hi && v % 16 == 0; };
    return step16(cfg->tile_m, 256) && step16(cfg->tile_n, 256) && step16(cfg->tile_k, 128) &&
           cfg->wg_size >= 32 && cfg->wg_size <= 1024 && cfg->wg_size % 32 == 0 && cfg->n_col_passes >= 1 &&
           cfg->n_col_passes <= 4;
}

int validate(const t0g_gemm_config *cfg) {
    if (!cfg) return fail(T0G_ERR_INVALID_ARG, "config is NULL");
    if (!native_tile(cfg) && !ref_shape(cfg))
        return fail(T0G_ERR_UNSUPPORTED_CONFIG,
                    "config %ux%u k%u wg%u passes %u is neither a gfx950 kernel (256x256/128x128/64x64 k64) nor in "
                    "the reference's GemmConfig space (tiles 16..256 in steps of 16, tile_k 16..128, wg_size a "
                    "multiple of 32, 1..4 column passes)",
                    cfg->tile_m, cfg->tile_n, cfg->tile_k, cfg->wg_size, cfg->n_col_passes);
    if (cfg->transpose > T0G_TT) return fail(T0G_ERR_INVALID_ARG, "bad transpose %u", cfg->transpose);
    if (cfg->epilogue > T0G_EPI_BIAS_ADD_RELU) return fail(T0G_ERR_INVALID_ARG, "bad epilogue %u", cfg->epilogue);
    if (cfg->split_k == T0G_STREAM_K) {
        if (native_tile(cfg) != &kTiles[0])
            return fail(T0G_ERR_UNSUPPORTED_CONFIG, "stream-K needs the gfx950 256x256 tile (got %ux%u wg%u)",
                        cfg->tile_m, cfg->tile_n, cfg->wg_size);
        return ok();
    }
    const uint32_t sk = cfg_split(cfg);
    if (sk > kMaxSplitK || (sk & (sk - 1)) != 0)
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "split_k=%u must be a power of two <= %u", sk, kMaxSplitK);
    return ok();
}

// ---- selection model ---------------------------------------------------------
// Modelled time (us) of one (tile, split) choice on MI355X's 256 CUs.  The
// busiest CU runs ceil(WGs / 256) workgroups, up to wg_per_cu at once; each
// wave of them costs t0_us, and their FLOPs go at the tile's per-CU rate for
// that occupancy.  Compulsory HBM bytes at 8 TB/s bound it from below.  A
// split-K adds the fp32 plane traffic and the reduce launch (fitted: 2.5 us +
// planes read at 4.5 TB/s + 0.25 us per plane of latency).
double model_time_us(const TileDef &t, uint32_t m, uint32_t k, uint32_t n, uint32_t sk) {
    const double tiles = (double)((m + t.bm - 1) / t.bm) * (double)((n + t.bn - 1) / t.bn);
    const double kc = (double)(((k + sk - 1) / sk + kTileK - 1) / kTileK * kTileK);
    const double wgs = tiles * sk;
    const double per_cu = ceil(wgs / kNumCUs);
    const double resident = per_cu < t.wg_per_cu ? per_cu : (double)t.wg_per_cu;
    const double waves = ceil(per_cu / t.wg_per_cu);
    const bool deep = tile_uses_deep(t, (uint64_t)wgs);
    const double rate = deep ? t.rate_deep
                        : t.wg_per_cu > 1
                            ? t.rate1 + (t.rate_full - t.rate1) * (resident - 1.0) / (double)(t.wg_per_cu - 1)
                            : t.rate1;
    const double flops_cu = per_cu * 2.0 * t.bm * t.bn * (kc > 0 ? kc : (double)kTileK);
    const double r = t.bm == 256 ? rate256(m, k, n) : rate;
    double t_us = (deep ? t.t0_deep_us : waves * t.t0_us) + flops_cu / r * 1e-3;
    const double bytes = 2.0 * ((double)m * k + (double)k * n) + 2.0 * (double)m * n;
    const double t_mem = bytes / kPeakBytes * 1e6;
    if (t_mem > t_us) t_us = t_mem;
    // The 256x256 kernels write their fp32 planes at about half the rate of the
    // smaller tiles' (measured on split 8 and 16: 1024x2048x11008, 512x4096x11008,
    // 256x4096x32768).
    if (sk > 1) t_us += 2.5 + (double)sk * m * n * 4.0 / (t.bm == 256 ? 2.5e6 : 4.5e6) + 0.25 * sk;
    return t_us;
}

// Stream-K on the 256x256 tile: every CU runs ceil(pairs / 256) K steps at
// the one-workgroup rate, plus the per-tile fixed cost and, when tiles are cut
// between workgroups, ~30 us for partial tiles and the extra tile prologues and
// epilogues (measured 22-44 us on MI355X over tile counts of 172-400).
double model_time_sk_us(uint32_t m, uint32_t k, uint32_t n) {
    const TileDef &t = kTiles[0];
    const uint64_t tiles = (uint64_t)((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
    const uint64_t ipt = (k + kTileK - 1) / kTileK;
    const uint64_t total = tiles * ipt;
    if (total == 0) return 1e300;
    const uint64_t per_cu = (total + kNumCUs - 1) / kNumCUs;
    const bool cut = total % kNumCUs != 0 || per_cu % ipt != 0;
    const double rate = kStreamKRateFactor * rate256(m, k, n);
    return t.t0_us + (double)per_cu * 2.0 * t.bm * t.bn * kTileK / rate * 1e-3 + (cut ? 30.0 : 5.0);
}

void select_config(uint32_t m, uint32_t k, uint32_t n, t0g_gemm_config *out, bool allow_stream_k) {
    const TileDef *best = &kTiles[0];
    uint32_t best_sk = 1;
    double best_t = 1e300;
    for (const TileDef &t : kTiles) {
        for (uint32_t sk = 1; sk <= kMaxSplitK; sk *= 2) {
            if (sk > 1 && k < sk * 4 * kTileK) break;   // keep >= 4 K tiles per split
            const double tt = model_time_us(t, m, k, n, sk);
            // On a near tie keep the earlier choice (bigger tile, fewer splits),
            // unless the later one needs fewer split planes: 128x128 split 4 took
            // 68.6 us on 1024x1024x32768 against 83.2 us for 256x256 split 16,
            // both modelled at 84.5 us.
            if (tt < best_t * 0.98 || (tt <= best_t * 1.02 && sk < best_sk)) {
                best_t = tt;
                best = &t;
                best_sk = sk;
            }
        }
    }
    // Stream-K only where data-parallel rounds quantise badly: a last round at
    // most an eighth full after at least one full one, and a modelled margin.
    // A part-empty round costs far less than its share of CUs suggests (the
    // busy CUs clock up under the board power limit), so stream-K measured
    // slower or equal at 144, 172, 576 and 1032 tiles (6144x11008x4096: 472 us
    // against 429 us) and faster at 258, 272 and 516 (4352x4096x8192: 230 us
    // against 309 us; 3072x11008x4096: 231 us against 252 us); the tuner
    // measures the rest.
    const TileDef &big = kTiles[0];
    const uint64_t tiles256 = (uint64_t)((m + big.bm - 1) / big.bm) * ((n + big.bn - 1) / big.bn);
    const uint64_t last_round = tiles256 % kNumCUs;
    if (allow_stream_k && tiles256 > kNumCUs && last_round != 0 && last_round * 8 <= kNumCUs &&
        model_time_sk_us(m, k, n) < 0.95 * best_t) {
        best = &kTiles[0];
        best_sk = T0G_STREAM_K;
    }
    make_config(*best, best_sk, out);
}

// A native config runs its own kernel.  A config of the reference's space
// (an RDNA3 tile, which says nothing about what is fast on 256 CDNA4 CUs) runs
// on the gfx950 tile the model rates fastest for the problem at that split.
const TileDef *plan_tile(const t0g_gemm_config *cfg, uint32_t m, uint32_t k, uint32_t n, uint32_t sk) {
    if (const TileDef *t = native_tile(cfg)) return t;
    if (sk == T0G_STREAM_K) return &kTiles[0];
    const TileDef *best = &kTiles[0];
    double best_t = 1e300;
    for (const TileDef &t : kTiles) {
        const double tt = model_time_us(t, m ? m : 1, k, n ? n : 1, sk ? sk : 1);
        if (tt < best_t * 0.98) {
            best_t = tt;
            best = &t;
        }
    }
    return best;
}

uint32_t legacy_chain(uint32_t epilogue) {
    if (epilogue == T0G_EPI_BIAS_ADD) return T0G_OP_BIAS_ADD;
    if (epilogue == T0G_EPI_BIAS_ADD_RELU) return T0G_OP_BIAS_ADD | (T0G_OP_RELU << 4);
    return 0;
}

int check_chain(uint32_t chain) {
    bool ended = false;
    for (uint32_t i = 0; i < kMaxChainOps; ++i) {
        const uint32_t op = (chain >> (4 * i)) & 15u;
        if (op == 0) {
            ended = true;
        } else if (ended || op > T0G_OP_CLAMP) {
            return fail(T0G_ERR_INVALID_ARG, "bad epilogue chain 0x%08x (op %u at position %u)", chain, op, i);
        }
    }
    return T0G_OK;
}

bool chain_has(uint32_t chain, uint32_t op) {
    for (uint32_t c = chain; c != 0; c >>= 4)
        if ((c & 15u) == op) return true;
    return false;
}

// lower_gemm declares bias, epi_scale, clamp_min, clamp_max after M, each only
// if some op of the chain uses it (src/t0/tile_ir.rs:670-683).
uint32_t chain_kernarg_bytes(uint32_t chain) {
    return (chain_has(chain, T0G_OP_BIAS_ADD) ? 8u : 0u) + (chain_has(chain, T0G_OP_SCALE) ? 4u : 0u) +
           (chain_has(chain, T0G_OP_CLAMP) ? 8u : 0u);
}

}  // namespace t0g

using namespace t0g;

extern "C" {

const char *t0g_last_error(void) { return g_last_error.c_str(); }
const char *t0g_version(void) { return "t0g 0.1.0 (gfx950)"; }

namespace {
struct RefPreset {
    const char *name;
    uint32_t tile_m, tile_n, tile_k, wg_size;
    uint8_t use_lds, double_buffer, wgp_mode;
    uint32_t n_col_passes;
};

// GemmConfig::tile_* (src/t0/gemm_gen.rs:88-145): field values as the
// reference sets them (wave32 workgroups, WGP mode on, swap_grid on, NT,
// no split, no padding).
const RefPreset kGemmPresets[] = {
    {"tile_16x64_k16", 16, 64, 16, 32, 1, 1, 1, 1},     {"tile_32x64_direct", 32, 64, 16, 64, 0, 0, 1, 1},
    {"tile_32x64_k16", 32, 64, 16, 64, 1, 1, 1, 1},     {"tile_32x64_k32", 32, 64, 32, 64, 1, 1, 1, 1},
    {"tile_32x128_k16", 32, 128, 16, 64, 1, 1, 1, 1},   {"tile_64x64_k16", 64, 64, 16, 64, 1, 1, 1, 1},
    {"tile_64x64_k32", 64, 64, 32, 64, 1, 1, 1, 1},     {"tile_128x64_k16", 128, 64, 16, 128, 1, 1, 1, 1},
    {"tile_64x128_k16", 64, 128, 16, 64, 1, 1, 1, 1},   {"tile_128x64_k32", 128, 64, 32, 128, 1, 1, 1, 1},
    {"tile_128x128_k16", 128, 128, 16, 128, 1, 1, 1, 1}, {"tile_64x64_k64", 64, 64, 64, 64, 1, 1, 1, 1},
    {"tile_128x128_2pass", 128, 64, 16, 128, 1, 1, 1, 2}, {"tile_64x128_2pass", 64, 64, 16, 64, 1, 1, 1, 2},
};

// TileGemm::tile_* (src/t0/tile_ir.rs:121-358): wg_size = tile_m (one wave32
// per 32 rows, TileGemm::wg_size), double-buffered, no split.  acc_swap (the
// _swap presets) is an RDNA3 register-pressure device with no field here.
const RefPreset kTilePresets[] = {
    {"tile_128x64_k16", 128, 64, 16, 128, 1, 1, 0, 1},       {"tile_64x64_k16", 64, 64, 16, 64, 1, 1, 0, 1},
    {"tile_64x64_k32", 64, 64, 32, 64, 1, 1, 0, 1},          {"tile_64x64_k64", 64, 64, 64, 64, 1, 1, 0, 1},
    {"tile_32x64_k16", 32, 64, 16, 32, 1, 1, 0, 1},          {"tile_128x64_k32", 128, 64, 32, 128, 1, 1, 0, 1},
    {"tile_64x128_k32", 64, 128, 32, 64, 1, 1, 0, 1},        {"tile_64x128_k16", 64, 128, 16, 64, 1, 1, 0, 1},
    {"tile_128x128_k16", 128, 128, 16, 128, 1, 1, 0, 1},     {"tile_128x128_k32", 128, 128, 32, 128, 1, 1, 1, 1},
    {"tile_128x128_k48", 128, 128, 48, 128, 1, 1, 0, 1},     {"tile_128x128_k16_swap", 128, 128, 16, 128, 1, 1, 0, 1},
    {"tile_128x128_k32_swap", 128, 128, 32, 128, 1, 1, 0, 1}, {"tile_256x64_k32_wgp", 256, 64, 32, 256, 1, 1, 1, 1},
    {"tile_256x64_k64_wgp", 256, 64, 64, 256, 1, 1, 1, 1},   {"tile_128x128_k64", 128, 128, 64, 128, 1, 1, 0, 1},
    {"tile_128x64_k64", 128, 64, 64, 128, 1, 1, 0, 1},
};

void from_preset(const RefPreset &p, t0g_gemm_config *out) {
    memset(out, 0, sizeof *out);
    out->tile_m = p.tile_m;
    out->tile_n = p.tile_n;
    out->tile_k = p.tile_k;
    out->wg_size = p.wg_size;
    out->use_lds = p.use_lds;
    out->double_buffer = p.double_buffer;
    out->wgp_mode = p.wgp_mode;
    out->n_col_passes = p.n_col_passes;
    out->swap_grid = 1;
    out->transpose = T0G_NT;
    out->epilogue = T0G_EPI_STORE_F32;
}

// The gfx950 kernels' own configs, named apart from the reference's presets.
bool native_preset(const char *name, t0g_gemm_config *out) {
    for (const TileDef &t : kTiles) {
        char buf[64];
        snprintf(buf, sizeof buf, "gfx950_%ux%u_k%u", t.bm, t.bn, kTileK);
        if (strcmp(buf, name) == 0) {
            make_config(t, 0, out);
            return true;
        }
    }
    return false;
}
}  // namespace

int t0g_config_preset(const char *name, t0g_gemm_config *out) {
    if (!name || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    for (const RefPreset &p : kGemmPresets)
        if (strcmp(p.name, name) == 0) {
            from_preset(p, out);
            return ok();
        }
    if (native_preset(name, out)) return ok();
    return fail(T0G_ERR_UNSUPPORTED_CONFIG, "unknown preset '%s'", name);
}

int t0g_tile_preset(const char *name, t0g_gemm_config *out) {
    if (!name || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    for (const RefPreset &p : kTilePresets)
        if (strcmp(p.name, name) == 0) {
            from_preset(p, out);
            return ok();
        }
    if (native_preset(name, out)) return ok();
    return fail(T0G_ERR_UNSUPPORTED_CONFIG, "unknown TileGemm preset '%s'", name);
}

int t0g_config_is_native(const t0g_gemm_config *cfg) { return cfg && native_tile(cfg) ? 1 : 0; }

int t0g_config_validate(const t0g_gemm_config *cfg) { return validate(cfg); }

uint32_t t0g_config_n_waves(const t0g_gemm_config *cfg) { return cfg ? cfg->wg_size / kWaveSize : 0; }

uint32_t t0g_config_lds_total(const t0g_gemm_config *cfg) {
    if (!cfg) return 0;
    const uint32_t per_buffer = (cfg->tile_m + cfg->tile_n) * cfg->tile_k * 2;
    return cfg->double_buffer ? 2 * per_buffer : per_buffer;
}

int t0g_config_name(const t0g_gemm_config *cfg, char *buf, size_t len) {
    if (!cfg || !buf || len == 0) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::string s = "t0_gemm_" + std::to_string(cfg->tile_m) + "x" + std::to_string(cfg->tile_n) + "_k" +
                    std::to_string(cfg->tile_k);
    s += cfg->use_lds ? (cfg->double_buffer ? "_ldsdb" : "_lds") : "_direct";
    if (cfg->split_k == T0G_STREAM_K) s += "_streamk";
    else if (cfg->split_k > 1) s += "_sk" + std::to_string(cfg->split_k);
    if (cfg->n_col_passes > 1) s += "_" + std::to_string(cfg->n_col_passes) + "p";
    if (!cfg->swap_grid) s += "_mg";
    if (cfg->wgp_mode) s += "_wgp";
    static const char *tr[] = {"", "_nn", "_tn", "_tt"};
    if (cfg->transpose <= T0G_TT) s += tr[cfg->transpose];
    if (cfg->epilogue == T0G_EPI_BIAS_ADD) s += "_bias";
    if (cfg->epilogue == T0G_EPI_BIAS_ADD_RELU) s += "_bias_relu";
    if (s.size() + 1 > len) return fail(T0G_ERR_INVALID_ARG, "name buffer too small (%zu < %zu)", len, s.size() + 1);
    memcpy(buf, s.c_str(), s.size() + 1);
    return ok();
}

int t0g_tile_config_name(const t0g_gemm_config *cfg, uint32_t chain, char *buf, size_t len) {
    if (!cfg || !buf || len == 0) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    char epi[64];
    int rc = t0g_epilogue_chain_name(chain ? chain : legacy_chain(cfg->epilogue), epi, sizeof epi);
    if (rc) return rc;
    std::string s = "tile_gemm_" + std::to_string(cfg->tile_m) + "x" + std::to_string(cfg->tile_n) + "_k" +
                    std::to_string(cfg->tile_k);
    if (cfg->double_buffer) s += "_db";
    if (cfg->split_k == T0G_STREAM_K) s += "_streamk";
    else if (cfg->split_k > 1) s += "_sk" + std::to_string(cfg->split_k);
    if (!cfg->swap_grid) s += "_mg";
    if (cfg->wgp_mode) s += "_wgp";
    static const char *tr[] = {"", "_nn", "_tn", "_tt"};
    if (cfg->transpose <= T0G_TT) s += tr[cfg->transpose];
    s += epi;
    if (s.size() + 1 > len) return fail(T0G_ERR_INVALID_ARG, "name buffer too small (%zu < %zu)", len, s.size() + 1);
    memcpy(buf, s.c_str(), s.size() + 1);
    return ok();
}

int t0g_auto_select(uint32_t m, uint32_t k, uint32_t n, t0g_gemm_config *out) {
    if (!out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (m == 0 || n == 0) return fail(T0G_ERR_INVALID_ARG, "auto_select: m=%u n=%u must be > 0", m, n);
    select_config(m, k, n, out);
    return ok();
}

// The tile ABI runs what t0g_tile_kernel_get + t0g_dispatch launch: NT or NN
// (TileTranspose has no other layouts, src/t0/tile_ir.rs:73-78), data-parallel
// or split-K (the library keeps the planes when build_kernargs_m leaves
// y_split_stride 0), never stream-K.  The reference's table is tuned for 96
// RDNA3 CUs; the choice here is the same 256-CU model as t0g_auto_select.
int t0g_tile_auto_select(uint32_t m, uint32_t k, uint32_t n, uint32_t transpose, t0g_gemm_config *out) {
    if (!out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (transpose != T0G_NT && transpose != T0G_NN)
        return fail(T0G_ERR_INVALID_ARG, "tile ABI layouts are NT and NN (got %u)", transpose);
    if (m == 0 || n == 0) return fail(T0G_ERR_INVALID_ARG, "tile_auto_select: m=%u n=%u must be > 0", m, n);
    select_config(m, k, n, out, false);
    out->transpose = transpose;
    return ok();
}

// The stream-K schedule has its own launch shape and argument block: it runs
// through t0g_gemm only, not through the reference's grid/kernarg/dispatch path.
static int no_stream_k(const t0g_gemm_config *cfg) {
    if (cfg->split_k == T0G_STREAM_K)
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "stream-K configs run through t0g_gemm only");
    return T0G_OK;
}

static int grid_common(const t0g_gemm_config *cfg, uint32_t m, uint32_t n, uint32_t sk, uint32_t *gx, uint32_t *gy) {
    if (!cfg || !gx || !gy) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = no_stream_k(cfg)) return rc;
    if (cfg->tile_m == 0 || cfg->tile_n == 0) return fail(T0G_ERR_INVALID_ARG, "zero tile size");
    const uint32_t eff_n = cfg->tile_n * (cfg->n_col_passes ? cfg->n_col_passes : 1);
    const uint32_t tm = (m + cfg->tile_m - 1) / cfg->tile_m;
    const uint32_t tn = (n + eff_n - 1) / eff_n;
    if (cfg->swap_grid) {
        *gx = tn * cfg->wg_size;
        *gy = tm * sk;
    } else {
        *gx = tm * cfg->wg_size;
        *gy = tn * sk;
    }
    return ok();
}

int t0g_compute_grid(const t0g_gemm_config *cfg, uint32_t m, uint32_t n, uint32_t *gx, uint32_t *gy) {
    return grid_common(cfg, m, n, 1, gx, gy);
}

int t0g_compute_grid_split_k(const t0g_gemm_config *cfg, uint32_t m, uint32_t n, uint32_t split_k, uint32_t *gx,
                             uint32_t *gy) {
    if (split_k == 0 || (split_k & (split_k - 1)) != 0)
        return fail(T0G_ERR_INVALID_ARG, "split_k=%u must be power of 2", split_k);
    return grid_common(cfg, m, n, split_k, gx, gy);
}

int t0g_compute_grid_auto(const t0g_gemm_config *cfg, uint32_t m, uint32_t n, uint32_t *gx, uint32_t *gy) {
    if (!cfg) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = no_stream_k(cfg)) return rc;
    const uint32_t sk = cfg_split(cfg);
    return sk > 1 ? t0g_compute_grid_split_k(cfg, m, n, sk, gx, gy) : t0g_compute_grid(cfg, m, n, gx, gy);
}

int t0g_tile_compute_grid(const t0g_gemm_config *cfg, uint32_t m, uint32_t n, uint32_t grid[3]) {
    if (!grid) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    int rc = grid_common(cfg, m, n, cfg ? cfg_split(cfg) : 1, &grid[0], &grid[1]);
    grid[2] = 1;
    return rc;
}

static void put_u64(uint8_t *p, uint64_t v) { memcpy(p, &v, 8); }   // x86-64 and gfx950 are little-endian
static void put_u32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }

int t0g_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                       const t0g_gemm_config *cfg, uint8_t out[40]) {
    if (!cfg || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = no_stream_k(cfg)) return rc;
    const uint32_t sk = cfg_split(cfg);
    const uint32_t y_stride = sk > 1 ? m * n * 4 : 0;
    put_u64(out + 0, x);
    put_u64(out + 8, wt);
    put_u64(out + 16, y);
    put_u32(out + 24, k);
    put_u32(out + 28, n);
    put_u32(out + 32, 0);
    put_u32(out + 36, y_stride);
    return ok();
}

int t0g_build_kernargs_with_bias(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                                 const t0g_gemm_config *cfg, uint64_t bias, uint8_t out[48]) {
    int rc = t0g_build_kernargs(x, wt, y, k, n, m, cfg, out);
    if (rc == T0G_OK) put_u64(out + 40, bias);
    return rc;
}

int t0g_build_kernargs_m(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                         const t0g_gemm_config *cfg, uint8_t out[44]) {
    if (!cfg || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (int rc = no_stream_k(cfg)) return rc;
    uint32_t shift = 0;
    switch (cfg_split(cfg)) {
        case 2: shift = 1; break;
        case 4: shift = 2; break;
        case 8: shift = 3; break;
        case 16: shift = 4; break;
        default: shift = 0; break;
    }
    put_u64(out + 0, x);
    put_u64(out + 8, wt);
    put_u64(out + 16, y);
    put_u32(out + 24, k);
    put_u32(out + 28, n);
    put_u32(out + 32, shift);
    put_u32(out + 36, 0);
    put_u32(out + 40, m);
    return ok();
}

int t0g_epilogue_chain(const uint32_t *ops, uint32_t n_ops, uint32_t *chain) {
    if (!chain || (n_ops && !ops)) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (n_ops > kMaxChainOps) return fail(T0G_ERR_INVALID_ARG, "%u epilogue ops, at most %u", n_ops, kMaxChainOps);
    uint32_t c = 0;
    for (uint32_t i = 0; i < n_ops; ++i) {
        if (ops[i] < T0G_OP_BIAS_ADD || ops[i] > T0G_OP_CLAMP)
            return fail(T0G_ERR_INVALID_ARG, "bad epilogue op %u", ops[i]);
        c |= ops[i] << (4 * i);
    }
    *chain = c;
    return ok();
}

int t0g_epilogue_chain_name(uint32_t chain, char *buf, size_t len) {
    if (!buf || !len) return fail(T0G_ERR_INVALID_ARG, "NULL buffer");
    int rc = check_chain(chain);
    if (rc) return rc;
    static const char *const kNames[] = {"", "bias", "scale", "relu", "silu", "gelu", "abs", "neg", "clamp"};
    std::string s;
    for (uint32_t c = chain; c != 0; c >>= 4) s += std::string("_") + kNames[c & 15u];
    if (s.size() + 1 > len) return fail(T0G_ERR_INVALID_ARG, "name buffer too small");
    memcpy(buf, s.c_str(), s.size() + 1);
    return ok();
}

int t0g_build_kernargs_m_epilogue(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                                  const t0g_gemm_config *cfg, uint32_t chain, uint64_t bias, float epi_scale,
                                  float clamp_min, float clamp_max, uint8_t out[64], size_t *len) {
    if (!out || !len) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    int rc = check_chain(chain);
    if (rc) return rc;
    if ((rc = t0g_build_kernargs_m(x, wt, y, k, n, m, cfg, out))) return rc;
    size_t off = 44;
    if (chain_has(chain, T0G_OP_BIAS_ADD)) {
        put_u64(out + off, bias);
        off += 8;
    }
    if (chain_has(chain, T0G_OP_SCALE)) {
        memcpy(out + off, &epi_scale, 4);
        off += 4;
    }
    if (chain_has(chain, T0G_OP_CLAMP)) {
        memcpy(out + off, &clamp_min, 4);
        memcpy(out + off + 4, &clamp_max, 4);
        off += 8;
    }
    *len = off;
    return ok();
}

uint32_t t0g_stream_k_begin(uint32_t total, uint32_t grid, uint32_t w) {
    return grid ? t0g_sk_begin(total, grid, w) : 0;
}

uint32_t t0g_stream_k_worker(uint32_t total, uint32_t grid, uint32_t it) {
    return grid && total >= grid ? t0g_sk_worker(total, grid, it) : 0;
}

int t0g_auto_select_backward_data(uint32_t m, uint32_t n_orig, uint32_t k_orig, t0g_gemm_config *out) {
    return t0g_auto_select(m, n_orig, k_orig, out);
}

int t0g_auto_select_backward_weight(uint32_t m, uint32_t n_orig, uint32_t k_orig, t0g_gemm_config *out) {
    return t0g_auto_select(n_orig, m, k_orig, out);
}

int t0g_build_kernargs_backward_data(uint64_t dy, uint64_t w, uint64_t dx, uint32_t m, uint32_t n_orig,
                                     uint32_t k_orig, const t0g_gemm_config *cfg, uint8_t out[40]) {
    return t0g_build_kernargs(dy, w, dx, n_orig, k_orig, m, cfg, out);
}

int t0g_build_kernargs_backward_weight(uint64_t dy_t, uint64_t x_t, uint64_t dw, uint32_t m, uint32_t n_orig,
                                       uint32_t k_orig, const t0g_gemm_config *cfg, uint8_t out[40]) {
    return t0g_build_kernargs(dy_t, x_t, dw, m, k_orig, n_orig, cfg, out);
}

int t0g_compute_grid_backward_data(const t0g_gemm_config *cfg, uint32_t m, uint32_t k_orig, uint32_t *gx,
                                   uint32_t *gy) {
    return t0g_compute_grid_auto(cfg, m, k_orig, gx, gy);
}

int t0g_compute_grid_backward_weight(const t0g_gemm_config *cfg, uint32_t n_orig, uint32_t k_orig, uint32_t *gx,
                                     uint32_t *gy) {
    return t0g_compute_grid_auto(cfg, n_orig, k_orig, gx, gy);
}

}  // extern "C"
