// Internal declarations shared by the host-side translation units of libt0g.
#ifndef T0G_INTERNAL_H
#define T0G_INTERNAL_H

#include <stdint.h>

#include <functional>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "t0g.h"

namespace t0g {

constexpr uint32_t kTileK = 64;
constexpr uint32_t kWaveSize = 64;
constexpr uint32_t kNumCUs = 256;
constexpr uint32_t kMaxSplitK = 64;
// 64-K stages per split from which the 64x64 deep ring splits K across its waves
constexpr uint32_t kKsplitMinStages = 24;
constexpr double kPeakFlops = 2.5e15;   // dense bf16 MFMA, MI355X
constexpr double kPeakBytes = 8.0e12;   // HBM3E, MI355X

// One entry of the MI355X tile table (see kTiles for the meaning of the
// timing fields).
struct TileDef {
    uint32_t bm, bn, wg;
    uint32_t wg_per_cu;     // workgroups one CU holds at once (LDS, registers)
    double t0_us;           // per-wave fixed cost: prologue, epilogue, launch share
    double rate1;           // per-CU bf16 FLOP/ns with one resident workgroup
    double rate_full;       // per-CU bf16 FLOP/ns with wg_per_cu resident workgroups
    double t0_deep_us;      // the deep-ring kernel (grids of at most one workgroup per CU):
    double rate_deep;       //   fixed cost and per-CU rate; 0 for tiles without one
    const char *symbol_prefix;
};
constexpr int kNumTiles = 3;
extern const TileDef kTiles[kNumTiles];
// The 64x64 and 128x128 tiles run their deep-ring kernels (suffix _d: one
// workgroup per CU, 64-K stages) when the grid gives each CU at most one
// workgroup.
inline bool tile_uses_deep(const TileDef &t, uint64_t workgroups) {
    return (t.bm == 64 || t.bm == 128) && workgroups <= kNumCUs;
}

extern thread_local std::string g_last_error;
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int ok();

const TileDef *find_tile(uint32_t tile_m, uint32_t tile_n, uint32_t tile_k, uint32_t wg_size);
void make_config(const TileDef &t, uint32_t split_k, t0g_gemm_config *out);
uint32_t cfg_split(const t0g_gemm_config *cfg);
// Accepts a native config (exactly one of the gfx950 kernels) or any config of
// the reference's GemmConfig / TileGemm space.
int validate(const t0g_gemm_config *cfg);
// The gfx950 tile of a native config (nullptr for a reference-space config).
const TileDef *native_tile(const t0g_gemm_config *cfg);
// The tile an m x n x k problem cut into sk K slices runs on under cfg: a
// native config's own, else the modelled fastest (validated cfg).
const TileDef *plan_tile(const t0g_gemm_config *cfg, uint32_t m, uint32_t k, uint32_t n, uint32_t sk);
// allow_stream_k = false: data-parallel configs only (the tile ABI launches).
void select_config(uint32_t m, uint32_t k, uint32_t n, t0g_gemm_config *out, bool allow_stream_k = true);
double model_time_us(const TileDef &t, uint32_t m, uint32_t k, uint32_t n, uint32_t sk);
double model_time_sk_us(uint32_t m, uint32_t k, uint32_t n);   // stream-K, 256x256 tile

// Epilogue chains (t0g_epilogue_op codes, 4 bits each, first op lowest).
constexpr uint32_t kMaxChainOps = 8;
uint32_t legacy_chain(uint32_t epilogue);          // t0g_epilogue -> chain
int check_chain(uint32_t chain);                   // codes valid, no gaps
bool chain_has(uint32_t chain, uint32_t op);
uint32_t chain_kernarg_bytes(uint32_t chain);      // tile_ir arguments after M

// Device time (ms) of each of `iters` t0g_gemm launches of d, after `warmup`
// untimed ones (t0g_runtime.cpp).
int time_gemm(t0g_device *dev, const t0g_gemm_desc *d, uint32_t warmup, uint32_t iters, std::vector<double> *ms);

// One kernel's entry in a code object's AMDGPU metadata (t0g_codeobj.cpp).
struct KernelMeta {
    uint32_t explicit_args_size;     // end of the last non-hidden argument: the caller's block
    uint32_t kernarg_segment_size;   // with the hidden arguments the runtime appends
    uint32_t group_segment_size;     // static LDS bytes
    uint32_t private_segment_size;   // scratch bytes per lane
    uint32_t max_workgroup_size;
    uint32_t wavefront_size;
};
// Metadata of kernel `symbol` in a gfx950 code object (bare ELF or clang
// offload bundle); refuses objects for other GPUs and malformed input.
int read_kernel_meta(const void *code_object, size_t size, const char *symbol, KernelMeta *out);

// Device address of device `ordinal`'s copy of the no-allocation scratch array
// (t0g_noalloc.hip); the device must be current on the first call for it.
int noalloc_scratch(int ordinal, uint64_t *ptr);
// Run `launch` (work on `stream` that uses device `ordinal`'s scratch) after the
// previous such work on any stream of that device, and record its end for the
// next one; under stream capture the caller orders the calls.  noalloc_scratch
// must have succeeded for the device.
int noalloc_scratch_use(int ordinal, hipStream_t stream, const std::function<int()> &launch);

}  // namespace t0g

#endif
