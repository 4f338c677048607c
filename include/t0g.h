/*
 * t0g.h -- C ABI of the MI355X (gfx950) bf16 GEMM path for the T0-GPU call surface.
 *
 * Drop-in boundary for the reference's GEMM hot path.  The reference is Rust
 * (GeisYaO/t0-gpu); each entry point below names the Rust item it replaces
 * (paths relative to the reference root).  Plain pointers, sizes and device
 * addresses only (uint64_t, like the reference's GpuBuffer::gpu_addr()).
 *
 * Errors: every fallible call returns a t0g_status (0 = OK) and leaves a
 * thread-local message in t0g_last_error().  The reference returns
 * Result<_, String> and panics on invalid GemmConfigs (src/t0/gemm_gen.rs:256-266,
 * src/t0/tile_ir.rs:630-655); here invalid configs return
 * T0G_ERR_UNSUPPORTED_CONFIG instead.  A device that saw a kernel/HIP failure or
 * a wait timeout is poisoned and refuses further work, as GpuRuntime does
 * (src/ignis/gpu_context.rs:150-157, 270-287).
 *
 * Threading: a t0g_device is safe to share between threads; its calls are
 * serialised by an internal mutex and run on one HIP stream (the reference
 * uses one in-order AQL queue, src/kfd/mod.rs:1290-1348).
 */
#ifndef T0G_H
#define T0G_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T0G_API __attribute__((visibility("default")))

typedef enum t0g_status {
    T0G_OK = 0,
    T0G_ERR_INVALID_ARG = 1,
    T0G_ERR_UNSUPPORTED_CONFIG = 2,
    T0G_ERR_HIP = 3,
    T0G_ERR_TIMEOUT = 4,
    T0G_ERR_POISONED = 5,
    T0G_ERR_NO_DEVICE = 6,
    T0G_ERR_OUT_OF_MEMORY = 7
} t0g_status;

/* GemmTranspose (src/t0/gemm_gen.rs:24-29) / TileTranspose (src/t0/tile_ir.rs:73-78),
 * extended with the layouts the reference builds by host transposes
 * (src/t0/gemm_gen.rs:482-542, src/ignis/ops/bf16_matmul.rs:215-308).
 * Operand storage, all row-major bf16:
 *   NT: A [M][lda>=K], B [N][ldb>=K]   C = A * B^T   (reference default: Y = X * WT^T)
 *   NN: A [M][lda>=K], B [K][ldb>=N]   C = A * B
 *   TN: A [K][lda>=M], B [K][ldb>=N]   C = A^T * B
 *   TT: A [K][lda>=M], B [N][ldb>=K]   C = A^T * B^T                              */
typedef enum t0g_transpose { T0G_NT = 0, T0G_NN = 1, T0G_TN = 2, T0G_TT = 3 } t0g_transpose;

/* EpilogueOp of gemm_gen (src/t0/gemm_gen.rs:41-49). */
typedef enum t0g_epilogue {
    T0G_EPI_STORE_F32 = 0,
    T0G_EPI_BIAS_ADD = 1,
    T0G_EPI_BIAS_ADD_RELU = 2
} t0g_epilogue;

/* EpilogueOp of tile_ir (src/t0/tile_ir.rs:41-62): the fused epilogue chain,
 * applied in order to every fp32 result before the output conversion
 * (emit_epilogue_on_vreg, src/t0/tile_ir.rs:2213-2339).  A chain is packed into
 * a uint32_t, 4 bits per op, first op in bits 0-3, 0 ends it (at most 8 ops);
 * t0g_epilogue_chain builds one.  The gemm_gen epilogues are the chains
 * {BIAS_ADD} and {BIAS_ADD, RELU}. */
typedef enum t0g_epilogue_op {
    T0G_OP_BIAS_ADD = 1,   /* x += bias[col]                 (needs bias: f32[N])   */
    T0G_OP_SCALE = 2,      /* x *= epi_scale                                        */
    T0G_OP_RELU = 3,       /* x = max(x, 0)                                         */
    T0G_OP_SILU = 4,       /* x = x * sigmoid(x)                                    */
    T0G_OP_GELU = 5,       /* x = x * sigmoid(1.702 x), the reference's approximation */
    T0G_OP_ABS = 6,        /* x = |x|                                               */
    T0G_OP_NEG = 7,        /* x = -x                                                */
    T0G_OP_CLAMP = 8       /* x = min(max(x, clamp_min), clamp_max)                 */
} t0g_epilogue_op;

typedef enum t0g_dtype { T0G_F32 = 0, T0G_BF16 = 1 } t0g_dtype;

/* GemmConfig (src/t0/gemm_gen.rs:56-84), also carrying a TileGemm
 * (src/t0/tile_ir.rs:85-117; wg_size = TileGemm::wg_size() = tile_m).  Same
 * fields and meaning.  Two kinds are valid:
 *   - native: one of the gfx950 kernels exactly (t0g_config_preset "gfx950_*":
 *     256x256 / 128x128 / 64x64, tile_k 64, wg_size 512 / 256 / 256, one pass);
 *     it runs that kernel.
 *   - reference space: every config gemm_gen::generate or lower_gemm takes
 *     (the 14 GemmConfig and 17 TileGemm presets, tiles 16..256 in steps of 16,
 *     tile_k 16..128, wave32 wg_size, 1..4 column passes).  Its grid in threads
 *     and kernargs keep the reference's meaning (t0g_compute_grid*,
 *     t0g_build_kernargs*); the runtime reads the problem from them and runs the
 *     gfx950 tile the 256-CU model picks for it (an RDNA3 tile shape carries no
 *     information about CDNA4).  Caller-owned split-K planes keep the
 *     reference's K partition: plane s = K slice [s K/sk, (s+1) K/sk).
 * split_k: 0 = None, or T0G_STREAM_K (native 256x256 only). */
typedef struct t0g_gemm_config {
    uint32_t tile_m;
    uint32_t tile_n;
    uint32_t tile_k;
    uint32_t wg_size;       /* threads per workgroup: the unit of the grid in threads */
    uint32_t split_k;       /* Option<u32>: 0 or 1 = no split */
    uint32_t lds_pad;       /* accepted for layout compatibility; the gfx950 kernels swizzle instead */
    uint32_t n_col_passes;  /* column passes: one workgroup's column block is tile_n * n_col_passes wide */
    uint8_t use_lds;
    uint8_t double_buffer;
    uint8_t swap_grid;      /* true: grid x -> N tiles, y -> M tiles (src/t0/gemm_gen.rs:286-296) */
    uint8_t wgp_mode;       /* RDNA3 only; ignored on CDNA4 */
    uint32_t transpose;     /* t0g_transpose */
    uint32_t epilogue;      /* t0g_epilogue */
} t0g_gemm_config;

/* split_k value selecting the stream-K schedule (no reference counterpart; the
 * reference evaluated and rejected stream-K on gfx1100): one workgroup per CU,
 * each taking an equal share of all (tile, 64-wide K step) pairs; tiles cut
 * between workgroups are summed in a fixed order, so results are deterministic.
 * 256x256 tile only; runs through t0g_gemm (not the reference-layout
 * t0g_kernel_get / t0g_dispatch path); operands that do not meet the fast
 * path's alignment fall back to the data-parallel 128x128 kernel. */
#define T0G_STREAM_K 0x80000000u

typedef struct t0g_device t0g_device;
typedef struct t0g_kernel t0g_kernel;

/* ---- library ------------------------------------------------------------ */
T0G_API const char *t0g_last_error(void);
T0G_API const char *t0g_version(void);

/* ---- configuration and selection (host only, no GPU needed) ------------ */

/* GemmConfig::tile_* presets (src/t0/gemm_gen.rs:88-145) by name, with the
 * reference's field values ("tile_16x64_k16" ... "tile_64x128_2pass", 14 in
 * all), plus the native configs "gfx950_256x256_k64", "gfx950_128x128_k64",
 * "gfx950_64x64_k64". */
T0G_API int t0g_config_preset(const char *name, t0g_gemm_config *out);
/* TileGemm::tile_* presets (src/t0/tile_ir.rs:121-358) by name, wg_size =
 * tile_m as TileGemm::wg_size() gives it ("tile_128x64_k16" ...
 * "tile_128x64_k64", 17 in all; the "_swap" ones without their acc_swap flag),
 * plus the native "gfx950_*" configs. */
T0G_API int t0g_tile_preset(const char *name, t0g_gemm_config *out);
/* generate() / lower_gemm()'s acceptance (src/t0/gemm_gen.rs:253-266,
 * src/t0/tile_ir.rs:624-655): native configs and the reference's config space
 * (see t0g_gemm_config); RDNA3-only limits (its VGPR estimate) do not apply. */
T0G_API int t0g_config_validate(const t0g_gemm_config *cfg);
/* 1 if cfg names one gfx950 kernel exactly (it then runs that kernel), 0 for
 * a reference-space config (it runs the tile the 256-CU model picks) or NULL.
 * No reference counterpart. */
T0G_API int t0g_config_is_native(const t0g_gemm_config *cfg);
/* GemmConfig::n_waves (src/t0/gemm_gen.rs:152): wg_size / 64 on wave64. */
T0G_API uint32_t t0g_config_n_waves(const t0g_gemm_config *cfg);
/* GemmConfig::lds_total (src/t0/gemm_gen.rs:162-170). */
T0G_API uint32_t t0g_config_lds_total(const t0g_gemm_config *cfg);
/* GemmConfig::name (src/t0/gemm_gen.rs:207-227), same tag scheme. */
T0G_API int t0g_config_name(const t0g_gemm_config *cfg, char *buf, size_t len);
/* TileGemm::name (src/t0/tile_ir.rs:398-430): "tile_gemm_<m>x<n>_k<k>[_db][_skN][_mg][_wgp][_nn]"
 * then the epilogue chain's "_op" tags (chain 0: cfg->epilogue's); TN/TT add
 * "_tn"/"_tt" and stream-K "_streamk", which TileGemm has no name for. */
T0G_API int t0g_tile_config_name(const t0g_gemm_config *cfg, uint32_t chain, char *buf, size_t len);

/* auto_select(m, k, n) -> GemmConfig (src/t0/gemm_gen.rs:320-322): table
 * re-derived for 256 CUs (NT layout, f32 store epilogue). */
T0G_API int t0g_auto_select(uint32_t m, uint32_t k, uint32_t n, t0g_gemm_config *out);
/* tile_auto_select(m, k, n, transpose) (src/t0/tile_ir.rs:471-568): a config
 * the tile ABI runs (t0g_tile_kernel_get + t0g_build_kernargs_m +
 * t0g_tile_compute_grid + t0g_dispatch).  transpose is NT or NN (TileTranspose,
 * src/t0/tile_ir.rs:73-78); the choice is the 256-CU model of t0g_auto_select
 * without stream-K.  Split-K configs are runnable: with the y_split_stride of 0
 * that build_kernargs_m writes, the library keeps the fp32 planes and reduces
 * them into Y in plane order (the reference leaves them to the caller,
 * src/t0/tile_ir.rs:3154-3157). */
T0G_API int t0g_tile_auto_select(uint32_t m, uint32_t k, uint32_t n, uint32_t transpose,
                                 t0g_gemm_config *out);

/* compute_grid (src/t0/gemm_gen.rs:286-296): grid in THREADS, x = tiles * wg_size. */
T0G_API int t0g_compute_grid(const t0g_gemm_config *cfg, uint32_t m, uint32_t n,
                             uint32_t *grid_x, uint32_t *grid_y);
/* compute_grid_split_k (src/t0/gemm_gen.rs:298-309); split_k must be a power of two. */
T0G_API int t0g_compute_grid_split_k(const t0g_gemm_config *cfg, uint32_t m, uint32_t n,
                                     uint32_t split_k, uint32_t *grid_x, uint32_t *grid_y);
/* compute_grid_auto (src/t0/gemm_gen.rs:402-409). */
T0G_API int t0g_compute_grid_auto(const t0g_gemm_config *cfg, uint32_t m, uint32_t n,
                                  uint32_t *grid_x, uint32_t *grid_y);
/* tile_ir::compute_grid (src/t0/tile_ir.rs:3193-3202): [x, y, 1] in threads. */
T0G_API int t0g_tile_compute_grid(const t0g_gemm_config *cfg, uint32_t m, uint32_t n,
                                  uint32_t grid[3]);

/* build_kernargs (src/t0/gemm_gen.rs:414-430): 40 bytes
 * [X u64 @0, WT u64 @8, Y u64 @16, K u32 @24, N u32 @28, split_k_shift u32 @32 (=0),
 *  y_split_stride u32 @36 (= M*N*4 when split_k > 1, else 0)].  Note the
 * reference's argument order (k, n, m). */
T0G_API int t0g_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                               uint32_t m, const t0g_gemm_config *cfg, uint8_t out[40]);
/* build_kernargs_with_bias (src/t0/gemm_gen.rs:438-456): 48 bytes, bias u64 @40. */
T0G_API int t0g_build_kernargs_with_bias(uint64_t x, uint64_t wt, uint64_t y, uint32_t k,
                                         uint32_t n, uint32_t m, const t0g_gemm_config *cfg,
                                         uint64_t bias, uint8_t out[48]);
/* tile_ir::build_kernargs_m (src/t0/tile_ir.rs:3173-3190): 44 bytes, M u32 @40,
 * split_k_shift = log2(split_k), y_split_stride = 0 (the reference value). */
T0G_API int t0g_build_kernargs_m(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                                 uint32_t m, const t0g_gemm_config *cfg, uint8_t out[44]);

/* TileGemm::with_epilogue (src/t0/tile_ir.rs:435-444): pack n_ops (<= 8)
 * t0g_epilogue_op values into a chain; n_ops = 0 gives the empty chain 0. */
T0G_API int t0g_epilogue_chain(const uint32_t *ops, uint32_t n_ops, uint32_t *chain);
/* The epilogue part of TileGemm::name (src/t0/tile_ir.rs:416-430): "" or
 * "_op_op..." ("_bias_relu", "_silu", ...). */
T0G_API int t0g_epilogue_chain_name(uint32_t chain, char *buf, size_t len);
/* tile_ir kernargs with the epilogue arguments lower_gemm declares after M
 * (src/t0/tile_ir.rs:661-683): [44-byte build_kernargs_m block][bias u64 if
 * the chain has BIAS_ADD][epi_scale f32 if SCALE][clamp_min f32, clamp_max f32
 * if CLAMP], packed (bias lands at the unaligned offset 44).  No reference
 * builder appends these; the layout is the one the generated kernel reads.
 * *len receives the size (44 .. 64 bytes). */
T0G_API int t0g_build_kernargs_m_epilogue(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                                          uint32_t m, const t0g_gemm_config *cfg, uint32_t chain,
                                          uint64_t bias, float epi_scale, float clamp_min,
                                          float clamp_max, uint8_t out[64], size_t *len);

/* Backward helpers (src/t0/gemm_gen.rs:482-542), same argument meaning:
 * forward Y[M,N] = X[M,K] * WT[N,K]^T. */
T0G_API int t0g_auto_select_backward_data(uint32_t m, uint32_t n_orig, uint32_t k_orig,
                                          t0g_gemm_config *out);
T0G_API int t0g_auto_select_backward_weight(uint32_t m, uint32_t n_orig, uint32_t k_orig,
                                            t0g_gemm_config *out);
T0G_API int t0g_build_kernargs_backward_data(uint64_t dy, uint64_t w, uint64_t dx, uint32_t m,
                                             uint32_t n_orig, uint32_t k_orig,
                                             const t0g_gemm_config *cfg, uint8_t out[40]);
T0G_API int t0g_build_kernargs_backward_weight(uint64_t dy_t, uint64_t x_t, uint64_t dw,
                                               uint32_t m, uint32_t n_orig, uint32_t k_orig,
                                               const t0g_gemm_config *cfg, uint8_t out[40]);
T0G_API int t0g_compute_grid_backward_data(const t0g_gemm_config *cfg, uint32_t m,
                                           uint32_t k_orig, uint32_t *grid_x, uint32_t *grid_y);
T0G_API int t0g_compute_grid_backward_weight(const t0g_gemm_config *cfg, uint32_t n_orig,
                                             uint32_t k_orig, uint32_t *grid_x, uint32_t *grid_y);

/* ---- device runtime (HIP) ------------------------------------------------ */

T0G_API int t0g_device_count(int *count);
/* KfdDevice::open + GpuRuntime::new (src/kfd/mod.rs:257-453, src/ignis/gpu_context.rs:86-147):
 * selects the HIP device, creates its stream, loads the gfx950 code object. */
T0G_API int t0g_device_open(int ordinal, t0g_device **out);
T0G_API int t0g_device_close(t0g_device *dev);
/* Run subsequent work on a caller-owned hipStream_t (NULL: back to the device's own).
 * On a change of stream the new stream first waits for the work issued on the
 * old one (the handle's split-K workspace and control block are shared by all
 * its launches, so they must not run at the same time). */
T0G_API int t0g_device_set_stream(t0g_device *dev, void *hip_stream);
T0G_API int t0g_device_get_stream(t0g_device *dev, void **hip_stream);
T0G_API int t0g_device_is_poisoned(t0g_device *dev, int *poisoned);

/* GpuRuntime::{alloc, alloc_zero} over its BufferPool (src/ignis/gpu_context.rs:21-76,
 * 437-446; KfdDevice::alloc_vram, src/kfd/mod.rs:572, when the pool has no buffer of
 * the size).  Sizes are rounded up to whole 4 KiB pages; a recycled buffer of the
 * same rounded size is reused, else hipMalloc.  Returns the device address. */
T0G_API int t0g_alloc(t0g_device *dev, size_t bytes, uint64_t *addr);
T0G_API int t0g_alloc_zero(t0g_device *dev, size_t bytes, uint64_t *addr);
/* GpuBuffer drop (src/kfd/mod.rs:1057-1081): hipFree, after waiting for the stream. */
T0G_API int t0g_free(t0g_device *dev, uint64_t addr);
/* GpuRuntime::recycle / BufferPool::recycle (src/ignis/gpu_context.rs:56-62, 457-459):
 * return a live buffer to the pool instead of freeing it; no wait.  Work already
 * queued on the device stream may still use it, so a later owner must use it in
 * that stream's order (t0g_memcpy_*, t0g_gemm on the same stream are). */
T0G_API int t0g_recycle(t0g_device *dev, uint64_t addr);
/* BufferPool::clear (src/ignis/gpu_context.rs:65-69): free every recycled buffer
 * (waits for the stream first). */
T0G_API int t0g_pool_clear(t0g_device *dev);
typedef struct t0g_pool_info {
    uint64_t cached_bytes;     /* BufferPool::cached_bytes: recycled, not yet reused */
    uint64_t cached_buffers;
    uint64_t live_bytes;       /* allocated and not freed or recycled */
    uint64_t live_buffers;
    uint64_t hits, misses;     /* allocations served from the pool / by hipMalloc */
} t0g_pool_info;
T0G_API int t0g_pool_stats(t0g_device *dev, t0g_pool_info *out);
/* GpuRuntime::alloc_f32 (src/ignis/gpu_context.rs:449-454): n floats, padded to
 * whole 512-byte blocks (at least one), zeroed in device-stream order. */
T0G_API int t0g_alloc_f32(t0g_device *dev, size_t n, uint64_t *addr);
/* GpuRuntime::{write_f32, read_f32} (src/ignis/gpu_context.rs:463-480): synchronous;
 * the read waits for queued work first, as read_f32 waits for idle. */
T0G_API int t0g_write_f32(t0g_device *dev, uint64_t addr, const float *src, size_t n);
T0G_API int t0g_read_f32(t0g_device *dev, uint64_t addr, float *dst, size_t n);
/* GpuRuntime::upload_f32 (src/ignis/gpu_context.rs:482-487): alloc_f32 + write_f32. */
T0G_API int t0g_upload_f32(t0g_device *dev, const float *src, size_t n, uint64_t *addr);
/* GpuBuffer::{write, read, zero} (src/kfd/mod.rs:1000-1055): synchronous. */
T0G_API int t0g_memcpy_h2d(t0g_device *dev, uint64_t dst, const void *src, size_t bytes);
T0G_API int t0g_memcpy_d2h(t0g_device *dev, void *dst, uint64_t src, size_t bytes);
T0G_API int t0g_memset(t0g_device *dev, uint64_t dst, int value, size_t bytes);

/* generate(&cfg) + compile + GpuKernel::load, cached by name as
 * GpuRuntime::ensure_kernel_t0 does (src/t0/gemm_gen.rs:253-281,
 * src/ignis/gpu_context.rs:171-218).  Selects the precompiled gfx950 kernel
 * for cfg; it takes the 40-byte (48 with a bias epilogue) gemm_gen kernargs. */
T0G_API int t0g_kernel_get(t0g_device *dev, const t0g_gemm_config *cfg, t0g_kernel **out);
/* tile_ir::lower_gemm twin (src/t0/tile_ir.rs:585): 44-byte kernargs with M @40
 * (+ bias u64 @44 with a bias epilogue, src/compile.rs:93-111 ordering). */
T0G_API int t0g_tile_kernel_get(t0g_device *dev, const t0g_gemm_config *cfg, t0g_kernel **out);
/* lower_gemm of a TileGemm with an epilogue chain (src/t0/tile_ir.rs:585, 661-683):
 * takes the kernargs of t0g_build_kernargs_m_epilogue for the same chain.
 * cfg->epilogue must be T0G_EPI_STORE_F32 (the chain replaces it). */
T0G_API int t0g_tile_kernel_get_epilogue(t0g_device *dev, const t0g_gemm_config *cfg, uint32_t chain,
                                         t0g_kernel **out);
/* A kernel's entry in a gfx950 code object's AMDGPU metadata note, read on the
 * host (no GPU needed).  The reference knows these from the kernel it generated
 * (T0Kernel::{kernarg_size, lds_size, wg_size}, src/t0/compile.rs:495-510). */
typedef struct t0g_kernel_meta {
    uint32_t kernarg_size;          /* bytes of the caller's argument block (explicit arguments) */
    uint32_t kernarg_segment_size;  /* the whole segment, with the runtime's hidden arguments   */
    uint32_t group_segment_size;    /* static LDS bytes                                          */
    uint32_t private_segment_size;  /* scratch bytes per lane                                    */
    uint32_t max_workgroup_size;    /* largest workgroup the kernel was built for                */
    uint32_t wavefront_size;
} t0g_kernel_meta;
/* code_object: a bare gfx950 ELF or a clang offload bundle holding one (size
 * bytes, read with bounds checks); objects for other GPUs are refused. */
T0G_API int t0g_code_object_kernel_meta(const void *code_object, size_t size, const char *symbol,
                                        t0g_kernel_meta *out);

/* GpuKernel::load(&device, &elf, &KernelLoadConfig{workgroup_size, lds_size})
 * (src/kfd/mod.rs:2559-2651, 2655): any gfx950 code object, launched raw.  The
 * kernel's argument size is read from the code object's metadata, and every
 * dispatch of it must pass exactly that many kernarg bytes (T0G_ERR_INVALID_ARG
 * otherwise, before anything reaches the GPU; this library's GEMM kernels take
 * 104).  A workgroup larger than the kernel was built for is refused here.
 * lds_size is the kernel's total LDS, as in KernelLoadConfig: the part beyond
 * the kernel's static LDS is requested as dynamic LDS at launch. */
T0G_API int t0g_kernel_load(t0g_device *dev, const void *code_object, size_t size,
                            const char *symbol, const uint32_t workgroup_size[3],
                            uint32_t lds_size, t0g_kernel **out);
/* CompiledKernel fields (src/t0/dsl.rs:8-21). */
T0G_API int t0g_kernel_info(const t0g_kernel *kernel, uint32_t *wg_size, uint32_t *lds_size,
                            uint32_t *kernarg_size, char *name, size_t name_len);

/* GpuRuntime::dispatch (src/ignis/gpu_context.rs:264-288): grid in THREADS,
 * kernargs as bytes; synchronous.  _async returns after enqueueing
 * (gpu_context.rs:332-342); t0g_wait_idle waits for all of them (gpu_context.rs:382). */
T0G_API int t0g_dispatch(t0g_device *dev, const t0g_kernel *kernel, const uint32_t grid_threads[3],
                         const void *kernargs, size_t kernargs_len);
T0G_API int t0g_dispatch_async(t0g_device *dev, const t0g_kernel *kernel,
                               const uint32_t grid_threads[3], const void *kernargs,
                               size_t kernargs_len);
T0G_API int t0g_wait_idle(t0g_device *dev);

/* ---- one-shot typed GEMM (no reference counterpart; replaces the
 *      select/kernargs/grid/dispatch/host-reduce sequence the reference's
 *      callers write out, e.g. examples/test_gemm_correctness.rs:150-215) ---- */
typedef struct t0g_gemm_desc {
    uint64_t a, b, c;               /* device addresses: bf16 A, bf16 B, f32|bf16 C */
    uint64_t bias;                  /* f32[N] for the bias epilogues, else 0 */
    uint64_t workspace;             /* fp32 split-K workspace, 0 = library-managed */
    uint64_t workspace_bytes;
    uint32_t m, n, k;
    uint32_t lda, ldb, ldc;         /* elements; 0 = packed */
    uint32_t transpose;             /* t0g_transpose */
    uint32_t out_dtype;             /* t0g_dtype */
    uint32_t epilogue;              /* t0g_epilogue (ignored when epi_chain != 0) */
    uint32_t split_k;               /* 0 = from config / auto_select, 1 = none, >1 forced */
    const t0g_gemm_config *config;  /* NULL = t0g_auto_select(m, k, n) */
    uint32_t epi_chain;             /* t0g_epilogue_chain; 0 = use epilogue */
    float epi_scale;                /* T0G_OP_SCALE operand */
    float clamp_min, clamp_max;     /* T0G_OP_CLAMP bounds */
} t0g_gemm_desc;

/* Enqueue C = op(A) * op(B) (+ epilogue) on the device stream (asynchronous).
 * split_k > 1: fp32 partial sums of each K slice, summed in plane order (by a
 * reduce kernel, or inside the GEMM kernel: t0g_set_split_k_mode). */
T0G_API int t0g_gemm(t0g_device *dev, const t0g_gemm_desc *desc);
/* t0g_gemm without allocating (no reference counterpart: for callers that cannot
 * allocate device memory, such as code under HIP graph capture, tight serving
 * loops or harnesses that forbid hipMalloc).  Same arguments and results as
 * t0g_gemm; the fp32 split-K planes go to desc->workspace if given, else to a
 * static per-device scratch array of T0G_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU it runs on until the process ends (a problem needing more
 * returns T0G_ERR_INVALID_ARG).  Stream-K configs run the data-parallel schedule
 * of the same tile.  Every call on one GPU shares that GPU's scratch, which keeps
 * the last call's partial sums. */
#define T0G_NOALLOC_SCRATCH_BYTES (64u << 20)
/* Calls that put planes in the scratch are taken one after another across all
 * handles and streams of a GPU (each waits for an event the previous one
 * recorded; no allocation), except under stream capture, where an event from
 * outside the capture cannot be waited for: captured calls on one GPU must be
 * ordered by the caller.  The instrumented timeline build is never used here
 * (loading it would allocate). */
T0G_API int t0g_gemm_noalloc(t0g_device *dev, const t0g_gemm_desc *desc);
/* Enqueue n GEMMs that do not depend on each other (no output of one is an
 * input or output of another) to run concurrently: round-robin over the device
 * stream and two side streams forked from it (default priority, each with its
 * own split-K workspace); work enqueued on the device stream afterwards runs
 * after all of them.  Stream-K configs take the data-parallel schedule here.
 * No reference counterpart: the reference's single AQL queue runs one kernel at
 * a time (src/kfd/mod.rs:1313-1319). */
T0G_API int t0g_gemm_group(t0g_device *dev, const t0g_gemm_desc *descs, uint32_t n);
/* Bytes of workspace t0g_gemm would use for desc (0 without split-K). */
T0G_API int t0g_gemm_workspace_size(const t0g_gemm_desc *desc, size_t *bytes);
/* Name of the gfx950 kernel symbol t0g_gemm would launch for desc. */
T0G_API int t0g_gemm_kernel_name(const t0g_gemm_desc *desc, char *buf, size_t len);

/* T0Kernel::compile(Target) / compile_with_info (src/t0/compile.rs:1115-1187)
 * plus build_kernargs and compute_grid, for callers that load and launch the
 * kernel themselves (GpuKernel::load + dispatch, or t0g_kernel_load +
 * t0g_dispatch): the kernels are precompiled, so "compiling" selects the
 * symbol t0g_gemm would launch for desc and returns the library's gfx950 code
 * object, the symbol's workgroup size and LDS, its argument block for desc's
 * operands and the grid in threads.  Host only.  Split-K (desc->split_k > 1 or
 * the config's) writes fp32 partial planes to C, plane s at
 * c + s * M * ldc * 4 bytes, which the caller sums in plane order as the
 * reference's callers do (examples/test_gemm_correctness.rs:190-207); this
 * needs out_dtype F32.  A stream-K config is compiled as the same tile without
 * the split (its launches need the device's flag words: t0g_gemm only). */
typedef struct t0g_compiled_kernel {
    const void *code_object;    /* gfx950 code object (clang offload bundle); static, owned by the library */
    size_t code_object_size;
    char name[96];              /* kernel symbol in it                        */
    uint32_t workgroup_size;    /* threads per workgroup along x (y = z = 1)  */
    uint32_t lds_size;          /* static LDS bytes                           */
    uint32_t kernarg_size;      /* bytes of kernargs[] to pass                */
    uint32_t grid[3];           /* grid in threads for desc's problem          */
    uint32_t splits;            /* fp32 planes written to C (1: C itself)      */
    uint8_t kernargs[160];      /* argument block for desc's problem           */
} t0g_compiled_kernel;
T0G_API int t0g_gemm_compile(const t0g_gemm_desc *desc, t0g_compiled_kernel *out);

/* ---- Ignis bf16_matmul caller path on f32 device tensors ------------------- *
 * src/ignis/ops/bf16_matmul.rs converts its f32 operands to bf16 on the CPU,
 * transposes and pads them there, runs an NT GEMM and unpads the result with a
 * second kernel.  Here the conversion runs on the GPU (t0g_f32_to_bf16, the
 * same rounding) into a library-managed scratch buffer, and the GEMM uses the
 * layout the operands already have (NN / NT / TN), unpadded: Y is written at
 * its final [rows][cols] stride.  All pointers are device addresses of packed
 * row-major arrays; the calls are asynchronous on the device stream. */

/* f32 -> bf16, RNE as (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
 * (src/ignis/ops/bf16_matmul.rs:372-375, no NaN special case). */
T0G_API int t0g_f32_to_bf16(t0g_device *dev, uint64_t src_f32, uint64_t dst_bf16, size_t n);
/* bf16_matmul::matmul forward (src/ignis/ops/bf16_matmul.rs:33-56, 160-211):
 * Y[M,N] = bf16(X[M,K]) * bf16(W[K,N]), f32 accumulate and output. */
T0G_API int t0g_matmul_f32(t0g_device *dev, uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t k,
                           uint32_t n);
/* gemm_backward_data (src/ignis/ops/bf16_matmul.rs:215-260):
 * dX[M,K] = bf16(dY[M,N]) * bf16(W[K,N])^T. */
T0G_API int t0g_matmul_backward_data_f32(t0g_device *dev, uint64_t dy, uint64_t w, uint64_t dx, uint32_t m,
                                         uint32_t k, uint32_t n);
/* gemm_backward_weight (src/ignis/ops/bf16_matmul.rs:265-308):
 * dW[K,N] = bf16(X[M,K])^T * bf16(dY[M,N]). */
T0G_API int t0g_matmul_backward_weight_f32(t0g_device *dev, uint64_t x, uint64_t dy, uint64_t dw, uint32_t m,
                                           uint32_t k, uint32_t n);
/* matmul_with_wt_bf16 (src/ignis/ops/bf16_matmul.rs:98-133): Y[M,N] =
 * bf16(X[M,K]) * WT[N,K]^T with WT already bf16. */
T0G_API int t0g_matmul_wt_bf16_f32(t0g_device *dev, uint64_t x, uint64_t wt_bf16, uint64_t y, uint32_t m,
                                   uint32_t k, uint32_t n);

/* GpuRuntime's bf16 weight cache (src/ignis/gpu_context.rs:100, 385-433), per
 * device handle.  get_or_create_bf16(tensor_id, f32_buf, n, convert_kernel):
 * the first call for tensor_id converts n f32 at f32_addr (t0g_f32_to_bf16's
 * rounding) into a buffer the cache owns and returns its device address; later
 * calls return that buffer without converting (the reference keys on the id
 * alone; a call with another n is refused with T0G_ERR_INVALID_ARG).  The
 * buffer stays valid until the id is invalidated or the cache cleared
 * (invalidate_bf16 / clear_bf16_cache: call after a weight update); t0g_free
 * and t0g_recycle refuse it.  Invalidated buffers go back to the handle's
 * pool, in device-stream order, so a training step's invalidate + get
 * reconverts into the same memory without a hipMalloc. */
T0G_API int t0g_bf16_cache_get(t0g_device *dev, uint64_t tensor_id, uint64_t f32_addr, size_t n,
                               uint64_t *bf16_addr);
T0G_API int t0g_bf16_cache_invalidate(t0g_device *dev, uint64_t tensor_id);
T0G_API int t0g_bf16_cache_clear(t0g_device *dev);
/* Cached tensors and the pool bytes they hold (no reference counterpart). */
T0G_API int t0g_bf16_cache_stats(t0g_device *dev, uint64_t *entries, uint64_t *bytes);
/* t0g_matmul_f32 / t0g_matmul_backward_data_f32 with W's bf16 copy taken from
 * the cache under w_id (converted on the first call only); X (dY) is
 * converted every call.  The caller invalidates w_id when W changes. */
T0G_API int t0g_matmul_f32_cached(t0g_device *dev, uint64_t x, uint64_t w, uint64_t w_id, uint64_t y,
                                  uint32_t m, uint32_t k, uint32_t n);
T0G_API int t0g_matmul_backward_data_f32_cached(t0g_device *dev, uint64_t dy, uint64_t w, uint64_t w_id,
                                                uint64_t dx, uint32_t m, uint32_t k, uint32_t n);

/* ---- GEMM autotuner and its on-disk cache ----------------------------------- *
 * GemmTuner (src/t0/auto_gemm.rs:28-417): benchmark the model's best candidate
 * configs on the GPU, keep the fastest, cache it in memory and as one JSON file
 * per problem under the cache directory (default $HOME/.t0_autotune, else
 * /tmp/.t0_autotune; auto_gemm.rs:484-490).  Files keep the reference's keys
 * (tile_m, tile_n, tile_k, wg_size, split_k, lds_pad, n_col_passes, wgp, swap,
 * tflops, all; auto_gemm.rs:364-391) and add "arch":"gfx950", the layout, the
 * output type and the problem size; a file without "arch":"gfx950" (one the
 * gfx1100 build wrote) or whose config is not valid here counts as a miss and
 * is re-tuned.  The key is (M, N, K, layout, output type); NT with f32 output
 * uses the reference's file name gemm_MxNxK.json, other keys add a suffix. */
typedef struct t0g_tuner t0g_tuner;

/* GemmTuneResult (src/t0/auto_gemm.rs:28-42); `all` is read with
 * t0g_tuner_ranking. */
typedef struct t0g_tune_result {
    t0g_gemm_config best;       /* best->transpose = layout tuned for */
    double best_tflops;
    uint32_t m, n, k;           /* key, in the reference's (M, N, K) order */
    uint32_t transpose;         /* t0g_transpose */
    uint32_t out_dtype;         /* t0g_dtype */
    int32_t from_cache;         /* 1: loaded from disk, 0: measured in this process */
    uint32_t n_all;             /* entries in the ranking */
    uint32_t reserved;
} t0g_tune_result;

/* GemmTuner::new / with_cache_dir (auto_gemm.rs:59-75); cache_dir NULL or "" =
 * the default.  max_candidates 8, n_iters 5. */
T0G_API int t0g_tuner_create(const char *cache_dir, t0g_tuner **out);
T0G_API int t0g_tuner_destroy(t0g_tuner *tuner);
/* global_tuner() (auto_gemm.rs:429-431): one process-wide tuner with the default directory. */
T0G_API int t0g_tuner_global(t0g_tuner **out);
T0G_API int t0g_tuner_set_params(t0g_tuner *tuner, uint32_t max_candidates, uint32_t n_iters);
T0G_API int t0g_tuner_get_params(t0g_tuner *tuner, uint32_t *max_candidates, uint32_t *n_iters,
                                 uint32_t *n_cached);
T0G_API int t0g_tuner_cache_dir(t0g_tuner *tuner, char *buf, size_t len);
/* The candidate list tune() benchmarks (auto_gemm.rs:107-112: the cost model's
 * best first): every MI355X tile x split_k in order of modelled time, at most
 * max entries.  Host only. */
T0G_API int t0g_tune_candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t max,
                                t0g_gemm_config *out, uint32_t *count);
/* GemmTuner::tune(rt, m, n, k) (auto_gemm.rs:82-163): memory, then disk, then
 * benchmark (random bf16 operands, device time by HIP events; the candidates
 * timed in three interleaved rounds of n_iters launches, each after warm-up
 * launches, and ranked by the median of their samples) and persist.  Synchronous. */
T0G_API int t0g_tuner_tune(t0g_tuner *tuner, t0g_device *dev, uint32_t m, uint32_t n, uint32_t k,
                           uint32_t transpose, uint32_t out_dtype, t0g_gemm_config *best);
/* Cached result without benchmarking: *found = 0 on a miss. */
T0G_API int t0g_tuner_lookup(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                             uint32_t out_dtype, t0g_tune_result *out, int *found);
/* Entry i of the ranking of a cached result (fastest first). */
T0G_API int t0g_tuner_ranking(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                              uint32_t out_dtype, uint32_t i, char *name, size_t name_len, double *tflops);
/* save_cache (auto_gemm.rs:364-391) of a result and its ranking, also into
 * memory; names[i] / tflops[i] for i < n_all. */
T0G_API int t0g_tuner_store(t0g_tuner *tuner, const t0g_tune_result *result, const char *const *names,
                            const double *tflops, uint32_t n_all);
/* invalidate / clear (auto_gemm.rs:393-403). */
T0G_API int t0g_tuner_invalidate(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                                 uint32_t out_dtype);
T0G_API int t0g_tuner_clear(t0g_tuner *tuner);
/* report (auto_gemm.rs:405-417) into buf; *needed = bytes including the NUL. */
T0G_API int t0g_tuner_report(t0g_tuner *tuner, char *buf, size_t len, size_t *needed);
/* tune_tile_ir(rt, m, n, k) -> TileIrTuneResult (src/t0/cost_model.rs:757-1013):
 * the tile ABI's configs (NT, f32 out, data-parallel or split-K; tuner NULL =
 * the global one), looked up in memory, then in <cache_dir>/tile_ir_MxNxK.json
 * (tile_ir_cache_path / load_tile_ir_cache, cost_model.rs:1059-1074), else
 * benchmarked as t0g_tuner_tune does and saved with save_tile_ir_cache's keys
 * (tile_m, tile_n, tile_k, split_k, wgp, tflops, all; cost_model.rs:1076-1093)
 * plus "arch":"gfx950", wg_size and the size.  A file without "arch":"gfx950"
 * (the gfx1100 build's) is a miss.  out->best runs through
 * t0g_tile_kernel_get; ranking names are TileGemm::name()s. */
T0G_API int t0g_tune_tile_ir(t0g_tuner *tuner, t0g_device *dev, uint32_t m, uint32_t n, uint32_t k,
                             t0g_tune_result *out);
T0G_API int t0g_tile_ir_lookup(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, t0g_tune_result *out,
                               int *found);
T0G_API int t0g_tile_ir_ranking(t0g_tuner *tuner, uint32_t m, uint32_t n, uint32_t k, uint32_t i, char *name,
                                size_t name_len, double *tflops);
/* save_tile_ir_cache of a result (NT, f32) and its ranking, also into memory. */
T0G_API int t0g_tile_ir_store(t0g_tuner *tuner, const t0g_tune_result *result, const char *const *names,
                              const double *tflops, uint32_t n_all);
/* auto_gemm(rt, a, b, c, m, n, k) (auto_gemm.rs:445-480): tune (NT, f32 out,
 * tuner NULL = the global one), then enqueue C[M][N] = A[M][K] * B[N][K]^T with
 * the best config; *tflops (may be NULL) = the cached measurement. */
T0G_API int t0g_auto_gemm(t0g_tuner *tuner, t0g_device *dev, uint64_t a, uint64_t b, uint64_t c, uint32_t m,
                          uint32_t n, uint32_t k, double *tflops);

/* ---- test hooks ------------------------------------------------------------ */
/* The stream-K partition (one range of (tile, K step) pairs per workgroup):
 * first pair of logical workgroup w (w = grid gives total), and the workgroup
 * whose range holds pair `it`.  Host only. */
T0G_API uint32_t t0g_stream_k_begin(uint32_t total, uint32_t grid, uint32_t w);
T0G_API uint32_t t0g_stream_k_worker(uint32_t total, uint32_t grid, uint32_t it);
/* Ready-flag waits of stream-K launches on dev that gave up (0 unless a
 * workgroup waited past its spin limit); waits for the device stream.  Any
 * wait on a stream that ran a stream-K launch (t0g_wait_idle, t0g_dispatch,
 * t0g_memcpy_*, ...) checks this count first and, if it is not 0, poisons the
 * device and returns T0G_ERR_TIMEOUT: the GEMM's cut tiles miss partial sums. */
T0G_API int t0g_stream_k_timeouts(t0g_device *dev, uint32_t *count);
/* Polls of a stream-K ready flag before a workgroup gives up (default 2^20,
 * about a tenth of a second); applies to launches made after the call. */
T0G_API int t0g_set_stream_k_spin_limit(uint32_t polls);
/* on != 0: later stream-K launches wait on a control word nothing sets, so
 * every wait of a cut tile gives up at the spin limit and the kernels still
 * exit (a host-forced timeout for testing the error path); 0 restores.  In a
 * split-K launch reduced inside the kernel, the same switch makes every
 * workgroup but a tile's last arrival give up waiting, so the last arrival
 * sums the whole tile (the result does not change). */
T0G_API int t0g_debug_stream_k_stall(int on);
/* How t0g_gemm runs split-K (no reference counterpart; the reference sums the
 * planes on the host): T0G_SPLIT_K_REDUCE_KERNEL (0) = fp32 planes
 * ([splits][M][N] in desc->workspace) plus the reduce kernel;
 * T0G_SPLIT_K_IN_KERNEL (1) = reduced inside the GEMM kernel wherever the plan
 * allows it (one launch; the K slices of a tile sum it in plane order), else as
 * 0; T0G_SPLIT_K_AUTO (2, the default) = in the kernel for two K slices on the
 * 64x64 and 128x128 deep-ring kernels (the second slice to finish adds the
 * first's partial, with no wait), else as 0.  All give the same bits.  With
 * more slices the in-kernel form is slower than the two launches on MI355X
 * (the slices wait for each other, and every partial crosses HBM twice); with
 * two it is faster (128x4096x4096: 13.8 against 14.1 us).  Process-wide, for
 * later calls. */
#define T0G_SPLIT_K_REDUCE_KERNEL 0u
#define T0G_SPLIT_K_IN_KERNEL 1u
#define T0G_SPLIT_K_AUTO 2u
T0G_API int t0g_set_split_k_mode(uint32_t mode);
/* Workgroup timeline, a diagnostic with no reference counterpart (the
 * reference times whole dispatches on the host clock).  on != 0: later
 * t0g_gemm launches run the same kernels from a second, instrumented code
 * object, whose 256x256, 128x128 and 64x64 fast kernels record, per
 * linear workgroup id (blockIdx.y * gridDim.x + blockIdx.x, the first
 * T0G_TIMELINE_SLOTS = 8192 of them), four u64 in a per-device array: the GPU's
 * constant 100 MHz clock at workgroup entry, after the K loop and after the
 * epilogue's stores completed, then XCC_ID << 32 | HW_ID (the XCD and the
 * CU/SIMD/wave of the recording wave).  Later launches overwrite earlier
 * ones' entries.  Process-wide; off by default (then it costs one uniform
 * branch per workgroup). */
T0G_API int t0g_set_timeline(int on);
/* Copy the first `entries` u64 of the device's timeline array (4 per workgroup)
 * to out, after the device stream has drained; *written: how many were copied
 * (at most 4 * 8192). */
T0G_API int t0g_timeline_read(t0g_device *dev, uint64_t *out, size_t entries, size_t *written);
/* Zero the device's timeline array (entries of workgroups that did not run stay 0). */
T0G_API int t0g_timeline_clear(t0g_device *dev);
/* Device-memory allocations this library has asked HIP for, process-wide
 * (every hipMalloc and every code-object load, which places the code in device
 * memory); lets a test show that an entry point such as t0g_gemm_noalloc
 * allocates nothing.  No reference counterpart. */
T0G_API int t0g_debug_device_alloc_count(uint64_t *count);
/* Make the n-th HIP call from now (n >= 1) fail with a simulated error;
 * n = 0 disarms.  Lets the error mapping and poisoning be tested without a
 * real device fault. */
T0G_API int t0g_debug_fail_hip_call(int n);
/* Wait timeout of t0g_wait_idle / t0g_dispatch in milliseconds (default 60000);
 * the reference polls for 5 s (src/kfd/mod.rs:1607-1642). */
T0G_API int t0g_set_wait_timeout_ms(uint32_t ms);

#ifdef __cplusplus
}
#endif

#endif /* T0G_H */
