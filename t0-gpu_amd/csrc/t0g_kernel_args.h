/* Kernel-argument block shared by the host runtime and the gfx950 kernels.
 * Every GEMM kernel in t0g_gemm_gfx950.hsaco takes exactly one T0gGemmArgs by
 * value; the host fills it and passes its bytes through hipModuleLaunchKernel's
 * HIP_LAUNCH_PARAM_BUFFER_POINTER, the HIP analogue of the reference writing a
 * kernarg blob into its AQL kernarg ring (src/kfd/mod.rs:2902). */
#ifndef T0G_KERNEL_ARGS_H
#define T0G_KERNEL_ARGS_H
#include <stdint.h>

typedef struct T0gGemmArgs {
    uint64_t a;              /* op(A) operand base address (bf16)                 */
    uint64_t b;              /* op(B) operand base address (bf16)                 */
    uint64_t c;              /* output base address (f32 or bf16)                 */
    uint64_t bias;           /* f32[N] bias for the bias epilogues, else 0        */
    uint64_t c_split_stride; /* bytes between split-K output planes               */
    uint32_t m, n, k;        /* problem size                                      */
    uint32_t lda, ldb, ldc;  /* leading dimensions in elements                    */
    uint32_t k_per_split;    /* K elements per split slice (multiple of tile_k)   */
    uint32_t tiles_m;        /* output tiles along M covered by the grid          */
    uint32_t tiles_n;        /* output tiles along N covered by the grid          */
    uint32_t epilogue;       /* epilogue chain, T0G_EPI_OP_* codes 4 bits each, first
                                op in bits 0-3, 0 ends the chain (0: plain store)   */
    uint32_t group_m;        /* tile-order group height (L2 reuse), >= 1          */
    uint32_t flags;          /* T0G_FLAG_* bits                                   */
    float epi_scale;         /* Scale operand                                     */
    float clamp_lo;          /* Clamp bounds                                      */
    float clamp_hi;
    uint32_t reserved;
} T0gGemmArgs;

/* Stream-K launch of the 256x256 tile: the GEMM's tiles x iterations_per_tile
 * K iterations (64 K values each) are dealt out in equal contiguous ranges to
 * `grid` workgroups; a tile cut between workgroups is finished by the one that
 * holds its last iteration (the owner), after it has added the fp32 partial
 * tiles the others left in their slots. */
typedef struct T0gGemmSkArgs {
    T0gGemmArgs g;           /* problem, operands, epilogue; k_per_split = k    */
    uint64_t partials;       /* f32 [grid][256 * 256]: one partial tile per workgroup */
    uint64_t sync;           /* u32: 16 control words (ticket, done, timeouts), then
                                one ready flag per workgroup; all zero between launches */
    uint32_t grid;           /* launched workgroups, <= tiles * iters_per_tile    */
    uint32_t iters_per_tile; /* ceil(k / 64)                                      */
    uint32_t spin_limit;     /* polls of a ready flag before counting a timeout   */
    uint32_t debug;          /* T0G_SK_DEBUG_* bits (0 in normal use)             */
    uint32_t reserved[2];    /* pads the block to 144 bytes (whole 16-byte words) */
} T0gGemmSkArgs;

/* Split-K with the reduction inside the GEMM kernel (suffix _r): the grid is
 * tiles x splits as for plain split-K; each workgroup writes its fp32 partial
 * tile (row-major [BM][BN]) to slot tile * splits + split of `partials`
 * (stores written through to memory), then increments the tile's arrival
 * counter.  The tile's result is summed in chunks (chunk c: elements
 * [c E / splits, (c + 1) E / splits) of the row-major tile, E = BM * BN), each
 * chunk by whichever workgroup claims it (sets its bit in the tile's claim
 * mask first): the workgroup of split c, once the tile is complete, or the
 * tile's last arrival for every chunk still unclaimed after its own.  Every
 * chunk sums the splits in order 0, 1, ... from 0.0, the order of
 * t0g_splitk_reduce, so the result does not depend on who summed it. */
typedef struct T0gGemmRedArgs {
    T0gGemmArgs g;           /* problem, operands, epilogue; c, ldc: the output  */
    uint64_t partials;       /* f32 [tiles * splits][BM * BN]                    */
    uint64_t sync;           /* u32: 16 control words, then one 128-byte line per
                                tile: arrival counter, 64-bit claim mask (bit c:
                                chunk c), done counter; all zero between launches */
    uint32_t grid;           /* launched workgroups = tiles * splits              */
    uint32_t splits;         /* K slices per tile: a power of two, 2 to 64        */
    uint32_t spin_limit;     /* polls a helper waits for its tile to complete     */
    uint32_t debug;          /* T0G_SK_DEBUG_* bits (0 in normal use)             */
    uint32_t tiles;          /* output tiles = tiles_m * tiles_n                  */
    uint32_t reserved;       /* pads the block to 144 bytes (whole 16-byte words) */
} T0gGemmRedArgs;
#define T0G_RED_ARRIVAL 16u      /* first tile line (after the control words)        */
#define T0G_RED_LINE_WORDS 32u   /* words per tile line: counters of different tiles
                                    never share a cache line                          */
#define T0G_RED_MAX_GRID 16384u  /* workgroups of one fused split-K launch, at most  */

#define T0G_SK_TILE 256u
#define T0G_SK_SLOT_BYTES (T0G_SK_TILE * T0G_SK_TILE * 4u)
#define T0G_SK_CTL_WORDS 16u
#define T0G_SK_TICKET 0u         /* control word: next logical workgroup id           */
#define T0G_SK_DONE 1u           /* control word: finished workgroups                 */
#define T0G_SK_TIMEOUTS 2u       /* control word: ready-flag waits that gave up, and
                                    workgroups that drew a ticket past the grid       */
#define T0G_SK_NEVER_SET 3u      /* control word nothing writes (stays 0)             */
#define T0G_SK_DEBUG_STALL 1u    /* owners wait on T0G_SK_NEVER_SET instead of the ready
                                    flags, so every wait runs to its spin limit and gives
                                    up: a host-forced timeout for testing error reporting */

#if defined(__HIPCC__)
#define T0G_HD __host__ __device__
#else
#define T0G_HD
#endif
/* First iteration of logical workgroup w (w = grid gives the total): the first
 * total % grid workgroups get one iteration more. */
static inline T0G_HD uint32_t t0g_sk_begin(uint32_t total, uint32_t grid, uint32_t w) {
    const uint32_t base = total / grid, rem = total % grid;
    return w * base + (w < rem ? w : rem);
}
/* Logical workgroup whose range holds iteration `it` (requires total >= grid). */
static inline T0G_HD uint32_t t0g_sk_worker(uint32_t total, uint32_t grid, uint32_t it) {
    const uint32_t base = total / grid, rem = total % grid, split = rem * (base + 1u);
    return it < split ? it / (base + 1u) : rem + (it - split) / base;
}

typedef struct T0gReduceArgs {
    uint64_t ws;             /* f32 planes [splits][m][ldw]                       */
    uint64_t c;              /* output (f32 or bf16) [m][ldc]                     */
    uint64_t bias;           /* f32[N] or 0                                       */
    uint64_t plane_elems;    /* elements between planes                           */
    uint32_t m, n, ldw, ldc;
    uint32_t splits;
    uint32_t epilogue;       /* epilogue chain, as in T0gGemmArgs                 */
    uint32_t grid_blocks;    /* launched workgroups (256 threads each)           */
    uint32_t flags;          /* T0G_REDUCE_* bits                                 */
    float epi_scale;
    float clamp_lo;
    float clamp_hi;
    uint32_t reserved;
} T0gReduceArgs;

typedef struct T0gConvertArgs {
    uint64_t src;            /* f32 [n]                                           */
    uint64_t dst;            /* bf16 [n]                                          */
    uint64_t n;              /* elements                                          */
    uint32_t grid_blocks;    /* launched workgroups (256 threads each)           */
    uint32_t flags;          /* T0G_CONVERT_VEC                                   */
} T0gConvertArgs;

#define T0G_FLAG_XCD_REMAP 1u   /* remap workgroup ids so each XCD owns a contiguous tile (128x128, 64x64: (split, tile)) range */
#define T0G_FLAG_C_VEC 2u       /* C base, row pitch and split-plane stride are 16-byte aligned */
#define T0G_FLAG_BIAS 4u        /* the chain reads bias[col]                                     */
#define T0G_FLAG_TIMELINE 8u    /* record the workgroup's timeline in t0g_timeline (diagnostics)   */
#define T0G_FLAG_C_CACHED 16u   /* 64x64 / 128x128 kernels: ordinary (not non-temporal) stores of C */
/* t0g_timeline: T0G_TIMELINE_SLOTS entries of 4 u64 per linear workgroup id: clock at entry, at
 * the end of the K loop and after the epilogue's stores completed (s_memrealtime, 100 MHz),
 * then XCC_ID << 32 | HW_ID of the wave that wrote it. */
#define T0G_TIMELINE_SLOTS 8192u
#define T0G_REDUCE_VEC 1u       /* planes 16-byte aligned, N % 4 == 0, C rows aligned for 4 elements */
#define T0G_REDUCE_BIAS 2u      /* the chain reads bias[col]                                     */
#define T0G_REDUCE_WAVE 4u      /* as VEC; each wave takes 512 consecutive elements per step     */
#define T0G_CONVERT_VEC 1u      /* src 16-byte and dst 8-byte aligned, n % 4 == 0: 16-byte loads */

/* Epilogue chain operations: tile_ir's EpilogueOp (src/t0/tile_ir.rs:41-62),
 * applied in chain order to each fp32 result before the output conversion. */
#define T0G_EPI_OP_BIAS_ADD 1u  /* x += bias[col]                                  */
#define T0G_EPI_OP_SCALE 2u     /* x *= epi_scale                                  */
#define T0G_EPI_OP_RELU 3u      /* x = max(x, 0)                                   */
#define T0G_EPI_OP_SILU 4u      /* x = x * sigmoid(x)                              */
#define T0G_EPI_OP_GELU 5u      /* x = x * sigmoid(1.702 x)                        */
#define T0G_EPI_OP_ABS 6u       /* x = |x|                                         */
#define T0G_EPI_OP_NEG 7u       /* x = -x                                          */
#define T0G_EPI_OP_CLAMP 8u     /* x = min(max(x, clamp_lo), clamp_hi)             */

#endif
