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

#define T0G_FLAG_XCD_REMAP 1u   /* remap block ids so each XCD owns a contiguous tile range */
#define T0G_FLAG_C_VEC 2u       /* C base, row pitch and split-plane stride are 16-byte aligned */
#define T0G_FLAG_BIAS 4u        /* the chain reads bias[col]                                     */
#define T0G_REDUCE_VEC 1u       /* planes 16-byte aligned, N % 4 == 0, C rows aligned for 4 elements */
#define T0G_REDUCE_BIAS 2u      /* the chain reads bias[col]                                     */
#define T0G_CONVERT_VEC 1u      /* src 32-byte and dst 16-byte aligned: 8 elements per step      */

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
