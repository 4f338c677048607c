// bf16 GEMM kernels for MI355X (gfx950, CDNA4), fp32 accumulation.
//
// Replaces the reference's runtime-generated RDNA3 GEMM kernels
// (src/t0/gemm_gen.rs:637-1348 generate_lds_db, src/t0/tile_ir.rs:585-1591
// lower_gemm).  Same math, C[M,N] = op(A)[M,K] * op(B)[K,N] with bf16 inputs
// and fp32 accumulation, written for the CDNA4 execution model:
//   * wave64, v_mfma_f32_32x32x16_bf16 (each wave owns a WTM x WTN sub-tile
//     built from 32x32 MFMA blocks, fp32 accumulators in AGPR/VGPR);
//   * one 64-element (128-byte) K slice per LDS row, XOR-swizzled in 16-byte
//     chunks so both the 16-byte fragment reads of a wave and the cooperative
//     tile stores are free of bank conflicts;
//   * double-buffered LDS with register staging: the global loads of K tile
//     t+1 are in flight while the MFMAs of tile t run; one barrier per tile;
//   * operands stored K-contiguous are copied as 16-byte chunks; operands
//     stored M/N-contiguous are read as 8x8 bf16 blocks and transposed in
//     registers, so NN / TN / TT need no host-side transpose (the reference
//     transposes on the CPU: src/ignis/ops/bf16_matmul.rs:390-424);
//   * M/N edges are clamped on load and masked on store (as tile_ir does,
//     src/t0/tile_ir.rs:934-946, 2462-2480); K tails are zero-filled, which the
//     reference leaves to the caller (src/t0/test_tile_gemm_suite.rs:62-99);
//   * split-K slices write fp32 planes at c + split * c_split_stride; the
//     deterministic plane-ordered reduction is t0g_splitk_reduce_*;
//   * block ids are remapped so each XCD (own L2) works on a contiguous,
//     M-grouped patch of output tiles.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "t0g_kernel_args.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

namespace t0g {

constexpr int kTileK = 64;       // bf16 elements of K per tile
constexpr int kRowBytes = 128;   // one LDS row holds the tile's K slice of one M/N row

// Chunk swizzle of an LDS row: chunk c of row r is stored at c ^ swz(r).
// swz takes all 8 values over any 8 consecutive rows, and over any 16
// consecutive rows the pair (r & 1, swz(r)) takes all 16 values, so 8 or 16
// lanes reading the same logical chunk of consecutive rows hit distinct banks.
__device__ __forceinline__ uint32_t swz(uint32_t row) { return (row & 7u) ^ ((row >> 3) & 1u); }

__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t chunk) {
    return row * kRowBytes + ((chunk ^ swz(row)) << 4);
}

__device__ __forceinline__ u32x4_t zero4() { return u32x4_t{0u, 0u, 0u, 0u}; }

__device__ __forceinline__ u32x4_t pack8(const uint16_t e[8]) {
    return u32x4_t{(uint32_t)e[0] | ((uint32_t)e[1] << 16), (uint32_t)e[2] | ((uint32_t)e[3] << 16),
                   (uint32_t)e[4] | ((uint32_t)e[5] << 16), (uint32_t)e[6] | ((uint32_t)e[7] << 16)};
}

// ---------------------------------------------------------------------------
// Operand stored K-contiguous: rows of the tile are rows of memory.
// ROWS tile rows x 8 chunks of 16 bytes; thread t copies chunk (t % 8) of rows
// t/8, t/8 + NT/8, ...  Eight consecutive lanes read one 128-byte row segment.
// ---------------------------------------------------------------------------
template <int ROWS, int NT, bool ALIGNED>
struct KMajorTile {
    static constexpr int kChunks = ROWS * 8 / NT;
    static constexpr int kRowsPerPass = NT / 8;
    static_assert(kChunks >= 1 && ROWS * 8 % NT == 0, "tile too small for the workgroup");

    u32x4_t v[kChunks];
    uint32_t off[kChunks];   // element offset of this thread's chunk at k = 0
    uint32_t lrow0;          // first LDS row of this thread
    uint32_t chunk;

    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t R, uint32_t ld) {
        chunk = tid & 7u;
        lrow0 = tid >> 3;
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            uint32_t r = row0 + lrow0 + i * kRowsPerPass;
            r = r < R ? r : R - 1;   // clamp: results of clamped rows are never stored
            off[i] = r * ld + chunk * 8;
        }
    }

    __device__ __forceinline__ void load(const uint16_t* __restrict__ base, uint32_t k0, uint32_t kend, bool full) {
        const uint16_t* p = base + k0;
        if (full) {
#pragma unroll
            for (int i = 0; i < kChunks; ++i) {
                if constexpr (ALIGNED) {
                    v[i] = *reinterpret_cast<const u32x4_t*>(p + off[i]);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) e[j] = p[off[i] + j];
                    v[i] = pack8(e);
                }
            }
        } else {
            const int valid = (int)kend - (int)(k0 + chunk * 8);   // elements of this chunk inside K
#pragma unroll
            for (int i = 0; i < kChunks; ++i) {
                if constexpr (ALIGNED) {
                    // K % 8 == 0 on this path: a chunk is entirely inside or outside.
                    v[i] = valid > 0 ? *reinterpret_cast<const u32x4_t*>(p + off[i]) : zero4();
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) e[j] = (j < valid) ? p[off[i] + j] : (uint16_t)0;
                    v[i] = pack8(e);
                }
            }
        }
    }

    __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
        for (int i = 0; i < kChunks; ++i)
            *reinterpret_cast<u32x4_t*>(lds + lds_off(lrow0 + i * kRowsPerPass, chunk)) = v[i];
    }
};

// ---------------------------------------------------------------------------
// Operand stored M/N-contiguous ([K][R] in memory).  The tile is cut into
// 8 (k) x 8 (r) blocks of bf16; thread t < ROWS owns block (k-block t % 8,
// r-block t / 8): eight 16-byte row loads, an 8x8 transpose in registers,
// eight 16-byte LDS stores into the K-contiguous LDS layout.
// ---------------------------------------------------------------------------
template <int ROWS, int NT, bool ALIGNED>
struct MNMajorTile {
    static_assert(ROWS <= NT, "one 8x8 block per thread at most");
    u32x4_t v[8];
    uint32_t kb, rb;
    uint32_t off;      // element offset of (k = kb*8, r = first column of the block) at k0 = 0
    uint32_t col0;     // first column (unclamped) of the block, unaligned path
    bool active;

    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t R, uint32_t ld) {
        active = tid < (uint32_t)ROWS;
        kb = tid & 7u;
        rb = tid >> 3;
        col0 = row0 + rb * 8;
        uint32_t c = col0;
        if constexpr (ALIGNED) c = c + 8 <= R ? c : R - 8;   // R % 8 == 0 and R >= 8 on this path
        off = kb * 8 * ld + c;
    }

    __device__ __forceinline__ void load(const uint16_t* __restrict__ base, uint32_t k0, uint32_t kend,
                                         bool full, uint32_t ld, uint32_t R) {
        if (!active) return;
        const uint16_t* p = base + (size_t)k0 * ld + off;
        const int krem = (int)kend - (int)(k0 + kb * 8);   // rows of this block inside K
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if constexpr (ALIGNED) {
                if (full || r < krem)
                    v[r] = *reinterpret_cast<const u32x4_t*>(p + r * ld);
                else
                    v[r] = zero4();
            } else {
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    e[j] = ((full || r < krem) && col0 + j < R) ? p[r * ld + j] : (uint16_t)0;
                v[r] = pack8(e);
            }
        }
    }

    __device__ __forceinline__ void store(char* lds) const {
        if (!active) return;
        // w[c] = the 8 k-values of column c: halves taken from v[2i], v[2i+1].
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int d = c >> 1;
            u32x4_t w;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t x = v[2 * i][d], y = v[2 * i + 1][d];
                w[i] = (c & 1) ? ((x >> 16) | (y & 0xFFFF0000u)) : ((x & 0xFFFFu) | (y << 16));
            }
            *reinterpret_cast<u32x4_t*>(lds + lds_off(rb * 8 + c, kb)) = w;
        }
    }
};

template <bool K_MAJOR, int ROWS, int NT, bool ALIGNED>
struct TileLoader;
template <int ROWS, int NT, bool ALIGNED>
struct TileLoader<true, ROWS, NT, ALIGNED> {
    KMajorTile<ROWS, NT, ALIGNED> t;
    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t R, uint32_t ld) { t.init(tid, row0, R, ld); }
    __device__ __forceinline__ void load(const uint16_t* base, uint32_t k0, uint32_t kend, bool full, uint32_t, uint32_t) {
        t.load(base, k0, kend, full);
    }
    __device__ __forceinline__ void store(char* lds) const { t.store(lds); }
};
template <int ROWS, int NT, bool ALIGNED>
struct TileLoader<false, ROWS, NT, ALIGNED> {
    MNMajorTile<ROWS, NT, ALIGNED> t;
    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t R, uint32_t ld) { t.init(tid, row0, R, ld); }
    __device__ __forceinline__ void load(const uint16_t* base, uint32_t k0, uint32_t kend, bool full, uint32_t ld, uint32_t R) {
        t.load(base, k0, kend, full, ld, R);
    }
    __device__ __forceinline__ void store(char* lds) const { t.store(lds); }
};

// ---------------------------------------------------------------------------
// The tile kernel body.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WAVES_M, int WAVES_N, bool A_K, bool B_K, bool OUT_BF16, bool ALIGNED>
__device__ __forceinline__ void gemm_tile(const T0gGemmArgs& p) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int SM = WTM / 32, SN = WTN / 32;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
    constexpr uint32_t A_BYTES = BM * kRowBytes, STAGE = (BM + BN) * kRowBytes;
    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    const uint32_t tid = threadIdx.x;

    // --- output tile of this workgroup ----------------------------------------
    uint32_t bid = blockIdx.x;
    const uint32_t nblk = p.tiles_m * p.tiles_n;   // grid x is exactly the tile count
    if ((p.flags & T0G_FLAG_XCD_REMAP) && (nblk & 7u) == 0) bid = (bid & 7u) * (nblk >> 3) + (bid >> 3);
    const uint32_t gm = p.group_m;
    const uint32_t per_group = gm * p.tiles_n;
    const uint32_t group = bid / per_group;
    const uint32_t first_m = group * gm;
    const uint32_t gsz = min(p.tiles_m - first_m, gm);
    const uint32_t in_group = bid - group * per_group;
    const uint32_t m0 = (first_m + in_group % gsz) * BM;
    const uint32_t n0 = (in_group / gsz) * BN;

    const uint32_t kbeg = blockIdx.y * p.k_per_split;
    const uint32_t kend = min(p.k, kbeg + p.k_per_split);
    const int nkt = kend > kbeg ? (int)((kend - kbeg + kTileK - 1) / kTileK) : 0;

    const uint16_t* __restrict__ A = reinterpret_cast<const uint16_t*>(p.a);
    const uint16_t* __restrict__ B = reinterpret_cast<const uint16_t*>(p.b);

    TileLoader<A_K, BM, NT, ALIGNED> la;
    TileLoader<B_K, BN, NT, ALIGNED> lb;
    la.init(tid, m0, p.m, p.lda);
    lb.init(tid, n0, p.n, p.ldb);

    // --- per-lane fragment addressing --------------------------------------------
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave / WAVES_N, wn = wave % WAVES_N;
    const uint32_t l32 = lane & 31u, g = lane >> 5;
    const uint32_t a_row = (wm * WTM + l32) * kRowBytes;
    const uint32_t b_row = A_BYTES + (wn * WTN + l32) * kRowBytes;
    uint32_t ch_off[kTileK / 16];
#pragma unroll
    for (int kk = 0; kk < kTileK / 16; ++kk) ch_off[kk] = (((uint32_t)(kk * 2) + g) ^ swz(l32)) << 4;

    f32x16_t acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j) acc[i][j] = f32x16_t{};

    if (nkt > 0) {
        la.load(A, kbeg, kend, kbeg + kTileK <= kend, p.lda, p.m);
        lb.load(B, kbeg, kend, kbeg + kTileK <= kend, p.ldb, p.n);
        la.store(smem);
        lb.store(smem + A_BYTES);
        __syncthreads();

        for (int kt = 0; kt < nkt; ++kt) {
            const char* cur = smem + (kt & 1) * STAGE;
            char* nxt = smem + ((kt + 1) & 1) * STAGE;
            const bool has_next = kt + 1 < nkt;
            if (has_next) {
                const uint32_t k0 = kbeg + (uint32_t)(kt + 1) * kTileK;
                const bool full = k0 + kTileK <= kend;
                la.load(A, k0, kend, full, p.lda, p.m);
                lb.load(B, k0, kend, full, p.ldb, p.n);
            }
#pragma unroll
            for (int kk = 0; kk < kTileK / 16; ++kk) {
                bf16x8_t af[SM], bfr[SN];
#pragma unroll
                for (int i = 0; i < SM; ++i)
                    af[i] = *reinterpret_cast<const bf16x8_t*>(cur + a_row + i * 32 * kRowBytes + ch_off[kk]);
#pragma unroll
                for (int j = 0; j < SN; ++j)
                    bfr[j] = *reinterpret_cast<const bf16x8_t*>(cur + b_row + j * 32 * kRowBytes + ch_off[kk]);
#pragma unroll
                for (int i = 0; i < SM; ++i)
#pragma unroll
                    for (int j = 0; j < SN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
            }
            if (has_next) {
                la.store(nxt);
                lb.store(nxt + A_BYTES);
            }
            __syncthreads();
        }
    }

    // --- epilogue: acc -> (+bias) -> (ReLU) -> f32 / bf16 (RNE) -----------------
    // 32x32 MFMA result layout: lane (l32, g), register r holds
    // row 8*(r/4) + 4*g + r%4, column l32 of the 32x32 block.
    const float* __restrict__ bias = reinterpret_cast<const float*>(p.bias);
    char* cbase = reinterpret_cast<char*>(p.c) + (size_t)blockIdx.y * p.c_split_stride;
#pragma unroll
    for (int j = 0; j < SN; ++j) {
        const uint32_t col = n0 + wn * WTN + j * 32 + l32;
        const bool col_ok = col < p.n;
        float bv = 0.0f;
        if (p.epilogue != 0 && col_ok) bv = bias[col];
#pragma unroll
        for (int i = 0; i < SM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                if (col_ok && row < p.m) {
                    float x = acc[i][j][r];
                    if (p.epilogue != 0) x = x + bv;
                    if (p.epilogue == 2) x = x > 0.0f ? x : 0.0f;
                    const size_t idx = (size_t)row * p.ldc + col;
                    if constexpr (OUT_BF16)
                        reinterpret_cast<__bf16*>(cbase)[idx] = (__bf16)x;
                    else
                        reinterpret_cast<float*>(cbase)[idx] = x;
                }
            }
        }
    }
}

// Plane-ordered split-K reduction: y = ((0 + p0) + p1) + ... in fp32, the
// order the reference's host loop uses (examples/test_gemm_correctness.rs:190-207),
// then the epilogue and the output conversion.
template <bool OUT_BF16>
__device__ __forceinline__ void splitk_reduce(const T0gReduceArgs& p) {
    const float* __restrict__ ws = reinterpret_cast<const float*>(p.ws);
    const float* __restrict__ bias = reinterpret_cast<const float*>(p.bias);
    const size_t total = (size_t)p.m * p.n;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)p.grid_blocks * 256) {
        const uint32_t row = (uint32_t)(idx / p.n), col = (uint32_t)(idx % p.n);
        const size_t w = (size_t)row * p.ldw + col;
        float acc = 0.0f;
        for (uint32_t s = 0; s < p.splits; ++s) acc = acc + ws[s * p.plane_elems + w];
        if (p.epilogue != 0) acc = acc + bias[col];
        if (p.epilogue == 2) acc = acc > 0.0f ? acc : 0.0f;
        const size_t o = (size_t)row * p.ldc + col;
        if constexpr (OUT_BF16)
            reinterpret_cast<__bf16*>(p.c)[o] = (__bf16)acc;
        else
            reinterpret_cast<float*>(p.c)[o] = acc;
    }
}

}  // namespace t0g

// ---------------------------------------------------------------------------
// Exported kernel symbols (looked up by name with hipModuleGetFunction).
// t0g_gemm_<BM>x<BN>_k64_<layout>_<out>[_u]   (_u: element-wise loads for
// shapes whose rows are not 16-byte aligned)
// ---------------------------------------------------------------------------
// 256x256 tiles hold 256 fp32 accumulators per lane: one wave per SIMD, the
// whole 512-entry VGPR+AGPR file.  Smaller tiles leave room for two workgroups
// per CU (LDS 64 KB or less each).
#define T0G_WPE_256x256 1, 1
#define T0G_WPE_128x128 1, 2
#define T0G_WPE_64x64 1, 4
#define T0G_GEMM(NAME, BM, BN, WM, WN, AK, BKM, OBF, AL)                                       \
    extern "C" __global__ void __launch_bounds__(64 * WM * WN)                                   \
        __attribute__((amdgpu_waves_per_eu(T0G_WPE_##BM##x##BN))) NAME(T0gGemmArgs p) {          \
        t0g::gemm_tile<BM, BN, WM, WN, AK, BKM, OBF, AL>(p);                                     \
    }

#define T0G_GEMM_LAYOUTS(PFX, BM, BN, WM, WN, OUTN, OBF, SFX, AL)          \
    T0G_GEMM(PFX##_nt_##OUTN##SFX, BM, BN, WM, WN, true, true, OBF, AL)    \
    T0G_GEMM(PFX##_nn_##OUTN##SFX, BM, BN, WM, WN, true, false, OBF, AL)   \
    T0G_GEMM(PFX##_tn_##OUTN##SFX, BM, BN, WM, WN, false, false, OBF, AL)  \
    T0G_GEMM(PFX##_tt_##OUTN##SFX, BM, BN, WM, WN, false, true, OBF, AL)

#define T0G_GEMM_TILE(PFX, BM, BN, WM, WN)                       \
    T0G_GEMM_LAYOUTS(PFX, BM, BN, WM, WN, f32, false, , true)    \
    T0G_GEMM_LAYOUTS(PFX, BM, BN, WM, WN, bf16, true, , true)

#define T0G_GEMM_TILE_U(PFX, BM, BN, WM, WN)                     \
    T0G_GEMM_LAYOUTS(PFX, BM, BN, WM, WN, f32, false, _u, false) \
    T0G_GEMM_LAYOUTS(PFX, BM, BN, WM, WN, bf16, true, _u, false)

T0G_GEMM_TILE(t0g_gemm_256x256_k64, 256, 256, 2, 2)
T0G_GEMM_TILE(t0g_gemm_128x128_k64, 128, 128, 2, 2)
T0G_GEMM_TILE(t0g_gemm_64x64_k64, 64, 64, 2, 2)
T0G_GEMM_TILE_U(t0g_gemm_128x128_k64, 128, 128, 2, 2)
T0G_GEMM_TILE_U(t0g_gemm_64x64_k64, 64, 64, 2, 2)

extern "C" __global__ void __launch_bounds__(256) t0g_splitk_reduce_f32(T0gReduceArgs p) {
    t0g::splitk_reduce<false>(p);
}
extern "C" __global__ void __launch_bounds__(256) t0g_splitk_reduce_bf16(T0gReduceArgs p) {
    t0g::splitk_reduce<true>(p);
}
