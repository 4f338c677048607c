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
//   * workgroup ids are remapped so each XCD (own L2) works on a contiguous
//     range of (K slice, M-grouped output tile) pairs.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "t0g_kernel_args.h"


typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
// Global-memory pointer types: with an explicit address space the compiler
// emits global_* instead of flat_* instructions (flat loads also count on
// lgkmcnt, so every LDS wait would wait for them as well).
typedef const __attribute__((address_space(1))) uint16_t gu16_t;
typedef __attribute__((address_space(1))) float gf32_t;
typedef __attribute__((address_space(1))) __bf16 gbf16_t;
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

namespace t0g {

constexpr int kRsrcWord3 = 0x00020000;   // gfx9-family raw buffer descriptor word 3

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

// Workgroup timeline (T0G_FLAG_TIMELINE), a diagnostic: built only into the
// second code object (T0G_TIMELINE defined), which the runtime launches while
// the host has the timeline switched on.  The fast kernels then record, per
// linear workgroup id, the constant 100 MHz clock at entry, after the K loop
// and after the epilogue's stores have completed, plus the XCC and hardware
// ids of the recording wave; the host reads the array with
// hipModuleGetGlobal.  The production code object carries none of it: even
// switched off, the marks moved the 4-wave 256x256 kernel's 11008x4096x1024
// launch by 2-5 %.
#ifdef T0G_TIMELINE
}  // namespace t0g
extern "C" {
__device__ __attribute__((aligned(256))) uint64_t t0g_timeline[T0G_TIMELINE_SLOTS * 4];
}
namespace t0g {
#endif

// Entry `ev` (0: entry, 1: end of the K loop, 2: stores completed, which also
// writes the ids) of this workgroup's record, written as it happens so that no
// clock value is held in registers across the K loop.
__device__ __forceinline__ void tl_mark(const T0gGemmArgs& p, int ev) {
#ifndef T0G_TIMELINE
    (void)p;
    (void)ev;
#else
    if (p.flags & T0G_FLAG_TIMELINE) {
        if (ev == 2) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the epilogue's stores have completed
        const uint64_t t = __builtin_amdgcn_s_memrealtime();
        const uint32_t slot = blockIdx.y * gridDim.x + blockIdx.x;
        if (threadIdx.x == 0 && slot < T0G_TIMELINE_SLOTS) {
            uint64_t* e = t0g_timeline + (uint64_t)slot * 4;
            e[ev] = t;
            if (ev == 2) {
                // XCC_ID is hardware register 20 on gfx950 (bits 3:0), HW_ID register 4
                const uint32_t xcc = (uint32_t)__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u;
                const uint32_t hw = (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);
                e[3] = ((uint64_t)xcc << 32) | hw;
            }
        }
    }
#endif
}

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

    __device__ __forceinline__ void load(gu16_t* __restrict__ base, uint32_t k0, uint32_t kend, bool full) {
        gu16_t* p = base + k0;
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

    __device__ __forceinline__ void load(gu16_t* __restrict__ base, uint32_t k0, uint32_t kend,
                                         bool full, uint32_t ld, uint32_t R) {
        if (!active) return;
        gu16_t* p = base + (size_t)k0 * ld + off;
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
    __device__ __forceinline__ void load(gu16_t* base, uint32_t k0, uint32_t kend, bool full, uint32_t, uint32_t) {
        t.load(base, k0, kend, full);
    }
    __device__ __forceinline__ void store(char* lds) const { t.store(lds); }
};
template <int ROWS, int NT, bool ALIGNED>
struct TileLoader<false, ROWS, NT, ALIGNED> {
    MNMajorTile<ROWS, NT, ALIGNED> t;
    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t R, uint32_t ld) { t.init(tid, row0, R, ld); }
    __device__ __forceinline__ void load(gu16_t* base, uint32_t k0, uint32_t kend, bool full, uint32_t ld, uint32_t R) {
        t.load(base, k0, kend, full, ld, R);
    }
    __device__ __forceinline__ void store(char* lds) const { t.store(lds); }
};

// ---------------------------------------------------------------------------
// Epilogue: acc -> epilogue chain -> f32 or bf16 (round to nearest even),
// masked to the M x N output.  32x32 MFMA result layout: lane
// (l32 = lane % 32, g = lane / 32), register r holds row 8*(r/4) + 4*g + r%4,
// column l32 of the 32x32 block.
// ---------------------------------------------------------------------------
// The bias values are fetched up front with range-checked buffer loads (columns
// past N read as 0) and retired with one explicit wait, so the per-element
// stores below carry no memory waits and stream out back to back.
template <int SN>
__device__ __forceinline__ void load_bias_cols(const T0gGemmArgs& p, uint32_t col0, uint32_t l32, float (&bv)[SN]) {
#pragma unroll
    for (int j = 0; j < SN; ++j) bv[j] = 0.0f;
    if (p.flags & T0G_FLAG_BIAS) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)p.bias, 0, (int)(p.n * 4u), (int)kRsrcWord3);
#pragma unroll
        for (int j = 0; j < SN; ++j)
            bv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (col0 + j * 32 + l32) * 4u, 0, 0));
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    }
}

// The epilogue chain (tile_ir's emit_epilogue_on_vreg, src/t0/tile_ir.rs:2213-2339):
// T0G_EPI_OP_* codes 4 bits each, first op in the low bits.  The chain is a
// kernel argument, so the decode loop branches uniformly.  SiLU and GELU use
// the hardware exp2 and reciprocal, as the reference does: sigmoid(y) =
// rcp(1 + exp2(-y * log2 e)); GELU is the reference's x * sigmoid(1.702 x).
struct EpiParams {
    uint32_t chain;
    float scale, lo, hi;
};

__device__ __forceinline__ float epi_sigmoid_mul(float x, float y) {
    const float e = __builtin_amdgcn_exp2f(-y * 1.44269504f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float apply_epilogue(float x, float bv, const EpiParams& e) {
    for (uint32_t c = e.chain; c != 0; c >>= 4) {
        switch (c & 15u) {
        case T0G_EPI_OP_BIAS_ADD: x = x + bv; break;
        case T0G_EPI_OP_SCALE: x = x * e.scale; break;
        case T0G_EPI_OP_RELU: x = x > 0.0f ? x : 0.0f; break;
        case T0G_EPI_OP_SILU: x = epi_sigmoid_mul(x, x); break;
        case T0G_EPI_OP_GELU: x = epi_sigmoid_mul(x, x * 1.702f); break;
        case T0G_EPI_OP_ABS: x = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) & 0x7FFFFFFFu); break;
        case T0G_EPI_OP_NEG: x = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) ^ 0x80000000u); break;
        case T0G_EPI_OP_CLAMP: x = __builtin_fminf(__builtin_fmaxf(x, e.lo), e.hi); break;
        default: break;
        }
    }
    return x;
}

template <class Args>
__device__ __forceinline__ EpiParams epi_of(const Args& p) {
    return EpiParams{p.epilogue, p.epi_scale, p.clamp_lo, p.clamp_hi};
}

// The chain over a lane's N output values: one decode per op rather than per
// value, which keeps the unrolled store loops small.
template <int N>
__device__ __forceinline__ void apply_epilogue_n(float (&v)[N], const float (&bv)[N], const EpiParams& e) {
    for (uint32_t c = e.chain; c != 0; c >>= 4) {
        const uint32_t op = c & 15u;
        if (op == T0G_EPI_OP_BIAS_ADD) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = v[i] + bv[i];
        } else if (op == T0G_EPI_OP_SCALE) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = v[i] * e.scale;
        } else if (op == T0G_EPI_OP_RELU) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = v[i] > 0.0f ? v[i] : 0.0f;
        } else if (op == T0G_EPI_OP_SILU) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = epi_sigmoid_mul(v[i], v[i]);
        } else if (op == T0G_EPI_OP_GELU) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = epi_sigmoid_mul(v[i], v[i] * 1.702f);
        } else if (op == T0G_EPI_OP_ABS) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v[i]) & 0x7FFFFFFFu);
        } else if (op == T0G_EPI_OP_NEG) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v[i]) ^ 0x80000000u);
        } else if (op == T0G_EPI_OP_CLAMP) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] = __builtin_fminf(__builtin_fmaxf(v[i], e.lo), e.hi);
        }
    }
}

// Output tile index and K slice of this workgroup (grid x is exactly the tile
// count, grid y the split count).  The dispatcher deals workgroups out to the
// 8 XCDs round-robin in linear order (x fastest).  With XCD_REMAP the linear id
// is permuted so that XCD c owns a contiguous range of slice-major (split,
// tile) order (xcd_range): the workgroups of one K slice share an L2, which
// then fetches each A and B panel of that slice once instead of once per XCD.
// Without split-K this is the plain tile remap.  (The 256x256 kernels keep the
// tile-only remap: measured, the extra prologue work cost their 4096^3 launch
// 1-1.5 %, more than the split-K shapes on that tile gain.)
struct GridPos {
    uint32_t tile, split;
};

// Linear workgroup id -> position in an order where XCD c (ids = c mod 8)
// holds one contiguous range: of `total` items, XCDs below total % 8 get
// total / 8 + 1 consecutive items and the others total / 8, so every id maps
// to a distinct item whatever the count (a bijection of [0, total)).
__device__ __forceinline__ uint32_t xcd_range(uint32_t id, uint32_t total) {
    const uint32_t x = id & 7u, q = total >> 3, r = total & 7u;
    return x * q + min(x, r) + (id >> 3);
}

__device__ __forceinline__ GridPos grid_pos(const T0gGemmArgs& p) {
    const uint32_t nblk = p.tiles_m * p.tiles_n;
    uint32_t tile = blockIdx.x, split = blockIdx.y;
    const uint64_t total = (uint64_t)nblk * gridDim.y;
    if ((p.flags & T0G_FLAG_XCD_REMAP) && total <= 0xFFFFFFFFull) {
        const uint32_t l = xcd_range(split * nblk + tile, (uint32_t)total);
        split = l / nblk;
        tile = l - split * nblk;
    }
    return GridPos{tile, split};
}

template <int SM, int SN, bool OUT_BF16>
__device__ __forceinline__ void store_tile(const T0gGemmArgs& p, const f32x16_t (&acc)[SM][SN], uint32_t row0,
                                           uint32_t col0, uint32_t l32, uint32_t g, uint32_t split) {
    const uint64_t cbase = p.c + (uint64_t)split * p.c_split_stride;
    float bv[SN];
    load_bias_cols<SN>(p, col0, l32, bv);
#pragma unroll
    for (int j = 0; j < SN; ++j) {
        const uint32_t col = col0 + j * 32 + l32;
        const bool col_ok = col < p.n;
#pragma unroll
        for (int i = 0; i < SM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = row0 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                if (col_ok && row < p.m) {
                    const float x = apply_epilogue(acc[i][j][r], bv[j], epi_of(p));
                    const uint64_t idx = (uint64_t)row * p.ldc + col;
                    if constexpr (OUT_BF16)
                        reinterpret_cast<gbf16_t*>(cbase)[idx] = (__bf16)x;
                    else
                        reinterpret_cast<gf32_t*>(cbase)[idx] = x;
                }
            }
        }
    }
}

// Epilogue of a tile that lies wholly inside C (and C rows are 16-byte
// aligned): each wave stages its WTM x WTN result through its own LDS region,
// 32 rows at a time, as f32 rows padded to WTN + 8 words -- the two lane
// halves of a 32x32 result sit 4 rows apart and so land in opposite halves of
// the 64 banks -- and writes whole rows back with 16-byte stores (4 f32 or
// 8 bf16 per lane), so every store instruction covers complete 128-byte lines.
template <int SN>
struct VecEpilogue {
    static constexpr int kWTN = SN * 32;
    static constexpr uint32_t kStride = (kWTN + 8) * 4;   // bytes per staged row
    static constexpr uint32_t kWaveBytes = 32 * kStride;   // LDS per wave
};

// WT: the 16-byte stores write through to memory (sc0 sc1) instead of going
// non-temporal into this XCD's L2, for data that workgroups on other XCDs read.
// PAIR: before the epilogue, add the tile's other K slice of a two-slice split:
// `partner` addresses that slice's fp32 partial at this wave tile's first
// element, row-major with `pld` floats per row, written through to memory by
// another workgroup; it is read past the caches (volatile: sc0 sc1) and added
// in plane order, (0 + p0) + p1, with own_first telling whether this
// workgroup's own values are p0.
template <int SM, int SN, bool OUT_BF16, bool WT = false, bool CACHED = false, bool PAIR = false>
__device__ __forceinline__ void store_tile_vec(const T0gGemmArgs& p, const f32x16_t (&acc)[SM][SN], uint32_t row0,
                                               uint32_t col0, uint32_t lane, uint32_t lds, bool vec, uint32_t split,
                                               uint64_t partner = 0, uint32_t pld = 0, bool own_first = false) {
    typedef VecEpilogue<SN> E;
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) float lds_f32;
    typedef __attribute__((address_space(3))) f32x4_t lds_f32x4;
    constexpr int kCols = OUT_BF16 ? 8 : 4;              // columns per lane and store
    constexpr int kLanesPerRow = E::kWTN / kCols;
    constexpr int kRowsPerPass = 64 / kLanesPerRow;
    constexpr int kPasses = 32 / kRowsPerPass;
    static_assert(kLanesPerRow <= 64 && 64 % kLanesPerRow == 0, "row must map onto whole lanes");
    const uint32_t l32 = lane & 31u, g = lane >> 5;
    const uint32_t rl = lane / kLanesPerRow, cl = (lane % kLanesPerRow) * kCols;
    // the partner's values for every (block, pass) this lane stores, all loads in flight at once
    f32x4_t pv[PAIR ? SM : 1][PAIR ? kPasses : 1][PAIR ? kCols / 4 : 1];
    if constexpr (PAIR) {
        typedef volatile __attribute__((address_space(1))) f32x4_t gvf32x4_t;
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass)
#pragma unroll
                for (int c = 0; c < kCols; c += 4)
                    pv[i][pass][c / 4] = *reinterpret_cast<gvf32x4_t*>(
                        (uintptr_t)(partner + ((uint64_t)(i * 32 + pass * kRowsPerPass + rl) * pld + cl + c) * 4u));
    }
    float bv[kCols];
#pragma unroll
    for (int c = 0; c < kCols; ++c) bv[c] = 0.0f;
    if (p.flags & T0G_FLAG_BIAS) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)p.bias, 0, (int)(p.n * 4u), (int)kRsrcWord3);
#pragma unroll
        for (int c = 0; c < kCols; ++c)
            bv[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (col0 + cl + c) * 4u, 0, 0));
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    }
    const uint64_t cbase = p.c + (uint64_t)split * p.c_split_stride;
    const uint32_t esize = OUT_BF16 ? 2u : 4u;
#pragma unroll
    for (int i = 0; i < SM; ++i) {
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = 8 * (r >> 2) + 4 * g + (r & 3);
                *reinterpret_cast<lds_f32*>((uintptr_t)(lds + row * E::kStride + (j * 32 + l32) * 4)) = acc[i][j][r];
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass) {
            const uint32_t rr = pass * kRowsPerPass + rl;
            float v[kCols];
#pragma unroll
            for (int c = 0; c < kCols; c += 4) {
                const f32x4_t q = *reinterpret_cast<const lds_f32x4*>((uintptr_t)(lds + rr * E::kStride + (cl + c) * 4));
                v[c] = q[0];
                v[c + 1] = q[1];
                v[c + 2] = q[2];
                v[c + 3] = q[3];
            }
            if constexpr (PAIR) {
#pragma unroll
                for (int c = 0; c < kCols; ++c) {
                    const float o = pv[i][pass][c / 4][c % 4];
                    v[c] = own_first ? (0.0f + v[c]) + o : (0.0f + o) + v[c];
                }
            }
            apply_epilogue_n<kCols>(v, bv, epi_of(p));
            const uint32_t grow = row0 + i * 32 + rr, gcol = col0 + cl;
            const uint64_t addr = cbase + ((uint64_t)grow * p.ldc + gcol) * esize;
            if (vec) {
                u32x4_t w;
                if constexpr (OUT_BF16) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const __bf16 lo = (__bf16)v[2 * c], hi = (__bf16)v[2 * c + 1];
                        w[c] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) w[c] = __builtin_bit_cast(uint32_t, v[c]);
                }
                // Non-temporal (unless WT or CACHED): C is not read again here, so
                // keep it from evicting A/B panels that later tiles on this XCD still
                // need.  CACHED: small split-K planes, read right after by the reduce.
                if constexpr (WT)
                    *reinterpret_cast<volatile __attribute__((address_space(1))) u32x4_t*>((uintptr_t)addr) = w;
                else if constexpr (CACHED)
                    *reinterpret_cast<__attribute__((address_space(1))) u32x4_t*>((uintptr_t)addr) = w;
                else
                    __builtin_nontemporal_store(w, reinterpret_cast<__attribute__((address_space(1))) u32x4_t*>((uintptr_t)addr));
            } else if (grow < p.m) {
#pragma unroll
                for (int c = 0; c < kCols; ++c) {
                    if (gcol + c < p.n) {
                        if constexpr (OUT_BF16)
                            reinterpret_cast<gbf16_t*>((uintptr_t)addr)[c] = (__bf16)v[c];
                        else
                            reinterpret_cast<gf32_t*>((uintptr_t)addr)[c] = v[c];
                    }
                }
            }
        }
        asm volatile("" ::: "memory");
    }
}

// ---------------------------------------------------------------------------
// Generic tile body: element-wise loads for rows that are not 16-byte
// aligned (K % 8 != 0 and the like); correctness path, not the fast path.
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
    const GridPos gp = grid_pos(p);
    const uint32_t bid = gp.tile;
    const uint32_t gm = p.group_m;
    const uint32_t per_group = gm * p.tiles_n;
    const uint32_t group = bid / per_group;
    const uint32_t first_m = group * gm;
    const uint32_t gsz = min(p.tiles_m - first_m, gm);
    const uint32_t in_group = bid - group * per_group;
    const uint32_t m0 = (first_m + in_group % gsz) * BM;
    const uint32_t n0 = (in_group / gsz) * BN;

    const uint32_t kbeg = gp.split * p.k_per_split;
    const uint32_t kend = min(p.k, kbeg + p.k_per_split);
    const int nkt = kend > kbeg ? (int)((kend - kbeg + kTileK - 1) / kTileK) : 0;

    gu16_t* __restrict__ A = reinterpret_cast<gu16_t*>(p.a);
    gu16_t* __restrict__ B = reinterpret_cast<gu16_t*>(p.b);

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

    store_tile<SM, SN, OUT_BF16>(p, acc, m0 + wm * WTM, n0 + wn * WTN, l32, g, gp.split);
}

// ---------------------------------------------------------------------------
// Fast tile body (16-byte aligned operands).
//
// Operands reach LDS through range-checked buffer loads straight into LDS
// (no VGPR staging).  The descriptor covers exactly the operand's extent, so
// rows past M/N or K past the operand read as zero without a clamp, and a K
// slice's tail is masked by sending the offset out of range.  The K loop is a
// ring of NS LDS stages of 32 K each; per stage s (two MFMA steps of K = 16):
//   issue the DMA of stage s + NS - 1 into the buffer stage s - 1 just freed
//   step 0: read step-1 fragments of stage s          | MFMAs of step 0
//   step 1: read step-0 fragments of stage s + 1      | MFMAs of step 1
//   wait until the DMA of stage s + 2 has landed; barrier
// Stage t's DMA thus has NS - 2 stages of MFMA work to arrive in, and the
// fragment reads of the next stage are in flight before the barrier, so the
// MFMA pipe does not drain at stage boundaries.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOob = 0x80000000u;    // offset past any descriptor range (operands < 2 GiB): loads return 0

// Descriptor over [base + shift, base + bytes).  A shift at or past the end
// gives an empty range (every load returns zero), never a wrapped one.
__device__ __forceinline__ rsrc_t make_rsrc(uint64_t base, uint32_t bytes, uint64_t shift) {
    const uint32_t rec = shift < bytes ? bytes - (uint32_t)shift : 0u;
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(base + shift), (short)0, (int)rec, kRsrcWord3);
}

__device__ __forceinline__ u32x4_t bload16(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Raw buffer descriptor words for [base + shift, base + bytes) (see make_rsrc).
__device__ __forceinline__ u32x4_t rsrc_words(uint64_t base, uint32_t bytes, uint64_t shift) {
    const uint32_t rec = shift < bytes ? bytes - (uint32_t)shift : 0u;
    const uint64_t a = base + shift;
    return u32x4_t{(uint32_t)a, (uint32_t)(a >> 32) & 0xFFFFu, rec, (uint32_t)kRsrcWord3};
}

// Descriptors read by the LDS-DMA asm are formed in scalar instructions only.
// A VALU write of an SGPR (v_readfirstlane, the form the compiler picks for a
// saturating subtract) needs wait states before a VMEM instruction reads that
// SGPR, and the compiler does not see the reads inside the asm: placed right
// before the first request of a group, it gave wrong results.  SALU writes
// need none (a VALU write read by SALU is interlocked).  The inputs are
// uniform: readfirstlane moves any the compiler holds in VGPRs to SGPRs.
__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
// {base + shift (48-bit address, high word masked), rec, word 3}
__device__ __forceinline__ u32x4_t rsrc_scalar(uint64_t base, uint64_t shift, uint32_t rec) {
    uint32_t lo, hi;
    asm("s_add_u32 %0, %2, %4\n\t"
        "s_addc_u32 %1, %3, %5\n\t"
        "s_and_b32 %1, %1, 0xffff"
        : "=&s"(lo), "=&s"(hi)
        : "s"(uniform_u32((uint32_t)base)), "s"(uniform_u32((uint32_t)(base >> 32))),
          "s"(uniform_u32((uint32_t)shift)), "s"(uniform_u32((uint32_t)(shift >> 32)))
        : "scc");
    return u32x4_t{lo, hi, rec, (uint32_t)kRsrcWord3};
}

// rsrc_words for shifts below 2^32 (the operands of the non-wide kernels):
// rec = max(bytes - shift, 0) by s_sub_u32 (SCC = borrow) and s_cselect.
__device__ __forceinline__ u32x4_t rsrc_words32(uint64_t base, uint32_t bytes, uint32_t shift) {
    uint32_t rec;
    asm("s_sub_u32 %0, %1, %2\n\t"
        "s_cselect_b32 %0, 0, %0"
        : "=&s"(rec)
        : "s"(uniform_u32(bytes)), "s"(uniform_u32(shift))
        : "scc");
    return rsrc_scalar(base, shift, rec);
}

// Wide form of rsrc_words for operands of any size: [base + shift, base + bytes)
// cut to its first 2 GiB (kOob stays out of range).  Callers shift it to the
// tile's first row (K-contiguous operands) or the stage's first k row
// (M/N-contiguous operands), so that every offset they use from there is below
// 2 GiB; the host checks the leading dimensions for that.  rec = min(max(bytes
// - shift, 0), kOob) in 64-bit scalar arithmetic.
__device__ __forceinline__ u32x4_t rsrc_words_wide(uint64_t base, uint64_t bytes, uint64_t shift) {
    uint32_t lo, hi;
    asm("s_sub_u32 %0, %2, %4\n\t"
        "s_subb_u32 %1, %3, %5\n\t"
        "s_cselect_b32 %0, 0, %0\n\t"       // borrow out: shift > bytes
        "s_cselect_b32 %1, 0, %1\n\t"
        "s_cmp_lg_u32 %1, 0\n\t"
        "s_cselect_b32 %0, 0x80000000, %0\n\t"
        "s_min_u32 %0, %0, 0x80000000"
        : "=&s"(lo), "=&s"(hi)
        : "s"(uniform_u32((uint32_t)bytes)), "s"(uniform_u32((uint32_t)(bytes >> 32))),
          "s"(uniform_u32((uint32_t)shift)), "s"(uniform_u32((uint32_t)(shift >> 32)))
        : "scc");
    static_assert(kOob == 0x80000000u, "the asm clamps to kOob");
    return rsrc_scalar(base, shift, lo);
}

// Bytes spanned by an operand of `rows` M/N rows and k K values with leading
// dimension ld: K-contiguous [rows][ld] or M/N-contiguous [k][ld].
template <bool K_MAJOR>
__device__ __forceinline__ uint64_t operand_bytes_wide(uint32_t rows, uint32_t k, uint32_t ld) {
    return K_MAJOR ? ((uint64_t)(rows - 1) * ld + k) * 2 : ((uint64_t)(k - 1) * ld + rows) * 2;
}

// 16-byte buffer load straight into LDS: lane l's data goes to LDS address
// m0 + 16 * l.  An SALU write of M0 needs one wait state before an LDS-DMA
// instruction reads it, hence the s_nop.  Completion is tracked by vmcnt only
// (callers wait with T0G_WAIT_VMCNT).
__device__ __forceinline__ void dma16(u32x4_t rsrc, uint32_t voff, uint32_t lds_m0) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %0, %1, 0 offen lds"
        :
        : "v"(voff), "s"(rsrc), "s"(lds_m0)
        : "memory", "m0");
}

// Grouped LDS DMA: the instruction's 12-bit immediate offset is added to both
// the descriptor offset and the LDS address (M0 + OFF + 16 * lane), so up to
// four 1 KB requests into consecutive LDS kilobytes share one M0 write: the
// group sets M0 once (dma_m0, with the wait state an SALU write of M0 needs
// before an LDS-DMA instruction reads it) and each request passes its piece's
// byte offset less OFF.  M0 is not otherwise used by this code (LDS
// instructions on gfx950 do not read it), so it holds between the requests.
__device__ __forceinline__ void dma_m0(uint32_t lds_base, uint32_t lds_off) {
    asm volatile(
        "s_add_u32 m0, %0, %1\n\t"
        "s_nop 0"
        :
        : "s"(lds_base), "s"(lds_off)
        : "memory", "m0", "scc");
}
template <uint32_t OFF>
__device__ __forceinline__ void dma16_off(u32x4_t rsrc, uint32_t voff) {
    static_assert(OFF < 4096, "12-bit immediate offset");
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen offset:%2 lds" : : "v"(voff), "s"(rsrc), "i"(OFF) : "memory");
}
// Request `slot` (0..3) of a group set up by dma_m0.
__device__ __forceinline__ void dma16_slot(u32x4_t rsrc, uint32_t voff, int slot) {
    switch (slot) {
        case 0: dma16_off<0>(rsrc, voff); break;
        case 1: dma16_off<1024>(rsrc, voff); break;
        case 2: dma16_off<2048>(rsrc, voff); break;
        default: dma16_off<3072>(rsrc, voff); break;
    }
}

// dma16 with the LDS address formed as lds_base + lds_off by one scalar add
// straight into M0.
__device__ __forceinline__ void dma16_at(u32x4_t rsrc, uint32_t voff, uint32_t lds_base, uint32_t lds_off) {
    asm volatile(
        "s_add_u32 m0, %2, %3\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %0, %1, 0 offen lds"
        :
        : "v"(voff), "s"(rsrc), "s"(lds_base), "s"(lds_off)
        : "memory", "m0", "scc");
}

// ---------------------------------------------------------------------------
// LDS layouts of the fast path (one pipeline stage holds BK = 32 or 64 K
// values of both operand tiles):
//   K-contiguous operand: one BK*2-byte row per M/N row; 16-byte chunk c of
//     row r is stored at chunk c ^ fk<BK>(r).  The 16 lanes of a ds_read_b128
//     phase read one logical chunk of 16 consecutive rows and touch distinct
//     banks.  One DMA instruction fills 1 KB = 16 rows (BK 32) or 8 whole
//     128-byte rows (BK 64, so every request is a full cache line).
//   M/N-contiguous operand: one row per k holding the tile's M/N extent; 32-byte
//     granule q of row k is stored at granule q ^ fm(k).  The 4 rows x 2
//     granules a half-wave of ds_read_b64_tr_b16 touches land in distinct banks.
// Both operands are copied global -> LDS by the buffer unit (LDS DMA): one
// wave instruction fills 1 KB, lane l writing the 16-byte slot l, so each lane
// fetches the global piece that the swizzle places in its slot.  Rows and K
// columns past the operand fall outside the descriptor range and read as zero.
// ---------------------------------------------------------------------------
// 32-bit LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Chunk swizzle of a K-contiguous row.  A 16-byte chunk's bank group (of 16)
// is (row * chunks_per_row + chunk) % 16.  BK 32 (4 chunks, 64 B rows): rows
// r, r+4, r+8, r+12 get four different values, so 16 consecutive rows reading
// one logical chunk cover all 16 groups.  BK 64 (8 chunks, 128 B rows): the 8
// rows of one parity among 16 consecutive rows get 8 different values.
// Neither depends on row bits >= 5, so 32-row sub-tiles are plain offsets.
template <uint32_t BK>
__device__ __forceinline__ uint32_t fk(uint32_t row) {
    if constexpr (BK == 32)
        return ((row >> 1) ^ (row >> 3)) & 3u;
    else
        return (row >> 1) & 7u;
}
__device__ __forceinline__ uint32_t fm(uint32_t k, uint32_t granules) {
    // {0, 2, 5, 7}[k % 4], reduced to the row's granule count
    return ((0x7520u >> ((k & 3u) * 4)) & 0xFu) & (granules - 1);
}

template <bool K_MAJOR, int ROWS, int NT, int SUBS, uint32_t BK>
struct DmaOperand;

// Fragment reads are ordinary LDS loads: the compiler inserts their lgkmcnt
// waits and the MFMA operand hazard padding.  (The LDS DMA is inline asm, so
// the compiler's wait-count pass never sees DMA in flight and adds no vmcnt
// drains before these reads.)
__device__ __forceinline__ bf16x8_t lds_load_b128(uint32_t addr) {
    return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>((uintptr_t)addr);
}
__device__ __forceinline__ void lds_load_tr16(uint32_t addr, short (&out)[4]) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(uintptr_t)addr);
    out[0] = v[0];
    out[1] = v[1];
    out[2] = v[2];
    out[3] = v[3];
}

// K-contiguous: LDS rows are M/N rows of BK*2 bytes.
template <int ROWS, int NT, int SUBS, uint32_t BK>
struct DmaOperand<true, ROWS, NT, SUBS, BK> {
    static constexpr int kWaves = NT / 64;
    static constexpr uint32_t kKRow = BK * 2;                      // bytes per LDS row
    static constexpr uint32_t kChunks = BK / 8;                    // 16-byte chunks per row
    static constexpr uint32_t kRowsPerInstr = 64 / kChunks;
    static constexpr int kInstr = ROWS * kKRow / 1024 / kWaves;   // per wave per stage
    static constexpr int kSteps = BK / 16;
    static_assert(kInstr >= 1 && ROWS * kKRow % (1024 * kWaves) == 0, "tile too small for the workgroup");
    static constexpr uint32_t kStageBytes = ROWS * kKRow;
    uint32_t off[kInstr];    // byte offset of the lane's piece at k = 0
    uint32_t kcol[kInstr];   // K column of the piece within the stage
    uint32_t wave;
    uint32_t frag[kSteps];   // LDS byte offset (within a stage) of the lane's chunk, per 16-wide K step

    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t ld, uint32_t wrow, uint32_t l32,
                                         uint32_t g) {
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t lane = tid & 63u;
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            const uint32_t q = i * kWaves + wave;
            const uint32_t r = kRowsPerInstr * q + lane / kChunks;
            const uint32_t c = (lane % kChunks) ^ fk<BK>(r);
            kcol[i] = c * 8;
            off[i] = ((row0 + r) * ld + c * 8) * 2;
        }
        const uint32_t row = wrow + l32;
#pragma unroll
        for (int kk = 0; kk < kSteps; ++kk) frag[kk] = row * kKRow + (((2u * kk + g) ^ fk<BK>(row)) << 4);
    }
    template <bool CHECK>
    __device__ __forceinline__ void issue(uint32_t lds, uint64_t base, uint32_t bytes, uint32_t ld, uint32_t k0,
                                          uint32_t kend) const {
        const u32x4_t r = rsrc(base, bytes, ld, k0);
#pragma unroll
        for (int i = 0; i < kInstr; ++i) issue_one<CHECK>(i, r, lds, k0, kend);
    }
    __device__ __forceinline__ u32x4_t rsrc(uint64_t base, uint32_t bytes, uint32_t, uint32_t k0) const {
        return rsrc_words32(base, bytes, k0 * 2u);
    }
    // CHECK: mask pieces at or past kend (a stage holding the K tail).  Without
    // it, pieces past kend read whatever follows in memory (or zero past the
    // descriptor range): fine for stages that are never consumed.
    template <bool CHECK>
    __device__ __forceinline__ void issue_one(int i, u32x4_t r, uint32_t lds, uint32_t k0, uint32_t kend) const {
        const uint32_t voff = CHECK ? (k0 + kcol[i] < kend ? off[i] : kOob) : off[i];
        dma16_at(r, voff, lds, (i * kWaves + wave) * 1024);
    }
    // Fragment of sub-tile `sub` (32 rows x 8 K values) for K step KK of the
    // stage at LDS address `stage`.
    template <int KK>
    __device__ __forceinline__ bf16x8_t read_one(uint32_t stage, int sub) const {
        return lds_load_b128(stage + frag[KK] + sub * 32 * kKRow);
    }
    // The same for a K step known at run time (uniform): kstep_off(kk) once,
    // then read_at per stage.  2*kk + g == 2*kk ^ g and the row offset has
    // zero chunk bits, so frag[kk] == frag[0] ^ (kk << 5).  Computed, not
    // selected from frag[]: a run-time index into the array makes the
    // compiler place it in LDS (18 KB more LDS, a store and reload in the
    // prologue, which cost the thin shapes 7 us per call).
    __device__ __forceinline__ uint32_t kstep_off(uint32_t kk) const { return frag[0] ^ (kk << 5); }
    __device__ __forceinline__ bf16x8_t read_at(uint32_t stage, int sub, uint32_t koff) const {
        return lds_load_b128(stage + koff + sub * 32 * kKRow);
    }
    template <int KK>
    __device__ __forceinline__ void read(uint32_t stage, bf16x8_t (&f)[SUBS]) const {
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) f[sub] = read_one<KK>(stage, sub);
    }
};

// M/N-contiguous: LDS rows are k rows of ROWS elements.
template <int ROWS, int NT, int SUBS, uint32_t BK>
struct DmaOperand<false, ROWS, NT, SUBS, BK> {
    static constexpr int kWaves = NT / 64;
    static constexpr uint32_t kRowB = ROWS * 2;
    static constexpr uint32_t kGranules = ROWS / 16;
    static constexpr uint32_t kStageBytes = BK * kRowB;
    static constexpr int kInstr = kStageBytes / 1024 / kWaves;
    static_assert(kInstr >= 1 && kStageBytes % (1024 * kWaves) == 0, "tile too small for the workgroup");
    static_assert(kGranules >= 4, "at least 4 granules per row");
    uint32_t off[kInstr];
    uint32_t krow[kInstr];
    uint32_t wave;
    uint32_t frag[SUBS];   // LDS byte offset (within a stage) of the lane's piece, K step 0, half 0

    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t ld, uint32_t wrow, uint32_t l32,
                                         uint32_t g) {
        (void)l32;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t lane = tid & 63u;
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            const uint32_t pos = (i * kWaves + wave) * 1024 + lane * 16;   // byte in the stage
            const uint32_t k = pos / kRowB;
            const uint32_t slot = (pos % kRowB) / 16;
            const uint32_t lg = (slot >> 1) ^ fm(k, kGranules);             // logical granule
            krow[i] = k;
            off[i] = (k * ld + row0 + lg * 16 + (slot & 1) * 8) * 2;
        }
        // ds_read_b64_tr_b16: in each 16-lane group, lane 4r+q points at k row
        // (base + r), columns colbase + 4q .. 4q+3; lane i then receives the 4
        // k values of column colbase + i.  The row is k = 16*kk + 8*g + 4*h + r;
        // fm depends on k % 4 = r only, so K step and half are plain offsets.
        const uint32_t r = (lane >> 2) & 3u, q = lane & 3u, gp = (lane >> 4) & 1u;
        const uint32_t k0 = 8 * g + r, f = fm(r, kGranules), gr = (wrow >> 4) + gp;
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) frag[sub] = k0 * kRowB + q * 8 + (((gr + 2 * sub) ^ f) << 5);
    }
    template <bool CHECK>
    __device__ __forceinline__ void issue(uint32_t lds, uint64_t base, uint32_t bytes, uint32_t ld, uint32_t k0,
                                          uint32_t kend) const {
        const u32x4_t r = rsrc(base, bytes, ld, k0);
#pragma unroll
        for (int i = 0; i < kInstr; ++i) issue_one<CHECK>(i, r, lds, k0, kend);
    }
    __device__ __forceinline__ u32x4_t rsrc(uint64_t base, uint32_t bytes, uint32_t ld, uint32_t k0) const {
        return rsrc_words32(base, bytes, k0 * ld * 2u);
    }
    // CHECK: mask pieces at or past kend (a stage holding the K tail).  Without
    // it, pieces past kend read whatever follows in memory (or zero past the
    // descriptor range): fine for stages that are never consumed.
    template <bool CHECK>
    __device__ __forceinline__ void issue_one(int i, u32x4_t r, uint32_t lds, uint32_t k0, uint32_t kend) const {
        const uint32_t voff = CHECK ? (k0 + krow[i] < kend ? off[i] : kOob) : off[i];
        dma16_at(r, voff, lds, (i * kWaves + wave) * 1024);
    }
    template <int KK>
    __device__ __forceinline__ void read(uint32_t stage, bf16x8_t (&f)[SUBS]) const {
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) f[sub] = read_one<KK>(stage, sub);
    }
    __device__ __forceinline__ uint32_t kstep_off(uint32_t kk) const { return kk * 16 * kRowB; }
    __device__ __forceinline__ bf16x8_t read_at(uint32_t stage, int sub, uint32_t koff) const {
        short v[8];
        short(&lo)[4] = *reinterpret_cast<short(*)[4]>(&v[0]);
        short(&hi)[4] = *reinterpret_cast<short(*)[4]>(&v[4]);
        lds_load_tr16(stage + frag[sub] + koff, lo);
        lds_load_tr16(stage + frag[sub] + koff + 4 * kRowB, hi);
        typedef short v8s __attribute__((ext_vector_type(8)));
        const v8s w = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
        return __builtin_bit_cast(bf16x8_t, w);
    }
    template <int KK>
    __device__ __forceinline__ bf16x8_t read_one(uint32_t stage, int sub) const {
        constexpr int O0 = KK * 16 * kRowB, O1 = (KK * 16 + 4) * kRowB;
        short v[8];
        short(&lo)[4] = *reinterpret_cast<short(*)[4]>(&v[0]);
        short(&hi)[4] = *reinterpret_cast<short(*)[4]>(&v[4]);
        lds_load_tr16(stage + frag[sub] + O0, lo);
        lds_load_tr16(stage + frag[sub] + O1, hi);
        typedef short v8s __attribute__((ext_vector_type(8)));
        const v8s w = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
        return __builtin_bit_cast(bf16x8_t, w);
    }
};

template <int SM, int SN>
__device__ __forceinline__ void mfma_step(f32x16_t (&acc)[SM][SN], const bf16x8_t (&fa)[SM],
                                          const bf16x8_t (&fb)[SN]) {
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
}

// s_waitcnt with only vmcnt = n (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
#define T0G_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14))

// Workgroup barrier without __syncthreads()'s release fence: the fence would
// wait for every LDS DMA in flight (vmcnt(0)), draining the prefetch ring.
// Callers retire exactly the DMA they need with T0G_WAIT_VMCNT first; the
// asm memory clobbers keep the compiler from moving LDS accesses across it.
// LDS reads still in flight at the barrier target the next stage's buffer,
// which nobody overwrites before the following barrier, so no lgkmcnt wait.
__device__ __forceinline__ void barrier_no_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One 16-wide K step (STEP of NSTEPS in a stage): SM rows of SN MFMAs on
// (fa, fb), interleaved with the LDS reads of the next step's fragments into
// (na, nb) -- from stage `cur`, or from `nxt` after the stage's last step --
// and with DMA instructions [DFIRST, DFIRST + DCOUNT) of the stage being
// filled.  sched_barrier pins the row order, so MFMAs stay queued while a DMA
// instruction issues.
// Per row of MFMAs, the DMA instructions and fragment reads are placed one at
// a time behind individual MFMAs (DMA, read, DMA, read, ...), so no two long
// issues sit between consecutive MFMAs.  Item t of a row with nd DMAs and nr
// reads: kind 0 = DMA, 1 = read; returns kind * 256 + index.
__host__ __device__ constexpr int row_item(int t, int nd, int nr) {
    const int both = nd < nr ? nd : nr;
    if (t < 2 * both) return (t & 1) * 256 + (t >> 1);
    return nd > nr ? (t - both) : 256 + (t - both);
}

template <int STEP, int NSTEPS, int DFIRST, int DCOUNT, bool CHECK, int RB = 0, int RE = -1, int RR = 0, int SM,
          int SN, class OpA, class OpB>
__device__ __forceinline__ void mfma_rows(f32x16_t (&acc)[SM][SN], const bf16x8_t (&fa)[SM], const bf16x8_t (&fb)[SN],
                                          bf16x8_t (&na)[SM], bf16x8_t (&nb)[SN], const OpA& la, const OpB& lb,
                                          uint32_t cur, uint32_t nxt, uint32_t fill, u32x4_t ra, u32x4_t rb,
                                          uint32_t kf, uint32_t kend) {
    // Rows [RB, RE) of the step; the next step's fragment reads go to rows
    // [RR, RE) (all of them: a step split in two calls gives the reads to the
    // second), the DMA instructions are spread over all rows of this call.
    constexpr int kRE = RE < 0 ? SM : RE;
    constexpr int NEXT_KK = (STEP + 1) % NSTEPS;
    const uint32_t rd = STEP + 1 < NSTEPS ? cur : nxt;
    constexpr int kRows = kRE - RB;
    constexpr int kPerRow = (DCOUNT + kRows - 1) / kRows;
    // Read placement: the next step's row r needs A[r] and all of B, so A[r]
    // is read in row r and B two fragments per row from the first read row
    // on: every fragment then has at least three rows of MFMAs to land.
    constexpr int kReadRows = kRE - RR;
#pragma unroll
    for (int i = RB; i < kRE; ++i) {
        const int bfirst = kReadRows > 0 ? 2 * (i - RR) : SN;
        const int blast = i == kRE - 1 ? SN : 2 * (i - RR) + 2;   // the last read row takes any B left
        const int nbr = i < RR ? 0 : (blast < SN ? blast : SN) - (bfirst < SN ? bfirst : SN);
        const int nar = i < RR ? 0 : (kReadRows == SM ? 1 : (i == RR ? SM : 0));
        const int nr = nbr + nar;
        const int nitems = kPerRow + nr;
        const int per_slot = (nitems + SN - 1) / SN;
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int u = 0; u < per_slot; ++u) {
                const int t = j * per_slot + u;
                if (t < nitems) {
                    const int it = row_item(t, kPerRow, nr);
                    if (it >= 256) {
                        const int q = it - 256;   // B reads of this row first, then its A reads
                        if (q < nbr)
                            nb[bfirst + q] = lb.template read_one<NEXT_KK>(rd + OpA::kStageBytes, bfirst + q);
                        else if (kReadRows == SM)
                            na[i] = la.template read_one<NEXT_KK>(rd, i);
                        else
                            na[q - nbr] = la.template read_one<NEXT_KK>(rd, q - nbr);
                    } else {
                        const int q = DFIRST + (i - RB) * kPerRow + it;
                        if (q < DFIRST + DCOUNT) {
                            if (q < OpA::kInstr)
                                la.template issue_one<CHECK>(q, ra, fill, kf, kend);
                            else
                                lb.template issue_one<CHECK>(q - OpA::kInstr, rb, fill + OpA::kStageBytes, kf, kend);
                        }
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// The K loop of the fast path (128x128 and 64x64 tiles): ring of NS >= 4
// stages of BK 32 or 64, DMA NS-1 stages ahead, one barrier per stage.  A
// stage's BK / 16 K steps alternate between two fragment register sets; the
// stage's DMA instructions are spread evenly over its steps.  BK 64 makes each
// K-contiguous LDS row a whole 128-byte line, so every DMA request fetches
// complete cache lines (the deep-ring kernels, one workgroup per CU).
template <bool CHECK, uint32_t BK, int NS, uint32_t A_BYTES, uint32_t STAGE, int kVmemPerStage, int SM, int SN,
          class OpA, class OpB>
__device__ __forceinline__ void k_pipeline(f32x16_t (&acc)[SM][SN], const OpA& la, const OpB& lb, const T0gGemmArgs& p,
                                           uint32_t a_bytes, uint32_t b_bytes, uint32_t kbeg, uint32_t kend, int nst,
                                           uint32_t lds0) {
    static_assert((BK == 32 || BK == 64) && NS >= 4, "ring of BK 32 or 64 stages");
    constexpr int kSteps = (int)BK / 16;
    // DMA instructions of the stage before K step i: [kD(i), kD(i + 1))
    constexpr int kPer = (kVmemPerStage + kSteps - 1) / kSteps;
#define T0G_KD(i) ((i) * kPer < kVmemPerStage ? (i) * kPer : kVmemPerStage)
    bf16x8_t fa0[SM], fb0[SN], fa1[SM], fb1[SN];
    {
        // Prologue: stages 0 .. NS-2 in flight; stages 0 and 1 must have landed.
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) {
            la.template issue<CHECK>(lds0 + s * STAGE, p.a, a_bytes, p.lda, kbeg + s * BK, kend);
            lb.template issue<CHECK>(lds0 + s * STAGE + A_BYTES, p.b, b_bytes, p.ldb, kbeg + s * BK, kend);
        }
        T0G_WAIT_VMCNT(kVmemPerStage * (NS - 3));
        barrier_no_fence();
        la.template read<0>(lds0, fa0);
        lb.template read<0>(lds0 + A_BYTES, fb0);

        uint32_t cur = 0;                 // byte offset of stage s's buffer
        uint32_t fill = (NS - 1) * STAGE; // buffer receiving stage s + NS - 1
        for (int s = 0; s < nst; ++s) {
            const uint32_t nxt = cur + STAGE == NS * STAGE ? 0 : cur + STAGE;
            const uint32_t kf = kbeg + (uint32_t)(s + NS - 1) * BK;
            const u32x4_t ra = la.rsrc(p.a, a_bytes, p.lda, kf);
            const u32x4_t rb = lb.rsrc(p.b, b_bytes, p.ldb, kf);
            // K step i of stage s reads step i + 1's fragments (the last step:
            // step 0 of stage s + 1, landed before the last barrier).
            mfma_rows<0, kSteps, T0G_KD(0), T0G_KD(1) - T0G_KD(0), CHECK>(
                acc, fa0, fb0, fa1, fb1, la, lb, lds0 + cur, lds0 + nxt, lds0 + fill, ra, rb, kf, kend);
            mfma_rows<1, kSteps, T0G_KD(1), T0G_KD(2) - T0G_KD(1), CHECK>(
                acc, fa1, fb1, fa0, fb0, la, lb, lds0 + cur, lds0 + nxt, lds0 + fill, ra, rb, kf, kend);
            if constexpr (kSteps == 4) {
                mfma_rows<2, kSteps, T0G_KD(2), T0G_KD(3) - T0G_KD(2), CHECK>(
                    acc, fa0, fb0, fa1, fb1, la, lb, lds0 + cur, lds0 + nxt, lds0 + fill, ra, rb, kf, kend);
                mfma_rows<3, kSteps, T0G_KD(3), T0G_KD(4) - T0G_KD(3), CHECK>(
                    acc, fa1, fb1, fa0, fb0, la, lb, lds0 + cur, lds0 + nxt, lds0 + fill, ra, rb, kf, kend);
            }
            T0G_WAIT_VMCNT(kVmemPerStage * (NS - 3));   // stage s+2 has landed
            barrier_no_fence();
            fill = cur;
            cur = nxt;
        }
    }
#undef T0G_KD
}

// Deep-ring K loop of the 64x64 tile (BK 64, one workgroup per CU, one 32x32
// MFMA block per wave): the fragments of a whole stage are read one stage
// ahead, right after the barrier that makes the stage visible, into one of
// two register sets, so every LDS read has a stage of MFMAs, DMA issue and
// the barrier to land.  Reading one K step ahead, as k_pipeline does, leaves
// the wave's single MFMA per step waiting on that step's reads: the thin
// 128x4096x4096 GEMM (64x64, split 2) went from 15.2 to 14.1 us per call,
// 256x256x32768 (split 16) from 15.3 to 13.7 us.  The 128x128 deep kernels
// (four MFMA blocks per wave) keep k_pipeline: on this loop they ran 84 ->
// 92 us on 1024x4096x11008.  MFMAs run in the same K order as k_pipeline's,
// so the results are the same bit for bit.
template <int KK, int SM, int SN, class OpA, class OpB>
__device__ __forceinline__ void read_step(const OpA& la, const OpB& lb, uint32_t stage, bf16x8_t (&fa)[SM],
                                          bf16x8_t (&fb)[SN]) {
#pragma unroll
    for (int i = 0; i < SM; ++i) fa[i] = la.template read_one<KK>(stage, i);
#pragma unroll
    for (int j = 0; j < SN; ++j) fb[j] = lb.template read_one<KK>(stage + OpA::kStageBytes, j);
}

template <int SM, int SN, class OpA, class OpB>
__device__ __forceinline__ void read_stage4(const OpA& la, const OpB& lb, uint32_t stage, bf16x8_t (&fa)[4][SM],
                                            bf16x8_t (&fb)[4][SN]) {
    read_step<0>(la, lb, stage, fa[0], fb[0]);
    read_step<1>(la, lb, stage, fa[1], fb[1]);
    read_step<2>(la, lb, stage, fa[2], fb[2]);
    read_step<3>(la, lb, stage, fa[3], fb[3]);
}

// One K step's MFMAs with DMA instructions [DFIRST, DFIRST + DCOUNT) of the
// stage being filled spread behind them.
template <int DFIRST, int DCOUNT, bool CHECK, int SM, int SN, class OpA, class OpB>
__device__ __forceinline__ void mfma_step_dma(f32x16_t (&acc)[SM][SN], const bf16x8_t (&fa)[SM],
                                              const bf16x8_t (&fb)[SN], const OpA& la, const OpB& lb, uint32_t fill,
                                              u32x4_t ra, u32x4_t rb, uint32_t kf, uint32_t kend) {
    constexpr int kSlots = SM * SN;
    constexpr int kPer = (DCOUNT + kSlots - 1) / kSlots;
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int q = DFIRST + (i * SN + j) * kPer + u;
                if (q < DFIRST + DCOUNT) {
                    if (q < OpA::kInstr)
                        la.template issue_one<CHECK>(q, ra, fill, kf, kend);
                    else
                        lb.template issue_one<CHECK>(q - OpA::kInstr, rb, fill + OpA::kStageBytes, kf, kend);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
}

// One stage: read stage `nxt` into (na, nb), multiply the current stage from
// (fa, fb), refill `fill` with stage kf's DMA, then wait for the stage two
// ahead and meet at the barrier.
template <bool CHECK, int NS, uint32_t STAGE, int kVmemPerStage, int SM, int SN, class OpA, class OpB>
__device__ __forceinline__ void deep_stage(f32x16_t (&acc)[SM][SN], const bf16x8_t (&fa)[4][SM],
                                           const bf16x8_t (&fb)[4][SN], bf16x8_t (&na)[4][SM], bf16x8_t (&nb)[4][SN],
                                           const OpA& la, const OpB& lb, const T0gGemmArgs& p, uint32_t a_bytes,
                                           uint32_t b_bytes, uint32_t nxt, uint32_t fill, uint32_t kf, uint32_t kend) {
    constexpr int kPer = (kVmemPerStage + 3) / 4;
#define T0G_KD4(i) ((i) * kPer < kVmemPerStage ? (i) * kPer : kVmemPerStage)
    read_stage4(la, lb, nxt, na, nb);
    const u32x4_t ra = la.rsrc(p.a, a_bytes, p.lda, kf);
    const u32x4_t rb = lb.rsrc(p.b, b_bytes, p.ldb, kf);
    mfma_step_dma<T0G_KD4(0), T0G_KD4(1) - T0G_KD4(0), CHECK>(acc, fa[0], fb[0], la, lb, fill, ra, rb, kf, kend);
    mfma_step_dma<T0G_KD4(1), T0G_KD4(2) - T0G_KD4(1), CHECK>(acc, fa[1], fb[1], la, lb, fill, ra, rb, kf, kend);
    mfma_step_dma<T0G_KD4(2), T0G_KD4(3) - T0G_KD4(2), CHECK>(acc, fa[2], fb[2], la, lb, fill, ra, rb, kf, kend);
    mfma_step_dma<T0G_KD4(3), T0G_KD4(4) - T0G_KD4(3), CHECK>(acc, fa[3], fb[3], la, lb, fill, ra, rb, kf, kend);
#undef T0G_KD4
    T0G_WAIT_VMCNT(kVmemPerStage * (NS - 3));   // the stage two ahead has landed
    barrier_no_fence();
}

template <bool CHECK, int NS, uint32_t A_BYTES, uint32_t STAGE, int kVmemPerStage, int SM, int SN, class OpA,
          class OpB>
__device__ __forceinline__ void k_pipeline_deep(f32x16_t (&acc)[SM][SN], const OpA& la, const OpB& lb,
                                                const T0gGemmArgs& p, uint32_t a_bytes, uint32_t b_bytes,
                                                uint32_t kbeg, uint32_t kend, int nst, uint32_t lds0) {
    static_assert(NS >= 4, "ring of at least 4 stages");
    constexpr uint32_t BK = 64;
    bf16x8_t fa0[4][SM], fb0[4][SN], fa1[4][SM], fb1[4][SN];
    // Prologue: stages 0 .. NS-2 in flight; stages 0 and 1 must have landed.
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        la.template issue<CHECK>(lds0 + s * STAGE, p.a, a_bytes, p.lda, kbeg + s * BK, kend);
        lb.template issue<CHECK>(lds0 + s * STAGE + A_BYTES, p.b, b_bytes, p.ldb, kbeg + s * BK, kend);
    }
    T0G_WAIT_VMCNT(kVmemPerStage * (NS - 3));
    barrier_no_fence();
    read_stage4(la, lb, lds0, fa0, fb0);

    uint32_t cur = 0;                  // byte offset of stage s's buffer
    uint32_t fill = (NS - 1) * STAGE;  // buffer receiving stage s + NS - 1
    for (int s = 0; s < nst; s += 2) {
        {
            const uint32_t nxt = cur + STAGE == NS * STAGE ? 0 : cur + STAGE;
            const uint32_t kf = kbeg + (uint32_t)(s + NS - 1) * BK;
            deep_stage<CHECK, NS, STAGE, kVmemPerStage>(acc, fa0, fb0, fa1, fb1, la, lb, p, a_bytes, b_bytes,
                                                        lds0 + nxt, lds0 + fill, kf, kend);
            fill = cur;
            cur = nxt;
        }
        if (s + 1 < nst) {
            const uint32_t nxt = cur + STAGE == NS * STAGE ? 0 : cur + STAGE;
            const uint32_t kf = kbeg + (uint32_t)(s + NS) * BK;
            deep_stage<CHECK, NS, STAGE, kVmemPerStage>(acc, fa1, fb1, fa0, fb0, la, lb, p, a_bytes, b_bytes,
                                                        lds0 + nxt, lds0 + fill, kf, kend);
            fill = cur;
            cur = nxt;
        }
    }
}

// K split across the waves (64x64 deep kernels): wave w multiplies the whole
// 64x64 tile (2 x 2 blocks of 32x32) for K step w of every 64-K stage, so each
// A and B row is read from LDS once per stage (4 fragment reads per wave
// instead of the 8 of the 2 x 2 wave grid, where every row was read by two
// waves).  The LDS DMA of a stage and the fragment reads of the next share the
// CU's LDS; halving the reads took the C4a loop from 10.0 to 8.4 us in a
// standalone model of this kernel, and a C4a call (128 x 4096 x 4096 NT,
// split 2, plus the reduce) from 14.2 to 13.75 us.  Fragments of the next stage are read one
// stage ahead, as in k_pipeline_deep; the four DMA instructions of the stage
// being filled go one behind each MFMA.  ksplit_sum() then adds the four
// partial tiles in wave order.
template <bool CHECK, int NS, uint32_t A_BYTES, uint32_t STAGE, int kVmemPerStage, class OpA, class OpB>
__device__ __forceinline__ void k_pipeline_ksplit(f32x16_t (&acc)[2][2], const OpA& la, const OpB& lb,
                                                  const T0gGemmArgs& p, uint32_t a_bytes, uint32_t b_bytes,
                                                  uint32_t kbeg, uint32_t kend, int nst, uint32_t lds0) {
    static_assert(NS >= 4, "ring of at least 4 stages");
    static_assert(kVmemPerStage == 4, "one DMA instruction behind each of the four MFMAs");
    constexpr uint32_t BK = 64;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ka = la.kstep_off(w), kb = lb.kstep_off(w);
    auto read4 = [&](uint32_t stage, bf16x8_t (&fa)[2], bf16x8_t (&fb)[2]) {
        fa[0] = la.read_at(stage, 0, ka);
        fa[1] = la.read_at(stage, 1, ka);
        fb[0] = lb.read_at(stage + A_BYTES, 0, kb);
        fb[1] = lb.read_at(stage + A_BYTES, 1, kb);
    };
    auto issue_q = [&](int q, u32x4_t ra, u32x4_t rb, uint32_t fill, uint32_t kf) {
        if (q < OpA::kInstr)
            la.template issue_one<CHECK>(q, ra, fill, kf, kend);
        else
            lb.template issue_one<CHECK>(q - OpA::kInstr, rb, fill + A_BYTES, kf, kend);
    };
    // one stage: read stage `nxt` into (na, nb), multiply (fa, fb) with the
    // DMA of stage kf into `fill` behind the MFMAs, wait for the stage two
    // ahead and meet at the barrier
    auto stage_step = [&](const bf16x8_t (&fa)[2], const bf16x8_t (&fb)[2], bf16x8_t (&na)[2], bf16x8_t (&nb)[2],
                          uint32_t nxt, uint32_t fill, uint32_t kf) {
        read4(nxt, na, nb);
        const u32x4_t ra = la.rsrc(p.a, a_bytes, p.lda, kf);
        const u32x4_t rb = lb.rsrc(p.b, b_bytes, p.ldb, kf);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                issue_q(i * 2 + j, ra, rb, fill, kf);
                __builtin_amdgcn_sched_barrier(0);
            }
        T0G_WAIT_VMCNT(kVmemPerStage * (NS - 3));   // the stage two ahead has landed
        barrier_no_fence();
    };
    bf16x8_t fa0[2], fb0[2], fa1[2], fb1[2];
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        la.template issue<CHECK>(lds0 + s * STAGE, p.a, a_bytes, p.lda, kbeg + s * BK, kend);
        lb.template issue<CHECK>(lds0 + s * STAGE + A_BYTES, p.b, b_bytes, p.ldb, kbeg + s * BK, kend);
    }
    T0G_WAIT_VMCNT(kVmemPerStage * (NS - 3));
    barrier_no_fence();
    read4(lds0, fa0, fb0);

    uint32_t cur = 0;
    uint32_t fill = (NS - 1) * STAGE;
    for (int s = 0; s < nst; s += 2) {
        {
            const uint32_t nxt = cur + STAGE == NS * STAGE ? 0 : cur + STAGE;
            stage_step(fa0, fb0, fa1, fb1, lds0 + nxt, lds0 + fill, kbeg + (uint32_t)(s + NS - 1) * BK);
            fill = cur;
            cur = nxt;
        }
        if (s + 1 < nst) {
            const uint32_t nxt = cur + STAGE == NS * STAGE ? 0 : cur + STAGE;
            stage_step(fa1, fb1, fa0, fb0, lds0 + nxt, lds0 + fill, kbeg + (uint32_t)(s + NS) * BK);
            fill = cur;
            cur = nxt;
        }
    }
}

// Sum the four waves' partial 64x64 tiles (each 2 x 2 blocks of 32x32 in the
// MFMA result layout) through LDS, in wave order ((w0 + w1) + w2) + w3, and
// return wave w's own 32x32 block (block w = the quadrant (w / 2, w % 2) the
// 2 x 2 wave grid's epilogue stores).  Needs 64 KB of LDS at `lds`; callers
// have finished with the ring (vmcnt(0) and a barrier).  Every wave writes all
// four blocks and reads four: a form that writes and reads only the three
// foreign blocks, with no barrier after the reads, ran 0.5-0.9 us slower per
// call on the thin shapes.  It ends with a barrier, before the epilogue reuses
// the LDS.
__device__ __forceinline__ f32x16_t ksplit_sum(const f32x16_t (&acc)[2][2], uint32_t lds) {
    typedef __attribute__((address_space(3))) float lds_f32;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            *reinterpret_cast<lds_f32*>((uintptr_t)(lds + ((w * 4 + b) * 1024 + e * 64 + lane) * 4)) = acc[b >> 1][b & 1][e];
    __syncthreads();
    f32x16_t r;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        float v = 0.0f;
#pragma unroll
        for (int src = 0; src < 4; ++src)
            v = v + *reinterpret_cast<const lds_f32*>((uintptr_t)(lds + ((src * 4 + w) * 1024 + e * 64 + lane) * 4));
        r[e] = v;
    }
    __syncthreads();
    return r;
}

}  // namespace t0g

#include "gemm_red.h"
#include "gemm_mfma16.h"

namespace t0g {

// Fast path: one BM x BN output tile per workgroup, operands streamed through
// LDS by DMA (k_pipeline), epilogue staged through LDS.  RED: split-K reduced
// inside the kernel (ra: the launch's T0gGemmRedArgs, p = ra->g).
template <int BM, int BN, int WAVES_M, int WAVES_N, bool A_K, bool B_K, bool OUT_BF16, uint32_t BK, int NS,
          bool RED = false, bool KS = false>
__device__ __forceinline__ void gemm_tile_fast(const T0gGemmArgs& p, const T0gGemmRedArgs* ra = nullptr) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int SM = WTM / 32, SN = WTN / 32;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
    static_assert((BK == 32 || BK == 64) && NS >= 4, "unsupported pipeline shape");
    using OpA = DmaOperand<A_K, BM, NT, SM, BK>;
    using OpB = DmaOperand<B_K, BN, NT, SN, BK>;
    constexpr uint32_t A_BYTES = OpA::kStageBytes, STAGE = OpA::kStageBytes + OpB::kStageBytes;
    constexpr int kVmemPerStage = OpA::kInstr + OpB::kInstr;
    __shared__ __attribute__((aligned(1024))) char smem[NS * STAGE];

    tl_mark(p, 0);
    const uint32_t tid = threadIdx.x;
    const GridPos gp = grid_pos(p);
    const uint32_t bid = gp.tile;
    const uint32_t gm = p.group_m;
    const uint32_t per_group = gm * p.tiles_n;
    const uint32_t group = bid / per_group;
    const uint32_t first_m = group * gm;
    const uint32_t gsz = min(p.tiles_m - first_m, gm);
    const uint32_t in_group = bid - group * per_group;
    const uint32_t m0 = (first_m + in_group % gsz) * BM;
    const uint32_t n0 = (in_group / gsz) * BN;

    const uint32_t kbeg = gp.split * p.k_per_split;
    const uint32_t kend = min(p.k, kbeg + p.k_per_split);
    const int nst = kend > kbeg ? (int)((kend - kbeg + BK - 1) / BK) : 0;

    const uint32_t a_bytes = (A_K ? (p.m - 1) * p.lda + p.k : (p.k - 1) * p.lda + p.m) * 2;
    const uint32_t b_bytes = (B_K ? (p.n - 1) * p.ldb + p.k : (p.k - 1) * p.ldb + p.n) * 2;

    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave / WAVES_N, wn = wave % WAVES_N;
    const uint32_t l32 = lane & 31u, g = lane >> 5;
    OpA la;
    OpB lb;
    la.init(tid, m0, p.lda, wm * WTM, l32, g);
    lb.init(tid, n0, p.ldb, wn * WTN, l32, g);

    f32x16_t acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j) acc[i][j] = f32x16_t{};
    // KS (64x64 deep ring only): K split across the waves (k_pipeline_ksplit),
    // whole-tile partials summed by ksplit_sum() after the loop.  The host
    // takes these kernels (suffix _ds, _dsr) for K ranges of 24 stages or more.
    constexpr bool KSPLIT = KS;
    static_assert(!KS || (BK == 64 && SM * SN == 1), "K split across the waves: 64x64 deep ring only");
    f32x16_t acc4[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc4[i][j] = f32x16_t{};

    if (nst > 0) {
        const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
        // Stages past a K tail need masked DMA; whole stages (the usual case)
        // skip the per-lane bound test.
        if constexpr (KSPLIT) {
            static_assert(WAVES_M == 2 && WAVES_N == 2, "four waves, one K step each");
            // operands with both 32-row sub-tiles of the tile, from row 0
            DmaOperand<A_K, BM, NT, 2, BK> ka;
            DmaOperand<B_K, BN, NT, 2, BK> kb;
            ka.init(tid, m0, p.lda, 0, l32, g);
            kb.init(tid, n0, p.ldb, 0, l32, g);
            if ((kend - kbeg) % BK == 0)
                k_pipeline_ksplit<false, NS, A_BYTES, STAGE, kVmemPerStage>(acc4, ka, kb, p, a_bytes, b_bytes, kbeg,
                                                                            kend, nst, lds0);
            else
                k_pipeline_ksplit<true, NS, A_BYTES, STAGE, kVmemPerStage>(acc4, ka, kb, p, a_bytes, b_bytes, kbeg,
                                                                           kend, nst, lds0);
        } else if constexpr (BK == 64 && SM * SN == 1) {
            if ((kend - kbeg) % BK == 0)
                k_pipeline_deep<false, NS, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg,
                                                                          kend, nst, lds0);
            else
                k_pipeline_deep<true, NS, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg,
                                                                         kend, nst, lds0);
        } else {
            if ((kend - kbeg) % BK == 0)
                k_pipeline<false, BK, NS, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg,
                                                                          kend, nst, lds0);
            else
                k_pipeline<true, BK, NS, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg,
                                                                         kend, nst, lds0);
        }
    }

    // Epilogue through LDS: 16-byte row stores for tiles wholly inside an
    // aligned C, per-element masked stores otherwise.
    static_assert((NT / 64) * VecEpilogue<SN>::kWaveBytes <= NS * STAGE, "epilogue staging must fit the LDS ring");
    T0G_WAIT_VMCNT(0);    // LDS DMA still in flight (stages past K) has landed
    barrier_no_fence();   // and every wave is done with the ring
    if constexpr (KSPLIT) {
        static_assert(4 * 4 * 16 * 64 * 4 <= NS * STAGE, "the partial tiles must fit the LDS ring");
        acc[0][0] = ksplit_sum(acc4, lds_addr(smem));
    }
    tl_mark(p, 1);
    if constexpr (RED) {
        // the partial tile, raw fp32, row-major into this workgroup's slot
        T0gGemmArgs q = p;
        q.c = ra->partials + (uint64_t)(gp.tile * ra->splits + gp.split) * (BM * BN * 4u);
        q.ldc = BN;
        q.c_split_stride = 0;
        q.epilogue = 0;
        q.flags = T0G_FLAG_C_VEC;
        store_tile_vec<SM, SN, false, true>(q, acc, wm * WTM, wn * WTN, lane,
                                            lds_addr(smem) + wave * VecEpilogue<SN>::kWaveBytes, true, 0);
        T0G_WAIT_VMCNT(0);    // the partial's stores have reached memory
        barrier_no_fence();
        if (ra->splits == 2u)
            red_pair<BM, BN, SM, SN, OUT_BF16>(*ra, acc, gp.tile, gp.split, m0, n0, wm * WTM, wn * WTN, lane,
                                               lds_addr(smem) + wave * VecEpilogue<SN>::kWaveBytes);
        else
            red_finish<BM, BN, NT, OUT_BF16>(*ra, gp.tile, gp.split, m0, n0, lds_addr(smem), NS * STAGE);
    } else {
        const bool vec = (p.flags & T0G_FLAG_C_VEC) && m0 + BM <= p.m && n0 + BN <= p.n;
        // the store form is chosen once per tile (a test of the flag next to each
        // store cost 0.27 us per call on 128 x 4096 x 4096 NN, where it is not set)
        if (p.flags & T0G_FLAG_C_CACHED)
            store_tile_vec<SM, SN, OUT_BF16, false, true>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane,
                                                          lds_addr(smem) + wave * VecEpilogue<SN>::kWaveBytes, vec,
                                                          gp.split);
        else
            store_tile_vec<SM, SN, OUT_BF16>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane,
                                             lds_addr(smem) + wave * VecEpilogue<SN>::kWaveBytes, vec, gp.split);
    }
    tl_mark(p, 2);
}

// Plane-ordered split-K reduction: y = ((0 + p0) + p1) + ... in fp32, the
// order the reference's host loop uses (examples/test_gemm_correctness.rs:190-207),
// then the epilogue and the output conversion.  Vector form (T0G_REDUCE_VEC):
// each thread owns 4 consecutive columns, loads up to 8 planes' float4 at once
// (all in flight together) and adds them in plane order.
template <bool OUT_BF16>
__device__ __forceinline__ void splitk_reduce(const T0gReduceArgs& p) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    const __attribute__((address_space(1))) float* ws = reinterpret_cast<const __attribute__((address_space(1))) float*>(p.ws);
    const __attribute__((address_space(1))) float* bias =
        reinterpret_cast<const __attribute__((address_space(1))) float*>(p.bias);
    if (p.flags & T0G_REDUCE_WAVE) {
        // Large outputs: each wave sums 128 items of 4 consecutive elements (of the
        // row-major M x N output) per grid step.  Per plane a lane makes two 16-byte
        // non-temporal loads, and each load instruction covers 1 KB of consecutive
        // plane; four planes are in flight.  Two 4-element stores follow.  The
        // workgroups cover the output in one step up to the grid cap.
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        typedef const __attribute__((address_space(1))) f32x4_t gf32x4_t;
        const uint64_t nq = p.n >> 2, total = (uint64_t)p.m * nq;
        const uint32_t lane = threadIdx.x & 63u;
        const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const uint64_t step = (uint64_t)p.grid_blocks * 4 * 128;
        for (uint64_t wb = ((uint64_t)blockIdx.x * 4 + wave) * 128; wb < total; wb += step) {
            uint64_t item[2] = {wb + lane, wb + 64 + lane};
            bool live[2] = {item[0] < total, item[1] < total};
            f32x4_t acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
            for (uint32_t s0 = 0; s0 < p.splits; s0 += 4) {
                f32x4_t v[4][2];
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        if (s0 + u < p.splits && live[h])
                            v[u][h] = __builtin_nontemporal_load(
                                reinterpret_cast<gf32x4_t*>(ws + (s0 + u) * p.plane_elems) + item[h]);
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u)
                    if (s0 + u < p.splits)
#pragma unroll
                        for (int h = 0; h < 2; ++h) acc[h] = acc[h] + v[u][h];
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (!live[h]) continue;
                const uint64_t row = item[h] / nq;
                const uint32_t col = (uint32_t)(item[h] - row * nq) * 4;
                float x[4] = {acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
                float bv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) bv[c] = (p.flags & T0G_REDUCE_BIAS) ? bias[col + c] : 0.0f;
                apply_epilogue_n<4>(x, bv, epi_of(p));
                const uint64_t o = row * p.ldc + col;
                if constexpr (OUT_BF16) {
                    const u32x2_t w2 = {(uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[0]) |
                                            ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[1]) << 16),
                                        (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[2]) |
                                            ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[3]) << 16)};
                    *reinterpret_cast<__attribute__((address_space(1))) u32x2_t*>((uintptr_t)(p.c + o * 2)) = w2;
                } else {
                    *reinterpret_cast<__attribute__((address_space(1))) f32x4_t*>((uintptr_t)(p.c + o * 4)) =
                        f32x4_t{x[0], x[1], x[2], x[3]};
                }
            }
        }
        return;
    }
    if (p.flags & T0G_REDUCE_VEC) {
        const uint32_t nq = p.n >> 2;
        const uint32_t total = p.m * nq;
        // blockDim.x: 256, or 64 for outputs too small to give every CU a 256-thread block
        for (uint32_t q = blockIdx.x * blockDim.x + threadIdx.x; q < total; q += p.grid_blocks * blockDim.x) {
            const uint32_t row = q / nq, col = (q - row * nq) * 4;
            const uint64_t w = (uint64_t)row * p.ldw + col;
            f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
            for (uint32_t s0 = 0; s0 < p.splits; s0 += 8) {
                f32x4_t v[8];
#pragma unroll
                for (uint32_t u = 0; u < 8; ++u)
                    if (s0 + u < p.splits)
                        v[u] = *reinterpret_cast<const __attribute__((address_space(1))) f32x4_t*>(
                            ws + (s0 + u) * p.plane_elems + w);
#pragma unroll
                for (uint32_t u = 0; u < 8; ++u)
                    if (s0 + u < p.splits) acc = acc + v[u];
            }
            float x[4] = {acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
            for (int c = 0; c < 4; ++c)
                x[c] = apply_epilogue(x[c], (p.flags & T0G_REDUCE_BIAS) ? bias[col + c] : 0.0f, epi_of(p));
            const uint64_t o = (uint64_t)row * p.ldc + col;
            if constexpr (OUT_BF16) {
                typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
                u32x2_t w2;
                w2[0] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[0]) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[1]) << 16);
                w2[1] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[2]) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x[3]) << 16);
                *reinterpret_cast<__attribute__((address_space(1))) u32x2_t*>((uintptr_t)(p.c + o * 2)) = w2;
            } else {
                const f32x4_t y = {x[0], x[1], x[2], x[3]};
                *reinterpret_cast<__attribute__((address_space(1))) f32x4_t*>((uintptr_t)(p.c + o * 4)) = y;
            }
        }
        return;
    }
    const size_t total = (size_t)p.m * p.n;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)p.grid_blocks * 256) {
        const uint32_t row = (uint32_t)(idx / p.n), col = (uint32_t)(idx % p.n);
        const size_t w = (size_t)row * p.ldw + col;
        float acc = 0.0f;
        for (uint32_t s = 0; s < p.splits; ++s) acc = acc + ws[s * p.plane_elems + w];
        acc = apply_epilogue(acc, (p.flags & T0G_REDUCE_BIAS) ? bias[col] : 0.0f, epi_of(p));
        const size_t o = (size_t)row * p.ldc + col;
        if constexpr (OUT_BF16)
            reinterpret_cast<gbf16_t*>((uintptr_t)p.c)[o] = (__bf16)acc;
        else
            reinterpret_cast<gf32_t*>((uintptr_t)p.c)[o] = acc;
    }
}

}  // namespace t0g

// f32 -> bf16 with the rounding of the reference's operand conversion
// (src/ignis/ops/bf16_matmul.rs:372-375): (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16,
// integer arithmetic, no special case for NaN.  HBM-bound: 6 bytes per element.
namespace t0g {
__device__ __forceinline__ uint32_t bf16_bits_ref(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}
}  // namespace t0g

// Vector form: each wave converts 128 items of 4 elements per grid step with
// two 16-byte non-temporal loads per lane, each instruction covering 1 KB of
// consecutive items (whole lines), and two 8-byte stores (512 consecutive bytes
// per instruction).  The host launches one step for every wave up to 2^20
// workgroups.  Measured against 8 elements per lane from 32 contiguous bytes in
// a grid of 8192 workgroups: 64 Mi elements in 58.4 against 66.6 us; a full grid
// of that form took 62.4 us, and more loads in flight per lane were slower.
// Whole waves run without per-lane bounds tests (those cost 61.2 us).
extern "C" __global__ void __launch_bounds__(256) t0g_f32_to_bf16_rne(T0gConvertArgs p) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) f32x4_t gf32x4_t;
    typedef __attribute__((address_space(1))) u32x2_t gu32x2_t;
    if (p.flags & T0G_CONVERT_VEC) {
        const uint64_t n4 = p.n >> 2;   // items of 4 elements
        const uint32_t lane = threadIdx.x & 63u;
        const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const uint64_t step = (uint64_t)p.grid_blocks * 4 * 128;
        gf32x4_t* const s = reinterpret_cast<gf32x4_t*>((uintptr_t)p.src);
        gu32x2_t* const d = reinterpret_cast<gu32x2_t*>((uintptr_t)p.dst);
        auto pack4 = [](f32x4_t v) {
            return u32x2_t{t0g::bf16_bits_ref(v[0]) | (t0g::bf16_bits_ref(v[1]) << 16),
                           t0g::bf16_bits_ref(v[2]) | (t0g::bf16_bits_ref(v[3]) << 16)};
        };
        for (uint64_t wb = ((uint64_t)blockIdx.x * 4 + wave) * 128; wb < n4; wb += step) {
            if (wb + 128 <= n4) {
                const f32x4_t a = __builtin_nontemporal_load(s + wb + lane);
                const f32x4_t b = __builtin_nontemporal_load(s + wb + 64 + lane);
                d[wb + lane] = pack4(a);
                d[wb + 64 + lane] = pack4(b);
            } else {
                const uint64_t i0 = wb + lane, i1 = wb + 64 + lane;
                if (i0 < n4) d[i0] = pack4(__builtin_nontemporal_load(s + i0));
                if (i1 < n4) d[i1] = pack4(__builtin_nontemporal_load(s + i1));
            }
        }
        return;
    }
    const uint64_t stride = (uint64_t)p.grid_blocks * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < p.n; i += stride)
        reinterpret_cast<__attribute__((address_space(1))) uint16_t*>((uintptr_t)p.dst)[i] =
            (uint16_t)t0g::bf16_bits_ref(reinterpret_cast<const __attribute__((address_space(1))) float*>((uintptr_t)p.src)[i]);
}

// ---------------------------------------------------------------------------
// Exported kernel symbols (looked up by name with hipModuleGetFunction).
// t0g_gemm_<BM>x<BN>_k64_<layout>_<out>[_u]   (_u: element-wise loads for
// shapes whose rows are not 16-byte aligned)
// ---------------------------------------------------------------------------
// 128x128 and 64x64 tiles leave room for two or four workgroups per CU (LDS
// 64 KB or less each); they keep a 4-deep ring of BK 32 stages.  (256x256 is
// defined further down.)
#define T0G_WPE_128x128 1, 2
#define T0G_WPE_64x64 1, 4
#define T0G_PIPE_128x128 32, 4
#define T0G_PIPE_64x64 32, 4
#define T0G_GEMM(NAME, BM, BN, WM, WN, AK, BKM, OBF, AL)                                       \
    extern "C" __global__ void __launch_bounds__(64 * WM * WN)                                   \
        __attribute__((amdgpu_waves_per_eu(T0G_WPE_##BM##x##BN))) NAME(T0gGemmArgs p) {          \
        if constexpr (AL)                                                                        \
            t0g::gemm_tile_fast<BM, BN, WM, WN, AK, BKM, OBF, T0G_PIPE_##BM##x##BN>(p);            \
        else                                                                                     \
            t0g::gemm_tile<BM, BN, WM, WN, AK, BKM, OBF, AL>(p);                                 \
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

// Deep-ring variants (suffix _d) of the 64x64 and 128x128 tiles for grids of
// at most one workgroup per CU (split-K and thin shapes): 128 KB of LDS per
// workgroup in stages of 64 K values, so every K-contiguous LDS row is a whole
// 128-byte line and each DMA request fetches full cache lines (half-line
// requests of the 32-K stages left a single workgroup per CU well short of
// the CU's fill rate: 256x256x32768 split 16 went from 17.7 to 15.0 us,
// 1024x4096x11008 on 128x128 tiles from 116 to 83 us).  64x64: 8 stages, 7 in
// flight; 128x128: 4 stages, 3 in flight.
#define T0G_PIPE_D_64x64 64, 8
#define T0G_PIPE_D_128x128 64, 4
#define T0G_GEMM_D(NAME, BM, BN, WM, WN, AK, BKM, OBF)                                                           \
    extern "C" __global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(1, 1)))       \
        NAME(T0gGemmArgs p) {                                                                                  \
        t0g::gemm_tile_fast<BM, BN, WM, WN, AK, BKM, OBF, T0G_PIPE_D_##BM##x##BN>(p);                           \
    }
#define T0G_GEMM_LAYOUTS_D(PFX, BM, BN, WM, WN, OUTN, OBF)                  \
    T0G_GEMM_D(PFX##_nt_##OUTN##_d, BM, BN, WM, WN, true, true, OBF)        \
    T0G_GEMM_D(PFX##_nn_##OUTN##_d, BM, BN, WM, WN, true, false, OBF)       \
    T0G_GEMM_D(PFX##_tn_##OUTN##_d, BM, BN, WM, WN, false, false, OBF)      \
    T0G_GEMM_D(PFX##_tt_##OUTN##_d, BM, BN, WM, WN, false, true, OBF)
#define T0G_GEMM_TILE_D(PFX, BM, BN, WM, WN)                \
    T0G_GEMM_LAYOUTS_D(PFX, BM, BN, WM, WN, f32, false)     \
    T0G_GEMM_LAYOUTS_D(PFX, BM, BN, WM, WN, bf16, true)

// 256x256: the 4-wave kernel (one wave of 128x128 per SIMD) for every layout.
#define T0G_GEMM_256(NAME, AK, BKM, OBF)                                                                  \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))         \
        NAME(T0gGemmArgs p) {                                                                             \
        t0g::gemm_tile_fast16<AK, BKM, OBF>(p);                                                          \
    }
#define T0G_GEMM_LAYOUTS_256(OUTN, OBF)                                 \
    T0G_GEMM_256(t0g_gemm_256x256_k64_nt_##OUTN, true, true, OBF)       \
    T0G_GEMM_256(t0g_gemm_256x256_k64_nn_##OUTN, true, false, OBF)      \
    T0G_GEMM_256(t0g_gemm_256x256_k64_tn_##OUTN, false, false, OBF)     \
    T0G_GEMM_256(t0g_gemm_256x256_k64_tt_##OUTN, false, true, OBF)
T0G_GEMM_LAYOUTS_256(f32, false)
T0G_GEMM_LAYOUTS_256(bf16, true)

// The same kernels for operands of 2^30 elements or more (suffix _x): buffer
// descriptors rebased per tile (K-contiguous operands) or per K stage
// (M/N-contiguous), 64-bit byte counts.
#define T0G_GEMM_256_X(NAME, AK, BKM, OBF)                                                                \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))         \
        NAME(T0gGemmArgs p) {                                                                             \
        t0g::gemm_tile_fast16<AK, BKM, OBF, true>(p);                                                    \
    }
#define T0G_GEMM_LAYOUTS_256_X(OUTN, OBF)                                   \
    T0G_GEMM_256_X(t0g_gemm_256x256_k64_nt_##OUTN##_x, true, true, OBF)     \
    T0G_GEMM_256_X(t0g_gemm_256x256_k64_nn_##OUTN##_x, true, false, OBF)    \
    T0G_GEMM_256_X(t0g_gemm_256x256_k64_tn_##OUTN##_x, false, false, OBF)   \
    T0G_GEMM_256_X(t0g_gemm_256x256_k64_tt_##OUTN##_x, false, true, OBF)
T0G_GEMM_LAYOUTS_256_X(f32, false)
T0G_GEMM_LAYOUTS_256_X(bf16, true)

// The same tiles on a stream-K schedule (suffix _sk, T0gGemmSkArgs).
#define T0G_GEMM_256_SK(NAME, AK, BKM, OBF)                                                               \
    extern "C" __global__ void __launch_bounds__(AK ? 512 : 256)                                         \
        __attribute__((amdgpu_waves_per_eu(AK ? 2 : 1, AK ? 2 : 1))) NAME(T0gGemmSkArgs s) {              \
        t0g::gemm_tile_sk<AK, BKM, OBF>(s);                                                              \
    }
#define T0G_GEMM_LAYOUTS_256_SK(OUTN, OBF)                                   \
    T0G_GEMM_256_SK(t0g_gemm_256x256_k64_nt_##OUTN##_sk, true, true, OBF)    \
    T0G_GEMM_256_SK(t0g_gemm_256x256_k64_nn_##OUTN##_sk, true, false, OBF)   \
    T0G_GEMM_256_SK(t0g_gemm_256x256_k64_tn_##OUTN##_sk, false, false, OBF)  \
    T0G_GEMM_256_SK(t0g_gemm_256x256_k64_tt_##OUTN##_sk, false, true, OBF)
T0G_GEMM_LAYOUTS_256_SK(f32, false)
T0G_GEMM_LAYOUTS_256_SK(bf16, true)
T0G_GEMM_TILE(t0g_gemm_128x128_k64, 128, 128, 2, 2)

// Split-K reduced inside the kernel (suffix _r, T0gGemmRedArgs): 128x128 and
// 256x256 tiles, every layout, f32 or bf16 out.
#define T0G_GEMM_R(NAME, BM, BN, WM, WN, AK, BKM, OBF)                                                   \
    extern "C" __global__ void __launch_bounds__(64 * WM * WN)                                           \
        __attribute__((amdgpu_waves_per_eu(T0G_WPE_##BM##x##BN))) NAME(T0gGemmRedArgs ra) {              \
        t0g::gemm_tile_fast<BM, BN, WM, WN, AK, BKM, OBF, T0G_PIPE_##BM##x##BN, true>(ra.g, &ra);       \
    }
#define T0G_GEMM_LAYOUTS_R(PFX, BM, BN, WM, WN, OUTN, OBF)                 \
    T0G_GEMM_R(PFX##_nt_##OUTN##_r, BM, BN, WM, WN, true, true, OBF)       \
    T0G_GEMM_R(PFX##_nn_##OUTN##_r, BM, BN, WM, WN, true, false, OBF)      \
    T0G_GEMM_R(PFX##_tn_##OUTN##_r, BM, BN, WM, WN, false, false, OBF)     \
    T0G_GEMM_R(PFX##_tt_##OUTN##_r, BM, BN, WM, WN, false, true, OBF)
T0G_GEMM_LAYOUTS_R(t0g_gemm_128x128_k64, 128, 128, 2, 2, f32, false)
T0G_GEMM_LAYOUTS_R(t0g_gemm_128x128_k64, 128, 128, 2, 2, bf16, true)
#define T0G_GEMM_256_R(NAME, AK, BKM, OBF)                                                                \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))         \
        NAME(T0gGemmRedArgs ra) {                                                                         \
        t0g::gemm_tile_fast16<AK, BKM, OBF, false, true>(ra.g, &ra);                                     \
    }
#define T0G_GEMM_LAYOUTS_256_R(OUTN, OBF)                                   \
    T0G_GEMM_256_R(t0g_gemm_256x256_k64_nt_##OUTN##_r, true, true, OBF)     \
    T0G_GEMM_256_R(t0g_gemm_256x256_k64_nn_##OUTN##_r, true, false, OBF)    \
    T0G_GEMM_256_R(t0g_gemm_256x256_k64_tn_##OUTN##_r, false, false, OBF)   \
    T0G_GEMM_256_R(t0g_gemm_256x256_k64_tt_##OUTN##_r, false, true, OBF)
T0G_GEMM_LAYOUTS_256_R(f32, false)
T0G_GEMM_LAYOUTS_256_R(bf16, true)
T0G_GEMM_TILE(t0g_gemm_64x64_k64, 64, 64, 2, 2)
T0G_GEMM_TILE_U(t0g_gemm_128x128_k64, 128, 128, 2, 2)
T0G_GEMM_TILE_U(t0g_gemm_64x64_k64, 64, 64, 2, 2)
T0G_GEMM_TILE_D(t0g_gemm_64x64_k64, 64, 64, 2, 2)
T0G_GEMM_TILE_D(t0g_gemm_128x128_k64, 128, 128, 2, 2)

// The 64x64 deep ring with K split across the four waves (suffix _ds): each
// wave multiplies the whole tile for one 16-wide K step of every stage, and the
// four partial tiles are summed through LDS after the loop.  For K ranges of
// 24 stages or more (the host's choice; the sum does not pay for shorter ones).
#define T0G_GEMM_DS(NAME, AK, BKM, OBF)                                                                       \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))             \
        NAME(T0gGemmArgs p) {                                                                                 \
        t0g::gemm_tile_fast<64, 64, 2, 2, AK, BKM, OBF, T0G_PIPE_D_64x64, false, true>(p);                    \
    }
#define T0G_GEMM_LAYOUTS_DS(OUTN, OBF)                                       \
    T0G_GEMM_DS(t0g_gemm_64x64_k64_nt_##OUTN##_ds, true, true, OBF)          \
    T0G_GEMM_DS(t0g_gemm_64x64_k64_nn_##OUTN##_ds, true, false, OBF)         \
    T0G_GEMM_DS(t0g_gemm_64x64_k64_tn_##OUTN##_ds, false, false, OBF)        \
    T0G_GEMM_DS(t0g_gemm_64x64_k64_tt_##OUTN##_ds, false, true, OBF)
T0G_GEMM_LAYOUTS_DS(f32, false)
T0G_GEMM_LAYOUTS_DS(bf16, true)

// Deep-ring kernels with the split-K reduced inside the kernel (suffix _dr).
#define T0G_GEMM_DR(NAME, BM, BN, WM, WN, AK, BKM, OBF)                                                          \
    extern "C" __global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(1, 1)))       \
        NAME(T0gGemmRedArgs ra) {                                                                              \
        t0g::gemm_tile_fast<BM, BN, WM, WN, AK, BKM, OBF, T0G_PIPE_D_##BM##x##BN, true>(ra.g, &ra);             \
    }
#define T0G_GEMM_LAYOUTS_DR(PFX, BM, BN, WM, WN, OUTN, OBF)                  \
    T0G_GEMM_DR(PFX##_nt_##OUTN##_dr, BM, BN, WM, WN, true, true, OBF)       \
    T0G_GEMM_DR(PFX##_nn_##OUTN##_dr, BM, BN, WM, WN, true, false, OBF)      \
    T0G_GEMM_DR(PFX##_tn_##OUTN##_dr, BM, BN, WM, WN, false, false, OBF)     \
    T0G_GEMM_DR(PFX##_tt_##OUTN##_dr, BM, BN, WM, WN, false, true, OBF)
#define T0G_GEMM_TILE_DR(PFX, BM, BN, WM, WN)                \
    T0G_GEMM_LAYOUTS_DR(PFX, BM, BN, WM, WN, f32, false)     \
    T0G_GEMM_LAYOUTS_DR(PFX, BM, BN, WM, WN, bf16, true)
T0G_GEMM_TILE_DR(t0g_gemm_64x64_k64, 64, 64, 2, 2)
T0G_GEMM_TILE_DR(t0g_gemm_128x128_k64, 128, 128, 2, 2)

// _ds with the split-K reduced inside the kernel (suffix _dsr).
#define T0G_GEMM_DSR(NAME, AK, BKM, OBF)                                                                      \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))             \
        NAME(T0gGemmRedArgs ra) {                                                                             \
        t0g::gemm_tile_fast<64, 64, 2, 2, AK, BKM, OBF, T0G_PIPE_D_64x64, true, true>(ra.g, &ra);             \
    }
#define T0G_GEMM_LAYOUTS_DSR(OUTN, OBF)                                      \
    T0G_GEMM_DSR(t0g_gemm_64x64_k64_nt_##OUTN##_dsr, true, true, OBF)        \
    T0G_GEMM_DSR(t0g_gemm_64x64_k64_nn_##OUTN##_dsr, true, false, OBF)       \
    T0G_GEMM_DSR(t0g_gemm_64x64_k64_tn_##OUTN##_dsr, false, false, OBF)      \
    T0G_GEMM_DSR(t0g_gemm_64x64_k64_tt_##OUTN##_dsr, false, true, OBF)
T0G_GEMM_LAYOUTS_DSR(f32, false)
T0G_GEMM_LAYOUTS_DSR(bf16, true)

extern "C" __global__ void __launch_bounds__(256) t0g_splitk_reduce_f32(T0gReduceArgs p) {
    t0g::splitk_reduce<false>(p);
}
extern "C" __global__ void __launch_bounds__(256) t0g_splitk_reduce_bf16(T0gReduceArgs p) {
    t0g::splitk_reduce<true>(p);
}
