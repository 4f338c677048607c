// 16x16x32 MFMA variant of the fast path, used for the 256x256 tile.
//
// Included by gemm_gfx950.hip after its DMA, swizzle and epilogue helpers.
// Same tiling as the 32x32x16 path (4 waves of 128x128, two 64 KB stages of
// 64 K values streamed into LDS by DMA), but each wave issues 64
// v_mfma_f32_16x16x32_bf16 per 32-wide K step on 8 x 8 sub-tiles of 16x16.
// At MI355X's board power limit the 16x16x32 form sustains a higher shader
// clock for the same FLOP rate per clock (it moves a quarter of the
// accumulator registers per instruction), so the GEMM gets more FLOP/s.
//
// MFMA operand layout (16x16x32 bf16): lane l holds A[l % 16][8*(l/16) .. +7]
// and B[8*(l/16) .. +7][l % 16]; the result lane l holds D[4*(l/16) + r][l % 16],
// r = 0..3.
#ifndef T0G_GEMM_MFMA16_H
#define T0G_GEMM_MFMA16_H

#include <type_traits>

namespace t0g {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// M/N-contiguous granule swizzle for the 16-wide fragments: {0,2,5,7}[k % 4]
// flipped by bit 3 of k, so the two 16-lane groups of a ds_read_b64_tr_b16
// half-wave (k rows 8 apart, same 16 columns) use the other 4 granules of the
// 256-byte bank window.
__device__ __forceinline__ uint32_t fm16(uint32_t k, uint32_t granules) {
    return (((0x7520u >> ((k & 3u) * 4)) & 0xFu) ^ ((k >> 3) & 1u)) & (granules - 1);
}

// WIDE: operands of any size (buffer descriptors rebased per tile or stage and
// cut to 2 GiB, 64-bit byte counts); otherwise operands below 2^30 elements,
// addressed from the operand base with 32-bit byte counts.
template <bool K_MAJOR, int ROWS, int NT, int SUBS, bool WIDE = false>
struct Op16;

// K-contiguous operand of a 256-row tile, 64 K values per stage: 128-byte LDS
// rows, chunk swizzle fk<64>.  A stage is 32 pieces of 1 KB, piece q = rows
// 8q .. 8q+7 at LDS offset q KB.  Whole stages: wave w issues pieces
// w kInstr + i, in groups of four consecutive pieces sharing one M0 write
// (dma_m0); the lanes' byte offsets, less the requests' immediate offsets, are
// kept in registers (the stage's K position is in the descriptor's base).
// Stages with a K tail (CHECK): wave w issues pieces i W + w, one M0 write
// each; for even W, fk<64> of those rows does not depend on i, so one K column
// serves all of a wave's instructions.
template <int ROWS, int NT, int SUBS, bool WIDE>
struct Op16<true, ROWS, NT, SUBS, WIDE> {
    typedef typename std::conditional<WIDE, uint64_t, uint32_t>::type bytes_t;
    static constexpr int kWaves = NT / 64;
    static constexpr uint32_t kKRow = 128;
    static constexpr int kInstr = ROWS * kKRow / 1024 / kWaves;
    static_assert(ROWS == 256 && (kWaves == 4 || kWaves == 8), "offset sharing assumes a 256-row tile, 4 or 8 waves");
    static constexpr uint32_t kStageBytes = ROWS * kKRow;
    uint64_t rowb;    // WIDE: byte offset of the tile's first row in the operand
    uint32_t off0;    // byte offset of instruction 0's piece at k = 0 (WIDE: from the tile's first row)
    uint32_t kcol;    // first K column of the lane's piece
    uint32_t step;    // bytes between instructions (8 W rows)
    uint32_t wave;
    uint32_t frag[2];   // per 32-wide K step: LDS offset of the lane's chunk in sub-tile 0
    // whole stages: byte offset of piece wave * kInstr + i, less (i % 4) KB (the
    // request's immediate offset).  Not negative: the piece's rows start at
    // 8 i, i.e. 16 i ld >= 1 KB * i bytes in, since ld >= K >= 64 here.
    uint32_t offs[kInstr];

    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t ld, uint32_t wrow) {
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t lane = tid & 63u;
        const uint32_t r = 8 * wave + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ fk<64>(r);
        kcol = c * 8;
        if constexpr (WIDE) {
            rowb = (uint64_t)row0 * ld * 2;
            off0 = (r * ld + c * 8) * 2;
        } else {
            rowb = 0;
            off0 = ((row0 + r) * ld + c * 8) * 2;
        }
        step = 16 * kWaves * ld;
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            const uint32_t rq = 8 * (wave * kInstr + i) + (lane >> 3);
            const uint32_t cq = (lane & 7u) ^ fk<64>(rq);
            const uint32_t o = WIDE ? (rq * ld + cq * 8) * 2 : ((row0 + rq) * ld + cq * 8) * 2;
            offs[i] = o - (uint32_t)(i & 3) * 1024u;
        }
        const uint32_t row = wrow + (lane & 15u), qk = lane >> 4;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) frag[kk] = row * kKRow + (((4u * kk + qk) ^ fk<64>(row)) << 4);
    }
    __device__ __forceinline__ u32x4_t rsrc(uint64_t base, bytes_t bytes, uint32_t, uint32_t k0) const {
        if constexpr (WIDE)
            return rsrc_words_wide(base + rowb, bytes > rowb ? bytes - rowb : 0u, (uint64_t)k0 * 2);
        else
            return rsrc_words32(base, bytes, k0 * 2);
    }
    // Requests of a stage go out in ascending i (the group's M0 is written at i % 4 == 0).
    template <bool CHECK>
    __device__ __forceinline__ void issue_one(int i, u32x4_t r, uint32_t lds, uint32_t k0, uint32_t kend) const {
        if (CHECK) {
            dma16(r, k0 + kcol < kend ? off0 + i * step : kOob, lds + (i * kWaves + wave) * 1024);
        } else {
            if ((i & 3) == 0) dma_m0(lds, (wave * kInstr + i) * 1024);
            dma16_slot(r, offs[i], i & 3);
        }
    }
    template <bool CHECK>
    __device__ __forceinline__ void issue(uint32_t lds, uint64_t base, bytes_t bytes, uint32_t ld, uint32_t k0,
                                          uint32_t kend) const {
        const u32x4_t r = rsrc(base, bytes, ld, k0);
#pragma unroll
        for (int i = 0; i < kInstr; ++i) issue_one<CHECK>(i, r, lds, k0, kend);
    }
    // Fragment of 16-row sub-tile `sub` for 32-wide K step KK.
    // The sub-tile offset is pointer arithmetic on an LDS pointer, so the
    // compiler folds it into the instruction's offset field instead of adding
    // it with VALU instructions.
    template <int KK>
    __device__ __forceinline__ bf16x8_t read_one(uint32_t stage, int sub) const {
        const __attribute__((address_space(3))) bf16x8_t* base =
            reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>((uintptr_t)(stage + frag[KK]));
        return base[sub * kKRow];   // sub * 16 rows of kKRow bytes, in 16-byte units
    }
};

// M/N-contiguous operand of a 256-column tile: LDS rows are k rows of 512
// bytes, granule swizzle fm16.  A stage is 32 pieces of 1 KB, piece q = k rows
// 2q, 2q+1 at LDS offset q KB.  Whole stages: wave w issues pieces
// w kInstr + i in groups of four sharing one M0 write, from byte offsets kept
// in registers less the requests' immediate offsets (not negative for
// ld >= 256: the piece starts 2 i k rows in; the host keeps smaller leading
// dimensions off these kernels).  Stages with a K tail (CHECK): wave w issues
// pieces i W + w, one M0 write each; their swizzle depends on i only through
// bit 0 of i (W = 4) or not at all (W = 8), so every instruction's byte offset
// is one of two bases plus i steps.
template <int ROWS, int NT, int SUBS, bool WIDE>
struct Op16<false, ROWS, NT, SUBS, WIDE> {
    typedef typename std::conditional<WIDE, uint64_t, uint32_t>::type bytes_t;
    static constexpr int kWaves = NT / 64;
    static constexpr uint32_t kRowB = ROWS * 2;
    static constexpr uint32_t kGranules = ROWS / 16;
    static constexpr uint32_t kStageBytes = 64 * kRowB;
    static constexpr int kInstr = kStageBytes / 1024 / kWaves;
    static_assert(ROWS == 256 && (kWaves == 4 || kWaves == 8), "offset sharing assumes a 256-column tile, 4 or 8 waves");
    static_assert(SUBS == 4 || SUBS == 8, "sub-tile granules are XORed into a 4- or 8-aligned base");
    uint32_t off[2];   // byte offsets of instructions 0 and 1 (less one instruction step) at k = 0
    uint32_t krow;     // k row of instruction 0's piece
    uint32_t step;     // bytes between instructions (2 W k rows)
    uint32_t wave;
    uint32_t frag0;    // K step 0, half 0, sub-tile 0; sub-tile s is frag0 ^ (s << 5)
    uint32_t offs[kInstr];   // whole stages: piece wave * kInstr + i, less (i % 4) KB

    __device__ __forceinline__ void init(uint32_t tid, uint32_t row0, uint32_t ld, uint32_t wrow) {
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t lane = tid & 63u;
        const uint32_t k = 2 * wave + (lane >> 5), slot = lane & 31u;
        krow = k;
        step = 4 * kWaves * ld;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t lg = (slot >> 1) ^ fm16(k + 2 * kWaves * i, kGranules);
            off[i] = (k * ld + row0 + lg * 16 + (slot & 1) * 8) * 2;
        }
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            const uint32_t kq = 2 * (wave * kInstr + i) + (lane >> 5);
            const uint32_t lg = (slot >> 1) ^ fm16(kq, kGranules);
            offs[i] = (kq * ld + row0 + lg * 16 + (slot & 1) * 8) * 2 - (uint32_t)(i & 3) * 1024u;
        }
        // ds_read_b64_tr_b16: 16-lane group q reads k rows 32*kk + 8q + 4h + r
        // (lane 4r + c: columns 4c .. 4c+3 of the 16-column sub-tile); lane i
        // of the group receives column i.  fm16 sees only k % 4 and bit 3 of k.
        // Sub-tile granule (wrow / 16 + s) ^ f, with wrow / 16 a multiple of
        // SUBS and s < SUBS, equals (wrow / 16 ^ f) ^ s: an XOR of bits 5 and up.
        const uint32_t q = lane >> 4, r = (lane >> 2) & 3u, c = lane & 3u;
        const uint32_t k0 = 8 * q + r, f = fm16(k0, kGranules);
        frag0 = k0 * kRowB + c * 8 + (((wrow >> 4) ^ f) << 5);
    }
    __device__ __forceinline__ u32x4_t rsrc(uint64_t base, bytes_t bytes, uint32_t ld, uint32_t k0) const {
        if constexpr (WIDE)
            return rsrc_words_wide(base, bytes, (uint64_t)k0 * ld * 2);
        else
            return rsrc_words32(base, bytes, k0 * ld * 2);
    }
    // Requests of a stage go out in ascending i (the group's M0 is written at i % 4 == 0).
    template <bool CHECK>
    __device__ __forceinline__ void issue_one(int i, u32x4_t r, uint32_t lds, uint32_t k0, uint32_t kend) const {
        if (CHECK) {
            dma16(r, k0 + krow + 2 * kWaves * i < kend ? off[i & 1] + i * step : kOob,
                  lds + (i * kWaves + wave) * 1024);
        } else {
            if ((i & 3) == 0) dma_m0(lds, (wave * kInstr + i) * 1024);
            dma16_slot(r, offs[i], i & 3);
        }
    }
    template <bool CHECK>
    __device__ __forceinline__ void issue(uint32_t lds, uint64_t base, bytes_t bytes, uint32_t ld, uint32_t k0,
                                          uint32_t kend) const {
        const u32x4_t r = rsrc(base, bytes, ld, k0);
#pragma unroll
        for (int i = 0; i < kInstr; ++i) issue_one<CHECK>(i, r, lds, k0, kend);
    }
    // The stage base is a multiple of 1 KB and the XOR touches bits 5..8 only, so
    // (stage + frag0) ^ (sub << 5) = stage + (frag0 ^ (sub << 5)) addresses
    // sub-tile `sub` of that stage; the K step's row offsets are pointer
    // arithmetic, folded into the instructions' offset fields.
    template <int KK>
    __device__ __forceinline__ bf16x8_t read_one(uint32_t stage, int sub) const {
        constexpr int O0 = KK * 32 * kRowB, O1 = (KK * 32 + 4) * kRowB;
        typedef short v4s __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4s lds_v4s;
        const __attribute__((address_space(3))) char* a = reinterpret_cast<const __attribute__((address_space(3))) char*>(
            (uintptr_t)(stage + (frag0 ^ ((uint32_t)sub << 5))));
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(a + O0));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(a + O1));
        typedef short v8s __attribute__((ext_vector_type(8)));
        const v8s w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(bf16x8_t, w);
    }
};

// v_mfma_f32_16x16x32_bf16 with the accumulator pinned to AGPRs.  Written as
// asm because the compiler's register allocation of 64 live 16x16 accumulators
// moves them between VGPRs and AGPRs on every K step.  The compiler does not
// see an MFMA here, so its wait-state bookkeeping for MFMA results does not
// apply: the accumulators are only read back by VALU after mfma16_drain().
__device__ __forceinline__ void mfma16(f32x4_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Wait states between the last MFMA writing an accumulator and VALU reads of
// it (8-pass XDL result to VALU read: at most 19), and between VALU writes of
// accumulators and their first use as MFMA source C.  The scheduling barrier
// keeps the compiler from moving accumulator reads or writes across it.  The
// accumulators must also never live in scratch: a spill store right after an
// asm MFMA would read its result too early (the Makefile rejects a build in
// which these kernels use scratch).
__device__ __forceinline__ void mfma16_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// One 32-wide K step, rows [RB, RE) of SM sub-tile rows, SN MFMAs per row.
// Next-step fragment reads go to rows [RR, RE): with all rows, A[r] in row r
// and B two per row; otherwise all reads spread evenly, B first.  DMA
// instructions [DFIRST, DFIRST + DCOUNT) are spread over the call's rows.
template <int STEP, int DFIRST, int DCOUNT, bool CHECK, int RB, int RE, int RR, int SM, int SN, class OpA, class OpB>
__device__ __forceinline__ void mfma16_rows(f32x4_t (&acc)[SM][SN], const bf16x8_t (&fa)[SM], const bf16x8_t (&fb)[SN],
                                            bf16x8_t (&na)[SM], bf16x8_t (&nb)[SN], const OpA& la, const OpB& lb,
                                            uint32_t cur, uint32_t nxt, uint32_t fill, u32x4_t ra, u32x4_t rb,
                                            uint32_t kf, uint32_t kend) {
    constexpr int NEXT_KK = (STEP + 1) % 2;
    const uint32_t rd = STEP == 0 ? cur : nxt;
    constexpr int kRows = RE - RB;
    constexpr int kPerRow = (DCOUNT + kRows - 1) / kRows;
    constexpr int kReadRows = RE - RR;
    constexpr bool kOwn = kReadRows == SM;   // every row reads: A[r] in row r
    constexpr int kReads = SM + SN;
    constexpr int kSpread = kReadRows > 0 ? (kReads + kReadRows - 1) / kReadRows : 0;
#pragma unroll
    for (int i = RB; i < RE; ++i) {
        int nbr = 0, nar = 0, bfirst = 0, qfirst = 0;
        if (i >= RR) {
            if (kOwn) {
                bfirst = 2 * (i - RR);
                const int blast = i == RE - 1 ? SN : bfirst + 2;
                nbr = (blast < SN ? blast : SN) - (bfirst < SN ? bfirst : SN);
                nar = 1;
            } else {
                qfirst = (i - RR) * kSpread;
                const int qlast = qfirst + kSpread < kReads ? qfirst + kSpread : kReads;
                nbr = qlast > qfirst ? qlast - qfirst : 0;   // reads q in [qfirst, qlast): B for q < SN, then A
            }
        }
        const int nr = nbr + nar;
        const int nitems = kPerRow + nr;
        const int per_slot = (nitems + SN - 1) / SN;
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            mfma16(acc[i][j], fa[i], fb[j]);
#pragma unroll
            for (int u = 0; u < per_slot; ++u) {
                const int t = j * per_slot + u;
                if (t < nitems) {
                    const int it = row_item(t, kPerRow, nr);
                    if (it >= 256) {
                        const int rq = it - 256;
                        if (kOwn) {
                            if (rq < nbr)
                                nb[bfirst + rq] = lb.template read_one<NEXT_KK>(rd + OpA::kStageBytes, bfirst + rq);
                            else
                                na[i] = la.template read_one<NEXT_KK>(rd, i);
                        } else {
                            const int q = qfirst + rq;
                            if (q < SN)
                                nb[q] = lb.template read_one<NEXT_KK>(rd + OpA::kStageBytes, q);
                            else
                                na[q - SN] = la.template read_one<NEXT_KK>(rd, q - SN);
                        }
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

// K loop: two 64 KB stages of 64 K values (two 32-wide steps each).  Halfway
// through step 1 of stage s one vmcnt(0)/lgkmcnt(0) wait and a barrier make
// stage s + 1 visible and free the buffer of stage s; the step's second half
// reads stage s + 1's first fragments and starts the DMA of stage s + 2 into
// the freed buffer (the A half), whose B half follows during step 0 of stage
// s + 1.  Each DMA so has half a stage or more to land before it is waited on.
// Stages past the end get an empty descriptor: their DMA writes zeros to LDS
// and reads no memory.
template <bool CHECK, uint32_t A_BYTES, uint32_t STAGE, int kVmemPerStage, int SM, int SN, class OpA, class OpB>
__device__ __forceinline__ void k_pipeline16(f32x4_t (&acc)[SM][SN], const OpA& la, const OpB& lb,
                                             const T0gGemmArgs& p, typename OpA::bytes_t a_bytes,
                                             typename OpB::bytes_t b_bytes, uint32_t kbeg,
                                             uint32_t kend, int nst, uint32_t lds0) {
    constexpr int kHalf = OpA::kInstr;   // the A half of a stage's DMA, then the B half
    static_assert(OpA::kInstr == OpB::kInstr, "equal A and B halves");
    bf16x8_t fa0[SM], fb0[SN], fa1[SM], fb1[SN];
    la.template issue<CHECK>(lds0, p.a, a_bytes, p.lda, kbeg, kend);
    lb.template issue<CHECK>(lds0 + A_BYTES, p.b, b_bytes, p.ldb, kbeg, kend);
    {
        const uint32_t k1 = kbeg + 64;
        la.template issue<CHECK>(lds0 + STAGE, p.a, k1 < kend ? a_bytes : typename OpA::bytes_t{0}, p.lda, k1, kend);
    }
    T0G_WAIT_VMCNT(kHalf);
    barrier_no_fence();
#pragma unroll
    for (int i = 0; i < SM; ++i) fa0[i] = la.template read_one<0>(lds0, i);
#pragma unroll
    for (int j = 0; j < SN; ++j) fb0[j] = lb.template read_one<0>(lds0 + A_BYTES, j);

    constexpr int kHalfRows = SM / 2;
    uint32_t cur = 0;
    for (int s = 0; s < nst; ++s) {
        const uint32_t nxt = cur ^ STAGE;
        const uint32_t k1 = kbeg + (uint32_t)(s + 1) * 64, k2 = k1 + 64;
        const u32x4_t rb1 = lb.rsrc(p.b, k1 < kend ? b_bytes : typename OpB::bytes_t{0}, p.ldb, k1);
        const u32x4_t ra2 = la.rsrc(p.a, k2 < kend ? a_bytes : typename OpA::bytes_t{0}, p.lda, k2);
        mfma16_rows<0, kHalf, kHalf, CHECK, 0, SM, 0>(acc, fa0, fb0, fa1, fb1, la, lb, lds0 + cur, lds0 + nxt,
                                                     lds0 + nxt, ra2, rb1, k1, kend);
        mfma16_rows<1, 0, 0, CHECK, 0, kHalfRows, kHalfRows>(acc, fa1, fb1, fa0, fb0, la, lb, lds0 + cur, lds0 + nxt,
                                                            lds0 + nxt, ra2, rb1, k1, kend);
        __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0)
        barrier_no_fence();
        mfma16_rows<1, 0, kHalf, CHECK, kHalfRows, SM, kHalfRows>(acc, fa1, fb1, fa0, fb0, la, lb, lds0 + cur,
                                                                 lds0 + nxt, lds0 + cur, ra2, rb1, k2, kend);
        cur = nxt;
    }
}

// Epilogue: each wave stages 32 rows x WTN columns of fp32 at a time through
// its own LDS region, rows padded to WTN + 4 words (the 16x16 result puts the
// four lane groups 4 rows apart; a 4-row step of 132 words moves 16 banks), and
// writes whole rows with 16-byte stores.
template <int SN>
struct VecEpilogue16 {
    static constexpr int kWTN = SN * 16;
    static constexpr uint32_t kStride = (kWTN + 4) * 4;
    static constexpr uint32_t kWaveBytes = 32 * kStride;
};

// Partial tiles that other workgroups left for this one (stream-K): `count`
// slots from `first`, summed in slot order onto the workgroup's own
// accumulators.  A slot holds a whole 256 x 256 f32 tile in accumulator order:
// sub-tile (i, j) of wave v is 1 KB at ((v * SM + i) * SN + j) KB, 16 bytes per
// lane; `frag` is this lane's offset of sub-tile (0, 0).
struct SkFixup {
    uint64_t base;
    uint32_t first, count;
    uint32_t frag;
};

// bf16 epilogue of a wave's SM x SN sub-tiles of a tile wholly inside an aligned
// C, converted in registers and staged as bf16.  The chain and the RNE
// conversion run on the MFMA result layout (lane (q, c) of sub-tile (i, j)
// holds rows 4q .. 4q+3 of column 16 j + c, one bias value per lane and j).
// Each 16-row band of the wave's tile then goes through LDS column-major, 32
// bytes (16 rows, four 8-byte pieces) per column: one ds_write_b64 per lane and
// sub-tile puts the lane's 4 rows in place.  ds_read_b64_tr_b16 hands lane i of
// a 16-lane group element i % 4 of the pieces that lanes 4 r + i / 4 (r =
// 0..3) of the group address; with lane 4 r + s of group g addressing column
// 16 g + 8 (s & 1) + r (+ 4 in the second read) and piece 2 p + (s >> 1), lane
// i = 4 s + e receives row 8 p + 4 (s >> 1) + e, columns 16 g + 8 (s & 1) ..
// + 7 (16 bytes), and one store instruction writes 8 rows x 64 columns: whole
// 128-byte lines.  Column col is placed at col ^ 4 in odd 8-column blocks and
// its pieces XORed with 2 when bit 3 and bit 4 of col differ, which puts the
// 32 lanes of every half-wave access -- writes: 16 columns x 2 pieces; reads:
// two groups of 8 columns x 2 pieces -- on distinct banks.  Against staging
// fp32 rows this halves the LDS bytes and takes a quarter of the LDS write
// instructions.  Two bands alternate between two regions, so a band's writes
// never wait for the previous band's reads.  `lds`: 2 * SN * 512 bytes of this
// wave's own.
__device__ __forceinline__ uint32_t bf16_stage_off(uint32_t col, uint32_t piece) {
    const uint32_t b3 = (col >> 3) & 1u, b4 = (col >> 4) & 1u;
    return (col ^ (b3 << 2)) * 32u + (piece ^ ((b3 ^ b4) << 1)) * 8u;
}

// One accumulator read out of its AGPR at this point of the program.  The
// register allocator otherwise copies every accumulator a VALU instruction
// uses into VGPRs right after the K loop -- all 128 (or 256) of them at once,
// more than the VGPRs left -- and spills.
__device__ __forceinline__ float acc_read(float a) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
    return v;
}

template <int SM, int SN>
__device__ __forceinline__ void store_tile_bf16_tr(const T0gGemmArgs& p, const f32x4_t (&acc)[SM][SN], uint32_t row0,
                                                   uint32_t col0, uint32_t lane, uint32_t lds) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) u32x2_t lds_u32x2;
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    static_assert(SN % 4 == 0, "the wave tile's columns come in blocks of 64");
    constexpr uint32_t kRegion = SN * 16 * 32;   // one band: 16 rows x 16 SN columns of bf16
    // The lane index through an opaque move: every address and bias value below
    // derives from it, so none of them is hoisted above the K loop's (volatile)
    // MFMAs and held in registers across it.
    asm volatile("v_mov_b32 %0, %0" : "+v"(lane));
    const uint32_t l16 = lane & 15u, q = lane >> 4;
    const EpiParams ep = epi_of(p);
    float bv[SN];
#pragma unroll
    for (int j = 0; j < SN; ++j)
        bv[j] = (p.flags & T0G_FLAG_BIAS)
                    ? reinterpret_cast<const __attribute__((address_space(1))) float*>(p.bias)[col0 + j * 16 + l16]
                    : 0.0f;
    // read side: lane 16 g + 4 r + s
    const uint32_t g = lane >> 4, r = (lane >> 2) & 3u, s = lane & 3u, e = lane & 3u;
    const uint32_t rcol = 16u * g + 8u * (s & 1u) + r, rpc = s >> 1;
    // the lane's own row and columns in the band after the two reads of pair pp
    const uint32_t srow = 4u * ((l16 >> 2) >> 1) + e, scol = 16u * g + 8u * ((l16 >> 2) & 1u);
    const uint64_t cb = p.c + ((uint64_t)(row0 + srow) * p.ldc + col0 + scol) * 2u;
#pragma unroll
    for (int i = 0; i < SM; ++i) {
        // one band at a time
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t reg = lds + (uint32_t)(i & 1) * kRegion;
        // the band's SN x 4 values through the chain at once (the chain is decoded
        // once per band)
        float v[SN * 4], b4[SN * 4];
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[4 * j + r] = acc_read(acc[i][j][r]);
                b4[4 * j + r] = bv[j];
            }
        apply_epilogue_n<SN * 4>(v, b4, ep);
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            u32x2_t w;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                w[h] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[4 * j + 2 * h]) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[4 * j + 2 * h + 1]) << 16);
            *reinterpret_cast<lds_u32x2*>((uintptr_t)(reg + bf16_stage_off(16u * j + l16, q))) = w;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int u = 0; u < SN / 4; ++u)
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                const uint32_t c0 = 64u * u + rcol, piece = 2u * pp + rpc;
                const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_v4s*)(uintptr_t)(reg + bf16_stage_off(c0, piece)));
                const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_v4s*)(uintptr_t)(reg + bf16_stage_off(c0 + 4u, piece)));
                u32x4_t w;
                w[0] = __builtin_bit_cast(uint32_t, __builtin_shufflevector(lo, lo, 0, 1));
                w[1] = __builtin_bit_cast(uint32_t, __builtin_shufflevector(lo, lo, 2, 3));
                w[2] = __builtin_bit_cast(uint32_t, __builtin_shufflevector(hi, hi, 0, 1));
                w[3] = __builtin_bit_cast(uint32_t, __builtin_shufflevector(hi, hi, 2, 3));
                const uint64_t addr = cb + ((uint64_t)(16u * i + 8u * pp) * p.ldc + 64u * u) * 2u;
                __builtin_nontemporal_store(
                    w, reinterpret_cast<__attribute__((address_space(1))) u32x4_t*>((uintptr_t)addr));
            }
    }
}

// WT: 16-byte stores write through to memory (sc0 sc1), as in store_tile_vec.
template <int SM, int SN, bool OUT_BF16, bool FIXUP = false, bool WT = false>
__device__ __forceinline__ void store_tile_vec16(const T0gGemmArgs& p, const f32x4_t (&acc)[SM][SN], uint32_t row0,
                                                 uint32_t col0, uint32_t lane, uint32_t lds, bool vec,
                                                 SkFixup fx = SkFixup{0, 0, 0, 0}) {
    if constexpr (OUT_BF16 && !FIXUP && !WT) {
        static_assert(2 * SN * 512 <= VecEpilogue16<SN>::kWaveBytes, "bf16 staging fits the wave's region");
        if (vec) {
            store_tile_bf16_tr<SM, SN>(p, acc, row0, col0, lane, lds);
            return;
        }
    }
    typedef VecEpilogue16<SN> E;
    typedef __attribute__((address_space(3))) float lds_f32;
    typedef __attribute__((address_space(3))) f32x4_t lds_f32x4;
    constexpr int kCols = OUT_BF16 ? 8 : 4;
    constexpr int kLanesPerRow = E::kWTN / kCols;
    constexpr int kRowsPerPass = 64 / kLanesPerRow;
    static_assert(kLanesPerRow <= 64 && 64 % kLanesPerRow == 0, "row must map onto whole lanes");
    static_assert(SM % 2 == 0, "32-row staging blocks");
    const uint32_t l16 = lane & 15u, q = lane >> 4;
    const uint32_t rl = lane / kLanesPerRow, cl = (lane % kLanesPerRow) * kCols;
    // Without partials to add first (FIXUP), the chain runs on the accumulator
    // layout before staging, 16 rows at a time on all of a lane's values (one
    // bias value per sub-tile column); with them, after the sums, on the rows
    // read back.  Bias reads past N return 0 (the descriptor's range).
    float bv[kCols], bl[SN];
#pragma unroll
    for (int c = 0; c < kCols; ++c) bv[c] = 0.0f;
#pragma unroll
    for (int j = 0; j < SN; ++j) bl[j] = 0.0f;
    if (p.flags & T0G_FLAG_BIAS) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)p.bias, 0, (int)(p.n * 4u), (int)kRsrcWord3);
        if constexpr (FIXUP) {
#pragma unroll
            for (int c = 0; c < kCols; ++c)
                bv[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (col0 + cl + c) * 4u, 0, 0));
        } else {
#pragma unroll
            for (int j = 0; j < SN; ++j)
                bl[j] = __builtin_bit_cast(float,
                                           __builtin_amdgcn_raw_buffer_load_b32(r, (col0 + j * 16 + l16) * 4u, 0, 0));
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    }
    const uint64_t cbase = p.c + (uint64_t)blockIdx.y * p.c_split_stride;
    const uint32_t esize = OUT_BF16 ? 2u : 4u;
#pragma unroll
    for (int i2 = 0; i2 < SM; i2 += 2) {
        f32x4_t x[2][SN];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int j = 0; j < SN; ++j) x[ii][j] = acc[i2 + ii][j];
        if constexpr (FIXUP) {
            // all of a slot's loads for this block are issued before any is used
            for (uint32_t s = 0; s < fx.count; ++s) {
                const uint64_t sb =
                    fx.base + (uint64_t)(fx.first + s) * T0G_SK_SLOT_BYTES + fx.frag + (uint32_t)(i2 * SN) * 1024u;
                f32x4_t t[2][SN];
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                    for (int j = 0; j < SN; ++j)
                        t[ii][j] = *reinterpret_cast<const volatile __attribute__((address_space(1))) f32x4_t*>(
                            (uintptr_t)(sb + (uint32_t)(ii * SN + j) * 1024u));
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                    for (int j = 0; j < SN; ++j) x[ii][j] += t[ii][j];
            }
        } else {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                float v[SN * 4], b4[SN * 4];
#pragma unroll
                for (int j = 0; j < SN; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        v[4 * j + r] = x[ii][j][r];
                        b4[4 * j + r] = bl[j];
                    }
                apply_epilogue_n<SN * 4>(v, b4, epi_of(p));
#pragma unroll
                for (int j = 0; j < SN; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) x[ii][j][r] = v[4 * j + r];
            }
        }
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int j = 0; j < SN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t row = 16 * ii + 4 * q + r;
                    *reinterpret_cast<lds_f32*>((uintptr_t)(lds + row * E::kStride + (j * 16 + l16) * 4)) =
                        x[ii][j][r];
                }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int pass = 0; pass < 32 / kRowsPerPass; ++pass) {
            const uint32_t rr = pass * kRowsPerPass + rl;
            float v[kCols];
#pragma unroll
            for (int c = 0; c < kCols; c += 4) {
                const f32x4_t qv = *reinterpret_cast<const lds_f32x4*>((uintptr_t)(lds + rr * E::kStride + (cl + c) * 4));
                v[c] = qv[0];
                v[c + 1] = qv[1];
                v[c + 2] = qv[2];
                v[c + 3] = qv[3];
            }
            if constexpr (FIXUP) apply_epilogue_n<kCols>(v, bv, epi_of(p));
            const uint32_t grow = row0 + i2 * 16 + rr, gcol = col0 + cl;
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
                if constexpr (WT)
                    *reinterpret_cast<volatile __attribute__((address_space(1))) u32x4_t*>((uintptr_t)addr) = w;
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

// Output tile of this workgroup: block ids remapped so each XCD (own L2) works
// on a contiguous patch, walked in groups of group_m tile rows.
template <int BM, int BN>
__device__ __forceinline__ void tile_of_index(const T0gGemmArgs& p, uint32_t bid, uint32_t& m0, uint32_t& n0) {
    const uint32_t gm = p.group_m;
    const uint32_t per_group = gm * p.tiles_n;
    const uint32_t group = bid / per_group;
    const uint32_t first_m = group * gm;
    const uint32_t gsz = min(p.tiles_m - first_m, gm);
    const uint32_t in_group = bid - group * per_group;
    m0 = (first_m + in_group % gsz) * BM;
    n0 = (in_group / gsz) * BN;
}

template <int BM, int BN>
__device__ __forceinline__ void tile_origin(const T0gGemmArgs& p, uint32_t& m0, uint32_t& n0) {
    uint32_t bid = blockIdx.x;
    const uint32_t nblk = p.tiles_m * p.tiles_n;
    if (p.flags & T0G_FLAG_XCD_REMAP) bid = xcd_range(bid, nblk);
    const uint32_t gm = p.group_m;
    const uint32_t per_group = gm * p.tiles_n;
    const uint32_t group = bid / per_group;
    const uint32_t first_m = group * gm;
    const uint32_t gsz = min(p.tiles_m - first_m, gm);
    const uint32_t in_group = bid - group * per_group;
    m0 = (first_m + in_group % gsz) * BM;
    n0 = (in_group / gsz) * BN;
}

// Split-K reduced in the kernel, after the K loop of a 256x256 tile (16x16x32
// result layout): the partial tile, raw fp32 and row-major, goes to this
// workgroup's slot (tile blockIdx.x, split blockIdx.y) through the same
// LDS-staged row stores as C (written through to memory), then the tile's
// arrival, chunk sums and cleanup.
template <int BM, int BN, int NT, int SM, int SN, bool OUT_BF16>
__device__ __forceinline__ void red_store_and_finish(const T0gGemmArgs& p, const T0gGemmRedArgs& ra,
                                                     const f32x4_t (&acc)[SM][SN], uint32_t row0, uint32_t col0,
                                                     uint32_t lane, uint32_t wave, uint32_t m0, uint32_t n0,
                                                     uint32_t lds, uint32_t lds_bytes) {
    T0gGemmArgs q = p;
    q.c = ra.partials + (uint64_t)(blockIdx.x * ra.splits + blockIdx.y) * (BM * BN * 4u);
    q.ldc = BN;
    q.c_split_stride = 0;
    q.epilogue = 0;
    q.flags = T0G_FLAG_C_VEC;
    store_tile_vec16<SM, SN, false, false, true>(q, acc, row0, col0, lane, lds + wave * VecEpilogue16<SN>::kWaveBytes,
                                                 true);
    T0G_WAIT_VMCNT(0);    // the partial's stores have reached memory
    barrier_no_fence();
    red_finish<BM, BN, NT, OUT_BF16>(ra, blockIdx.x, blockIdx.y, m0, n0, lds, lds_bytes);
}

// The 256x256 fast path on 16x16x32 MFMAs (2 x 2 waves of 128 x 128).  RED:
// split-K reduced inside the kernel (ra: the launch's T0gGemmRedArgs, p = ra->g).
template <bool A_K, bool B_K, bool OUT_BF16, bool WIDE = false, bool RED = false>
__device__ __forceinline__ void gemm_tile_fast16(const T0gGemmArgs& p, const T0gGemmRedArgs* ra = nullptr) {
    constexpr int BM = 256, BN = 256, WAVES_M = 2, WAVES_N = 2;
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int SM = WTM / 16, SN = WTN / 16;
    using OpA = Op16<A_K, BM, NT, SM, WIDE>;
    using OpB = Op16<B_K, BN, NT, SN, WIDE>;
    constexpr uint32_t A_BYTES = OpA::kStageBytes, STAGE = OpA::kStageBytes + OpB::kStageBytes;
    constexpr int kVmemPerStage = OpA::kInstr + OpB::kInstr;
    __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];

    tl_mark(p, 0);
    const uint32_t tid = threadIdx.x;
    uint32_t m0, n0;
    tile_origin<BM, BN>(p, m0, n0);

    const uint32_t kbeg = blockIdx.y * p.k_per_split;
    const uint32_t kend = min(p.k, kbeg + p.k_per_split);
    const int nst = kend > kbeg ? (int)((kend - kbeg + 63) / 64) : 0;

    typename OpA::bytes_t a_bytes;
    typename OpB::bytes_t b_bytes;
    if constexpr (WIDE) {
        a_bytes = operand_bytes_wide<A_K>(p.m, p.k, p.lda);
        b_bytes = operand_bytes_wide<B_K>(p.n, p.k, p.ldb);
    } else {
        a_bytes = (A_K ? (p.m - 1) * p.lda + p.k : (p.k - 1) * p.lda + p.m) * 2;
        b_bytes = (B_K ? (p.n - 1) * p.ldb + p.k : (p.k - 1) * p.ldb + p.n) * 2;
    }

    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave / WAVES_N, wn = wave % WAVES_N;
    OpA la;
    OpB lb;
    la.init(tid, m0, p.lda, wm * WTM);
    lb.init(tid, n0, p.ldb, wn * WTN);

    f32x4_t acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j) acc[i][j] = f32x4_t{};

    if (nst > 0) {
        mfma16_drain();
        const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
        if ((kend - kbeg) % 64 == 0)
            k_pipeline16<false, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg, kend, nst, lds0);
        else
            k_pipeline16<true, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg, kend, nst, lds0);
    }

    static_assert((NT / 64) * VecEpilogue16<SN>::kWaveBytes <= 2 * STAGE, "epilogue staging must fit the stages");
    mfma16_drain();
    T0G_WAIT_VMCNT(0);
    barrier_no_fence();
    tl_mark(p, 1);
    if constexpr (RED) {
        red_store_and_finish<BM, BN, NT, SM, SN, OUT_BF16>(p, *ra, acc, wm * WTM, wn * WTN, lane, wave, m0, n0,
                                                           lds_addr(smem), 2 * STAGE);
    } else {
        const bool vec = (p.flags & T0G_FLAG_C_VEC) && m0 + BM <= p.m && n0 + BN <= p.n;
        store_tile_vec16<SM, SN, OUT_BF16>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane,
                                           lds_addr(smem) + wave * VecEpilogue16<SN>::kWaveBytes, vec);
    }
    tl_mark(p, 2);
}


// Ping-pong pipeline of the 8-wave stream-K 256x256 kernel (NN, NT).  Waves 0-3 (group 0) and
// 4-7 (group 1) share the four SIMDs, one of each per SIMD, and alternate
// between a load phase (fragment reads, DMA issue, waits) and a compute phase
// (32 MFMAs and nothing else), offset by one phase: while one wave of a SIMD
// multiplies, the other one feeds LDS and its registers.  A wave's VMEM
// instruction holds up its own next MFMA for a good part of the texture
// unit's 16 cycles per 1 KB request; here that time falls on the other wave's
// MFMAs.  Every phase ends at a workgroup barrier; group 1 starts one barrier
// late and group 0 ends one barrier late.
//
// Stage s (64 K values) spans four phases: 4s (group 0 loads step 0), 4s + 1
// (group 1 loads step 0), 4s + 2 and 4s + 3 (step 1).  The DMA of stage s + 1
// goes into the buffer of stage s - 1, free since the barrier closing phase
// 4s - 1, and must be complete at the barrier closing phase 4s + 3.  Group 1
// sends its share in phase 4s + 1 and retires it in phase 4s + 3; group 0
// sends its A share in phase 4s and its B share in phase 4s + 2 and retires
// both at the end of its compute phase 4s + 3, so no phase carries more than
// half of the CU's DMA requests for the stage.
template <bool CHECK, uint32_t A_BYTES, uint32_t STAGE, int SM, int SN, class OpA, class OpB>
__device__ __forceinline__ void k_pipeline_pp(f32x4_t (&acc)[SM][SN], const OpA& la, const OpB& lb,
                                              const T0gGemmArgs& p, typename OpA::bytes_t a_bytes,
                                              typename OpB::bytes_t b_bytes,
                                              uint32_t kbeg, uint32_t kend, int nst, uint32_t lds0, uint32_t group) {
    bf16x8_t fa[SM], fb[SN];
    la.template issue<CHECK>(lds0, p.a, a_bytes, p.lda, kbeg, kend);
    lb.template issue<CHECK>(lds0 + A_BYTES, p.b, b_bytes, p.ldb, kbeg, kend);
    T0G_WAIT_VMCNT(0);
    barrier_no_fence();
    if (group != 0) barrier_no_fence();
    for (int s = 0; s < nst; ++s) {
        const uint32_t cur = lds0 + ((s & 1) ? STAGE : 0u), nxt = lds0 + ((s & 1) ? 0u : STAGE);
        // load phase, K step 0: fragment reads first, so their latency runs
        // while the DMA issues
#pragma unroll
        for (int i = 0; i < SM; ++i) fa[i] = la.template read_one<0>(cur, i);
#pragma unroll
        for (int j = 0; j < SN; ++j) fb[j] = lb.template read_one<0>(cur + A_BYTES, j);
        asm volatile("" ::: "memory");
        if (s + 1 < nst) {
            const uint32_t k1 = kbeg + (uint32_t)(s + 1) * 64;
            la.template issue<CHECK>(nxt, p.a, a_bytes, p.lda, k1, kend);
            if (group != 0) lb.template issue<CHECK>(nxt + A_BYTES, p.b, b_bytes, p.ldb, k1, kend);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        barrier_no_fence();
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j) mfma16(acc[i][j], fa[i], fb[j]);
        barrier_no_fence();
        // load phase, K step 1
#pragma unroll
        for (int i = 0; i < SM; ++i) fa[i] = la.template read_one<1>(cur, i);
#pragma unroll
        for (int j = 0; j < SN; ++j) fb[j] = lb.template read_one<1>(cur + A_BYTES, j);
        if (group == 0) {
            asm volatile("" ::: "memory");
            if (s + 1 < nst) lb.template issue<CHECK>(nxt + A_BYTES, p.b, b_bytes, p.ldb, kbeg + (uint32_t)(s + 1) * 64, kend);
            __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        } else {
            __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0)
        }
        barrier_no_fence();
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j) mfma16(acc[i][j], fa[i], fb[j]);
        if (group == 0) T0G_WAIT_VMCNT(0);
        barrier_no_fence();
    }
    if (group == 0) barrier_no_fence();
}

// ---- stream-K ------------------------------------------------------------------
// The 256x256 kernels above on a stream-K schedule (T0gGemmSkArgs): `grid`
// workgroups, one per CU, each take an equal contiguous range of the GEMM's
// (tile, 64-wide K iteration) pairs, tiles in index order and K ascending
// within a tile.  A workgroup walks the tiles of its range from the last to the
// first.  The last tile of its range is usually cut (its K tail belongs to the
// next workgroups): the workgroup writes that partial tile to its slot, makes
// it visible at device scope and raises its ready flag; it does this first, so
// the partial is ready early.  Every other tile of its range it owns (its range
// holds the tile's last K iteration): it computes its part, waits for the ready
// flags of the lower workgroups that hold the rest of the tile (those wrote
// the partial at the start of their own work), adds their partials in slot
// order and runs the epilogue.
//
// Waits only go to lower logical ids, and logical ids are tickets drawn from a
// device counter as each workgroup starts, so every workgroup waited for has
// already started and never waits for a later one: no deadlock, whether or not
// the whole grid is resident.  A wait gives up after spin_limit polls (and
// counts a timeout) so that every workgroup ends.  The last workgroup to finish
// resets the ticket and done counters; owners clear the flags they consumed:
// the control block is all zero again for the next launch.
// Partial tiles and ready flags cross XCDs, whose L2 caches are not coherent
// with each other for this memory.  Instead of fences (a release writes back,
// an acquire invalidates, the whole L2 of the XCD, which costs every other
// workgroup there its cached operand panels), partials are written and read
// with volatile accesses, which bypass the caches, and flags with relaxed
// device-scope atomics; vmcnt(0) and a barrier order the partial's stores
// before the flag.
typedef volatile __attribute__((address_space(1))) f32x4_t gvf32x4_t;

template <int SM, int SN>
__device__ __forceinline__ void store_partial16(const f32x4_t (&acc)[SM][SN], uint64_t slot_frag) {
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
            *reinterpret_cast<gvf32x4_t*>((uintptr_t)(slot_frag + (uint32_t)(i * SN + j) * 1024u)) = acc[i][j];
}

// Loop state lives in LDS and is read back after the K loop: the pipeline
// needs nearly all SGPRs, and values kept live across it would be spilled.
struct SkRange {
    uint32_t w, t;   // logical workgroup id, current tile
};

// threadIdx.x through an opaque move: values derived from it in one phase of
// the tile loop cannot be hoisted out of the loop and kept live (in VGPRs)
// across the other phase's K loop.
__device__ __forceinline__ uint32_t opaque_tid() {
    uint32_t t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((uint32_t)threadIdx.x));
    return t;
}

// A fresh, wave-uniform copy of a kernel-argument block kept in LDS: the
// kernarg values themselves would otherwise be held in SGPRs for the whole
// tile loop.  The asm barrier makes every phase read LDS again.
template <class T>
__device__ __forceinline__ T lds_args(const T& src) {
    static_assert(sizeof(T) % 16 == 0, "whole 16-byte words");
    asm volatile("" ::: "memory");
    typedef const __attribute__((address_space(3))) u32x4_t lds_u32x4;
    const uint32_t base = lds_addr(reinterpret_cast<const char*>(&src));
    uint32_t w[sizeof(T) / 4];
#pragma unroll
    for (uint32_t i = 0; i < sizeof(T) / 16; ++i) {
        const u32x4_t v = *reinterpret_cast<lds_u32x4*>((uintptr_t)(base + 16 * i));
#pragma unroll
        for (int c = 0; c < 4; ++c) w[4 * i + c] = (uint32_t)__builtin_amdgcn_readfirstlane(v[c]);
    }
    return __builtin_bit_cast(T, w);
}

__device__ __forceinline__ SkRange sk_state(const SkRange* st) {
    const volatile SkRange* v = st;
    return SkRange{(uint32_t)__builtin_amdgcn_readfirstlane(v->w), (uint32_t)__builtin_amdgcn_readfirstlane(v->t)};
}

template <bool A_K, bool B_K, bool OUT_BF16>
__device__ __forceinline__ void gemm_tile_sk(const T0gGemmSkArgs& kargs) {
    constexpr bool PP = A_K;   // same kernel choice per layout as the data-parallel 256x256 kernels
    constexpr int BM = 256, BN = 256, WAVES_M = 2, WAVES_N = PP ? 4 : 2;
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int SM = WTM / 16, SN = WTN / 16;
    using OpA = Op16<A_K, BM, NT, SM>;
    using OpB = Op16<B_K, BN, NT, SN>;
    constexpr uint32_t A_BYTES = OpA::kStageBytes, STAGE = OpA::kStageBytes + OpB::kStageBytes;
    constexpr int kVmemPerStage = OpA::kInstr + OpB::kInstr;
    static_assert((NT / 64) * SM * SN * 1024 == T0G_SK_SLOT_BYTES, "a partial tile fills one slot");
    static_assert((NT / 64) * VecEpilogue16<SN>::kWaveBytes <= 2 * STAGE, "epilogue staging must fit the stages");
    typedef __attribute__((address_space(1))) uint32_t gu32_t;
    static_assert(sizeof(T0gGemmSkArgs) % 16 == 0, "argument block copied in 16-byte words");
    __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];
    __shared__ SkRange s_state;
    __shared__ __attribute__((aligned(16))) T0gGemmSkArgs s_args;

    if (threadIdx.x == 0) {
        s_args = kargs;
        gu32_t* const ctl = reinterpret_cast<gu32_t*>((uintptr_t)kargs.sync);
        const uint32_t w = __hip_atomic_fetch_add(ctl + T0G_SK_TICKET, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t total = kargs.g.tiles_m * kargs.g.tiles_n * kargs.iters_per_tile;
        const uint32_t it0 = t0g_sk_begin(total, kargs.grid, w), it1 = t0g_sk_begin(total, kargs.grid, w + 1);
        s_state.w = w;
        s_state.t = it1 > it0 ? (it1 - 1) / kargs.iters_per_tile : 0xFFFFFFFFu;   // all ones: empty range
        if (w >= kargs.grid) {
            // control block not at zero (a launch overlapping this one): do nothing
            // rather than touch slots and flags past the grid
            s_state.t = 0xFFFFFFFFu;
            __hip_atomic_fetch_add(ctl + T0G_SK_TIMEOUTS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();

    for (;;) {
        f32x4_t acc[SM][SN];
        {
            const T0gGemmSkArgs s = lds_args(s_args);
            const T0gGemmArgs& p = s.g;
            const uint32_t tid = opaque_tid();
            const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
            const uint32_t wm = wave / WAVES_N, wn = wave % WAVES_N;
            const SkRange st = sk_state(&s_state);
            if (st.t == 0xFFFFFFFFu) break;
            const uint32_t ipt = s.iters_per_tile, total = p.tiles_m * p.tiles_n * ipt;
            const uint32_t tb = st.t * ipt;
            const uint32_t it0 = t0g_sk_begin(total, s.grid, st.w), it1 = t0g_sk_begin(total, s.grid, st.w + 1);
            const uint32_t kb = it0 > tb ? it0 - tb : 0u, ke = it1 < tb + ipt ? it1 - tb : ipt;
            uint32_t m0, n0;
            tile_of_index<BM, BN>(p, st.t, m0, n0);
            const uint32_t kbeg = kb * 64u, kend = min(p.k, ke * 64u);
            const int nst = (int)(ke - kb);
            const uint32_t a_bytes = (A_K ? (p.m - 1) * p.lda + p.k : (p.k - 1) * p.lda + p.m) * 2;
            const uint32_t b_bytes = (B_K ? (p.n - 1) * p.ldb + p.k : (p.k - 1) * p.ldb + p.n) * 2;
            const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
            OpA la;
            OpB lb;
            la.init(tid, m0, p.lda, wm * WTM);
            lb.init(tid, n0, p.ldb, wn * WTN);
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j) acc[i][j] = f32x4_t{};
            mfma16_drain();
            if constexpr (PP) {
                const uint32_t group = wave >> 2;
                if ((kend - kbeg) % 64 == 0)
                    k_pipeline_pp<false, A_BYTES, STAGE>(acc, la, lb, p, a_bytes, b_bytes, kbeg, kend, nst, lds0,
                                                         group);
                else
                    k_pipeline_pp<true, A_BYTES, STAGE>(acc, la, lb, p, a_bytes, b_bytes, kbeg, kend, nst, lds0,
                                                        group);
            } else {
                if ((kend - kbeg) % 64 == 0)
                    k_pipeline16<false, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg, kend,
                                                                       nst, lds0);
                else
                    k_pipeline16<true, A_BYTES, STAGE, kVmemPerStage>(acc, la, lb, p, a_bytes, b_bytes, kbeg, kend,
                                                                      nst, lds0);
            }
            mfma16_drain();
            T0G_WAIT_VMCNT(0);
            barrier_no_fence();
        }

        // after the K loop: everything is recomputed from the LDS state
        const T0gGemmSkArgs s = lds_args(s_args);
        const T0gGemmArgs& p = s.g;
        gu32_t* const ctl = reinterpret_cast<gu32_t*>((uintptr_t)s.sync);
        const uint32_t tid = opaque_tid();
        const uint32_t lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t wm = wave / WAVES_N, wn = wave % WAVES_N;
        const SkRange st = sk_state(&s_state);
        const uint32_t ipt = s.iters_per_tile, total = p.tiles_m * p.tiles_n * ipt;
        const uint32_t tb = st.t * ipt;
        const uint32_t it0 = t0g_sk_begin(total, s.grid, st.w), it1 = t0g_sk_begin(total, s.grid, st.w + 1);
        const uint32_t frag = wave * (uint32_t)(SM * SN) * 1024u + lane * 16u;
        gu32_t* const ready = ctl + T0G_SK_CTL_WORDS;
        if (it1 < tb + ipt) {
            // the tile's K tail belongs to later workgroups: leave the partial
            store_partial16<SM, SN>(acc, s.partials + (uint64_t)st.w * T0G_SK_SLOT_BYTES + frag);
            T0G_WAIT_VMCNT(0);
            __syncthreads();
            if (tid == 0) __hip_atomic_store(ready + st.w, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            const uint32_t first = tb < it0 ? t0g_sk_worker(total, s.grid, tb) : st.w;
            if (first < st.w) {
                if (tid == 0) {
                    const bool stall = (s.debug & T0G_SK_DEBUG_STALL) != 0u;
                    for (uint32_t j = first; j < st.w; ++j) {
                        gu32_t* const flag = stall ? ctl + T0G_SK_NEVER_SET : ready + j;
                        for (uint32_t n = 0;
                             __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u; ++n) {
                            if (n >= s.spin_limit) {
                                __hip_atomic_fetch_add(ctl + T0G_SK_TIMEOUTS, 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
                                break;
                            }
                            __builtin_amdgcn_s_sleep(2);
                        }
                    }
                }
                __syncthreads();
            }
            uint32_t m0, n0;
            tile_of_index<BM, BN>(p, st.t, m0, n0);
            const bool vec = (p.flags & T0G_FLAG_C_VEC) && m0 + BM <= p.m && n0 + BN <= p.n;
            store_tile_vec16<SM, SN, OUT_BF16, true>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane,
                                                     lds_addr(smem) + wave * VecEpilogue16<SN>::kWaveBytes, vec,
                                                     SkFixup{s.partials, first, st.w - first, frag});
            if (first < st.w) {
                __syncthreads();
                if (tid == 0)
                    for (uint32_t j = first; j < st.w; ++j)
                        __hip_atomic_store(ready + j, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        // next tile down, or done; the barrier also ends the epilogue's use of LDS
        // before the next K loop's DMA
        __syncthreads();
        if (tid == 0) s_state.t = tb > it0 ? st.t - 1 : 0xFFFFFFFFu;
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        gu32_t* const ctl = reinterpret_cast<gu32_t*>((uintptr_t)kargs.sync);
        const uint32_t done = __hip_atomic_fetch_add(ctl + T0G_SK_DONE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == kargs.grid - 1) {
            __hip_atomic_store(ctl + T0G_SK_TICKET, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl + T0G_SK_DONE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace t0g

#endif
