// Split-K with the reduction inside the GEMM kernel (T0gGemmRedArgs, kernels
// with suffix _r).  Included by gemm_gfx950.hip after its DMA and epilogue
// helpers.
//
// A separate reduce kernel costs a second dependent launch (about 3.7 us of
// launch-to-launch time on MI355X, more than the reduce itself on the
// HBM-bound shapes) plus its own pass over the planes.  Here every workgroup
// of a tile's K slices writes its fp32 partial tile to its slot, and the
// tile's sum is formed by the same kernel:
//   * arrival: once the partial's stores have completed, thread 0 increments
//     the tile's arrival counter; the increment that completes the tile makes
//     its workgroup the tile's last arrival;
//   * chunks: the tile's row-major elements are cut into `splits` chunks,
//     chunk s belonging to split s.  A workgroup sums a chunk after claiming
//     it: a fetch-or of the chunk's bit into the tile's 64-bit claim mask, the
//     chunk being its own if the bit was clear.  An earlier arrival waits a
//     bounded number of polls for the tile to complete, then claims its own
//     chunk, or leaves if the wait ran out.  The last arrival sums its own
//     chunk, then claims every chunk still clear with one more fetch-or and
//     sums those.  So each chunk is summed exactly once, and no workgroup
//     depends on another one being resident: no deadlock and no error path;
//   * order: a chunk's elements are summed over the splits in order 0, 1, ...
//     starting from 0.0 -- the plane order of t0g_splitk_reduce and of the
//     reference's host loop -- so the result is the same bit for bit whoever
//     sums it, and equal to the two-kernel path's.
// Partials cross XCDs, whose L2 caches are not coherent with each other for
// this memory.  Release and acquire fences would write back and invalidate
// the whole L2 of the XCD for every workgroup (evicting the operand panels of
// the workgroups still in their K loops); instead the partials are written
// through to memory (sc0 sc1 stores, completed by vmcnt(0) before the
// arrival), read back by LDS DMA that bypasses the caches (sc0 sc1), and
// counters and claim masks are relaxed device-scope atomics, each tile's in a
// cache line of its own.  A tile's done counter counts its workgroups out;
// the last one clears the tile's line, so every launch finds it at zero.
// Counter values past `splits` can only come from two launches sharing the
// control block at once: they are counted in T0G_SK_TIMEOUTS, which the host
// reports as an error.
#ifndef T0G_GEMM_RED_H
#define T0G_GEMM_RED_H

namespace t0g {

typedef __attribute__((address_space(1))) uint32_t gred_u32_t;

// dma16 with sc0 sc1: the 16 bytes come from memory, not from a cache that
// may hold an older copy.
__device__ __forceinline__ void dma16_sys(u32x4_t rsrc, uint32_t voff, uint32_t lds_m0) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %0, %1, 0 offen sc0 sc1 lds"
        :
        : "v"(voff), "s"(rsrc), "s"(lds_m0)
        : "memory", "m0");
}

// Sum chunk c of tile `tile` over its splits into C (rows and columns of the
// tile that fall outside M x N are skipped).  The chunk's splits x ce values
// are staged in LDS by DMA (every 1 KB piece of a round in flight at once), in
// rounds of at most lds_bytes, then each thread sums 4 consecutive elements.
template <int BM, int BN, int NT, bool OUT_BF16>
__device__ __forceinline__ void red_chunk(const T0gGemmRedArgs& ra, uint32_t tile, uint32_t c, uint32_t m0,
                                          uint32_t n0, uint32_t lds, uint32_t lds_bytes) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
    const T0gGemmArgs& p = ra.g;
    constexpr uint32_t E = (uint32_t)BM * BN;
    constexpr int kWaves = NT / 64;
    const uint32_t S = ra.splits;
    const uint32_t ce = E / S;                       // elements per chunk (a multiple of 256)
    uint32_t sub = lds_bytes / (4u * S);             // elements per round: powers of two throughout
    if (sub > ce) sub = ce;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t slot_bytes = E * 4u;
    const u32x4_t rsrc = rsrc_words(ra.partials, (uint32_t)((uint64_t)ra.grid * slot_bytes), 0);
    const uint32_t pieces_per_plane = sub * 4u / 1024u;
    const EpiParams ep = epi_of(p);
    for (uint32_t r0 = 0; r0 < ce; r0 += sub) {
        const uint32_t e0 = c * ce + r0;
        const uint32_t pieces = S * pieces_per_plane;
        for (uint32_t q = wave; q < pieces; q += kWaves) {
            const uint32_t s = q / pieces_per_plane, piece = q - s * pieces_per_plane;
            const uint32_t goff = (tile * S + s) * slot_bytes + e0 * 4u + piece * 1024u;
            dma16_sys(rsrc, goff + lane * 16u, lds + s * sub * 4u + piece * 1024u);
        }
        T0G_WAIT_VMCNT(0);
        barrier_no_fence();
        for (uint32_t g4 = tid; g4 < sub / 4u; g4 += NT) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            for (uint32_t s = 0; s < S; ++s)
                acc = acc + *reinterpret_cast<const lds_f32x4*>((uintptr_t)(lds + s * sub * 4u + g4 * 16u));
            const uint32_t e = e0 + g4 * 4u;
            const uint32_t row = m0 + e / BN, col = n0 + e % BN;
            float v[4] = {acc[0], acc[1], acc[2], acc[3]}, bv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                bv[k] = ((p.flags & T0G_FLAG_BIAS) && col + k < p.n)
                            ? reinterpret_cast<const __attribute__((address_space(1))) float*>(p.bias)[col + k]
                            : 0.0f;
            apply_epilogue_n<4>(v, bv, ep);
            if (row >= p.m) continue;
            const uint64_t o = (uint64_t)row * p.ldc + col;
            if ((p.flags & T0G_FLAG_C_VEC) && col + 4 <= p.n) {
                if constexpr (OUT_BF16) {
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    u32x2 w;
                    w[0] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[0]) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[1]) << 16);
                    w[1] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[2]) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[3]) << 16);
                    *reinterpret_cast<__attribute__((address_space(1))) u32x2*>((uintptr_t)(p.c + o * 2)) = w;
                } else {
                    const f32x4 y = {v[0], v[1], v[2], v[3]};
                    *reinterpret_cast<__attribute__((address_space(1))) f32x4*>((uintptr_t)(p.c + o * 4)) = y;
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (col + k < p.n) {
                        if constexpr (OUT_BF16)
                            reinterpret_cast<gbf16_t*>((uintptr_t)p.c)[o + k] = (__bf16)v[k];
                        else
                            reinterpret_cast<gf32_t*>((uintptr_t)p.c)[o + k] = v[k];
                    }
                }
            }
        }
        barrier_no_fence();   // the next round's DMA reuses the LDS
    }
}

// After the workgroup's partial tile is in its slot (its write-through stores
// completed and the workgroup past a barrier): arrival, chunk claims and sums,
// and the end-of-launch cleanup.  lds / lds_bytes: LDS the kernel no longer
// needs.
template <int BM, int BN, int NT, bool OUT_BF16>
__device__ __forceinline__ void red_finish(const T0gGemmRedArgs& ra, uint32_t tile, uint32_t split, uint32_t m0,
                                           uint32_t n0, uint32_t lds, uint32_t lds_bytes) {
    __shared__ uint32_t s_red[3];
    gred_u32_t* const ctl = reinterpret_cast<gred_u32_t*>((uintptr_t)ra.sync);
    // the tile's own 128-byte line: arrival counter, 64-bit claim mask, done counter
    gred_u32_t* const arrival = ctl + T0G_RED_ARRIVAL + tile * T0G_RED_LINE_WORDS;
    gred_u32_t* const claim = arrival + 1;
    gred_u32_t* const done = arrival + 3;
    const uint32_t S = ra.splits;
    const uint32_t tid = threadIdx.x;
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(arrival, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev >= S) __hip_atomic_fetch_add(ctl + T0G_SK_TIMEOUTS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t last = prev + 1u == S;
        uint32_t complete = last;
        if (!last && prev < S) {
            // polls spaced by about 500 clocks: the tile's other slices finish
            // within a few microseconds, and denser polling of the same lines
            // by every waiting workgroup slows the arrivals themselves
            gred_u32_t* const w = (ra.debug & T0G_SK_DEBUG_STALL) ? ctl + T0G_SK_NEVER_SET : arrival;
            for (uint32_t n = 0; n < ra.spin_limit; ++n) {
                if (__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= S) {
                    complete = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
        }
        uint32_t mine = 0;
        if (complete) {
            const uint32_t bit = 1u << (split & 31u);
            mine = (__hip_atomic_fetch_or(claim + (split >> 5), bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                    bit) == 0u;
        }
        s_red[0] = last;
        s_red[1] = mine;
    }
    __syncthreads();
    const uint32_t last = s_red[0], mine = s_red[1];
    if (mine) red_chunk<BM, BN, NT, OUT_BF16>(ra, tile, split, m0, n0, lds, lds_bytes);
    if (last) {
        __syncthreads();   // s_red reused
        if (tid == 0) {
            // every chunk whose workgroup has not claimed it (it gave up waiting)
            const uint32_t all_lo = S >= 32u ? 0xFFFFFFFFu : (1u << S) - 1u;
            const uint32_t all_hi = S >= 64u ? 0xFFFFFFFFu : S > 32u ? (1u << (S - 32u)) - 1u : 0u;
            s_red[1] = ~__hip_atomic_fetch_or(claim, all_lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & all_lo;
            s_red[2] = all_hi ? ~__hip_atomic_fetch_or(claim + 1, all_hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                                    all_hi
                              : 0u;
        }
        __syncthreads();
        const uint32_t free_lo = __builtin_amdgcn_readfirstlane(s_red[1]);
        const uint32_t free_hi = __builtin_amdgcn_readfirstlane(s_red[2]);
        for (uint32_t c = 0; c < S; ++c) {
            const uint32_t word = c < 32u ? free_lo : free_hi;
            if ((word >> (c & 31u)) & 1u) red_chunk<BM, BN, NT, OUT_BF16>(ra, tile, c, m0, n0, lds, lds_bytes);
        }
    }
    __syncthreads();
    if (tid == 0) {
        // the tile's last workgroup out: every other one has finished with the line
        const uint32_t out = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (out + 1u == S) {
            for (uint32_t w = 0; w < 4u; ++w)
                __hip_atomic_store(arrival + w, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (out >= S) {
            __hip_atomic_fetch_add(ctl + T0G_SK_TIMEOUTS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Two K slices: no wait at all.  Both workgroups of the tile have written
// their partials through to memory (vmcnt(0), then a barrier) when thread 0
// increments the tile's arrival counter.  The first to arrive leaves.  The
// second finds the other slice's partial complete in memory, adds it to its
// own values in plane order -- (0 + p0) + p1, the reduce kernel's order, so
// the bits equal the two-kernel path's whichever slice arrives second -- and
// stores the output through the epilogue; it also clears the counter for the
// next launch (both workgroups are done with it).  This takes three memory
// round trips after the K loop (partial, counter, the other partial), where
// red_finish's arrival, wait, claim and done counter take six.
template <int BM, int BN, int SM, int SN, bool OUT_BF16>
__device__ __forceinline__ void red_pair(const T0gGemmRedArgs& ra, const f32x16_t (&acc)[SM][SN], uint32_t tile,
                                         uint32_t split, uint32_t m0, uint32_t n0, uint32_t wrow, uint32_t wcol,
                                         uint32_t lane, uint32_t lds_stage) {
    __shared__ uint32_t s_pair;
    const T0gGemmArgs& p = ra.g;
    gred_u32_t* const ctl = reinterpret_cast<gred_u32_t*>((uintptr_t)ra.sync);
    gred_u32_t* const arrival = ctl + T0G_RED_ARRIVAL + tile * T0G_RED_LINE_WORDS;
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(arrival, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev >= 2u) __hip_atomic_fetch_add(ctl + T0G_SK_TIMEOUTS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == 1u) __hip_atomic_store(arrival, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_pair = prev;
    }
    __syncthreads();
    if (s_pair != 1u) return;
    constexpr uint32_t kSlot = (uint32_t)BM * BN * 4u;
    const uint64_t partner = ra.partials + (uint64_t)(tile * 2u + (split ^ 1u)) * kSlot + ((uint64_t)wrow * BN + wcol) * 4u;
    const bool vec = (p.flags & T0G_FLAG_C_VEC) && m0 + BM <= p.m && n0 + BN <= p.n;
    store_tile_vec<SM, SN, OUT_BF16, false, false, true>(p, acc, m0 + wrow, n0 + wcol, lane, lds_stage, vec, 0,
                                                         partner, BN, split == 0u);
}

}  // namespace t0g

#endif
