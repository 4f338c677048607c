// Device half of the C ABI: HIP device/stream/memory, the embedded gfx950
// code object, the reference-layout dispatch path and the typed GEMM entry.
//
// The reference talks to /dev/kfd directly: VRAM allocation, an AQL queue
// with a doorbell, an ELF loader that patches RSRC1 (src/kfd/mod.rs).  Here
// those become hipMalloc, one HIP stream per device handle and
// hipModuleLoadData / hipModuleLaunchKernel on a code object built ahead of
// time by hipcc for gfx950.
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <string.h>
#include <time.h>

#include <algorithm>
#include <atomic>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "t0g.h"
#include "t0g_internal.h"
#include "t0g_kernel_args.h"

// The gfx950 code object, embedded at build time (T0G_HSACO_FILE is set by the Makefile).
__asm__(".section .rodata.t0g_hsaco,\"a\",@progbits\n"
        ".p2align 12\n"
        ".hidden t0g_hsaco_begin\n"
        ".globl t0g_hsaco_begin\n"
        "t0g_hsaco_begin:\n"
        ".incbin \"" T0G_HSACO_FILE "\"\n"
        ".hidden t0g_hsaco_end\n"
        ".globl t0g_hsaco_end\n"
        "t0g_hsaco_end:\n"
        ".byte 0\n"
        ".previous\n");
extern "C" const unsigned char t0g_hsaco_begin[];
extern "C" const unsigned char t0g_hsaco_end[];
// The same kernels with the workgroup timeline compiled in (T0G_HSACO_TL_FILE),
// loaded on a device the first time the timeline is used there.
__asm__(".section .rodata.t0g_hsaco_tl,\"a\",@progbits\n"
        ".p2align 12\n"
        ".hidden t0g_hsaco_tl_begin\n"
        ".globl t0g_hsaco_tl_begin\n"
        "t0g_hsaco_tl_begin:\n"
        ".incbin \"" T0G_HSACO_TL_FILE "\"\n"
        ".byte 0\n"
        ".previous\n");
extern "C" const unsigned char t0g_hsaco_tl_begin[];

namespace t0g {

enum class KernelKind { GemmGen, TileGemm, Raw };

}  // namespace t0g

struct t0g_kernel {
    t0g::KernelKind kind;
    t0g_gemm_config cfg;          // GemmGen / TileGemm
    hipFunction_t fn = nullptr;   // Raw
    uint32_t wg[3] = {1, 1, 1};
    uint32_t lds = 0;
    uint32_t dyn_lds = 0;         // Raw: LDS requested at launch beyond the kernel's static LDS
    uint32_t kernarg_size = 0;    // Raw: exact argument block size, from the code object's metadata
    uint32_t chain = 0;           // TileGemm: epilogue chain its kernargs carry
    std::string name;
};

struct t0g_device {
    int ordinal = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t order_event = nullptr;   // orders launches across t0g_device_set_stream
    hipModule_t module = nullptr;
    hipModule_t module_tl = nullptr;   // the timeline build of the same kernels (loaded on first use)
    std::mutex mu;
    bool poisoned = false;
    std::string poison_reason;
    std::unordered_map<std::string, hipFunction_t> fns;
    std::unordered_map<std::string, hipFunction_t> fns_tl;
    std::vector<std::unique_ptr<t0g_kernel>> kernels;
    std::unordered_map<std::string, t0g_kernel *> kernel_cache;
    std::vector<hipModule_t> extra_modules;
    std::unordered_map<uint64_t, size_t> allocations;   // live buffers -> their 4 KiB-rounded size
    // BufferPool (src/ignis/gpu_context.rs:21-76): recycled buffers by size
    std::unordered_map<size_t, std::vector<uint64_t>> pool;
    size_t pool_bytes = 0;
    uint64_t pool_hits = 0, pool_misses = 0;
    uint64_t ws = 0;
    size_t ws_bytes = 0;
    uint64_t conv = 0;         // bf16 operand scratch of the matmul entry points
    size_t conv_bytes = 0;
    // GpuRuntime::bf16_cache (src/ignis/gpu_context.rs:100): tensor id -> its bf16 copy.
    // The buffers come from the pool but belong to the cache (not to `allocations`, so
    // t0g_free / t0g_recycle refuse them); invalidating an id returns its buffer to the pool.
    struct Bf16Copy {
        uint64_t addr;
        size_t n;       // elements converted
        size_t bytes;   // pool size of the buffer
    };
    std::unordered_map<uint64_t, Bf16Copy> bf16_cache;
    uint32_t num_cus = 0;      // compute units: the stream-K grid
    uint64_t scratch = 0;      // this device's no-allocation scratch (0: unavailable, see scratch_error)
    std::string scratch_error;
    uint64_t sk_sync = 0;      // stream-K control words and ready flags (zero between launches)
    hipStream_t sk_stream = nullptr;   // stream of a stream-K launch whose timeout word is not yet checked
    // t0g_gemm_group: side streams (default priority), each with its own split-K
    // workspace, and the events that fork them from and join them back into `stream`
    static constexpr int kSides = 2;
    hipStream_t side[kSides] = {};
    uint64_t side_ws[kSides] = {};
    size_t side_ws_bytes[kSides] = {};
    hipEvent_t fork_ev = nullptr;
    hipEvent_t join_ev[kSides] = {};
};

namespace t0g {

static std::atomic<int> g_fail_countdown{0};
static std::atomic<uint32_t> g_wait_timeout_ms{60000};
// Polls of a stream-K ready flag (each followed by a short s_sleep: about a
// tenth of a second in all at the default, against microseconds for a real
// wait) before a workgroup gives up and counts a timeout.
static std::atomic<uint32_t> g_sk_spin_limit{1u << 20};
static std::atomic<uint32_t> g_sk_debug{0};
// Split-K: 0 = reduce inside the GEMM kernel where the plan allows it (the _r
// kernels), 1 = always partial planes plus the separate reduce kernel.
static std::atomic<uint32_t> g_split_mode{T0G_SPLIT_K_AUTO};
// Workgroup timeline recording (t0g_set_timeline): a diagnostic, off by default.
static std::atomic<int> g_timeline{0};
// Polls a workgroup of a fused split-K launch waits for its tile's other K
// slices before leaving its chunk to the tile's last arrival (a few tens of
// microseconds: within one wave of workgroups the slices finish together).
constexpr uint32_t kRedSpinLimit = 256;

// Every HIP call goes through here so a test can make the n-th one fail.
static bool injected_failure() {
    int c = g_fail_countdown.load();
    while (c > 0) {
        if (g_fail_countdown.compare_exchange_weak(c, c - 1)) return c == 1;
    }
    return false;
}

#define T0G_HIP(expr) (::t0g::injected_failure() ? hipErrorLaunchFailure : (expr))

// Device-memory allocations this library has asked HIP for (hipMalloc and
// code-object loads), process-wide, so a test can show that an entry point
// allocates nothing.
static std::atomic<uint64_t> g_device_allocs{0};

static hipError_t dev_malloc(void **p, size_t bytes) {
    g_device_allocs.fetch_add(1);
    return hipMalloc(p, bytes);
}

static hipError_t module_load(hipModule_t *m, const void *image) {
    g_device_allocs.fetch_add(1);
    return hipModuleLoadData(m, image);
}

static int hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorOutOfMemory ? T0G_ERR_OUT_OF_MEMORY : T0G_ERR_HIP, "%s failed: %s (%d)", what,
                hipGetErrorString(e), (int)e);
}

// A failure of work already sent to the device poisons the handle, as the
// reference's GpuRuntime does after a dispatch timeout.
static int poison(t0g_device *dev, int code) {
    dev->poisoned = true;
    dev->poison_reason = g_last_error;
    return code;
}

static int check_usable(t0g_device *dev) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    if (dev->poisoned)
        return fail(T0G_ERR_POISONED, "device poisoned by an earlier failure: %s", dev->poison_reason.c_str());
    hipError_t e = T0G_HIP(hipSetDevice(dev->ordinal));
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    return T0G_OK;
}

static double now_ms() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

// Once a stream that ran a stream-K launch has drained: a ready-flag wait that
// gave up, or a launch that found the control block busy, left cut tiles
// without some of their partial sums, so the result is wrong and the device is
// poisoned with T0G_ERR_TIMEOUT, as the reference poisons its runtime after a
// dispatch timeout (src/ignis/gpu_context.rs:150-157).
static int check_stream_k(t0g_device *dev) {
    if (!dev->sk_stream || dev->sk_stream != dev->stream) return T0G_OK;
    dev->sk_stream = nullptr;
    uint32_t count = 0;
    hipError_t e = T0G_HIP(hipMemcpy(&count, (const void *)(dev->sk_sync + 4 * T0G_SK_TIMEOUTS), 4,
                                     hipMemcpyDeviceToHost));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipMemcpy(stream-K timeout count)"));
    if (count)
        return poison(dev, fail(T0G_ERR_TIMEOUT,
                                "stream-K: %u ready-flag wait(s) gave up or launches overlapped; cut tiles miss "
                                "partial sums",
                                count));
    return T0G_OK;
}

// Wait for the stream with a time limit (the reference polls the AQL read
// pointer for 5 s, src/kfd/mod.rs:1607-1642).  Timeout poisons the device.
// The first 200 us poll without sleeping, as the reference does: a sleep of
// the kernel's timer granularity (~60 us with the default timer slack) would
// otherwise dominate a short GEMM's synchronous call.  Longer waits sleep
// 20 us between polls.
static int wait_stream(t0g_device *dev) {
    const double t0 = now_ms();
    const uint32_t limit = g_wait_timeout_ms.load();
    for (;;) {
        hipError_t e = T0G_HIP(hipStreamQuery(dev->stream));
        if (e == hipSuccess) return check_stream_k(dev);
        if (e != hipErrorNotReady) return poison(dev, hip_fail(e, "hipStreamQuery"));
        const double waited = now_ms() - t0;
        if (waited > limit)
            return poison(dev, fail(T0G_ERR_TIMEOUT, "GPU wait timed out after %u ms", limit));
        if (waited > 0.2) {
            timespec ts = {0, 20000};
            nanosleep(&ts, nullptr);
        }
    }
}

static int load_timeline_module(t0g_device *dev) {
    if (dev->module_tl) return T0G_OK;
    hipError_t e = T0G_HIP(module_load(&dev->module_tl, t0g_hsaco_tl_begin));
    if (e != hipSuccess) {
        dev->module_tl = nullptr;
        return hip_fail(e, "hipModuleLoadData(timeline code object)");
    }
    return T0G_OK;
}

// timeline: the kernel from the timeline build of the code object.
static int get_function(t0g_device *dev, const std::string &name, hipFunction_t *out, bool timeline = false) {
    auto &fns = timeline ? dev->fns_tl : dev->fns;
    auto it = fns.find(name);
    if (it != fns.end()) {
        *out = it->second;
        return T0G_OK;
    }
    if (timeline) {
        int rc = load_timeline_module(dev);
        if (rc) return rc;
    }
    hipFunction_t f = nullptr;
    hipError_t e = T0G_HIP(hipModuleGetFunction(&f, timeline ? dev->module_tl : dev->module, name.c_str()));
    if (e != hipSuccess) return hip_fail(e, ("hipModuleGetFunction(" + name + ")").c_str());
    fns.emplace(name, f);
    *out = f;
    return T0G_OK;
}

static int launch(t0g_device *dev, hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx,
                  void *args, size_t args_size) {
    void *extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &args_size,
                     HIP_LAUNCH_PARAM_END};
    hipError_t e = T0G_HIP(hipModuleLaunchKernel(f, gx, gy, gz, bx, 1, 1, 0, dev->stream, nullptr, extra));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipModuleLaunchKernel"));
    return T0G_OK;
}

static const char *layout_tag(uint32_t t) {
    static const char *tags[] = {"nt", "nn", "tn", "tt"};
    return tags[t & 3];
}

static bool a_k_major(uint32_t t) { return t == T0G_NT || t == T0G_NN; }
static bool b_k_major(uint32_t t) { return t == T0G_NT || t == T0G_TT; }

// A fully resolved GEMM launch (both the typed API and the reference-layout
// dispatch path end here).
struct GemmPlan {
    const TileDef *tile;
    uint32_t transpose;
    bool out_bf16;
    bool aligned;
    uint32_t splits;
    uint32_t k_per_split;
    uint32_t tiles_m, tiles_n;
    uint32_t wg;   // threads per workgroup of the chosen kernel
    bool stream_k;
    uint32_t sk_ipt;   // stream-K: 64-wide K steps per tile
    bool fused;        // split-K reduced inside the GEMM kernel (_r symbol)
    std::string symbol;
};

// Stream-K grid: one workgroup per CU (at most 256, the table's CU count),
// never more than there are (tile, K step) pairs.
static uint32_t sk_grid(const GemmPlan &p, uint32_t num_cus) {
    const uint64_t total = (uint64_t)p.tiles_m * p.tiles_n * p.sk_ipt;
    uint64_t g = num_cus ? num_cus : kNumCUs;
    if (g > kNumCUs) g = kNumCUs;
    return (uint32_t)(total < g ? total : g);
}

// How the kernels address the operands.
//   Fast: 16-byte aligned rows and operands below 2^30 elements; the buffer
//     descriptors span the whole operand (0x80000000 is their always-out-of-range
//     offset).
//   Wide: aligned operands of 2^30 elements or more, 256x256 kernels only (_x):
//     the descriptors are rebased to the tile's first row (K-contiguous operand)
//     or the stage's first k row (M/N-contiguous) and cut to 2 GiB; the offsets
//     used from there stay below 2 GiB for leading dimensions below these bounds
//     (256 rows of a K-contiguous tile; 64 k rows plus one row of a stage).
//   Elementwise: everything else (_u kernels, 32-bit element offsets).
enum class OperandPath { Fast, Wide, Elementwise };
constexpr uint32_t kMaxKMajorLd = 1u << 22;
constexpr uint32_t kMaxMnMajorLd = (1u << 24) - 256;

// The 256x256 kernels issue a stage's DMA in groups of four 1 KB requests
// sharing one M0 value; each request's offset register holds its piece's byte
// offset less up to 3 KB (the instruction's immediate offset adds it back).  An
// M/N-contiguous operand's piece i of wave 0 starts 2 i k rows, i.e. 4 i ld
// bytes, in: not below i KB only for ld >= 256.  Smaller leading dimensions of
// M/N-contiguous operands therefore stay off those kernels (a K-contiguous
// operand on a whole-stage loop has ld >= K >= 64, which is enough there).
static bool ld_fits_256(uint32_t t, uint32_t lda, uint32_t ldb) {
    return (a_k_major(t) || lda >= 256) && (b_k_major(t) || ldb >= 256);
}

static OperandPath operand_path(uint64_t a, uint64_t b, uint32_t m, uint32_t n, uint32_t k, uint32_t lda,
                                uint32_t ldb, uint32_t t) {
    if ((a & 15) || (b & 15) || (lda & 7) || (ldb & 7)) return OperandPath::Elementwise;
    if (a_k_major(t) ? (k & 7) != 0 : ((m & 7) != 0 || m < 8)) return OperandPath::Elementwise;
    if (b_k_major(t) ? (k & 7) != 0 : ((n & 7) != 0 || n < 8)) return OperandPath::Elementwise;
    const uint64_t a_elems = a_k_major(t) ? (uint64_t)m * lda : (uint64_t)k * lda;
    const uint64_t b_elems = b_k_major(t) ? (uint64_t)n * ldb : (uint64_t)k * ldb;
    if (a_elems < (1ull << 30) && b_elems < (1ull << 30)) return OperandPath::Fast;
    if (lda < (a_k_major(t) ? kMaxKMajorLd : kMaxMnMajorLd) && ldb < (b_k_major(t) ? kMaxKMajorLd : kMaxMnMajorLd) &&
        ld_fits_256(t, lda, ldb))
        return OperandPath::Wide;
    return OperandPath::Elementwise;
}

// allow_fused: the caller can run the in-kernel split-K reduction (its sync
// words exist; not concurrent with another such launch of this device).
// exact_split: K is cut into exactly split_req slices of k / split_req (the
// caller guarantees the division and a multiple of 8 per slice: the fp32
// planes are the caller's, with the reference's partition); otherwise slices
// are rounded to whole 64-K stages and the split may shrink.
// fits_256: ld_fits_256() of the operands.
static int make_plan(const TileDef *tile, uint32_t transpose, bool out_bf16, OperandPath path, bool fits_256,
                     uint32_t m, uint32_t n, uint32_t k, uint32_t split_req, GemmPlan *p, bool allow_fused = false,
                     bool exact_split = false) {
    const bool aligned = path != OperandPath::Elementwise, wide = path == OperandPath::Wide;
    bool stream_k = split_req == T0G_STREAM_K;
    if (stream_k) split_req = 1;
    if (!aligned && tile->bm == 256) tile = &kTiles[1];   // no element-wise-load variant of the 256x256 tile
    if (!fits_256 && tile->bm == 256) tile = &kTiles[1];
    if (wide) tile = &kTiles[0];                           // the wide kernels are 256x256 only
    if (tile->bm != 256 || k == 0 || wide) stream_k = false;   // the data-parallel kernel then
    p->stream_k = stream_k;
    p->sk_ipt = stream_k ? (k + kTileK - 1) / kTileK : 0;
    p->tile = tile;
    p->transpose = transpose;
    p->out_bf16 = out_bf16;
    p->aligned = aligned;
    p->tiles_m = (m + tile->bm - 1) / tile->bm;
    p->tiles_n = (n + tile->bn - 1) / tile->bn;
    uint32_t sk = split_req ? split_req : 1;
    uint32_t kps = k;
    if (exact_split && sk > 1) {
        kps = k / sk;
    } else if (sk > 1) {
        kps = ((k + sk - 1) / sk + kTileK - 1) / kTileK * kTileK;
        sk = (k + kps - 1) / kps;
        if (sk <= 1) {
            sk = 1;
            kps = k;
        }
    }
    if (kps == 0) kps = kTileK;   // K == 0: one empty slice, C = 0 (+ epilogue)
    p->splits = sk;
    p->k_per_split = kps;
    const bool partial = sk > 1;
    // At most one workgroup per CU: the 64x64 and 128x128 tiles switch to their
    // deep-ring variants (the CU's LDS then holds one workgroup with 128 KB of
    // 64-K stages, whole cache lines per DMA request).
    const uint64_t red_grid = (uint64_t)p->tiles_m * p->tiles_n * sk;
    const bool deep = tile_uses_deep(*tile, red_grid) && aligned && !wide;
    // In-kernel reduction: a power-of-two split whose chunks (the tile cut in
    // `splits` equal parts) hold 256 elements or more, one wave of workgroups
    // (a slice waits only for slices running at the same time) and slots
    // addressable by a 32-bit buffer descriptor.  The 64x64 tile has it in its
    // deep-ring kernel only.
    // T0G_SPLIT_K_AUTO: in the kernel for two slices on the deep rings, whose
    // red_pair finish has the second slice add the first's partial without a wait
    const uint32_t mode = g_split_mode.load();
    const bool want_fused = mode == T0G_SPLIT_K_IN_KERNEL || (mode == T0G_SPLIT_K_AUTO && sk == 2 && deep);
    p->fused = partial && allow_fused && want_fused && aligned && !wide && !stream_k &&
               (tile->bm != 64 || deep) && (sk & (sk - 1)) == 0 && sk <= kMaxSplitK &&
               (uint64_t)sk * 256 <= (uint64_t)tile->bm * tile->bn &&
               red_grid <= (uint64_t)kNumCUs * tile->wg_per_cu && red_grid <= T0G_RED_MAX_GRID &&
               red_grid * tile->bm * tile->bn * 4 < (1ull << 31);
    // The 256x256 kernels run 4 waves (one 128x128 wave tile per SIMD), except
    // the stream-K ones with a K-contiguous A (NN, NT), which keep the 8-wave
    // ping-pong schedule.
    p->wg = (tile->bm == 256 && !(stream_k && a_k_major(transpose))) ? 256u : tile->wg;
    // The 64x64 deep ring splits K across its four waves (_ds, _dsr) for K
    // ranges of kKsplitMinStages 64-K stages or more: the loop then reads each
    // fragment once per stage instead of twice, and the closing sum of the four
    // partial tiles (about 0.5 us) is paid back.  Per call, split against
    // unsplit: 32 stages (128x4096x4096 NT, split 2) 13.8 against 14.2 us;
    // 16 stages (256x256x1024 NT) 6.76 against 6.64 us; 4 stages (256^3)
    // 4.91 against 4.30 us.
    const bool ksplit = deep && tile->bm == 64 && (kps + 63) / 64 >= kKsplitMinStages;
    const char *deep_sfx = ksplit ? (p->fused ? "_dsr" : "_ds") : (p->fused ? "_dr" : "_d");
    p->symbol = std::string(tile->symbol_prefix) + "_" + layout_tag(transpose) + "_" +
                ((out_bf16 && (!partial || p->fused)) ? "bf16" : "f32") +
                (aligned ? (wide ? "_x" : deep ? deep_sfx : p->fused ? "_r" : "") : "_u") + (stream_k ? "_sk" : "");
    if ((uint64_t)p->tiles_m * p->tiles_n > 0x7FFFFFFFull)
        return fail(T0G_ERR_INVALID_ARG, "too many output tiles (%u x %u)", p->tiles_m, p->tiles_n);
    if (stream_k && (uint64_t)p->tiles_m * p->tiles_n * p->sk_ipt > 0x7FFFFFFFull)
        return fail(T0G_ERR_INVALID_ARG, "stream-K: too many (tile, K step) pairs for %ux%ux%u", m, n, k);
    return T0G_OK;
}

// The element-wise kernels (operands the fast path cannot take) use 32-bit
// element offsets.
static int check_extent(const char *what, uint64_t rows, uint64_t ld) {
    if (rows * ld >= (1ull << 31))
        return fail(T0G_ERR_INVALID_ARG,
                    "%s spans %llu elements; unaligned operands (taken element-wise) must stay below 2^31", what,
                    (unsigned long long)(rows * ld));
    return T0G_OK;
}

static int ensure_workspace(t0g_device *dev, size_t bytes) {
    if (dev->ws_bytes >= bytes) return T0G_OK;
    if (dev->ws) {
        hipError_t e = T0G_HIP(hipFree((void *)dev->ws));   // hipFree waits for work using it
        dev->ws = 0;
        dev->ws_bytes = 0;
        if (e != hipSuccess) return poison(dev, hip_fail(e, "hipFree(workspace)"));
    }
    void *p = nullptr;
    hipError_t e = T0G_HIP(dev_malloc(&p, bytes));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
    dev->ws = (uint64_t)p;
    dev->ws_bytes = bytes;
    return T0G_OK;
}

struct GemmOperands {
    uint64_t a, b, c, bias;
    uint32_t m, n, k, lda, ldb, ldc;
    uint32_t chain;            // epilogue chain (t0g_epilogue_op codes)
    float epi_scale, clamp_lo, clamp_hi;
    uint64_t c_split_stride;   // reference-layout path: caller-owned planes
};

// Stream-K control words and ready flags, allocated and zeroed once per device;
// every launch leaves them zero again.
// Also the control block of the in-kernel split-K reduction (arrival and claim
// words after the control words); the two kinds of launch never overlap.
static int ensure_sk_sync(t0g_device *dev) {
    if (dev->sk_sync) return T0G_OK;
    // a fused launch has at most T0G_RED_MAX_GRID / 2 tiles (two slices or more each)
    const size_t bytes =
        (T0G_SK_CTL_WORDS + std::max<size_t>(kNumCUs, (size_t)T0G_RED_LINE_WORDS * (T0G_RED_MAX_GRID / 2))) * 4;
    void *ptr = nullptr;
    hipError_t e = T0G_HIP(dev_malloc(&ptr, bytes));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(stream-K flags)");
    e = T0G_HIP(hipMemsetAsync(ptr, 0, bytes, dev->stream));
    if (e != hipSuccess) {
        (void)hipFree(ptr);
        return hip_fail(e, "hipMemsetAsync(stream-K flags)");
    }
    dev->sk_sync = (uint64_t)ptr;
    return T0G_OK;
}

// The GEMM kernel's argument block for a plan.  With splits > 1 and no
// caller-owned planes (o.c_split_stride == 0) the kernel writes fp32 planes to
// `ws` and *reduce is set: the reduce kernel then produces C.
// allow_timeline = false: never the instrumented code object (its first use loads
// a module, which allocates device memory).
static void fill_gemm_args(const GemmPlan &p, const GemmOperands &o, uint64_t ws, T0gGemmArgs *out, bool *reduce_out,
                           bool allow_timeline = true) {
    T0gGemmArgs &args = *out;
    memset(&args, 0, sizeof args);
    args.a = o.a;
    args.b = o.b;
    args.m = o.m;
    args.n = o.n;
    args.k = o.k;
    args.lda = o.lda;
    args.ldb = o.ldb;
    args.k_per_split = p.k_per_split;
    args.tiles_m = p.tiles_m;
    args.tiles_n = p.tiles_n;
    args.group_m = 8;
    args.flags = T0G_FLAG_XCD_REMAP | (allow_timeline && g_timeline.load() ? T0G_FLAG_TIMELINE : 0u);
    const bool reduce = p.splits > 1 && o.c_split_stride == 0 && !p.fused;
    if (reduce) {
        args.c = ws;
        args.ldc = o.n;
        args.c_split_stride = (uint64_t)o.m * o.n * 4;
        args.epilogue = 0;
        // Many small planes (split 8 or more, 16 MiB in all at most) are stored
        // cached by the 64x64 and 128x128 kernels, so the reduce kernel reads them
        // from the Infinity Cache: 256 x 256 x 32768 (16 planes of 256 KB) 14.06 ->
        // 13.69 us per call.  Two planes of 2 MB (128 x 4096 x 4096) measured 0.1 us
        // slower that way, and final C stores of unsplit 2048^3 0.4 us slower.
        if (p.splits >= 8 && args.c_split_stride * p.splits <= (16ull << 20)) args.flags |= T0G_FLAG_C_CACHED;
    } else {
        args.c = o.c;
        args.ldc = o.ldc;
        args.c_split_stride = o.c_split_stride;
        args.epilogue = o.chain;
        args.epi_scale = o.epi_scale;
        args.clamp_lo = o.clamp_lo;
        args.clamp_hi = o.clamp_hi;
        args.bias = o.bias;
        if (chain_has(o.chain, T0G_OP_BIAS_ADD)) args.flags |= T0G_FLAG_BIAS;
    }
    const uint64_t esize = reduce || !p.out_bf16 ? 4 : 2;
    if ((args.c & 15) == 0 && ((uint64_t)args.ldc * esize) % 16 == 0 && args.c_split_stride % 16 == 0)
        args.flags |= T0G_FLAG_C_VEC;
    *reduce_out = reduce;
}

// Launch the plan's GEMM kernel.  With splits > 1 and no caller-owned planes
// the partial planes go to `ws` and the reduce kernel produces C.
static int run_plan(t0g_device *dev, const GemmPlan &p, const GemmOperands &o, uint64_t ws,
                    bool allow_timeline = true) {
    T0gGemmArgs args;
    bool reduce = false;
    fill_gemm_args(p, o, ws, &args, &reduce, allow_timeline);
    hipFunction_t f = nullptr;
    int rc = get_function(dev, p.symbol, &f, (args.flags & T0G_FLAG_TIMELINE) != 0);
    if (rc) return rc;
    if (p.fused) {
        T0gGemmRedArgs ra;
        memset(&ra, 0, sizeof ra);
        ra.g = args;
        ra.partials = ws;
        ra.sync = dev->sk_sync;
        ra.tiles = p.tiles_m * p.tiles_n;
        ra.grid = ra.tiles * p.splits;
        ra.splits = p.splits;
        ra.spin_limit = kRedSpinLimit;
        ra.debug = g_sk_debug.load();
        dev->sk_stream = dev->stream;
        return launch(dev, f, p.tiles_m * p.tiles_n, p.splits, 1, p.wg, &ra, sizeof ra);
    }
    if (p.stream_k) {
        T0gGemmSkArgs sa;
        memset(&sa, 0, sizeof sa);
        sa.g = args;
        sa.partials = ws;
        sa.sync = dev->sk_sync;
        sa.grid = sk_grid(p, dev->num_cus);
        sa.iters_per_tile = p.sk_ipt;
        sa.spin_limit = g_sk_spin_limit.load();
        sa.debug = g_sk_debug.load();
        dev->sk_stream = dev->stream;
        return launch(dev, f, sa.grid, 1, 1, p.wg, &sa, sizeof sa);
    }
    rc = launch(dev, f, p.tiles_m * p.tiles_n, p.splits, 1, p.wg, &args, sizeof args);
    if (rc || !reduce) return rc;

    hipFunction_t fr = nullptr;
    rc = get_function(dev, p.out_bf16 ? "t0g_splitk_reduce_bf16" : "t0g_splitk_reduce_f32", &fr);
    if (rc) return rc;
    T0gReduceArgs r;
    memset(&r, 0, sizeof r);
    r.ws = ws;
    r.c = o.c;
    r.bias = o.bias;
    r.plane_elems = (uint64_t)o.m * o.n;
    r.m = o.m;
    r.n = o.n;
    r.ldw = o.n;
    r.ldc = o.ldc;
    r.splits = p.splits;
    r.epilogue = o.chain;
    r.epi_scale = o.epi_scale;
    r.clamp_lo = o.clamp_lo;
    r.clamp_hi = o.clamp_hi;
    if (chain_has(o.chain, T0G_OP_BIAS_ADD)) r.flags |= T0G_REDUCE_BIAS;
    const uint64_t out_esize = p.out_bf16 ? 2 : 4;
    // Large outputs (2^21 elements or more) take the wave-contiguous form, one grid
    // step per wave: the MLP's 1024 x 4096 x 11008 split 4 (GEMM + reduce) went from
    // 88.5 to 87.2 us against the earlier 8-columns-per-thread form.  Small outputs
    // keep 4 columns per thread with 8 planes in flight and 64-thread blocks: the
    // 8-column form had taken 256 x 256 from 3.9 to 6.6 us (too few loads in
    // flight to cover latency).
    const bool vec4 = (ws & 15) == 0 && (o.n & 3) == 0 && (o.c & (4 * out_esize - 1)) == 0 &&
                      ((uint64_t)o.ldc * out_esize) % (4 * out_esize) == 0;
    const bool wave = vec4 && (uint64_t)o.m * o.n >= (1ull << 21);
    const bool vec = vec4 && !wave && (uint64_t)o.m * (o.n / 4) < (1ull << 31);
    if (wave) r.flags |= T0G_REDUCE_WAVE;
    if (vec) r.flags |= T0G_REDUCE_VEC;
    const uint64_t total = (wave || vec) ? (uint64_t)o.m * (o.n / 4) : (uint64_t)o.m * o.n;
    // 4-wide outputs of fewer than 256 full blocks run 64-thread blocks, so every CU
    // shares the plane reads (256 x 256: 64 CUs -> 256)
    const uint32_t threads = (vec && total < 256u * 256u) ? 64u : 256u;
    uint64_t blocks = wave ? (total + 511) / 512 : (total + threads - 1) / threads;
    const uint64_t cap = wave ? (1u << 20) : 4096;
    if (blocks > cap) blocks = cap;
    r.grid_blocks = (uint32_t)blocks;
    return launch(dev, fr, (uint32_t)blocks, 1, 1, threads, &r, sizeof r);
}

static int resolve_desc(const t0g_gemm_desc *d, t0g_gemm_config *cfg, GemmPlan *plan, GemmOperands *o,
                        bool allow_fused = false) {
    if (!d) return fail(T0G_ERR_INVALID_ARG, "desc is NULL");
    if (d->transpose > T0G_TT) return fail(T0G_ERR_INVALID_ARG, "bad transpose %u", d->transpose);
    if (d->out_dtype > T0G_BF16) return fail(T0G_ERR_INVALID_ARG, "bad out_dtype %u", d->out_dtype);
    if (d->epilogue > T0G_EPI_BIAS_ADD_RELU) return fail(T0G_ERR_INVALID_ARG, "bad epilogue %u", d->epilogue);
    const uint32_t chain = d->epi_chain ? d->epi_chain : legacy_chain(d->epilogue);
    if (int rc0 = check_chain(chain)) return rc0;
    if (chain_has(chain, T0G_OP_BIAS_ADD) && !d->bias)
        return fail(T0G_ERR_INVALID_ARG, "bias epilogue without a bias pointer");
    const uint32_t t = d->transpose;
    o->a = d->a;
    o->b = d->b;
    o->c = d->c;
    o->bias = d->bias;
    o->m = d->m;
    o->n = d->n;
    o->k = d->k;
    o->lda = d->lda ? d->lda : (a_k_major(t) ? d->k : d->m);
    o->ldb = d->ldb ? d->ldb : (b_k_major(t) ? d->k : d->n);
    o->ldc = d->ldc ? d->ldc : d->n;
    o->chain = chain;
    o->epi_scale = d->epi_scale;
    o->clamp_lo = d->clamp_min;
    o->clamp_hi = d->clamp_max;
    o->c_split_stride = 0;
    if (o->ldc < o->n) return fail(T0G_ERR_INVALID_ARG, "ldc=%u < n=%u", o->ldc, o->n);
    if (a_k_major(t) ? o->lda < o->k : o->lda < o->m) return fail(T0G_ERR_INVALID_ARG, "lda=%u too small", o->lda);
    if (b_k_major(t) ? o->ldb < o->k : o->ldb < o->n) return fail(T0G_ERR_INVALID_ARG, "ldb=%u too small", o->ldb);
    int rc;
    if (d->config) {
        *cfg = *d->config;
    } else {
        select_config(d->m ? d->m : 1, d->k, d->n ? d->n : 1, cfg);
    }
    cfg->transpose = t;
    cfg->epilogue = d->epi_chain ? (uint32_t)T0G_EPI_STORE_F32 : d->epilogue;
    if ((rc = validate(cfg))) return rc;
    const uint32_t sk = d->split_k ? d->split_k : cfg_split(cfg);
    if (sk == T0G_STREAM_K && native_tile(cfg) != &kTiles[0])
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "stream-K needs the gfx950 256x256 tile");
    if (sk > kMaxSplitK && sk != T0G_STREAM_K)
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "split_k=%u > %u", sk, kMaxSplitK);
    const TileDef *tile = plan_tile(cfg, d->m, d->k, d->n, sk);
    const OperandPath path = operand_path(d->a, d->b, d->m, d->n, d->k, o->lda, o->ldb, t);
    if (path == OperandPath::Elementwise) {
        if ((rc = check_extent("A", a_k_major(t) ? d->m : d->k, o->lda))) return rc;
        if ((rc = check_extent("B", b_k_major(t) ? d->n : d->k, o->ldb))) return rc;
    }
    return make_plan(tile, t, d->out_dtype == T0G_BF16, path, ld_fits_256(t, o->lda, o->ldb), d->m, d->n, d->k, sk,
                     plan, allow_fused);
}

// Device workspace a plan needs: stream-K partial slots, fused split-K tile
// slots, or split-K planes.
static size_t plan_workspace(const GemmPlan &p, uint32_t m, uint32_t n, uint32_t num_cus) {
    if (p.stream_k) return (size_t)sk_grid(p, num_cus) * T0G_SK_SLOT_BYTES;
    if (p.fused) return (size_t)p.tiles_m * p.tiles_n * p.splits * p.tile->bm * p.tile->bn * 4;
    if (p.splits > 1) return (size_t)p.splits * m * n * 4;
    return 0;
}

}  // namespace t0g

using namespace t0g;

extern "C" {

int t0g_stream_k_timeouts(t0g_device *dev, uint32_t *count) {
    if (!dev || !count) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    *count = 0;
    if (!dev->sk_sync) return ok();
    if ((rc = wait_stream(dev))) return rc;
    hipError_t e = T0G_HIP(hipMemcpy(count, (const void *)(dev->sk_sync + 4 * T0G_SK_TIMEOUTS), 4,
                                     hipMemcpyDeviceToHost));
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy(stream-K timeouts)");
    return ok();
}

int t0g_debug_device_alloc_count(uint64_t *count) {
    if (!count) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *count = g_device_allocs.load();
    return ok();
}

int t0g_debug_fail_hip_call(int n) {
    if (n < 0) return fail(T0G_ERR_INVALID_ARG, "n must be >= 0");
    g_fail_countdown.store(n);
    return ok();
}

int t0g_set_wait_timeout_ms(uint32_t ms) {
    if (ms == 0) return fail(T0G_ERR_INVALID_ARG, "timeout must be > 0");
    g_wait_timeout_ms.store(ms);
    return ok();
}

int t0g_set_stream_k_spin_limit(uint32_t polls) {
    g_sk_spin_limit.store(polls);
    return ok();
}

int t0g_debug_stream_k_stall(int on) {
    g_sk_debug.store(on ? T0G_SK_DEBUG_STALL : 0u);
    return ok();
}

int t0g_set_split_k_mode(uint32_t mode) {
    if (mode > 2)
        return fail(T0G_ERR_INVALID_ARG, "split-K mode %u (0: reduce kernel, 1: in-kernel reduce, 2: auto)", mode);
    g_split_mode.store(mode);
    return ok();
}

int t0g_set_timeline(int on) {
    g_timeline.store(on ? 1 : 0);
    return ok();
}

// The module's t0g_timeline array (device address and size).
static int timeline_global(t0g_device *dev, hipDeviceptr_t *ptr, size_t *bytes) {
    int rc = load_timeline_module(dev);
    if (rc) return rc;
    hipError_t e = T0G_HIP(hipModuleGetGlobal(ptr, bytes, dev->module_tl, "t0g_timeline"));
    if (e != hipSuccess) return hip_fail(e, "hipModuleGetGlobal(t0g_timeline)");
    return T0G_OK;
}

int t0g_timeline_read(t0g_device *dev, uint64_t *out, size_t entries, size_t *written) {
    if (!dev || !written || (!out && entries)) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *written = 0;
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    hipDeviceptr_t p = nullptr;
    size_t bytes = 0;
    if ((rc = timeline_global(dev, &p, &bytes))) return rc;
    const size_t n = entries < bytes / 8 ? entries : bytes / 8;
    if ((rc = wait_stream(dev))) return rc;   // the recorded launches have finished
    hipError_t e = T0G_HIP(hipMemcpyAsync(out, p, n * 8, hipMemcpyDeviceToHost, dev->stream));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipMemcpy D2H (timeline)"));
    if ((rc = wait_stream(dev))) return rc;
    *written = n;
    return ok();
}

int t0g_timeline_clear(t0g_device *dev) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    hipDeviceptr_t p = nullptr;
    size_t bytes = 0;
    if ((rc = timeline_global(dev, &p, &bytes))) return rc;
    hipError_t e = T0G_HIP(hipMemsetAsync(p, 0, bytes, dev->stream));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipMemset (timeline)"));
    if ((rc = wait_stream(dev))) return rc;
    return ok();
}

int t0g_device_count(int *count) {
    if (!count) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    int n = 0;
    hipError_t e = T0G_HIP(hipGetDeviceCount(&n));
    if (e == hipErrorNoDevice || (e == hipSuccess && n == 0)) {
        *count = 0;
        return ok();
    }
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    *count = n;
    return ok();
}

int t0g_device_open(int ordinal, t0g_device **out) {
    if (!out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *out = nullptr;
    int n = 0;
    hipError_t e = T0G_HIP(hipGetDeviceCount(&n));
    if (e == hipErrorNoDevice || (e == hipSuccess && n == 0)) return fail(T0G_ERR_NO_DEVICE, "no HIP device");
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (ordinal < 0 || ordinal >= n) return fail(T0G_ERR_INVALID_ARG, "device %d out of range [0,%d)", ordinal, n);
    if ((e = T0G_HIP(hipSetDevice(ordinal))) != hipSuccess) return hip_fail(e, "hipSetDevice");
    hipDeviceProp_t prop;
    if ((e = T0G_HIP(hipGetDeviceProperties(&prop, ordinal))) != hipSuccess)
        return hip_fail(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(T0G_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only", ordinal,
                    prop.gcnArchName);
    std::unique_ptr<t0g_device> dev(new t0g_device);
    dev->ordinal = ordinal;
    dev->num_cus = prop.multiProcessorCount > 0 ? (uint32_t)prop.multiProcessorCount : kNumCUs;
    if ((e = T0G_HIP(hipStreamCreateWithFlags(&dev->own_stream, hipStreamNonBlocking))) != hipSuccess)
        return hip_fail(e, "hipStreamCreate");
    dev->stream = dev->own_stream;
    // set-up of t0g_gemm_noalloc's scratch, with this device current; a failure
    // only disables that entry point
    if (noalloc_scratch(ordinal, &dev->scratch) != T0G_OK) {
        dev->scratch = 0;
        dev->scratch_error = g_last_error;
    }
    if ((e = T0G_HIP(module_load(&dev->module, t0g_hsaco_begin))) != hipSuccess) {
        (void)hipStreamDestroy(dev->own_stream);
        return hip_fail(e, "hipModuleLoadData(gfx950 GEMM code object)");
    }
    *out = dev.release();
    return ok();
}

int t0g_device_close(t0g_device *dev) {
    if (!dev) return ok();
    (void)hipSetDevice(dev->ordinal);
    if (!dev->poisoned) (void)hipStreamSynchronize(dev->stream);
    if (dev->ws) (void)hipFree((void *)dev->ws);
    if (dev->conv) (void)hipFree((void *)dev->conv);
    if (dev->sk_sync) (void)hipFree((void *)dev->sk_sync);
    for (int i = 0; i < t0g_device::kSides; ++i) {
        if (dev->side[i]) {
            if (!dev->poisoned) (void)hipStreamSynchronize(dev->side[i]);
            (void)hipStreamDestroy(dev->side[i]);
        }
        if (dev->side_ws[i]) (void)hipFree((void *)dev->side_ws[i]);
        if (dev->join_ev[i]) (void)hipEventDestroy(dev->join_ev[i]);
    }
    if (dev->fork_ev) (void)hipEventDestroy(dev->fork_ev);
    for (const auto &a : dev->allocations) (void)hipFree((void *)a.first);
    for (const auto &c : dev->bf16_cache) (void)hipFree((void *)c.second.addr);
    for (const auto &bucket : dev->pool)
        for (uint64_t a : bucket.second) (void)hipFree((void *)a);
    for (hipModule_t m : dev->extra_modules) (void)hipModuleUnload(m);
    if (dev->module) (void)hipModuleUnload(dev->module);
    if (dev->module_tl) (void)hipModuleUnload(dev->module_tl);
    if (dev->order_event) (void)hipEventDestroy(dev->order_event);
    if (dev->own_stream) (void)hipStreamDestroy(dev->own_stream);
    delete dev;
    return ok();
}

// The handle's split-K workspace and the control block of its stream-K and
// in-kernel split-K launches are shared by everything it launches, so a
// switch of stream makes the new stream wait for the work issued on the old
// one: two launches of one handle never run at the same time.
int t0g_device_set_stream(t0g_device *dev, void *hip_stream) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    hipStream_t next = hip_stream ? (hipStream_t)hip_stream : dev->own_stream;
    if (next != dev->stream) {
        int rc = check_usable(dev);
        if (rc) return rc;
        hipError_t e = hipSuccess;
        if (!dev->order_event &&
            (e = T0G_HIP(hipEventCreateWithFlags(&dev->order_event, hipEventDisableTiming))) != hipSuccess)
            return hip_fail(e, "hipEventCreateWithFlags");
        if ((e = T0G_HIP(hipEventRecord(dev->order_event, dev->stream))) != hipSuccess)
            return hip_fail(e, "hipEventRecord");
        if ((e = T0G_HIP(hipStreamWaitEvent(next, dev->order_event, 0))) != hipSuccess)
            return hip_fail(e, "hipStreamWaitEvent");
        // A stream-K launch whose timeout count is not yet checked is now ordered
        // before everything on the new stream, so the new stream's waits check it.
        if (dev->sk_stream == dev->stream) dev->sk_stream = next;
    }
    dev->stream = next;
    return ok();
}

int t0g_device_get_stream(t0g_device *dev, void **hip_stream) {
    if (!dev || !hip_stream) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *hip_stream = (void *)dev->stream;
    return ok();
}

int t0g_device_is_poisoned(t0g_device *dev, int *poisoned) {
    if (!dev || !poisoned) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *poisoned = dev->poisoned ? 1 : 0;
    return ok();
}

// The pool's size key: whole 4 KiB pages, as BufferPool::alloc rounds.
static size_t pool_size(size_t bytes) { return ((bytes ? bytes : 1) + 4095) & ~(size_t)4095; }

static int alloc_locked(t0g_device *dev, size_t bytes, uint64_t *addr) {
    const size_t size = pool_size(bytes);
    auto it = dev->pool.find(size);
    if (it != dev->pool.end() && !it->second.empty()) {
        *addr = it->second.back();
        it->second.pop_back();
        dev->pool_bytes -= size;
        dev->pool_hits++;
    } else {
        void *p = nullptr;
        hipError_t e = T0G_HIP(dev_malloc(&p, size));
        if (e != hipSuccess) return hip_fail(e, "hipMalloc");
        *addr = (uint64_t)p;
        dev->pool_misses++;
    }
    dev->allocations[*addr] = size;
    return T0G_OK;
}

int t0g_alloc(t0g_device *dev, size_t bytes, uint64_t *addr) {
    if (!dev || !addr) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *addr = 0;
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    if ((rc = alloc_locked(dev, bytes, addr))) return rc;
    return ok();
}

int t0g_alloc_zero(t0g_device *dev, size_t bytes, uint64_t *addr) {
    int rc = t0g_alloc(dev, bytes, addr);
    if (rc) return rc;
    return t0g_memset(dev, *addr, 0, bytes);
}

int t0g_free(t0g_device *dev, uint64_t addr) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    if (!dev->allocations.count(addr))
        return fail(T0G_ERR_INVALID_ARG, "0x%llx is not a live buffer of t0g_alloc (never allocated, freed or recycled)",
                    (unsigned long long)addr);
    (void)hipSetDevice(dev->ordinal);
    if (!dev->poisoned) {
        int rc = wait_stream(dev);   // the reference frees without waiting (src/kfd/mod.rs:1057-1081)
        if (rc) return rc;
    }
    dev->allocations.erase(addr);
    hipError_t e = T0G_HIP(hipFree((void *)addr));
    if (e != hipSuccess) return hip_fail(e, "hipFree");
    return ok();
}

int t0g_recycle(t0g_device *dev, uint64_t addr) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    auto it = dev->allocations.find(addr);
    if (it == dev->allocations.end())
        return fail(T0G_ERR_INVALID_ARG, "0x%llx is not a live buffer of t0g_alloc (never allocated, freed or recycled)",
                    (unsigned long long)addr);
    const size_t size = it->second;
    dev->allocations.erase(it);
    dev->pool[size].push_back(addr);
    dev->pool_bytes += size;
    return ok();
}

int t0g_pool_clear(t0g_device *dev) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    (void)hipSetDevice(dev->ordinal);
    if (!dev->poisoned) {
        int rc = wait_stream(dev);   // recycled buffers may still be read by queued work
        if (rc) return rc;
    }
    hipError_t first = hipSuccess;
    for (auto &bucket : dev->pool)
        for (uint64_t a : bucket.second) {
            hipError_t e = T0G_HIP(hipFree((void *)a));
            if (e != hipSuccess && first == hipSuccess) first = e;
        }
    dev->pool.clear();
    dev->pool_bytes = 0;
    if (first != hipSuccess) return hip_fail(first, "hipFree(pooled buffer)");
    return ok();
}

int t0g_pool_stats(t0g_device *dev, t0g_pool_info *out) {
    if (!dev || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::lock_guard<std::mutex> lk(dev->mu);
    memset(out, 0, sizeof *out);
    out->cached_bytes = dev->pool_bytes;
    for (const auto &bucket : dev->pool) out->cached_buffers += bucket.second.size();
    out->live_buffers = dev->allocations.size();
    for (const auto &a : dev->allocations) out->live_bytes += a.second;
    out->hits = dev->pool_hits;
    out->misses = dev->pool_misses;
    return ok();
}

// alloc_f32 pads to whole 512-byte blocks, at least one (src/ignis/gpu_context.rs:449-454).
static size_t f32_bytes(size_t n) { return ((n * 4 > 512 ? n * 4 : 512) + 511) & ~(size_t)511; }

int t0g_alloc_f32(t0g_device *dev, size_t n, uint64_t *addr) {
    if (!dev || !addr) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *addr = 0;
    if (n > (SIZE_MAX - 1024) / 4) return fail(T0G_ERR_INVALID_ARG, "%zu floats overflow a size", n);
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    const size_t bytes = f32_bytes(n);
    if ((rc = alloc_locked(dev, bytes, addr))) return rc;
    // zeroed in stream order: work enqueued later on the device stream sees zeros
    hipError_t e = T0G_HIP(hipMemsetAsync((void *)*addr, 0, bytes, dev->stream));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipMemsetAsync"));
    return ok();
}

int t0g_write_f32(t0g_device *dev, uint64_t addr, const float *src, size_t n) {
    if (n > SIZE_MAX / 4) return fail(T0G_ERR_INVALID_ARG, "%zu floats overflow a size", n);
    return t0g_memcpy_h2d(dev, addr, src, n * 4);
}

int t0g_read_f32(t0g_device *dev, uint64_t addr, float *dst, size_t n) {
    if (n > SIZE_MAX / 4) return fail(T0G_ERR_INVALID_ARG, "%zu floats overflow a size", n);
    return t0g_memcpy_d2h(dev, dst, addr, n * 4);   // waits for the stream first, as read_f32 waits for idle
}

int t0g_upload_f32(t0g_device *dev, const float *src, size_t n, uint64_t *addr) {
    if (!addr || (!src && n)) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    int rc = t0g_alloc_f32(dev, n, addr);
    if (rc) return rc;
    if ((rc = t0g_write_f32(dev, *addr, src, n))) {
        (void)t0g_recycle(dev, *addr);
        *addr = 0;
        return rc;
    }
    return ok();
}

int t0g_memcpy_h2d(t0g_device *dev, uint64_t dst, const void *src, size_t bytes) {
    if (!dev || (!src && bytes)) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    hipError_t e = T0G_HIP(hipMemcpyAsync((void *)dst, src, bytes, hipMemcpyHostToDevice, dev->stream));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipMemcpy H2D"));
    if ((rc = wait_stream(dev))) return rc;
    return ok();
}

int t0g_memcpy_d2h(t0g_device *dev, void *dst, uint64_t src, size_t bytes) {
    if (!dev || (!dst && bytes)) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    hipError_t e = T0G_HIP(hipMemcpyAsync(dst, (const void *)src, bytes, hipMemcpyDeviceToHost, dev->stream));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipMemcpy D2H"));
    if ((rc = wait_stream(dev))) return rc;
    return ok();
}

int t0g_memset(t0g_device *dev, uint64_t dst, int value, size_t bytes) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    hipError_t e = T0G_HIP(hipMemsetAsync((void *)dst, value, bytes, dev->stream));
    if (e != hipSuccess) return poison(dev, hip_fail(e, "hipMemset"));
    if ((rc = wait_stream(dev))) return rc;
    return ok();
}

// chain != 0 (TileGemm only): an explicit epilogue chain; its arguments follow
// M in the kernargs.  Otherwise the chain is cfg->epilogue's.
static int kernel_get_common(t0g_device *dev, const t0g_gemm_config *cfg, KernelKind kind, uint32_t chain,
                             t0g_kernel **out) {
    if (!dev || !cfg || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *out = nullptr;
    int rc = validate(cfg);
    if (rc) return rc;
    if (cfg->split_k == T0G_STREAM_K)
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "stream-K configs run through t0g_gemm only");
    if ((rc = check_chain(chain))) return rc;
    if (chain && cfg->epilogue != T0G_EPI_STORE_F32)
        return fail(T0G_ERR_INVALID_ARG, "an epilogue chain replaces cfg->epilogue, which must be STORE_F32");
    if (cfg->transpose != T0G_NT && cfg->transpose != T0G_NN)
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "reference-layout kernels are NT or NN");
    char name[160], epi[64];
    t0g_config_name(cfg, name, sizeof name);
    t0g_epilogue_chain_name(chain, epi, sizeof epi);
    strncat(name, epi, sizeof name - strlen(name) - 1);
    std::string key = std::string(kind == KernelKind::TileGemm ? "tile:" : "gen:") + name;
    std::lock_guard<std::mutex> lk(dev->mu);
    auto it = dev->kernel_cache.find(key);
    if (it != dev->kernel_cache.end()) {
        *out = it->second;
        return ok();
    }
    std::unique_ptr<t0g_kernel> k(new t0g_kernel);
    k->kind = kind;
    k->cfg = *cfg;
    k->wg[0] = cfg->wg_size;
    k->lds = t0g_config_lds_total(cfg);
    k->chain = chain ? chain : legacy_chain(cfg->epilogue);
    if (kind == KernelKind::GemmGen)
        k->kernarg_size = cfg->epilogue != T0G_EPI_STORE_F32 ? 48 : 40;
    else
        k->kernarg_size = 44 + chain_kernarg_bytes(k->chain);
    k->name = name;
    *out = k.get();
    dev->kernel_cache.emplace(key, k.get());
    dev->kernels.push_back(std::move(k));
    return ok();
}

int t0g_kernel_get(t0g_device *dev, const t0g_gemm_config *cfg, t0g_kernel **out) {
    return kernel_get_common(dev, cfg, KernelKind::GemmGen, 0, out);
}

int t0g_tile_kernel_get(t0g_device *dev, const t0g_gemm_config *cfg, t0g_kernel **out) {
    return kernel_get_common(dev, cfg, KernelKind::TileGemm, 0, out);
}

int t0g_tile_kernel_get_epilogue(t0g_device *dev, const t0g_gemm_config *cfg, uint32_t chain, t0g_kernel **out) {
    return kernel_get_common(dev, cfg, KernelKind::TileGemm, chain, out);
}

int t0g_kernel_load(t0g_device *dev, const void *code_object, size_t size, const char *symbol,
                    const uint32_t workgroup_size[3], uint32_t lds_size, t0g_kernel **out) {
    if (!dev || !code_object || !symbol || !workgroup_size || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    *out = nullptr;
    // The argument size, LDS and largest workgroup come from the code object,
    // so a dispatch that does not fit the kernel is refused on the host.
    KernelMeta meta;
    int rc = read_kernel_meta(code_object, size, symbol, &meta);
    if (rc) return rc;
    uint64_t threads = 1;
    for (int i = 0; i < 3; i++) threads *= workgroup_size[i] ? workgroup_size[i] : 1;
    if (threads > meta.max_workgroup_size)
        return fail(T0G_ERR_INVALID_ARG, "workgroup of %llu threads; %s was built for at most %u",
                    (unsigned long long)threads, symbol, meta.max_workgroup_size);
    std::lock_guard<std::mutex> lk(dev->mu);
    if ((rc = check_usable(dev))) return rc;
    hipModule_t m = nullptr;
    hipError_t e = T0G_HIP(module_load(&m, code_object));
    if (e != hipSuccess) return hip_fail(e, "hipModuleLoadData");
    hipFunction_t f = nullptr;
    e = T0G_HIP(hipModuleGetFunction(&f, m, symbol));
    if (e != hipSuccess) {
        (void)hipModuleUnload(m);
        return hip_fail(e, "hipModuleGetFunction");
    }
    dev->extra_modules.push_back(m);
    std::unique_ptr<t0g_kernel> k(new t0g_kernel);
    k->kind = KernelKind::Raw;
    memset(&k->cfg, 0, sizeof k->cfg);
    k->fn = f;
    for (int i = 0; i < 3; i++) k->wg[i] = workgroup_size[i] ? workgroup_size[i] : 1;
    k->lds = lds_size > meta.group_segment_size ? lds_size : meta.group_segment_size;
    k->dyn_lds = lds_size > meta.group_segment_size ? lds_size - meta.group_segment_size : 0;
    k->kernarg_size = meta.explicit_args_size;
    k->name = symbol;
    *out = k.get();
    dev->kernels.push_back(std::move(k));
    return ok();
}

int t0g_kernel_info(const t0g_kernel *kernel, uint32_t *wg_size, uint32_t *lds_size, uint32_t *kernarg_size,
                    char *name, size_t name_len) {
    if (!kernel) return fail(T0G_ERR_INVALID_ARG, "kernel is NULL");
    if (wg_size) *wg_size = kernel->wg[0] * kernel->wg[1] * kernel->wg[2];
    if (lds_size) *lds_size = kernel->lds;
    if (kernarg_size) *kernarg_size = kernel->kernarg_size;
    if (name && name_len) {
        snprintf(name, name_len, "%s", kernel->name.c_str());
    }
    return ok();
}

static uint32_t rd_u32(const uint8_t *p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}
static uint64_t rd_u64(const uint8_t *p) {
    uint64_t v;
    memcpy(&v, p, 8);
    return v;
}

static int gemm_locked(t0g_device *dev, const t0g_gemm_desc *d, bool allow_fused = true);

// A reference-space config (an RDNA3 tile): the problem is the one the
// reference's kernel for cfg computes from this grid and these kernargs, and
// the gfx950 tile the model picks computes it.  The grid covers tiles_m row
// blocks of tile_m and tiles_n column blocks of tile_n * n_col_passes
// (compute_grid, src/t0/gemm_gen.rs:286-309); rows stop at M (tile_ir's
// boundary masking, src/t0/tile_ir.rs:2374-2481; gemm_gen's M is the grid's)
// and columns at N, which is also Y's row pitch.  o: the decoded kernargs
// (m = M, n = N, ldc = N).
static int dispatch_ref(t0g_device *dev, const t0g_kernel *kn, uint32_t tiles_m, uint32_t tiles_n, uint32_t sk,
                        GemmOperands o, uint32_t y_split_stride) {
    const t0g_gemm_config &cfg = kn->cfg;
    const uint64_t rows = std::min<uint64_t>(o.m, (uint64_t)tiles_m * cfg.tile_m);
    const uint64_t cols = std::min<uint64_t>(o.n, (uint64_t)tiles_n * cfg.tile_n * cfg.n_col_passes);
    o.m = (uint32_t)rows;
    o.n = (uint32_t)cols;
    if (sk > 1 && y_split_stride != 0) {
        // Caller-owned planes, summed by the caller in plane order
        // (examples/test_gemm_correctness.rs:190-207): plane s at Y + s * y_split_stride
        // holds K slice [s K/sk, (s+1) K/sk), as the reference's kernel cuts it
        // (k_end = K >> split_k_shift, k_start = split id * k_end; src/t0/gemm_gen.rs:728-752).
        if (o.k % (cfg.tile_k * sk) != 0)
            return fail(T0G_ERR_UNSUPPORTED_CONFIG, "K=%u must be a multiple of tile_k*split_k=%u", o.k,
                        cfg.tile_k * sk);
        if (y_split_stride % 4 != 0)
            return fail(T0G_ERR_INVALID_ARG, "y_split_stride=%u is not a whole number of f32", y_split_stride);
        if (rows && cols && (uint64_t)y_split_stride / 4 < (rows - 1) * o.ldc + cols)
            return fail(T0G_ERR_INVALID_ARG, "y_split_stride=%u bytes cannot hold a %llux%llu plane of pitch %u",
                        y_split_stride, (unsigned long long)rows, (unsigned long long)cols, o.ldc);
        if (o.chain != 0)
            return fail(T0G_ERR_UNSUPPORTED_CONFIG,
                        "an epilogue on caller-owned split-K planes would be applied to every partial sum; "
                        "leave y_split_stride 0 (tile ABI) for a reduced, epilogued Y");
        if (rows == 0 || cols == 0) return ok();
        const TileDef *tile = plan_tile(&cfg, o.m, o.k, o.n, sk);
        const OperandPath path = operand_path(o.a, o.b, o.m, o.n, o.k, o.lda, o.ldb, cfg.transpose);
        int rc;
        if (path == OperandPath::Elementwise) {
            if ((rc = check_extent("X", o.m, o.lda))) return rc;
            if ((rc = check_extent("WT", cfg.transpose == T0G_NN ? o.k : o.n, o.ldb))) return rc;
        }
        GemmPlan p;
        if ((rc = make_plan(tile, cfg.transpose, false, path, ld_fits_256(cfg.transpose, o.lda, o.ldb), o.m, o.n, o.k,
                            sk, &p, false, true)))
            return rc;
        o.c_split_stride = y_split_stride;
        return run_plan(dev, p, o, 0);
    }
    // One output (no split, or tile_ir's y_split_stride 0, whose planes the
    // library keeps): the whole auto-selected plan, split and workspace included.
    if (rows == 0 || cols == 0) return ok();
    t0g_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = o.a;
    d.b = o.b;
    d.c = o.c;
    d.bias = o.bias;
    d.m = o.m;
    d.n = o.n;
    d.k = o.k;
    d.lda = o.lda;
    d.ldb = o.ldb;
    d.ldc = o.ldc;
    d.transpose = cfg.transpose;
    d.out_dtype = T0G_F32;
    d.epi_chain = o.chain;
    d.epi_scale = o.epi_scale;
    d.clamp_min = o.clamp_lo;
    d.clamp_max = o.clamp_hi;
    return gemm_locked(dev, &d);
}

// Interpret reference-layout kernargs + a thread grid for a GEMM kernel handle
// and launch the equivalent gfx950 GEMM (see t0g_kernel_get / t0g_tile_kernel_get).
static int dispatch_gemm(t0g_device *dev, const t0g_kernel *kn, const uint32_t grid[3], const uint8_t *ka,
                         size_t len) {
    const t0g_gemm_config &cfg = kn->cfg;
    if (len < kn->kernarg_size)
        return fail(T0G_ERR_INVALID_ARG, "kernargs are %zu bytes, %s needs %u", len, kn->name.c_str(),
                    kn->kernarg_size);
    const uint32_t wg = cfg.wg_size;
    if (grid[0] % wg != 0) return fail(T0G_ERR_INVALID_ARG, "grid x=%u is not a multiple of wg_size %u", grid[0], wg);
    if (grid[2] != 1) return fail(T0G_ERR_INVALID_ARG, "grid z must be 1 (got %u)", grid[2]);
    const uint32_t sk = cfg_split(&cfg);
    const uint32_t gx = grid[0] / wg, gy = grid[1];
    if (gy % sk != 0) return fail(T0G_ERR_INVALID_ARG, "grid y=%u is not a multiple of split_k %u", gy, sk);
    const uint32_t tiles_m = cfg.swap_grid ? gy / sk : gx;
    const uint32_t tiles_n = cfg.swap_grid ? gx : gy / sk;
    GemmOperands o;
    memset(&o, 0, sizeof o);
    o.a = rd_u64(ka + 0);
    o.b = rd_u64(ka + 8);
    o.c = rd_u64(ka + 16);
    o.k = rd_u32(ka + 24);
    o.n = rd_u32(ka + 28);
    const uint32_t y_split_stride = rd_u32(ka + 36);
    if (kn->kind == KernelKind::TileGemm) {
        // lower_gemm's argument order after M: bias, epi_scale, clamp_min, clamp_max
        // (src/t0/tile_ir.rs:661-683), each present only if the chain uses it.
        o.m = rd_u32(ka + 40);
        size_t off = 44;
        if (chain_has(kn->chain, T0G_OP_BIAS_ADD)) {
            o.bias = rd_u64(ka + off);
            off += 8;
        }
        if (chain_has(kn->chain, T0G_OP_SCALE)) {
            memcpy(&o.epi_scale, ka + off, 4);
            off += 4;
        }
        if (chain_has(kn->chain, T0G_OP_CLAMP)) {
            memcpy(&o.clamp_lo, ka + off, 4);
            memcpy(&o.clamp_hi, ka + off + 4, 4);
        }
    } else if (cfg.epilogue != T0G_EPI_STORE_F32) {
        o.bias = rd_u64(ka + 40);
    }
    if (o.m == 0) o.m = tiles_m * cfg.tile_m;   // gemm_gen kernargs carry no M: the grid covers it exactly
    o.chain = kn->chain;
    o.lda = o.k;
    o.ldb = cfg.transpose == T0G_NN ? o.n : o.k;
    o.ldc = o.n;
    if (!native_tile(&cfg)) return dispatch_ref(dev, kn, tiles_m, tiles_n, sk, o, y_split_stride);
    // tile_ir split-K: build_kernargs_m always writes y_split_stride = 0 and
    // leaves the planes to the caller (src/t0/tile_ir.rs:3154-3157, 3179), so a
    // stride of 0 here means the library keeps the fp32 planes in its own
    // workspace and reduces them into Y in plane order, epilogue chain last.
    const bool lib_planes = kn->kind == KernelKind::TileGemm && sk > 1 && y_split_stride == 0;
    if (sk > 1 && !lib_planes) {
        if (y_split_stride == 0)
            return fail(T0G_ERR_INVALID_ARG,
                        "split_k=%u with y_split_stride=0 would make every K slice store to the same Y", sk);
        if (o.k % (sk * kTileK) != 0)
            return fail(T0G_ERR_UNSUPPORTED_CONFIG, "K=%u must be a multiple of tile_k*split_k=%u", o.k, sk * kTileK);
        if ((uint64_t)y_split_stride < (uint64_t)o.m * o.n * 4)
            return fail(T0G_ERR_INVALID_ARG, "y_split_stride=%u smaller than one M*N f32 plane", y_split_stride);
        // the reference's kernel would apply the epilogue to every partial plane
        // (bias added split_k times); the planes stay plain partial sums here
        if (o.chain != 0)
            return fail(T0G_ERR_UNSUPPORTED_CONFIG,
                        "an epilogue on caller-owned split-K planes would be applied to every partial sum; "
                        "leave y_split_stride 0 (tile ABI) for a reduced, epilogued Y");
        o.c_split_stride = y_split_stride;
    }
    int rc;
    const TileDef *tile = find_tile(cfg.tile_m, cfg.tile_n, cfg.tile_k, cfg.wg_size);
    const OperandPath path = operand_path(o.a, o.b, o.m, o.n, o.k, o.lda, o.ldb, cfg.transpose);
    if (path == OperandPath::Elementwise) {
        if ((rc = check_extent("X", o.m, o.lda))) return rc;
        if ((rc = check_extent("WT", cfg.transpose == T0G_NN ? o.k : o.n, o.ldb))) return rc;
    }
    GemmPlan p;
    if ((rc = make_plan(tile, cfg.transpose, false, path, ld_fits_256(cfg.transpose, o.lda, o.ldb), o.m, o.n, o.k, sk,
                        &p, lib_planes)))
        return rc;
    if (p.tile != tile)   // another tile than the caller's grid was built for: refuse rather than re-grid
        return fail(T0G_ERR_UNSUPPORTED_CONFIG,
                    "tile %ux%u cannot take these operands (rows must be 16-byte aligned with K %% 8 == 0; "
                    "operands of 2^30 elements or more need the 256x256 tile)",
                    cfg.tile_m, cfg.tile_n);
    if (lib_planes) {
        // the plan's own split of K (any K); the grid must cover the whole output,
        // since the reduce reads every element of the planes
        if (tiles_m < p.tiles_m || tiles_n < p.tiles_n)
            return fail(T0G_ERR_INVALID_ARG, "grid covers %ux%u tiles; split-K over %ux%u needs %ux%u", tiles_m,
                        tiles_n, o.m, o.n, p.tiles_m, p.tiles_n);
        if (o.m == 0 || o.n == 0) return ok();
        uint64_t ws = 0;
        if (p.fused && (rc = ensure_sk_sync(dev))) return rc;
        if (p.splits > 1) {
            if ((rc = ensure_workspace(dev, plan_workspace(p, o.m, o.n, dev->num_cus)))) return rc;
            ws = dev->ws;
        }
        return run_plan(dev, p, o, ws);
    }
    p.tiles_m = tiles_m;
    p.tiles_n = tiles_n;
    p.splits = sk;
    p.k_per_split = sk > 1 ? o.k / sk : (o.k ? o.k : kTileK);
    if (tiles_m == 0 || tiles_n == 0) return ok();
    return run_plan(dev, p, o, 0);
}

static int dispatch_common(t0g_device *dev, const t0g_kernel *kernel, const uint32_t grid[3], const void *ka,
                           size_t len, bool sync) {
    if (!dev || !kernel || !grid || (!ka && len)) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    if (kernel->kind == KernelKind::Raw) {
        const uint32_t bx = kernel->wg[0], by = kernel->wg[1], bz = kernel->wg[2];
        if (grid[0] % bx || grid[1] % by || grid[2] % bz)
            return fail(T0G_ERR_INVALID_ARG, "grid (%u,%u,%u) is not a multiple of the workgroup", grid[0], grid[1],
                        grid[2]);
        if (len != kernel->kernarg_size)
            return fail(T0G_ERR_INVALID_ARG, "kernargs are %zu bytes; %s takes exactly %u (code object metadata)", len,
                        kernel->name.c_str(), kernel->kernarg_size);
        std::vector<uint8_t> buf((const uint8_t *)ka, (const uint8_t *)ka + len);
        size_t sz = len;
        void *extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, buf.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                         HIP_LAUNCH_PARAM_END};
        hipError_t e = T0G_HIP(hipModuleLaunchKernel(kernel->fn, grid[0] / bx, grid[1] / by, grid[2] / bz, bx, by, bz,
                                                     kernel->dyn_lds, dev->stream, nullptr, extra));
        if (e != hipSuccess) return poison(dev, hip_fail(e, "hipModuleLaunchKernel"));
    } else {
        rc = dispatch_gemm(dev, kernel, grid, (const uint8_t *)ka, len);
        if (rc) return rc;
    }
    if (sync && (rc = wait_stream(dev))) return rc;
    return ok();
}

int t0g_dispatch(t0g_device *dev, const t0g_kernel *kernel, const uint32_t grid_threads[3], const void *kernargs,
                 size_t kernargs_len) {
    return dispatch_common(dev, kernel, grid_threads, kernargs, kernargs_len, true);
}

int t0g_dispatch_async(t0g_device *dev, const t0g_kernel *kernel, const uint32_t grid_threads[3],
                       const void *kernargs, size_t kernargs_len) {
    return dispatch_common(dev, kernel, grid_threads, kernargs, kernargs_len, false);
}

int t0g_wait_idle(t0g_device *dev) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    if ((rc = wait_stream(dev))) return rc;
    return ok();
}

int t0g_gemm_workspace_size(const t0g_gemm_desc *d, size_t *bytes) {
    if (!bytes) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    t0g_gemm_config cfg;
    GemmPlan p;
    GemmOperands o;
    int rc = resolve_desc(d, &cfg, &p, &o, true);
    if (rc) return rc;
    *bytes = plan_workspace(p, d->m, d->n, kNumCUs);
    return ok();
}

int t0g_gemm_kernel_name(const t0g_gemm_desc *d, char *buf, size_t len) {
    if (!buf || !len) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    t0g_gemm_config cfg;
    GemmPlan p;
    GemmOperands o;
    int rc = resolve_desc(d, &cfg, &p, &o, true);
    if (rc) return rc;
    snprintf(buf, len, "%s", p.symbol.c_str());
    return ok();
}

int t0g_gemm_compile(const t0g_gemm_desc *d, t0g_compiled_kernel *out) {
    if (!d || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    memset(out, 0, sizeof *out);
    t0g_gemm_config cfg;
    GemmPlan p;
    GemmOperands o;
    int rc = resolve_desc(d, &cfg, &p, &o);
    if (rc) return rc;
    // Planes go into C, so C's size must not depend on a split the caller did not
    // ask for: a split comes only from desc->split_k or an explicit config.  An
    // auto-selected split, or stream-K (its launches need the device's flag
    // words), compiles as the same tile without the split.
    const bool asked = d->split_k > 1 || (d->split_k == 0 && d->config && cfg_split(d->config) > 1 &&
                                          d->config->split_k != T0G_STREAM_K);
    if (p.stream_k || (p.splits > 1 && !asked)) {
        t0g_gemm_config dp = cfg;
        dp.split_k = 0;
        t0g_gemm_desc d2 = *d;
        d2.config = &dp;
        d2.split_k = 1;
        if ((rc = resolve_desc(&d2, &cfg, &p, &o))) return rc;
    }
    if (p.splits > 1) {
        if (d->out_dtype != T0G_F32)
            return fail(T0G_ERR_UNSUPPORTED_CONFIG, "a split-K kernel writes fp32 planes: out_dtype must be F32");
        if (o.chain)
            return fail(T0G_ERR_UNSUPPORTED_CONFIG, "an epilogue cannot be applied to split-K partial planes");
        o.c_split_stride = (uint64_t)o.m * o.ldc * 4;
    }
    if ((uint64_t)p.tiles_m * p.tiles_n * p.wg > 0xFFFFFFFFull)
        return fail(T0G_ERR_INVALID_ARG, "%u x %u tiles: the grid in threads exceeds 32 bits", p.tiles_m, p.tiles_n);
    T0gGemmArgs args;
    bool reduce = false;
    fill_gemm_args(p, o, 0, &args, &reduce);
    const size_t co_size = (size_t)(t0g_hsaco_end - t0g_hsaco_begin);
    KernelMeta meta;
    if ((rc = read_kernel_meta(t0g_hsaco_begin, co_size, p.symbol.c_str(), &meta))) return rc;
    if (meta.explicit_args_size != sizeof args)
        return fail(T0G_ERR_HIP, "%s takes %u argument bytes, this library builds %zu", p.symbol.c_str(),
                    meta.explicit_args_size, sizeof args);
    out->code_object = t0g_hsaco_begin;
    out->code_object_size = co_size;
    snprintf(out->name, sizeof out->name, "%s", p.symbol.c_str());
    out->workgroup_size = p.wg;
    out->lds_size = meta.group_segment_size;
    out->kernarg_size = (uint32_t)sizeof args;
    out->grid[0] = p.tiles_m * p.tiles_n * p.wg;
    out->grid[1] = p.splits;
    out->grid[2] = 1;
    out->splits = p.splits;
    memcpy(out->kernargs, &args, sizeof args);
    return ok();
}

// t0g_gemm with dev->mu held.  allow_fused = false: split-K with the separate
// reduce kernel (launches that may overlap another on this device).
static int gemm_locked(t0g_device *dev, const t0g_gemm_desc *d, bool allow_fused) {
    t0g_gemm_config cfg;
    GemmPlan p;
    GemmOperands o;
    int rc = resolve_desc(d, &cfg, &p, &o, allow_fused);
    if (rc) return rc;
    if ((rc = check_usable(dev))) return rc;
    if (d->m == 0 || d->n == 0) return ok();
    uint64_t ws = 0;
    if ((p.stream_k || p.fused) && (rc = ensure_sk_sync(dev))) return rc;
    if (p.splits > 1 || p.stream_k) {
        const size_t need = plan_workspace(p, d->m, d->n, dev->num_cus);
        if (d->workspace) {
            if (d->workspace_bytes < need)
                return fail(T0G_ERR_INVALID_ARG, "workspace of %llu bytes, split-K needs %zu",
                            (unsigned long long)d->workspace_bytes, need);
            ws = d->workspace;
        } else {
            if ((rc = ensure_workspace(dev, need))) return rc;
            ws = dev->ws;
        }
    }
    if ((rc = run_plan(dev, p, o, ws))) return rc;
    return ok();
}

int t0g_gemm(t0g_device *dev, const t0g_gemm_desc *d) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    return gemm_locked(dev, d);
}

// t0g_gemm without allocating: the split-K planes go to the caller's workspace or
// to the device's static scratch array; stream-K configs take the data-parallel
// schedule of the same tile (their flag words would be allocated).  No hipMalloc,
// hipFree or other allocating call is made here.
int t0g_gemm_noalloc(t0g_device *dev, const t0g_gemm_desc *d) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    if (!dev->scratch)
        return fail(T0G_ERR_HIP, "no-allocation scratch unavailable on device %d: %s", dev->ordinal,
                    dev->scratch_error.c_str());
    t0g_gemm_config cfg;
    GemmPlan p;
    GemmOperands o;
    int rc = resolve_desc(d, &cfg, &p, &o);
    if (rc) return rc;
    if (p.stream_k) {
        t0g_gemm_config dp = cfg;
        dp.split_k = 0;
        t0g_gemm_desc d2 = *d;
        d2.config = &dp;
        d2.split_k = 1;
        if ((rc = resolve_desc(&d2, &cfg, &p, &o))) return rc;
    }
    if ((rc = check_usable(dev))) return rc;
    if (d->m == 0 || d->n == 0) return ok();
    uint64_t ws = 0;
    if (p.splits > 1) {
        const size_t need = (size_t)p.splits * d->m * d->n * 4;
        if (d->workspace) {
            if (d->workspace_bytes < need)
                return fail(T0G_ERR_INVALID_ARG, "workspace of %llu bytes, split-K needs %zu",
                            (unsigned long long)d->workspace_bytes, need);
            ws = d->workspace;
        } else {
            if (need > (size_t)T0G_NOALLOC_SCRATCH_BYTES)
                return fail(T0G_ERR_INVALID_ARG,
                            "split-K of %ux%u over %u planes needs %zu bytes of scratch; t0g_gemm_noalloc has %u "
                            "(ask for fewer splits with desc.split_k, or pass a workspace)",
                            d->m, d->n, p.splits, need, (unsigned)T0G_NOALLOC_SCRATCH_BYTES);
            ws = dev->scratch;
        }
    }
    // never the timeline build: its first use loads a code object, which allocates
    if (ws != 0 && ws == dev->scratch)
        rc = noalloc_scratch_use(dev->ordinal, dev->stream, [&] { return run_plan(dev, p, o, ws, false); });
    else
        rc = run_plan(dev, p, o, ws, false);
    if (rc) return rc;
    return ok();
}

// Independent GEMMs, round-robin over the device stream and the side streams.
// Stream-K and the in-kernel split-K reduction keep one control block per
// device, so grouped GEMMs take the data-parallel schedule and the separate
// reduce kernel instead (such launches must not overlap).
int t0g_gemm_group(t0g_device *dev, const t0g_gemm_desc *descs, uint32_t n) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    if (n && !descs) return fail(T0G_ERR_INVALID_ARG, "descs is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    if (n <= 1) return n ? gemm_locked(dev, descs) : ok();
    const int sides = (int)std::min<uint32_t>(n - 1, t0g_device::kSides);
    hipError_t e;
    for (int i = 0; i < sides; ++i) {
        if (!dev->side[i] && (e = T0G_HIP(hipStreamCreateWithFlags(&dev->side[i], hipStreamNonBlocking))) != hipSuccess) {
            dev->side[i] = nullptr;
            return hip_fail(e, "hipStreamCreate(side stream)");
        }
        if (!dev->join_ev[i] &&
            (e = T0G_HIP(hipEventCreateWithFlags(&dev->join_ev[i], hipEventDisableTiming))) != hipSuccess) {
            dev->join_ev[i] = nullptr;
            return hip_fail(e, "hipEventCreate(join)");
        }
    }
    if (!dev->fork_ev && (e = T0G_HIP(hipEventCreateWithFlags(&dev->fork_ev, hipEventDisableTiming))) != hipSuccess) {
        dev->fork_ev = nullptr;
        return hip_fail(e, "hipEventCreate(fork)");
    }
    // validate every descriptor before anything is enqueued
    for (uint32_t i = 0; i < n; ++i) {
        t0g_gemm_config cfg;
        GemmPlan p;
        GemmOperands o;
        if ((rc = resolve_desc(&descs[i], &cfg, &p, &o))) return fail(rc, "descs[%u]: %s", i, g_last_error.c_str());
    }
    if ((e = T0G_HIP(hipEventRecord(dev->fork_ev, dev->stream))) != hipSuccess)
        return poison(dev, hip_fail(e, "hipEventRecord(fork)"));
    for (int i = 0; i < sides; ++i)
        if ((e = T0G_HIP(hipStreamWaitEvent(dev->side[i], dev->fork_ev, 0))) != hipSuccess)
            return poison(dev, hip_fail(e, "hipStreamWaitEvent(fork)"));
    // A side stream's GEMM runs with that stream's workspace swapped into
    // dev->ws, and the slots are swapped back afterwards, so a workspace that a
    // GEMM grows (freeing the old one) is kept by whichever stream grew it.
    auto swap_side = [dev](int s) {
        std::swap(dev->stream, dev->side[s]);
        std::swap(dev->ws, dev->side_ws[s]);
        std::swap(dev->ws_bytes, dev->side_ws_bytes[s]);
    };
    int first_rc = T0G_OK;
    for (uint32_t i = 0; i < n && !first_rc; ++i) {
        t0g_gemm_desc d = descs[i];
        t0g_gemm_config cfg;
        GemmPlan p;
        GemmOperands o;
        (void)resolve_desc(&d, &cfg, &p, &o);
        t0g_gemm_config dp_cfg;
        if (p.stream_k) {   // the same tile, data-parallel
            dp_cfg = cfg;
            dp_cfg.split_k = 0;
            d.config = &dp_cfg;
            d.split_k = 1;
        }
        const int s = (int)(i % (uint32_t)(sides + 1)) - 1;   // -1: the device stream
        if (s >= 0) swap_side(s);
        first_rc = gemm_locked(dev, &d, false);   // concurrent launches: no shared control block
        if (s >= 0) swap_side(s);
    }
    // join whatever was enqueued, also after a failure
    for (int i = 0; i < sides; ++i) {
        if ((e = T0G_HIP(hipEventRecord(dev->join_ev[i], dev->side[i]))) != hipSuccess ||
            (e = T0G_HIP(hipStreamWaitEvent(dev->stream, dev->join_ev[i], 0))) != hipSuccess)
            return poison(dev, hip_fail(e, "join of a side stream"));
    }
    return first_rc ? first_rc : ok();
}

}  // extern "C"

namespace t0g {

// Device time of `iters` back-to-back t0g_gemm launches of d (after `warmup`
// untimed ones): one HIP event between consecutive launches on the device
// stream, so each duration covers one whole GEMM (partials and reduce).
int time_gemm(t0g_device *dev, const t0g_gemm_desc *d, uint32_t warmup, uint32_t iters, std::vector<double> *ms) {
    if (!dev || !d || !ms || iters == 0) return fail(T0G_ERR_INVALID_ARG, "time_gemm: bad argument");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    std::vector<hipEvent_t> ev(iters + 1, nullptr);
    auto destroy = [&ev]() {
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
    };
    for (hipEvent_t &e : ev) {
        hipError_t he = T0G_HIP(hipEventCreate(&e));
        if (he != hipSuccess) {
            e = nullptr;
            destroy();
            return hip_fail(he, "hipEventCreate");
        }
    }
    for (uint32_t i = 0; i < warmup && !rc; ++i) rc = gemm_locked(dev, d);
    for (uint32_t i = 0; i <= iters && !rc; ++i) {
        hipError_t he = T0G_HIP(hipEventRecord(ev[i], dev->stream));
        if (he != hipSuccess) rc = poison(dev, hip_fail(he, "hipEventRecord"));
        else if (i < iters) rc = gemm_locked(dev, d);
    }
    if (!rc) rc = wait_stream(dev);
    if (!rc) {
        ms->assign(iters, 0.0);
        for (uint32_t i = 0; i < iters && !rc; ++i) {
            float t = 0.f;
            hipError_t he = T0G_HIP(hipEventElapsedTime(&t, ev[i], ev[i + 1]));
            if (he != hipSuccess) rc = hip_fail(he, "hipEventElapsedTime");
            (*ms)[i] = t;
        }
    }
    destroy();
    return rc;
}

}  // namespace t0g

extern "C" {

// ---- Ignis bf16_matmul caller path ------------------------------------------

static int convert_locked(t0g_device *dev, uint64_t src, uint64_t dst, uint64_t n) {
    if (n == 0) return T0G_OK;
    hipFunction_t f = nullptr;
    int rc = get_function(dev, "t0g_f32_to_bf16_rne", &f);
    if (rc) return rc;
    T0gConvertArgs a;
    memset(&a, 0, sizeof a);
    a.src = src;
    a.dst = dst;
    a.n = n;
    const bool vec = (src & 15) == 0 && (dst & 7) == 0 && (n & 3) == 0;
    if (vec) a.flags |= T0G_CONVERT_VEC;
    // vector form: 512 items of 4 elements per workgroup and grid step, one step
    // per wave up to 2^20 workgroups; element form: 256 elements, 8192 workgroups
    uint64_t blocks = vec ? (n / 4 + 511) / 512 : (n + 255) / 256;
    const uint64_t cap = vec ? (1u << 20) : 8192;
    if (blocks > cap) blocks = cap;
    a.grid_blocks = (uint32_t)blocks;
    return launch(dev, f, (uint32_t)blocks, 1, 1, 256, &a, sizeof a);
}

static int ensure_conv(t0g_device *dev, size_t bytes) {
    if (dev->conv_bytes >= bytes) return T0G_OK;
    if (dev->conv) {
        hipError_t e = T0G_HIP(hipFree((void *)dev->conv));   // waits for work using it
        dev->conv = 0;
        dev->conv_bytes = 0;
        if (e != hipSuccess) return poison(dev, hip_fail(e, "hipFree(conversion scratch)"));
    }
    void *p = nullptr;
    hipError_t e = T0G_HIP(dev_malloc(&p, bytes));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(conversion scratch)");
    dev->conv = (uint64_t)p;
    dev->conv_bytes = bytes;
    return T0G_OK;
}

static size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Convert the f32 operands that need it into the scratch buffer, then run one
// GEMM with f32 output.  a_elems / b_elems: elements of A and B (0: already bf16).
static int matmul_common(t0g_device *dev, uint64_t a_f32, size_t a_elems, uint64_t b, size_t b_elems,
                         uint64_t c, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    if (!a_f32 || !b || !c) return fail(T0G_ERR_INVALID_ARG, "NULL operand");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    const size_t a_bytes = round256(a_elems * 2), b_bytes = round256(b_elems * 2);
    if ((rc = ensure_conv(dev, a_bytes + b_bytes + 256))) return rc;
    const uint64_t a16 = dev->conv, b16 = b_elems ? dev->conv + a_bytes : b;
    if ((rc = convert_locked(dev, a_f32, a16, a_elems))) return rc;
    if (b_elems && (rc = convert_locked(dev, b, b16, b_elems))) return rc;
    t0g_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = a16;
    d.b = b16;
    d.c = c;
    d.m = m;
    d.n = n;
    d.k = k;
    d.transpose = transpose;
    d.out_dtype = T0G_F32;
    return gemm_locked(dev, &d);
}

int t0g_f32_to_bf16(t0g_device *dev, uint64_t src, uint64_t dst, size_t n) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    if (n && (!src || !dst)) return fail(T0G_ERR_INVALID_ARG, "NULL buffer");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    if ((rc = convert_locked(dev, src, dst, n))) return rc;
    return ok();
}

int t0g_matmul_f32(t0g_device *dev, uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t k, uint32_t n) {
    // Y = X * W: X [M][K] is K-contiguous, W [K][N] is N-contiguous -> NN.
    int rc = matmul_common(dev, x, (size_t)m * k, w, (size_t)k * n, y, m, n, k, T0G_NN);
    return rc ? rc : ok();
}

int t0g_matmul_backward_data_f32(t0g_device *dev, uint64_t dy, uint64_t w, uint64_t dx, uint32_t m, uint32_t k,
                                 uint32_t n) {
    // dX[M,K] = dY[M,N] * W[K,N]^T: contraction over N; dY rows and W rows are N-contiguous -> NT.
    int rc = matmul_common(dev, dy, (size_t)m * n, w, (size_t)k * n, dx, m, k, n, T0G_NT);
    return rc ? rc : ok();
}

int t0g_matmul_backward_weight_f32(t0g_device *dev, uint64_t x, uint64_t dy, uint64_t dw, uint32_t m, uint32_t k,
                                   uint32_t n) {
    // dW[K,N] = X[M,K]^T * dY[M,N]: contraction over M; both operands are M-major -> TN.
    int rc = matmul_common(dev, x, (size_t)m * k, dy, (size_t)m * n, dw, k, n, m, T0G_TN);
    return rc ? rc : ok();
}

int t0g_matmul_wt_bf16_f32(t0g_device *dev, uint64_t x, uint64_t wt_bf16, uint64_t y, uint32_t m, uint32_t k,
                           uint32_t n) {
    // Y = X * WT^T with WT [N][K] bf16 -> NT; only X needs converting.
    int rc = matmul_common(dev, x, (size_t)m * k, wt_bf16, 0, y, m, n, k, T0G_NT);
    return rc ? rc : ok();
}

// ---- bf16 weight cache (GpuRuntime::get_or_create_bf16 and friends) ----------

// The cached bf16 copy of tensor `id`, converting n f32 at f32_addr on a miss.
static int bf16_cache_get_locked(t0g_device *dev, uint64_t id, uint64_t f32_addr, size_t n, uint64_t *out) {
    auto it = dev->bf16_cache.find(id);
    if (it != dev->bf16_cache.end()) {
        if (it->second.n != n)
            return fail(T0G_ERR_INVALID_ARG,
                        "tensor %llu is cached with %zu elements, asked for %zu (invalidate it after a resize)",
                        (unsigned long long)id, it->second.n, n);
        *out = it->second.addr;
        return T0G_OK;
    }
    uint64_t addr = 0;
    int rc = alloc_locked(dev, round256(n * 2), &addr);
    if (rc) return rc;
    const size_t bytes = dev->allocations[addr];
    dev->allocations.erase(addr);   // owned by the cache from here on
    if ((rc = convert_locked(dev, f32_addr, addr, n))) {
        dev->pool[bytes].push_back(addr);
        dev->pool_bytes += bytes;
        return rc;
    }
    dev->bf16_cache[id] = t0g_device::Bf16Copy{addr, n, bytes};
    *out = addr;
    return T0G_OK;
}

static void bf16_cache_drop_locked(t0g_device *dev, std::unordered_map<uint64_t, t0g_device::Bf16Copy>::iterator it) {
    // Back to the pool: work already queued on the device stream may still read it, and a
    // later owner uses it in that stream's order.
    dev->pool[it->second.bytes].push_back(it->second.addr);
    dev->pool_bytes += it->second.bytes;
    dev->bf16_cache.erase(it);
}

int t0g_bf16_cache_get(t0g_device *dev, uint64_t tensor_id, uint64_t f32_addr, size_t n, uint64_t *bf16_addr) {
    if (!dev || !bf16_addr) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    if (!f32_addr || n == 0) return fail(T0G_ERR_INVALID_ARG, "empty tensor");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    if ((rc = bf16_cache_get_locked(dev, tensor_id, f32_addr, n, bf16_addr))) return rc;
    return ok();
}

int t0g_bf16_cache_invalidate(t0g_device *dev, uint64_t tensor_id) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    auto it = dev->bf16_cache.find(tensor_id);
    if (it != dev->bf16_cache.end()) bf16_cache_drop_locked(dev, it);
    return ok();
}

int t0g_bf16_cache_clear(t0g_device *dev) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    while (!dev->bf16_cache.empty()) bf16_cache_drop_locked(dev, dev->bf16_cache.begin());
    return ok();
}

int t0g_bf16_cache_stats(t0g_device *dev, uint64_t *entries, uint64_t *bytes) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    std::lock_guard<std::mutex> lk(dev->mu);
    uint64_t b = 0;
    for (const auto &c : dev->bf16_cache) b += c.second.bytes;
    if (entries) *entries = dev->bf16_cache.size();
    if (bytes) *bytes = b;
    return ok();
}

// matmul / gemm_backward_data with W's bf16 copy taken from the cache: only the
// activation operand is converted per call.
static int matmul_cached(t0g_device *dev, uint64_t a_f32, size_t a_elems, uint64_t w, uint64_t w_id, size_t w_elems,
                         uint64_t c, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose) {
    if (!dev) return fail(T0G_ERR_INVALID_ARG, "device is NULL");
    if (!a_f32 || !w || !c) return fail(T0G_ERR_INVALID_ARG, "NULL operand");
    std::lock_guard<std::mutex> lk(dev->mu);
    int rc = check_usable(dev);
    if (rc) return rc;
    if (m == 0 || n == 0) return ok();
    uint64_t w16 = 0;
    if (w_elems && (rc = bf16_cache_get_locked(dev, w_id, w, w_elems, &w16))) return rc;
    if ((rc = ensure_conv(dev, round256(a_elems * 2) + 256))) return rc;
    if ((rc = convert_locked(dev, a_f32, dev->conv, a_elems))) return rc;
    t0g_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = dev->conv;
    d.b = w_elems ? w16 : dev->conv;   // K == 0: the GEMM reads no operand
    d.c = c;
    d.m = m;
    d.n = n;
    d.k = k;
    d.transpose = transpose;
    d.out_dtype = T0G_F32;
    if ((rc = gemm_locked(dev, &d))) return rc;
    return ok();
}

int t0g_matmul_f32_cached(t0g_device *dev, uint64_t x, uint64_t w, uint64_t w_id, uint64_t y, uint32_t m, uint32_t k,
                          uint32_t n) {
    return matmul_cached(dev, x, (size_t)m * k, w, w_id, (size_t)k * n, y, m, n, k, T0G_NN);
}

int t0g_matmul_backward_data_f32_cached(t0g_device *dev, uint64_t dy, uint64_t w, uint64_t w_id, uint64_t dx,
                                        uint32_t m, uint32_t k, uint32_t n) {
    return matmul_cached(dev, dy, (size_t)m * n, w, w_id, (size_t)k * n, dx, m, k, n, T0G_NT);
}

}  // extern "C"
