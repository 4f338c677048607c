"""Runtime paths on the GPU, through the C ABI: the tile ABI's own sequence with
split-K (tile_auto_select -> lower_gemm/load -> build_kernargs_m -> compute_grid
-> dispatch, src/t0/tile_ir.rs:471-568, 3148-3202), raw code objects with their
argument size checked on the host (GpuKernel::load, src/kfd/mod.rs:2559-2651),
T0Kernel::compile for callers that launch themselves, async dispatch + wait_idle
(src/ignis/gpu_context.rs:332-384), stream-K failures reported as errors
(gpu_context.rs:150-157), the buffer pool and f32 helpers (gpu_context.rs:21-76,
437-487) and tune_tile_ir (src/t0/cost_model.rs:788-1097)."""
import struct
import sys

import numpy as np
import pytest

import oracle as o
import t0g

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def rt():
    r = t0g.GpuRuntime.new(0)
    yield r
    r.close()


def check_parity(c_gpu, c_ref, k, label):
    ok, relf, maxabs, bound = o.parity(c_gpu, c_ref, k)
    _log(f"[parity] {label}: relF={relf:.3e} max|d|={maxabs:.3e} (bound {bound:.3e})")
    assert ok, f"{label}: relF={relf:.3e} max|d|={maxabs:.3e} bound={bound:.3e}"


# ---- the tile ABI with split-K --------------------------------------------------

TILE_SHAPES = [
    (128, 4096, 4096),    # C4a: thin M (benchmark config 4)
    (256, 32768, 256),    # C4b: deep K (benchmark config 4)
    (200, 3000, 136),     # ragged M/N and a K that no split divides
]


@pytest.mark.parametrize("layout", ["NT", "NN"])
@pytest.mark.parametrize("m,k,n", TILE_SHAPES)
def test_tile_abi_sequence_with_auto_selected_split(rt, layout, m, k, n):
    """The reference's tile_ir sequence as a caller writes it, on the configs
    tile_auto_select hands out (split-K on the HBM-bound shapes): build_kernargs_m
    leaves y_split_stride 0, and Y holds the reduced product."""
    tr = t0g.LAYOUTS[layout]
    cfg = t0g.tile_auto_select(m, k, n, tr)
    _log(f"[case] tile ABI {m}x{k}x{n} {layout}: {t0g.tile_config_name(cfg)}")
    kern = rt.ensure_tile_kernel(cfg)
    assert kern.info()["kernarg_size"] == 44
    x = o.rand_bf16_lcg(m * k, m * 7 + k)                                   # U(-0.5, 0.5) inputs (config 4)
    b = o.rand_bf16_lcg(k * n, n * 11 + k)
    ref = o.gemm(layout, x, b, m, n, k)
    xa, ba = rt.upload(x), rt.upload(b)
    y = rt.upload(np.full((m + 8, n), -9999.0, dtype=np.float32))          # sentinel rows past M
    try:
        ka = t0g.build_kernargs_m(xa, ba, y, k, n, m, cfg)
        assert struct.unpack_from("<I", ka, 36)[0] == 0                     # the reference's stride
        rt.dispatch(kern, t0g.tile_compute_grid(cfg, m, n), ka)
        got = rt.read(y, (m + 8, n), np.float32)
        check_parity(got[:m], ref, k, f"tile ABI {t0g.tile_config_name(cfg)} {m}x{k}x{n}")
        assert np.all(got[m:] == -9999.0)
        # the same problem on the caller-owned-plane contract: a stride at @36 makes
        # the kernel write plain K-slice planes that the caller sums (gemm_gen style)
        sk = max(cfg.split_k, 1)
        if sk > 1 and k % (64 * sk) == 0:
            planes = rt.alloc(sk * m * n * 4)
            try:
                ka2 = bytearray(ka)
                ka2[36:40] = struct.pack("<I", m * n * 4)
                ka2[16:24] = struct.pack("<Q", planes)
                rt.dispatch(kern, t0g.tile_compute_grid(cfg, m, n), bytes(ka2))
                p = rt.read(planes, (sk, m, n), np.float32)
                check_parity(o.splitk_reduce(p), ref, k, f"caller planes sk={sk}")
                kps = k // sk
                part = o.gemm_krange(layout, x, b, m, n, k, kps, 2 * kps)
                check_parity(p[1], part, kps, "plane 1")
            finally:
                rt.free(planes)
    finally:
        for a in (xa, ba, y):
            rt.free(a)


def test_tile_abi_split_with_epilogue_chain(rt):
    """A split tile kernel with a chain: the library reduces the planes in plane order
    and applies the chain once (bias is not added per plane)."""
    m, k, n = 128, 4096, 1024
    cfg = t0g.GemmConfig.preset("gfx950_128x128_k64").copy(split_k=8)
    chain = t0g.epilogue_chain(["bias", "relu"])
    kern = rt.ensure_tile_kernel(cfg, chain)
    x = o.rand_bf16_lcg(m * k, 3)
    wt = o.rand_bf16_lcg(n * k, 4)
    bias = (np.arange(n, dtype=np.float32) % 7 - 3) * 0.25
    ref32 = o.gemm("NT", x, wt, m, n, k)
    ref = o.epilogue_chain(ref32, ["bias", "relu"], bias=bias)
    xa, wa, ba = rt.upload(x), rt.upload(wt), rt.upload(bias)
    y = rt.alloc(m * n * 4)
    try:
        ka = t0g.build_kernargs_m_epilogue(xa, wa, y, k, n, m, cfg, chain, bias=ba)
        rt.dispatch(kern, t0g.tile_compute_grid(cfg, m, n), ka)
        got = rt.read(y, (m, n), np.float32)
        check_parity(got, ref, k, "tile ABI sk8 bias+relu")
        # bit-exact to the plane-ordered reduce of the same kernel's planes, chained
        planes = rt.alloc(8 * m * n * 4)
        try:
            plain = rt.ensure_tile_kernel(cfg)
            ka2 = bytearray(t0g.build_kernargs_m(xa, wa, planes, k, n, m, cfg))
            ka2[36:40] = struct.pack("<I", m * n * 4)
            rt.dispatch(plain, t0g.tile_compute_grid(cfg, m, n), bytes(ka2))
            p = rt.read(planes, (8, m, n), np.float32)
            exp = o.epilogue_chain(o.splitk_reduce(p), ["bias", "relu"], bias=bias)
            assert np.array_equal(got, exp)
        finally:
            rt.free(planes)
        # a chain on caller-owned planes is refused before anything runs
        bad = bytearray(ka)
        bad[36:40] = struct.pack("<I", m * n * 4)
        with pytest.raises(t0g.T0gError) as e:
            rt.dispatch(kern, t0g.tile_compute_grid(cfg, m, n), bytes(bad))
        assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG
        assert not rt.is_poisoned()
    finally:
        for a in (xa, wa, ba, y):
            rt.free(a)


# ---- raw code objects: argument size from the code object's metadata ------------

def _hsaco():
    import os
    with open(os.path.join(os.path.dirname(t0g.LIB_PATH), "t0g_gemm_gfx950.hsaco"), "rb") as f:
        return f.read()


def test_raw_dispatch_with_the_wrong_argument_size_is_refused(rt):
    """A kernarg block that does not match the kernel is refused on the host (it never
    reaches the GPU) and the device stays usable; an oversized workgroup is refused at load."""
    blob = _hsaco()
    kern = rt.load_kernel(blob, "t0g_gemm_128x128_k64_nt_f32", (256, 1, 1))
    assert kern.info()["kernarg_size"] == 104
    for size in (0, 40, 88, 103, 105, 144):
        with pytest.raises(t0g.T0gError) as e:
            rt.dispatch(kern, [256, 1, 1], b"\0" * size)
        assert e.value.code == t0g.ERR_INVALID_ARG and "exactly 104" in str(e.value)
    with pytest.raises(t0g.T0gError) as e:
        rt.load_kernel(blob, "t0g_gemm_128x128_k64_nt_f32", (1024, 1, 1))
    assert e.value.code == t0g.ERR_INVALID_ARG
    with pytest.raises(t0g.T0gError):
        rt.load_kernel(blob, "no_such_kernel", (256, 1, 1))
    assert not rt.is_poisoned()


@pytest.mark.parametrize("layout,m,n,k,sk", [("NT", 256, 384, 128, 0), ("NN", 300, 200, 520, 0),
                                             ("TN", 512, 512, 1024, 0), ("NT", 128, 1024, 2048, 4)])
def test_compile_load_dispatch(rt, layout, m, n, k, sk):
    """T0Kernel::compile -> GpuKernel::load -> dispatch, the way a caller that launches
    kernels itself does it: the code object, symbol, LDS, argument block and grid come
    from t0g_gemm_compile; an explicitly split plan writes K-slice planes into C (a split
    auto_select would pick is not taken: C stays one plane)."""
    a_mk = o.rand_bf16_lcg(m * k, 21).reshape(m, k)
    b_nk = o.rand_bf16_lcg(n * k, 22).reshape(n, k)
    a_st = a_mk if layout[0] == "N" else np.ascontiguousarray(a_mk.T)
    b_st = b_nk if layout[1] == "T" else np.ascontiguousarray(b_nk.T)
    ref = o.gemm("NT", a_mk, b_nk, m, n, k)
    da, db = rt.upload(a_st), rt.upload(b_st)
    cfg = t0g.GemmConfig.preset("gfx950_128x128_k64").copy(split_k=sk) if sk else None
    planes = max(sk, 1)
    dc = rt.alloc(planes * m * n * 4)
    try:
        d = t0g.gemm_desc(da, db, dc, m, n, k, transpose=layout, config=cfg)
        ck = t0g.gemm_compile(d)
        _log(f"[case] compile {layout} {m}x{n}x{k}: {ck.name.decode()} grid {list(ck.grid)} splits {ck.splits}")
        assert ck.splits == planes, "C holds one plane per split: the plan must match the allocation"
        kern = rt.load_kernel(ck.elf(), ck.name.decode(), (ck.workgroup_size, 1, 1), ck.lds_size)
        rt.dispatch(kern, list(ck.grid), ck.args())
        p = rt.read(dc, (ck.splits, m, n), np.float32)
        check_parity(o.splitk_reduce(p) if ck.splits > 1 else p[0], ref, k, f"compiled {ck.name.decode()}")
    finally:
        for a in (da, db, dc):
            rt.free(a)


def test_dispatch_async_then_wait_idle(rt):
    """dispatch_async enqueues and returns; wait_idle waits for all of them
    (gpu_context.rs:332-384).  Eight GEMMs into eight outputs, one wait."""
    cfg = t0g.GemmConfig.preset("gfx950_64x64_k64")
    kern = rt.ensure_gemm_kernel(cfg)
    m, k, n = 128, 256, 192
    outs, refs, ins = [], [], []
    try:
        for i in range(8):
            x = o.rand_bf16_xorshift(m * k, 100 + i)
            wt = o.rand_bf16_xorshift(n * k, 200 + i)
            refs.append(o.gemm_nt_naive(x, wt, m, k, n))
            xa, wa = rt.upload(x), rt.upload(wt)
            y = rt.alloc(m * n * 4)
            ins += [xa, wa]
            outs.append(y)
            gx, gy = t0g.compute_grid_auto(cfg, m, n)
            rt.dispatch_async(kern, [gx, gy, 1], t0g.build_kernargs(xa, wa, y, k, n, m, cfg))
        rt.wait_idle()
        for i, y in enumerate(outs):
            check_parity(rt.read(y, (m, n), np.float32), refs[i], k, f"async dispatch {i}")
    finally:
        for a in ins + outs:
            rt.free(a)


# ---- stream-K failures are errors ----------------------------------------------

def test_stream_k_wait_that_gives_up_poisons_the_device():
    """Host-forced: later stream-K launches wait on a control word nothing sets, with a
    spin limit of 64 polls, so every wait of a cut tile gives up and every kernel exits.
    The next wait on the stream returns T0G_ERR_TIMEOUT and the device is poisoned."""
    r = t0g.GpuRuntime.new(0)
    try:
        m, n, k = 512, 512, 4096       # 4 tiles x 64 K steps over 256 workgroups: every tile cut 64 ways
        a = r.upload(o.rand_bf16_xorshift(m * k, 5))
        b = r.upload(o.rand_bf16_xorshift(k * n, 6))
        c = r.alloc(m * n * 4)
        sk = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
        r.gemm(a, b, c, m, n, k, transpose="NN", config=sk)   # a normal launch first: no error
        r.wait_idle()
        assert r.stream_k_timeouts() == 0
        t0g.set_stream_k_spin_limit(64)
        t0g.debug_stream_k_stall(True)
        try:
            r.gemm(a, b, c, m, n, k, transpose="NN", config=sk)
            with pytest.raises(t0g.T0gError) as e:
                r.wait_idle()
            assert e.value.code == t0g.ERR_TIMEOUT and "stream-K" in str(e.value)
        finally:
            t0g.debug_stream_k_stall(False)
            t0g.set_stream_k_spin_limit(1 << 20)
        assert r.is_poisoned()
        with pytest.raises(t0g.T0gError) as e:
            r.gemm(a, b, c, m, n, k, transpose="NN", config=sk)
        assert e.value.code == t0g.ERR_POISONED
    finally:
        r.close()


def test_stream_k_give_up_is_reported_after_a_stream_switch():
    """As above, but the caller switches the handle to another stream right after the
    stalled launch: the new stream is ordered after it, so its first wait still reads the
    timeout count, returns T0G_ERR_TIMEOUT and poisons the device."""
    from hip_rt import Stream
    r = t0g.GpuRuntime.new(0)
    side = Stream()
    try:
        m, n, k = 512, 512, 4096
        a = r.upload(o.rand_bf16_xorshift(m * k, 5))
        b = r.upload(o.rand_bf16_xorshift(k * n, 6))
        c = r.alloc(m * n * 4)
        sk = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
        t0g.set_stream_k_spin_limit(64)
        t0g.debug_stream_k_stall(True)
        try:
            r.gemm(a, b, c, m, n, k, transpose="NN", config=sk)
            r.set_stream(side.ptr)
            with pytest.raises(t0g.T0gError) as e:
                r.wait_idle()
            assert e.value.code == t0g.ERR_TIMEOUT and "stream-K" in str(e.value)
        finally:
            t0g.debug_stream_k_stall(False)
            t0g.set_stream_k_spin_limit(1 << 20)
        assert r.is_poisoned()
    finally:
        r.close()
        side.destroy()


# ---- grouped GEMMs keep each stream's workspace ------------------------------------

def test_gemm_group_workspace_growth_on_the_device_stream():
    """Regression: a group whose first GEMM (device stream) grows the split-K workspace,
    then a plain split-K GEMM that fits the old size.  The plain GEMM must use the grown
    workspace (the old one was freed), and its result must match the oracle."""
    r = t0g.GpuRuntime.new(0)
    bufs = []
    try:
        def up(arr):
            a = r.upload(arr)
            bufs.append(a)
            return a

        def out(nbytes):
            a = r.alloc(nbytes)
            bufs.append(a)
            return a

        cfg = t0g.GemmConfig.preset("gfx950_64x64_k64").copy(split_k=4)
        sm, sn, sk_ = 128, 128, 2048                      # small: 4 planes x 64 KB
        x_s = o.rand_bf16_lcg(sm * sk_, 1)
        w_s = o.rand_bf16_lcg(sn * sk_, 2)
        xs, ws = up(x_s), up(w_s)
        ys = out(sm * sn * 4)
        r.gemm(xs, ws, ys, sm, sn, sk_, config=cfg)                       # workspace W0 (small)
        bm, bn, bk = 512, 512, 2048                        # big: 4 planes x 1 MB, grows W0 -> W1
        x_b = o.rand_bf16_lcg(bm * bk, 3)
        w_b = o.rand_bf16_lcg(bn * bk, 4)
        xb, wb = up(x_b), up(w_b)
        yb, y2 = out(bm * bn * 4), out(sm * sn * 4)
        d_big = t0g.gemm_desc(xb, wb, yb, bm, bn, bk, config=cfg)
        d_side = t0g.gemm_desc(xs, ws, y2, sm, sn, sk_, config=cfg)
        r.gemm_group([d_big, d_side])
        ys2 = out(sm * sn * 4)
        r.gemm(xs, ws, ys2, sm, sn, sk_, config=cfg)                      # fits W0's size: must use W1
        r.wait_idle()
        ref_s = o.gemm("NT", x_s, w_s, sm, sn, sk_)
        check_parity(r.read(ys2, (sm, sn), np.float32), ref_s, sk_, "split-K after the group")
        check_parity(r.read(yb, (bm, bn), np.float32), o.gemm("NT", x_b, w_b, bm, bn, bk), bk, "group big")
        check_parity(r.read(y2, (sm, sn), np.float32), ref_s, sk_, "group side")
        assert np.array_equal(r.read(ys, (sm, sn), np.float32), r.read(ys2, (sm, sn), np.float32))
    finally:
        for a in bufs:
            r.free(a)
        r.close()


def _hip_runtime():
    """The HIP runtime libt0g.so is linked against (its streams are what
    t0g_device_set_stream takes)."""
    import ctypes
    hip = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    return hip


def test_stream_switch_orders_split_k_launches():
    """t0g_device_set_stream: work issued after a switch of stream waits for the work
    issued on the old one, so two split-K GEMMs that share the handle's workspace run
    one after the other.  A large split-K GEMM on stream A, a switch to stream B and at
    once a small one whose planes go to the same workspace: both match the oracle."""
    import ctypes
    hip = _hip_runtime()
    r = t0g.GpuRuntime.new(0)
    streams = [ctypes.c_void_p(), ctypes.c_void_p()]
    for s in streams:
        assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    bufs = []
    try:
        def up(arr):
            a = r.upload(arr)
            bufs.append(a)
            return a

        def out(nbytes):
            a = r.alloc(nbytes)
            bufs.append(a)
            return a

        cfg = t0g.GemmConfig.preset("gfx950_64x64_k64").copy(split_k=4)
        bm, bn, bk = 1024, 1024, 8192
        sm, sn, sk_ = 256, 256, 4096
        x_b, w_b = o.rand_bf16_lcg(bm * bk, 21), o.rand_bf16_lcg(bn * bk, 22)
        x_s, w_s = o.rand_bf16_lcg(sm * sk_, 23), o.rand_bf16_lcg(sn * sk_, 24)
        xb, wb, xs, ws = up(x_b), up(w_b), up(x_s), up(w_s)
        yb, ys = out(bm * bn * 4), out(sm * sn * 4)
        r.wait_idle()
        _log("[case] split-K 1024x1024x8192 on stream A, then 256x256x4096 on stream B")
        r.set_stream(streams[0].value)
        r.gemm(xb, wb, yb, bm, bn, bk, config=cfg)
        r.set_stream(streams[1].value)
        r.gemm(xs, ws, ys, sm, sn, sk_, config=cfg)
        for s in streams:
            assert hip.hipStreamSynchronize(s) == 0
        r.set_stream(None)
        check_parity(r.read(yb, (bm, bn), np.float32), o.gemm("NT", x_b, w_b, bm, bn, bk), bk, "stream A")
        check_parity(r.read(ys, (sm, sn), np.float32), o.gemm("NT", x_s, w_s, sm, sn, sk_), sk_, "stream B")
    finally:
        r.set_stream(None)
        for a in bufs:
            r.free(a)
        r.close()
        for s in streams:
            hip.hipStreamDestroy(s)


# ---- buffer pool and f32 helpers ------------------------------------------------

def test_pool_reuses_recycled_buffers(rt):
    """BufferPool (gpu_context.rs:21-76): a recycled buffer comes back for the next
    allocation of the same 4 KiB-rounded size; clear frees the cached ones."""
    rt.pool_clear()
    s0 = rt.pool_stats()
    a = rt.alloc(10000)
    rt.recycle(a)
    st = rt.pool_stats()
    assert st["cached_buffers"] == 1 and st["cached_bytes"] == 12288
    b = rt.alloc(12000)                 # same rounded size (3 pages): the same buffer
    assert b == a
    assert rt.pool_stats()["hits"] == s0["hits"] + 1 and rt.pool_stats()["cached_buffers"] == 0
    c = rt.alloc(20000)                 # another size: a new buffer
    assert c != b
    rt.recycle(b)
    for op in (rt.recycle, rt.free):    # a recycled address is no longer live
        with pytest.raises(t0g.T0gError) as e:
            op(b)
        assert e.value.code == t0g.ERR_INVALID_ARG
    rt.free(c)
    rt.pool_clear()
    st = rt.pool_stats()
    assert st["cached_buffers"] == 0 and st["cached_bytes"] == 0


def test_f32_helpers_roundtrip(rt):
    """alloc_f32 pads to 512-byte blocks and zeroes; upload_f32 / read_f32 / write_f32
    (gpu_context.rs:449-487)."""
    z = rt.alloc_f32(3)
    assert np.array_equal(rt.read_f32(z, 128), np.zeros(128, np.float32))   # 512 bytes, all zero
    data = np.linspace(-2, 2, 1000, dtype=np.float32)
    u = rt.upload_f32(data)
    assert np.array_equal(rt.read_f32(u, 1000), data)
    rt.write_f32(u, data[::-1].copy())
    assert np.array_equal(rt.read_f32(u, 1000), data[::-1])
    rt.recycle(z)
    z2 = rt.alloc_f32(100)               # same 4 KiB size class: reused, and zeroed again
    assert z2 == z
    assert np.array_equal(rt.read_f32(z2, 128), np.zeros(128, np.float32))
    for x in (u, z2):
        rt.free(x)


def test_recycled_operands_feed_a_gemm(rt):
    """An Ignis-style loop: allocate, run, recycle, allocate again; the GEMM reads the
    recycled buffers in stream order."""
    m, k, n = 256, 512, 256
    for it in range(3):
        x = o.rand_bf16_lcg(m * k, 40 + it)
        wt = o.rand_bf16_lcg(n * k, 50 + it)
        xa, wa = rt.upload(x), rt.upload(wt)
        y = rt.alloc_f32(m * n)
        rt.gemm(xa, wa, y, m, n, k)
        got = rt.read_f32(y, m * n).reshape(m, n)
        check_parity(got, o.gemm("NT", x, wt, m, n, k), k, f"pooled loop {it}")
        for a in (xa, wa, y):
            rt.recycle(a)
    assert rt.pool_stats()["hits"] >= 6
    rt.pool_clear()


# ---- tune_tile_ir ---------------------------------------------------------------

def test_tune_tile_ir_on_the_thin_shape(rt, tmp_path):
    """tune_tile_ir (cost_model.rs:788-1013) on benchmark config 4's thin shape: the best
    config runs through the tile ABI against the oracle, the second call is a hit, and a
    new tuner reads tile_ir_128x4096x4096.json."""
    m, n, k = 128, 4096, 4096
    with t0g.GemmTuner.with_cache_dir(tmp_path / "tt") as tuner:
        tuner.max_candidates = 4
        tuner.n_iters = 3
        r = tuner.tune_tile_ir(rt, m, n, k)
        ranking = tuner.tile_ir_ranking(m, n, k)
        _log(f"[tune_tile_ir] best {t0g.tile_config_name(r.best)} {r.best_tflops:.1f} TF; {ranking}")
        assert r.from_cache == 0 and r.best.split_k != t0g.STREAM_K and r.best_tflops > 50
        assert ranking[0][0] == t0g.tile_config_name(r.best)
        assert all(nm.startswith("tile_gemm_") for nm, _ in ranking)
        assert tuner.tune_tile_ir(rt, m, n, k).best_tflops == r.best_tflops
        assert (tmp_path / "tt" / "tile_ir_128x4096x4096.json").exists()
        best = r.best
    with t0g.GemmTuner.with_cache_dir(tmp_path / "tt") as again:
        assert again.tile_ir_lookup(m, n, k).from_cache == 1
    kern = rt.ensure_tile_kernel(best)
    x = o.rand_bf16_lcg(m * k, 8)
    wt = o.rand_bf16_lcg(n * k, 9)
    xa, wa = rt.upload(x), rt.upload(wt)
    y = rt.alloc(m * n * 4)
    try:
        rt.dispatch(kern, t0g.tile_compute_grid(best, m, n), t0g.build_kernargs_m(xa, wa, y, k, n, m, best))
        check_parity(rt.read(y, (m, n), np.float32), o.gemm("NT", x, wt, m, n, k), k, "tuned tile config")
    finally:
        for a in (xa, wa, y):
            rt.free(a)


# ---- workgroup timeline (diagnostic) -------------------------------------------

@pytest.mark.parametrize("preset,m,n,k,sk,layout", [
    ("gfx950_256x256_k64", 1024, 768, 512, 0, "NN"),      # 12 workgroups, 8-wave ping-pong kernel
    ("gfx950_256x256_k64", 512, 768, 384, 0, "NT"),       # 6 workgroups, 8-wave ping-pong kernel
    ("gfx950_256x256_k64", 512, 512, 384, 0, "TN"),       # 4 workgroups, 4-wave kernel
    ("gfx950_128x128_k64", 256, 640, 1024, 4, "NT"),      # 10 tiles x 4 K slices, deep-ring kernel
    ("gfx950_64x64_k64", 1024, 1024, 128, 0, "NN"),       # 256 workgroups, 4-stage ring kernel
])
def test_timeline_records_every_workgroup(rt, preset, m, n, k, sk, layout):
    """With t0g_set_timeline on, launches run the instrumented build of the kernels
    and each workgroup leaves one entry: entry clock <= end of its K loop <= its
    stores completed, an XCD id below 8; the result is unchanged.  Off again, the
    production kernels run and record nothing."""
    _log(f"[case] timeline {preset} {m}x{n}x{k} sk={sk} {layout}")
    a_mk = o.rand_bf16_lcg(m * k, 31 + m).reshape(m, k)
    b_nk = o.rand_bf16_lcg(n * k, 37 + n).reshape(n, k)
    a = rt.upload(a_mk if layout[0] == "N" else np.ascontiguousarray(a_mk.T))
    b = rt.upload(b_nk if layout[1] == "T" else np.ascontiguousarray(b_nk.T))
    c = rt.alloc(m * n * 4)
    cfg = t0g.GemmConfig.preset(preset)
    d = t0g.gemm_desc(a, b, c, m, n, k, transpose=layout, config=cfg, split_k=sk)
    tile = cfg.tile_m
    wgs = ((m + tile - 1) // tile) * ((n + tile - 1) // tile) * max(sk, 1)
    try:
        rt.timeline_clear()
        t0g.set_timeline(True)
        rt.gemm_desc(d)
        rt.wait_idle()
        tl = rt.timeline_read()
    finally:
        t0g.set_timeline(False)
    rows = tl[tl[:, 0] != 0]
    assert len(rows) == wgs and not tl[wgs:].any(), f"{len(rows)} entries for {wgs} workgroups"
    assert np.all(rows[:, 0] <= rows[:, 1]) and np.all(rows[:, 1] <= rows[:, 2])
    assert np.all((rows[:, 3] >> np.uint64(32)) < 8)
    span_us = (rows[:, 2].max() - rows[:, 0].min()) * t0g.TIMELINE_TICK_NS / 1e3
    assert 0 < span_us < 1e5
    check_parity(rt.read(c, (m, n), np.float32), o.gemm("NT", a_mk, b_nk, m, n, k), k, f"timeline {preset}")
    rt.timeline_clear()
    rt.gemm_desc(d)
    rt.wait_idle()
    assert not rt.timeline_read().any(), "a launch with the timeline off recorded entries"
    for x in (a, b, c):
        rt.free(x)
