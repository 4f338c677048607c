"""t0g_gemm_noalloc against t0g_gemm, through the C ABI: the same results, bit for
bit, on two calls in a row (the second smaller, reusing the device's scratch
array), for split-K plans whose planes live in that scratch, a stream-K config
(run data-parallel without allocating) and a caller workspace; a problem that
needs more scratch than the array holds is refused before anything runs."""
import struct
import sys

import numpy as np
import pytest

import oracle as o
import t0g


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def gemm_noalloc(rt, desc):
    rt.gemm_noalloc(desc)


def _sections(elf):
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    hdr = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    names = elf[hdr[shstrndx][4]:hdr[shstrndx][4] + hdr[shstrndx][5]]
    out = {}
    for h in hdr:
        nm = names[h[0]:names.index(b"\0", h[0])].decode()
        out[nm] = h
    return out


def test_scratch_is_exported_from_the_device_code_object():
    """Host-side (no GPU): the fatbin inside libt0g.so exports the scratch array as a
    GLOBAL symbol of the gfx950 code object under the name the library registers with
    the HIP runtime.  An array the runtime cannot find by that name makes it abort
    while loading the library's code object (seen once, with the array inside an
    anonymous namespace: the symbol was local)."""
    with open(t0g.LIB_PATH, "rb") as f:
        lib = f.read()
    sec = _sections(lib)
    fat = lib[sec[".hip_fatbin"][4]:sec[".hip_fatbin"][4] + sec[".hip_fatbin"][5]]
    assert fat.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    n, = struct.unpack_from("<Q", fat, 24)
    pos, dev = 32, None
    for _ in range(n):
        off, size, idl = struct.unpack_from("<QQQ", fat, pos)
        ident = fat[pos + 24:pos + 24 + idl].decode()
        pos += 24 + idl
        if "gfx950" in ident:
            dev = fat[off:off + size]
    assert dev is not None, "no gfx950 code object in libt0g.so's fatbin"
    ds = _sections(dev)
    dynsym, dynstr = ds[".dynsym"], ds[".dynstr"]
    strtab = dev[dynstr[4]:dynstr[4] + dynstr[5]]
    found = {}
    for i in range(dynsym[5] // 24):
        st_name, st_info, _, _, _, st_size = struct.unpack_from("<IBBHQQ", dev, dynsym[4] + 24 * i)
        nm = strtab[st_name:strtab.index(b"\0", st_name)].decode()
        found[nm] = (st_info >> 4, st_size)
    registered = [nm for nm in found if "scratch" in nm]
    assert registered, f"no scratch symbol exported: {sorted(found)}"
    bind, size = found[registered[0]]
    assert bind == 1 and size == 64 << 20   # STB_GLOBAL, T0G_NOALLOC_SCRATCH_BYTES
    assert registered[0].encode() in lib     # the host side registers that same name


@pytest.fixture(scope="module")
def rt():
    r = t0g.GpuRuntime.new(0)
    yield r
    r.close()


def _pair(rt, layout, m, n, k, seed, cfg=None, out=t0g.BF16, split_k=0):
    """Run one problem through t0g_gemm and through t0g_gemm_noalloc; return both
    outputs and the oracle's fp32 product."""
    a_mk = o.rand_bf16_lcg(m * k, seed).reshape(m, k)
    b_nk = o.rand_bf16_lcg(n * k, seed + 1).reshape(n, k)
    a_st = a_mk if layout[0] == "N" else np.ascontiguousarray(a_mk.T)
    b_st = b_nk if layout[1] == "T" else np.ascontiguousarray(b_nk.T)
    esz, dt = (2, np.uint16) if out == t0g.BF16 else (4, np.float32)
    da, db = rt.upload(a_st), rt.upload(b_st)
    c1, c2 = rt.alloc(m * n * esz), rt.alloc(m * n * esz)
    try:
        rt.memset(c1, 0xFF, m * n * esz)
        rt.memset(c2, 0xEE, m * n * esz)
        d1 = t0g.gemm_desc(da, db, c1, m, n, k, transpose=layout, out_dtype=out, config=cfg, split_k=split_k)
        d2 = t0g.gemm_desc(da, db, c2, m, n, k, transpose=layout, out_dtype=out, config=cfg, split_k=split_k)
        rt.gemm_desc(d1)
        gemm_noalloc(rt, d2)
        rt.wait_idle()
        return rt.read(c1, (m, n), dt), rt.read(c2, (m, n), dt), o.gemm("NT", a_mk, b_nk, m, n, k)
    finally:
        for x in (da, db, c1, c2):
            rt.free(x)


def _check(ref_gemm, got, ref32, k, out, label):
    """Bit-equal to t0g_gemm's output; against the oracle, the fp32 output passes the
    full gate, the bf16 one the relF part (its rounding alone can exceed max|d|)."""
    assert np.array_equal(got, ref_gemm), f"{label}: t0g_gemm_noalloc differs from t0g_gemm"
    g32 = got if out == t0g.F32 else o.bf16_to_f32(got)
    ok, relf, maxabs, bound = o.parity(g32, ref32, k)
    _log(f"[noalloc] {label}: identical to t0g_gemm; relF={relf:.3e} max|d|={maxabs:.3e} (bound {bound:.3e})")
    assert (ok if out == t0g.F32 else relf <= 5e-3), label


@pytest.mark.parametrize("first,second", [
    (("NT", 128, 4096, 4096), ("NT", 64, 1024, 2048)),      # benchmark config 4a, then a smaller split
    (("NN", 256, 256, 32768), ("NN", 128, 192, 8192)),      # benchmark config 4b (split 16), then smaller
    (("TN", 512, 512, 4096), ("NT", 200, 136, 3000)),       # a ragged, K-tail second call
])
@pytest.mark.gpu
def test_noalloc_matches_gemm_two_calls_in_a_row(rt, first, second):
    for i, (layout, m, n, k) in enumerate((first, second)):
        cfg = t0g.auto_select(m, k, n)
        _log(f"[case] noalloc call {i + 1}: {layout} {m}x{n}x{k} ({cfg.name()})")
        r_gemm, r_noalloc, ref32 = _pair(rt, layout, m, n, k, 31 + i, out=t0g.F32)
        _check(r_gemm, r_noalloc, ref32, k, t0g.F32, f"{layout} {m}x{n}x{k} f32")
        r_gemm, r_noalloc, ref32 = _pair(rt, layout, m, n, k, 31 + i, out=t0g.BF16)
        _check(r_gemm, r_noalloc, ref32, k, t0g.BF16, f"{layout} {m}x{n}x{k} bf16")


@pytest.mark.gpu
def test_noalloc_forced_split_and_stream_k(rt):
    """A forced split (planes in the scratch) and a stream-K config (data-parallel here):
    each equal to t0g_gemm with the same plan."""
    p128 = t0g.GemmConfig.preset("gfx950_128x128_k64")
    r_gemm, r_noalloc, ref32 = _pair(rt, "NT", 512, 384, 4096, 41, cfg=p128, out=t0g.F32, split_k=8)
    _check(r_gemm, r_noalloc, ref32, 4096, t0g.F32, "forced split 8")
    sk = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
    dp = t0g.GemmConfig.preset("gfx950_256x256_k64")
    m, n, k = 1024, 768, 2048
    a = o.rand_bf16_lcg(m * k, 43)
    b = o.rand_bf16_lcg(k * n, 44)
    da, db = rt.upload(a), rt.upload(b)
    c1, c2 = rt.alloc(m * n * 4), rt.alloc(m * n * 4)
    try:
        rt.gemm(da, db, c1, m, n, k, transpose="NN", config=dp)
        gemm_noalloc(rt, t0g.gemm_desc(da, db, c2, m, n, k, transpose="NN", config=sk))
        got, want = rt.read(c2, (m, n), np.float32), rt.read(c1, (m, n), np.float32)
        assert np.array_equal(got, want)
        ok, relf, _, _ = o.parity(got, o.gemm("NN", a, b, m, n, k), k)
        assert ok, relf
    finally:
        for x in (da, db, c1, c2):
            rt.free(x)


@pytest.mark.gpu
def test_noalloc_caller_workspace(rt):
    m, n, k = 256, 512, 8192
    a = o.rand_bf16_lcg(m * k, 51)
    b = o.rand_bf16_lcg(n * k, 52)
    cfg = t0g.GemmConfig.preset("gfx950_64x64_k64").copy(split_k=4)
    da, db = rt.upload(a), rt.upload(b)
    c, ws = rt.alloc(m * n * 4), rt.alloc(4 * m * n * 4)
    try:
        gemm_noalloc(rt, t0g.gemm_desc(da, db, c, m, n, k, config=cfg, workspace=ws, workspace_bytes=4 * m * n * 4))
        ok, relf, _, _ = o.parity(rt.read(c, (m, n), np.float32), o.gemm("NT", a, b, m, n, k), k)
        assert ok, relf
        with pytest.raises(t0g.T0gError) as e:   # a workspace too small for the planes
            gemm_noalloc(rt, t0g.gemm_desc(da, db, c, m, n, k, config=cfg, workspace=ws, workspace_bytes=1024))
        assert e.value.code == t0g.ERR_INVALID_ARG
    finally:
        for x in (da, db, c, ws):
            rt.free(x)


@pytest.mark.gpu
def test_noalloc_refuses_more_scratch_than_it_has(rt):
    """4096 x 4096 with 8 planes needs 512 MiB: refused before anything is launched,
    and the device stays usable."""
    d = t0g.gemm_desc(1 << 20, 1 << 21, 1 << 22, 4096, 4096, 4096,
                      config=t0g.GemmConfig.preset("gfx950_128x128_k64"), split_k=8)
    with pytest.raises(t0g.T0gError) as e:
        gemm_noalloc(rt, d)
    assert e.value.code == t0g.ERR_INVALID_ARG and "scratch" in str(e.value)
    assert not rt.is_poisoned()


@pytest.mark.gpu
def test_noalloc_first_call_on_a_fresh_handle_allocates_nothing():
    """The property the entry point exists for.  On a handle that has launched nothing
    (no split-K workspace, no control block, no kernel looked up yet) the first call, a
    split-K plan whose planes go to the scratch, makes no device allocation: the library's
    count of hipMalloc calls and code-object loads does not move.  The same holds with the
    timeline diagnostic switched on (its instrumented code object is never loaded here).
    t0g_gemm on the same handle does allocate (its workspace), which shows the count sees it."""
    m, n, k = 128, 4096, 4096
    a = o.rand_bf16_lcg(m * k, 61)
    b = o.rand_bf16_lcg(n * k, 62)
    ref = o.gemm("NT", a, b, m, n, k)
    fresh = t0g.GpuRuntime.new(0)
    try:
        da, db, c = fresh.upload(a), fresh.upload(b), fresh.alloc(m * n * 4)
        desc = t0g.gemm_desc(da, db, c, m, n, k, split_k=2)
        assert t0g.gemm_workspace_size(desc) == 2 * m * n * 4          # a split plan: planes in the scratch
        before = t0g.device_alloc_count()
        fresh.gemm_noalloc(desc)
        fresh.wait_idle()
        assert t0g.device_alloc_count() == before, "t0g_gemm_noalloc allocated device memory"
        ok, relf, maxabs, _ = o.parity(fresh.read(c, (m, n), np.float32), ref, k)
        assert ok, (relf, maxabs)
        t0g.set_timeline(1)
        try:
            fresh.memset(c, 0, m * n * 4)
            before = t0g.device_alloc_count()
            fresh.gemm_noalloc(desc)
            fresh.wait_idle()
            assert t0g.device_alloc_count() == before, "the timeline build was loaded"
        finally:
            t0g.set_timeline(0)
        assert o.parity(fresh.read(c, (m, n), np.float32), ref, k)[0]
        before = t0g.device_alloc_count()
        fresh.gemm_desc(desc)                       # t0g_gemm: its workspace is a hipMalloc
        fresh.wait_idle()
        assert t0g.device_alloc_count() > before
        for x in (da, db, c):
            fresh.free(x)
    finally:
        fresh.close()


@pytest.mark.gpu
def test_noalloc_calls_from_two_handles_take_the_scratch_in_turn():
    """Two handles (two streams) on one GPU, each enqueueing split-K calls into the shared
    scratch with no wait in between: each call waits for the previous user's event, so
    every result equals the same problem run alone through t0g_gemm."""
    h1, h2 = t0g.GpuRuntime.new(0), t0g.GpuRuntime.new(0)
    bufs = []
    try:
        probs = []
        for i, (h, (m, n, k)) in enumerate([(h1, (256, 2048, 8192)), (h2, (512, 1024, 4096)),
                                             (h1, (128, 4096, 4096)), (h2, (256, 256, 32768))]):
            a = o.rand_bf16_lcg(m * k, 70 + i)
            b = o.rand_bf16_lcg(n * k, 80 + i)
            da, db, c = h.upload(a), h.upload(b), h.alloc(m * n * 4)
            bufs.append((h, (da, db, c)))
            d = t0g.gemm_desc(da, db, c, m, n, k, split_k=8)
            assert t0g.gemm_workspace_size(d) > 0
            probs.append((h, d, a, b, c, m, n, k))
        for h, d, *_ in probs:                      # enqueued back to back on two streams
            h.gemm_noalloc(d)
        h1.wait_idle()
        h2.wait_idle()
        for h, d, a, b, c, m, n, k in probs:
            got = h.read(c, (m, n), np.float32)
            h.memset(c, 0, m * n * 4)
            h.gemm_desc(d)                          # alone, library workspace
            h.wait_idle()
            assert np.array_equal(got, h.read(c, (m, n), np.float32)), f"{m}x{n}x{k}"
            assert o.parity(got, o.gemm("NT", a, b, m, n, k), k)[0]
    finally:
        for h, xs in bufs:
            for x in xs:
                h.free(x)
        h1.close()
        h2.close()


@pytest.mark.gpu
def test_noalloc_under_hip_graph_capture():
    """A split-K call captured into a HIP graph on a caller stream and replayed: every
    replay, with eager work and synchronisations in between, equals the eager call bit
    for bit, and replaying allocates nothing."""
    from hip_rt import Graph, Stream
    m, n, k = 256, 1024, 8192
    a = o.rand_bf16_lcg(m * k, 91)
    b = o.rand_bf16_lcg(n * k, 92)
    h = t0g.GpuRuntime.new(0)
    s = Stream()
    g = None
    try:
        da, db = h.upload(a), h.upload(b)
        c_eager, c_graph, c_other = h.alloc(m * n * 4), h.alloc(m * n * 4), h.alloc(m * n * 4)
        d_eager = t0g.gemm_desc(da, db, c_eager, m, n, k, split_k=4)
        d_graph = t0g.gemm_desc(da, db, c_graph, m, n, k, split_k=4)
        h.gemm_noalloc(d_eager)
        h.wait_idle()
        want = h.read(c_eager, (m, n), np.float32)
        assert o.parity(want, o.gemm("NT", a, b, m, n, k), k)[0]
        h.set_stream(s.ptr)
        g = Graph(s, lambda: h.gemm_noalloc(d_graph))
        before = t0g.device_alloc_count()
        for rep in range(3):
            h.memset(c_graph, 0, m * n * 4)
            g.launch(s)
            s.synchronize()
            got = h.read(c_graph, (m, n), np.float32)
            assert np.array_equal(got, want), f"replay {rep}"
            h.gemm_noalloc(t0g.gemm_desc(db, da, c_other, 256, 256, 1024, split_k=2))   # eager work between
            h.wait_idle()
        assert t0g.device_alloc_count() == before
        h.set_stream(None)
        for x in (da, db, c_eager, c_graph, c_other):
            h.free(x)
    finally:
        if g is not None:
            g.destroy()
        h.close()
        s.destroy()
