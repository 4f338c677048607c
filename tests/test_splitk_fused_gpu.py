"""Split-K reduced inside the GEMM kernel (the _r and _dr kernels), through the C ABI.

The in-kernel reduction sums every chunk of a tile over its K slices in plane
order from 0.0, the order of the separate reduce kernel and of the reference's
host loop (examples/test_gemm_correctness.rs:190-207).  So each case runs once
reduced in the kernel and once as planes plus the reduce kernel
(t0g_set_split_k_mode) and the two outputs must be identical bit for bit; the
result is also checked against the oracle.  Cases cover every kernel that has an
in-kernel form (128x128, 256x256 in its 8-wave and 4-wave kernels, the 64x64
and 128x128 deep-ring kernels of grids with one workgroup per CU), all
layouts, f32 and bf16 output, ragged M/N edges, K tails, epilogue chains,
repeated launches (the control words must be back at zero after each), the
host-forced path in which every workgroup but a tile's last arrival gives up
waiting, so the last arrival sums the whole tile, and a seeded sweep of random
aligned problems (24 committed; 400 pass with T0G_FUSED_SWEEP_CASES=400).
Two slices on the deep rings take the no-wait pair sum (the second slice to
arrive adds the first's partial), the default for them: it has cases of its own,
two handles running it at once on two streams, and replays of a captured HIP
graph."""
import sys

import numpy as np
import pytest

import oracle as o
import t0g

pytestmark = pytest.mark.gpu

P128 = t0g.GemmConfig.preset("gfx950_128x128_k64")
P256 = t0g.GemmConfig.preset("gfx950_256x256_k64")
P64 = t0g.GemmConfig.preset("gfx950_64x64_k64")


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def rt():
    r = t0g.GpuRuntime.new(0)
    yield r
    t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)
    t0g.debug_stream_k_stall(False)
    assert r.stream_k_timeouts() == 0
    r.close()


def _operands(layout, m, n, k, seed):
    a_mk = o.rand_bf16_lcg(m * k, seed).reshape(m, k)
    b_nk = o.rand_bf16_lcg(n * k, seed + 1).reshape(n, k)
    a_st = a_mk if layout[0] == "N" else np.ascontiguousarray(a_mk.T)
    b_st = b_nk if layout[1] == "T" else np.ascontiguousarray(b_nk.T)
    return a_mk, b_nk, a_st, b_st


def _run(rt, da, db, m, n, k, layout, cfg, sk, out, mode, epilogue_ops=None, bias=0, repeat=1):
    esz, dt = (2, np.uint16) if out == t0g.BF16 else (4, np.float32)
    t0g.set_split_k_mode(mode)
    try:
        d = t0g.gemm_desc(da, db, 0, m, n, k, transpose=layout, out_dtype=out, config=cfg, split_k=sk,
                          epilogue_ops=epilogue_ops, bias=bias)
        name = t0g.gemm_kernel_name(d)
        dc = rt.alloc(m * n * esz)
        try:
            rt.memset(dc, 0xFF, m * n * esz)
            d.c = dc
            for _ in range(repeat):
                rt.gemm_desc(d)
            rt.wait_idle()
            return name, rt.read(dc, (m, n), dt)
        finally:
            rt.free(dc)
    finally:
        t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)


CASES = [
    # layout, m, n, k, config, split: what it exercises
    ("NT", 128, 4096, 4096, P128, 8),      # benchmark config 4a
    ("NT", 256, 256, 32768, P128, 64),     # benchmark config 4b: 64 slices per tile, 64-element chunks of 4 rows
    ("NN", 256, 256, 32768, P256, 64),     # one 256x256 tile in 64 slices (8-wave kernel)
    ("NN", 1024, 4096, 11008, P256, 4),    # the MLP's Y = H W2: 64 tiles x 4 slices, K tail per slice
    ("NT", 1024, 4096, 11008, P256, 4),    # the MLP's dX = dH W1^T
    ("TN", 512, 768, 4096, P256, 8),       # 4-wave 256x256 kernel (M-contiguous A)
    ("TT", 384, 512, 2048, P256, 4),       # ragged M on the 4-wave kernel
    ("TN", 200, 296, 4096, P128, 4),       # ragged M and N on 128x128
    ("NN", 320, 136, 3000, P128, 4),       # K tail: 3000 in slices of 768
    ("TT", 128, 128, 8192, P128, 32),      # a single tile in 32 slices
    ("NT", 128, 4096, 4096, P64, 2),       # benchmark config 4a on the 64x64 deep-ring kernel
    ("NT", 256, 256, 32768, P64, 16),      # benchmark config 4b: 16 slices, 256-element chunks
    ("NN", 192, 320, 5000, P64, 4),        # K tail on the 64x64 deep-ring kernel
    ("TN", 104, 200, 3000, P64, 8),        # ragged M and N, M-contiguous A (rows of 16-byte multiples)
    ("TT", 64, 64, 4096, P64, 16),         # a single 64x64 tile in 16 slices
    # two slices: the second to arrive adds the first's partial (red_pair)
    ("TN", 104, 200, 3000, P64, 2),        # ragged edges (masked stores), K tail, K split across the waves
    ("NN", 320, 136, 3000, P128, 2),       # ragged, 128x128 deep ring
    ("NT", 256, 512, 1024, P64, 2),        # 8 stages per slice: the 2 x 2 wave grid (_dr)
    ("TT", 192, 256, 4096, P128, 2),       # TT on 128x128
]


@pytest.mark.parametrize("out", [t0g.F32, t0g.BF16])
@pytest.mark.parametrize("layout,m,n,k,cfg,sk", CASES)
def test_fused_equals_reduce_kernel(rt, layout, m, n, k, cfg, sk, out):
    _log(f"[case] fused split-K {layout} {m}x{n}x{k} {cfg.tile_m}x{cfg.tile_n} sk={sk} out={out}")
    a_mk, b_nk, a_st, b_st = _operands(layout, m, n, k, 101 + m + sk)
    da, db = rt.upload(a_st), rt.upload(b_st)
    try:
        name_f, fused = _run(rt, da, db, m, n, k, layout, cfg, sk, out, t0g.SPLIT_K_IN_KERNEL)
        name_r, planes = _run(rt, da, db, m, n, k, layout, cfg, sk, out, t0g.SPLIT_K_REDUCE_KERNEL)
        fused_sfx = ("_r", "_dr", "_dsr")
        assert name_f.endswith(fused_sfx) and not name_r.endswith(fused_sfx), (name_f, name_r)
        deep = cfg.tile_m < 256 and (m + cfg.tile_m - 1) // cfg.tile_m * ((n + cfg.tile_n - 1) // cfg.tile_n) * sk <= 256
        assert name_f.endswith(("_dr", "_dsr")) == deep, name_f
        # the 64x64 deep ring splits K across its waves from 24 stages of 64 per slice,
        # in both modes alike
        stages = ((k + sk - 1) // sk + 63) // 64   # 64-K stages per slice (slices round up to whole stages)
        ksplit = deep and cfg.tile_m == 64 and stages >= 24
        assert name_f.endswith("_dsr") == ksplit and name_r.endswith("_ds") == ksplit, (name_f, name_r)
        assert np.array_equal(fused, planes), f"{name_f} differs from planes + reduce kernel"
        got = fused if out == t0g.F32 else o.bf16_to_f32(fused)
        ok, relf, maxabs, bound = o.parity(got, o.gemm("NT", a_mk, b_nk, m, n, k), k)
        _log(f"[parity] {name_f}: identical to the reduce kernel; relF={relf:.3e} max|d|={maxabs:.3e}")
        assert ok if out == t0g.F32 else relf <= 5e-3
    finally:
        rt.free(da)
        rt.free(db)


@pytest.mark.parametrize("layout,m,n,k,cfg,sk", [CASES[0], CASES[3], CASES[7], CASES[9], CASES[10], CASES[12],
                                                  CASES[15], CASES[16]])
def test_fused_epilogue_chain(rt, layout, m, n, k, cfg, sk):
    """bias + SiLU + clamp applied once, after the sum (not per slice)."""
    a_mk, b_nk, a_st, b_st = _operands(layout, m, n, k, 7 + n)
    bias = np.linspace(-0.5, 0.5, n, dtype=np.float32)
    da, db, dbias = rt.upload(a_st), rt.upload(b_st), rt.upload(bias)
    ops = ["bias", "silu", "clamp"]
    try:
        t0g.set_split_k_mode(t0g.SPLIT_K_IN_KERNEL)
        d = t0g.gemm_desc(da, db, 0, m, n, k, transpose=layout, config=cfg, split_k=sk, epilogue_ops=ops,
                          bias=dbias, clamp=(-0.05, 0.1))
        dc = rt.alloc(m * n * 4)
        try:
            d.c = dc
            rt.gemm_desc(d)
            fused = rt.read(dc, (m, n), np.float32)
            t0g.set_split_k_mode(t0g.SPLIT_K_REDUCE_KERNEL)
            rt.gemm_desc(d)
            planes = rt.read(dc, (m, n), np.float32)
        finally:
            t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)
            rt.free(dc)
        assert np.array_equal(fused, planes)
        ref = o.epilogue_chain(o.gemm("NT", a_mk, b_nk, m, n, k), ops, bias=bias, clamp=(-0.05, 0.1))
        ok, relf, maxabs, _ = o.parity(fused, ref, k)
        assert ok, (relf, maxabs)
    finally:
        for x in (da, db, dbias):
            rt.free(x)


@pytest.mark.parametrize("case", [0, 9, 10])
def test_fused_repeated_launches_and_stall(rt, case):
    """Eight launches back to back give the same bits (the arrival and claim words
    are reset by every launch); with the host-forced stall every tile is summed by
    its last arrival alone, with the same bits; no launch counts a timeout."""
    layout, m, n, k, cfg, sk = CASES[case]
    a_mk, b_nk, a_st, b_st = _operands(layout, m, n, k, 55)
    da, db = rt.upload(a_st), rt.upload(b_st)
    try:
        _, once = _run(rt, da, db, m, n, k, layout, cfg, sk, t0g.F32, t0g.SPLIT_K_IN_KERNEL)
        _, eight = _run(rt, da, db, m, n, k, layout, cfg, sk, t0g.F32, t0g.SPLIT_K_IN_KERNEL, repeat=8)
        assert np.array_equal(once, eight)
        t0g.debug_stream_k_stall(True)
        try:
            _, alone = _run(rt, da, db, m, n, k, layout, cfg, sk, t0g.F32, t0g.SPLIT_K_IN_KERNEL, repeat=3)
        finally:
            t0g.debug_stream_k_stall(False)
        assert np.array_equal(once, alone)
        assert rt.stream_k_timeouts() == 0
        assert not rt.is_poisoned()
    finally:
        rt.free(da)
        rt.free(db)


# T0G_FUSED_SWEEP_CASES: a longer run of the seeded sweep below for one-off checks.
N_SWEEP = int(__import__("os").environ.get("T0G_FUSED_SWEEP_CASES", "24"))


@pytest.mark.parametrize("i", range(N_SWEEP))
def test_fused_random_problem(rt, i):
    """Seeded random problems whose rows are 16-byte aligned (so the in-kernel form
    applies wherever its grid conditions hold): layout, M, N, K, tile, a power-of-two
    split, both outputs.  The in-kernel result must equal planes + reduce kernel bit
    for bit and pass the oracle gate."""
    rng = np.random.default_rng(7000 + i)
    layout = ["NT", "NN", "TN", "TT"][i % 4]
    cfg = [P64, P128, P256][int(rng.integers(0, 3))]
    m = 8 * int(rng.integers(1, 97))
    n = 8 * int(rng.integers(1, 97))
    sk = int(rng.choice([2, 4, 8, 16]))
    k = 8 * int(rng.integers(8 * sk, 8 * sk + 400))
    out = t0g.BF16 if i % 2 else t0g.F32
    _log(f"[case] fused sweep {i}: {layout} {m}x{n}x{k} {cfg.tile_m}x{cfg.tile_n} sk={sk} out={out}")
    a_mk, b_nk, a_st, b_st = _operands(layout, m, n, k, 300 + i)
    da, db = rt.upload(a_st), rt.upload(b_st)
    try:
        name_f, fused = _run(rt, da, db, m, n, k, layout, cfg, sk, out, t0g.SPLIT_K_IN_KERNEL)
        name_r, planes = _run(rt, da, db, m, n, k, layout, cfg, sk, out, t0g.SPLIT_K_REDUCE_KERNEL)
        _log(f"[kernel] {name_f} / {name_r}")
        assert np.array_equal(fused, planes), f"{name_f} differs from {name_r} + reduce kernel"
        got = fused if out == t0g.F32 else o.bf16_to_f32(fused)
        ok, relf, maxabs, bound = o.parity(got, o.gemm("NT", a_mk, b_nk, m, n, k), k)
        assert ok if out == t0g.F32 else relf <= 5e-3, (relf, maxabs, bound)
    finally:
        rt.free(da)
        rt.free(db)


def test_two_slice_sums_on_two_handles_at_once():
    """The two-slice sum, the default for C4a's shape, keeps its arrival counters in the
    handle's control block: two handles on two streams, eight launches each enqueued in
    turn with no wait, give every output equal bit for bit to a single launch's."""
    from hip_rt import Stream
    m, n, k = 128, 4096, 4096
    a = o.rand_bf16_lcg(m * k, 71)
    b = o.rand_bf16_lcg(n * k, 72)
    streams = [Stream(), Stream()]
    hs = [t0g.GpuRuntime.new(0), t0g.GpuRuntime.new(0)]
    try:
        t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)
        ops, outs = [], []
        for h, s in zip(hs, streams):
            h.set_stream(s.ptr)
            da, db = h.upload(a), h.upload(b)
            cs = [h.alloc(m * n * 4) for _ in range(8)]
            ops.append((da, db))
            outs.append(cs)
        names = {t0g.gemm_kernel_name(t0g.gemm_desc(ops[0][0], ops[0][1], outs[0][0], m, n, k, config=P64,
                                                    split_k=2))}
        assert names == {"t0g_gemm_64x64_k64_nt_f32_dsr"}, names
        for i in range(8):
            for h, (da, db), cs in zip(hs, ops, outs):
                h.gemm(da, db, cs[i], m, n, k, config=P64, split_k=2)
        for h in hs:
            h.wait_idle()
        want = hs[0].read(outs[0][0], (m, n), np.float32)
        assert o.parity(want, o.gemm("NT", a, b, m, n, k), k)[0]
        for j, (h, cs) in enumerate(zip(hs, outs)):
            for i, c in enumerate(cs):
                assert np.array_equal(h.read(c, (m, n), np.float32), want), f"handle {j} launch {i}"
        for h in hs:
            assert h.stream_k_timeouts() == 0
            assert not h.is_poisoned()
            h.set_stream(None)
    finally:
        for h in hs:
            h.close()
        for s in streams:
            s.destroy()


def test_two_slice_sum_under_hip_graph_capture():
    """A two-slice launch captured into a HIP graph (after an eager call set up the
    workspace and control block; the launch itself enqueues only the kernel, and the
    counters clear themselves) and replayed: every replay, with eager work and
    synchronisations in between, equals the eager call bit for bit."""
    from hip_rt import Graph, Stream
    m, n, k = 128, 4096, 4096
    a = o.rand_bf16_lcg(m * k, 81)
    b = o.rand_bf16_lcg(n * k, 82)
    h = t0g.GpuRuntime.new(0)
    s = Stream()
    g = None
    try:
        t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)
        h.set_stream(s.ptr)
        da, db = h.upload(a), h.upload(b)
        c_eager, c_graph, c_other = h.alloc(m * n * 2), h.alloc(m * n * 2), h.alloc(64 * 64 * 4)
        d_eager = t0g.gemm_desc(da, db, c_eager, m, n, k, out_dtype=t0g.BF16, config=P64, split_k=2)
        d_graph = t0g.gemm_desc(da, db, c_graph, m, n, k, out_dtype=t0g.BF16, config=P64, split_k=2)
        assert t0g.gemm_kernel_name(d_graph) == "t0g_gemm_64x64_k64_nt_bf16_dsr"
        h.gemm_desc(d_eager)
        h.wait_idle()
        want = h.read(c_eager, (m, n), np.uint16)
        g = Graph(s, lambda: h.gemm_desc(d_graph))
        for rep in range(4):
            h.memset(c_graph, 0xFF, m * n * 2)
            g.launch(s)
            s.synchronize()
            assert np.array_equal(h.read(c_graph, (m, n), np.uint16), want), f"replay {rep}"
            h.gemm(db, da, c_other, 64, 64, 4096, config=P64, split_k=2)   # eager two-slice work between
            h.wait_idle()
        assert h.stream_k_timeouts() == 0
        h.set_stream(None)
        for x in (da, db, c_eager, c_graph, c_other):
            h.free(x)
    finally:
        if g is not None:
            g.destroy()
        h.close()
        s.destroy()
