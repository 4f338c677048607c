"""Stream-K schedule on the GPU: parity with the oracle on shapes that cut
tiles two ways, many ways (up to 15 partials per tile), with K tails and ragged
edges, in all layouts and both output types; bit-exact agreement with the
data-parallel kernel where no tile is cut; repeat launches (the control block
is reset by every launch); fused epilogues after the fixup; no timed-out waits."""
import sys

import numpy as np
import pytest

import oracle as o
import t0g

pytestmark = pytest.mark.gpu

SK = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
DP = t0g.GemmConfig.preset("gfx950_256x256_k64")


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def rt():
    r = t0g.GpuRuntime.new(0)
    yield r
    assert r.stream_k_timeouts() == 0
    r.close()


def _operands(layout, m, n, k, seed):
    a_mk = o.rand_bf16_xorshift(m * k, seed).reshape(m, k)
    b_nk = o.rand_bf16_xorshift(n * k, seed + 1).reshape(n, k)
    a_st = a_mk if layout in ("NT", "NN") else np.ascontiguousarray(a_mk.T)
    b_st = b_nk if layout in ("NT", "TT") else np.ascontiguousarray(b_nk.T)
    return a_st, b_st


def _run(rt, da, db, m, n, k, layout, cfg, out=t0g.F32, **kw):
    esz = 4 if out == t0g.F32 else 2
    dc = rt.alloc(m * n * esz)
    try:
        rt.memset(dc, 0xFF, m * n * esz)
        rt.gemm(da, db, dc, m, n, k, transpose=layout, config=cfg, out_dtype=out, **kw)
        rt.wait_idle()
        return rt.read(dc, (m, n), np.float32 if out == t0g.F32 else np.uint16)
    finally:
        rt.free(dc)


SHAPES = [
    # (m, n, k): what it exercises
    (1024, 2816, 4096),   # 44 tiles x 64 steps over 256 workgroups: 11 steps each, ~6 per tile
    (512, 768, 1000),     # K tail; 6 tiles x 16 steps = 96 workgroups of 1 step: 15 partials per tile
    (1000, 1000, 640),    # ragged M and N edges, 16 tiles x 10 steps
    (2048, 2048, 256),    # 64 tiles x 4 steps, one step per workgroup
    (1536, 2560, 3072),   # uneven ranges (2880 steps over 256)
    (256, 256, 64),       # a single step: grid of one
]


@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_stream_k_parity(rt, layout, m, n, k):
    _log(f"[case] stream-K {layout} {m}x{n}x{k}")
    a_st, b_st = _operands(layout, m, n, k, m + n + k)
    ref = o.gemm(layout, a_st, b_st, m, n, k)
    da, db = rt.upload(a_st), rt.upload(b_st)
    try:
        c = _run(rt, da, db, m, n, k, layout, SK)
        ok, relf, maxabs, bound = o.parity(c, ref, k)
        _log(f"[parity] stream-K {layout} {m}x{n}x{k}: relF={relf:.3e} max|d|={maxabs:.3e} (bound {bound:.3e})")
        assert ok
        again = _run(rt, da, db, m, n, k, layout, SK)
        assert np.array_equal(c, again), "stream-K results must not depend on timing"
        c16 = _run(rt, da, db, m, n, k, layout, SK, out=t0g.BF16)
        assert np.array_equal(c16, o.f32_to_bf16_rne(c)), "bf16 output != RNE(fp32 output)"
    finally:
        rt.free(da)
        rt.free(db)


@pytest.mark.parametrize("layout", ["NN", "TN"])
def test_stream_k_without_cuts_equals_data_parallel(rt, layout):
    """4096^3: 256 tiles x 64 steps on 256 workgroups, each owns one whole tile, so
    the sums are the data-parallel kernel's, bit for bit."""
    m = n = k = 4096
    a_st, b_st = _operands(layout, m, n, k, 77)
    da, db = rt.upload(a_st), rt.upload(b_st)
    try:
        c_sk = _run(rt, da, db, m, n, k, layout, SK, out=t0g.BF16)
        c_dp = _run(rt, da, db, m, n, k, layout, DP, out=t0g.BF16)
        assert np.array_equal(c_sk, c_dp)
    finally:
        rt.free(da)
        rt.free(db)


def test_stream_k_mlp_shape_sampled_rows(rt):
    """The MLP forward shape the schedule is for (1024 x 11008 x 4096, 172 tiles):
    oracle rows sampled across all four tile rows."""
    m, n, k = 1024, 11008, 4096
    a_st, b_st = _operands("NN", m, n, k, 5)
    da, db = rt.upload(a_st), rt.upload(b_st)
    try:
        c = _run(rt, da, db, m, n, k, "NN", SK)
        rows = np.array([0, 1, 255, 256, 300, 511, 512, 777, 1023])
        ref = o.gemm_rows("NN", a_st, b_st, m, n, k, rows)
        ok, relf, maxabs, bound = o.parity(c[rows], ref, k)
        _log(f"[parity] stream-K MLP rows: relF={relf:.3e} max|d|={maxabs:.3e}")
        assert ok
    finally:
        rt.free(da)
        rt.free(db)


def test_stream_k_epilogue_chain_after_fixup(rt):
    m, n, k = 512, 768, 1000
    a_st, b_st = _operands("NT", m, n, k, 9)
    bias = np.linspace(-1, 1, n, dtype=np.float32)
    da, db, dbias = rt.upload(a_st), rt.upload(b_st), rt.upload(bias)
    try:
        kw = dict(epilogue_ops=["bias", "silu"], bias=dbias)
        c = _run(rt, da, db, m, n, k, "NT", SK, **kw)
        ref = o.epilogue_chain(o.gemm("NT", a_st, b_st, m, n, k), ["bias", "silu"], bias=bias)
        ok, relf, maxabs, _ = o.parity(c, ref, k)
        assert ok, f"relF={relf:.3e} max|d|={maxabs:.3e}"
        c16 = _run(rt, da, db, m, n, k, "NT", SK, out=t0g.BF16, **kw)
        assert np.array_equal(c16, o.f32_to_bf16_rne(c))
    finally:
        for x in (da, db, dbias):
            rt.free(x)


def test_stream_k_back_to_back_launches(rt):
    """Different shapes queued without waiting in between: each launch finds the
    ticket counter and ready flags at zero."""
    cases = [(512, 768, 1000, "NT"), (1024, 2816, 4096, "NN"), (256, 256, 64, "TT"), (512, 768, 1000, "NT")]
    bufs, outs = [], []
    try:
        for i, (m, n, k, lay) in enumerate(cases):
            a_st, b_st = _operands(lay, m, n, k, 100 + (i % 3))
            da, db, dc = rt.upload(a_st), rt.upload(b_st), rt.alloc(m * n * 4)
            bufs += [da, db, dc]
            outs.append((dc, a_st, b_st, m, n, k, lay))
        for dc, a_st, b_st, m, n, k, lay in outs:
            rt.gemm(bufs[bufs.index(dc) - 2], bufs[bufs.index(dc) - 1], dc, m, n, k, transpose=lay, config=SK)
        rt.wait_idle()
        for dc, a_st, b_st, m, n, k, lay in outs:
            c = rt.read(dc, (m, n), np.float32)
            ok, relf, maxabs, _ = o.parity(c, o.gemm(lay, a_st, b_st, m, n, k), k)
            assert ok, f"{lay} {m}x{n}x{k}: relF={relf:.3e} max|d|={maxabs:.3e}"
    finally:
        for x in bufs:
            rt.free(x)
