"""The 64x64 deep ring with K split across its four waves (kernels _ds and _dsr), which
the planner takes for K slices of 24 stages of 64 or more: every layout, no split and
split-K (planes + reduce kernel, the two-slice sum and the general in-kernel sum), K
tails, ragged edges and both outputs, against the CPU oracle.  Each case also runs
twice (the same bits) and, where it splits, once more with planes + reduce kernel,
whose bits every in-kernel form must equal (the sum is in plane order either way).
The operands are U(-0.5, 0.5) rounded to bf16, so the sums cancel as in the benchmark
data; the random sweep elsewhere stays below 24 stages and never reaches these kernels."""
import sys

import numpy as np
import pytest

import oracle as o
import t0g

pytestmark = pytest.mark.gpu

P64 = t0g.GemmConfig.preset("gfx950_64x64_k64")
AUTO, REDUCE, IN_KERNEL = t0g.SPLIT_K_AUTO, t0g.SPLIT_K_REDUCE_KERNEL, t0g.SPLIT_K_IN_KERNEL

# layout, M, N, K, split, split-K mode, kernel suffix
CASES = [
    ("NT", 256, 256, 2048, 1, AUTO, "_ds"),         # 16 tiles, 32 stages each, no split
    ("NN", 192, 320, 6200, 4, REDUCE, "_ds"),       # slices of 1600 (25 stages), 1400 in the last
    ("TN", 104, 200, 3100, 2, AUTO, "_dsr"),        # ragged edges, two slices summed in the kernel, K tail
    ("TT", 200, 136, 6000, 4, IN_KERNEL, "_dsr"),   # four slices summed in the kernel (chunk claims)
    ("NT", 64, 64, 16384, 8, REDUCE, "_ds"),        # a single tile in 8 slices of 32 stages
    ("NN", 128, 4096, 4096, 2, AUTO, "_dsr"),       # benchmark config 4a's shape, NN
]


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def rt():
    r = t0g.GpuRuntime.new(0)
    yield r
    t0g.set_split_k_mode(AUTO)
    r.close()


def _uniform_half(n, seed):
    rng = np.random.default_rng(seed)
    return o.f32_to_bf16_rne(rng.random(n, dtype=np.float32) - np.float32(0.5))


def _run(rt, da, db, m, n, k, layout, split, out, mode):
    t0g.set_split_k_mode(mode)
    try:
        d = t0g.gemm_desc(da, db, 0, m, n, k, transpose=layout, out_dtype=out, config=P64, split_k=split)
        name = t0g.gemm_kernel_name(d)
        esz, dt = (2, np.uint16) if out == t0g.BF16 else (4, np.float32)
        dc = rt.alloc(m * n * esz)
        try:
            rt.memset(dc, 0xFF, m * n * esz)
            d.c = dc
            rt.gemm_desc(d)
            rt.wait_idle()
            return name, rt.read(dc, (m, n), dt)
        finally:
            rt.free(dc)
    finally:
        t0g.set_split_k_mode(AUTO)


@pytest.mark.parametrize("out", [t0g.F32, t0g.BF16])
@pytest.mark.parametrize("layout,m,n,k,split,mode,sfx", CASES)
def test_k_split_kernels_against_the_oracle(rt, layout, m, n, k, split, mode, sfx, out):
    _log(f"[case] K split across the waves: {layout} {m}x{n}x{k} split {split} mode {mode} out {out}")
    a_mk = _uniform_half(m * k, 11 + m + k).reshape(m, k)
    b_nk = _uniform_half(n * k, 13 + n + k).reshape(n, k)
    a_st = a_mk if layout[0] == "N" else np.ascontiguousarray(a_mk.T)
    b_st = b_nk if layout[1] == "T" else np.ascontiguousarray(b_nk.T)
    da, db = rt.upload(a_st), rt.upload(b_st)
    try:
        name, got = _run(rt, da, db, m, n, k, layout, split, out, mode)
        assert name.startswith("t0g_gemm_64x64_k64_") and name.endswith(sfx), name
        _, again = _run(rt, da, db, m, n, k, layout, split, out, mode)
        assert np.array_equal(got, again), f"{name}: a second run differs"
        if split > 1:
            name_p, planes = _run(rt, da, db, m, n, k, layout, split, out, REDUCE)
            assert name_p.endswith("_ds"), name_p
            assert np.array_equal(got, planes), f"{name} differs from {name_p} + reduce kernel"
        ref = o.gemm("NT", a_mk, b_nk, m, n, k)
        c = got if out == t0g.F32 else o.bf16_to_f32(got)
        ok, relf, maxabs, bound = o.parity(c, ref, k)
        _log(f"[parity] {name}: relF={relf:.3e} max|d|={maxabs:.3e} (bound {bound:.3e})")
        assert ok if out == t0g.F32 else relf <= 5e-3
        if out == t0g.BF16:
            # the bf16 output is RNE of the same kernel's fp32 result
            _, f32 = _run(rt, da, db, m, n, k, layout, split, t0g.F32, mode)
            assert np.array_equal(got, o.f32_to_bf16_rne(f32))
    finally:
        rt.free(da)
        rt.free(db)


@pytest.mark.parametrize("layout,m,n,k,split,mode,sfx", [
    ("NT", 256, 256, 2048, 1, AUTO, "_ds"),        # the chain in the GEMM kernel's own store
    ("TN", 104, 200, 3100, 2, AUTO, "_dsr"),       # applied once, after the two-slice sum
    ("NN", 192, 320, 6200, 4, REDUCE, "_ds"),      # applied by the reduce kernel
])
def test_k_split_kernels_with_an_epilogue_chain(rt, layout, m, n, k, split, mode, sfx):
    """bias + SiLU + scale + clamp on the K-split kernels, f32 against the oracle's chain and
    bf16 equal to RNE of the same kernel's f32 output."""
    _log(f"[case] K split + epilogue chain: {layout} {m}x{n}x{k} split {split} mode {mode}")
    a_mk = _uniform_half(m * k, 17 + m + k).reshape(m, k)
    b_nk = _uniform_half(n * k, 19 + n + k).reshape(n, k)
    a_st = a_mk if layout[0] == "N" else np.ascontiguousarray(a_mk.T)
    b_st = b_nk if layout[1] == "T" else np.ascontiguousarray(b_nk.T)
    bias = ((np.arange(n, dtype=np.float32) % 5) - 2.0) * 0.25
    ops = ["bias", "silu", "scale", "clamp"]
    da, db, dbias = rt.upload(a_st), rt.upload(b_st), rt.upload(bias)
    outs = {}
    try:
        t0g.set_split_k_mode(mode)
        for out, esz, dt in ((t0g.F32, 4, np.float32), (t0g.BF16, 2, np.uint16)):
            d = t0g.gemm_desc(da, db, 0, m, n, k, transpose=layout, out_dtype=out, config=P64, split_k=split,
                              epilogue_ops=ops, bias=dbias, epi_scale=1.5, clamp=(-0.2, 0.6))
            name = t0g.gemm_kernel_name(d)
            assert name.startswith("t0g_gemm_64x64_k64_") and name.endswith(sfx), name
            dc = rt.alloc(m * n * esz)
            try:
                rt.memset(dc, 0xFF, m * n * esz)
                d.c = dc
                rt.gemm_desc(d)
                rt.wait_idle()
                outs[out] = rt.read(dc, (m, n), dt)
            finally:
                rt.free(dc)
    finally:
        t0g.set_split_k_mode(AUTO)
        for x in (da, db, dbias):
            rt.free(x)
    ref = o.epilogue_chain(o.gemm("NT", a_mk, b_nk, m, n, k), ops, bias=bias, scale=1.5, clamp=(-0.2, 0.6))
    ok, relf, maxabs, bound = o.parity(outs[t0g.F32], ref, k)
    _log(f"[parity] chain: relF={relf:.3e} max|d|={maxabs:.3e} (bound {bound:.3e})")
    assert ok
    assert np.array_equal(outs[t0g.BF16], o.f32_to_bf16_rne(outs[t0g.F32]))
