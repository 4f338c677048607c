"""Seeded sweep of random GEMM problems through t0g_gemm against the CPU oracle.

Each case draws a layout (NT/NN/TN/TT), M, N and K, a config (auto_select's or one of
the three tiles), a split-K count, padded leading dimensions (some of them not a
multiple of 8, which routes the operands to the element-wise kernels) and the
output type; every third case also an epilogue chain of one to four ops with
random bias, scale and clamp bounds (checked against the oracle's restatement of
the chain).  Even cases draw A and B from the reference's LCG (one-sided, U[-0.5, 0]); odd
cases from U(-0.5, 0.5), rounded to bf16, so sums cancel as they do in the benchmark's
data.  Checked per case: parity of the fp32 result with the oracle
(relF <= 5e-3, max|d| <= 1e-2 sqrt(K/256)), a second run equal bit for bit, and
for bf16 output, equality with RNE of the same config's fp32 output.  The padding
columns hold random values, so a kernel that reads past the logical operand
breaks parity."""
import sys

import numpy as np
import pytest

import oracle as o
import t0g

pytestmark = pytest.mark.gpu

import os

# T0G_SWEEP_CASES / T0G_SWEEP_SEED0: a longer sweep, or another slice of seeds, for
# one-off correctness runs; the default is the committed 48-case sweep.
N_CASES = int(os.environ.get("T0G_SWEEP_CASES", "48"))
SEED0 = int(os.environ.get("T0G_SWEEP_SEED0", "1000"))
PRESETS = [None, "gfx950_256x256_k64", "gfx950_128x128_k64", "gfx950_64x64_k64"]


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def rt():
    r = t0g.GpuRuntime.new(0)
    yield r
    r.close()


def _case(i):
    rng = np.random.default_rng(SEED0 + i)
    layout = ["NT", "NN", "TN", "TT"][i % 4]
    m = int(rng.integers(1, 701))
    n = int(rng.integers(1, 701))
    k = int(rng.integers(1, 1201))
    preset = PRESETS[int(rng.integers(0, len(PRESETS)))]
    splits = [s for s in (1, 2, 3, 4, 8) if s == 1 or k >= s * 64]
    split = 0 if preset is None else int(rng.choice(splits))
    pads = [int(rng.choice([0, 0, 8, 13])) for _ in range(3)]
    out = t0g.BF16 if rng.integers(0, 2) else t0g.F32
    chain = None
    if i % 3 == 2:
        names = ["bias", "scale", "relu", "silu", "gelu", "abs", "neg", "clamp"]
        chain = [names[int(x)] for x in rng.integers(0, len(names), int(rng.integers(1, 5)))]
    return rng, layout, m, n, k, preset, split, pads, out, chain


def _stored(logical, pad, rng):
    """logical [rows][cols] bf16 bits in a [rows][cols + pad] array whose padding holds random bf16."""
    rows, cols = logical.shape
    full = o.rand_bf16_lcg(rows * (cols + pad), int(rng.integers(1, 1 << 30))).reshape(rows, cols + pad)
    full[:, :cols] = logical
    return np.ascontiguousarray(full)


# Long K on the 64x64 tile: K a multiple of 8 from 1536 to 5000 and M, N up to 400, so the
# grid stays at one workgroup per CU and slices of 24 stages or more reach the deep ring's
# K-split kernels (_ds, and _dsr where two slices are summed in the kernel); the short-K
# sweep above never gets there.  Padding of 13 elements still sends some cases to the
# element-wise kernels.  16 committed; 120 pass with T0G_SWEEP_LONG_CASES=120.
N_LONG = int(os.environ.get("T0G_SWEEP_LONG_CASES", "16"))


def _case_long(j):
    rng = np.random.default_rng(SEED0 + 50000 + j)
    layout = ["NT", "NN", "TN", "TT"][j % 4]
    # M (N) is the contiguous dimension of A (B) in TN/TT (NN/TN): a multiple of 8 there keeps
    # the rows 16-byte aligned for the fast kernels; elsewhere it is ragged
    m = 8 * int(rng.integers(1, 51)) if layout in ("TN", "TT") else int(rng.integers(1, 401))
    n = 8 * int(rng.integers(1, 51)) if layout in ("NN", "TN") else int(rng.integers(1, 401))
    k = 8 * int(rng.integers(192, 626))
    preset = "gfx950_64x64_k64" if j % 8 != 7 else None
    split = 0 if preset is None else int(rng.choice([1, 1, 2, 2, 4]))
    pads = [int(rng.choice([0, 0, 0, 8, 8, 13])) if j % 4 == 2 else int(rng.choice([0, 0, 8])) for _ in range(3)]
    out = t0g.BF16 if rng.integers(0, 2) else t0g.F32
    chain = None
    if j % 3 == 1:
        names = ["bias", "scale", "relu", "silu", "gelu", "abs", "neg", "clamp"]
        chain = [names[int(x)] for x in rng.integers(0, len(names), int(rng.integers(1, 5)))]
    return rng, layout, m, n, k, preset, split, pads, out, chain


def _plan_name(case):
    _, layout, m, n, k, preset, split, pads, out, chain = case
    a_cols = (k if layout in ("NT", "NN") else m) + pads[0]
    b_cols = (k if layout in ("NT", "TT") else n) + pads[1]
    kw = dict(transpose=layout, lda=a_cols, ldb=b_cols, ldc=n + pads[2], split_k=split, out_dtype=t0g.F32)
    if preset is not None:
        kw["config"] = t0g.GemmConfig.preset(preset)
    if chain:
        kw.update(epilogue_ops=chain, bias=0x40000)
    return t0g.gemm_kernel_name(t0g.gemm_desc(0x10000, 0x20000, 0x30000, m, n, k, **kw))


def test_long_k_sweep_reaches_the_k_split_kernels():
    names = [_plan_name(_case_long(j)) for j in range(N_LONG)]
    assert sum(nm.endswith(("_ds", "_dsr")) for nm in names) >= N_LONG // 3, names


@pytest.mark.parametrize("j", range(N_LONG))
def test_random_problem_long_k(rt, j):
    _check(rt, 1000 + j, _case_long(j), f"long-K sweep {j}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_problem(rt, i):
    _check(rt, i, _case(i), f"sweep {i}")


def _check(rt, i, case, tag):
    rng, layout, m, n, k, preset, split, pads, out, chain = case
    _log(f"[case] {tag}: {layout} {m}x{n}x{k} data={'lcg' if i % 2 == 0 else 'two-sided'} "
         f"preset={preset} split={split} pads={pads} "
         f"out={'bf16' if out == t0g.BF16 else 'f32'} chain={chain}")
    if i % 2 == 0:
        a_mk = o.rand_bf16_lcg(m * k, 7 * i + 1).reshape(m, k)
        b_nk = o.rand_bf16_lcg(n * k, 7 * i + 2).reshape(n, k)
    else:
        drng = np.random.default_rng(SEED0 + 7919 + i)
        a_mk = o.f32_to_bf16_rne(drng.uniform(-0.5, 0.5, (m, k)).astype(np.float32))
        b_nk = o.f32_to_bf16_rne(drng.uniform(-0.5, 0.5, (n, k)).astype(np.float32))
    a_log = a_mk if layout in ("NT", "NN") else np.ascontiguousarray(a_mk.T)
    b_log = b_nk if layout in ("NT", "TT") else np.ascontiguousarray(b_nk.T)
    a_st = _stored(a_log, pads[0], rng)
    b_st = _stored(b_log, pads[1], rng)
    lda, ldb, ldc = a_st.shape[1], b_st.shape[1], n + pads[2]
    kw = dict(transpose=layout, lda=lda, ldb=ldb, ldc=ldc, split_k=split)
    if preset is not None:
        kw["config"] = t0g.GemmConfig.preset(preset)
    bias = None
    if chain:
        bias = (rng.standard_normal(n) * 0.05).astype(np.float32)
        scale = float(rng.uniform(-2.0, 2.0))
        lo = float(rng.uniform(-0.1, 0.0))
        kw.update(epilogue_ops=chain, epi_scale=scale, clamp=(lo, lo + float(rng.uniform(0.01, 0.2))))
    da, db = rt.upload(a_st), rt.upload(b_st)
    dc = rt.alloc(m * ldc * 4)
    dc2 = rt.alloc(m * ldc * 4)
    dbias = rt.upload(bias) if bias is not None else 0
    if bias is not None:
        kw["bias"] = dbias
    try:
        desc = t0g.gemm_desc(da, db, dc, m, n, k, out_dtype=t0g.F32, **kw)
        _log(f"[kernel] {t0g.gemm_kernel_name(desc)}")
        rt.memset(dc, 0xFF, m * ldc * 4)
        rt.gemm(da, db, dc, m, n, k, out_dtype=t0g.F32, **kw)
        rt.memset(dc2, 0, m * ldc * 4)
        rt.gemm(da, db, dc2, m, n, k, out_dtype=t0g.F32, **kw)
        rt.wait_idle()
        c = rt.read(dc, (m, ldc), np.float32)[:, :n]
        c2 = rt.read(dc2, (m, ldc), np.float32)[:, :n]
        assert np.array_equal(c.view(np.uint32), c2.view(np.uint32)), "two runs differ"
        ref = o.gemm("NT", a_mk, b_nk, m, n, k)
        if chain:
            ref = o.epilogue_chain(ref, chain, bias=bias, scale=kw["epi_scale"], clamp=kw["clamp"])
        ok, relf, maxabs, bound = o.parity(c, ref, k)
        _log(f"[parity] {tag}: relF={relf:.3e} max|d|={maxabs:.3e} (bound {bound:.3e})")
        assert ok, f"relF={relf:.3e} max|d|={maxabs:.3e} bound={bound:.3e}"
        if out == t0g.BF16:
            rt.memset(dc2, 0xFF, m * ldc * 2)
            rt.gemm(da, db, dc2, m, n, k, out_dtype=t0g.BF16, **kw)
            rt.wait_idle()
            c16 = rt.read(dc2, (m, ldc), np.uint16)[:, :n]
            assert np.array_equal(c16, o.f32_to_bf16_rne(c)), "bf16 output is not RNE of the fp32 output"
    finally:
        for x in (da, db, dc, dc2, dbias):
            if x:
                rt.free(x)
