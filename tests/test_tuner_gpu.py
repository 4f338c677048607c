"""GEMM autotuner on the GPU (src/t0/auto_gemm.rs:82-238, 445-480): benchmark,
cache hit, disk persistence, auto_gemm's result against the oracle, and every
config the tuner may pick computing the same product within the parity gate."""
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


def test_tune_4096(rt, tmp_path):
    """test_tune_4096 (auto_gemm.rs:544-577): 4 candidates, 3 iterations; the best is
    fast, the ranking is sorted and made of candidates, the second call is a cache hit and
    a new tuner finds the result on disk."""
    _log("[case] tune 4096^3 NT f32")
    with t0g.GemmTuner.with_cache_dir(tmp_path / "tune") as tuner:
        tuner.max_candidates = 4
        tuner.n_iters = 3
        cfg = tuner.tune(rt, 4096, 4096, 4096)
        r = tuner.lookup(4096, 4096, 4096)
        ranking = tuner.ranking(4096, 4096, 4096)
        _log(f"[tune] best {cfg.name()} {r.best_tflops:.1f} TF; ranking {ranking}")
        assert r.from_cache == 0
        assert r.best_tflops > 500.0
        assert ranking[0][0] == cfg.name()
        assert [t for _, t in ranking] == sorted((t for _, t in ranking), reverse=True)
        cand_names = [c.name() for c in t0g.tune_candidates(4096, 4096, 4096, "NT", 4)]
        assert len(ranking) == 4 and {n for n, _ in ranking} == set(cand_names)
        assert tuner.tune(rt, 4096, 4096, 4096).name() == cfg.name()
        assert (tmp_path / "tune" / "gemm_4096x4096x4096.json").exists()
    with t0g.GemmTuner.with_cache_dir(tmp_path / "tune") as again:
        r2 = again.lookup(4096, 4096, 4096)
        assert r2.from_cache == 1 and r2.best.name() == cfg.name()
        assert abs(r2.best_tflops - r.best_tflops) < 0.01
        assert again.tune(rt, 4096, 4096, 4096).name() == cfg.name()


def test_auto_gemm_matches_the_oracle(rt, tmp_path):
    """auto_gemm(rt, a, b, c, m, n, k): NT, f32 output, with the tuned config."""
    m, n, k = 512, 384, 1024
    _log(f"[case] auto_gemm {m}x{n}x{k}")
    a = o.rand_bf16_xorshift(m * k, m * 1000 + k).reshape(m, k)
    b = o.rand_bf16_xorshift(n * k, n * 2000 + k).reshape(n, k)
    ref = o.gemm("NT", a, b, m, n, k)
    da, db = rt.upload(a), rt.upload(b)
    dc = rt.alloc(m * n * 4)
    try:
        with t0g.GemmTuner.with_cache_dir(tmp_path / "auto") as tuner:
            tuner.max_candidates = 3
            tuner.n_iters = 3
            for attempt in range(2):
                rt.memset(dc, 0, m * n * 4)
                tf = t0g.auto_gemm(rt, da, db, dc, m, n, k, tuner=tuner)
                c = rt.read(dc, (m, n), np.float32)
                ok, relf, maxabs, bound = o.parity(c, ref, k)
                _log(f"[parity] auto_gemm call {attempt}: {tf:.1f} TF relF={relf:.3e} max|d|={maxabs:.3e}")
                assert ok and tf > 0
            assert len(tuner) == 1
    finally:
        for x in (da, db, dc):
            rt.free(x)


@pytest.mark.parametrize("layout,out", [("NT", t0g.F32), ("NN", t0g.BF16), ("TN", t0g.F32)])
def test_every_candidate_computes_the_same_product(rt, layout, out):
    """Whatever the tuner picks, the result passes the parity gate: each candidate config
    of a 320x256x2048 problem runs through t0g_gemm and is checked against the oracle;
    bf16 outputs must be RNE of the candidate's own fp32 output."""
    m, n, k = 320, 256, 2048
    a_mk = o.rand_bf16_xorshift(m * k, 11).reshape(m, k)
    b_nk = o.rand_bf16_xorshift(n * k, 12).reshape(n, k)
    ref = o.gemm("NT", a_mk, b_nk, m, n, k)
    a_st = a_mk if layout in ("NT", "NN") else np.ascontiguousarray(a_mk.T)
    b_st = b_nk if layout in ("NT", "TT") else np.ascontiguousarray(b_nk.T)
    da, db = rt.upload(a_st), rt.upload(b_st)
    dc = rt.alloc(m * n * 4)
    dc16 = rt.alloc(m * n * 2)
    try:
        cands = t0g.tune_candidates(m, n, k, layout, 64)
        assert len(cands) >= 3
        for cfg in cands:
            _log(f"[case] candidate {cfg.name()} {layout}")
            rt.gemm(da, db, dc, m, n, k, transpose=layout, config=cfg)
            if out == t0g.BF16:
                rt.gemm(da, db, dc16, m, n, k, transpose=layout, config=cfg, out_dtype=t0g.BF16)
            rt.wait_idle()
            c = rt.read(dc, (m, n), np.float32)
            ok, relf, maxabs, bound = o.parity(c, ref, k)
            assert ok, f"{cfg.name()}: relF={relf:.3e} max|d|={maxabs:.3e}"
            if out == t0g.BF16:
                assert np.array_equal(rt.read(dc16, (m, n), np.uint16), o.f32_to_bf16_rne(c)), cfg.name()
    finally:
        for x in (da, db, dc, dc16):
            rt.free(x)


def test_tune_other_layout_and_output(rt, tmp_path):
    with t0g.GemmTuner.with_cache_dir(tmp_path / "nn") as tuner:
        tuner.max_candidates = 3
        tuner.n_iters = 2
        cfg = tuner.tune(rt, 1024, 2048, 512, transpose="NN", out_dtype=t0g.BF16)
        assert cfg.transpose == t0g.NN
        assert (tmp_path / "nn" / "gemm_1024x2048x512_nn_bf16.json").exists()
        assert tuner.lookup(1024, 2048, 512) is None
