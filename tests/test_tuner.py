"""GEMM autotuner: the on-disk cache, the candidate list and the tuner API
(src/t0/auto_gemm.rs), host side.  The benchmark itself runs in
test_tuner_gpu.py."""
import json
import os

import pytest

import t0g


def _tuner(tmp_path, sub="cache"):
    return t0g.GemmTuner.with_cache_dir(tmp_path / sub)


def test_tuner_new():
    """test_tuner_new (auto_gemm.rs:535-541): 8 candidates, 5 iterations, empty."""
    with t0g.GemmTuner.new() as t:
        assert t.max_candidates == 8
        assert t.n_iters == 5
        assert len(t) == 0


def test_cache_dir_default(monkeypatch):
    """test_cache_dir_default (auto_gemm.rs:529-533) and default_cache_dir (484-490)."""
    monkeypatch.setenv("HOME", "/some/home")
    with t0g.GemmTuner.new() as t:
        assert t.cache_dir == "/some/home/.t0_autotune"
        assert "t0_autotune" in t.cache_dir
    monkeypatch.delenv("HOME")
    with t0g.GemmTuner.new() as t:
        assert t.cache_dir == "/tmp/.t0_autotune"


def test_params_are_settable_and_checked(tmp_path):
    with _tuner(tmp_path) as t:
        t.max_candidates = 4
        t.n_iters = 3
        assert (t.max_candidates, t.n_iters) == (4, 3)
        with pytest.raises(t0g.T0gError) as e:
            t.n_iters = 0
        assert e.value.code == t0g.ERR_INVALID_ARG


def test_cache_roundtrip(tmp_path):
    """test_cache_roundtrip (auto_gemm.rs:580-610): save, then a new tuner on the same
    directory loads the same config and TFLOPS, marked from_cache, with its ranking."""
    cfg = t0g.GemmConfig.preset("gfx950_128x128_k64").copy(split_k=4)
    ranking = [(cfg.name(), 79.2), ("t0_gemm_64x64_k64_ldsdb", 65.3)]
    with _tuner(tmp_path) as t:
        t.save_cache(4096, 4096, 4096, cfg, 79.2, ranking)
        r = t.lookup(4096, 4096, 4096)
        assert r is not None and r.from_cache == 0
    with _tuner(tmp_path) as t2:
        r = t2.lookup(4096, 4096, 4096)
        assert r is not None
        assert (r.best.tile_m, r.best.tile_n, r.best.tile_k, r.best.split_k) == (128, 128, 64, 4)
        assert abs(r.best_tflops - 79.2) < 0.1
        assert r.from_cache == 1
        assert r.best.name() == cfg.name()
        assert t2.ranking(4096, 4096, 4096) == [(n, pytest.approx(v, abs=0.01)) for n, v in ranking]
        assert len(t2) == 1
        assert "[cached]" in t2.report()


def test_cache_file_keeps_the_reference_keys(tmp_path):
    """The file holds every key save_cache writes (auto_gemm.rs:373-386), parseable as
    JSON, plus the architecture, layout, output type and size."""
    cfg = t0g.GemmConfig.preset("gfx950_256x256_k64")
    with _tuner(tmp_path) as t:
        t.save_cache(1024, 11008, 4096, cfg, 991.44, [(cfg.name(), 991.44)])
    path = tmp_path / "cache" / "gemm_1024x11008x4096.json"
    js = json.loads(path.read_text())
    for key in ("tile_m", "tile_n", "tile_k", "wg_size", "split_k", "lds_pad", "n_col_passes", "wgp", "swap",
                "tflops", "all"):
        assert key in js, key
    assert js["split_k"] == 1 and js["swap"] is True and js["wgp"] is False
    assert js["arch"] == "gfx950" and js["layout"] == "nt" and js["out"] == "f32"
    assert (js["m"], js["n"], js["k"]) == (1024, 11008, 4096)
    assert js["all"] == [[cfg.name(), 991.44]]


def test_file_names_per_layout_and_output(tmp_path):
    cfg = t0g.GemmConfig.preset("gfx950_64x64_k64")
    with _tuner(tmp_path) as t:
        t.save_cache(64, 128, 256, cfg, 1.0, transpose="NN", out_dtype=t0g.BF16)
        t.save_cache(64, 128, 256, cfg, 2.0, transpose="TN")
        t.save_cache(64, 128, 256, cfg, 3.0)
        assert t.lookup(64, 128, 256, "NN", t0g.BF16).best.transpose == t0g.NN
        assert t.lookup(64, 128, 256, "NN") is None
    assert sorted(os.listdir(tmp_path / "cache")) == [
        "gemm_64x128x256.json", "gemm_64x128x256_nn_bf16.json", "gemm_64x128x256_tn.json"]


def _write(tmp_path, name, text):
    d = tmp_path / "cache"
    d.mkdir(exist_ok=True)
    (d / name).write_text(text)


def test_reference_written_file_is_a_miss(tmp_path):
    """A file the gfx1100 build wrote (the JSON of the reference's test_parse_json_helpers,
    auto_gemm.rs:518-526, has no architecture and an RDNA3 tile) is not used here."""
    _write(tmp_path, "gemm_4096x4096x4096.json",
           '{"tile_m":128,"tile_n":64,"tile_k":32,"wg_size":128,"tflops":79.21,"split_k":1}')
    with _tuner(tmp_path) as t:
        assert t.lookup(4096, 4096, 4096) is None


def test_gfx1100_tile_with_gfx950_tag_is_a_miss(tmp_path):
    _write(tmp_path, "gemm_4096x4096x4096.json",
           '{"tile_m":128,"tile_n":64,"tile_k":32,"wg_size":128,"tflops":79.21,"split_k":1,"arch":"gfx950"}')
    with _tuner(tmp_path) as t:
        assert t.lookup(4096, 4096, 4096) is None


def test_hand_written_file_with_whitespace_loads(tmp_path):
    _write(tmp_path, "gemm_512x512x512.json",
           '{\n  "tile_m": 64, "tile_n": 64, "tile_k": 64, "wg_size": 256,\n  "split_k": 2,\n'
           '  "tflops": 12.5, "arch": "gfx950",\n  "all": [ ["a", 12.5] , ["b",3] ]\n}\n')
    with _tuner(tmp_path) as t:
        r = t.lookup(512, 512, 512)
        assert r is not None and r.best.name() == "t0_gemm_64x64_k64_ldsdb_sk2"
        assert r.best_tflops == 12.5
        assert t.ranking(512, 512, 512) == [("a", 12.5), ("b", 3.0)]


@pytest.mark.parametrize("text", [
    "", "{", '{"tile_m":', '{"tile_m":256,"tile_n":256,"tile_k":64,"arch":"gfx950"}',
    '{"tile_m":256,"tile_n":256,"tile_k":64,"wg_size":512,"tflops":1,"arch":"gfx950","m":1}',
    '{"tile_m":256,"tile_n":256,"tile_k":64,"wg_size":512,"tflops":1,"arch":"gfx950","layout":"nn"}',
    '{"tile_m":99999999999,"tile_n":256,"tile_k":64,"wg_size":512,"tflops":1,"arch":"gfx950"}',
    '{"tile_m":256,"tile_n":256,"tile_k":64,"wg_size":512,"tflops":1,"arch":"gfx950","split_k":3}',
])
def test_broken_or_foreign_files_are_misses(tmp_path, text):
    _write(tmp_path, "gemm_4096x4096x4096.json", text)
    with _tuner(tmp_path) as t:
        assert t.lookup(4096, 4096, 4096) is None


def test_broken_ranking_keeps_the_config(tmp_path):
    _write(tmp_path, "gemm_8x8x8.json",
           '{"tile_m":64,"tile_n":64,"tile_k":64,"wg_size":256,"tflops":1.5,"arch":"gfx950","all":[["x",]]}')
    with _tuner(tmp_path) as t:
        r = t.lookup(8, 8, 8)
        assert r is not None and r.n_all == 0


def test_invalidate_and_clear(tmp_path):
    """invalidate / clear (auto_gemm.rs:393-403); clear leaves files it did not write."""
    cfg = t0g.GemmConfig.preset("gfx950_128x128_k64")
    with _tuner(tmp_path) as t:
        t.save_cache(256, 256, 256, cfg, 1.0)
        t.save_cache(512, 512, 512, cfg, 2.0)
        t.invalidate(256, 256, 256)
        assert t.lookup(256, 256, 256) is None
        assert not (tmp_path / "cache" / "gemm_256x256x256.json").exists()
        assert t.lookup(512, 512, 512) is not None
        t.clear()
        assert len(t) == 0
        assert not (tmp_path / "cache").exists()
        t.save_cache(512, 512, 512, cfg, 2.0)
        t.save_tile_ir_cache(512, 512, 512, cfg, 2.0)
        _write(tmp_path, "notes.json", "{}")
        t.clear()
        assert os.listdir(tmp_path / "cache") == ["notes.json"]   # gemm_* and tile_ir_* are this tuner's


def test_store_rejects_bad_input(tmp_path):
    with _tuner(tmp_path) as t:
        bad = t0g.GemmConfig.preset("gfx950_128x128_k64").copy(tile_m=96)
        with pytest.raises(t0g.T0gError) as e:
            t.save_cache(64, 64, 64, bad, 1.0)
        assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG
        with pytest.raises(t0g.T0gError) as e:
            t.save_cache(0, 64, 64, t0g.GemmConfig.preset("gfx950_64x64_k64"), 1.0)
        assert e.value.code == t0g.ERR_INVALID_ARG
        with pytest.raises(t0g.T0gError):
            t.save_cache(64, 64, 64, t0g.GemmConfig.preset("gfx950_64x64_k64"), 1.0, [('a"b', 1.0)])
        with pytest.raises(t0g.T0gError):
            t.lookup(64, 64, 64, transpose=7)


def test_unwritable_directory_is_an_error_for_store(tmp_path):
    (tmp_path / "file").write_text("x")
    with t0g.GemmTuner.with_cache_dir(tmp_path / "file" / "sub") as t:
        with pytest.raises(t0g.T0gError):
            t.save_cache(64, 64, 64, t0g.GemmConfig.preset("gfx950_64x64_k64"), 1.0)


SHAPES = [(256, 256, 256), (4096, 4096, 4096), (8192, 8192, 8192), (128, 4096, 4096), (256, 256, 32768),
          (1024, 11008, 4096), (1024, 4096, 11008), (11008, 4096, 1024), (4096, 11008, 1024), (100, 300, 72)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_candidates_start_with_auto_select(m, n, k):
    """The benchmark list is the model's ranking: its head is auto_select's choice (for the
    NT layout), every entry is a valid distinct config, splits keep >= 4 K tiles each."""
    cands = t0g.tune_candidates(m, n, k, "NT", 64)
    assert cands[0].name() == t0g.auto_select(m, k, n).name()
    names = [c.name() for c in cands]
    assert len(set(names)) == len(names)
    for c in cands:
        c.validate()
        sk = max(1, c.split_k)
        assert sk == 1 or sk == t0g.STREAM_K or k >= sk * 4 * 64
    assert sum(c.split_k == t0g.STREAM_K for c in cands) == 1
    assert len(t0g.tune_candidates(m, n, k, "NT", 3)) == min(3, len(cands))
    assert all(c.transpose == t0g.TN for c in t0g.tune_candidates(m, n, k, "TN", 8))


def test_candidates_cover_every_tile():
    cands = t0g.tune_candidates(4096, 4096, 4096, "NT", 64)
    assert {(c.tile_m, c.tile_n) for c in cands} == {(256, 256), (128, 128), (64, 64)}
    assert len(cands) == 3 * 5 + 1   # 3 tiles x split 1..16 (64 K tiles, >= 4 per split), and stream-K


# ---- tune_tile_ir's cache (src/t0/cost_model.rs:1030-1097) ----------------------

def test_tile_ir_cache_roundtrip(tmp_path):
    """save_tile_ir_cache then load_tile_ir_cache on a new tuner: the same tile, split
    and TFLOPS, from_cache, the TileGemm-named ranking (cost_model.rs:1076-1093)."""
    cfg = t0g.GemmConfig.preset("gfx950_128x128_k64").copy(split_k=8)
    ranking = [(t0g.tile_config_name(cfg), 271.3), ("tile_gemm_64x64_k64_db_sk2", 200.0)]
    with _tuner(tmp_path) as t:
        t.save_tile_ir_cache(128, 4096, 4096, cfg, 271.3, ranking)
        assert t.tile_ir_lookup(128, 4096, 4096).from_cache == 0
        assert t.lookup(128, 4096, 4096) is None          # a separate cache from GemmTuner's
    js = json.loads((tmp_path / "cache" / "tile_ir_128x4096x4096.json").read_text())
    for key in ("tile_m", "tile_n", "tile_k", "split_k", "wgp", "tflops", "all"):   # the reference's keys
        assert key in js, key
    assert (js["tile_m"], js["tile_n"], js["tile_k"], js["split_k"], js["wgp"]) == (128, 128, 64, 8, False)
    assert js["arch"] == "gfx950"
    with _tuner(tmp_path) as t2:
        r = t2.tile_ir_lookup(128, 4096, 4096)
        assert r is not None and r.from_cache == 1
        assert (r.best.tile_m, r.best.tile_n, r.best.split_k, r.best.wg_size) == (128, 128, 8, 256)
        assert r.best.transpose == t0g.NT and abs(r.best_tflops - 271.3) < 0.01
        assert t2.tile_ir_ranking(128, 4096, 4096) == [(n, pytest.approx(v, abs=0.01)) for n, v in ranking]
        assert "tile_ir 128x4096x4096" in t2.report()


def test_tile_ir_file_of_the_gfx1100_build_is_a_miss(tmp_path):
    """The file save_tile_ir_cache writes on gfx1100 (no arch; an RDNA3 tile) is re-tuned here."""
    _write(tmp_path, "tile_ir_4096x4096x4096.json",
           '{"tile_m":128,"tile_n":128,"tile_k":32,"split_k":1,"wgp":false,"tflops":84.70,'
           '"all":[["tile_gemm_128x128_k32_db",84.70]]}')
    with _tuner(tmp_path) as t:
        assert t.tile_ir_lookup(4096, 4096, 4096) is None


def test_tile_ir_file_without_wg_size_loads(tmp_path):
    """load_tile_ir_cache reads no workgroup size (cost_model.rs:1059-1074): the tile gives it."""
    _write(tmp_path, "tile_ir_256x256x32768.json",
           '{"tile_m":64,"tile_n":64,"tile_k":64,"split_k":16,"wgp":false,"tflops":243.1,"arch":"gfx950"}')
    with _tuner(tmp_path) as t:
        r = t.tile_ir_lookup(256, 256, 32768)
        assert r is not None and (r.best.wg_size, r.best.split_k) == (256, 16)
        assert t0g.tile_config_name(r.best) == "tile_gemm_64x64_k64_db_sk16"


@pytest.mark.parametrize("text", [
    '{"tile_m":256,"tile_n":256,"tile_k":64,"split_k":2147483648,"wgp":false,"tflops":1,"arch":"gfx950"}',
    '{"tile_m":96,"tile_n":64,"tile_k":64,"split_k":1,"wgp":false,"tflops":1,"arch":"gfx950"}',
    '{"tile_m":64,"tile_n":64,"tile_k":64,"split_k":1,"wgp":false,"arch":"gfx950"}',
])
def test_tile_ir_bad_files_are_misses(tmp_path, text):
    _write(tmp_path, "tile_ir_64x64x64.json", text)
    with _tuner(tmp_path) as t:
        assert t.tile_ir_lookup(64, 64, 64) is None


def test_tile_ir_store_refuses_stream_k(tmp_path):
    with _tuner(tmp_path) as t:
        sk = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
        with pytest.raises(t0g.T0gError) as e:
            t.save_tile_ir_cache(4352, 4096, 8192, sk, 1.0)
        assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG
