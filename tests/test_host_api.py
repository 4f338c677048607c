"""Host-side checks of the C ABI (no GPU): symbol table, GemmConfig mirror,
selection, grids, kernarg byte layouts and the error paths.

Byte layouts and grid formulas are the reference's (src/t0/gemm_gen.rs:286-309,
402-456; src/t0/tile_ir.rs:3173-3202); the assertions follow its own unit tests
(src/t0/gemm_gen.rs:548-584, 620-630; src/t0/tile_ir.rs:2875-2894)."""
import ctypes
import os
import re
import struct

import pytest

import t0g
from conftest import ROOT


def _declared_symbols():
    with open(os.path.join(ROOT, "include", "t0g.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"T0G_API\s+[^;(]*?\b(t0g_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    syms = _declared_symbols()
    assert len(syms) >= 40
    lib = t0g.library()
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_rust_binding_declares_every_entry_point():
    """INTEGRATION.md's extern "C" block declares each function of the header with
    the header's parameter count (the binding a Rust caller would paste)."""
    with open(os.path.join(ROOT, "include", "t0g.h")) as f:
        header = f.read()
    with open(os.path.join(ROOT, "INTEGRATION.md")) as f:
        doc = f.read()

    def nargs(a):
        a = " ".join(a.split())
        return 0 if a in ("", "void") else a.count(",") + 1

    c_fns = {n: nargs(a) for n, a in re.findall(r"T0G_API\s+[^;(]*?\b(t0g_\w+)\s*\(([^;]*?)\);", header, re.S)}
    rust_fns = {n: nargs(a) for n, a in re.findall(r"pub fn (t0g_\w+)\(([^;]*?)\)\s*(?:->[^;]*)?;", doc, re.S)}
    assert sorted(set(c_fns) - set(rust_fns)) == []
    assert {n: (rust_fns[n], c_fns[n]) for n in c_fns if rust_fns[n] != c_fns[n]} == {}


def test_binding_constants_match_the_header():
    """Every enum value and numeric #define of the header that the Python binding
    mirrors (T0G_X as t0g.X) has the header's value."""
    with open(os.path.join(ROOT, "include", "t0g.h")) as f:
        body = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    vals = {}
    for blk in re.findall(r"enum\s*\w*\s*\{(.*?)\}", body, re.S):
        nxt = 0
        for ent in (e.strip() for e in blk.split(",")):
            m = re.match(r"T0G_(\w+)\s*(?:=\s*(-?\w+))?$", ent)
            if not m:
                continue
            if m.group(2) is not None:
                nxt = int(m.group(2), 0)
            vals[m.group(1)] = nxt
            nxt += 1
    for name, v, sh in re.findall(r"#define T0G_(\w+)\s+\(?(0x[0-9a-fA-F]+|\d+)u?(?:\s*<<\s*(\d+))?\)?", body):
        vals[name] = int(v, 0) << (int(sh) if sh else 0)
    mirrored = {n: (v, getattr(t0g, n)) for n, v in vals.items() if hasattr(t0g, n)}
    assert len(mirrored) >= 25
    for n in ("SPLIT_K_REDUCE_KERNEL", "SPLIT_K_IN_KERNEL", "SPLIT_K_AUTO", "STREAM_K", "BF16", "TT"):
        assert n in mirrored, n
    assert {n: x for n, x in mirrored.items() if x[0] != x[1]} == {}


def test_library_links_no_oracle():
    with open(t0g.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"oracle_gemm" not in blob and b"liboracle" not in blob


def test_version_and_last_error():
    assert "gfx950" in t0g.version()
    with pytest.raises(t0g.T0gError) as e:
        t0g.GemmConfig.preset("tile_96x64_k16")   # no such preset in gemm_gen.rs:88-145
    assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG
    assert "unknown preset" in t0g.last_error()


@pytest.mark.parametrize("name,bm,bn,wg", [("gfx950_256x256_k64", 256, 256, 512), ("gfx950_128x128_k64", 128, 128, 256),
                                           ("gfx950_64x64_k64", 64, 64, 256)])
def test_presets_and_derived_fields(name, bm, bn, wg):
    c = t0g.GemmConfig.preset(name)
    c.validate()
    assert (c.tile_m, c.tile_n, c.tile_k, c.wg_size) == (bm, bn, 64, wg)
    assert c.n_waves() == wg // 64                 # wave64
    assert c.lds_total() == 2 * (bm + bn) * 64 * 2  # lds_total: 2 buffers x (X + WT) tiles
    assert c.name() == f"t0_gemm_{bm}x{bn}_k64_ldsdb"
    assert c.copy(split_k=4).name() == f"t0_gemm_{bm}x{bn}_k64_ldsdb_sk4"
    assert c.copy(swap_grid=0).name().endswith("_mg")
    assert c.copy(transpose=t0g.NN).name().endswith("_nn")
    assert c.copy(epilogue=t0g.EPI_BIAS_ADD).name().endswith("_bias")
    assert c.copy(epilogue=t0g.EPI_BIAS_ADD_RELU).name().endswith("_bias_relu")


def test_invalid_configs_are_errors_not_panics():
    c = t0g.GemmConfig.preset("gfx950_128x128_k64")
    # outside both the native set and the reference's space (gemm_gen.rs:684-803 panics on these)
    for bad in (dict(tile_m=8), dict(tile_m=24), dict(tile_m=272), dict(tile_n=8), dict(tile_k=8), dict(tile_k=24),
                dict(tile_k=144), dict(wg_size=0), dict(wg_size=48), dict(wg_size=2048), dict(n_col_passes=0),
                dict(n_col_passes=5), dict(split_k=3), dict(split_k=128)):
        with pytest.raises(t0g.T0gError) as e:
            c.copy(**bad).validate()
        assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG, bad
    with pytest.raises(t0g.T0gError) as e:
        c.copy(transpose=4).validate()
    assert e.value.code == t0g.ERR_INVALID_ARG
    # stream-K needs the native 256x256 kernel, not merely a 256x256 tile shape
    with pytest.raises(t0g.T0gError):
        t0g.GemmConfig.preset("gfx950_256x256_k64").copy(wg_size=256, split_k=t0g.STREAM_K).validate()
    with pytest.raises(t0g.T0gError):
        t0g.GemmConfig.preset("tile_64x64_k16").copy(split_k=t0g.STREAM_K).validate()


def test_off_native_variants_are_reference_space_configs():
    # what used to be refused (another tile_k, wg_size, pass count or no LDS) is now a config of
    # the reference's space: valid, and run on the modelled tile rather than its own kernel
    c = t0g.GemmConfig.preset("gfx950_128x128_k64")
    assert c.is_native()
    for var in (dict(tile_m=96), dict(tile_k=16), dict(wg_size=128), dict(n_col_passes=2), dict(double_buffer=0)):
        v = c.copy(**var)
        v.validate()
        assert not v.is_native(), var


# GemmConfig::tile_* (src/t0/gemm_gen.rs:88-145): (name, tile_m, tile_n, tile_k, wg_size, use_lds, passes)
GEMM_PRESETS = [("tile_16x64_k16", 16, 64, 16, 32, 1, 1), ("tile_32x64_direct", 32, 64, 16, 64, 0, 1),
                ("tile_32x64_k16", 32, 64, 16, 64, 1, 1), ("tile_32x64_k32", 32, 64, 32, 64, 1, 1),
                ("tile_32x128_k16", 32, 128, 16, 64, 1, 1), ("tile_64x64_k16", 64, 64, 16, 64, 1, 1),
                ("tile_64x64_k32", 64, 64, 32, 64, 1, 1), ("tile_128x64_k16", 128, 64, 16, 128, 1, 1),
                ("tile_64x128_k16", 64, 128, 16, 64, 1, 1), ("tile_128x64_k32", 128, 64, 32, 128, 1, 1),
                ("tile_128x128_k16", 128, 128, 16, 128, 1, 1), ("tile_64x64_k64", 64, 64, 64, 64, 1, 1),
                ("tile_128x128_2pass", 128, 64, 16, 128, 1, 2), ("tile_64x128_2pass", 64, 64, 16, 64, 1, 2)]


@pytest.mark.parametrize("name,bm,bn,bk,wg,lds,passes", GEMM_PRESETS)
def test_reference_gemm_presets(name, bm, bn, bk, wg, lds, passes):
    c = t0g.GemmConfig.preset(name)
    c.validate()
    assert not c.is_native()
    assert (c.tile_m, c.tile_n, c.tile_k, c.wg_size, c.use_lds, c.double_buffer, c.n_col_passes) == \
        (bm, bn, bk, wg, lds, lds, passes)
    assert (c.split_k, c.lds_pad, c.swap_grid, c.wgp_mode, c.transpose, c.epilogue) == (0, 0, 1, 1, t0g.NT, 0)
    # GemmConfig::name (gemm_gen.rs:207-227): lds tag, pass tag, then _wgp
    tag = "_ldsdb" if lds else "_direct"
    ptag = f"_{passes}p" if passes > 1 else ""
    assert c.name() == f"t0_gemm_{bm}x{bn}_k{bk}{tag}{ptag}_wgp"
    assert c.copy(split_k=4).name() == f"t0_gemm_{bm}x{bn}_k{bk}{tag}_sk4{ptag}_wgp"
    assert c.lds_total() == (bm + bn) * bk * 2 * (2 if lds else 1)   # lds_total (gemm_gen.rs:162-170)
    # compute_grid (gemm_gen.rs:286-309): threads of the caller's wg_size, columns per pass block
    tm, tn = -(-1000 // bm), -(-3000 // (bn * passes))
    assert t0g.compute_grid(c, 1000, 3000) == (tn * wg, tm)
    assert t0g.compute_grid_split_k(c, 1000, 3000, 4) == (tn * wg, tm * 4)
    assert t0g.compute_grid(c.copy(swap_grid=0), 1000, 3000) == (tm * wg, tn)


def test_reference_gemm_preset_count_and_sweep_list():
    assert len(GEMM_PRESETS) == 14
    # sweep_configs() (gemm_gen.rs:233-245) draws on these presets; all are valid configs here
    for name in ("tile_16x64_k16", "tile_32x64_k16", "tile_32x64_k32", "tile_32x128_k16", "tile_64x64_k16",
                 "tile_64x64_k32", "tile_128x64_k16", "tile_64x128_k16", "tile_128x64_k32"):
        t0g.GemmConfig.preset(name).validate()


# TileGemm::tile_* (src/t0/tile_ir.rs:121-358): (name, tile_m, tile_n, tile_k, wgp)
TILE_PRESETS = [("tile_128x64_k16", 128, 64, 16, 0), ("tile_64x64_k16", 64, 64, 16, 0),
                ("tile_64x64_k32", 64, 64, 32, 0), ("tile_64x64_k64", 64, 64, 64, 0),
                ("tile_32x64_k16", 32, 64, 16, 0), ("tile_128x64_k32", 128, 64, 32, 0),
                ("tile_64x128_k32", 64, 128, 32, 0), ("tile_64x128_k16", 64, 128, 16, 0),
                ("tile_128x128_k16", 128, 128, 16, 0), ("tile_128x128_k32", 128, 128, 32, 1),
                ("tile_128x128_k48", 128, 128, 48, 0), ("tile_128x128_k16_swap", 128, 128, 16, 0),
                ("tile_128x128_k32_swap", 128, 128, 32, 0), ("tile_256x64_k32_wgp", 256, 64, 32, 1),
                ("tile_256x64_k64_wgp", 256, 64, 64, 1), ("tile_128x128_k64", 128, 128, 64, 0),
                ("tile_128x64_k64", 128, 64, 64, 0)]


@pytest.mark.parametrize("name,bm,bn,bk,wgp", TILE_PRESETS)
def test_reference_tile_presets(name, bm, bn, bk, wgp):
    c = t0g.GemmConfig.tile_preset(name)
    c.validate()
    assert not c.is_native()
    assert (c.tile_m, c.tile_n, c.tile_k, c.wg_size, c.wgp_mode, c.double_buffer, c.split_k) == \
        (bm, bn, bk, bm, wgp, 1, 0)                                   # TileGemm::wg_size() = tile_m
    # tile_ir::compute_grid (tile_ir.rs:3193-3202)
    assert t0g.tile_compute_grid(c, 129, 65) == [-(-65 // bn) * bm, -(-129 // bm), 1]
    db_wgp = "_db" + ("_wgp" if wgp else "")
    assert t0g.tile_config_name(c) == f"tile_gemm_{bm}x{bn}_k{bk}{db_wgp}"


def test_reference_configs_run_on_the_modelled_native_tile():
    # a reference config names an RDNA3 tile; the kernel is the gfx950 tile the 256-CU model picks
    ref = t0g.GemmConfig.preset("tile_64x64_k16")
    d = t0g.gemm_desc(0x10000, 0x20000, 0x30000, 4096, 4096, 4096, config=ref)
    assert t0g.gemm_kernel_name(d) == "t0g_gemm_256x256_k64_nt_f32"
    d = t0g.gemm_desc(0x10000, 0x20000, 0x30000, 4096, 4096, 4096, config=ref.copy(split_k=4))
    assert t0g.gemm_kernel_name(d).startswith("t0g_gemm_256x256_k64_nt_f32")
    assert t0g.gemm_workspace_size(d) == 4 * 4096 * 4096 * 4          # the config's split is kept
    # a native config still runs its own kernel, whatever the model would pick
    nat = t0g.GemmConfig.preset("gfx950_64x64_k64")
    d = t0g.gemm_desc(0x10000, 0x20000, 0x30000, 4096, 4096, 4096, config=nat)
    assert t0g.gemm_kernel_name(d).startswith("t0g_gemm_64x64_k64_nt_f32")


def test_auto_select_reference_assertions():
    # src/t0/gemm_gen.rs:548-573
    c = t0g.auto_select(256, 256, 256)
    assert 16 <= c.tile_m <= 256 and c.wg_size >= 32
    c = t0g.auto_select(1024, 1024, 1024)
    assert c.tile_m >= 64
    c = t0g.auto_select(8192, 8192, 8192)
    assert c.tile_m >= 64
    c = t0g.auto_select(128, 4096, 4096)
    assert 128 % c.tile_m == 0
    for m, k, n in [(256, 256, 256), (4096, 4096, 4096), (8192, 8192, 8192), (128, 4096, 4096),
                    (256, 32768, 256), (1024, 4096, 11008), (1024, 11008, 4096), (11008, 1024, 4096), (1, 1, 1)]:
        t0g.auto_select(m, k, n).validate()


def test_auto_select_table_for_256_cus():
    big = t0g.auto_select(8192, 8192, 8192)
    assert (big.tile_m, big.tile_n, big.split_k) == (256, 256, 0)
    sq = t0g.auto_select(4096, 4096, 4096)
    assert (sq.tile_m, sq.tile_n, sq.split_k) == (256, 256, 0)   # 256 tiles: one per CU
    thin = t0g.auto_select(128, 4096, 4096)
    tiles = (-(-128 // thin.tile_m)) * (-(-4096 // thin.tile_n)) * max(thin.split_k, 1)
    assert tiles >= 128                                            # thin M is spread with split-K
    deep = t0g.auto_select(256, 32768, 256)
    assert deep.split_k >= 8                                       # 256x256 output, K=32768: split K
    assert t0g.tile_auto_select(128, 256, 64, t0g.NN).transpose == t0g.NN


def test_compute_grid_formulas():
    c = t0g.GemmConfig.preset("gfx950_128x128_k64")
    assert t0g.compute_grid(c, 1000, 300) == (3 * 256, 8)          # ceil(300/128)*wg, ceil(1000/128)
    assert t0g.compute_grid(c.copy(swap_grid=0), 1000, 300) == (8 * 256, 3)
    assert t0g.compute_grid_split_k(c, 256, 256, 4) == (2 * 256, 2 * 4)
    with pytest.raises(t0g.T0gError):
        t0g.compute_grid_split_k(c, 256, 256, 3)
    assert t0g.compute_grid_auto(c.copy(split_k=8), 256, 512) == (4 * 256, 16)
    assert t0g.compute_grid_auto(c, 256, 512) == (4 * 256, 2)
    assert t0g.tile_compute_grid(c.copy(split_k=2), 129, 65) == [1 * 256, 2 * 2, 1]


def test_build_kernargs_layout():
    c = t0g.GemmConfig.preset("gfx950_64x64_k64")
    ka = t0g.build_kernargs(0x1000, 0x2000, 0x3000, 64, 96, 128, c)
    assert len(ka) == 40
    assert struct.unpack("<QQQIIII", ka) == (0x1000, 0x2000, 0x3000, 64, 96, 0, 0)
    ka = t0g.build_kernargs(0x1000, 0x2000, 0x3000, 512, 96, 128, c.copy(split_k=4))
    assert struct.unpack("<QQQIIII", ka)[6] == 128 * 96 * 4          # y_split_stride = M*N*4
    kb = t0g.build_kernargs_with_bias(0x1000, 0x2000, 0x3000, 64, 64, 128, c, 0x4000)
    assert len(kb) == 48 and struct.unpack("<Q", kb[40:48])[0] == 0x4000   # gemm_gen.rs:620-630
    km = t0g.build_kernargs_m(1, 2, 3, 64, 96, 77, c.copy(split_k=8))
    assert len(km) == 44 and struct.unpack("<QQQIIIII", km) == (1, 2, 3, 64, 96, 3, 0, 77)


def test_backward_helpers_argument_mapping():
    m, n_orig, k_orig = 1024, 4096, 11008
    cd = t0g.auto_select_backward_data(m, n_orig, k_orig)
    assert cd.as_dict() == t0g.auto_select(m, n_orig, k_orig).as_dict()
    cw = t0g.auto_select_backward_weight(m, n_orig, k_orig)
    assert cw.as_dict() == t0g.auto_select(n_orig, m, k_orig).as_dict()
    ka = t0g.build_kernargs_backward_data(10, 20, 30, m, n_orig, k_orig, cd)
    assert struct.unpack("<QQQII", ka[:32]) == (10, 20, 30, n_orig, k_orig)     # K=N_orig, N=K_orig
    kw = t0g.build_kernargs_backward_weight(10, 20, 30, m, n_orig, k_orig, cw)
    assert struct.unpack("<QQQII", kw[:32]) == (10, 20, 30, m, k_orig)          # K=M, N=K_orig
    assert t0g.compute_grid_backward_data(cd, m, k_orig) == t0g.compute_grid_auto(cd, m, k_orig)
    assert t0g.compute_grid_backward_weight(cw, n_orig, k_orig) == t0g.compute_grid_auto(cw, n_orig, k_orig)


def test_gemm_plan_selection_host_only():
    d = t0g.gemm_desc(0x10000, 0x20000, 0x30000, 4096, 4096, 4096, transpose="NN", out_dtype=t0g.BF16)
    assert t0g.gemm_kernel_name(d) == "t0g_gemm_256x256_k64_nn_bf16"
    assert t0g.gemm_workspace_size(d) == 0
    d = t0g.gemm_desc(0x10000, 0x20000, 0x30000, 33, 50, 100)          # K % 8 != 0: element-wise loads
    assert t0g.gemm_kernel_name(d).endswith("_u")
    d = t0g.gemm_desc(0x10000, 0x20000, 0x30000, 256, 256, 32768)
    assert "_nt_f32" in t0g.gemm_kernel_name(d)            # split-K: f32 partial planes
    ws = t0g.gemm_workspace_size(d)
    cfg = t0g.auto_select(256, 32768, 256)
    assert ws == cfg.split_k * 256 * 256 * 4
    d = t0g.gemm_desc(0x10000, 0x20000, 0x30000, 64, 64, 64, split_k=4)
    assert t0g.gemm_workspace_size(d) == 0        # K=64 is one tile: nothing to split
    with pytest.raises(t0g.T0gError) as e:
        t0g.gemm_kernel_name(t0g.gemm_desc(1, 2, 3, 64, 64, 64, ldc=10))
    assert e.value.code == t0g.ERR_INVALID_ARG
    with pytest.raises(t0g.T0gError):
        t0g.gemm_kernel_name(t0g.gemm_desc(1, 2, 3, 64, 64, 64, epilogue=t0g.EPI_BIAS_ADD))   # no bias pointer


def test_split_k_mode_selects_the_reduction():
    """By default (auto) split-K writes fp32 planes for the reduce kernel, except two K
    slices on a deep-ring kernel, which are summed inside it (_dr, _dsr); the reduce
    kernel mode always writes planes; the in-kernel mode takes the _r kernel, or _dr /
    _dsr where the grid runs the deep-ring kernel (both write the output dtype and sum
    the planes themselves), and only where its plan conditions hold; an unknown mode is
    refused."""
    def name(m=128, n=4096, **kw):
        return t0g.gemm_kernel_name(t0g.gemm_desc(0x10000, 0x20000, 0x30000, m, n, 4096, transpose="NT",
                                                  out_dtype=t0g.BF16, **kw))
    c128 = t0g.GemmConfig.preset("gfx950_128x128_k64")
    c64 = t0g.GemmConfig.preset("gfx950_64x64_k64")
    # 32 tiles x 8 slices: one workgroup per CU, so the deep-ring kernel writes the planes
    assert name(config=c128, split_k=8) == "t0g_gemm_128x128_k64_nt_f32_d"
    # two slices on the deep ring: summed in the kernel by default
    assert name(config=c64, split_k=2) == "t0g_gemm_64x64_k64_nt_bf16_dsr"   # 32 stages per slice
    assert name(config=c128, split_k=2) == "t0g_gemm_128x128_k64_nt_bf16_dr"
    assert name(m=64, n=512, config=c64, split_k=4) == "t0g_gemm_64x64_k64_nt_f32_d"   # 16
    t0g.set_split_k_mode(t0g.SPLIT_K_REDUCE_KERNEL)
    try:
        assert name(config=c64, split_k=2) == "t0g_gemm_64x64_k64_nt_f32_ds"
        assert name(config=c128, split_k=2) == "t0g_gemm_128x128_k64_nt_f32_d"
    finally:
        t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)
    t0g.set_split_k_mode(t0g.SPLIT_K_IN_KERNEL)
    try:
        assert name(config=c128, split_k=8) == "t0g_gemm_128x128_k64_nt_bf16_dr"
        assert name(m=256, config=c128, split_k=8) == "t0g_gemm_128x128_k64_nt_bf16_r"   # 512 workgroups
        # 2048 K per split (32 stages of 64): the deep ring with K split across its waves
        assert name(config=c64, split_k=2) == "t0g_gemm_64x64_k64_nt_bf16_dsr"
        assert name(m=64, n=512, config=c64, split_k=2) == "t0g_gemm_64x64_k64_nt_bf16_dsr"
        assert name(m=64, n=512, config=c64, split_k=4) == "t0g_gemm_64x64_k64_nt_bf16_dr"   # 16 stages
        assert name(config=c64, split_k=16) == "t0g_gemm_64x64_k64_nt_f32"       # 2048 workgroups: no _r kernel
        assert name(m=64, n=512, config=c64, split_k=16) == "t0g_gemm_64x64_k64_nt_bf16_dr"
        assert name(m=64, n=512, config=c64, split_k=32) == "t0g_gemm_64x64_k64_nt_f32_d"   # 128-element chunks
        assert name(config=c128, split_k=6) == "t0g_gemm_128x128_k64_nt_f32_d"   # not a power of two
        assert name(config=c128) == "t0g_gemm_128x128_k64_nt_bf16_d"              # no split, nothing to sum
        with pytest.raises(t0g.T0gError) as e:
            t0g.set_split_k_mode(3)
        assert e.value.code == t0g.ERR_INVALID_ARG
    finally:
        t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)
    assert name(config=c128, split_k=8) == "t0g_gemm_128x128_k64_nt_f32_d"
    # more workgroups than CUs: the 4-stage ring kernel, two workgroups per CU
    assert t0g.gemm_kernel_name(t0g.gemm_desc(0x10000, 0x20000, 0x30000, 4096, 4096, 4096, out_dtype=t0g.BF16,
                                              config=c128)) == "t0g_gemm_128x128_k64_nt_bf16"


def test_no_device_on_this_host_is_an_error():
    if t0g.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(t0g.T0gError) as e:
        t0g.GpuRuntime.new(0)
    assert e.value.code == t0g.ERR_NO_DEVICE


def test_gemm_group_argument_checks():
    """t0g_gemm_group rejects a NULL device before touching the GPU, with or without
    descriptors."""
    lib = t0g._lib
    d = t0g.gemm_desc(1, 2, 3, 64, 64, 64)
    arr = (t0g.GemmDesc * 1)(d)
    assert lib.t0g_gemm_group(None, arr, 1) == t0g.ERR_INVALID_ARG
    assert "device" in lib.t0g_last_error().decode()
    assert lib.t0g_gemm_group(None, None, 0) == t0g.ERR_INVALID_ARG


def test_injected_hip_failure_maps_to_error():
    t0g.debug_fail_hip_call(1)
    try:
        with pytest.raises(t0g.T0gError) as e:
            t0g.GpuRuntime.new(0)
        assert e.value.code == t0g.ERR_HIP and "failed" in str(e.value)
    finally:
        t0g.debug_fail_hip_call(0)


def test_epilogue_chain_packing_names_and_kernargs():
    """tile_ir EpilogueOp chains (src/t0/tile_ir.rs:41-62): packing, TileGemm::name's
    epilogue tags (src/t0/tile_ir.rs:416-430) and lower_gemm's argument order after M
    (bias, epi_scale, clamp_min, clamp_max; src/t0/tile_ir.rs:661-683)."""
    c = t0g.epilogue_chain(["bias", "relu"])
    assert c == t0g.OP_BIAS_ADD | (t0g.OP_RELU << 4)
    assert t0g.epilogue_chain_name(c) == "_bias_relu"
    assert t0g.epilogue_chain_name(0) == ""
    assert t0g.epilogue_chain_name(t0g.epilogue_chain(["gelu", "neg", "abs", "clamp"])) == "_gelu_neg_abs_clamp"
    with pytest.raises(t0g.T0gError):
        t0g.epilogue_chain([9])
    with pytest.raises(t0g.T0gError):
        t0g.epilogue_chain(["relu"] * 9)
    with pytest.raises(t0g.T0gError):
        t0g.epilogue_chain_name(0x30)                 # a gap before an op
    cfg = t0g.GemmConfig.preset("gfx950_64x64_k64")
    base = t0g.build_kernargs_m(1, 2, 3, 64, 32, 16, cfg)
    ka = t0g.build_kernargs_m_epilogue(1, 2, 3, 64, 32, 16, cfg, t0g.epilogue_chain(["relu"]))
    assert ka == base                                 # ReLU needs no arguments
    chain = t0g.epilogue_chain(["bias", "scale", "clamp", "silu"])
    ka = t0g.build_kernargs_m_epilogue(1, 2, 3, 64, 32, 16, cfg, chain, bias=0x1122334455667788,
                                       epi_scale=0.5, clamp=(-2.0, 3.0))
    assert len(ka) == 64 and ka[:44] == base
    assert struct.unpack_from("<Qfff", ka, 44) == (0x1122334455667788, 0.5, -2.0, 3.0)
    ka = t0g.build_kernargs_m_epilogue(1, 2, 3, 64, 32, 16, cfg, t0g.epilogue_chain(["clamp", "scale"]),
                                       epi_scale=4.0, clamp=(0.0, 1.0))
    assert len(ka) == 56 and struct.unpack_from("<fff", ka, 44) == (4.0, 0.0, 1.0)


def test_desc_chain_validation():
    d = t0g.gemm_desc(0x1000, 0x2000, 0x3000, 256, 256, 256, transpose="NN", epilogue_ops=["bias", "silu"])
    with pytest.raises(t0g.T0gError) as e:             # BiasAdd without a bias pointer
        t0g.gemm_kernel_name(d)
    assert e.value.code == t0g.ERR_INVALID_ARG
    d = t0g.gemm_desc(0x1000, 0x2000, 0x3000, 256, 256, 256, transpose="NN", epilogue_ops=["gelu", "clamp"],
                      clamp=(-1.0, 1.0))
    assert t0g.gemm_kernel_name(d).startswith("t0g_gemm_")


@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
def test_operand_size_limits(layout):
    """Operands below 2^30 elements take the fast kernels; larger aligned ones the wide
    256x256 kernels (_x: descriptors rebased per tile or K stage), whatever the config
    asked for, as long as the leading dimension stays below 2^22 (K-contiguous) or
    2^24 - 256 (M/N-contiguous) elements; the rest goes element-wise (_u, 32-bit element
    offsets), where 2^31 elements or more are refused with an error."""
    k, n = 16384, 256
    a, b = 1 << 12, 1 << 40   # 16-byte aligned device addresses (not dereferenced here)

    def name(m, a=a, k=k, **kw):
        return t0g.gemm_kernel_name(t0g.gemm_desc(a, b, 0, m, n, k, transpose=layout, out_dtype=t0g.BF16, **kw))

    below = (1 << 30) // k - 8   # a multiple of 8: M-contiguous rows stay 16-byte aligned
    assert name(below) == f"t0g_gemm_256x256_k64_{layout.lower()}_bf16"
    for m in ((1 << 30) // k, (1 << 31) // k, (1 << 34) // k):                    # 1 GiB .. 32 GiB of A
        assert name(m) == f"t0g_gemm_256x256_k64_{layout.lower()}_bf16_x", m
    c128 = t0g.GemmConfig.preset("gfx950_128x128_k64")
    assert name((1 << 31) // k, config=c128).endswith("_bf16_x")                   # forced onto 256x256
    assert name((1 << 31) // k, config=c128.copy(split_k=2)) == f"t0g_gemm_256x256_k64_{layout.lower()}_f32_x"
    sk = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
    assert name((1 << 31) // k, config=sk).endswith("_bf16_x")                     # no wide stream-K kernel
    # unaligned A: element-wise, refused once A spans 2^31 elements
    assert name((1 << 31) // k - 8, a=a + 2).endswith("_u")
    with pytest.raises(t0g.T0gError) as e:
        name((1 << 31) // k, a=a + 2)
    assert e.value.code == t0g.ERR_INVALID_ARG
    # leading dimensions past the wide kernels' offset range: element-wise
    a_k = layout in ("NT", "NN")
    big_ld = (1 << 22) if a_k else (1 << 24)
    m = 1 << 12 if a_k else big_ld - 512      # A of about 2^34 (K-contiguous) or 2^31 (M/N-contiguous) elements
    kk = k if a_k else 128
    assert name(m, k=kk, lda=big_ld - 512).endswith("_x")
    with pytest.raises(t0g.T0gError) as e:    # past the bound: element-wise, which cannot take 2^31 elements
        name(m, k=kk, lda=big_ld)
    assert e.value.code == t0g.ERR_INVALID_ARG


def test_k_split_kernels_from_24_stages_per_slice():
    """The 64x64 deep ring splits K across its waves (_ds, or _dsr summed in the kernel) from
    24 stages of 64 K values per slice; one stage less keeps the 2 x 2 wave grid (_d, _dr)."""
    c64 = t0g.GemmConfig.preset("gfx950_64x64_k64")

    def name(k, split, out=t0g.BF16):
        return t0g.gemm_kernel_name(t0g.gemm_desc(0x10000, 0x20000, 0x30000, 64, 64, k, transpose="NT",
                                                  out_dtype=out, config=c64, split_k=split))
    assert name(23 * 64, 1) == "t0g_gemm_64x64_k64_nt_bf16_d"
    assert name(24 * 64, 1) == "t0g_gemm_64x64_k64_nt_bf16_ds"
    assert name(23 * 64 + 8, 1) == "t0g_gemm_64x64_k64_nt_bf16_ds"     # a 24th stage with a K tail
    assert name(2 * 23 * 64, 2) == "t0g_gemm_64x64_k64_nt_bf16_dr"     # two slices: summed in the kernel
    assert name(2 * 24 * 64, 2) == "t0g_gemm_64x64_k64_nt_bf16_dsr"
    assert name(4 * 24 * 64, 4) == "t0g_gemm_64x64_k64_nt_f32_ds"      # four slices: planes + reduce
    t0g.set_split_k_mode(t0g.SPLIT_K_REDUCE_KERNEL)
    try:
        assert name(2 * 24 * 64, 2) == "t0g_gemm_64x64_k64_nt_f32_ds"
        assert name(2 * 23 * 64, 2) == "t0g_gemm_64x64_k64_nt_f32_d"
    finally:
        t0g.set_split_k_mode(t0g.SPLIT_K_AUTO)
