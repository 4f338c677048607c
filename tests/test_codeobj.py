"""Host-side checks (no GPU) of the code-object metadata reader, the compile
entry point (T0Kernel::compile, src/t0/compile.rs:1115-1187) and the tile ABI's
selection (tile_auto_select, src/t0/tile_ir.rs:471-568).

The metadata reader is checked against the built gfx950 code object, whose
argument blocks are known from t0g_kernel_args.h (T0gGemmArgs 104 bytes,
T0gGemmSkArgs and T0gGemmRedArgs 144), and against malformed or foreign input it must refuse
without reading out of bounds."""
import ctypes
import os
import random
import struct

import pytest

import t0g

HSACO = os.path.join(os.path.dirname(t0g.LIB_PATH), "t0g_gemm_gfx950.hsaco")


@pytest.fixture(scope="module")
def blob():
    with open(HSACO, "rb") as f:
        return f.read()


def _bundle_entries(blob):
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    assert blob.startswith(magic)
    n = struct.unpack_from("<Q", blob, len(magic))[0]
    pos, out = len(magic) + 8, []
    for _ in range(n):
        off, size, idl = struct.unpack_from("<QQQ", blob, pos)
        pos += 24
        out.append((blob[pos:pos + idl].decode(), off, size))
        pos += idl
    return out


def _gfx950_elf(blob):
    for ident, off, size in _bundle_entries(blob):
        if "gfx950" in ident:
            return blob[off:off + size]
    raise AssertionError("no gfx950 entry")


@pytest.mark.parametrize("symbol,args,lds,wg", [
    ("t0g_gemm_256x256_k64_nt_f32", 104, 131072, 256),
    ("t0g_gemm_256x256_k64_tn_bf16", 104, 131072, 256),
    ("t0g_gemm_128x128_k64_nn_f32", 104, None, 256),
    ("t0g_gemm_64x64_k64_nt_f32_d", 104, 131072, 256),
    ("t0g_gemm_64x64_k64_nn_bf16_ds", 104, 131072, 256),
    ("t0g_gemm_64x64_k64_tn_f32_dsr", 144, None, 256),
    ("t0g_gemm_256x256_k64_nn_bf16_sk", 144, None, 512),
    ("t0g_gemm_256x256_k64_tt_f32_sk", 144, None, 256),
    ("t0g_gemm_256x256_k64_nn_bf16_r", 144, None, 256),
    ("t0g_gemm_128x128_k64_nt_f32_r", 144, None, 256),
    ("t0g_splitk_reduce_bf16", 80, 0, 256),
    ("t0g_f32_to_bf16_rne", 32, 0, 256),
])
def test_metadata_of_the_built_code_object(blob, symbol, args, lds, wg):
    for obj in (blob, _gfx950_elf(blob)):   # the bundle and the bare ELF inside it
        m = t0g.code_object_kernel_meta(obj, symbol)
        assert m.kernarg_size == args
        assert m.kernarg_segment_size >= args   # plus hidden arguments, where used
        assert m.max_workgroup_size == wg
        assert m.wavefront_size == 64
        assert m.private_segment_size == 0
        if lds is not None:
            assert m.group_segment_size == lds


def test_argument_block_sizes_match_the_header(blob):
    """The sizes the runtime packs are the ones every kernel of each kind reads."""
    names = set()
    for ident, off, size in _bundle_entries(blob):
        if "gfx950" in ident:
            elf = blob[off:off + size]
            # kernel names: the NUL-terminated ".kd" symbols in the string tables
            for part in elf.split(b"\0"):
                if part.endswith(b".kd") and part.startswith(b"t0g_gemm_"):
                    names.add(part[:-3].decode())
    assert len(names) >= 60
    for s in sorted(names):
        want = 144 if s.endswith(("_sk", "_r", "_dr", "_dsr")) else 104   # T0gGemmSkArgs / T0gGemmRedArgs
        assert t0g.code_object_kernel_meta(blob, s).kernarg_size == want, s


def test_unknown_symbol_and_garbage_are_refused(blob):
    with pytest.raises(t0g.T0gError) as e:
        t0g.code_object_kernel_meta(blob, "no_such_kernel")
    assert e.value.code == t0g.ERR_INVALID_ARG and "no kernel named" in str(e.value)
    for junk in (b"", b"\x7fELF", b"hello world" * 10, b"__CLANG_OFFLOAD_BUNDLE__" + b"\xff" * 8):
        with pytest.raises(t0g.T0gError):
            t0g.code_object_kernel_meta(junk, "t0g_gemm_256x256_k64_nt_f32")


def test_code_object_for_another_gpu_is_refused(blob):
    elf = bytearray(_gfx950_elf(blob))
    flags = struct.unpack_from("<I", elf, 0x30)[0]
    struct.pack_into("<I", elf, 0x30, (flags & ~0xFF) | 0x4C)   # gfx942's mach
    with pytest.raises(t0g.T0gError) as e:
        t0g.code_object_kernel_meta(bytes(elf), "t0g_gemm_256x256_k64_nt_f32")
    assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG and "0x4c" in str(e.value)


def test_truncated_and_corrupted_objects_never_crash(blob):
    """Every truncation point of the metadata note's neighbourhood and random byte
    flips give a clean answer or a clean error (the reader is bounds-checked)."""
    elf = _gfx950_elf(blob)
    rng = random.Random(1234)
    cuts = sorted(set([0, 1, 4, 16, 63, 64, 100, len(elf) // 2, len(elf) - 1] +
                      [rng.randrange(len(elf)) for _ in range(60)]))
    for cut in cuts:
        try:
            t0g.code_object_kernel_meta(elf[:cut], "t0g_gemm_256x256_k64_nt_f32")
        except t0g.T0gError:
            pass
    for _ in range(200):
        b = bytearray(elf)
        for _ in range(8):
            b[rng.randrange(len(b))] = rng.randrange(256)
        try:
            t0g.code_object_kernel_meta(bytes(b), "t0g_gemm_256x256_k64_nt_f32")
        except t0g.T0gError:
            pass


def _args(ck):
    """Decode a T0gGemmArgs block (t0g_kernel_args.h)."""
    raw = ck.args()
    a, b, c, bias, stride = struct.unpack_from("<5Q", raw, 0)
    ints = struct.unpack_from("<12I", raw, 40)
    keys = ["m", "n", "k", "lda", "ldb", "ldc", "k_per_split", "tiles_m", "tiles_n", "epilogue", "group_m", "flags"]
    d = dict(zip(keys, ints))
    d.update(a=a, b=b, c=c, bias=bias, c_split_stride=stride)
    return d


def test_compile_returns_what_t0g_gemm_launches(blob):
    d = t0g.gemm_desc(1 << 20, 1 << 26, 1 << 30, 4096, 4096, 4096, transpose="NN", out_dtype=t0g.BF16)
    ck = t0g.gemm_compile(d)
    assert ck.name.decode() == t0g.gemm_kernel_name(d) == "t0g_gemm_256x256_k64_nn_bf16"
    assert ck.elf() == blob                       # the library's own code object
    assert (ck.workgroup_size, ck.lds_size, ck.kernarg_size, ck.splits) == (256, 131072, 104, 1)
    assert list(ck.grid) == [256 * 256, 1, 1]
    f = _args(ck)
    assert (f["a"], f["b"], f["c"]) == (1 << 20, 1 << 26, 1 << 30)
    assert (f["m"], f["n"], f["k"], f["lda"], f["ldb"], f["ldc"]) == (4096,) * 6
    assert (f["tiles_m"], f["tiles_n"], f["k_per_split"]) == (16, 16, 4096)
    meta = t0g.code_object_kernel_meta(ck.elf(), ck.name.decode())
    assert meta.kernarg_size == ck.kernarg_size and meta.group_segment_size == ck.lds_size


def test_compile_split_k_writes_planes_to_c():
    cfg = t0g.GemmConfig.preset("gfx950_128x128_k64").copy(split_k=8)
    d = t0g.gemm_desc(1 << 20, 1 << 26, 1 << 30, 128, 4096, 4096, config=cfg)
    ck = t0g.gemm_compile(d)
    assert ck.splits == 8 and list(ck.grid) == [32 * 256, 8, 1]
    f = _args(ck)
    assert f["c"] == 1 << 30 and f["c_split_stride"] == 128 * 4096 * 4 and f["k_per_split"] == 512
    with pytest.raises(t0g.T0gError) as e:   # planes are fp32
        t0g.gemm_compile(t0g.gemm_desc(1 << 20, 1 << 26, 1 << 30, 128, 4096, 4096, config=cfg, out_dtype=t0g.BF16))
    assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG


@pytest.mark.parametrize("layout,m,n,lda,ldb,tile", [
    ("NN", 384, 200, 0, 248, 128), ("NN", 384, 248, 0, 256, 256), ("NN", 4096, 4096, 0, 0, 256),
    ("TN", 200, 200, 248, 248, 128), ("TN", 256, 256, 256, 256, 256), ("TN", 248, 512, 248, 512, 128),
    ("TT", 200, 320, 200, 0, 128), ("TT", 256, 320, 264, 0, 256),
    ("NT", 200, 200, 0, 0, 256)])
def test_small_mn_contiguous_ld_stays_off_the_256_kernels(layout, m, n, lda, ldb, tile):
    """The 256x256 kernels' grouped LDS DMA needs ld >= 256 for M/N-contiguous
    operands (offset registers hold a piece's offset less up to 3 KB); K-contiguous
    operands are unaffected.  The 256x256 preset with a smaller such ld runs on the
    128x128 kernels, with stream-K asked for too."""
    cfg = t0g.GemmConfig.preset("gfx950_256x256_k64")
    for c in (cfg, cfg.copy(split_k=t0g.STREAM_K)):
        d = t0g.gemm_desc(1 << 20, 1 << 26, 1 << 30, m, n, 512, transpose=layout, lda=lda, ldb=ldb, config=c)
        assert t0g.gemm_kernel_name(d).startswith(f"t0g_gemm_{tile}x{tile}_k64_{layout.lower()}_")


def test_compile_stream_k_falls_back_to_the_same_tile():
    cfg = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
    ck = t0g.gemm_compile(t0g.gemm_desc(1 << 20, 1 << 26, 1 << 30, 4352, 8192, 4096, transpose="NN", config=cfg))
    assert ck.name.decode() == "t0g_gemm_256x256_k64_nn_f32" and ck.splits == 1


@pytest.mark.parametrize("m,k,n", [(128, 4096, 4096), (256, 32768, 256), (4096, 4096, 4096), (4352, 8192, 4096),
                                   (1024, 4096, 11008), (1, 1, 1), (200, 192, 136)])
def test_tile_auto_select_gives_tile_abi_configs(m, k, n):
    for tr in (t0g.NT, t0g.NN):
        c = t0g.tile_auto_select(m, k, n, tr)
        c.validate()
        assert c.transpose == tr
        assert c.split_k != t0g.STREAM_K
        gx, gy, gz = t0g.tile_compute_grid(c, m, n)   # the tile ABI's grid exists for it
        assert gz == 1 and gx % c.wg_size == 0
    for tr in (t0g.TN, t0g.TT):   # TileTranspose has NT and NN only
        with pytest.raises(t0g.T0gError) as e:
            t0g.tile_auto_select(m, k, n, tr)
        assert e.value.code == t0g.ERR_INVALID_ARG


def test_tile_auto_select_splits_the_hbm_bound_shapes():
    """The thin and deep benchmark shapes get split-K on the tile ABI too (the
    reference's table splits shapes with few tiles, tile_ir.rs:524-560)."""
    assert t0g.tile_auto_select(128, 4096, 4096).split_k > 1
    assert t0g.tile_auto_select(256, 32768, 256).split_k > 1
    sq = t0g.tile_auto_select(4096, 4096, 4096)
    assert (sq.tile_m, sq.tile_n, sq.split_k) == (256, 256, 0)
    assert t0g.auto_select(4352, 8192, 4096).split_k == t0g.STREAM_K   # auto_select may take stream-K ...
    assert t0g.tile_auto_select(4352, 8192, 4096).split_k != t0g.STREAM_K   # ... the tile ABI never


def test_tile_config_name_follows_tilegemm_name():
    """TileGemm::name's format (src/t0/tile_ir.rs:398-431): tile, k, _db, _skN, _mg, _wgp, _nn, epilogue."""
    c = t0g.GemmConfig.preset("gfx950_128x128_k64")
    assert t0g.tile_config_name(c) == "tile_gemm_128x128_k64_db"
    assert t0g.tile_config_name(c.copy(split_k=8)) == "tile_gemm_128x128_k64_db_sk8"
    assert t0g.tile_config_name(c.copy(transpose=t0g.NN, swap_grid=0)) == "tile_gemm_128x128_k64_db_mg_nn"
    relu = t0g.epilogue_chain(["relu"])
    bias_relu = t0g.epilogue_chain(["bias", "relu"])
    assert t0g.tile_config_name(c, relu).endswith("_relu")          # tile_ir.rs:4952
    assert t0g.tile_config_name(c, bias_relu).endswith("_bias_relu")   # tile_ir.rs:4985
    assert "_relu" not in t0g.tile_config_name(c)                     # tile_ir.rs:5015


@pytest.mark.parametrize("layout,m,n,k", [("TN", 512, 512, 1024), ("NN", 300, 200, 520), ("NT", 128, 4096, 4096)])
def test_compile_takes_no_split_the_caller_did_not_ask_for(layout, m, n, k):
    """C holds one plane per split, so a compiled plan splits only when desc.split_k or an
    explicit config asks: auto_select's split for the shape is compiled as the same tile
    without it (C stays M x N)."""
    d = t0g.gemm_desc(1 << 20, 1 << 26, 1 << 30, m, n, k, transpose=layout)
    auto = t0g.auto_select(m, k, n)
    ck = t0g.gemm_compile(d)
    assert ck.splits == 1 and ck.grid[1] == 1
    assert f"{auto.tile_m}x{auto.tile_n}" in ck.name.decode()
    assert _args(ck)["c_split_stride"] == 0 and _args(ck)["k_per_split"] == k
    asked = t0g.gemm_compile(t0g.gemm_desc(1 << 20, 1 << 26, 1 << 30, m, n, k, transpose=layout, split_k=2))
    assert asked.splits == 2 and asked.grid[1] == 2
