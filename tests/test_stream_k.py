"""Stream-K schedule, host side: the partition of (tile, K step) pairs over
workgroups that the kernels compute (t0g_kernel_args.h), and the config and
plan rules around T0G_STREAM_K.  GPU parity is in test_stream_k_gpu.py."""
import pytest

import t0g


def _ranges(total, grid):
    return [(t0g.stream_k_begin(total, grid, w), t0g.stream_k_begin(total, grid, w + 1)) for w in range(grid)]


CASES = [(1, 1), (4, 4), (96, 96), (160, 160), (2816, 256), (2880, 256), (11008, 256), (16384, 256),
         (257, 256), (511, 256), (100003, 256), (64 * 172, 256)]


@pytest.mark.parametrize("total,grid", CASES)
def test_partition_covers_every_pair_once(total, grid):
    r = _ranges(total, grid)
    assert r[0][0] == 0 and r[-1][1] == total == t0g.stream_k_begin(total, grid, grid)
    sizes = [e - b for b, e in r]
    assert all(r[i][1] == r[i + 1][0] for i in range(grid - 1))
    assert max(sizes) - min(sizes) <= 1 and min(sizes) >= 1
    for w, (b, e) in enumerate(r):
        for it in {b, e - 1, (b + e) // 2}:
            assert t0g.stream_k_worker(total, grid, it) == w


@pytest.mark.parametrize("tiles,ipt", [(172, 64), (64, 172), (688, 16), (44, 64), (6, 16), (16, 10), (64, 4),
                                       (256, 64), (60, 48), (1, 1), (1, 4)])
def test_each_workgroup_leaves_at_most_one_partial(tiles, ipt):
    """What the kernel relies on: a workgroup's last tile is the only one it may not
    finish (its first job, done before any wait); every other tile in its range it
    owns, and the partials it adds come from lower workgroups only; every tile has
    exactly one owner, and every partial exactly one consumer."""
    total = tiles * ipt
    grid = min(256, total)
    owners = {}
    consumers = {}
    for w, (b, e) in enumerate(_ranges(total, grid)):
        t_first, t_last = b // ipt, (e - 1) // ipt
        for t in range(t_last, t_first - 1, -1):
            tb = t * ipt
            owner = e >= tb + ipt
            if not owner:
                assert t == t_last, "only the first tile processed can be left unfinished"
                continue
            assert t not in owners
            owners[t] = w
            first = t0g.stream_k_worker(total, grid, tb) if tb < b else w
            assert first <= w
            for j in range(first, w):
                assert j not in consumers
                consumers[j] = w
                jb, je = t0g.stream_k_begin(total, grid, j), t0g.stream_k_begin(total, grid, j + 1)
                assert (je - 1) // ipt == t and je < tb + ipt, "contributor j leaves its partial of tile t"
    assert sorted(owners) == list(range(tiles))
    leaving = [w for w, (b, e) in enumerate(_ranges(total, grid)) if e % ipt != 0]
    assert sorted(consumers) == leaving


def test_stream_k_config_rules():
    cfg = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
    cfg.validate()
    assert cfg.name() == "t0_gemm_256x256_k64_ldsdb_streamk"
    for preset in ("gfx950_128x128_k64", "gfx950_64x64_k64"):
        bad = t0g.GemmConfig.preset(preset).copy(split_k=t0g.STREAM_K)
        with pytest.raises(t0g.T0gError) as e:
            bad.validate()
        assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG
    # the reference's grid / kernarg path has no stream-K launch
    for call in (lambda: t0g.compute_grid_auto(cfg, 1024, 1024), lambda: t0g.tile_compute_grid(cfg, 1024, 1024),
                 lambda: t0g.build_kernargs(0, 0, 0, 64, 64, 64, cfg),
                 lambda: t0g.build_kernargs_m(0, 0, 0, 64, 64, 64, cfg)):
        with pytest.raises(t0g.T0gError) as e:
            call()
        assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG


@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
def test_stream_k_plan(layout):
    cfg = t0g.GemmConfig.preset("gfx950_256x256_k64").copy(split_k=t0g.STREAM_K)
    m, n, k = 1024, 11008, 4096
    a, b = 1 << 20, 1 << 30
    d = t0g.gemm_desc(a, b, 0, m, n, k, transpose=layout, out_dtype=t0g.BF16, config=cfg)
    assert t0g.gemm_kernel_name(d) == f"t0g_gemm_256x256_k64_{layout.lower()}_bf16_sk"
    assert t0g.gemm_workspace_size(d) == 256 * 256 * 256 * 4   # one 256 KB slot per CU
    small = t0g.gemm_desc(a, b, 0, 256, 256, 128, transpose=layout, config=cfg)
    assert t0g.gemm_workspace_size(small) == 2 * 256 * 256 * 4   # 1 tile x 2 K steps: two workgroups
    # unaligned operands: the data-parallel 128x128 kernel instead
    u = t0g.gemm_desc(a + 2, b, 0, m, n, k, transpose=layout, config=cfg)
    assert t0g.gemm_kernel_name(u).startswith("t0g_gemm_128x128_k64_") and t0g.gemm_workspace_size(u) == 0
    # K = 0: nothing to split
    z = t0g.gemm_desc(a, b, 0, m, n, 0, transpose=layout, config=cfg)
    assert not t0g.gemm_kernel_name(z).endswith("_sk")
    # forcing it through desc.split_k on a 128x128 config is refused
    c128 = t0g.GemmConfig.preset("gfx950_128x128_k64")
    with pytest.raises(t0g.T0gError):
        t0g.gemm_kernel_name(t0g.gemm_desc(a, b, 0, m, n, k, transpose=layout, config=c128, split_k=t0g.STREAM_K))


@pytest.mark.parametrize("m,n,k,sk", [
    # tile counts just past one or two rounds of 256: data-parallel needs a nearly empty
    # last round (measured on MI355X: 4352x4096x8192, 272 tiles, 230 us stream-K vs 309 us;
    # 3072x11008x4096, 516 tiles, 231 vs 252 us; 1536x11008x32768, 258 tiles, 902 vs 1009 us
    # for split 4)
    (4352, 4096, 8192, True), (4352, 4096, 4096, True), (3072, 11008, 4096, True), (1536, 11008, 32768, True),
    # fuller last rounds, or a thin last round after four full ones, stay data-parallel
    # (measured: 144 tiles a tie, 576 tiles slower, 1032 tiles 472 vs 429 us)
    (4608, 4608, 8192, False), (3072, 3072, 8192, False), (6144, 6144, 6144, False), (6144, 11008, 4096, False),
    (8448, 8192, 8192, False),
    # The benchmark shapes keep their schedules (measured slower with stream-K: MLP 97 vs 88 us)
    (4096, 4096, 4096, False), (8192, 8192, 8192, False), (128, 4096, 4096, False), (256, 256, 32768, False),
    (1024, 11008, 4096, False), (1024, 4096, 11008, False), (11008, 4096, 1024, False), (256, 256, 256, False)])
def test_auto_select_takes_stream_k_only_with_a_margin(m, n, k, sk):
    cfg = t0g.auto_select(m, k, n)
    assert (cfg.split_k == t0g.STREAM_K) == sk, cfg.name()
    if sk:
        assert (cfg.tile_m, cfg.tile_n) == (256, 256)
