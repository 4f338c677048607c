"""The reference's own callers, with the reference's own GemmConfig / TileGemm
values, through the C ABI unchanged: kernel_get -> build_kernargs* ->
compute_grid* -> dispatch, grids in threads of the caller's wave32 wg_size,
split-K planes at Y + s * y_split_stride summed on the host in plane order.

Each config here is of the reference's space (an RDNA3 tile), so the library
reads the problem back from the grid and kernargs and runs the gfx950 tile its
model picks; the planes follow the reference's K partition, K / split_k each.
Gate: the north-star parity (relF <= 5e-3, max|d| <= 1e-2 sqrt(K/256)) against
the oracle, per plane against the oracle's sum over that plane's K slice.
"""
import numpy as np
import pytest

import oracle as o
import t0g
from test_gemm_gpu import Buffers, _log, check_parity

pytestmark = pytest.mark.gpu

SENTINEL = -9999.0


@pytest.fixture(scope="module")
def rt():
    r = t0g.GpuRuntime.new(0)
    yield r
    r.close()


@pytest.fixture
def bufs(rt):
    b = Buffers(rt)
    yield b
    b.free()


def _dispatch_gemm_gen(rt, bufs, cfg, m, k, n, x, wt, margin=256):
    """The sequence of examples/test_gemm_correctness.rs:118-215 (planes in one buffer)
    with a sentinel after the last plane; returns the planes [sk][M][N]."""
    sk = max(cfg.split_k, 1)
    kern = rt.ensure_gemm_kernel(cfg)
    info = kern.info()
    assert info["kernarg_size"] == 40 and info["wg_size"] == cfg.wg_size
    xa, wa = bufs.up(x), bufs.up(wt)
    y = bufs.up(np.full(sk * m * n + margin, SENTINEL, dtype=np.float32))
    ka = t0g.build_kernargs(xa, wa, y, k, n, m, cfg)
    gx, gy = t0g.compute_grid_auto(cfg, m, n)
    rt.dispatch(kern, [gx, gy, 1], ka)
    raw = rt.read(y, (sk * m * n + margin,), np.float32)
    assert np.all(raw[sk * m * n:] == SENTINEL), "write past the last plane"
    return raw[:sk * m * n].reshape(sk, m, n)


def _check_planes(planes, x, wt, m, k, n, label):
    sk = planes.shape[0]
    assert not np.any(planes == SENTINEL), f"{label}: part of a plane left unwritten"
    ref = o.gemm("NT", x, wt, m, n, k)
    check_parity(o.splitk_reduce(planes), ref, k, label)
    if sk > 1:
        ks = k // sk
        for s in range(sk):
            exp = o.gemm_krange("NT", x, wt, m, n, k, s * ks, (s + 1) * ks)
            check_parity(planes[s], exp, ks, f"{label} plane {s}")


# examples/test_gemm_correctness.rs:67-86: its 8 configs x its 6 sizes (M, K, N), with its
# divisibility filter (:150-154) and its seeds (:128-129)
HARNESS_CFGS = [("tile_64x64_k16", 0), ("tile_64x64_k32", 0), ("tile_128x64_k32", 0), ("tile_128x64_k32", 2),
                ("tile_64x64_k16", 4), ("tile_64x64_k16", 8), ("tile_32x128_k16", 0), ("tile_32x128_k16", 4)]
HARNESS_SIZES = [(64, 64, 64), (128, 128, 128), (256, 256, 256), (64, 256, 64), (128, 1024, 256), (256, 512, 512)]


@pytest.mark.parametrize("preset,sk", HARNESS_CFGS)
def test_gemm_correctness_harness(rt, bufs, preset, sk):
    cfg = t0g.GemmConfig.preset(preset).copy(split_k=sk)
    assert not cfg.is_native()
    ran = 0
    for (m, k, n) in HARNESS_SIZES:
        skk = max(sk, 1)
        if m % cfg.tile_m or n % (cfg.tile_n * cfg.n_col_passes) or k % (cfg.tile_k * skk):
            continue
        label = f"harness {preset} sk={sk} {m}x{k}x{n}"
        _log(f"[case] {label}")
        x = o.rand_bf16_xorshift(m * k, m * 1000 + k)
        wt = o.rand_bf16_xorshift(n * k, n * 2000 + k)
        planes = _dispatch_gemm_gen(rt, bufs, cfg, m, k, n, x, wt)
        _check_planes(planes, x, wt, m, k, n, label)
        # the reference harness's own pass criterion (:245-247) holds as well
        assert np.max(np.abs(o.splitk_reduce(planes) - o.gemm("NT", x, wt, m, n, k))) < 0.01 * k
        bufs.free()
        ran += 1
    assert ran > 0


ALL_GEMM_PRESETS = ["tile_16x64_k16", "tile_32x64_direct", "tile_32x64_k16", "tile_32x64_k32", "tile_32x128_k16",
                    "tile_64x64_k16", "tile_64x64_k32", "tile_128x64_k16", "tile_64x128_k16", "tile_128x64_k32",
                    "tile_128x128_k16", "tile_64x64_k64", "tile_128x128_2pass", "tile_64x128_2pass"]


@pytest.mark.parametrize("preset", ALL_GEMM_PRESETS)
@pytest.mark.parametrize("sk", [0, 2, 16])
def test_every_gemm_preset(rt, bufs, preset, sk):
    """Every GemmConfig preset (gemm_gen.rs:88-145), split None / 2 / 16 (the largest the
    reference's split_k_shift table takes, gemm_gen.rs:684), on a square and an uneven
    shape; the two-pass presets cover all N columns in one dispatch."""
    cfg = t0g.GemmConfig.preset(preset).copy(split_k=sk)
    for (m, k, n) in [(256, 1024, 256), (384, 2048, 768)]:
        label = f"preset {preset} sk={sk} {m}x{k}x{n}"
        _log(f"[case] {label}")
        x = o.rand_bf16_xorshift(m * k, m * 1000 + k)
        wt = o.rand_bf16_xorshift(n * k, n * 2000 + k)
        planes = _dispatch_gemm_gen(rt, bufs, cfg, m, k, n, x, wt)
        _check_planes(planes, x, wt, m, k, n, label)
        bufs.free()


def test_gemm_gen_bias_epilogue_48_byte_kernargs(rt, bufs):
    """build_kernargs_with_bias (gemm_gen.rs:438-456) on a reference preset with
    EpilogueOp::BiasAddReluStoreF32."""
    cfg = t0g.GemmConfig.preset("tile_64x64_k32").copy(epilogue=t0g.EPI_BIAS_ADD_RELU)
    m, k, n = 192, 320, 256
    x = o.rand_bf16_xorshift(m * k, 5)
    wt = o.rand_bf16_xorshift(n * k, 6)
    bias = np.linspace(-2.0, 2.0, n, dtype=np.float32)
    ref = o.epilogue_chain(o.gemm("NT", x, wt, m, n, k), ["bias", "relu"], bias=bias)
    kern = rt.ensure_gemm_kernel(cfg)
    assert kern.info()["kernarg_size"] == 48
    xa, wa, ba = bufs.up(x), bufs.up(wt), bufs.up(bias)
    y = bufs.alloc(m * n * 4, fill=0)
    ka = t0g.build_kernargs_with_bias(xa, wa, y, k, n, m, cfg, ba)
    gx, gy = t0g.compute_grid_auto(cfg, m, n)
    rt.dispatch(kern, [gx, gy, 1], ka)
    check_parity(rt.read(y, (m, n), np.float32), ref, k, "gemm_gen bias+relu tile_64x64_k32")


def test_gemm_gen_split_with_zero_stride_is_reduced(rt, bufs):
    """A gemm_gen split with y_split_stride 0 (every K slice of the reference's kernel would
    store to the same Y) is summed into Y by the library."""
    cfg = t0g.GemmConfig.preset("tile_64x64_k16").copy(split_k=4)
    m, k, n = 128, 512, 192
    x = o.rand_bf16_xorshift(m * k, 11)
    wt = o.rand_bf16_xorshift(n * k, 12)
    kern = rt.ensure_gemm_kernel(cfg)
    xa, wa = bufs.up(x), bufs.up(wt)
    y = bufs.up(np.full(m * n + 64, SENTINEL, dtype=np.float32))
    ka = bytearray(t0g.build_kernargs(xa, wa, y, k, n, m, cfg))
    ka[36:40] = (0).to_bytes(4, "little")
    gx, gy = t0g.compute_grid_auto(cfg, m, n)
    rt.dispatch(kern, [gx, gy, 1], bytes(ka))
    got = rt.read(y, (m * n + 64,), np.float32)
    assert np.all(got[m * n:] == SENTINEL)
    check_parity(got[:m * n].reshape(m, n), o.gemm("NT", x, wt, m, n, k), k, "gemm_gen sk=4 stride 0")


def test_caller_planes_refuse_a_k_the_reference_cannot_split(rt, bufs):
    cfg = t0g.GemmConfig.preset("tile_64x64_k16").copy(split_k=4)
    kern = rt.ensure_gemm_kernel(cfg)
    m, k, n = 64, 96, 64                       # 96 % (16 * 4) != 0
    ka = t0g.build_kernargs(0x1000, 0x2000, 0x3000, k, n, m, cfg)
    gx, gy = t0g.compute_grid_auto(cfg, m, n)
    with pytest.raises(t0g.T0gError) as e:
        rt.dispatch(kern, [gx, gy, 1], ka)
    assert e.value.code == t0g.ERR_UNSUPPORTED_CONFIG
    assert not rt.is_poisoned()


# src/t0/test_tile_gemm_suite.rs:161-208 (test_tg_combo_sequential): TileGemmConfig 128x64 k16
# and 32x64 k16 (wg_size = tile_m), 44-byte kernargs with K and N padded to the tile, M exact
def _c128():
    return t0g.GemmConfig.tile_preset("tile_128x64_k16")


def _c32():
    return t0g.GemmConfig.tile_preset("tile_32x64_k16")


TILE_SUITE = [(128, 128, 128, "c128"), (256, 256, 256, "c32"), (128, 1024, 512, "c128"), (256, 512, 128, "c128"),
              (512, 512, 512, "c128"), (1024, 1024, 1024, "c128"), (33, 100, 50, "c32"), (129, 65, 17, "c128"),
              (100, 300, 200, "c32"), (1000, 768, 512, "c128")]


@pytest.mark.parametrize("m,k,n,which", TILE_SUITE)
def test_tile_gemm_suite_combo(rt, bufs, m, k, n, which):
    cfg = _c128() if which == "c128" else _c32()
    assert cfg.wg_size == cfg.tile_m
    label = f"tile suite {which} {m}x{k}x{n}"
    _log(f"[case] {label}")
    k_pad = (k + cfg.tile_k - 1) // cfg.tile_k * cfg.tile_k
    m_pad = (m + cfg.tile_m - 1) // cfg.tile_m * cfg.tile_m
    n_pad = (n + cfg.tile_n - 1) // cfg.tile_n * cfg.tile_n
    xb = o.make_bf16_suite(m * k, 42 + m).reshape(m, k)
    wb = o.make_bf16_suite(n * k, 137 + n).reshape(n, k)
    xp = np.zeros((m, k_pad), np.uint16)
    xp[:, :k] = xb
    # WT is allocated for the n_pad rows the kernargs' N names (the suite allocates n rows and
    # lets the RDNA3 kernel read past them; here every read stays inside the buffer)
    wp = np.zeros((n_pad, k_pad), np.uint16)
    wp[:n, :k] = wb
    kern = rt.ensure_tile_kernel(cfg)
    assert kern.info()["kernarg_size"] == 44
    xa, wa = bufs.up(xp), bufs.up(wp)
    y = bufs.up(np.full((m_pad + 1, n_pad), SENTINEL, dtype=np.float32))
    ka = t0g.build_kernargs_m(xa, wa, y, k_pad, n_pad, m, cfg)
    grid = t0g.tile_compute_grid(cfg, m, n)
    rt.dispatch(kern, grid, ka)
    got = rt.read(y, (m_pad + 1, n_pad), np.float32)
    ref = o.gemm("NT", xb, wb, m, n, k)
    check_parity(got[:m, :n], ref, k, label)
    assert np.all(got[m:] == SENTINEL), f"{label}: rows at or past M were written"
    # the suite's own criteria (:196-197): every |err| <= 1.0 and below its per-case bound
    err = np.abs(got[:m, :n] - ref)
    assert np.count_nonzero(err > 1.0) == 0


@pytest.mark.parametrize("preset", ["tile_128x64_k32", "tile_128x128_k48", "tile_256x64_k32_wgp", "tile_64x128_k16"])
def test_tile_presets_split_k_library_planes(rt, bufs, preset):
    """TileGemm presets with split_k 4 and build_kernargs_m's y_split_stride 0
    (tile_ir.rs:3179): the library keeps and reduces the planes."""
    cfg = t0g.GemmConfig.tile_preset(preset).copy(split_k=4)
    m, k, n = 300, 1536, 200
    a = o.make_bf16_suite(m * k, 3).reshape(m, k)
    b = o.make_bf16_suite(n * k, 4).reshape(n, k)
    kern = rt.ensure_tile_kernel(cfg)
    aa, ba = bufs.up(a), bufs.up(b)
    y = bufs.up(np.full((m + 2, n), SENTINEL, dtype=np.float32))
    rt.dispatch(kern, t0g.tile_compute_grid(cfg, m, n), t0g.build_kernargs_m(aa, ba, y, k, n, m, cfg))
    got = rt.read(y, (m + 2, n), np.float32)
    check_parity(got[:m], o.gemm("NT", a, b, m, n, k), k, f"tile {preset} sk=4 {m}x{k}x{n}")
    assert np.all(got[m:] == SENTINEL)


# src/ignis/ops/bf16_matmul.rs:140-211: select_config(m) picks tile_16x64_k16 / tile_32x64_k16 /
# tile_64x64_k16; X and W are converted (RNE) and padded (X flat, WT transposed and padded in 2D),
# Y is [m_pad][n_pad], kernargs carry K = k_pad, N = n_pad and the unpadded m, and the grid is
# compute_grid_auto(cfg, m, n_pad)
def _ignis_select(m):
    return t0g.GemmConfig.preset("tile_16x64_k16" if m <= 16 else "tile_32x64_k16" if m <= 32 else "tile_64x64_k16")


def _pad(v, t):
    return (v + t - 1) // t * t


@pytest.mark.parametrize("m,k,n", [(1, 64, 50), (7, 128, 64), (16, 256, 200), (20, 64, 130), (32, 512, 96),
                                   (33, 256, 256), (100, 1024, 300), (512, 4096, 1104)])
def test_ignis_forward_presets(rt, bufs, m, k, n):
    cfg = _ignis_select(m)
    m_pad, n_pad, k_pad = _pad(m, cfg.tile_m), _pad(n, cfg.tile_n), _pad(k, cfg.tile_k)
    assert k_pad == k   # the reference pads X flat, which keeps rows apart only when k % tile_k == 0
    rng = np.random.default_rng(m * 7 + n)
    x = rng.standard_normal((m, k), dtype=np.float32)
    w = (rng.standard_normal((k, n), dtype=np.float32) * 0.05).astype(np.float32)
    xb = o.f32_to_bf16_rne(x)
    wtb = o.f32_to_bf16_rne(np.ascontiguousarray(w.T))
    xp = np.zeros(m_pad * k_pad, np.uint16)
    xp[:m * k] = xb.reshape(-1)
    wp = np.zeros((n_pad, k_pad), np.uint16)
    wp[:n, :k] = wtb
    label = f"ignis forward {cfg.name()} {m}x{k}x{n}"
    _log(f"[case] {label}")
    kern = rt.ensure_gemm_kernel(cfg)
    xa, wa = bufs.up(xp), bufs.up(wp)
    y = bufs.up(np.full((m_pad, n_pad), SENTINEL, dtype=np.float32))
    ka = t0g.build_kernargs(xa, wa, y, k_pad, n_pad, m, cfg)
    gx, gy = t0g.compute_grid_auto(cfg, m, n_pad)
    rt.dispatch(kern, [gx, gy, 1], ka)
    got = rt.read(y, (m_pad, n_pad), np.float32)
    assert not np.any(got == SENTINEL)   # the whole padded tile grid is written, as the reference's kernel does
    ref = o.gemm("NT", xb.reshape(m, k), wtb, m, n, k)
    check_parity(got[:m, :n], ref, k, label)


# examples/test_gemm_backward.rs:118-287: GemmConfig::tile_64x64_k16 for both gradients, its 7
# sizes (M, K, N) and seeds; dX = dY * W through build_kernargs_backward_data on W = WT^T
# (host transpose), dW = dY^T * X through build_kernargs_backward_weight on dY^T and X^T
BACKWARD_SIZES = [(64, 64, 64), (128, 128, 128), (256, 256, 256), (128, 256, 512), (64, 512, 128), (256, 128, 256),
                  (512, 256, 128)]


@pytest.mark.parametrize("m,k,n", BACKWARD_SIZES)
def test_gemm_backward_harness(rt, bufs, m, k, n):
    cfg = t0g.GemmConfig.preset("tile_64x64_k16")
    x = o.rand_bf16_xorshift(m * k, m * 100 + k)
    w = o.rand_bf16_xorshift(n * k, n * 200 + k)          # WT [N][K]
    dy = o.rand_bf16_xorshift(m * n, m * 300 + n)
    kern = rt.ensure_gemm_kernel(cfg)
    _log(f"[case] backward harness tile_64x64_k16 {m}x{k}x{n}")
    # dX[M][K] = dY[M][N] * WT[N][K]
    w_t = o.transpose_bf16(w, n, k)                        # W [K][N]
    dya, wa = bufs.up(dy), bufs.up(w_t)
    dx = bufs.up(np.full(m * k + 64, SENTINEL, dtype=np.float32))
    ka = t0g.build_kernargs_backward_data(dya, wa, dx, m, n, k, cfg)
    gx, gy = t0g.compute_grid_backward_data(cfg, m, k)
    rt.dispatch(kern, [gx, gy, 1], ka)
    got = rt.read(dx, (m * k + 64,), np.float32)
    assert np.all(got[m * k:] == SENTINEL)
    check_parity(got[:m * k].reshape(m, k), o.gemm("NN", dy, w, m, k, n), n, f"backward dX {m}x{k}x{n}")
    # dW[N][K] = dY^T[N][M] * X[M][K]
    dy_t = o.transpose_bf16(dy, m, n)                      # [N][M]
    x_t = o.transpose_bf16(x, m, k)                        # [K][M]
    dyta, xta = bufs.up(dy_t), bufs.up(x_t)
    dw = bufs.up(np.full(n * k + 64, SENTINEL, dtype=np.float32))
    ka = t0g.build_kernargs_backward_weight(dyta, xta, dw, m, n, k, cfg)
    gx, gy = t0g.compute_grid_backward_weight(cfg, n, k)
    rt.dispatch(kern, [gx, gy, 1], ka)
    got = rt.read(dw, (n * k + 64,), np.float32)
    assert np.all(got[n * k:] == SENTINEL)
    check_parity(got[:n * k].reshape(n, k), o.gemm("TN", dy, x, n, k, m), m, f"backward dW {m}x{k}x{n}")
