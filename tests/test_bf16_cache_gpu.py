"""GpuRuntime's bf16 weight cache (src/ignis/gpu_context.rs:100, 385-433) through the
C ABI: get_or_create_bf16 converts once per tensor id, invalidate_bf16 makes the next
use reconvert, clear_bf16_cache drops every entry; the cached matmul entry points take
W's copy from it.  Results against the oracle on the RNE-converted operands."""
import numpy as np
import pytest

import oracle as o
import t0g
from test_gemm_gpu import Buffers, _log, check_parity

pytestmark = pytest.mark.gpu


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


def test_get_or_create_converts_once(rt, bufs):
    rt.clear_bf16_cache()
    rng = np.random.default_rng(1)
    w = rng.standard_normal(10007, dtype=np.float32)
    wa = bufs.up(w)
    a1 = rt.get_or_create_bf16(7, wa, w.size)
    rt.wait_idle()
    assert np.array_equal(rt.read(a1, (w.size,), np.uint16), o.f32_to_bf16_rne(w))
    assert rt.bf16_cache_stats()[0] == 1
    # the f32 tensor changes, the id does not: the cache keeps the first conversion
    rt.write(wa, -w)
    a2 = rt.get_or_create_bf16(7, wa, w.size)
    rt.wait_idle()
    assert a2 == a1
    assert np.array_equal(rt.read(a2, (w.size,), np.uint16), o.f32_to_bf16_rne(w))
    # after invalidate_bf16 the next call converts the tensor as it is now
    rt.invalidate_bf16(7)
    assert rt.bf16_cache_stats()[0] == 0
    a3 = rt.get_or_create_bf16(7, wa, w.size)
    rt.wait_idle()
    assert np.array_equal(rt.read(a3, (w.size,), np.uint16), o.f32_to_bf16_rne(-w))
    # another size under the same id is a caller error, not a silent short buffer
    with pytest.raises(t0g.T0gError) as e:
        rt.get_or_create_bf16(7, wa, w.size - 1)
    assert e.value.code == t0g.ERR_INVALID_ARG
    # the cache owns its buffers
    with pytest.raises(t0g.T0gError):
        rt.free(a3)
    rt.clear_bf16_cache()
    assert rt.bf16_cache_stats() == (0, 0)
    assert not rt.is_poisoned()


@pytest.mark.parametrize("m,k,n", [(1, 4, 2), (100, 300, 72), (1024, 4096, 1104)])
def test_cached_matmul_forward_and_backward_data(rt, bufs, m, k, n):
    rt.clear_bf16_cache()
    rng = np.random.default_rng(m + 3 * n)
    x = rng.standard_normal((m, k), dtype=np.float32)
    w = rng.standard_normal((k, n), dtype=np.float32) * 0.1
    w_new = rng.standard_normal((k, n), dtype=np.float32) * 0.1
    dy = rng.standard_normal((m, n), dtype=np.float32)
    x16, dy16 = o.f32_to_bf16_rne(x), o.f32_to_bf16_rne(dy)
    xa, wa, dya = bufs.up(x), bufs.up(w), bufs.up(dy)
    y, dx = bufs.alloc(4 * m * n, fill=0), bufs.alloc(4 * m * k, fill=0)
    wid = 0xABCD0000 + m

    def expect(wmat):
        w16 = o.f32_to_bf16_rne(wmat)
        return (o.gemm("NN", x16, w16, m, n, k), o.gemm("NT", dy16, w16, m, k, n))

    _log(f"[case] cached matmul {m}x{k}x{n}")
    for step in range(2):                       # the second step converts nothing
        rt.matmul_f32_cached(xa, wa, wid, y, m, k, n)
        rt.matmul_backward_data_f32_cached(dya, wa, wid, dx, m, k, n)
        rt.wait_idle()
        ey, edx = expect(w)
        check_parity(rt.read(y, (m, n), np.float32), ey, k, f"cached forward step {step}")
        check_parity(rt.read(dx, (m, k), np.float32), edx, n, f"cached backward data step {step}")
        assert rt.bf16_cache_stats()[0] == 1
    # a weight update without invalidate is not seen (the cache's contract) ...
    rt.write(wa, w_new)
    rt.matmul_f32_cached(xa, wa, wid, y, m, k, n)
    rt.wait_idle()
    stale = rt.read(y, (m, n), np.float32)
    check_parity(stale, expect(w)[0], k, "stale weight copy")
    # ... and with it, the next call converts the updated weight
    rt.invalidate_bf16(wid)
    rt.matmul_f32_cached(xa, wa, wid, y, m, k, n)
    rt.matmul_backward_data_f32_cached(dya, wa, wid, dx, m, k, n)
    rt.wait_idle()
    ey, edx = expect(w_new)
    check_parity(rt.read(y, (m, n), np.float32), ey, k, "forward after invalidate")
    check_parity(rt.read(dx, (m, k), np.float32), edx, n, "backward data after invalidate")
    # the uncached entry point gives the same bits
    y2 = bufs.alloc(4 * m * n, fill=0)
    rt.matmul_f32(xa, wa, y2, m, k, n)
    rt.wait_idle()
    assert np.array_equal(rt.read(y2, (m, n), np.float32), rt.read(y, (m, n), np.float32))
    rt.clear_bf16_cache()
