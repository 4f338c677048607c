"""Pins the CPU oracle (oracle/ref_gemm.c) before anything is checked against it.

Each check is chosen so a plausible restatement mistake fails it:
  * reference-held torch goldens (benchmarks/torch_ref, copied as data) pin the
    NT orientation and the fp32 result; a transposed operand or a dropped K term
    is shown to miss them by orders of magnitude;
  * the fast multithreaded variant must equal the naive reference loop bit for bit
    in every layout (layouts differ only by exact data movement);
  * all-ones inputs give C = K exactly (examples/hello_gemm_gen.rs:72-133);
  * random cases sit inside the fp32 sequential-sum error bound around an exact
    fp64 sum (bf16 products are exact in fp64);
  * bf16 rounding helpers are checked on IEEE tie cases; the PRNGs against an
    independent big-integer restatement and their documented ranges.
"""
import math
import os

import numpy as np
import pytest

import oracle as o
from conftest import GOLDEN

TR = os.path.join(GOLDEN, "torch_ref")


def _bin(name, dtype, shape):
    return np.fromfile(os.path.join(TR, name), dtype=dtype).reshape(shape)


def test_golden_manifest_intact():
    import hashlib
    with open(os.path.join(TR, "MANIFEST.txt")) as f:
        for line in f:
            digest, name = line.split()
            with open(os.path.join(TR, name), "rb") as g:
                assert hashlib.sha256(g.read()).hexdigest() == digest, name


@pytest.mark.parametrize("w_name,ref_name", [("w_gate.bin", "h_gate_f32ref.bin"), ("w_up.bin", "h_up_f32ref.bin")])
def test_nt_gemm_matches_torch_golden(w_name, ref_name):
    x = _bin("x.bin", np.uint16, (64, 256))
    w = _bin(w_name, np.uint16, (512, 256))
    ref = _bin(ref_name, np.float32, (64, 512))
    y = o.gemm_nt_naive(x, w, 64, 256, 512)
    # torch's fp32 mm sums in another order; both are within a few ulp of the exact sum.
    assert np.abs(y - ref).max() <= 1e-6
    assert np.array_equal(o.gemm("NT", x, w, 64, 512, 256), y)


def test_second_gemm_matches_torch_golden():
    s = _bin("swiglu_bf16_trunc.bin", np.uint16, (64, 512))
    wd = _bin("w_down.bin", np.uint16, (256, 512))
    ref = _bin("y_bf16_f32acc.bin", np.float32, (64, 256))
    y = o.gemm("NT", s, wd, 64, 256, 512)
    assert np.abs(y - ref).max() <= 1e-6


def test_golden_discriminates_plausible_mistakes():
    x = _bin("x.bin", np.uint16, (64, 256))
    w = _bin("w_gate.bin", np.uint16, (512, 256))
    ref = _bin("h_gate_f32ref.bin", np.float32, (64, 512))
    wrong_orientation = o.gemm("NN", x, w, 64, 512, 256)        # B read as [K][N]
    assert np.abs(wrong_orientation - ref).max() > 0.1
    dropped_term = o.gemm("NT", np.ascontiguousarray(x[:, :255]), np.ascontiguousarray(w[:, :255]), 64, 512, 255)
    assert np.abs(dropped_term - ref).max() > 1e-3
    bf16_out = o.bf16_to_f32(o.f32_to_bf16_rne(o.gemm("NT", x, w, 64, 512, 256)))
    assert np.abs(bf16_out - ref).max() > 1e-4                   # output rounding is visible too


def test_bf16_golden_is_rounded_fp32_result():
    """h_gate_bf16acc is torch's bf16 GEMM: bf16-valued and within bf16 rounding of the fp32 golden."""
    ref = _bin("h_gate_f32ref.bin", np.float32, (64, 512))
    b16 = _bin("h_gate_bf16acc.bin", np.float32, (64, 512))
    assert np.all((b16.view(np.uint32) & 0xFFFF) == 0)
    assert np.all(np.abs(b16 - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-30)


def bf16_ulp_distance(a16, b16):
    """|a - b| in bf16 ulps (sign-magnitude bit patterns mapped onto one ordered integer line)."""
    def line(b):
        b = np.asarray(b).astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(line(a16) - line(b16))


# torch's bf16-output GEMMs (benchmarks/gen_torch_ref.py: torch.mm on bf16 operands, fp32
# accumulation, bf16 result), the goldens src/t0/precision_vs_torch.rs:115-118 compares against
BF16_GOLDENS = [("x.bin", (64, 256), "w_gate.bin", (512, 256), "h_gate_bf16acc.bin"),
                ("x.bin", (64, 256), "w_up.bin", (512, 256), "h_up_bf16acc.bin"),
                ("swiglu_bf16_trunc.bin", (64, 512), "w_down.bin", (256, 512), "y_bf16chain.bin")]


@pytest.mark.parametrize("a_name,a_shape,b_name,b_shape,gold", BF16_GOLDENS)
def test_bf16_output_mode_matches_torch_bf16_gemm(a_name, a_shape, b_name, b_shape, gold):
    """The oracle's bf16 output (RNE of its fp32 result, t0g's bf16 mode) equals torch's bf16
    GEMM to within one bf16 ulp everywhere, and exactly on all but a few entries (torch sums
    in another order, so a result next to a rounding boundary may round the other way)."""
    a = _bin(a_name, np.uint16, a_shape)
    b = _bin(b_name, np.uint16, b_shape)
    m, k = a_shape
    n = b_shape[0]
    g = _bin(gold, np.float32, (m, n))
    assert np.array_equal(o.bf16_to_f32(o.f32_to_bf16_rne(g)), g)   # the golden is bf16-valued
    got = o.f32_to_bf16_rne(o.gemm("NT", a, b, m, n, k))
    d = bf16_ulp_distance(got, o.f32_to_bf16_rne(g))
    assert d.max() <= 1 and np.count_nonzero(d) <= 8, (d.max(), np.count_nonzero(d))
    # a truncating output (RTZ) or a wrong operand misses it by far more
    trunc = o.f32_to_bf16_trunc(o.gemm("NT", a, b, m, n, k))
    assert np.count_nonzero(bf16_ulp_distance(trunc, o.f32_to_bf16_rne(g))) > a_shape[0] * n // 10


@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
@pytest.mark.parametrize("m,n,k", [(37, 23, 61), (64, 128, 300), (1, 5, 1), (16, 1, 7)])
def test_fast_oracle_bit_equal_to_naive_loop(layout, m, n, k):
    a_nk = o.rand_bf16_xorshift(m * k, m * 1000 + k).reshape(m, k)   # op(A) as [M][K]
    b_nk = o.rand_bf16_xorshift(n * k, n * 2000 + k).reshape(n, k)   # op(B)^T as [N][K]
    naive = o.gemm_nt_naive(a_nk, b_nk, m, k, n)
    a_st = a_nk if layout in ("NT", "NN") else np.ascontiguousarray(a_nk.T)
    b_st = b_nk if layout in ("NT", "TT") else np.ascontiguousarray(b_nk.T)
    fast = o.gemm(layout, a_st, b_st, m, n, k, threads=3)
    assert np.array_equal(fast.view(np.uint32), naive.view(np.uint32))


def test_gemm_rows_matches_full_product():
    m, n, k = 96, 40, 130
    for layout in ("NT", "NN", "TN", "TT"):
        a = o.rand_bf16_lcg(m * k, 5)
        b = o.rand_bf16_lcg(n * k, 6)
        full = o.gemm(layout, a, b, m, n, k)
        rows = np.array([0, 7, 95, 31])
        assert np.array_equal(o.gemm_rows(layout, a, b, m, n, k, rows), full[rows])


@pytest.mark.parametrize("k", [1, 256, 4096, 32768])
def test_all_ones_known_answer(k):
    m, n = 4, 8
    ones = np.full(m * k, 0x3F80, dtype=np.uint16)
    onesb = np.full(n * k, 0x3F80, dtype=np.uint16)
    assert np.all(o.gemm_nt_naive(ones, onesb, m, k, n) == float(k))
    assert np.all(o.gemm("NT", ones, onesb, m, n, k) == float(k))


@pytest.mark.parametrize("m,n,k", [(32, 48, 256), (8, 8, 4096)])
def test_within_fp32_sequential_sum_bound_of_exact(m, n, k):
    a = o.rand_bf16_xorshift(m * k, 11).reshape(m, k)
    b = o.rand_bf16_xorshift(n * k, 12).reshape(n, k)
    c = o.gemm("NT", a, b, m, n, k).astype(np.float64)
    af = o.bf16_to_f32(a).astype(np.float64)
    bf = o.bf16_to_f32(b).astype(np.float64)
    exact = af @ bf.T
    absum = np.abs(af) @ np.abs(bf).T
    gamma = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    assert np.all(np.abs(c - exact) <= gamma * absum + 1e-30)


def test_bf16_rounding_helpers():
    def f(bits):
        return np.array([bits], dtype=np.uint32).view(np.float32)[0]
    # RNE ties go to even, above-half rounds up, below-half down.
    assert o.f32_to_bf16_rne(np.float32(f(0x3F808000)))[()] == 0x3F80
    assert o.f32_to_bf16_rne(np.float32(f(0x3F818000)))[()] == 0x3F82
    assert o.f32_to_bf16_rne(np.float32(f(0x3F808001)))[()] == 0x3F81
    assert o.f32_to_bf16_rne(np.float32(f(0x3F807FFF)))[()] == 0x3F80
    assert o.f32_to_bf16_trunc(np.float32(f(0x3F80FFFF)))[()] == 0x3F80
    assert o.bf16_to_f32(np.array([0x3F80, 0xC000], dtype=np.uint16)).tolist() == [1.0, -2.0]
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32)
    r = o.bf16_to_f32(o.f32_to_bf16_rne(x))
    assert np.all(np.abs(r - x) <= np.abs(x) * 2.0 ** -8)   # half an ulp of an 8-bit significand


def test_xorshift_generator_matches_integer_restatement():
    seed = 256 * 1000 + 256
    got = o.rand_bf16_xorshift(6, seed)
    s = seed ^ 0xDEADBEEFCAFEBABE
    mask = (1 << 64) - 1
    expect = []
    for _ in range(6):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        f = (np.float32(s >> 32) / np.float32(4294967295.0)) * np.float32(2.0) - np.float32(1.0)
        expect.append(int(o.f32_to_bf16_rne(np.float32(f))[()]))
    assert got.tolist() == expect
    vals = o.bf16_to_f32(o.rand_bf16_xorshift(100000, 7))
    assert vals.min() >= -1.0 and vals.max() <= 1.0 and abs(vals.mean()) < 0.01


def test_lcg_generators_range_and_restatement():
    got = o.rand_bf16_lcg(4, 42 + 128)
    rng = 42 + 128
    mask = (1 << 64) - 1
    expect = []
    for _ in range(4):
        rng = (rng * 6364136223846793005 + 1442695040888963407) & mask
        f = np.float32(rng >> 33) / np.float32(2.0 ** 31) - np.float32(1.0)
        expect.append(int((np.float32(f * np.float32(0.5))).view(np.uint32) >> 16))
    assert got.tolist() == expect
    # (rng >> 33) / 2^31 lies in [0, 1), so the reference's "random" values are
    # one-sided: f in [-1, 0), times 0.5 -> [-0.5, 0].  Restated as is.
    vals = o.bf16_to_f32(o.rand_bf16_lcg(100000, 3))
    assert vals.min() >= -0.5 and vals.max() <= 0.0 and abs(vals.mean() + 0.25) < 0.01
    suite = o.bf16_to_f32(o.make_bf16_suite(100000, 42))
    assert suite.min() >= -1.0 and suite.max() <= 0.99
    w = o.linear_init_f32(4096, 16, seed=42)
    scale = np.float32(np.sqrt(2.0 / 4096))
    assert w.min() >= -scale and w.max() <= 0.0 and abs(float(w.mean()) + 0.5 * scale) < 0.01 * scale


def test_randn_generator_moments():
    v = o.bf16_to_f32(o.randn_bf16(200001, 2, 0.02)).astype(np.float64)
    assert abs(v.mean()) < 2e-4 and abs(v.std() - 0.02) < 2e-4


def test_splitk_partials_sum_in_plane_order():
    m, n, k, sk = 16, 24, 512, 4
    a = o.rand_bf16_lcg(m * k, 1)
    b = o.rand_bf16_lcg(n * k, 2)
    planes = np.stack([o.gemm_krange("NT", a, b, m, n, k, s * k // sk, (s + 1) * k // sk) for s in range(sk)])
    y = o.splitk_reduce(planes)
    manual = np.zeros((m, n), dtype=np.float32)
    for s in range(sk):
        manual = manual + planes[s]
    assert np.array_equal(y, manual)
    assert np.abs(y - o.gemm("NT", a, b, m, n, k)).max() < 1e-4
    ones = np.full(m * k, 0x3F80, dtype=np.uint16)
    onesb = np.full(n * k, 0x3F80, dtype=np.uint16)
    p1 = np.stack([o.gemm_krange("NT", ones, onesb, m, n, k, s * 128, (s + 1) * 128) for s in range(4)])
    assert np.all(o.splitk_reduce(p1) == float(k))


def test_parity_gate_rejects_wrong_results():
    m, n, k = 64, 64, 256
    a = o.rand_bf16_xorshift(m * k, 1)
    b = o.rand_bf16_xorshift(n * k, 2)
    c = o.gemm("NT", a, b, m, n, k)
    assert o.parity(c, c, k)[0]
    bad = c.copy()
    bad[3, 5] += 0.02
    assert not o.parity(bad, c, k)[0]
    assert not o.parity(c.T.copy(), c, k)[0]


def test_parity_gate_subnormal_regime():
    """Entries below 2^-100 count in max|d| only: a device result that flushes a
    subnormal reciprocal passes, an error in ordinary values still fails, and a
    tiny value in the place of an ordinary one fails through relF."""
    x = np.linspace(-84.0, -88.5, 4096).astype(np.float32).reshape(64, 64)   # exp(-x) < FLT_MAX
    ref = o.epilogue_chain(x, ["silu"])                 # CPU fp32, subnormal reciprocals kept
    assert np.abs(ref).max() < 1e-34 and (np.abs(ref) >= 2.0 ** -126).all()
    e = np.exp(np.float32(-1.0) * x.astype(np.float64))
    flushed = np.where(1.0 / (1.0 + e) < 2.0 ** -126, 0.0, ref).astype(np.float32)
    assert (flushed == 0).any() and o.parity(flushed, ref, 256)[0]
    mixed_ref = ref.copy()
    mixed_ref[0, :8] = 1.0
    assert o.parity(flushed.copy() + (mixed_ref - ref), mixed_ref, 256)[0]
    wrong = mixed_ref.copy()
    wrong[0, 3] = 1.02                                  # 2 % off in an ordinary entry
    assert not o.parity(wrong, mixed_ref, 256)[0]
    dropped = mixed_ref.copy()
    dropped[0, :8] = 1e-35                              # ordinary values replaced by tiny ones
    assert not o.parity(dropped, mixed_ref, 256)[0]
    # an output that is simply wrong over a reference made only of tiny values: relF has
    # nothing to measure there, and max|d| = 1e-3 is inside the K-scaled bound
    garbage = np.full_like(ref, 1e-3)
    assert not o.parity(garbage, ref, 256)[0]
    assert not o.parity(-flushed + 2.0 ** -80, ref, 256)[0]
    # an entry of an ordinary matrix that cancels to exactly 0.0 in the CPU's sum keeps the
    # GPU's fp32 summation noise, which is fine; an error there at the matrix's own scale is not
    rng = np.random.default_rng(3)
    dense = rng.standard_normal((64, 64)).astype(np.float32)
    dense[5, 7] = 0.0
    noisy = dense.copy()
    noisy[5, 7] = 3e-8
    assert o.parity(noisy, dense, 256)[0]
    noisy[5, 7] = 0.008              # inside max|d|'s bound (0.01), not counted in relF
    assert not o.parity(noisy, dense, 256)[0]


def test_epilogue_chain_known_answers():
    """Each epilogue op against values fixed by the mathematics (not by retyping the
    oracle's formulas): exact results for the piecewise ops, the identity
    f(x) - f(-x) = x that any x * sigmoid(a x) satisfies, sigmoid's value at known
    points computed in fp64, and chain order."""
    x = np.array([[-3.0, -0.5, 0.0, 0.25, 2.0, 40.0, -40.0]], dtype=np.float32)
    bias = np.array([1.0, 1.0, -1.0, 0.5, -4.0, 0.0, 0.0], dtype=np.float32)
    assert np.array_equal(o.epilogue_chain(x, ["relu"]), [[0, 0, 0, 0.25, 2.0, 40.0, 0]])
    assert np.array_equal(o.epilogue_chain(x, ["abs"]), np.abs(x))
    assert np.array_equal(o.epilogue_chain(x, ["neg"]), -x)
    assert np.array_equal(o.epilogue_chain(x, ["clamp"], clamp=(-1.0, 1.0)), [[-1, -0.5, 0, 0.25, 1, 1, -1]])
    assert np.array_equal(o.epilogue_chain(x, ["scale"], scale=0.5), x * 0.5)
    assert np.array_equal(o.epilogue_chain(x, ["bias"], bias=bias), x + bias)
    # order matters: bias then ReLU is not ReLU then bias
    assert np.array_equal(o.epilogue_chain(x, ["bias", "relu"], bias=bias), [[0, 0.5, 0, 0.75, 0, 40.0, 0]])
    assert np.array_equal(o.epilogue_chain(x, ["relu", "bias"], bias=bias), [[1, 1, -1, 0.75, -2.0, 40.0, 0]])
    # x*sigmoid(a x) - (-x)*sigmoid(-a x) = x for any a: pins the sign and the form
    for op in ("silu", "gelu"):
        f = o.epilogue_chain(x, [op]).astype(np.float64)
        g = o.epilogue_chain(-x, [op]).astype(np.float64)
        assert np.allclose(f - g, x, rtol=0, atol=2e-6), op
    # values at x = 1 (fp64 sigmoid): silu(1) = 1/(1+e^-1), gelu(1) = 1/(1+e^-1.702)
    one = np.ones((1, 1), dtype=np.float32)
    assert abs(float(o.epilogue_chain(one, ["silu"])[0, 0]) - 1 / (1 + math.exp(-1.0))) < 1e-6
    assert abs(float(o.epilogue_chain(one, ["gelu"])[0, 0]) - 1 / (1 + math.exp(-1.702))) < 1e-6
    # saturation: large |x| gives x or 0, without NaN
    s = o.epilogue_chain(x, ["silu"])
    assert s[0, 5] == 40.0 and abs(s[0, 6]) < 1e-12 and np.isfinite(s).all()
