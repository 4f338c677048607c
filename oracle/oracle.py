"""numpy front end of the CPU oracle (oracle/ref_gemm.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker (or as the timed CPU baseline); the
product path never imports it.  See ref_gemm.c for the reference lines each
function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


if not os.path.exists(LIB_PATH):
    build()

_lib = ctypes.CDLL(LIB_PATH)
_sz = ctypes.c_size_t
_p = ctypes.c_void_p


def _sig(name, restype, *argtypes):
    f = getattr(_lib, name)
    f.restype = restype
    f.argtypes = list(argtypes)
    return f


_sig("oracle_f32_to_bf16_rne", ctypes.c_uint16, ctypes.c_float)
_sig("oracle_f32_to_bf16_trunc", ctypes.c_uint16, ctypes.c_float)
_sig("oracle_bf16_to_f32", ctypes.c_float, ctypes.c_uint16)
_sig("oracle_f32_to_bf16_rne_array", None, _p, _p, _sz)
_sig("oracle_bf16_to_f32_array", None, _p, _p, _sz)
_sig("oracle_rand_bf16_xorshift", None, _p, _sz, ctypes.c_uint64)
_sig("oracle_rand_bf16_lcg", None, _p, _sz, ctypes.c_uint64)
_sig("oracle_make_bf16_suite", None, _p, _sz, ctypes.c_uint64)
_sig("oracle_linear_init_f32", None, _p, _sz, _sz, ctypes.c_uint64)
_sig("oracle_randn_bf16", None, _p, _sz, ctypes.c_uint64, ctypes.c_double)
_sig("oracle_gemm_nt_naive", None, _p, _p, _p, _sz, _sz, _sz)
_sig("oracle_gemm_nt_naive_rows", None, _p, _p, _p, _sz, _sz, _sz, _sz, _sz)
_sig("oracle_gemm", None, ctypes.c_int, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _sz, ctypes.c_int)
_sig("oracle_gemm_krange", None, ctypes.c_int, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _sz, _sz, ctypes.c_int)
_sig("oracle_splitk_reduce", None, _p, _p, _sz, _sz)
_sig("oracle_transpose_bf16", None, _p, _p, _sz, _sz)
_sig("oracle_num_threads", ctypes.c_int)

LAYOUT = {"NT": 0, "NN": 1, "TN": 2, "TT": 3}


def _u16(a):
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, a.dtype
    return a


def f32_to_bf16_rne(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _lib.oracle_f32_to_bf16_rne_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def f32_to_bf16_trunc(x):
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_to_f32(x):
    x = _u16(x)
    out = np.empty(x.shape, dtype=np.float32)
    _lib.oracle_bf16_to_f32_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def rand_bf16_xorshift(n, seed):
    out = np.empty(n, dtype=np.uint16)
    _lib.oracle_rand_bf16_xorshift(out.ctypes.data, n, seed)
    return out


def rand_bf16_lcg(n, seed):
    out = np.empty(n, dtype=np.uint16)
    _lib.oracle_rand_bf16_lcg(out.ctypes.data, n, seed)
    return out


def make_bf16_suite(n, seed):
    out = np.empty(n, dtype=np.uint16)
    _lib.oracle_make_bf16_suite(out.ctypes.data, n, seed)
    return out


def linear_init_f32(in_features, out_features, seed=42):
    out = np.empty((in_features, out_features), dtype=np.float32)
    _lib.oracle_linear_init_f32(out.ctypes.data, in_features, out_features, seed)
    return out


def randn_bf16(n, seed, sigma=1.0):
    out = np.empty(n, dtype=np.uint16)
    _lib.oracle_randn_bf16(out.ctypes.data, n, seed, sigma)
    return out


def gemm_nt_naive(x, wt, m, k, n, rows=None):
    """Faithful single-thread reference loop; rows=(begin, end) computes a row block only."""
    x, wt = _u16(x), _u16(wt)
    y = np.zeros((m, n), dtype=np.float32)
    if rows is None:
        _lib.oracle_gemm_nt_naive(x.ctypes.data, wt.ctypes.data, y.ctypes.data, m, k, n)
    else:
        _lib.oracle_gemm_nt_naive_rows(x.ctypes.data, wt.ctypes.data, y.ctypes.data, m, k, n, rows[0], rows[1])
    return y


def gemm(layout, a, b, m, n, k, lda=None, ldb=None, threads=0):
    """Bit-identical fast restatement, any of NT/NN/TN/TT (see ref_gemm.c)."""
    lay = LAYOUT[layout] if isinstance(layout, str) else layout
    a, b = _u16(a), _u16(b)
    a_mk = lay in (0, 1)
    b_kn = lay in (1, 2)
    lda = lda or (k if a_mk else m)
    ldb = ldb or (n if b_kn else k)
    c = np.empty((m, n), dtype=np.float32)
    _lib.oracle_gemm(lay, a.ctypes.data, b.ctypes.data, c.ctypes.data, m, n, k, lda, ldb, n, threads)
    return c


def gemm_rows(layout, a, b, m, n, k, rows, threads=0):
    """Rows `rows` (an index array) of the product, with the same per-element order."""
    lay = LAYOUT[layout] if isinstance(layout, str) else layout
    a = _u16(a).reshape(-1)
    rows = np.asarray(rows)
    if lay in (0, 1):   # A stored [M][K]: take the rows
        a_sub = a.reshape(m, k)[rows]
        return gemm(lay, a_sub, b, len(rows), n, k, threads=threads)
    a_sub = np.ascontiguousarray(a.reshape(k, m)[:, rows])   # A stored [K][M]: take the columns
    return gemm(lay, a_sub, b, len(rows), n, k, threads=threads)


def gemm_krange(layout, a, b, m, n, k, k_begin, k_end, threads=0):
    lay = LAYOUT[layout] if isinstance(layout, str) else layout
    a, b = _u16(a), _u16(b)
    a_mk = lay in (0, 1)
    b_kn = lay in (1, 2)
    lda = k if a_mk else m
    ldb = n if b_kn else k
    c = np.empty((m, n), dtype=np.float32)
    _lib.oracle_gemm_krange(lay, a.ctypes.data, b.ctypes.data, c.ctypes.data, m, n, lda, ldb, n, k_begin, k_end,
                            threads)
    return c


def splitk_reduce(planes):
    planes = np.ascontiguousarray(planes, dtype=np.float32)
    sk = planes.shape[0]
    y = np.empty(planes.shape[1:], dtype=np.float32)
    _lib.oracle_splitk_reduce(planes.ctypes.data, y.ctypes.data, y.size, sk)
    return y


def transpose_bf16(a, rows, cols):
    a = _u16(a)
    out = np.empty(rows * cols, dtype=np.uint16)
    _lib.oracle_transpose_bf16(a.ctypes.data, out.ctypes.data, rows, cols)
    return out.reshape(cols, rows)


def num_threads():
    return _lib.oracle_num_threads()


# Entries whose reference magnitude is below 2^-100 are judged by max|d| alone.
# The hardware exp2 and reciprocal of the SiLU/GELU epilogue (v_exp_f32,
# v_rcp_f32: the instructions the reference emits, src/t0/tile_ir.rs:2270-2317)
# flush subnormal results, so x * rcp(1 + exp(-x)) is 0 on the device where the
# fp32 CPU expectation keeps a subnormal reciprocal: for x near -88 the two
# differ by up to |x| * 2^-126 ~ 1e-36.  A matrix made only of such values
# (the reference's LCG inputs are all <= 0, so every GEMM output of a long K is
# positive and [silu, scale < 0, silu] sends all of them there) would otherwise
# fail relF on differences of 1e-36.
RELF_FLOOR = 2.0 ** -100
# Those entries must still lie within TINY_ABS + 5e-3 * rms(the other entries)
# of the reference: the relF scale where the matrix has ordinary values (an
# entry that cancels to exactly 0.0 in the CPU's fp32 sum keeps the GPU's
# summation noise), and TINY_ABS, far above the flush differences (~1e-36) and
# far below any result that is merely wrong, where every entry is tiny.
TINY_ABS = 2.0 ** -90


def parity(c_gpu, c_ref, k):
    """The north-star gate: relF <= 5e-3 and max|d| <= 1e-2 * sqrt(K/256).  Returns (ok, relF, maxabs, bound).

    relF is taken over the entries with |ref| >= RELF_FLOOR; the others must lie within
    TINY_ABS + 5e-3 * rms(ref over the former) of the reference."""
    c_gpu = np.asarray(c_gpu, dtype=np.float64)
    c_ref = np.asarray(c_ref, dtype=np.float64)
    diff = c_gpu - c_ref
    big = np.abs(c_ref) >= RELF_FLOOR
    nref = np.linalg.norm(c_ref[big])
    relf = float(np.linalg.norm(diff[big]) / nref) if nref > 0 else 0.0
    maxabs = float(np.max(np.abs(diff))) if diff.size else 0.0
    n_big = int(np.count_nonzero(big))
    tiny_bound = TINY_ABS + (5e-3 * nref / np.sqrt(n_big) if n_big else 0.0)
    tiny_ok = not np.any(np.abs(diff[~big]) > tiny_bound)
    bound = 1e-2 * np.sqrt(max(k, 1) / 256.0)
    return (relf <= 5e-3 and maxabs <= bound and tiny_ok), relf, maxabs, bound


# Epilogue chain: tile_ir's EpilogueOp (src/t0/tile_ir.rs:41-62) as applied by
# emit_epilogue_on_vreg (src/t0/tile_ir.rs:2213-2339), in fp32 and in chain
# order.  SiLU is the CPU expectation of the reference's own GPU test
# (src/t0/tile_ir.rs:5113-5117: x * 1/(1 + exp(-x))); GELU is the sigmoid
# approximation the reference emits (src/t0/tile_ir.rs:2283-2317:
# x * sigmoid(1.702 x)), not the tanh form its doc comment names.
EPI_BIAS, EPI_SCALE, EPI_RELU, EPI_SILU, EPI_GELU, EPI_ABS, EPI_NEG, EPI_CLAMP = range(1, 9)
EPI_NAMES = {"bias": EPI_BIAS, "scale": EPI_SCALE, "relu": EPI_RELU, "silu": EPI_SILU, "gelu": EPI_GELU,
             "abs": EPI_ABS, "neg": EPI_NEG, "clamp": EPI_CLAMP}


def _sigmoid_f32(y):
    with np.errstate(over="ignore"):
        return np.float32(1.0) / (np.float32(1.0) + np.exp(-y))


def epilogue_chain(c, ops, bias=None, scale=1.0, clamp=(0.0, 0.0)):
    """Apply a tile_ir epilogue chain (op codes or names) to fp32 results c[M][N]."""
    x = np.array(c, dtype=np.float32, copy=True)
    for op in ops:
        op = EPI_NAMES[op] if isinstance(op, str) else op
        if op == EPI_BIAS:
            x = x + np.asarray(bias, dtype=np.float32)[None, :]
        elif op == EPI_SCALE:
            x = x * np.float32(scale)
        elif op == EPI_RELU:
            x = np.maximum(x, np.float32(0.0))
        elif op == EPI_SILU:
            x = x * _sigmoid_f32(x)
        elif op == EPI_GELU:
            x = x * _sigmoid_f32(x * np.float32(1.702))
        elif op == EPI_ABS:
            x = np.abs(x)
        elif op == EPI_NEG:
            x = -x
        elif op == EPI_CLAMP:
            x = np.minimum(np.maximum(x, np.float32(clamp[0])), np.float32(clamp[1]))
        else:
            raise ValueError(f"unknown epilogue op {op}")
    return x
