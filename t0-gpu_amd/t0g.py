"""Python binding of libt0g (the MI355X bf16 GEMM path) over its C ABI.

Mirrors the reference's GEMM call surface so that callers and tests read like
the reference's own Rust code:

    cfg = auto_select(m, k, n)                    # src/t0/gemm_gen.rs:320
    gx, gy = compute_grid_auto(cfg, m, n)         # src/t0/gemm_gen.rs:402
    ka = build_kernargs(x, wt, y, k, n, m, cfg)   # src/t0/gemm_gen.rs:414
    rt = GpuRuntime.new()                         # src/ignis/gpu_context.rs:86
    kern = rt.ensure_gemm_kernel(cfg)             # generate + compile + load
    rt.dispatch(kern, [gx, gy, 1], ka)            # src/ignis/gpu_context.rs:264

plus a typed one-shot `GpuRuntime.gemm(...)`.  Every compute call runs the
gfx950 kernels in lib/libt0g.so; there is no CPU fallback: if the library is
missing the import fails loudly.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libt0g.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()' "
        f"or make -C t0-gpu_amd)")

_lib = ctypes.CDLL(LIB_PATH)

OK = 0
ERR_INVALID_ARG = 1
ERR_UNSUPPORTED_CONFIG = 2
ERR_HIP = 3
ERR_TIMEOUT = 4
ERR_POISONED = 5
ERR_NO_DEVICE = 6
ERR_OUT_OF_MEMORY = 7

NT, NN, TN, TT = 0, 1, 2, 3
LAYOUTS = {"NT": NT, "NN": NN, "TN": TN, "TT": TT}
EPI_STORE_F32, EPI_BIAS_ADD, EPI_BIAS_ADD_RELU = 0, 1, 2
F32, BF16 = 0, 1
STREAM_K = 0x80000000   # GemmConfig.split_k value selecting the stream-K schedule
# tile_ir EpilogueOp (src/t0/tile_ir.rs:41-62): the fused epilogue chain
OP_BIAS_ADD, OP_SCALE, OP_RELU, OP_SILU, OP_GELU, OP_ABS, OP_NEG, OP_CLAMP = range(1, 9)
EPILOGUE_OPS = {"bias": OP_BIAS_ADD, "scale": OP_SCALE, "relu": OP_RELU, "silu": OP_SILU,
                "gelu": OP_GELU, "abs": OP_ABS, "neg": OP_NEG, "clamp": OP_CLAMP}


class T0gError(RuntimeError):
    """A failed C-ABI call: `code` is the t0g_status, the message is t0g_last_error()."""

    def __init__(self, code, msg):
        super().__init__(f"[t0g status {code}] {msg}")
        self.code = code


class GemmConfig(ctypes.Structure):
    """GemmConfig (src/t0/gemm_gen.rs:56-84); split_k 0 means None."""

    _fields_ = [
        ("tile_m", ctypes.c_uint32),
        ("tile_n", ctypes.c_uint32),
        ("tile_k", ctypes.c_uint32),
        ("wg_size", ctypes.c_uint32),
        ("split_k", ctypes.c_uint32),
        ("lds_pad", ctypes.c_uint32),
        ("n_col_passes", ctypes.c_uint32),
        ("use_lds", ctypes.c_uint8),
        ("double_buffer", ctypes.c_uint8),
        ("swap_grid", ctypes.c_uint8),
        ("wgp_mode", ctypes.c_uint8),
        ("transpose", ctypes.c_uint32),
        ("epilogue", ctypes.c_uint32),
    ]

    @staticmethod
    def preset(name):
        """GemmConfig::tile_* (src/t0/gemm_gen.rs:88-145) or a native "gfx950_*" config."""
        cfg = GemmConfig()
        _check(_lib.t0g_config_preset(name.encode(), ctypes.byref(cfg)))
        return cfg

    @staticmethod
    def tile_preset(name):
        """TileGemm::tile_* (src/t0/tile_ir.rs:121-358), wg_size = tile_m."""
        cfg = GemmConfig()
        _check(_lib.t0g_tile_preset(name.encode(), ctypes.byref(cfg)))
        return cfg

    def is_native(self):
        return bool(_lib.t0g_config_is_native(ctypes.byref(self)))

    def copy(self, **changes):
        c = GemmConfig()
        ctypes.memmove(ctypes.byref(c), ctypes.byref(self), ctypes.sizeof(GemmConfig))
        for k, v in changes.items():
            setattr(c, k, v)
        return c

    def validate(self):
        _check(_lib.t0g_config_validate(ctypes.byref(self)))

    def n_waves(self):
        return _lib.t0g_config_n_waves(ctypes.byref(self))

    def lds_total(self):
        return _lib.t0g_config_lds_total(ctypes.byref(self))

    def name(self):
        buf = ctypes.create_string_buffer(128)
        _check(_lib.t0g_config_name(ctypes.byref(self), buf, len(buf)))
        return buf.value.decode()

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}

    def __repr__(self):
        return f"GemmConfig({self.name()})"


class GemmDesc(ctypes.Structure):
    _fields_ = [
        ("a", ctypes.c_uint64),
        ("b", ctypes.c_uint64),
        ("c", ctypes.c_uint64),
        ("bias", ctypes.c_uint64),
        ("workspace", ctypes.c_uint64),
        ("workspace_bytes", ctypes.c_uint64),
        ("m", ctypes.c_uint32),
        ("n", ctypes.c_uint32),
        ("k", ctypes.c_uint32),
        ("lda", ctypes.c_uint32),
        ("ldb", ctypes.c_uint32),
        ("ldc", ctypes.c_uint32),
        ("transpose", ctypes.c_uint32),
        ("out_dtype", ctypes.c_uint32),
        ("epilogue", ctypes.c_uint32),
        ("split_k", ctypes.c_uint32),
        ("config", ctypes.POINTER(GemmConfig)),
        ("epi_chain", ctypes.c_uint32),
        ("epi_scale", ctypes.c_float),
        ("clamp_min", ctypes.c_float),
        ("clamp_max", ctypes.c_float),
    ]


class KernelMeta(ctypes.Structure):
    """A kernel's entry in a gfx950 code object's AMDGPU metadata (t0g_kernel_meta)."""

    _fields_ = [
        ("kernarg_size", ctypes.c_uint32),
        ("kernarg_segment_size", ctypes.c_uint32),
        ("group_segment_size", ctypes.c_uint32),
        ("private_segment_size", ctypes.c_uint32),
        ("max_workgroup_size", ctypes.c_uint32),
        ("wavefront_size", ctypes.c_uint32),
    ]


class CompiledKernel(ctypes.Structure):
    """T0Kernel::compile output for a problem (t0g_compiled_kernel): code object,
    symbol, launch shape and argument block."""

    _fields_ = [
        ("code_object", ctypes.c_void_p),
        ("code_object_size", ctypes.c_size_t),
        ("name", ctypes.c_char * 96),
        ("workgroup_size", ctypes.c_uint32),
        ("lds_size", ctypes.c_uint32),
        ("kernarg_size", ctypes.c_uint32),
        ("grid", ctypes.c_uint32 * 3),
        ("splits", ctypes.c_uint32),
        ("kernargs", ctypes.c_uint8 * 160),
    ]

    def elf(self):
        """The code object's bytes (CompiledKernel.elf)."""
        return ctypes.string_at(self.code_object, self.code_object_size)

    def args(self):
        return bytes(self.kernargs[:self.kernarg_size])


class PoolInfo(ctypes.Structure):
    _fields_ = [
        ("cached_bytes", ctypes.c_uint64),
        ("cached_buffers", ctypes.c_uint64),
        ("live_bytes", ctypes.c_uint64),
        ("live_buffers", ctypes.c_uint64),
        ("hits", ctypes.c_uint64),
        ("misses", ctypes.c_uint64),
    ]


_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_p = ctypes.c_void_p
_cfgp = ctypes.POINTER(GemmConfig)
_u32p = ctypes.POINTER(ctypes.c_uint32)


def _sig(name, restype, *argtypes):
    f = getattr(_lib, name)
    f.restype = restype
    f.argtypes = list(argtypes)
    return f


_sig("t0g_last_error", ctypes.c_char_p)
_sig("t0g_version", ctypes.c_char_p)
_sig("t0g_config_preset", ctypes.c_int, ctypes.c_char_p, _cfgp)
_sig("t0g_tile_preset", ctypes.c_int, ctypes.c_char_p, _cfgp)
_sig("t0g_config_validate", ctypes.c_int, _cfgp)
_sig("t0g_config_is_native", ctypes.c_int, _cfgp)
_sig("t0g_config_n_waves", _u32, _cfgp)
_sig("t0g_config_lds_total", _u32, _cfgp)
_sig("t0g_config_name", ctypes.c_int, _cfgp, ctypes.c_char_p, ctypes.c_size_t)
_sig("t0g_tile_config_name", ctypes.c_int, _cfgp, _u32, ctypes.c_char_p, ctypes.c_size_t)
_sig("t0g_code_object_kernel_meta", ctypes.c_int, _p, ctypes.c_size_t, ctypes.c_char_p, ctypes.POINTER(KernelMeta))
_sig("t0g_auto_select", ctypes.c_int, _u32, _u32, _u32, _cfgp)
_sig("t0g_tile_auto_select", ctypes.c_int, _u32, _u32, _u32, _u32, _cfgp)
_sig("t0g_compute_grid", ctypes.c_int, _cfgp, _u32, _u32, _u32p, _u32p)
_sig("t0g_compute_grid_split_k", ctypes.c_int, _cfgp, _u32, _u32, _u32, _u32p, _u32p)
_sig("t0g_compute_grid_auto", ctypes.c_int, _cfgp, _u32, _u32, _u32p, _u32p)
_sig("t0g_tile_compute_grid", ctypes.c_int, _cfgp, _u32, _u32, _u32p)
_sig("t0g_build_kernargs", ctypes.c_int, _u64, _u64, _u64, _u32, _u32, _u32, _cfgp, ctypes.c_char_p)
_sig("t0g_build_kernargs_with_bias", ctypes.c_int, _u64, _u64, _u64, _u32, _u32, _u32, _cfgp, _u64,
     ctypes.c_char_p)
_sig("t0g_build_kernargs_m", ctypes.c_int, _u64, _u64, _u64, _u32, _u32, _u32, _cfgp, ctypes.c_char_p)
_sig("t0g_epilogue_chain", ctypes.c_int, _u32p, _u32, _u32p)
_sig("t0g_epilogue_chain_name", ctypes.c_int, _u32, ctypes.c_char_p, ctypes.c_size_t)
_sig("t0g_build_kernargs_m_epilogue", ctypes.c_int, _u64, _u64, _u64, _u32, _u32, _u32, _cfgp, _u32, _u64,
     ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_char_p, ctypes.POINTER(ctypes.c_size_t))
_sig("t0g_auto_select_backward_data", ctypes.c_int, _u32, _u32, _u32, _cfgp)
_sig("t0g_auto_select_backward_weight", ctypes.c_int, _u32, _u32, _u32, _cfgp)
_sig("t0g_build_kernargs_backward_data", ctypes.c_int, _u64, _u64, _u64, _u32, _u32, _u32, _cfgp,
     ctypes.c_char_p)
_sig("t0g_build_kernargs_backward_weight", ctypes.c_int, _u64, _u64, _u64, _u32, _u32, _u32, _cfgp,
     ctypes.c_char_p)
_sig("t0g_compute_grid_backward_data", ctypes.c_int, _cfgp, _u32, _u32, _u32p, _u32p)
_sig("t0g_compute_grid_backward_weight", ctypes.c_int, _cfgp, _u32, _u32, _u32p, _u32p)
_sig("t0g_device_count", ctypes.c_int, ctypes.POINTER(ctypes.c_int))
_sig("t0g_device_open", ctypes.c_int, ctypes.c_int, ctypes.POINTER(_p))
_sig("t0g_device_close", ctypes.c_int, _p)
_sig("t0g_device_set_stream", ctypes.c_int, _p, _p)
_sig("t0g_device_get_stream", ctypes.c_int, _p, ctypes.POINTER(_p))
_sig("t0g_device_is_poisoned", ctypes.c_int, _p, ctypes.POINTER(ctypes.c_int))
_sig("t0g_alloc", ctypes.c_int, _p, ctypes.c_size_t, ctypes.POINTER(_u64))
_sig("t0g_alloc_zero", ctypes.c_int, _p, ctypes.c_size_t, ctypes.POINTER(_u64))
_sig("t0g_free", ctypes.c_int, _p, _u64)
_sig("t0g_recycle", ctypes.c_int, _p, _u64)
_sig("t0g_pool_clear", ctypes.c_int, _p)
_sig("t0g_pool_stats", ctypes.c_int, _p, ctypes.POINTER(PoolInfo))
_sig("t0g_alloc_f32", ctypes.c_int, _p, ctypes.c_size_t, ctypes.POINTER(_u64))
_sig("t0g_write_f32", ctypes.c_int, _p, _u64, _p, ctypes.c_size_t)
_sig("t0g_read_f32", ctypes.c_int, _p, _u64, _p, ctypes.c_size_t)
_sig("t0g_upload_f32", ctypes.c_int, _p, _p, ctypes.c_size_t, ctypes.POINTER(_u64))
_sig("t0g_memcpy_h2d", ctypes.c_int, _p, _u64, _p, ctypes.c_size_t)
_sig("t0g_memcpy_d2h", ctypes.c_int, _p, _p, _u64, ctypes.c_size_t)
_sig("t0g_memset", ctypes.c_int, _p, _u64, ctypes.c_int, ctypes.c_size_t)
_sig("t0g_kernel_get", ctypes.c_int, _p, _cfgp, ctypes.POINTER(_p))
_sig("t0g_tile_kernel_get", ctypes.c_int, _p, _cfgp, ctypes.POINTER(_p))
_sig("t0g_tile_kernel_get_epilogue", ctypes.c_int, _p, _cfgp, _u32, ctypes.POINTER(_p))
_sig("t0g_kernel_load", ctypes.c_int, _p, _p, ctypes.c_size_t, ctypes.c_char_p, _u32p, _u32,
     ctypes.POINTER(_p))
_sig("t0g_kernel_info", ctypes.c_int, _p, _u32p, _u32p, _u32p, ctypes.c_char_p, ctypes.c_size_t)
_sig("t0g_dispatch", ctypes.c_int, _p, _p, _u32p, _p, ctypes.c_size_t)
_sig("t0g_dispatch_async", ctypes.c_int, _p, _p, _u32p, _p, ctypes.c_size_t)
_sig("t0g_wait_idle", ctypes.c_int, _p)
_sig("t0g_gemm", ctypes.c_int, _p, ctypes.POINTER(GemmDesc))
_sig("t0g_gemm_workspace_size", ctypes.c_int, ctypes.POINTER(GemmDesc), ctypes.POINTER(ctypes.c_size_t))
_sig("t0g_gemm_group", ctypes.c_int, _p, ctypes.POINTER(GemmDesc), _u32)
_sig("t0g_gemm_noalloc", ctypes.c_int, _p, ctypes.POINTER(GemmDesc))
_sig("t0g_gemm_kernel_name", ctypes.c_int, ctypes.POINTER(GemmDesc), ctypes.c_char_p, ctypes.c_size_t)
_sig("t0g_gemm_compile", ctypes.c_int, ctypes.POINTER(GemmDesc), ctypes.POINTER(CompiledKernel))
_sig("t0g_f32_to_bf16", ctypes.c_int, _p, _u64, _u64, ctypes.c_size_t)
_sig("t0g_matmul_f32", ctypes.c_int, _p, _u64, _u64, _u64, _u32, _u32, _u32)
_sig("t0g_matmul_backward_data_f32", ctypes.c_int, _p, _u64, _u64, _u64, _u32, _u32, _u32)
_sig("t0g_matmul_backward_weight_f32", ctypes.c_int, _p, _u64, _u64, _u64, _u32, _u32, _u32)
_sig("t0g_matmul_wt_bf16_f32", ctypes.c_int, _p, _u64, _u64, _u64, _u32, _u32, _u32)
_sig("t0g_bf16_cache_get", ctypes.c_int, _p, _u64, _u64, ctypes.c_size_t, ctypes.POINTER(_u64))
_sig("t0g_bf16_cache_invalidate", ctypes.c_int, _p, _u64)
_sig("t0g_bf16_cache_clear", ctypes.c_int, _p)
_sig("t0g_bf16_cache_stats", ctypes.c_int, _p, ctypes.POINTER(_u64), ctypes.POINTER(_u64))
_sig("t0g_matmul_f32_cached", ctypes.c_int, _p, _u64, _u64, _u64, _u64, _u32, _u32, _u32)
_sig("t0g_matmul_backward_data_f32_cached", ctypes.c_int, _p, _u64, _u64, _u64, _u64, _u32, _u32, _u32)


class TuneResult(ctypes.Structure):
    """GemmTuneResult (src/t0/auto_gemm.rs:28-42) without the ranking (GemmTuner.ranking)."""

    _fields_ = [
        ("best", GemmConfig),
        ("best_tflops", ctypes.c_double),
        ("m", ctypes.c_uint32),
        ("n", ctypes.c_uint32),
        ("k", ctypes.c_uint32),
        ("transpose", ctypes.c_uint32),
        ("out_dtype", ctypes.c_uint32),
        ("from_cache", ctypes.c_int32),
        ("n_all", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


_tunerp = ctypes.POINTER(_p)
_sig("t0g_tuner_create", ctypes.c_int, ctypes.c_char_p, _tunerp)
_sig("t0g_tuner_destroy", ctypes.c_int, _p)
_sig("t0g_tuner_global", ctypes.c_int, _tunerp)
_sig("t0g_tuner_set_params", ctypes.c_int, _p, _u32, _u32)
_sig("t0g_tuner_get_params", ctypes.c_int, _p, _u32p, _u32p, _u32p)
_sig("t0g_tuner_cache_dir", ctypes.c_int, _p, ctypes.c_char_p, ctypes.c_size_t)
_sig("t0g_tune_candidates", ctypes.c_int, _u32, _u32, _u32, _u32, _u32, _cfgp, _u32p)
_sig("t0g_tuner_tune", ctypes.c_int, _p, _p, _u32, _u32, _u32, _u32, _u32, _cfgp)
_sig("t0g_tuner_lookup", ctypes.c_int, _p, _u32, _u32, _u32, _u32, _u32, ctypes.POINTER(TuneResult),
     ctypes.POINTER(ctypes.c_int))
_sig("t0g_tuner_ranking", ctypes.c_int, _p, _u32, _u32, _u32, _u32, _u32, _u32, ctypes.c_char_p, ctypes.c_size_t,
     ctypes.POINTER(ctypes.c_double))
_sig("t0g_tuner_store", ctypes.c_int, _p, ctypes.POINTER(TuneResult), ctypes.POINTER(ctypes.c_char_p),
     ctypes.POINTER(ctypes.c_double), _u32)
_sig("t0g_tuner_invalidate", ctypes.c_int, _p, _u32, _u32, _u32, _u32, _u32)
_sig("t0g_tuner_clear", ctypes.c_int, _p)
_sig("t0g_tuner_report", ctypes.c_int, _p, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t))
_sig("t0g_auto_gemm", ctypes.c_int, _p, _p, _u64, _u64, _u64, _u32, _u32, _u32, ctypes.POINTER(ctypes.c_double))
_sig("t0g_tune_tile_ir", ctypes.c_int, _p, _p, _u32, _u32, _u32, ctypes.POINTER(TuneResult))
_sig("t0g_tile_ir_lookup", ctypes.c_int, _p, _u32, _u32, _u32, ctypes.POINTER(TuneResult), ctypes.POINTER(ctypes.c_int))
_sig("t0g_tile_ir_ranking", ctypes.c_int, _p, _u32, _u32, _u32, _u32, ctypes.c_char_p, ctypes.c_size_t,
     ctypes.POINTER(ctypes.c_double))
_sig("t0g_tile_ir_store", ctypes.c_int, _p, ctypes.POINTER(TuneResult), ctypes.POINTER(ctypes.c_char_p),
     ctypes.POINTER(ctypes.c_double), _u32)
_sig("t0g_stream_k_begin", _u32, _u32, _u32, _u32)
_sig("t0g_stream_k_worker", _u32, _u32, _u32, _u32)
_sig("t0g_stream_k_timeouts", ctypes.c_int, _p, _u32p)
_sig("t0g_debug_device_alloc_count", ctypes.c_int, ctypes.POINTER(_u64))
_sig("t0g_debug_fail_hip_call", ctypes.c_int, ctypes.c_int)
_sig("t0g_set_wait_timeout_ms", ctypes.c_int, _u32)
_sig("t0g_set_stream_k_spin_limit", ctypes.c_int, _u32)
_sig("t0g_debug_stream_k_stall", ctypes.c_int, ctypes.c_int)
_sig("t0g_set_split_k_mode", ctypes.c_int, _u32)
_sig("t0g_set_timeline", ctypes.c_int, ctypes.c_int)
_sig("t0g_timeline_read", ctypes.c_int, _p, ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t,
     ctypes.POINTER(ctypes.c_size_t))
_sig("t0g_timeline_clear", ctypes.c_int, _p)


def _check(rc):
    if rc != OK:
        raise T0gError(rc, _lib.t0g_last_error().decode(errors="replace"))


def last_error():
    return _lib.t0g_last_error().decode(errors="replace")


def version():
    return _lib.t0g_version().decode()


def library():
    """The loaded ctypes.CDLL (for symbol-level tests)."""
    return _lib


# ---- selection, grids, kernargs (host only) ---------------------------------

def auto_select(m, k, n):
    cfg = GemmConfig()
    _check(_lib.t0g_auto_select(m, k, n, ctypes.byref(cfg)))
    return cfg


def tile_auto_select(m, k, n, transpose=NT):
    cfg = GemmConfig()
    _check(_lib.t0g_tile_auto_select(m, k, n, transpose, ctypes.byref(cfg)))
    return cfg


def _grid2(fn, *args):
    gx, gy = ctypes.c_uint32(), ctypes.c_uint32()
    _check(fn(*args, ctypes.byref(gx), ctypes.byref(gy)))
    return gx.value, gy.value


def compute_grid(cfg, m, n):
    return _grid2(_lib.t0g_compute_grid, ctypes.byref(cfg), m, n)


def compute_grid_split_k(cfg, m, n, split_k):
    return _grid2(_lib.t0g_compute_grid_split_k, ctypes.byref(cfg), m, n, split_k)


def compute_grid_auto(cfg, m, n):
    return _grid2(_lib.t0g_compute_grid_auto, ctypes.byref(cfg), m, n)


def tile_compute_grid(cfg, m, n):
    g = (ctypes.c_uint32 * 3)()
    _check(_lib.t0g_tile_compute_grid(ctypes.byref(cfg), m, n, g))
    return [g[0], g[1], g[2]]


def build_kernargs(x, wt, y, k, n, m, cfg):
    buf = ctypes.create_string_buffer(40)
    _check(_lib.t0g_build_kernargs(x, wt, y, k, n, m, ctypes.byref(cfg), buf))
    return buf.raw


def build_kernargs_with_bias(x, wt, y, k, n, m, cfg, bias):
    buf = ctypes.create_string_buffer(48)
    _check(_lib.t0g_build_kernargs_with_bias(x, wt, y, k, n, m, ctypes.byref(cfg), bias, buf))
    return buf.raw


def build_kernargs_m(x, wt, y, k, n, m, cfg):
    buf = ctypes.create_string_buffer(44)
    _check(_lib.t0g_build_kernargs_m(x, wt, y, k, n, m, ctypes.byref(cfg), buf))
    return buf.raw


def build_kernargs_m_epilogue(x, wt, y, k, n, m, cfg, chain, bias=0, epi_scale=1.0, clamp=(0.0, 0.0)):
    """build_kernargs_m + the epilogue arguments lower_gemm declares after M (src/t0/tile_ir.rs:661-683)."""
    buf = ctypes.create_string_buffer(64)
    ln = ctypes.c_size_t()
    _check(_lib.t0g_build_kernargs_m_epilogue(x, wt, y, k, n, m, ctypes.byref(cfg), chain, bias, epi_scale,
                                              clamp[0], clamp[1], buf, ctypes.byref(ln)))
    return buf.raw[:ln.value]


def auto_select_backward_data(m, n_orig, k_orig):
    cfg = GemmConfig()
    _check(_lib.t0g_auto_select_backward_data(m, n_orig, k_orig, ctypes.byref(cfg)))
    return cfg


def auto_select_backward_weight(m, n_orig, k_orig):
    cfg = GemmConfig()
    _check(_lib.t0g_auto_select_backward_weight(m, n_orig, k_orig, ctypes.byref(cfg)))
    return cfg


def build_kernargs_backward_data(dy, w, dx, m, n_orig, k_orig, cfg):
    buf = ctypes.create_string_buffer(40)
    _check(_lib.t0g_build_kernargs_backward_data(dy, w, dx, m, n_orig, k_orig, ctypes.byref(cfg), buf))
    return buf.raw


def build_kernargs_backward_weight(dy_t, x_t, dw, m, n_orig, k_orig, cfg):
    buf = ctypes.create_string_buffer(40)
    _check(_lib.t0g_build_kernargs_backward_weight(dy_t, x_t, dw, m, n_orig, k_orig, ctypes.byref(cfg), buf))
    return buf.raw


def compute_grid_backward_data(cfg, m, k_orig):
    return _grid2(_lib.t0g_compute_grid_backward_data, ctypes.byref(cfg), m, k_orig)


def compute_grid_backward_weight(cfg, n_orig, k_orig):
    return _grid2(_lib.t0g_compute_grid_backward_weight, ctypes.byref(cfg), n_orig, k_orig)


def epilogue_chain(ops):
    """TileGemm::with_epilogue (src/t0/tile_ir.rs:440): op codes or names -> packed chain."""
    codes = [EPILOGUE_OPS[o] if isinstance(o, str) else int(o) for o in ops]
    arr = (ctypes.c_uint32 * max(1, len(codes)))(*codes)
    out = ctypes.c_uint32()
    _check(_lib.t0g_epilogue_chain(arr, len(codes), ctypes.byref(out)))
    return out.value


def epilogue_chain_name(chain):
    buf = ctypes.create_string_buffer(96)
    _check(_lib.t0g_epilogue_chain_name(chain, buf, len(buf)))
    return buf.value.decode()


def gemm_desc(a, b, c, m, n, k, transpose=NT, out_dtype=F32, lda=0, ldb=0, ldc=0, split_k=0,
              epilogue=EPI_STORE_F32, bias=0, workspace=0, workspace_bytes=0, config=None,
              epilogue_ops=None, epi_scale=1.0, clamp=(0.0, 0.0)):
    """epilogue_ops: a tile_ir epilogue chain (op codes or names); overrides `epilogue`."""
    d = GemmDesc()
    d.a, d.b, d.c, d.bias = a, b, c, bias
    d.workspace, d.workspace_bytes = workspace, workspace_bytes
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb, d.ldc = lda, ldb, ldc
    d.transpose = LAYOUTS[transpose] if isinstance(transpose, str) else transpose
    d.out_dtype = out_dtype
    d.epilogue = epilogue
    d.split_k = split_k
    d.config = ctypes.pointer(config) if config is not None else None
    d.epi_chain = epilogue_chain(epilogue_ops) if epilogue_ops else 0
    d.epi_scale = epi_scale
    d.clamp_min, d.clamp_max = clamp
    return d


def gemm_workspace_size(desc):
    n = ctypes.c_size_t()
    _check(_lib.t0g_gemm_workspace_size(ctypes.byref(desc), ctypes.byref(n)))
    return n.value


def gemm_kernel_name(desc):
    buf = ctypes.create_string_buffer(128)
    _check(_lib.t0g_gemm_kernel_name(ctypes.byref(desc), buf, len(buf)))
    return buf.value.decode()


def gemm_compile(desc):
    """T0Kernel::compile + build_kernargs + compute_grid for desc (host only)."""
    out = CompiledKernel()
    _check(_lib.t0g_gemm_compile(ctypes.byref(desc), ctypes.byref(out)))
    return out


def code_object_kernel_meta(code_object, symbol):
    """KernelMeta of `symbol` in a gfx950 code object (bytes), read on the host."""
    blob = bytes(code_object)
    buf = ctypes.create_string_buffer(blob, len(blob))
    meta = KernelMeta()
    _check(_lib.t0g_code_object_kernel_meta(buf, len(blob), symbol.encode(), ctypes.byref(meta)))
    return meta


def tile_config_name(cfg, chain=0):
    """TileGemm::name (src/t0/tile_ir.rs:398-430)."""
    buf = ctypes.create_string_buffer(160)
    _check(_lib.t0g_tile_config_name(ctypes.byref(cfg), chain, buf, len(buf)))
    return buf.value.decode()


def set_stream_k_spin_limit(polls):
    _check(_lib.t0g_set_stream_k_spin_limit(polls))


def debug_stream_k_stall(on):
    _check(_lib.t0g_debug_stream_k_stall(1 if on else 0))


SPLIT_K_REDUCE_KERNEL, SPLIT_K_IN_KERNEL, SPLIT_K_AUTO = 0, 1, 2


def set_split_k_mode(mode):
    """SPLIT_K_REDUCE_KERNEL: planes + reduce kernel; SPLIT_K_IN_KERNEL: split-K reduced
    inside the GEMM kernel where the plan allows it; SPLIT_K_AUTO (default): in the kernel
    for two K slices on the deep-ring tiles, else planes.  Same bits every way."""
    _check(_lib.t0g_set_split_k_mode(mode))


TIMELINE_SLOTS = 8192
TIMELINE_TICK_NS = 10.0   # the GPU's constant 100 MHz clock


def set_timeline(on):
    """Record per-workgroup timelines of later GEMM launches (diagnostic)."""
    _check(_lib.t0g_set_timeline(1 if on else 0))


def device_alloc_count():
    """Device allocations (hipMalloc, code-object loads) the library has made in this process."""
    c = _u64()
    _check(_lib.t0g_debug_device_alloc_count(ctypes.byref(c)))
    return c.value


def debug_fail_hip_call(n):
    _check(_lib.t0g_debug_fail_hip_call(n))


def set_wait_timeout_ms(ms):
    _check(_lib.t0g_set_wait_timeout_ms(ms))


def device_count():
    n = ctypes.c_int()
    _check(_lib.t0g_device_count(ctypes.byref(n)))
    return n.value


class Kernel:
    """A GpuKernel handle (owned by its GpuRuntime)."""

    def __init__(self, handle):
        self.handle = handle

    def info(self):
        wg, lds, ka = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        name = ctypes.create_string_buffer(128)
        _check(_lib.t0g_kernel_info(self.handle, ctypes.byref(wg), ctypes.byref(lds), ctypes.byref(ka), name,
                                    len(name)))
        return {"wg_size": wg.value, "lds_size": lds.value, "kernarg_size": ka.value, "name": name.value.decode()}


class GpuRuntime:
    """GpuRuntime (src/ignis/gpu_context.rs:86-147) over one HIP device."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def new(ordinal=0):
        h = ctypes.c_void_p()
        _check(_lib.t0g_device_open(ordinal, ctypes.byref(h)))
        return GpuRuntime(h)

    def close(self):
        if self.handle:
            _check(_lib.t0g_device_close(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def stream_k_timeouts(self):
        v = ctypes.c_uint32()
        _check(_lib.t0g_stream_k_timeouts(self.handle, ctypes.byref(v)))
        return v.value

    def set_stream(self, hip_stream_ptr):
        _check(_lib.t0g_device_set_stream(self.handle, ctypes.c_void_p(hip_stream_ptr or None)))

    def stream(self):
        s = ctypes.c_void_p()
        _check(_lib.t0g_device_get_stream(self.handle, ctypes.byref(s)))
        return s.value

    def is_poisoned(self):
        v = ctypes.c_int()
        _check(_lib.t0g_device_is_poisoned(self.handle, ctypes.byref(v)))
        return bool(v.value)

    # memory (src/ignis/gpu_context.rs:437-487, src/kfd/mod.rs:947-1055)
    def alloc(self, nbytes):
        a = ctypes.c_uint64()
        _check(_lib.t0g_alloc(self.handle, nbytes, ctypes.byref(a)))
        return a.value

    def alloc_zero(self, nbytes):
        a = ctypes.c_uint64()
        _check(_lib.t0g_alloc_zero(self.handle, nbytes, ctypes.byref(a)))
        return a.value

    def free(self, addr):
        _check(_lib.t0g_free(self.handle, addr))

    def recycle(self, addr):
        """GpuRuntime::recycle: back to the buffer pool instead of freed."""
        _check(_lib.t0g_recycle(self.handle, addr))

    def pool_clear(self):
        _check(_lib.t0g_pool_clear(self.handle))

    def pool_stats(self):
        info = PoolInfo()
        _check(_lib.t0g_pool_stats(self.handle, ctypes.byref(info)))
        return {f: getattr(info, f) for f, _ in PoolInfo._fields_}

    def alloc_f32(self, n):
        """GpuRuntime::alloc_f32: n floats, 512-byte padded, zeroed."""
        a = ctypes.c_uint64()
        _check(_lib.t0g_alloc_f32(self.handle, n, ctypes.byref(a)))
        return a.value

    def write_f32(self, addr, data):
        import numpy as np
        arr = np.ascontiguousarray(data, dtype=np.float32)
        _check(_lib.t0g_write_f32(self.handle, addr, arr.ctypes.data, arr.size))

    def read_f32(self, addr, n):
        """GpuRuntime::read_f32: waits for queued work, then copies n floats."""
        import numpy as np
        out = np.empty(n, dtype=np.float32)
        _check(_lib.t0g_read_f32(self.handle, addr, out.ctypes.data, n))
        return out

    def upload_f32(self, data):
        """GpuRuntime::upload_f32: alloc_f32 + write_f32."""
        import numpy as np
        arr = np.ascontiguousarray(data, dtype=np.float32)
        a = ctypes.c_uint64()
        _check(_lib.t0g_upload_f32(self.handle, arr.ctypes.data, arr.size, ctypes.byref(a)))
        return a.value

    def write(self, addr, array):
        """Host numpy array -> device (GpuBuffer::write)."""
        import numpy as np
        arr = np.ascontiguousarray(array)
        _check(_lib.t0g_memcpy_h2d(self.handle, addr, arr.ctypes.data, arr.nbytes))

    def read(self, addr, shape, dtype):
        """Device -> new host numpy array (GpuBuffer::read)."""
        import numpy as np
        out = np.empty(shape, dtype=dtype)
        _check(_lib.t0g_memcpy_d2h(self.handle, out.ctypes.data, addr, out.nbytes))
        return out

    def upload(self, array):
        import numpy as np
        arr = np.ascontiguousarray(array)
        addr = self.alloc(arr.nbytes)
        self.write(addr, arr)
        return addr

    def timeline_clear(self):
        _check(_lib.t0g_timeline_clear(self.handle))

    def timeline_read(self, workgroups=TIMELINE_SLOTS):
        """[workgroups][4] uint64: clock at entry, after the K loop, after the stores
        (ticks of TIMELINE_TICK_NS), then XCC_ID << 32 | HW_ID; rows of workgroups
        that did not run are zero."""
        import numpy as np
        out = np.zeros((workgroups, 4), dtype=np.uint64)
        n = ctypes.c_size_t()
        _check(_lib.t0g_timeline_read(self.handle, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                      out.size, ctypes.byref(n)))
        return out

    def memset(self, addr, value, nbytes):
        _check(_lib.t0g_memset(self.handle, addr, value, nbytes))

    # kernels and dispatch
    def ensure_gemm_kernel(self, cfg):
        h = ctypes.c_void_p()
        _check(_lib.t0g_kernel_get(self.handle, ctypes.byref(cfg), ctypes.byref(h)))
        return Kernel(h)

    def ensure_tile_kernel(self, cfg, epilogue_chain=0):
        """lower_gemm(&spec) + load; epilogue_chain: the spec's tile_ir epilogue (packed)."""
        h = ctypes.c_void_p()
        if epilogue_chain:
            _check(_lib.t0g_tile_kernel_get_epilogue(self.handle, ctypes.byref(cfg), epilogue_chain,
                                                     ctypes.byref(h)))
        else:
            _check(_lib.t0g_tile_kernel_get(self.handle, ctypes.byref(cfg), ctypes.byref(h)))
        return Kernel(h)

    def load_kernel(self, code_object, symbol, workgroup_size, lds_size=0):
        h = ctypes.c_void_p()
        wg = (ctypes.c_uint32 * 3)(*workgroup_size)
        buf = ctypes.create_string_buffer(bytes(code_object), len(code_object))
        _check(_lib.t0g_kernel_load(self.handle, buf, len(code_object), symbol.encode(), wg, lds_size,
                                    ctypes.byref(h)))
        return Kernel(h)

    def _dispatch(self, fn, kernel, grid, kernargs):
        g = (ctypes.c_uint32 * 3)(*grid)
        buf = ctypes.create_string_buffer(bytes(kernargs), len(kernargs))
        _check(fn(self.handle, kernel.handle, g, buf, len(kernargs)))

    def dispatch(self, kernel, grid, kernargs):
        self._dispatch(_lib.t0g_dispatch, kernel, grid, kernargs)

    def dispatch_async(self, kernel, grid, kernargs):
        self._dispatch(_lib.t0g_dispatch_async, kernel, grid, kernargs)

    def wait_idle(self):
        _check(_lib.t0g_wait_idle(self.handle))

    def gemm_desc(self, desc):
        _check(_lib.t0g_gemm(self.handle, ctypes.byref(desc)))

    def gemm_noalloc(self, desc):
        """t0g_gemm without allocating: split-K planes in the device's static scratch
        array (T0G_NOALLOC_SCRATCH_BYTES) or desc.workspace."""
        _check(_lib.t0g_gemm_noalloc(self.handle, ctypes.byref(desc)))

    def gemm_group(self, descs):
        """Enqueue independent GEMMs (GemmDesc list) to run concurrently."""
        arr = (GemmDesc * max(1, len(descs)))(*descs)
        _check(_lib.t0g_gemm_group(self.handle, arr, len(descs)))

    def gemm(self, a, b, c, m, n, k, **kw):
        """Enqueue C = op(A) op(B) on the device stream (asynchronous)."""
        self.gemm_desc(gemm_desc(a, b, c, m, n, k, **kw))

    # Ignis bf16_matmul caller path (src/ignis/ops/bf16_matmul.rs) on f32 device tensors
    def f32_to_bf16(self, src, dst, n):
        _check(_lib.t0g_f32_to_bf16(self.handle, src, dst, n))

    def matmul_f32(self, x, w, y, m, k, n):
        """bf16_matmul::matmul forward: Y[M,N] = bf16(X[M,K]) bf16(W[K,N])."""
        _check(_lib.t0g_matmul_f32(self.handle, x, w, y, m, k, n))

    def matmul_backward_data_f32(self, dy, w, dx, m, k, n):
        """gemm_backward_data: dX[M,K] = bf16(dY[M,N]) bf16(W[K,N])^T."""
        _check(_lib.t0g_matmul_backward_data_f32(self.handle, dy, w, dx, m, k, n))

    def matmul_backward_weight_f32(self, x, dy, dw, m, k, n):
        """gemm_backward_weight: dW[K,N] = bf16(X[M,K])^T bf16(dY[M,N])."""
        _check(_lib.t0g_matmul_backward_weight_f32(self.handle, x, dy, dw, m, k, n))

    def matmul_wt_bf16_f32(self, x, wt_bf16, y, m, k, n):
        """matmul_with_wt_bf16: Y[M,N] = bf16(X[M,K]) WT[N,K]^T."""
        _check(_lib.t0g_matmul_wt_bf16_f32(self.handle, x, wt_bf16, y, m, k, n))

    # GpuRuntime::{get_or_create_bf16, invalidate_bf16, clear_bf16_cache} (src/ignis/gpu_context.rs:385-433)
    def get_or_create_bf16(self, tensor_id, f32_addr, n):
        out = _u64()
        _check(_lib.t0g_bf16_cache_get(self.handle, tensor_id, f32_addr, n, ctypes.byref(out)))
        return out.value

    def invalidate_bf16(self, tensor_id):
        _check(_lib.t0g_bf16_cache_invalidate(self.handle, tensor_id))

    def clear_bf16_cache(self):
        _check(_lib.t0g_bf16_cache_clear(self.handle))

    def bf16_cache_stats(self):
        e, b = _u64(), _u64()
        _check(_lib.t0g_bf16_cache_stats(self.handle, ctypes.byref(e), ctypes.byref(b)))
        return e.value, b.value

    def matmul_f32_cached(self, x, w, w_id, y, m, k, n):
        """matmul with W's bf16 copy from the cache under w_id."""
        _check(_lib.t0g_matmul_f32_cached(self.handle, x, w, w_id, y, m, k, n))

    def matmul_backward_data_f32_cached(self, dy, w, w_id, dx, m, k, n):
        _check(_lib.t0g_matmul_backward_data_f32_cached(self.handle, dy, w, w_id, dx, m, k, n))


# ---- autotuner (src/t0/auto_gemm.rs) -----------------------------------------

def _layout(t):
    return LAYOUTS[t.upper()] if isinstance(t, str) else int(t)


def tune_candidates(m, n, k, transpose=NT, max_count=64):
    """The configs GemmTuner.tune benchmarks, best modelled first."""
    arr = (GemmConfig * max_count)()
    cnt = ctypes.c_uint32()
    _check(_lib.t0g_tune_candidates(m, n, k, _layout(transpose), max_count, arr, ctypes.byref(cnt)))
    return [arr[i].copy() for i in range(cnt.value)]


class GemmTuner:
    """GemmTuner (src/t0/auto_gemm.rs:46-417): GPU-benchmarked config choice with
    an in-memory and on-disk cache (one JSON file per problem)."""

    def __init__(self, handle, owned=True):
        self.handle = handle
        self._owned = owned

    @staticmethod
    def new():
        h = _p()
        _check(_lib.t0g_tuner_create(None, ctypes.byref(h)))
        return GemmTuner(h)

    @staticmethod
    def with_cache_dir(path):
        h = _p()
        _check(_lib.t0g_tuner_create(os.fsencode(str(path)), ctypes.byref(h)))
        return GemmTuner(h)

    @staticmethod
    def global_tuner():
        h = _p()
        _check(_lib.t0g_tuner_global(ctypes.byref(h)))
        return GemmTuner(h, owned=False)

    def close(self):
        if self.handle and self._owned:
            _check(_lib.t0g_tuner_destroy(self.handle))
        self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _params(self):
        mc, it, nc = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        _check(_lib.t0g_tuner_get_params(self.handle, ctypes.byref(mc), ctypes.byref(it), ctypes.byref(nc)))
        return mc.value, it.value, nc.value

    @property
    def max_candidates(self):
        return self._params()[0]

    @max_candidates.setter
    def max_candidates(self, v):
        _check(_lib.t0g_tuner_set_params(self.handle, v, self.n_iters))

    @property
    def n_iters(self):
        return self._params()[1]

    @n_iters.setter
    def n_iters(self, v):
        _check(_lib.t0g_tuner_set_params(self.handle, self.max_candidates, v))

    def __len__(self):
        return self._params()[2]

    @property
    def cache_dir(self):
        buf = ctypes.create_string_buffer(4096)
        _check(_lib.t0g_tuner_cache_dir(self.handle, buf, len(buf)))
        return buf.value.decode()

    def tune(self, rt, m, n, k, transpose=NT, out_dtype=F32):
        """GemmTuner::tune(rt, m, n, k) -> best GemmConfig (argument order as the reference)."""
        cfg = GemmConfig()
        _check(_lib.t0g_tuner_tune(self.handle, rt.handle, m, n, k, _layout(transpose), out_dtype,
                                   ctypes.byref(cfg)))
        return cfg

    def lookup(self, m, n, k, transpose=NT, out_dtype=F32):
        """The cached TuneResult (memory, then disk) or None."""
        r = TuneResult()
        found = ctypes.c_int()
        _check(_lib.t0g_tuner_lookup(self.handle, m, n, k, _layout(transpose), out_dtype, ctypes.byref(r),
                                     ctypes.byref(found)))
        return r if found.value else None

    def ranking(self, m, n, k, transpose=NT, out_dtype=F32):
        """GemmTuneResult::all: [(config name, TFLOPS)], fastest first."""
        r = self.lookup(m, n, k, transpose, out_dtype)
        if r is None:
            return []
        out = []
        buf = ctypes.create_string_buffer(256)
        tf = ctypes.c_double()
        for i in range(r.n_all):
            _check(_lib.t0g_tuner_ranking(self.handle, m, n, k, _layout(transpose), out_dtype, i, buf, len(buf),
                                          ctypes.byref(tf)))
            out.append((buf.value.decode(), tf.value))
        return out

    def save_cache(self, m, n, k, best, best_tflops, all_=(), transpose=NT, out_dtype=F32):
        """save_cache (src/t0/auto_gemm.rs:364-391) of a result and its ranking."""
        r = TuneResult()
        r.best = best
        r.best_tflops = best_tflops
        r.m, r.n, r.k = m, n, k
        r.transpose = _layout(transpose)
        r.out_dtype = out_dtype
        names = (ctypes.c_char_p * max(1, len(all_)))(*[nm.encode() for nm, _ in all_])
        tfs = (ctypes.c_double * max(1, len(all_)))(*[t for _, t in all_])
        _check(_lib.t0g_tuner_store(self.handle, ctypes.byref(r), names, tfs, len(all_)))

    def invalidate(self, m, n, k, transpose=NT, out_dtype=F32):
        _check(_lib.t0g_tuner_invalidate(self.handle, m, n, k, _layout(transpose), out_dtype))

    def clear(self):
        _check(_lib.t0g_tuner_clear(self.handle))

    def tune_tile_ir(self, rt, m, n, k):
        """tune_tile_ir(rt, m, n, k) (src/t0/cost_model.rs:788-1013) -> TuneResult."""
        r = TuneResult()
        _check(_lib.t0g_tune_tile_ir(self.handle, rt.handle, m, n, k, ctypes.byref(r)))
        return r

    def tile_ir_lookup(self, m, n, k):
        r = TuneResult()
        found = ctypes.c_int()
        _check(_lib.t0g_tile_ir_lookup(self.handle, m, n, k, ctypes.byref(r), ctypes.byref(found)))
        return r if found.value else None

    def tile_ir_ranking(self, m, n, k):
        """TileIrTuneResult::all: [(TileGemm name, TFLOPS)], fastest first."""
        r = self.tile_ir_lookup(m, n, k)
        if r is None:
            return []
        out = []
        buf = ctypes.create_string_buffer(256)
        tf = ctypes.c_double()
        for i in range(r.n_all):
            _check(_lib.t0g_tile_ir_ranking(self.handle, m, n, k, i, buf, len(buf), ctypes.byref(tf)))
            out.append((buf.value.decode(), tf.value))
        return out

    def save_tile_ir_cache(self, m, n, k, best, best_tflops, all_=()):
        """save_tile_ir_cache (src/t0/cost_model.rs:1076-1093)."""
        r = TuneResult()
        r.best = best
        r.best_tflops = best_tflops
        r.m, r.n, r.k = m, n, k
        names = (ctypes.c_char_p * max(1, len(all_)))(*[nm.encode() for nm, _ in all_])
        tfs = (ctypes.c_double * max(1, len(all_)))(*[t for _, t in all_])
        _check(_lib.t0g_tile_ir_store(self.handle, ctypes.byref(r), names, tfs, len(all_)))

    def report(self):
        need = ctypes.c_size_t()
        _check(_lib.t0g_tuner_report(self.handle, None, 0, ctypes.byref(need)))
        buf = ctypes.create_string_buffer(need.value)
        _check(_lib.t0g_tuner_report(self.handle, buf, len(buf), ctypes.byref(need)))
        return buf.value.decode()


def auto_gemm(rt, a, b, c, m, n, k, tuner=None):
    """auto_gemm(rt, a, b, c, m, n, k) (src/t0/auto_gemm.rs:445-480): tune (NT, f32 out)
    and run C = A * B^T with the best config, synchronously; returns the cached TFLOPS."""
    tf = ctypes.c_double()
    _check(_lib.t0g_auto_gemm(tuner.handle if tuner is not None else None, rt.handle, a, b, c, m, n, k, ctypes.byref(tf)))
    return tf.value


def tune_tile_ir(rt, m, n, k, tuner=None):
    """tune_tile_ir(rt, m, n, k) -> TileIrTuneResult (src/t0/cost_model.rs:788-1013),
    on the global tuner unless one is given."""
    r = TuneResult()
    _check(_lib.t0g_tune_tile_ir(tuner.handle if tuner is not None else None, rt.handle, m, n, k, ctypes.byref(r)))
    return r


def stream_k_begin(total, grid, w):
    """First (tile, K step) pair of stream-K workgroup w (w = grid: the total)."""
    return _lib.t0g_stream_k_begin(total, grid, w)


def stream_k_worker(total, grid, it):
    """The stream-K workgroup whose range holds pair `it`."""
    return _lib.t0g_stream_k_worker(total, grid, it)
