"""ctypes view of the ggml-base C ABI (include/ggml_host.h), the same entry
points the OpenASR Rust host binds in
crates/openasr-core/src/ggml_runtime/ffi.rs:399-1057, plus loading of the
MI355X plugin through the verified loader (ffi.rs:415-434,
ggml_runtime/backend.rs:1290-1444).

This is the host side of the drop-in boundary as tests, the benchmark and
the smoke check drive it. Nothing here computes: every op runs inside
libggml-mi355x.so on the GPU.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
LIB_DIR = ROOT / "lib"
BASE_PATH = LIB_DIR / "libggml-base.so"
PLUGIN_PATH = LIB_DIR / "libggml-mi355x.so"

GGML_MAX_DIMS = 4
GGML_MAX_SRC = 10

# element types (ffi.rs:343-351)
F32, F16, Q4_0, Q8_0, Q3_K, Q4_K, Q8_K, I32, I64 = 0, 1, 2, 8, 11, 12, 15, 26, 27
TYPE_NAMES = {F32: "f32", F16: "f16", Q8_0: "q8_0", Q3_K: "q3_K", Q4_K: "q4_K", I32: "i32"}

GGML_ROPE_TYPE_NEOX = 2
GGML_PREC_DEFAULT, GGML_PREC_F32 = 0, 10
STATUS_SUCCESS = 0
BUFFER_USAGE_WEIGHTS, BUFFER_USAGE_COMPUTE = 1, 2


class ggml_init_params(C.Structure):
    _fields_ = [("mem_size", C.c_size_t), ("mem_buffer", C.c_void_p), ("no_alloc", C.c_bool)]


class ggml_tensor(C.Structure):
    _fields_ = [
        ("type", C.c_int),
        ("buffer", C.c_void_p),
        ("ne", C.c_int64 * 4),
        ("nb", C.c_size_t * 4),
        ("op", C.c_int),
        ("op_params", C.c_int32 * 16),
        ("flags", C.c_int32),
        ("src", C.c_void_p * GGML_MAX_SRC),
        ("view_src", C.c_void_p),
        ("view_offs", C.c_size_t),
        ("data", C.c_void_p),
        ("name", C.c_char * 64),
        ("extra", C.c_void_p),
        ("padding", C.c_char * 8),
    ]


class cancel_capability(C.Structure):
    _fields_ = [("mechanism", C.c_int), ("observation_granularity", C.c_int)]


assert C.sizeof(ggml_tensor) == 336

T = C.c_void_p  # ggml_tensor *
CTX = C.c_void_p

_base = None


def _sig(lib, name, restype, *argtypes):
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = list(argtypes)


def base() -> C.CDLL:
    """Load libggml-base.so (RTLD_GLOBAL, so the plugin resolves its imports)."""
    global _base
    if _base is not None:
        return _base
    if not BASE_PATH.exists():
        raise RuntimeError(f"{BASE_PATH} is missing: run `python -m openasr_amd.build` first")
    lib = C.CDLL(str(BASE_PATH), mode=C.RTLD_GLOBAL)
    i64, sz, f, i = C.c_int64, C.c_size_t, C.c_float, C.c_int
    _sig(lib, "ggml_init", CTX, ggml_init_params)
    _sig(lib, "ggml_free", None, CTX)
    _sig(lib, "ggml_tensor_overhead", sz)
    _sig(lib, "ggml_graph_overhead_custom", sz, sz, C.c_bool)
    _sig(lib, "ggml_nbytes", sz, T)
    _sig(lib, "ggml_nelements", i64, T)
    _sig(lib, "ggml_row_size", sz, i, i64)
    _sig(lib, "ggml_type_size", sz, i)
    _sig(lib, "ggml_blck_size", i64, i)
    _sig(lib, "ggml_is_contiguous", C.c_bool, T)
    _sig(lib, "ggml_set_name", T, T, C.c_char_p)
    _sig(lib, "ggml_new_tensor_1d", T, CTX, i, i64)
    _sig(lib, "ggml_new_tensor_2d", T, CTX, i, i64, i64)
    _sig(lib, "ggml_new_tensor_3d", T, CTX, i, i64, i64, i64)
    _sig(lib, "ggml_new_tensor_4d", T, CTX, i, i64, i64, i64, i64)
    _sig(lib, "ggml_set_input", None, T)
    _sig(lib, "ggml_set_output", None, T)
    for name in ("ggml_add", "ggml_sub", "ggml_mul", "ggml_div", "ggml_mul_mat", "ggml_get_rows", "ggml_cpy"):
        _sig(lib, name, T, CTX, T, T)
    for name in ("ggml_silu", "ggml_gelu", "ggml_gelu_erf", "ggml_relu", "ggml_cont", "ggml_argmax",
                 "ggml_argmax_first", "ggml_transpose", "ggml_soft_max"):
        _sig(lib, name, T, CTX, T)
    _sig(lib, "ggml_scale", T, CTX, T, f)
    _sig(lib, "ggml_rms_norm", T, CTX, T, f)
    _sig(lib, "ggml_norm", T, CTX, T, f)
    _sig(lib, "ggml_mul_mat_set_prec", None, T, i)
    _sig(lib, "ggml_set_rows", T, CTX, T, T, T)
    _sig(lib, "ggml_soft_max_ext", T, CTX, T, T, f, f)
    _sig(lib, "ggml_flash_attn_ext", T, CTX, T, T, T, T, f, f, f)
    _sig(lib, "ggml_flash_attn_ext_set_prec", None, T, i)
    _sig(lib, "ggml_rope_ext", T, CTX, T, T, T, i, i, i, f, f, f, f, f, f)
    _sig(lib, "ggml_reshape_1d", T, CTX, T, i64)
    _sig(lib, "ggml_reshape_2d", T, CTX, T, i64, i64)
    _sig(lib, "ggml_reshape_3d", T, CTX, T, i64, i64, i64)
    _sig(lib, "ggml_reshape_4d", T, CTX, T, i64, i64, i64, i64)
    _sig(lib, "ggml_repeat", T, CTX, T, T)
    _sig(lib, "ggml_repeat_4d", T, CTX, T, i64, i64, i64, i64)
    _sig(lib, "ggml_view_1d", T, CTX, T, i64, sz)
    _sig(lib, "ggml_view_2d", T, CTX, T, i64, i64, sz, sz)
    _sig(lib, "ggml_view_3d", T, CTX, T, i64, i64, i64, sz, sz, sz)
    _sig(lib, "ggml_view_4d", T, CTX, T, i64, i64, i64, i64, sz, sz, sz, sz)
    _sig(lib, "ggml_permute", T, CTX, T, i, i, i, i)
    _sig(lib, "ggml_im2col", T, CTX, T, T, i, i, i, i, i, i, C.c_bool, i)
    _sig(lib, "ggml_conv_2d", T, CTX, T, T, i, i, i, i, i, i)
    for name in ("ggml_sin", "ggml_cos"):
        _sig(lib, name, T, CTX, T)
    _sig(lib, "ggml_concat", T, CTX, T, T, i)
    _sig(lib, "ggml_cast", T, CTX, T, i)
    _sig(lib, "ggml_new_graph_custom", C.c_void_p, CTX, sz, C.c_bool)
    _sig(lib, "ggml_build_forward_expand", None, C.c_void_p, T)
    _sig(lib, "ggml_graph_n_nodes", i, C.c_void_p)
    _sig(lib, "ggml_graph_node", T, C.c_void_p, i)
    _sig(lib, "ggml_quantize_chunk", sz, i, C.c_void_p, C.c_void_p, i64, i64, i64, C.c_void_p)
    _sig(lib, "ggml_fp16_to_fp32", f, C.c_uint16)
    _sig(lib, "ggml_fp32_to_fp16", C.c_uint16, f)
    _sig(lib, "ggml_backend_tensor_set", i, T, C.c_void_p, sz, sz)
    _sig(lib, "ggml_backend_tensor_get", i, T, C.c_void_p, sz, sz)
    _sig(lib, "ggml_backend_tensor_memset", i, T, C.c_uint8, sz, sz)
    _sig(lib, "ggml_backend_alloc_ctx_tensors_from_buft", C.c_void_p, CTX, C.c_void_p)
    _sig(lib, "ggml_backend_buffer_free", None, C.c_void_p)
    _sig(lib, "ggml_backend_buffer_set_usage", None, C.c_void_p, i)
    _sig(lib, "ggml_backend_buffer_clear", None, C.c_void_p, C.c_uint8)
    _sig(lib, "ggml_backend_buffer_get_size", sz, C.c_void_p)
    _sig(lib, "ggml_backend_buft_alloc_buffer", C.c_void_p, C.c_void_p, sz)
    _sig(lib, "ggml_backend_buft_name", C.c_char_p, C.c_void_p)
    _sig(lib, "ggml_backend_buft_get_alignment", sz, C.c_void_p)
    _sig(lib, "ggml_backend_name", C.c_char_p, C.c_void_p)
    _sig(lib, "ggml_backend_free", None, C.c_void_p)
    _sig(lib, "ggml_backend_get_default_buffer_type", C.c_void_p, C.c_void_p)
    _sig(lib, "ggml_backend_synchronize", None, C.c_void_p)
    _sig(lib, "ggml_backend_graph_compute", i, C.c_void_p, C.c_void_p)
    _sig(lib, "ggml_backend_graph_compute_with_abort", i, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
         C.POINTER(cancel_capability))
    _sig(lib, "ggml_backend_supports_op", C.c_bool, C.c_void_p, T)
    _sig(lib, "ggml_backend_dev_name", C.c_char_p, C.c_void_p)
    _sig(lib, "ggml_backend_dev_description", C.c_char_p, C.c_void_p)
    _sig(lib, "ggml_backend_dev_type", i, C.c_void_p)
    _sig(lib, "ggml_backend_dev_init", C.c_void_p, C.c_void_p, C.c_char_p)
    _sig(lib, "ggml_backend_dev_buffer_type", C.c_void_p, C.c_void_p)
    _sig(lib, "ggml_backend_dev_supports_op", C.c_bool, C.c_void_p, T)
    _sig(lib, "ggml_backend_reg_name", C.c_char_p, C.c_void_p)
    _sig(lib, "ggml_backend_reg_dev_count", sz, C.c_void_p)
    _sig(lib, "ggml_backend_reg_dev_get", C.c_void_p, C.c_void_p, sz)
    _sig(lib, "ggml_backend_reg_get_proc_address", C.c_void_p, C.c_void_p, C.c_char_p)
    _sig(lib, "ggml_backend_load_verified_v3_utf8", C.c_void_p, C.c_char_p, C.c_void_p, sz, C.c_char_p,
         C.c_char_p, C.c_char_p, C.c_char_p)
    _sig(lib, "ggml_backend_probe_verified_v3_utf8", C.c_bool, C.c_char_p, C.c_void_p, sz, C.c_char_p,
         C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, sz)
    _sig(lib, "ggml_backend_host_abi_fingerprint", C.c_char_p)
    _sig(lib, "ggml_gallocr_new", C.c_void_p, C.c_void_p)
    _sig(lib, "ggml_gallocr_free", None, C.c_void_p)
    _sig(lib, "ggml_gallocr_alloc_graph", C.c_bool, C.c_void_p, C.c_void_p)
    _sig(lib, "ggml_gallocr_get_buffer_size", sz, C.c_void_p, i)
    _sig(lib, "ggml_backend_cpu_buffer_type", C.c_void_p)
    _sig(lib, "oa_synth_normal", None, C.c_uint64, C.c_uint64, i64, i64, f, f, C.c_void_p)
    _sig(lib, "oa_synth_uniform_i32", None, C.c_uint64, C.c_uint64, i64, C.c_int32, C.c_void_p)
    _base = lib
    return lib


def tensor(ptr) -> ggml_tensor:
    return ggml_tensor.from_address(ptr)


# ----------------------------------------------------------------- plugin --

_plugin = None


class Plugin:
    """The MI355X backend plugin, loaded the way the OpenASR host loads a HIP
    pack: verified load with ABI fingerprint, provider "hip" and device
    target "gfx950", then device 0 initialised as a backend."""

    def __init__(self, path: Path = PLUGIN_PATH, device_target: str = "gfx950"):
        lib = base()
        if not Path(path).exists():
            raise RuntimeError(f"{path} is missing: run `python -m openasr_amd.build` first")
        fp = lib.ggml_backend_host_abi_fingerprint()
        self.reg = lib.ggml_backend_load_verified_v3_utf8(str(path).encode(), None, 0, fp, b"hip",
                                                          device_target.encode(), b"")
        if not self.reg:
            raise RuntimeError("MI355X plugin failed verified loading (no gfx950 device, or ABI mismatch)")
        if lib.ggml_backend_reg_dev_count(self.reg) < 1:
            raise RuntimeError("MI355X plugin reports no devices")
        self.dev = lib.ggml_backend_reg_dev_get(self.reg, 0)
        self.backend = lib.ggml_backend_dev_init(self.dev, None)
        if not self.backend:
            raise RuntimeError("MI355X backend init failed")
        self.buft = lib.ggml_backend_get_default_buffer_type(self.backend)
        self.cdll = C.CDLL(str(path))  # same mapping as the verified load; used for direct helpers
        self.cdll.ggml_backend_mi355x_profile_graph.restype = C.c_int
        self.cdll.ggml_backend_mi355x_profile_graph.argtypes = [C.c_void_p, C.c_void_p, C.c_int,
                                                               C.POINTER(C.c_float), C.c_int, C.c_char_p, C.c_int]
        self.cdll.ggml_backend_mi355x_set_hip_graphs.restype = None
        self.cdll.ggml_backend_mi355x_set_hip_graphs.argtypes = [C.c_void_p, C.c_bool]

    @property
    def name(self) -> str:
        return base().ggml_backend_name(self.backend).decode()

    def profile(self, graph, iters: int, max_steps: int = 4096):
        ms = (C.c_float * max_steps)()
        labels = C.create_string_buffer(max_steps * 96)
        n = self.cdll.ggml_backend_mi355x_profile_graph(self.backend, graph, iters, ms, max_steps, labels, 96)
        if n < 0:
            raise RuntimeError("profile_graph failed")
        out = []
        for k in range(min(n, max_steps)):
            lab = labels.raw[k * 96:(k + 1) * 96].split(b"\0", 1)[0].decode()
            out.append((lab, float(ms[k])))
        return out


def plugin() -> Plugin:
    global _plugin
    if _plugin is None:
        _plugin = Plugin()
    return _plugin


# --------------------------------------------------------------- graphs ----

NP_OF = {F32: np.float32, F16: np.uint16, I32: np.int32, I64: np.int64}


class Graph:
    """A ggml context + graph built through the C ABI and allocated on one
    backend buffer type, with numpy transfers for inputs and outputs."""

    def __init__(self, n_tensors: int = 4096, graph_size: int = 8192):
        lib = base()
        mem = lib.ggml_tensor_overhead() * n_tensors + lib.ggml_graph_overhead_custom(graph_size, False) + (1 << 16)
        self.ctx = lib.ggml_init(ggml_init_params(mem, None, True))
        self.wctx = lib.ggml_init(ggml_init_params(lib.ggml_tensor_overhead() * n_tensors, None, True))
        self.graph_size = graph_size
        self.gf = None
        self.galloc = None
        self.wbuf = None
        self.lib = lib

    # tensors
    def new(self, typ, *ne, name=None, weight=False):
        ctx = self.wctx if weight else self.ctx
        fn = {1: self.lib.ggml_new_tensor_1d, 2: self.lib.ggml_new_tensor_2d, 3: self.lib.ggml_new_tensor_3d,
              4: self.lib.ggml_new_tensor_4d}[len(ne)]
        t = fn(ctx, typ, *ne)
        if not t:
            raise RuntimeError("ggml_new_tensor failed")
        if name:
            self.lib.ggml_set_name(t, name.encode())
        if not weight:
            self.lib.ggml_set_input(t)
        return t

    def build(self, *outputs):
        self.gf = self.lib.ggml_new_graph_custom(self.ctx, self.graph_size, False)
        for o in outputs:
            self.lib.ggml_set_output(o)
            self.lib.ggml_build_forward_expand(self.gf, o)
        return self.gf

    def allocate(self, buft):
        """Weights context -> its own WEIGHTS buffer; graph tensors -> gallocr."""
        lib = self.lib
        self.wbuf = lib.ggml_backend_alloc_ctx_tensors_from_buft(self.wctx, buft)
        if self.wbuf:
            lib.ggml_backend_buffer_set_usage(self.wbuf, BUFFER_USAGE_WEIGHTS)
        self.galloc = lib.ggml_gallocr_new(buft)
        if not lib.ggml_gallocr_alloc_graph(self.galloc, self.gf):
            raise RuntimeError("graph allocation failed")

    def set(self, t, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        n = self.lib.ggml_nbytes(t)
        if arr.nbytes != n:
            raise ValueError(f"set: {arr.nbytes} bytes for a {n}-byte tensor")
        if self.lib.ggml_backend_tensor_set(t, arr.ctypes.data, 0, n) != 0:
            raise RuntimeError("ggml_backend_tensor_set failed")

    def get(self, t, dtype=None, shape=None) -> np.ndarray:
        tt = tensor(t)
        n = self.lib.ggml_nbytes(t)
        dtype = dtype or NP_OF.get(tt.type, np.uint8)
        out = np.empty(n // np.dtype(dtype).itemsize, dtype=dtype)
        if self.lib.ggml_backend_tensor_get(t, out.ctypes.data, 0, n) != 0:
            raise RuntimeError("ggml_backend_tensor_get failed")
        if shape is None and tt.type in NP_OF:
            shape = tuple(int(tt.ne[i]) for i in range(3, -1, -1))
        return out.reshape(shape) if shape is not None else out

    def compute(self, backend) -> int:
        return self.lib.ggml_backend_graph_compute(backend, self.gf)

    def free(self):
        lib = self.lib
        if self.galloc:
            lib.ggml_gallocr_free(self.galloc)
            self.galloc = None
        if self.wbuf:
            lib.ggml_backend_buffer_free(self.wbuf)
            self.wbuf = None
        if self.ctx:
            lib.ggml_free(self.ctx)
            self.ctx = None
        if self.wctx:
            lib.ggml_free(self.wctx)
            self.wctx = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------ memory ABI v1 -----
# ctypes mirror of include/ggml_backend_memory.h (the host's #[repr(C)]
# structs, crates/openasr-core/src/ggml_runtime/ffi.rs:144-332) and a thin
# wrapper that drives it the way backend_memory.rs:140-330 does: resolve the
# registry proc, check size / version / required entries, and call every
# list-returning function twice (count, then fill).

MEM_DOMAIN_DEVICE_LOCAL = 1
MEM_REQUEST_BUFFER, MEM_REQUEST_HOST_IMPORT, MEM_REQUEST_GRAPH_PRIVATE, MEM_REQUEST_TRANSFER = 1, 2, 3, 4
MEM_QUOTE_PROVISIONAL = 1 << 0
MEM_QUOTE_OPAQUE_DRIVER_COSTS = 1 << 2
MEM_STATS_BUDGET_UNAVAILABLE = 1 << 0
MEM_CLAIM_EXACT, MEM_CLAIM_CONSERVATIVE_UPPER, MEM_CLAIM_PROVISIONAL = 1 << 0, 1 << 1, 1 << 6
MEM_HEALTHY, MEM_DEGRADED, MEM_QUARANTINED, MEM_DEVICE_LOST = 0, 1, 2, 3


class mem_domain_id(C.Structure):
    _fields_ = [("physical_device_uuid", C.c_uint8 * 16), ("heap_index", C.c_uint32), ("kind", C.c_uint32)]


class mem_domain(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("flags", C.c_uint32), ("id", mem_domain_id), ("name", C.c_char * 48)]


class mem_request(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("kind", C.c_uint32), ("flags", C.c_uint32), ("usage", C.c_uint32),
                ("request_id", C.c_uint64), ("backend", C.c_void_p), ("peer_backend", C.c_void_p),
                ("buft", C.c_void_p), ("graph", C.c_void_p), ("host_ptr", C.c_void_p),
                ("requested_bytes", C.c_uint64), ("currently_allocated_bytes", C.c_uint64),
                ("max_tensor_bytes", C.c_uint64)]


class mem_claim(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("flags", C.c_uint32), ("request_id", C.c_uint64),
                ("domain", mem_domain_id), ("payload_requested_bytes", C.c_uint64),
                ("committed_before_bytes", C.c_uint64), ("committed_after_upper_bytes", C.c_uint64),
                ("commit_peak_extra_upper_bytes", C.c_uint64), ("resident_after_upper_bytes", C.c_uint64),
                ("retained_after_use_upper_bytes", C.c_uint64), ("releasable_after_use_upper_bytes", C.c_uint64)]


class mem_quote(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("flags", C.c_uint32), ("residual_flags", C.c_uint32),
                ("residual_request_count", C.c_uint32), ("provisional_requested_upper_bytes", C.c_uint64),
                ("stats_generation", C.c_uint64), ("quote_token", C.c_uint64), ("request_fingerprint", C.c_uint64)]


class mem_stats(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("flags", C.c_uint32), ("domain", mem_domain_id),
                ("generation", C.c_uint64), ("timestamp_monotonic_ns", C.c_uint64), ("total_bytes", C.c_uint64),
                ("budget_bytes", C.c_uint64), ("device_used_bytes", C.c_uint64), ("device_free_bytes", C.c_uint64),
                ("backend_owned_live_bytes", C.c_uint64), ("backend_owned_cached_bytes", C.c_uint64),
                ("backend_owned_workspace_bytes", C.c_uint64), ("backend_owned_high_water_bytes", C.c_uint64),
                ("allocation_count", C.c_uint64), ("allocation_failure_count", C.c_uint64),
                ("health", C.c_uint32), ("last_ggml_status", C.c_int32), ("last_native_error", C.c_int64),
                ("quarantine_generation", C.c_uint64)]


class mem_quarantine(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("flags", C.c_uint32), ("reason", C.c_uint32),
                ("ggml_status", C.c_int32), ("native_error", C.c_int64), ("message", C.c_char * 96)]


_U32P = C.POINTER(C.c_uint32)
MEM_GET_DOMAINS = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(mem_domain), _U32P)
MEM_QUOTE = C.CFUNCTYPE(C.c_int, C.POINTER(mem_request), C.c_uint32, C.POINTER(mem_quote), C.POINTER(mem_claim),
                        _U32P)
MEM_RESERVE = C.CFUNCTYPE(C.c_int, C.POINTER(mem_request), C.c_uint32, C.POINTER(mem_quote), C.POINTER(mem_claim),
                          _U32P)
MEM_GET_STATS = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.POINTER(mem_stats), _U32P)
MEM_TRIM = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint64)
MEM_QUARANTINE = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(mem_quarantine))


class mem_api(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("capabilities", C.c_uint64),
                ("get_domains", MEM_GET_DOMAINS), ("quote", MEM_QUOTE), ("reserve_private", MEM_RESERVE),
                ("get_stats", MEM_GET_STATS), ("trim", MEM_TRIM), ("quarantine", MEM_QUARANTINE)]


MEM_API_GET = C.CFUNCTYPE(C.POINTER(mem_api))


class MemoryStatusError(RuntimeError):
    def __init__(self, operation: str, status: int):
        super().__init__(f"memory ABI {operation} returned ggml status {status}")
        self.operation, self.status = operation, status


def _check(operation: str, status: int) -> None:
    if status != 0:
        raise MemoryStatusError(operation, status)


def _array(cls, n: int):
    arr = (cls * max(n, 1))()
    for x in arr:
        x.struct_size = C.sizeof(cls)
    return arr


class MemoryApi:
    """The v1 table of one backend, resolved through its registry."""

    def __init__(self, reg, device, backend):
        proc = base().ggml_backend_reg_get_proc_address(reg, b"ggml_backend_memory_get_api_v1")
        if not proc:
            raise RuntimeError("memory ABI unavailable")
        api = MEM_API_GET(proc)()
        if not api:
            raise RuntimeError("memory ABI unavailable")
        self.raw = api.contents
        if (self.raw.struct_size < C.sizeof(mem_api) or self.raw.abi_version != 1
                or not all((self.raw.get_domains, self.raw.quote, self.raw.reserve_private, self.raw.get_stats))):
            raise RuntimeError("memory ABI incompatible")
        self.device, self.backend = device, backend

    def domains(self):
        n = C.c_uint32(0)
        _check("domains/count", self.raw.get_domains(self.device, None, C.byref(n)))
        arr, cap = _array(mem_domain, n.value), C.c_uint32(n.value)
        _check("domains", self.raw.get_domains(self.device, arr, C.byref(cap)))
        return list(arr)[:cap.value]

    def quote(self, requests):
        reqs = (mem_request * max(len(requests), 1))(*requests)
        q = mem_quote(struct_size=C.sizeof(mem_quote))
        n = C.c_uint32(0)
        _check("quote/count", self.raw.quote(reqs, len(requests), C.byref(q), None, C.byref(n)))
        claims, cap = _array(mem_claim, n.value), C.c_uint32(n.value)
        _check("quote", self.raw.quote(reqs, len(requests), C.byref(q), claims, C.byref(cap)))
        return q, list(claims)[:cap.value]

    def reserve_private(self, requests, q):
        reqs = (mem_request * max(len(requests), 1))(*requests)
        n = C.c_uint32(0)
        _check("reserve_private/count", self.raw.reserve_private(reqs, len(requests), C.byref(q), None, C.byref(n)))
        claims, cap = _array(mem_claim, n.value), C.c_uint32(n.value)
        _check("reserve_private", self.raw.reserve_private(reqs, len(requests), C.byref(q), claims, C.byref(cap)))
        return list(claims)[:cap.value]

    def stats(self):
        n = C.c_uint32(0)
        _check("stats/count", self.raw.get_stats(self.device, self.backend, None, C.byref(n)))
        arr, cap = _array(mem_stats, n.value), C.c_uint32(n.value)
        _check("stats", self.raw.get_stats(self.device, self.backend, arr, C.byref(cap)))
        return list(arr)[:cap.value]

    def trim(self, flags: int = 0) -> None:
        _check("trim", self.raw.trim(self.backend, flags))

    def quarantine(self, reason: int, status: int, message: bytes) -> None:
        q = mem_quarantine(struct_size=C.sizeof(mem_quarantine), reason=reason, ggml_status=status, message=message)
        _check("quarantine", self.raw.quarantine(self.backend, C.byref(q)))


def mem_request_of(kind: int, backend=None, buft=None, graph=None, requested: int = 0, current: int = 0,
                   request_id: int = 0, usage: int = 0) -> mem_request:
    return mem_request(struct_size=C.sizeof(mem_request), kind=kind, usage=usage, request_id=request_id,
                       backend=backend, buft=buft, graph=graph, requested_bytes=requested,
                       currently_allocated_bytes=current)


# --------------------------------------------------------------- helpers ---

def synth_normal(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    base().oa_synth_normal(seed, stream, first, n, mean, std, out.ctypes.data)
    return out


def quantize(typ: int, x: np.ndarray) -> np.ndarray:
    """ggml_quantize_chunk over a [rows, k] f32 matrix -> raw ggml bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    lib = base()
    out = np.empty(rows * lib.ggml_row_size(typ, k), dtype=np.uint8)
    lib.ggml_quantize_chunk(typ, x.ctypes.data, out.ctypes.data, 0, rows, k, None)
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)
