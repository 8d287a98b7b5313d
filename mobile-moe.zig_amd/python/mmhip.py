"""ctypes binding of libmmhip (include/mmhip.h) plus seeded synthetic-weight
generators for the GGUF block formats on this path.

The binding is thin on purpose: every call goes straight to the C ABI, and a
missing or unloadable libmmhip raises instead of degrading to anything else.

Block formats (src/dequant.zig:305-311, 372-377 in the reference):
  Q8_0     34 B  = f16 d, int8 qs[32]
  IQ2_XXS  66 B  = f16 d, u16 qs[32]  (256 weights)
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(_HERE)
# MMHIP_LIBRARY selects another build of the same library (e.g. the host
# sanitizer build, lib/libmmhip_san.so).
LIB_PATH = os.environ.get("MMHIP_LIBRARY") or os.path.join(PKG_DIR, "lib", "libmmhip.so")

F32, F16, Q8_0, IQ2_XXS = 0, 1, 8, 16
BLOCK_SIZE = {F32: 1, F16: 1, Q8_0: 32, IQ2_XXS: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, IQ2_XXS: 66}

OK, ERR_UNAVAILABLE, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_NOMEM = 0, -1, -2, -3, -4, -5

_c_void_p = ctypes.c_void_p
_u32, _u64, _i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32
_fp = ctypes.POINTER(ctypes.c_float)


class MoeWeights(ctypes.Structure):
    _fields_ = [
        ("hidden_size", _u32), ("moe_intermediate", _u32), ("shared_intermediate", _u32),
        ("n_routed_experts", _u32), ("expert_type", _u32), ("shared_type", _u32),
        ("router_type", _u32), ("routed_scaling_factor", ctypes.c_float),
        ("router_host", _c_void_p), ("expert_gate_host", _c_void_p), ("expert_up_host", _c_void_p),
        ("expert_down_host", _c_void_p), ("shared_gate_host", _c_void_p),
        ("shared_up_host", _c_void_p), ("shared_down_host", _c_void_p),
    ]


class RouteParams(ctypes.Structure):
    _fields_ = [("throttle_level", _i32), ("active_expert_limit", _u32),
                ("deferral_bias_host", _fp)]


class GemvGroup(ctypes.Structure):
    _fields_ = [("w", _c_void_p), ("first", _u64), ("n_mats", _u64), ("x_dev", _c_void_p), ("x_stride", _u64),
                ("y_dev", _c_void_p), ("y_stride", _u64)]


class Shape(ctypes.Structure):
    _fields_ = [("m", _u32), ("n", _u32), ("k", _u32), ("dim", _u32)]


class OpSchedule(ctypes.Structure):
    _fields_ = [("op", _u32), ("backend", _u32), ("precision", _u32), ("sync_after", _u32),
                ("shape", Shape), ("estimated_us", _u64)]


class PlanHParams(ctypes.Structure):
    _fields_ = [("hidden_size", _u32), ("intermediate_size", _u32), ("num_heads", _u32),
                ("head_dim", _u32), ("seq_len_hint", _u32), ("leading_dense_layers", _u32),
                ("n_routed_experts", _u32), ("weight_precision", _u32)]


class PerfEntry(ctypes.Structure):
    _fields_ = [("op", _u32), ("precision", _u32), ("shape", Shape), ("cpu_us", _u64), ("gpu_us", _u64)]


# name -> (restype, argtypes)
class GgufInfo(ctypes.Structure):
    _fields_ = [("version", _u32), ("tensor_count", _u64), ("metadata_count", _u64), ("n_tensors", _u64),
                ("n_keys", _u64), ("alignment", _u64), ("data_offset", _u64), ("file_size", _u64)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", _u32), ("dims", _u64 * 4), ("type", _u32), ("offset", _u64),
                ("n_elements", _u64), ("n_bytes", _u64), ("data", _c_void_p)]


_SIGS = {
    "mmhip_last_error": (ctypes.c_char_p, []),
    "mmhip_is_available": (ctypes.c_int, []),
    "mmhip_device_count": (ctypes.c_int, []),
    "mmhip_version": (ctypes.c_char_p, []),
    "mmhip_init": (ctypes.c_int, [ctypes.POINTER(_c_void_p), ctypes.c_int]),
    "mmhip_destroy": (None, [_c_void_p]),
    "mmhip_synchronize": (ctypes.c_int, [_c_void_p]),
    "mmhip_stream": (_c_void_p, [_c_void_p]),
    "mmhip_num_cu": (ctypes.c_int, [_c_void_p]),
    "mmhip_profile_enable": (ctypes.c_int, [_c_void_p, ctypes.c_int]),
    "mmhip_profile_read": (ctypes.c_int, [_c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(_u64)]),
    "mmhip_malloc": (ctypes.c_int, [_c_void_p, ctypes.POINTER(_c_void_p), ctypes.c_size_t]),
    "mmhip_free": (ctypes.c_int, [_c_void_p, _c_void_p]),
    "mmhip_memcpy_h2d": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_size_t]),
    "mmhip_memcpy_d2h": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_size_t]),
    "mmhip_memset_dev": (ctypes.c_int, [_c_void_p, _c_void_p, ctypes.c_int, ctypes.c_size_t]),
    "mmhip_weight_upload": (ctypes.c_int, [_c_void_p, _c_void_p, _u32, _u64, _u64, _u64,
                                           ctypes.POINTER(_c_void_p)]),
    "mmhip_weight_from_device": (ctypes.c_int, [_c_void_p, _c_void_p, _u32, _u64, _u64, _u64,
                                                ctypes.POINTER(_c_void_p)]),
    "mmhip_weight_free": (None, [_c_void_p, _c_void_p]),
    "mmhip_weight_device_bytes": (_u64, [_c_void_p]),
    "mmhip_mat_vec_mul": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u32, _c_void_p, _u64, _u64]),
    "mmhip_batch_mat_mul": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u32, _c_void_p, _u64, _u64, _u64]),
    "mmhip_dequantize": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u32, _u64]),
    "mmhip_forget": (ctypes.c_int, [_c_void_p, _c_void_p]),
    "mmhip_dequantize_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u32, _u64]),
    "mmhip_quantize_q8_0": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u64]),
    "mmhip_sample_greedy": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u64]),
    "mmhip_argmax_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u64]),
    "mmhip_quantize_q8_0_rows_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _u64, _u64, _u32]),
    "mmhip_dequantize_q8_0_rows_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _u64, _c_void_p, _u64, _u32]),
    "mmhip_gemv_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _u64, _c_void_p, _c_void_p]),
    "mmhip_gemv_grouped_dev": (ctypes.c_int, [_c_void_p, ctypes.POINTER(GemvGroup), _u32]),
    "mmhip_gemv_batched_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _u64, _u64, _c_void_p, _u64,
                                              _c_void_p, _u64]),
    "mmhip_qmm_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _u64, _c_void_p, _c_void_p, _u64, ctypes.c_int]),
    "mmhip_qmm_dev_noalloc": (ctypes.c_int, [_c_void_p, _c_void_p, _u64, _c_void_p, _c_void_p, _u64, ctypes.c_int]),
    "mmhip_moe_layer_create": (ctypes.c_int, [_c_void_p, ctypes.POINTER(MoeWeights), ctypes.POINTER(_c_void_p)]),
    "mmhip_moe_layer_destroy": (None, [_c_void_p, _c_void_p]),
    "mmhip_moe_ffn": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _u32,
                                     ctypes.POINTER(RouteParams), _c_void_p, _c_void_p]),
    "mmhip_moe_ffn_dev": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _u32,
                                         ctypes.POINTER(RouteParams), _c_void_p, _c_void_p]),
    "mmhip_moe_expert_counts": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p]),
    "mmhip_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_c_void_p)]),
    "mmhip_gguf_close": (None, [_c_void_p]),
    "mmhip_gguf_get_info": (ctypes.c_int, [_c_void_p, ctypes.POINTER(GgufInfo)]),
    "mmhip_gguf_tensor_at": (ctypes.c_int, [_c_void_p, _u64, ctypes.POINTER(GgufTensor)]),
    "mmhip_gguf_find_tensor": (ctypes.c_int, [_c_void_p, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]),
    "mmhip_gguf_key_at": (ctypes.c_char_p, [_c_void_p, _u64]),
    "mmhip_gguf_meta_type": (ctypes.c_int, [_c_void_p, ctypes.c_char_p]),
    "mmhip_gguf_meta_int": (ctypes.c_int, [_c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "mmhip_gguf_meta_float": (ctypes.c_int, [_c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "mmhip_gguf_meta_string": (ctypes.c_int, [_c_void_p, ctypes.c_char_p, ctypes.POINTER(_c_void_p),
                                              ctypes.POINTER(_u64)]),
    "mmhip_gguf_meta_array": (ctypes.c_int, [_c_void_p, ctypes.c_char_p, ctypes.POINTER(_u32), ctypes.POINTER(_u64),
                                             ctypes.POINTER(_c_void_p), ctypes.POINTER(_u64)]),
    "mmhip_weight_upload_gguf": (ctypes.c_int, [_c_void_p, _c_void_p, ctypes.c_char_p, ctypes.POINTER(_c_void_p)]),
    "mmhip_weight_upload_gguf_rows": (ctypes.c_int, [_c_void_p, _c_void_p, ctypes.POINTER(ctypes.c_char_p), _u32,
                                                     ctypes.POINTER(_c_void_p)]),
    "mmhip_moe_layer_create_gguf": (ctypes.c_int, [_c_void_p, _c_void_p, _u32, ctypes.POINTER(_c_void_p)]),
    "mmhip_plan_layer": (ctypes.c_int, [_u32, ctypes.POINTER(PlanHParams), ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.POINTER(PerfEntry), ctypes.c_size_t,
                                        ctypes.POINTER(OpSchedule), ctypes.c_size_t,
                                        ctypes.POINTER(ctypes.c_size_t)]),
    "mmhip_plan_critical_path_us": (_u64, [ctypes.POINTER(OpSchedule), ctypes.c_size_t]),
    "mmhip_plan_device_mask": (_u32, [ctypes.POINTER(OpSchedule), ctypes.c_size_t]),
}

_lib: Optional[ctypes.CDLL] = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libmmhip.so (raises if it is missing: there is no other path)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"libmmhip not built: {path} is missing (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class MmhipError(RuntimeError):
    def __init__(self, what: str, code: int, msg: Optional[str] = None):
        if msg is None:
            msg = load_library().mmhip_last_error().decode(errors="replace")
        super().__init__(f"{what} failed ({code}): {msg}")
        self.code = code


def _enc(s: str) -> bytes:
    """GGUF names and keys are byte strings; non-UTF-8 bytes round-trip."""
    return s.encode("utf-8", "surrogateescape")


def _dec(b: bytes) -> str:
    return b.decode("utf-8", "surrogateescape")


def check(rc: int, what: str) -> int:
    if rc < 0:
        raise MmhipError(what, rc)
    return rc


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class DeviceArray:
    """Device buffer owned through the library's allocator."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = _c_void_p()
        check(ctx.lib.mmhip_malloc(ctx.handle, ctypes.byref(p), self.nbytes), "mmhip_malloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, ctx: "Context", arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(ctx, arr.nbytes)
        check(ctx.lib.mmhip_memcpy_h2d(ctx.handle, d.ptr, _ptr(arr), arr.nbytes), "mmhip_memcpy_h2d")
        return d

    def to_numpy(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        check(self.ctx.lib.mmhip_memcpy_d2h(self.ctx.handle, _ptr(out), self.ptr, out.nbytes), "mmhip_memcpy_d2h")
        return out

    def zero(self):
        check(self.ctx.lib.mmhip_memset_dev(self.ctx.handle, self.ptr, 0, self.nbytes), "mmhip_memset_dev")

    def free(self):
        if self.ptr:
            self.ctx.lib.mmhip_free(self.ctx.handle, self.ptr)
            self.ptr = None


class Weight:
    def __init__(self, ctx: "Context", handle: int, ggml_type: int, rows: int, cols: int, count: int):
        self.ctx, self.handle = ctx, handle
        self.type, self.rows, self.cols, self.count = ggml_type, rows, cols, count

    @property
    def device_bytes(self) -> int:
        return int(self.ctx.lib.mmhip_weight_device_bytes(self.handle))

    def free(self):
        if self.handle:
            self.ctx.lib.mmhip_weight_free(self.ctx.handle, self.handle)
            self.handle = None


class Context:
    """One device context (the reference's OpenCLBackend object)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _c_void_p()
        check(self.lib.mmhip_init(ctypes.byref(h), device), "mmhip_init")
        self.handle = h.value

    def close(self):
        if self.handle:
            self.lib.mmhip_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- plumbing --
    @property
    def stream(self) -> int:
        return self.lib.mmhip_stream(self.handle)

    @property
    def num_cu(self) -> int:
        return self.lib.mmhip_num_cu(self.handle)

    def synchronize(self):
        check(self.lib.mmhip_synchronize(self.handle), "mmhip_synchronize")

    def profile(self, enable: bool):
        check(self.lib.mmhip_profile_enable(self.handle, 1 if enable else 0), "mmhip_profile_enable")

    def profile_read(self, family: str):
        ms = ctypes.c_double()
        n = _u64()
        check(self.lib.mmhip_profile_read(self.handle, family.encode(), ctypes.byref(ms), ctypes.byref(n)),
              "mmhip_profile_read")
        return ms.value, n.value

    # -- weights --
    def upload(self, raw: np.ndarray, ggml_type: int, rows: int, cols: int, count: int = 1) -> Weight:
        raw = np.ascontiguousarray(raw)
        h = _c_void_p()
        check(self.lib.mmhip_weight_upload(self.handle, _ptr(raw), ggml_type, rows, cols, count, ctypes.byref(h)),
              "mmhip_weight_upload")
        return Weight(self, h.value, ggml_type, rows, cols, count)

    def upload_gguf(self, g: "Gguf", name: str) -> Weight:
        """One-time upload of a GGUF tensor (rows = dims[1], cols = dims[0], count = dims[2])."""
        t = g.tensor(name)
        if t is None:
            raise KeyError(name)
        h = _c_void_p()
        check(self.lib.mmhip_weight_upload_gguf(self.handle, g.handle, _enc(name), ctypes.byref(h)),
              "mmhip_weight_upload_gguf")
        d = t["dims"]
        return Weight(self, h.value, t["type"], d[1], d[0], d[2])

    def upload_gguf_rows(self, g: "Gguf", names) -> Weight:
        """One weight of the named matrices' rows stacked in order (e.g. q_a then kv_a)."""
        ts = [g.tensor(n) for n in names]
        if any(t is None for t in ts):
            raise KeyError([n for n, t in zip(names, ts) if t is None])
        arr = (ctypes.c_char_p * len(names))(*[_enc(n) for n in names])
        h = _c_void_p()
        check(self.lib.mmhip_weight_upload_gguf_rows(self.handle, g.handle, arr, len(names), ctypes.byref(h)),
              "mmhip_weight_upload_gguf_rows")
        return Weight(self, h.value, ts[0]["type"], sum(t["dims"][1] for t in ts), ts[0]["dims"][0], 1)

    def weight_from_device(self, raw: DeviceArray, ggml_type: int, rows: int, cols: int, count: int = 1) -> Weight:
        h = _c_void_p()
        check(self.lib.mmhip_weight_from_device(self.handle, raw.ptr, ggml_type, rows, cols, count,
                                                ctypes.byref(h)), "mmhip_weight_from_device")
        return Weight(self, h.value, ggml_type, rows, cols, count)

    # -- engine seam (host slices) --
    def mat_vec_mul(self, raw: np.ndarray, ggml_type: int, x: np.ndarray, out_dim: int, in_dim: int,
                    resident: bool = False) -> np.ndarray:
        """matVecMulUnified. The C ABI keeps the upload resident keyed by the
        host pointer; resident=False drops it after the call, since a later
        numpy array may reuse the same address."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(out_dim, dtype=np.float32)
        try:
            check(self.lib.mmhip_mat_vec_mul(self.handle, _ptr(out), _ptr(raw), ggml_type, _ptr(x), out_dim,
                                             in_dim), "mmhip_mat_vec_mul")
        finally:
            if not resident:
                self.forget(raw)
        return out

    def batch_mat_mul(self, raw: np.ndarray, ggml_type: int, xin: np.ndarray, out_dim: int, batch: int,
                      in_dim: int, resident: bool = False) -> np.ndarray:
        """batchMatMulUnified: out [batch][out_dim]."""
        xin = np.ascontiguousarray(xin, dtype=np.float32)
        out = np.empty((batch, out_dim), dtype=np.float32)
        try:
            check(self.lib.mmhip_batch_mat_mul(self.handle, _ptr(out), _ptr(raw), ggml_type, _ptr(xin), out_dim,
                                               batch, in_dim), "mmhip_batch_mat_mul")
        finally:
            if not resident:
                self.forget(raw)
        return out

    def dequantize(self, raw: np.ndarray, ggml_type: int, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        check(self.lib.mmhip_dequantize(self.handle, _ptr(out), _ptr(raw), ggml_type, n), "mmhip_dequantize")
        return out

    def quantize_q8_0(self, x: np.ndarray) -> np.ndarray:
        """quantizeQ8_0 (dequant.zig:98-130) on the device: raw 34-byte blocks."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.empty(((x.size + 31) // 32) * 34, dtype=np.uint8)
        check(self.lib.mmhip_quantize_q8_0(self.handle, _ptr(out), _ptr(x), x.size), "mmhip_quantize_q8_0")
        return out

    def sample_greedy(self, logits: np.ndarray) -> int:
        """sampleGreedy (inference.zig:376-386) on the device."""
        logits = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
        out = np.zeros(1, dtype=np.uint32)
        check(self.lib.mmhip_sample_greedy(self.handle, _ptr(out), _ptr(logits), logits.size), "mmhip_sample_greedy")
        return int(out[0])

    def argmax_dev(self, out: "DeviceArray", logits: "DeviceArray", n: int, out_offset: int = 0):
        check(self.lib.mmhip_argmax_dev(self.handle, out.ptr + out_offset, logits.ptr, n), "mmhip_argmax_dev")

    def forget(self, raw: np.ndarray):
        check(self.lib.mmhip_forget(self.handle, _ptr(raw)), "mmhip_forget")

    # -- device twins --
    def gemv_batched_dev(self, w: Weight, first: int, n: int, x: DeviceArray, x_stride: int, y: DeviceArray,
                         y_stride: int):
        check(self.lib.mmhip_gemv_batched_dev(self.handle, w.handle, first, n, x.ptr, x_stride, y.ptr, y_stride),
              "mmhip_gemv_batched_dev")

    def gemv_groups(self, groups) -> ctypes.Array:
        """groups: (weight, first, n_mats, x, x_stride, y, y_stride) tuples ->
        the mmhip_gemv_group array mmhip_gemv_grouped_dev takes (built once,
        reusable)."""
        arr = (GemvGroup * len(groups))()
        for i, (w, first, n, x, xs, y, ys) in enumerate(groups):
            arr[i] = GemvGroup(w.handle, first, n, x.ptr, xs, y.ptr, ys)
        return arr

    def gemv_grouped_dev(self, groups):
        """mmhip_gemv_grouped_dev: several GEMV groups (tuples as gemv_groups,
        or its array) in one launch."""
        arr = groups if isinstance(groups, ctypes.Array) else self.gemv_groups(groups)
        check(self.lib.mmhip_gemv_grouped_dev(self.handle, arr, len(arr)), "mmhip_gemv_grouped_dev")

    def qmm_dev(self, w: Weight, mat: int, x: DeviceArray, y: DeviceArray, batch: int, out_layout: int = 0):
        check(self.lib.mmhip_qmm_dev(self.handle, w.handle, mat, x.ptr, y.ptr, batch, out_layout), "mmhip_qmm_dev")

    def qmm_dev_noalloc(self, w: Weight, mat: int, x: DeviceArray, y: DeviceArray, batch: int, out_layout: int = 0):
        """mmhip_qmm_dev_noalloc: the same product with the library's fixed
        per-device scratch; allocates nothing."""
        check(self.lib.mmhip_qmm_dev_noalloc(self.handle, w.handle, mat, x.ptr, y.ptr, batch, out_layout),
              "mmhip_qmm_dev_noalloc")

    def dequantize_dev(self, out: DeviceArray, raw: DeviceArray, ggml_type: int, n: int):
        check(self.lib.mmhip_dequantize_dev(self.handle, out.ptr, raw.ptr, ggml_type, n), "mmhip_dequantize_dev")

    def quantize_q8_0_rows_dev(self, blocks: DeviceArray, x: DeviceArray, x_stride: int, n_rows: int, row_len: int,
                               blocks_offset: int = 0, x_offset: int = 0):
        """KVCache.put's Q8_0 branch for n_rows rows (byte offsets into the buffers)."""
        check(self.lib.mmhip_quantize_q8_0_rows_dev(self.handle, blocks.ptr + blocks_offset, x.ptr + x_offset,
                                                    x_stride, n_rows, row_len), "mmhip_quantize_q8_0_rows_dev")

    def dequantize_q8_0_rows_dev(self, out: DeviceArray, out_stride: int, blocks: DeviceArray, n_rows: int,
                                 row_len: int, out_offset: int = 0, blocks_offset: int = 0):
        """getKVCompressed / getKPe's Q8_0 branch for n_rows rows."""
        check(self.lib.mmhip_dequantize_q8_0_rows_dev(self.handle, out.ptr + out_offset, out_stride,
                                                      blocks.ptr + blocks_offset, n_rows, row_len),
              "mmhip_dequantize_q8_0_rows_dev")


class Gguf:
    """A memory-mapped GGUF v3 file (gguf.loadFromFile / parse, gguf.zig:266-413)."""

    NOT_FOUND = -6

    def __init__(self, path):
        self.lib = load_library()
        h = _c_void_p()
        check(self.lib.mmhip_gguf_open(os.fsencode(path), ctypes.byref(h)), "mmhip_gguf_open")
        self.handle = h.value

    def close(self):
        if self.handle:
            self.lib.mmhip_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        i = GgufInfo()
        check(self.lib.mmhip_gguf_get_info(self.handle, ctypes.byref(i)), "mmhip_gguf_get_info")
        return {f: getattr(i, f) for f, _ in GgufInfo._fields_}

    @staticmethod
    def _tensor_dict(t: GgufTensor) -> dict:
        return dict(name=_dec(t.name), n_dims=t.n_dims, dims=tuple(t.dims), type=t.type, offset=t.offset,
                    n_elements=t.n_elements, n_bytes=t.n_bytes, data=t.data)

    def tensors(self) -> list:
        out = []
        for i in range(self.info()["n_tensors"]):
            t = GgufTensor()
            check(self.lib.mmhip_gguf_tensor_at(self.handle, i, ctypes.byref(t)), "mmhip_gguf_tensor_at")
            out.append(self._tensor_dict(t))
        return out

    def tensor(self, name: str) -> Optional[dict]:
        t = GgufTensor()
        rc = self.lib.mmhip_gguf_find_tensor(self.handle, _enc(name), ctypes.byref(t))
        if rc == self.NOT_FOUND:
            return None
        check(rc, "mmhip_gguf_find_tensor")
        return self._tensor_dict(t)

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's mapped bytes."""
        t = self.tensor(name)
        if t is None or not t["data"]:
            raise KeyError(name)
        return np.ctypeslib.as_array(ctypes.cast(t["data"], ctypes.POINTER(ctypes.c_uint8)), (t["n_bytes"],)).copy()

    def keys(self) -> list:
        return [_dec(self.lib.mmhip_gguf_key_at(self.handle, i)) for i in range(self.info()["n_keys"])]

    def meta_type(self, key: str) -> Optional[int]:
        rc = self.lib.mmhip_gguf_meta_type(self.handle, _enc(key))
        return None if rc < 0 else rc

    def meta_int(self, key: str) -> Optional[int]:
        v = ctypes.c_int64()
        rc = self.lib.mmhip_gguf_meta_int(self.handle, _enc(key), ctypes.byref(v))
        return None if rc == self.NOT_FOUND else (check(rc, "mmhip_gguf_meta_int"), v.value)[1]

    def meta_float(self, key: str) -> Optional[float]:
        v = ctypes.c_double()
        rc = self.lib.mmhip_gguf_meta_float(self.handle, _enc(key), ctypes.byref(v))
        return None if rc == self.NOT_FOUND else (check(rc, "mmhip_gguf_meta_float"), v.value)[1]

    def meta_string(self, key: str) -> Optional[bytes]:
        p, n = _c_void_p(), _u64()
        rc = self.lib.mmhip_gguf_meta_string(self.handle, _enc(key), ctypes.byref(p), ctypes.byref(n))
        if rc == self.NOT_FOUND:
            return None
        check(rc, "mmhip_gguf_meta_string")
        return ctypes.string_at(p.value, n.value) if n.value else b""

    def meta_array(self, key: str) -> Optional[tuple]:
        """(element type, length, payload bytes)."""
        et, n, p, nb = _u32(), _u64(), _c_void_p(), _u64()
        rc = self.lib.mmhip_gguf_meta_array(self.handle, _enc(key), ctypes.byref(et), ctypes.byref(n),
                                            ctypes.byref(p), ctypes.byref(nb))
        if rc == self.NOT_FOUND:
            return None
        check(rc, "mmhip_gguf_meta_array")
        return et.value, n.value, (ctypes.string_at(p.value, nb.value) if nb.value else b"")


class MoeLayer:
    """Device-resident MoE FFN layer (moeFFN + Scheduler.route on the GPU)."""

    def __init__(self, ctx: Context, *, hidden: int, inter: int, n_experts: int, expert_type: int,
                 router: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray,
                 shared: Optional[tuple] = None, shared_inter: Optional[int] = None,
                 shared_type: Optional[int] = None, router_type: int = F32, routed_scaling_factor: float = 1.0):
        self.ctx = ctx
        self.hidden, self.inter, self.n_experts = hidden, inter, n_experts
        self._keep = [router, gate, up, down] + (list(shared) if shared else [])
        w = MoeWeights()
        w.hidden_size, w.moe_intermediate, w.n_routed_experts = hidden, inter, n_experts
        w.shared_intermediate = shared_inter if shared_inter is not None else inter
        w.expert_type = expert_type
        w.shared_type = shared_type if shared_type is not None else expert_type
        w.router_type = router_type
        w.routed_scaling_factor = routed_scaling_factor
        w.router_host, w.expert_gate_host = _ptr(router), _ptr(gate)
        w.expert_up_host, w.expert_down_host = _ptr(up), _ptr(down)
        if shared:
            w.shared_gate_host, w.shared_up_host, w.shared_down_host = (_ptr(s) for s in shared)
        h = _c_void_p()
        check(ctx.lib.mmhip_moe_layer_create(ctx.handle, ctypes.byref(w), ctypes.byref(h)), "mmhip_moe_layer_create")
        self.handle = h.value
        self._plan = None  # the PlanDispatch this layer is bound to, if any

    @classmethod
    def from_gguf(cls, ctx: Context, g: "Gguf", layer: int) -> "MoeLayer":
        """Model.bindLayer's FFN tensors (model.zig:289-395) of blk.<layer>, uploaded once."""
        gate = g.tensor(f"blk.{layer}.ffn_gate_exps.weight")
        if gate is None:
            raise KeyError(f"blk.{layer}.ffn_gate_exps.weight")
        self = cls.__new__(cls)
        self.ctx, self._keep = ctx, [g]
        self.hidden, self.inter, self.n_experts = gate["dims"][0], gate["dims"][1], gate["dims"][2]
        h = _c_void_p()
        check(ctx.lib.mmhip_moe_layer_create_gguf(ctx.handle, g.handle, layer, ctypes.byref(h)),
              "mmhip_moe_layer_create_gguf")
        self.handle = h.value
        self._plan = None
        return self

    def free(self):
        if self.handle:
            self.ctx.lib.mmhip_moe_layer_destroy(self.ctx.handle, self.handle)
            self.handle = None

    @staticmethod
    def route_params(level: int = 0, active_expert_limit: int = 0, deferral_bias: Optional[np.ndarray] = None):
        rp = RouteParams()
        rp.throttle_level = level
        rp.active_expert_limit = active_expert_limit
        rp.deferral_bias_host = (deferral_bias.ctypes.data_as(_fp) if deferral_bias is not None else None)
        return rp

    def ffn(self, hidden: np.ndarray, level: int = 0, active_expert_limit: int = 0,
            deferral_bias: Optional[np.ndarray] = None):
        """moeFFN for the tokens in `hidden`. A layer bound to a PlanDispatch
        runs only through it: a direct call raises MmhipError (ERR_INVALID),
        so no layer's routed experts run twice for one token."""
        if self._plan is not None:
            raise MmhipError("moe_ffn", ERR_INVALID,
                             "the layer is bound to a PlanDispatch; its FFN runs at the plan's ffn_gate_up")
        return self._ffn(hidden, level, active_expert_limit, deferral_bias)

    def _ffn(self, hidden: np.ndarray, level: int = 0, active_expert_limit: int = 0,
             deferral_bias: Optional[np.ndarray] = None):
        hidden = np.ascontiguousarray(hidden, dtype=np.float32).reshape(-1, self.hidden)
        t = hidden.shape[0]
        out = np.empty_like(hidden)
        ids = np.empty((t, 4), dtype=np.uint32)
        wts = np.empty((t, 4), dtype=np.float32)
        rp = self.route_params(level, active_expert_limit, deferral_bias)
        k = check(self.ctx.lib.mmhip_moe_ffn(self.ctx.handle, self.handle, _ptr(hidden), _ptr(out), t,
                                             ctypes.byref(rp), _ptr(ids), _ptr(wts)), "mmhip_moe_ffn")
        return out, ids[:, :k], wts[:, :k]

    def ffn_dev(self, hidden: DeviceArray, out: DeviceArray, n_tokens: int, rp: Optional[RouteParams] = None):
        if self._plan is not None:
            raise MmhipError("moe_ffn_dev", ERR_INVALID,
                             "the layer is bound to a PlanDispatch; its FFN runs at the plan's ffn_gate_up")
        rp = rp if rp is not None else self.route_params()
        check(self.ctx.lib.mmhip_moe_ffn_dev(self.ctx.handle, self.handle, hidden.ptr, out.ptr, n_tokens,
                                             ctypes.byref(rp), None, None), "mmhip_moe_ffn_dev")

    def expert_counts(self) -> np.ndarray:
        out = np.zeros(self.n_experts, dtype=np.uint64)
        check(self.ctx.lib.mmhip_moe_expert_counts(self.ctx.handle, self.handle, _ptr(out)), "mmhip_moe_expert_counts")
        return out


# ----------------------------------------------------------------------------
# Operator planner (OpScheduler / LayerPlan, scheduler.zig:265-552); host only
# ----------------------------------------------------------------------------

OP = dict(matMulQ8_0=0, matMulQ4_K=1, matMulF32=2, matVecMulQ8_0=3, matVecMulF32=4, rmsNorm=5, siluMul=6, rope=7,
          softmax=8, dot=9, attention=10, ffn_gate_up=11, ffn_down=12)
PREC = dict(q8_0=0, q4_k=1, f32=2, f16=3, iq2_xxs=4)
BACKEND_CPU, BACKEND_GPU, BACKEND_NPU = 0, 1, 2


def plan_layer(layer: int, *, hidden_size: int, intermediate_size: int, num_heads: int, head_dim: int,
               leading_dense_layers: int, n_routed_experts: int, weight_precision: int = 0, seq_len_hint: int = 0,
               has_gpu: bool = False, has_npu: bool = False, throttle_level: int = 0, perf_db=()):
    """OpScheduler.init + planLayer. perf_db: iterable of (op, precision,
    (m, n, k, dim), cpu_us, gpu_us). Returns a list of OpSchedule."""
    lib = load_library()
    hp = PlanHParams(hidden_size, intermediate_size, num_heads, head_dim, seq_len_hint, leading_dense_layers,
                     n_routed_experts, weight_precision)
    entries = (PerfEntry * max(1, len(perf_db)))()
    for i, (op, prec, shp, cpu_us, gpu_us) in enumerate(perf_db):
        entries[i].op, entries[i].precision = op, prec
        entries[i].shape = Shape(*shp)
        entries[i].cpu_us, entries[i].gpu_us = cpu_us, gpu_us
    out = (OpSchedule * 16)()
    n = ctypes.c_size_t()
    check(lib.mmhip_plan_layer(layer, ctypes.byref(hp), int(has_gpu), int(has_npu), throttle_level, entries,
                               len(perf_db), out, 16, ctypes.byref(n)), "mmhip_plan_layer")
    return list(out[:n.value])


def _ops_array(ops):
    arr = (OpSchedule * max(1, len(ops)))()
    for i, o in enumerate(ops):
        arr[i] = o
    return arr


def plan_critical_path_us(ops) -> int:
    """LayerPlan.estimatedCriticalPathUs."""
    return load_library().mmhip_plan_critical_path_us(_ops_array(ops), len(ops))


def plan_device_mask(ops) -> int:
    """LayerPlan.deviceMask (bit 0 CPU, 1 GPU, 2 NPU)."""
    return load_library().mmhip_plan_device_mask(_ops_array(ops), len(ops))


def op_schedule(op: int, backend: int, precision: int, estimated_us: int, sync_after: bool, shape=(0, 0, 0, 0)):
    return OpSchedule(op, backend, precision, int(sync_after), Shape(*shape), estimated_us)


class PlanDispatch:
    """The GPU side of HeteroExecutor.executeLayer (hetero_executor.zig:88-127,
    the body dispatchGpu lacks at 154-159), as zig/hip_backend.zig's
    PlanDispatch does: the device runs the whole moeFFN in one call, so
    ffn_gate_up issues it for the token in `hidden`, siluMul is already done
    inside it, and ffn_down hands the result back (hidden <- ffn_out,
    inference.zig:1009). Other ops raise MmhipError with ERR_UNSUPPORTED (the
    executor keeps them on its CPU path); siluMul or ffn_down without a
    preceding ffn_gate_up raise it with ERR_INVALID.

    The reference's plan for a MoE layer names only the shared expert's
    gate/up, siluMul and down (scheduler.zig:466-501) and leaves the routed
    experts to moeFFN; here the plan's FFN ops carry the whole layer. A layer
    therefore runs through exactly one of the two paths: binding it to a
    PlanDispatch makes its direct ffn / ffn_dev calls (moeFFN's path) raise
    ERR_INVALID until release(), and a layer binds to one PlanDispatch at a
    time."""

    def __init__(self, moe: Optional["MoeLayer"], level: int = 0):
        if moe is not None and moe._plan is not None:
            raise MmhipError("plan dispatch", ERR_INVALID, "the MoE layer is already bound to a PlanDispatch")
        self.moe, self.level = moe, level
        self.ffn_out = None
        if moe is not None:
            moe._plan = self

    def release(self) -> None:
        """Unbinds the layer: moeFFN's direct calls work again."""
        if self.moe is not None and self.moe._plan is self:
            self.moe._plan = None
        self.moe = None
        self.ffn_out = None

    def dispatch_gpu(self, op: OpSchedule, hidden: np.ndarray) -> None:
        if op.op == OP["ffn_gate_up"]:
            if self.moe is None:
                raise MmhipError("plan dispatch", ERR_UNSUPPORTED, "no MoE layer for ffn_gate_up")
            self.ffn_out = self.moe._ffn(hidden, level=self.level)[0].reshape(hidden.shape)
        elif op.op == OP["siluMul"]:
            if self.ffn_out is None:
                raise MmhipError("plan dispatch", ERR_INVALID, "siluMul before ffn_gate_up")
        elif op.op == OP["ffn_down"]:
            if self.ffn_out is None:
                raise MmhipError("plan dispatch", ERR_INVALID, "ffn_down before ffn_gate_up")
            hidden[...] = self.ffn_out
            self.ffn_out = None
        else:
            raise MmhipError("plan dispatch", ERR_UNSUPPORTED, f"op {op.op} does not run on this backend")


# ----------------------------------------------------------------------------
# Seeded synthetic weights (raw GGUF bytes)
# ----------------------------------------------------------------------------

def f16_bits(values: np.ndarray) -> np.ndarray:
    """IEEE round-to-nearest-even binary16 bit patterns (numpy's conversion)."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def make_q8_0(rng: np.random.Generator, rows: int, cols: int, count: int = 1, d_sigma: float = 0.02) -> np.ndarray:
    """Q8_0 blocks: qs ~ U{-127..127}, d = f16(|N(0, d_sigma)| / 127)."""
    nb = (cols + 31) // 32
    n = count * rows * nb
    blk = np.empty((n, 34), dtype=np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, d_sigma, n)) / 127.0)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:] = rng.integers(-127, 128, (n, 32), dtype=np.int64).astype(np.int8).view(np.uint8)
    return blk.reshape(-1)


def make_iq2_xxs(rng: np.random.Generator, rows: int, cols: int, count: int = 1, d_scale: float = 4e-4) -> np.ndarray:
    """IQ2_XXS superblocks: per 32-weight sub-block four random grid indices,
    four random 7-bit sign codes and a random 4-bit scale;
    d = f16(|N(0, 1)| * d_scale)."""
    assert cols % 256 == 0
    n = count * rows * (cols // 256)
    sb = np.empty((n, 66), dtype=np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, 1.0, n)) * d_scale)
    sb[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    idx = rng.integers(0, 256, (n, 8, 4), dtype=np.uint32)
    codes = rng.integers(0, 128, (n, 8, 4), dtype=np.uint32)
    ls = rng.integers(0, 16, (n, 8), dtype=np.uint32)
    aux0 = idx[..., 0] | (idx[..., 1] << 8) | (idx[..., 2] << 16) | (idx[..., 3] << 24)
    aux1 = codes[..., 0] | (codes[..., 1] << 7) | (codes[..., 2] << 14) | (codes[..., 3] << 21) | (ls << 28)
    words = np.stack([aux0, aux1], axis=-1).astype(np.uint32)  # [n, 8, 2]
    sb[:, 2:] = words.reshape(n, 16).view(np.uint8).reshape(n, 64)
    return sb.reshape(-1)


def make_weight(rng: np.random.Generator, ggml_type: int, rows: int, cols: int, count: int = 1) -> np.ndarray:
    if ggml_type == Q8_0:
        return make_q8_0(rng, rows, cols, count)
    if ggml_type == IQ2_XXS:
        return make_iq2_xxs(rng, rows, cols, count)
    if ggml_type == F32:
        return rng.normal(0.0, 0.02, count * rows * cols).astype(np.float32).view(np.uint8)
    if ggml_type == F16:
        return f16_bits(rng.normal(0.0, 0.02, count * rows * cols)).view(np.uint8)
    raise ValueError(f"unsupported type {ggml_type}")


def tensor_bytes(ggml_type: int, rows: int, cols: int, count: int = 1) -> int:
    bs, bb = BLOCK_SIZE[ggml_type], BLOCK_BYTES[ggml_type]
    return count * rows * ((cols + bs - 1) // bs) * bb


def max_abs_rel(y: np.ndarray, ref: np.ndarray) -> float:
    """max|y - ref| / max|ref| (the path's parity metric)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / den) if den > 0 else float(np.max(np.abs(y - ref)))
