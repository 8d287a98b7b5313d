"""ctypes binding of liboracle.so, the C restatement of the reference CPU
path (oracle.h). TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, Q8_0, IQ2_XXS = 0, 1, 8, 16
NORMAL, LIGHT, MEDIUM, HEAVY = 0, 1, 2, 3
TARGET_GPU, TARGET_CPU, TARGET_SKIPPED = 0, 1, 2

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u32, _u64 = ctypes.c_uint32, ctypes.c_uint64


class Throttle(ctypes.Structure):
    _fields_ = [("level", ctypes.c_int), ("active_expert_limit", _u32), ("hot_experts_on_cpu", ctypes.c_int)]


class ExpertStats(ctypes.Structure):
    _fields_ = [("counts", _vp), ("n_experts", _u32), ("n_layers", _u32), ("total_tokens", _u64)]


class MoeDesc(ctypes.Structure):
    _fields_ = [("hidden", _u32), ("moe_inter", _u32), ("shared_inter", _u32), ("n_experts", _u32),
                ("expert_type", _u32), ("shared_type", _u32), ("router_type", _u32),
                ("router", _vp), ("expert_gate", _vp), ("expert_up", _vp), ("expert_down", _vp),
                ("shared_gate", _vp), ("shared_up", _vp), ("shared_down", _vp),
                ("routed_scaling_factor", ctypes.c_float), ("deferral_bias", _vp)]


_SIGS = {
    "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float, ctypes.POINTER(ctypes.c_int)]),
    "orc_block_size": (_u64, [_u32]),
    "orc_block_bytes": (_u64, [_u32]),
    "orc_tensor_bytes": (_u64, [_u32, _u64]),
    "orc_iq2xxs_grid": (_u64, [_u32]),
    "orc_ksigns": (ctypes.c_uint8, [_u32]),
    "orc_dequantize_q8_0": (None, [_vp, _u64, _vp]),
    "orc_quantize_q8_0": (None, [_vp, _u64, _vp]),
    "orc_sample_greedy": (_u32, [_vp, _u64]),
    "orc_quantize_q8_0_rows": (None, [_vp, _u64, _u64, _u32, _vp]),
    "orc_dequantize_q8_0_rows": (None, [_vp, _u64, _u32, _vp]),
    "orc_dequantize_iq2xxs_block": (None, [_vp, _vp]),
    "orc_dequantize_iq2xxs": (None, [_vp, _u64, _vp]),
    "orc_dequantize": (ctypes.c_int, [_vp, _u32, _u64, _vp]),
    "orc_matvec_q8_0": (None, [_vp, _vp, _vp, _sz, _sz]),
    "orc_matmul_q8_0": (None, [_vp, _vp, _vp, _sz, _sz, _sz]),
    "orc_matvec_f32": (None, [_vp, _vp, _vp, _sz, _sz]),
    "orc_dot": (ctypes.c_float, [_vp, _vp, _sz]),
    "orc_silu": (ctypes.c_float, [ctypes.c_float]),
    "orc_topk": (_sz, [_vp, _sz, _sz, _vp, _vp]),
    "orc_mat_vec_mul_unified": (ctypes.c_int, [_vp, _vp, _u32, _vp, _sz, _sz]),
    "orc_batch_mat_mul_unified": (ctypes.c_int, [_vp, _vp, _u32, _vp, _sz, _sz, _sz]),
    "orc_throttle_set": (None, [ctypes.POINTER(Throttle), ctypes.c_int]),
    "orc_route": (_u32, [_vp, _u32, ctypes.POINTER(Throttle), ctypes.c_float, _vp, _u32, _vp, _vp, _vp, _vp]),
    "orc_pool_create": (_vp, [ctypes.c_int]),
    "orc_pool_destroy": (None, [_vp]),
    "orc_moe_ffn": (ctypes.c_int, [ctypes.POINTER(MoeDesc), _vp, _vp, _u32, ctypes.POINTER(Throttle),
                                   _vp, _vp, _vp, _vp]),
    "orc_moe_ffn_batch": (ctypes.c_int, [ctypes.POINTER(MoeDesc), _vp, _vp, _u32, ctypes.POINTER(Throttle),
                                         _vp, _vp, _u32, _vp, _vp]),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} missing (make -C oracle)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(v: float):
    """f32ToF16 (dequant.zig:50-95): (code, defect) with defect 0 (a correct
    code), 1 (the reference traps; low 16 bits returned) or 2 (the reference
    returns this corrupted code)."""
    d = ctypes.c_int(0)
    r = lib().orc_f32_to_f16(v, ctypes.byref(d))
    return r, d.value


def sample_greedy(logits: np.ndarray) -> int:
    """sampleGreedy (inference.zig:376-386)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
    return int(lib().orc_sample_greedy(_p(logits), logits.size))


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """quantizeQ8_0 (dequant.zig:98-130): f32 values -> raw 34-byte blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(((x.size + 31) // 32) * 34, dtype=np.uint8)
    lib().orc_quantize_q8_0(_p(x), x.size, _p(out))
    return out


def quantize_q8_0_rows(x: np.ndarray, row_len: int) -> np.ndarray:
    """KVCache.put's Q8_0 branch per row: [n_rows][row_len] f32 -> blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_rows = x.size // row_len
    out = np.empty(n_rows * ((row_len + 31) // 32) * 34, dtype=np.uint8)
    lib().orc_quantize_q8_0_rows(_p(x), row_len, n_rows, row_len, _p(out))
    return out


def dequantize_q8_0_rows(blocks: np.ndarray, n_rows: int, row_len: int) -> np.ndarray:
    """getKVCompressed / getKPe's dequantization per row."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty((n_rows, row_len), dtype=np.float32)
    lib().orc_dequantize_q8_0_rows(_p(blocks), n_rows, row_len, _p(out))
    return out


def ksigns(code: int) -> int:
    return lib().orc_ksigns(code)


def grid(idx: int) -> int:
    return lib().orc_iq2xxs_grid(idx)


def tensor_bytes(t: int, n: int) -> int:
    return lib().orc_tensor_bytes(t, n)


def dequantize(raw: np.ndarray, t: int, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw)
    out = np.empty(n, dtype=np.float32)
    rc = lib().orc_dequantize(_p(raw), t, n, _p(out))
    if rc:
        raise ValueError(f"orc_dequantize rc={rc}")
    return out


def matvec_q8_0(raw, x, out_dim, in_dim) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(out_dim, dtype=np.float32)
    lib().orc_matvec_q8_0(_p(out), _p(raw), _p(x), out_dim, in_dim)
    return out


def matmul_q8_0(raw, b, m, n, k) -> np.ndarray:
    """qmm.matMulQ8_0: returns C [m][n] (out_dim x batch)."""
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_q8_0(_p(out), _p(raw), _p(b), m, n, k)
    return out


def matvec_f32(w, x, out_dim, in_dim) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(out_dim, dtype=np.float32)
    lib().orc_matvec_f32(_p(out), _p(w), _p(x), out_dim, in_dim)
    return out


def dot(a, b) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().orc_dot(_p(a), _p(b), a.size)


def silu(x: float) -> float:
    return lib().orc_silu(x)


def topk(scores, k):
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    idx = np.zeros(max(k, 1), dtype=np.uint32)
    sc = np.zeros(max(k, 1), dtype=np.float32)
    n = lib().orc_topk(_p(scores), scores.size, k, _p(idx), _p(sc))
    return idx[:n], sc[:n]


def mat_vec_mul_unified(raw, t, x, out_dim, in_dim) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(out_dim, dtype=np.float32)
    rc = lib().orc_mat_vec_mul_unified(_p(out), _p(raw), t, _p(x), out_dim, in_dim)
    if rc:
        raise ValueError(f"orc_mat_vec_mul_unified rc={rc}")
    return out


def batch_mat_mul_unified(raw, t, xin, out_dim, batch, in_dim) -> np.ndarray:
    xin = np.ascontiguousarray(xin, dtype=np.float32)
    out = np.empty((batch, out_dim), dtype=np.float32)
    rc = lib().orc_batch_mat_mul_unified(_p(out), _p(raw), t, _p(xin), out_dim, batch, in_dim)
    if rc:
        raise ValueError(f"orc_batch_mat_mul_unified rc={rc}")
    return out


def throttle(level: int, active_expert_limit: int = 0) -> Throttle:
    th = Throttle()
    lib().orc_throttle_set(ctypes.byref(th), level)
    if active_expert_limit:
        th.active_expert_limit = active_expert_limit
    return th


class Stats:
    def __init__(self, n_layers: int, n_experts: int):
        self.counts = np.zeros(n_layers * n_experts, dtype=np.uint64)
        self.s = ExpertStats(self.counts.ctypes.data, n_experts, n_layers, 0)


def route(scores, level=NORMAL, rsf=1.0, stats: Stats = None, layer=0, active_expert_limit=0):
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    th = throttle(level, active_expert_limit)
    ids = np.zeros(4, dtype=np.uint32)
    w = np.zeros(4, dtype=np.float32)
    targets = np.zeros(4, dtype=np.int32)
    deferred = np.zeros(1, dtype=np.int32)
    k = lib().orc_route(ctypes.addressof(stats.s) if stats else None, layer, ctypes.byref(th), rsf,
                        _p(scores), scores.size, _p(ids), _p(w), _p(targets), _p(deferred))
    return ids[:k], w[:k], targets[:k], bool(deferred[0])


class Pool:
    """thread_pool.ThreadPool equivalent (n workers, FIFO)."""

    def __init__(self, n_threads: int = 4):
        self.h = lib().orc_pool_create(n_threads)
        self.n = n_threads

    def close(self):
        if self.h:
            lib().orc_pool_destroy(self.h)
            self.h = None


class Moe:
    """moeFFN with the reference's data layout (raw GGUF bytes per tensor)."""

    def __init__(self, *, hidden, inter, n_experts, expert_type, router, gate, up, down, shared=None,
                 shared_inter=None, shared_type=None, router_type=F32, routed_scaling_factor=1.0,
                 deferral_bias=None):
        self._keep = [router, gate, up, down] + (list(shared) if shared else []) + [deferral_bias]
        d = MoeDesc()
        d.hidden, d.moe_inter, d.n_experts = hidden, inter, n_experts
        d.shared_inter = shared_inter if shared_inter is not None else inter
        d.expert_type = expert_type
        d.shared_type = shared_type if shared_type is not None else expert_type
        d.router_type = router_type
        d.router, d.expert_gate, d.expert_up, d.expert_down = _p(router), _p(gate), _p(up), _p(down)
        if shared:
            d.shared_gate, d.shared_up, d.shared_down = (_p(s) for s in shared)
        d.routed_scaling_factor = routed_scaling_factor
        d.deferral_bias = _p(deferral_bias) if deferral_bias is not None else None
        self.d = d
        self.hidden = hidden

    def ffn(self, hidden, level=NORMAL, pool: Pool = None, stats: Stats = None, layer=0, active_expert_limit=0):
        hidden = np.ascontiguousarray(hidden, dtype=np.float32).reshape(-1, self.hidden)
        t = hidden.shape[0]
        out = np.empty_like(hidden)
        ids = np.zeros((t, 4), dtype=np.uint32)
        w = np.zeros((t, 4), dtype=np.float32)
        th = throttle(level, active_expert_limit)
        k = lib().orc_moe_ffn_batch(ctypes.byref(self.d), pool.h if pool else None,
                                    ctypes.addressof(stats.s) if stats else None, layer, ctypes.byref(th),
                                    _p(hidden), _p(out), t, _p(ids), _p(w))
        if k < 0:
            raise ValueError(f"orc_moe_ffn_batch rc={k}")
        return out, ids[:, :k], w[:, :k]
