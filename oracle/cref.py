"""ctypes wrapper of oracle/liboracle.so (oracle/expert_ref.c) -- TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py).

Arrays are numpy: packed weights uint32 [S, N, K*bits/32], scales/biases as
uint16 bit patterns [S, N, K/group] in the activation dtype ("bf16"/"f16"),
activations and results as float32 values exactly representable in that
dtype.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
DT = {"f16": 1, "bf16": 2}


class OProj(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("b", ctypes.c_void_p),
                ("bits", ctypes.c_int32), ("group", ctypes.c_int32), ("N", ctypes.c_int32),
                ("K", ctypes.c_int32), ("meta_dt", ctypes.c_int32)]


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class CRef:
    def __init__(self, path: Path):
        self.lib = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        self.lib.oracle_qmv.argtypes = [ctypes.POINTER(OProj), ctypes.c_int, P, P]
        self.lib.oracle_moe_layer.argtypes = [ctypes.POINTER(OProj)] * 6 + [
            P, ctypes.c_int, ctypes.c_int, P, P, ctypes.c_int, ctypes.c_float, ctypes.c_int, P, P]
        self.lib.oracle_moe_layer.restype = ctypes.c_int
        self.lib.oracle_router.argtypes = [P, P, P] + [ctypes.c_int] * 6 + [ctypes.c_float, P, P]
        self.lib.oracle_round_array.argtypes = [P, P, ctypes.c_int, ctypes.c_int]
        self.lib.oracle_set_threads.argtypes = [ctypes.c_int]
        self._keep = []

    def set_threads(self, n: int) -> None:
        """OpenMP threads of the moe_layer / qmv loops (0: all processors)."""
        self.lib.oracle_set_threads(int(n))

    def proj(self, arr, dt: str) -> OProj:
        """arr = (w uint32 [S,N,W], s uint16 [S,N,G], b uint16 [S,N,G], bits, group)."""
        w, s, b, bits, group = arr
        w = np.ascontiguousarray(w, dtype=np.uint32)
        s = np.ascontiguousarray(s, dtype=np.uint16)
        b = np.ascontiguousarray(b, dtype=np.uint16)
        self._keep += [w, s, b]
        N = w.shape[-2]
        K = w.shape[-1] * 32 // bits
        return OProj(w.ctypes.data, s.ctypes.data, b.ctypes.data, bits, group, N, K, DT[dt])

    def qmv(self, arr, slot, v, dt):
        p = self.proj(arr, dt)
        v = _f32(v)
        out = np.zeros(p.N, dtype=np.float32)
        self.lib.oracle_qmv(ctypes.byref(p), slot, v.ctypes.data, out.ctypes.data)
        return out

    def moe_layer(self, x, slots, weights, arena, dt, *, shared=None, limit=10.0,
                  fp32_swiglu=False, return_terms=False):
        """arena/shared: {"gate_proj"|"up_proj"|"down_proj": (w, s, b, bits, group)}."""
        x = _f32(x)
        T, d = x.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        k = slots.shape[1]
        weights = _f32(weights)
        g, u, dn = (self.proj(arena[p], dt) for p in ("gate_proj", "up_proj", "down_proj"))
        if shared is not None:
            sg, su, sd = (ctypes.byref(self.proj(shared[p], dt))
                          for p in ("gate_proj", "up_proj", "down_proj"))
        else:
            sg = su = sd = None
        out = np.zeros((T, d), dtype=np.float32)
        terms = np.zeros((T, d), dtype=np.float32)
        rc = self.lib.oracle_moe_layer(ctypes.byref(g), ctypes.byref(u), ctypes.byref(dn), sg, su,
                                       sd, x.ctypes.data, T, k, slots.ctypes.data,
                                       weights.ctypes.data, DT[dt], float(limit), int(fp32_swiglu),
                                       out.ctypes.data, terms.ctypes.data)
        self._keep.clear()
        if rc:
            raise MemoryError("oracle_moe_layer")
        return (out, terms) if return_terms else out

    def router(self, x, wg, bias, k, score_func=0, norm=True, scale=1.0):
        x, wg = _f32(x), _f32(wg)
        T, d = x.shape
        E = wg.shape[0]
        b = _f32(bias) if bias is not None else None
        idx = np.zeros((T, k), dtype=np.int32)
        w = np.zeros((T, k), dtype=np.float32)
        self.lib.oracle_router(x.ctypes.data, wg.ctypes.data, b.ctypes.data if b is not None else None,
                               T, d, E, k, score_func, int(norm), float(scale), idx.ctypes.data,
                               w.ctypes.data)
        return idx, w

    def round_array(self, a, dt):
        a = _f32(a).ravel()
        out = np.empty_like(a)
        self.lib.oracle_round_array(a.ctypes.data, out.ctypes.data, a.size, DT[dt])
        return out


def load() -> CRef:
    return CRef(HERE / "liboracle.so")
