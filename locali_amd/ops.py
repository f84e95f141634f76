"""torch-facing wrappers over the liblocali_amd.so C ABI.

Tensors must already live on the GPU; the wrappers pass raw device pointers
and the current HIP stream, check shapes on the host, and raise on any error.
PyTorch supplies device memory, streams, data movement (index selects,
concatenation) and the dtype casts the reference itself makes (activations to
fp16 for an fp16-metadata tier, dsv4_arena.py:172-173; the output back to x's
dtype, arena.py:547); every product and sum runs in the library's HIP
kernels.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import (COMBINE_FP32, COMBINE_ROUNDED, DT_BF16, DT_F16, DT_F32, SCORE_SIGMOID,
                   SCORE_SOFTMAX, SCORE_SQRTSOFTPLUS, check, lib)

__all__ = [
    "ProjArena", "ExpertArenaT", "RouterSpec", "Workspace", "router", "dispatch",
    "expert_decode", "decode_gateup", "decode_down_combine", "router_logits", "decode_gateup_select",
    "expert_grouped", "combine", "combine_routes",
    "forward", "arena_fill",
    "COMBINE_ROUNDED", "COMBINE_FP32",
]

DTYPES = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}
SCORE_FUNCS = {"sqrtsoftplus": SCORE_SQRTSOFTPLUS, "sigmoid": SCORE_SIGMOID,
               "softmax": SCORE_SOFTMAX}


def _stream() -> int:
    """The current HIP stream of the current device (raw handle)."""
    return torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())


_STREAMS: dict = {}


def current_stream(device=None) -> torch.cuda.Stream:
    """torch.cuda.current_stream(device), one Stream object per raw stream
    (the torch call costs several microseconds; this lookup about one)."""
    idx = torch._C._cuda_getDevice() if device is None or torch.device(device).index is None \
        else torch.device(device).index
    raw = torch._C._cuda_getCurrentRawStream(idx)
    s = _STREAMS.get((idx, raw))
    if s is None:
        s = _STREAMS[(idx, raw)] = torch.cuda.current_stream(idx)
    return s


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr()


def _dt(t: torch.Tensor) -> int:
    try:
        return DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


@dataclass
class ProjArena:
    """One projection across all arena slots, in MLX affine layout:
    weight uint32 [S, rows, cols*bits/32], scales/biases [S, rows, cols/group]."""
    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    bits: int
    group_size: int

    @property
    def n_slots(self) -> int:
        return int(self.weight.shape[0])

    @property
    def rows(self) -> int:
        return int(self.weight.shape[1])

    @property
    def cols(self) -> int:
        return int(self.weight.shape[2]) * 32 // self.bits

    def struct(self) -> _lib.QProj:
        w, s, b = self.weight, self.scales, self.biases
        key = (w.data_ptr(), s.data_ptr(), b.data_ptr(), tuple(w.shape), tuple(s.shape), self.bits,
               self.group_size, w.dtype, s.dtype)
        cached = self.__dict__.get("_struct")
        if cached is not None and cached[0] == key:
            return cached[1]
        st = self._build_struct()
        self.__dict__["_struct"] = (key, st)
        return st

    def _build_struct(self) -> _lib.QProj:
        w, s, b = self.weight, self.scales, self.biases
        if w.dtype not in (torch.int32, torch.uint32):
            raise TypeError("packed weights must be 32-bit")
        if s.shape != b.shape or s.dtype != b.dtype:
            raise ValueError("scales and biases must match")
        if s.shape[:2] != w.shape[:2] or s.shape[2] * self.group_size != self.cols:
            raise ValueError(f"metadata shape {tuple(s.shape)} does not fit weight {tuple(w.shape)}")
        return _lib.QProj(_ptr(w), _ptr(s), _ptr(b), self.bits, self.group_size, self.rows,
                          self.cols, _dt(s), self.n_slots)


@dataclass
class ExpertArenaT:
    gate: ProjArena
    up: ProjArena
    down: ProjArena

    def struct(self) -> _lib.ExpertArena:
        parts = (self.gate.struct(), self.up.struct(), self.down.struct())
        cached = self.__dict__.get("_struct")
        if cached is None or any(a is not b for a, b in zip(cached[0], parts)):
            cached = self.__dict__["_struct"] = (parts, _lib.ExpertArena(*parts))
        return cached[1]

    @property
    def d_model(self) -> int:
        return self.gate.cols

    @property
    def d_ff(self) -> int:
        return self.gate.rows

    @property
    def n_slots(self) -> int:
        return self.gate.n_slots


@dataclass
class RouterSpec:
    """The gate's tensors (tf:modeling_deepseek_v4.py:1028-1033, 1062)."""
    weight: torch.Tensor                      # [E, d]
    top_k: int
    score_func: str = "sqrtsoftplus"
    norm_topk: bool = True
    routed_scale: float = 1.0
    score_bias: torch.Tensor | None = None    # [E] fp32
    tid2eid: torch.Tensor | None = None       # [vocab, top_k] int32

    def struct(self) -> _lib.Router:
        key = (self.weight.data_ptr(), tuple(self.weight.shape), self.weight.dtype, self.top_k, self.score_func,
               self.norm_topk, self.routed_scale,
               None if self.score_bias is None else self.score_bias.data_ptr(),
               None if self.tid2eid is None else (self.tid2eid.data_ptr(), tuple(self.tid2eid.shape)))
        cached = self.__dict__.get("_struct")
        if cached is not None and cached[0] == key:
            return cached[1]
        st = self._build_struct()
        self.__dict__["_struct"] = (key, st)
        return st

    def _build_struct(self) -> _lib.Router:
        E = int(self.weight.shape[0])
        bias = self.score_bias
        if bias is not None and (bias.dtype != torch.float32 or bias.numel() != E):
            raise ValueError("score_bias must be fp32 [n_experts]")
        t2e = self.tid2eid
        if t2e is not None and (t2e.dtype != torch.int32 or t2e.dim() != 2 or t2e.shape[1] != self.top_k):
            raise ValueError("tid2eid must be int32 [vocab, top_k]")
        return _lib.Router(_ptr(self.weight), _dt(self.weight), E, self.top_k,
                           SCORE_FUNCS[self.score_func], int(self.norm_topk),
                           float(self.routed_scale), _ptr(bias), _ptr(t2e),
                           int(t2e.shape[0]) if t2e is not None else 0)

    @property
    def n_experts(self) -> int:
        return int(self.weight.shape[0])


class Workspace:
    """Zero-initialised device scratch, grown on demand (growth allocates, so
    size it once up front for allocation-free steady state)."""

    def __init__(self, device=None):
        self.device = torch.device(device or "cuda")
        self.buf = torch.zeros(0, dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf.numel() < nbytes:
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self.buf

    def reserve(self, tokens, d_model, d_ff, n_experts, top_k, has_shared) -> torch.Tensor:
        return self.get(workspace_bytes(tokens, d_model, d_ff, n_experts, top_k, has_shared))

    def scratch(self, name: str, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
        """A named intermediate kept between calls (calls on one stream
        reuse it in order)."""
        cache = self.__dict__.setdefault("_scratch", {})
        t = cache.get(name)
        if t is None or t.shape != shape or t.dtype != dtype:
            t = cache[name] = torch.empty(shape, dtype=dtype, device=self.device)
        return t


_WS_BYTES: dict = {}


def workspace_bytes(tokens, d_model, d_ff, n_experts, top_k, has_shared) -> int:
    key = (int(tokens), int(d_model), int(d_ff), int(n_experts), int(top_k), bool(has_shared))
    n = _WS_BYTES.get(key)
    if n is None:
        n = _WS_BYTES[key] = int(lib().locali_moe_workspace_bytes(*key[:5], int(key[5])))
    return n


def _flat(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1]).contiguous()


def router(spec: RouterSpec, x: torch.Tensor, ws: Workspace, *, input_ids=None, logits=None,
           slot_of_expert=None, n_slots: int = 0):
    """Returns (idx int32 [T,k], weights fp32 [T,k], route_slot int32 [T,k] | None)."""
    x2 = _flat(x)
    T, d = x2.shape
    k = spec.top_k
    idx = torch.empty(T, k, dtype=torch.int32, device=x.device)
    w = torch.empty(T, k, dtype=torch.float32, device=x.device)
    rs = torch.empty(T, k, dtype=torch.int32, device=x.device) if slot_of_expert is not None else None
    buf = ws.reserve(T, d, 1, spec.n_experts, k, 0)
    ids = None
    if input_ids is not None:
        ids = input_ids.reshape(-1).to(device=x.device, dtype=torch.int32).contiguous()
    lg = logits.reshape(T, -1).contiguous() if logits is not None else None
    if lg is not None and lg.dtype != torch.float32:
        raise TypeError("logits must be fp32")
    st = spec.struct()
    rc = lib().locali_moe_router(ctypes.byref(st), _ptr(x2), _dt(x2), T, d, _ptr(ids), _ptr(lg),
                                 _ptr(slot_of_expert), n_slots, _ptr(idx), _ptr(w), _ptr(rs),
                                 _ptr(buf), buf.numel(), _stream())
    check(rc, "locali_moe_router")
    return idx, w, rs


def dispatch(route_slot: torch.Tensor, n_slots: int):
    """Stable slot sort: (sorted_route int32 [T*k], seg_start int32 [n_slots+1])."""
    T, k = route_slot.shape
    sorted_route = torch.empty(T * k, dtype=torch.int32, device=route_slot.device)
    seg = torch.empty(n_slots + 1, dtype=torch.int32, device=route_slot.device)
    rc = lib().locali_moe_dispatch(_ptr(route_slot.contiguous()), T, k, n_slots, _ptr(sorted_route),
                                   _ptr(seg), _stream())
    check(rc, "locali_moe_dispatch")
    return sorted_route, seg


def _decode_ws(ws, arena, T, k, shared):
    ws = ws if ws is not None else Workspace()
    return ws.reserve(T, arena.d_model, arena.d_ff, 1, k, shared is not None)


def expert_decode(arena: ExpertArenaT, shared: ExpertArenaT | None, x: torch.Tensor,
                  route_slot: torch.Tensor, weights: torch.Tensor, *, swiglu_limit=10.0,
                  fp32_swiglu=False, combine_mode=COMBINE_ROUNDED, hidden=None, ws=None):
    x2 = _flat(x)
    T = x2.shape[0]
    k = route_slot.shape[-1]
    routes = T * k + (T if shared is not None else 0)
    if hidden is None:
        hidden = (ws.scratch("decode_hidden", (routes, arena.d_ff), x2.dtype) if ws is not None
                  else torch.empty(routes, arena.d_ff, dtype=x2.dtype, device=x.device))
    out = torch.empty_like(x2)
    buf = _decode_ws(ws, arena, T, k, shared)
    a = arena.struct()
    s = shared.struct() if shared is not None else None
    rc = lib().locali_moe_expert_decode(ctypes.byref(a), ctypes.byref(s) if s is not None else None,
                                        _ptr(x2), _dt(x2), T, k, _ptr(route_slot.contiguous()),
                                        _ptr(weights.contiguous()), float(swiglu_limit),
                                        int(fp32_swiglu), int(combine_mode), _ptr(hidden), _ptr(out),
                                        _ptr(buf), buf.numel(), _stream())
    check(rc, "locali_moe_expert_decode")
    return out.reshape(x.shape)


def decode_gateup(arena: ExpertArenaT, shared: ExpertArenaT | None, x: torch.Tensor,
                  route_slot: torch.Tensor, hidden: torch.Tensor, ws: "Workspace", *,
                  swiglu_limit=10.0, fp32_swiglu=False):
    """Stage 1 of expert_decode: hidden[r] = swiglu(gate_r(x), up_r(x)); the
    down stage's prepared inputs stay in `ws`."""
    x2 = _flat(x)
    k = route_slot.shape[-1]
    buf = _decode_ws(ws, arena, x2.shape[0], k, shared)
    a = arena.struct()
    s = shared.struct() if shared is not None else None
    rc = lib().locali_moe_decode_gateup(ctypes.byref(a), ctypes.byref(s) if s is not None else None,
                                        _ptr(x2), _dt(x2), x2.shape[0], k, _ptr(route_slot),
                                        float(swiglu_limit), int(fp32_swiglu), _ptr(hidden),
                                        _ptr(buf), buf.numel(), _stream())
    check(rc, "locali_moe_decode_gateup")
    return hidden


def decode_down_combine(arena: ExpertArenaT, shared: ExpertArenaT | None, route_slot: torch.Tensor,
                        weights: torch.Tensor, out: torch.Tensor, ws: "Workspace", *,
                        combine_mode=COMBINE_ROUNDED):
    """Stage 2 of expert_decode (same workspace as stage 1): down projection,
    weighted combine, shared add."""
    T, k = route_slot.shape
    buf = _decode_ws(ws, arena, T, k, shared)
    a = arena.struct()
    s = shared.struct() if shared is not None else None
    rc = lib().locali_moe_decode_down_combine(ctypes.byref(a), ctypes.byref(s) if s is not None else None,
                                              _dt(out), T, k, _ptr(route_slot), _ptr(weights),
                                              int(combine_mode), _ptr(out), _ptr(buf), buf.numel(),
                                              _stream())
    check(rc, "locali_moe_decode_down_combine")
    return out


def router_logits(spec: RouterSpec, x: torch.Tensor, logits=None):
    """fp32 logits [T, E] = x . Wg^T (the decode forward's logits kernel; T <= 8)."""
    x2 = _flat(x)
    T, d = x2.shape
    out = torch.empty(T, spec.n_experts, dtype=torch.float32, device=x.device) if logits is None else logits
    st = spec.struct()
    rc = lib().locali_moe_router_logits(ctypes.byref(st), _ptr(x2), _dt(x2), T, d, _ptr(out), _stream())
    check(rc, "locali_moe_router_logits")
    return out


def decode_gateup_select(spec: RouterSpec, arena: ExpertArenaT, shared: ExpertArenaT | None,
                         slot_of_expert: torch.Tensor, x: torch.Tensor, logits: torch.Tensor,
                         hidden: torch.Tensor, ws: "Workspace", *, input_ids=None, swiglu_limit=10.0,
                         fp32_swiglu=False, idx=None, weights=None, route_slot=None):
    """The decode forward's gate/up kernel with the routes selected inside it
    from `logits`; returns (idx, weights, route_slot). decode_down_combine on
    the same workspace finishes the layer."""
    x2 = _flat(x)
    T = x2.shape[0]
    k = spec.top_k
    dev = x.device
    idx = torch.empty(T, k, dtype=torch.int32, device=dev) if idx is None else idx
    weights = torch.empty(T, k, dtype=torch.float32, device=dev) if weights is None else weights
    route_slot = torch.empty(T, k, dtype=torch.int32, device=dev) if route_slot is None else route_slot
    buf = _decode_ws(ws, arena, T, k, shared)
    ids = None
    if input_ids is not None:
        ids = input_ids.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
    r, a = spec.struct(), arena.struct()
    s = shared.struct() if shared is not None else None
    rc = lib().locali_moe_decode_gateup_select(ctypes.byref(r), ctypes.byref(a),
                                               ctypes.byref(s) if s is not None else None,
                                               _ptr(slot_of_expert), _ptr(x2), _dt(x2), T, _ptr(ids),
                                               _ptr(logits.contiguous()), float(swiglu_limit), int(fp32_swiglu),
                                               _ptr(idx), _ptr(weights), _ptr(route_slot), _ptr(hidden),
                                               _ptr(buf), buf.numel(), _stream())
    check(rc, "locali_moe_decode_gateup_select")
    return idx, weights, route_slot


def expert_grouped(arena: ExpertArenaT, shared: ExpertArenaT | None, x: torch.Tensor,
                   idx: torch.Tensor, slot_of_expert: torch.Tensor, weights: torch.Tensor,
                   ws: Workspace, *, n_experts=None, swiglu_limit=10.0, fp32_swiglu=False,
                   combine_mode=COMBINE_ROUNDED):
    x2 = _flat(x)
    T = x2.shape[0]
    k = idx.shape[-1]
    E = int(n_experts or slot_of_expert.numel())
    buf = ws.reserve(T, arena.d_model, arena.d_ff, E, k, shared is not None)
    out = torch.empty_like(x2)
    a = arena.struct()
    s = shared.struct() if shared is not None else None
    rc = lib().locali_moe_expert_grouped(ctypes.byref(a), ctypes.byref(s) if s is not None else None,
                                         _ptr(x2), _dt(x2), T, k, E, _ptr(idx.contiguous()),
                                         _ptr(slot_of_expert), _ptr(weights.contiguous()),
                                         float(swiglu_limit), int(fp32_swiglu), int(combine_mode),
                                         _ptr(out), _ptr(buf), buf.numel(), _stream())
    check(rc, "locali_moe_expert_grouped")
    return out.reshape(x.shape)


def expert_grouped_stages(arena: ExpertArenaT, shared: ExpertArenaT | None, x: torch.Tensor,
                          idx: torch.Tensor, slot_of_expert: torch.Tensor, weights: torch.Tensor,
                          ws: Workspace, *, n_experts=None, swiglu_limit=10.0, fp32_swiglu=False,
                          combine_mode=COMBINE_ROUNDED):
    """expert_grouped that also returns its intermediates
    (locali_moe_expert_grouped_stages): (out, h [routes, d_ff], y [routes,
    d_model]) with route r = t * top_k + j, and the shared expert's route of
    token t at T * top_k + t."""
    x2 = _flat(x)
    T = x2.shape[0]
    k = idx.shape[-1]
    E = int(n_experts or slot_of_expert.numel())
    routes = T * k + (T if shared is not None else 0)
    buf = ws.reserve(T, arena.d_model, arena.d_ff, E, k, shared is not None)
    out = torch.empty_like(x2)
    h = torch.empty(routes, arena.d_ff, dtype=x2.dtype, device=x2.device)
    y = torch.empty(routes, arena.d_model, dtype=x2.dtype, device=x2.device)
    pos = torch.empty(T * k, dtype=torch.int32, device=x2.device)
    a = arena.struct()
    s = shared.struct() if shared is not None else None
    rc = lib().locali_moe_expert_grouped_stages(ctypes.byref(a), ctypes.byref(s) if s is not None else None,
                                                _ptr(x2), _dt(x2), T, k, E, _ptr(idx.contiguous()),
                                                _ptr(slot_of_expert), _ptr(weights.contiguous()),
                                                float(swiglu_limit), int(fp32_swiglu), int(combine_mode),
                                                _ptr(out), _ptr(h), _ptr(y), _ptr(pos), _ptr(buf), buf.numel(),
                                                _stream())
    check(rc, "locali_moe_expert_grouped_stages")
    order = torch.cat([pos.long(), torch.arange(T * k, routes, device=x2.device)])
    return out.reshape(x.shape), h[order], y[order]


def combine(y: torch.Tensor, weights: torch.Tensor, shared_y=None, mode=COMBINE_ROUNDED):
    T, k, d = y.shape
    out = torch.empty(T, d, dtype=y.dtype, device=y.device)
    rc = lib().locali_moe_combine(_ptr(y.contiguous()), _ptr(shared_y), _ptr(weights.contiguous()),
                                  _dt(y), T, k, d, int(mode), _ptr(out), _stream())
    check(rc, "locali_moe_combine")
    return out


def combine_routes(y: torch.Tensor, route_pos: torch.Tensor, weights: torch.Tensor, out_dtype,
                   shared_y=None, mode=COMBINE_ROUNDED):
    """out[t] = combine over j of y[route_pos[t, j]] (rows skipped where
    route_pos < 0) with weights[t, j], in j order; y rows in fp32, fp16 or
    bf16, out and shared_y in out_dtype (locali_moe_combine_routes)."""
    T, k = route_pos.shape
    d = y.shape[-1]
    out = torch.empty(T, d, dtype=out_dtype, device=y.device)
    if shared_y is not None and shared_y.dtype != out_dtype:
        raise TypeError("shared_y must be in the output dtype")
    rc = lib().locali_moe_combine_routes(_ptr(y.contiguous()), _dt(y), _ptr(route_pos.contiguous()),
                                         _ptr(shared_y), _ptr(weights.contiguous()), DTYPES[out_dtype],
                                         T, k, d, int(mode), _ptr(out), _stream())
    check(rc, "locali_moe_combine_routes")
    return out


def forward(spec: RouterSpec, arena: ExpertArenaT, shared: ExpertArenaT | None,
            slot_of_expert: torch.Tensor, x: torch.Tensor, ws: Workspace, *, input_ids=None,
            swiglu_limit=10.0, fp32_swiglu=False, out=None, idx=None, weights=None):
    """Whole MoE layer (router, dispatch, experts, combine, shared) on an
    all-resident arena. Returns (out, idx, weights)."""
    x2 = _flat(x)
    T, d = x2.shape
    k = spec.top_k
    buf = ws.reserve(T, d, arena.d_ff, spec.n_experts, k, shared is not None)
    out = torch.empty_like(x2) if out is None else out
    idx = torch.empty(T, k, dtype=torch.int32, device=x.device) if idx is None else idx
    weights = torch.empty(T, k, dtype=torch.float32, device=x.device) if weights is None else weights
    ids = None
    if input_ids is not None:
        ids = input_ids.reshape(-1).to(device=x.device, dtype=torch.int32).contiguous()
    r = spec.struct()
    a = arena.struct()
    s = shared.struct() if shared is not None else None
    rc = lib().locali_moe_forward(ctypes.byref(r), ctypes.byref(a),
                                  ctypes.byref(s) if s is not None else None, _ptr(slot_of_expert),
                                  _ptr(x2), _dt(x2), T, _ptr(ids), float(swiglu_limit),
                                  int(fp32_swiglu), _ptr(out), _ptr(idx), _ptr(weights), _ptr(buf),
                                  buf.numel(), _stream())
    check(rc, "locali_moe_forward")
    return out.reshape(x.shape), idx, weights


def arena_fill(dst: torch.Tensor, src: torch.Tensor, stream=None) -> None:
    """Asynchronous host -> HBM copy of src (pinned host tensor) into dst."""
    if src.is_cuda or not dst.is_cuda:
        raise ValueError("arena_fill copies a host tensor into a device tensor")
    nbytes = src.numel() * src.element_size()
    if nbytes != dst.numel() * dst.element_size():
        raise ValueError("arena_fill size mismatch")
    st = stream.cuda_stream if stream is not None else _stream()
    rc = lib().locali_moe_arena_fill(_ptr(dst), ctypes.c_void_p(src.data_ptr()), nbytes, st)
    check(rc, "locali_moe_arena_fill")


def arena_fill_batch_ptrs(pieces, stream) -> None:
    """arena_fill_batch over raw (dst device address, src host address,
    bytes) triples, for callers that keep their own address arithmetic."""
    table = (_lib.FillPiece * max(len(pieces), 1))(*(_lib.FillPiece(d, s, n) for d, s, n in pieces))
    rc = lib().locali_moe_arena_fill_batch(table, len(pieces), stream.cuda_stream)
    check(rc, "locali_moe_arena_fill_batch")


def slot_table(arrays) -> tuple:
    """(dst_base, slot_bytes, n_slots) of slot-major device arrays, in record
    order, for arena_fill_slots (n_slots: the smallest leading dimension)."""
    base = (ctypes.c_void_p * len(arrays))(*(a.data_ptr() for a in arrays))
    per = (ctypes.c_size_t * len(arrays))(*(a[0].numel() * a.element_size() for a in arrays))
    return base, per, min(int(a.shape[0]) for a in arrays)


def arena_fill_slots(table, slots, sources, stream) -> None:
    """Asynchronous fills of whole experts (locali_moe_arena_fill_slots):
    expert i's records lie back to back in host memory at address sources[i]
    and land in slot slots[i] of the arrays of `table` (slot_table). Pinned
    sources go through the copy kernel; the host memory must stay until the
    stream has passed the copy."""
    n = len(slots)
    base, per, n_slots = table
    sl = (ctypes.c_int32 * max(n, 1))(*slots)
    src = (ctypes.c_void_p * max(n, 1))(*sources)
    rc = lib().locali_moe_arena_fill_slots(base, per, len(base), n_slots, sl, src, n, stream.cuda_stream)
    check(rc, "locali_moe_arena_fill_slots")


def arena_fill_batch(pieces, stream=None) -> None:
    """Asynchronous host -> HBM copies of several (dst device tensor, src host
    tensor) pairs in one call: pinned, 16-byte aligned sources go through one
    kernel that reads the host memory directly (locali_moe_arena_fill_batch).
    The host tensors must stay alive until the stream has passed the copy."""
    table = (_lib.FillPiece * max(len(pieces), 1))()
    for i, (dst, src) in enumerate(pieces):
        if src.is_cuda or not dst.is_cuda:
            raise ValueError("arena_fill_batch copies host tensors into device tensors")
        nbytes = src.numel() * src.element_size()
        if nbytes != dst.numel() * dst.element_size():
            raise ValueError("arena_fill_batch size mismatch")
        table[i] = _lib.FillPiece(dst.data_ptr(), src.data_ptr(), nbytes)
    st = stream.cuda_stream if stream is not None else _stream()
    rc = lib().locali_moe_arena_fill_batch(table, len(pieces), st)
    check(rc, "locali_moe_arena_fill_batch")
