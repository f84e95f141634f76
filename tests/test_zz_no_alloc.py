"""locali_moe_forward_noalloc through the C ABI: the whole-layer forward with
its scratch in the library's static per-GPU array against locali_moe_forward
with a caller workspace. The same kernels run on the same inputs, so outputs,
routes and weights must be identical bit for bit: for two calls in a row, the
second smaller than the first (what the first left in the shared array must
not leak into the second), on the full-width layer (d_model 4096, 256 experts
+ shared, d_ff 2048, 2-bit g64 bf16) and on the small fp16 layer; and a call
that needs more scratch than the array holds is refused before any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from gpu_helpers import banner
from locali_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _noalloc(spec, arena, shared, slot_of, x):
    """One call of locali_moe_forward_noalloc by ctypes; (rc, out, idx, weights)."""
    T = x.shape[0]
    k = spec.top_k
    out = torch.empty_like(x)
    idx = torch.empty(T, k, dtype=torch.int32, device=DEV)
    wts = torch.empty(T, k, dtype=torch.float32, device=DEV)
    r, a = spec.struct(), arena.struct()
    s = shared.struct() if shared is not None else None
    rc = _lib.lib().locali_moe_forward_noalloc(
        ctypes.byref(r), ctypes.byref(a), ctypes.byref(s) if s is not None else None, slot_of.data_ptr(),
        x.data_ptr(), ops.DTYPES[x.dtype], T, None, 10.0, 0, out.data_ptr(), idx.data_ptr(),
        wts.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return rc, out, idx, wts


@pytest.mark.parametrize("shape", ["full_width", "small_fp16"])
def test_noalloc_forward_equals_workspace_forward(shape):
    if shape == "full_width":
        d, E, dff, bits, dtype, calls = 4096, 256, 2048, 2, torch.bfloat16, (64, 1)
    else:
        d, E, dff, bits, dtype, calls = 1024, 32, 512, 4, torch.float16, (8, 2)
    banner(f"forward_noalloc {shape} calls {calls}")
    arena = synth.expert_arena(E + 1, d, dff, bits_gate_up=bits, dtype=dtype, seed=71, device=DEV)
    shared = synth.expert_arena(1, d, dff, bits_gate_up=bits, dtype=dtype, seed=72, device=DEV,
                                zero_slot=False)
    w, bias = synth.uniform_router(E, d, dtype, seed=73, device=DEV, bias_std=0.01)
    spec = ops.RouterSpec(w, 6, routed_scale=1.5, score_bias=bias)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    for i, T in enumerate(calls):
        x = synth.activations(T, d, dtype, seed=74 + i, device=DEV)
        rc, out, idx, wts = _noalloc(spec, arena, shared, slot_of, x)
        _lib.check(rc, "locali_moe_forward_noalloc")
        ref, ridx, rw = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace())
        torch.cuda.synchronize()
        assert torch.equal(idx, ridx) and torch.equal(wts, rw), f"call {i} (T={T}) routes"
        assert torch.equal(out, ref), f"call {i} (T={T}) output"


def test_noalloc_refuses_more_than_its_scratch():
    banner("forward_noalloc size limit")
    d, E, dff = 4096, 256, 2048
    arena = synth.expert_arena(3, d, dff, dtype=torch.bfloat16, seed=75, device=DEV)
    w, _ = synth.uniform_router(E, d, torch.bfloat16, seed=76, device=DEV)
    spec = ops.RouterSpec(w, 6, routed_scale=1.5)
    slot_of = torch.zeros(E, dtype=torch.int32, device=DEV)
    T = 128                                   # needs about 31.7 MiB of scratch
    assert ops.workspace_bytes(T, d, dff, E, 6, False) > (16 << 20)
    x = torch.zeros(T, d, dtype=torch.bfloat16, device=DEV)
    rc, *_ = _noalloc(spec, arena, None, slot_of, x)
    assert rc == -2
    assert b"static scratch holds" in _lib.lib().locali_moe_last_error()


def _capture_first_main():
    """Body of test_noalloc_first_call_under_graph_capture, run in a fresh
    process so that the library's first noalloc call on the device (the
    scratch lookup and its clear) happens while a graph is being captured."""
    torch.cuda.set_device(0)
    d, E, dff = 4096, 256, 2048
    arena = synth.expert_arena(E + 1, d, dff, dtype=torch.bfloat16, seed=81, device=DEV)
    shared = synth.expert_arena(1, d, dff, dtype=torch.bfloat16, seed=82, device=DEV, zero_slot=False)
    w, bias = synth.uniform_router(E, d, torch.bfloat16, seed=83, device=DEV, bias_std=0.01)
    spec = ops.RouterSpec(w, 6, routed_scale=1.5, score_bias=bias)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    xs = [synth.activations(1, d, torch.bfloat16, seed=84 + i, device=DEV) for i in range(3)]
    x = xs[0].clone()
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        rc, out, idx, wts = _noalloc(spec, arena, shared, slot_of, x)
    _lib.check(rc, "locali_moe_forward_noalloc (captured)")
    for rep, xi in enumerate(xs):
        x.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        ref, ridx, rw = ops.forward(spec, arena, shared, slot_of, xi, ops.Workspace())
        torch.cuda.synchronize()
        assert torch.equal(idx, ridx) and torch.equal(wts, rw), f"replay {rep} routes"
        assert torch.equal(out, ref), f"replay {rep} output"
        # an eager noalloc call between replays shares the same scratch
        rc2, out2, _, _ = _noalloc(spec, arena, shared, slot_of, xi)
        _lib.check(rc2, "locali_moe_forward_noalloc (eager)")
        torch.cuda.synchronize()
        assert torch.equal(out2, ref), f"eager call after replay {rep}"
    print("capture-first ok", flush=True)


def test_noalloc_first_call_under_graph_capture():
    """The first noalloc call of a process made inside torch.cuda.graph
    capture: every replay (inputs changed between replays, an eager noalloc
    call after each) equals the workspace forward bit for bit."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    banner("forward_noalloc first call under graph capture (fresh process)")
    here = Path(__file__).resolve().parent
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([str(here.parent), str(here)]))
    proc = subprocess.run([sys.executable, "-c", "import test_zz_no_alloc as t; t._capture_first_main()"],
                          cwd=here, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=110)
    assert proc.returncode == 0 and "capture-first ok" in proc.stdout, proc.stdout[-3000:]
