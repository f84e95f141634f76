"""CPU oracle for the streamed-MoE hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import anything from this package, and only as the checker (or, for
the baseline, as the CPU stand-in that is timed beside the GPU). The product
package ``locali_amd`` never imports it and has no CPU fallback.

Modules:
  scheduler   pure-Python restatement of the SLRU / LFU-decay slot planner
              (reference native/locali_core.c:39-325, tests/test_locali_native.py:11-62)
  affine      numpy affine 2/4/8-bit pack / unpack / dequant / qmv
              (MLX affine layout used by reference dsv4_kernels.py:21-97)
  moe         router, expert pipeline (clamped SwiGLU), combine and dispatch
              restated from reference dsv4_arena.py:146-235 and arena.py:460-681
  cref        ctypes wrapper of expert_ref.c, an independent C restatement of
              the expert arithmetic (OpenMP) used for large sizes and as the
              CPU baseline
"""
