"""Helpers shared by the GPU parity tests: torch arenas -> oracle numpy form,
tolerance checks and a one-line case banner printed before each GPU step."""

from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import affine

# North-star tolerance for expert outputs (bf16 against the fp32/fp64 oracle).
RTOL, ATOL = 1e-2, 2e-3


def banner(msg: str) -> None:
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def dt_name(dtype) -> str:
    return {torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]


def proj_numpy(p, float_meta: bool, slots=None):
    """ProjArena -> (w uint32, scales, biases, bits, group) on the host; scales
    and biases as float64 values (numpy oracle) or uint16 bits (C oracle).
    `slots` selects arena slots on the device before the copy."""
    w, s, b = p.weight, p.scales, p.biases
    if slots is not None:
        sel = torch.as_tensor(slots, dtype=torch.long, device=w.device)
        w, s, b = w[sel], s[sel], b[sel]
    w = w.detach().cpu().contiguous().view(torch.int32).numpy().view(np.uint32)
    if float_meta:
        s = s.detach().cpu().double().numpy()
        b = b.detach().cpu().double().numpy()
    else:
        s = s.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
        b = b.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    return w, s, b, p.bits, p.group_size


def arena_numpy(arena, float_meta=True, slots=None):
    return {name: proj_numpy(p, float_meta, slots)
            for name, p in (("gate_proj", arena.gate), ("up_proj", arena.up), ("down_proj", arena.down))}


def values(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_close(got, want, what, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {bad.sum()} / {bad.size} outside rtol={rtol} atol={atol}; first at {tuple(i)}: "
            f"got {got[tuple(i)]!r} want {want[tuple(i)]!r}")


def assert_close_terms(got, want, terms, what, rtol=RTOL, atol=ATOL):
    """Combined outputs are sums of terms each rounded to 16 bits; one
    last-place flip of a term of magnitude m moves the result by up to
    2^-7 m (bf16 spacing, a superset of fp16's). The bound adds that to the
    stated tolerance (1e-2 rel, 2e-3 abs), with terms = sum of |rounded term| per element."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    tol = atol + rtol * np.abs(want) + 2.0 ** -7 * np.asarray(terms, dtype=np.float64)
    bad = np.abs(got - want) > tol
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {bad.sum()} / {bad.size} outside the term-rounding bound; first at {tuple(i)}: "
            f"got {got[tuple(i)]!r} want {want[tuple(i)]!r} terms {np.asarray(terms)[tuple(i)]!r}")


def exact_fraction(got, want) -> float:
    return float(np.mean(np.asarray(got) == np.asarray(want)))


def ulp(v, dtype) -> np.ndarray:
    """Spacing of the 16-bit format at |v| (bf16: 8 significant bits, fp16:
    11), subnormal spacing below the smallest normal."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    if dtype == torch.bfloat16:
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
        return 2.0 ** (e - 7)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def ulp_distance(got, want, dtype) -> np.ndarray:
    """|got - want| in units of the format's spacing at want (a value one
    rounding step away from want, on either side, is at distance 1 or less:
    at a power of two the spacing below is half the one above)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return np.abs(got - want) / ulp(want, dtype)
