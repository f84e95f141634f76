"""The C ABI boundary: liblocali_amd.so loads on a host without a GPU and
exports every function include/*.h declares, the Python bindings cover all of
them, and argument checking fails loudly (no compute call is made here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from locali_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
DECL = re.compile(r"^\s*(?:LOCALI_API\s+)?[A-Za-z_][\w\s\*]*?\b(locali_\w+)\s*\(", re.M)


def declared() -> set[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in DECL.finditer(text):
            names.add(m.group(1))
    return names


def test_headers_declare_the_planner_and_gpu_entry_points():
    names = declared()
    planner = {"locali_cache_create", "locali_cache_create_policy", "locali_cache_destroy",
               "locali_cache_note_token", "locali_cache_plan", "locali_cache_peek",
               "locali_cache_probation_size", "locali_cache_protected_size"}
    assert planner <= names
    assert {"locali_moe_router", "locali_moe_dispatch", "locali_moe_expert_decode",
            "locali_moe_expert_grouped", "locali_moe_combine", "locali_moe_arena_fill",
            "locali_moe_arena_fill_batch",
            "locali_moe_forward", "locali_moe_workspace_bytes"} <= names


def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(declared()) if not hasattr(handle, n)]
    assert not missing, f"declared in include/*.h but not exported: {missing}"


def test_python_bindings_cover_the_headers():
    assert declared() == set(_lib.EXPORTS)


def test_argument_errors_are_reported_without_a_gpu():
    lib = _lib.lib()
    rc = lib.locali_moe_dispatch(None, -1, 6, 257, None, None, None)
    assert rc == -1
    assert lib.locali_moe_last_error().startswith(b"dispatch:")


def test_empty_batch_returns_without_touching_anything():
    """tokens == 0 is a no-op that succeeds (no pointer is read, no GPU is
    needed)."""
    lib = _lib.lib()
    assert lib.locali_moe_dispatch(None, 0, 6, 257, None, None, None) == 0
    assert lib.locali_moe_combine(None, None, None, 2, 0, 6, 4096, 0, None, None) == 0


def test_workspace_size_is_positive_and_monotone():
    lib = _lib.lib()
    a = lib.locali_moe_workspace_bytes(1, 4096, 2048, 256, 6, 1)
    b = lib.locali_moe_workspace_bytes(64, 4096, 2048, 256, 6, 1)
    assert 0 < a < b
    assert lib.locali_moe_workspace_bytes(0, 4096, 2048, 256, 6, 1) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.LocaliError):
        _lib.lib()


@pytest.mark.parametrize("slot", [-1, 97, 1 << 30])
def test_fill_slots_refuses_a_slot_outside_the_arena(slot):
    """A slot outside [0, n_slots) is an argument error, reported before any
    copy is queued (the pointers are never dereferenced, so fakes do)."""
    lib = _lib.lib()
    n_arrays, n_slots = 9, 97
    base = (ctypes.c_void_p * n_arrays)(*([0x1000] * n_arrays))
    per = (ctypes.c_size_t * n_arrays)(*([4096] * n_arrays))
    slots = (ctypes.c_int32 * 2)(3, slot)
    src = (ctypes.c_void_p * 2)(0x2000, 0x3000)
    rc = lib.locali_moe_arena_fill_slots(base, per, n_arrays, n_slots, slots, src, 2, None)
    assert rc == -1
    assert b"outside [0, 97)" in lib.locali_moe_last_error()
