"""The C ABI library loads, exports every declared symbol, and validates
arguments on the host (no GPU needed: every case below fails before launch)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_symbols():
    names = []
    for h in HEADERS:
        text = h.read_text()
        names += re.findall(r"^LS_API\s+[\w\s\*]+?\b(ls_\w+)\s*\(", text, flags=re.M)
    return names


def test_header_declares_symbols():
    names = declared_symbols()
    assert "ls_verify_greedy" in names and len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    from longspark_amd import _lib
    lib = _lib.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert set(declared_symbols()) == set(_lib.exported_symbols())


def test_version_and_error_strings():
    from longspark_amd import _lib
    assert b"gfx950" in _lib.lib().ls_version()
    assert isinstance(_lib.lib().ls_last_error(), bytes)


def test_greedy_host_validation_codes():
    from longspark_amd import _lib
    lib = _lib.lib()
    dummy = ctypes.c_void_p(16)
    # width < 2
    st = lib.ls_verify_greedy(dummy, _lib.LS_BF16, 100, dummy, _lib.LS_I32, 16, 1, 1, 4, 1, 100,
                              None, dummy, dummy, None, None, dummy, 1 << 20, dummy, 1 << 20, None)
    assert st == _lib.LS_ERR_SHAPE and b"width" in lib.ls_last_error()
    # row stride smaller than vocab
    st = lib.ls_verify_greedy(dummy, _lib.LS_BF16, 10, dummy, _lib.LS_I32, 16, 1, 1, 4, 16, 100,
                              None, dummy, dummy, None, None, dummy, 1 << 20, dummy, 1 << 20, None)
    assert st == _lib.LS_ERR_SHAPE
    # bad dtype
    st = lib.ls_verify_greedy(dummy, 99, 100, dummy, _lib.LS_I32, 16, 1, 1, 4, 16, 100,
                              None, dummy, dummy, None, None, dummy, 1 << 20, dummy, 1 << 20, None)
    assert st == _lib.LS_ERR_DTYPE
    # workspace too small
    st = lib.ls_verify_greedy(dummy, _lib.LS_BF16, 100, dummy, _lib.LS_I32, 16, 1, 1, 4, 16, 100,
                              None, dummy, dummy, None, None, dummy, 4, dummy, 4, None)
    assert st == _lib.LS_ERR_WORKSPACE
    c, s = _lib.workspace_sizes("ls_verify_greedy_workspace", 128, 16, 151936)
    assert c > 0 and s == 0


def test_python_wrappers_reject_cpu_tensors():
    from longspark_amd import verify
    logits = torch.zeros(32, 100, dtype=torch.bfloat16)
    cand = torch.zeros(2, 16, dtype=torch.int32)
    with pytest.raises(ValueError):
        verify.verify_greedy(logits=logits, candidates=cand, width=16)
