"""The C-ABI library loads on a host without a GPU and exports every entry
point ``include/kairyu_quant.h`` declares (no compute calls here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from kairyu_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "kairyu_quant.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|int64_t|const char\*|size_t)\s+(kq_\w+)\s*\(", text, re.M))


def test_header_declarations_are_bound():
    declared = declared_symbols()
    assert declared, "no declarations parsed"
    assert declared == set(_native.exported_symbols())


def test_library_loads_and_exports_every_symbol():
    lib = _native.library()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.kq_version() >= 100
    assert isinstance(lib.kq_last_error(), bytes)


def test_exported_symbols_in_dynamic_table():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(kq_\w+)", out))
    assert declared_symbols() <= exported


def test_tiled_operand_size():
    lib = _native.library()
    # tiles (2 units x 2 stages x 256 words) + table (2 units x 3 group pairs x 32)
    assert lib.kq_w4a16_tiled_words(24, 256, 48, 0) == 2 * 2 * 256 + 2 * 3 * 32
    assert lib.kq_w4a16_tiled_words(28672, 4096, 128, 0) == 1792 * 32 * 256 + 1792 * 16 * 32
    # one zero: scale-only table (16 words per unit and pair) + groups x n/8 zero words
    assert lib.kq_w4a16_tiled_words(24, 256, 48, 1) == 2 * 2 * 256 + 2 * 3 * 16 + 6 * 3
    assert (lib.kq_w4a16_tiled_words(28672, 4096, 128, 1)
            == 1792 * 32 * 256 + 1792 * 16 * 16 + 32 * 3584)
    assert lib.kq_w4a16_tiled_words(20, 256, 128, 0) == -1  # n % 8
    assert lib.kq_w4a16_tiled_words(24, 256, 12, 0) == -1   # group % 8


def test_bad_shapes_fail_closed_without_touching_the_device():
    # validation happens on the host before any launch: negative / zero sizes
    with pytest.raises(ValueError, match="bad shape"):
        _native.call("kq_w8a8_i8_gemm", None, None, None, None, None, -1, None, 0, None,
                     -1, 4, 4, None, 0, None)
    with pytest.raises(RuntimeError, match="fp16 or bf16"):
        _native.call("kq_act_quant_i8", None, 2, 1, 8, 8, None, None, None)
    with pytest.raises(ValueError, match="gidx_mode"):
        _native.call("kq_w4a16_gptq_gemm", None, 0, None, None, None, None, None, 7, None, -1,
                     None, 1, 8, 8, 8, None, 0, None)


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setenv("KAIRYU_AMD_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _native.library()
    monkeypatch.delenv("KAIRYU_AMD_LIB")
    monkeypatch.setattr(_native, "_lib", None)
    assert isinstance(_native.library(), ctypes.CDLL)
