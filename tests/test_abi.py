"""The C ABI library without a GPU: it loads, exports every function
include/bark_hip.h declares, and reports errors (no device, bad arguments)
through return codes and bark_hip_last_error() instead of crashing."""
from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "bark_hip.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(bark_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(pkg):
    declared = header_functions()
    assert len(declared) >= 14
    L = pkg.lib()
    for name in declared:
        assert hasattr(L, name), name
    # the Python bindings cover exactly the header
    assert sorted(pkg.HEADER_SYMBOLS) == declared
    out = subprocess.run(["nm", "-D", "--defined-only", str(pkg.lib_path())], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (bark_hip_\w+)", out))
    assert set(declared) <= exported


def test_header_compiles_as_c(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "bark_hip.h"\nint main(void) { return BARK_HIP_OK; }\n')
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", str(ROOT / "include"), "-c", str(src), "-o",
                    str(tmp_path / "t.o")], check=True)


@pytest.mark.skipif(
    subprocess.run([sys.executable, "-c", "import torch,sys; sys.exit(0 if torch.cuda.is_available() else 1)"]).returncode
    == 0,
    reason="a GPU is visible",
)
def test_no_device_is_an_error_not_a_crash(pkg):
    """The Backend::Auto fall-back (src/inference.rs:219-229) needs a failing
    create to come back as an error code."""
    L = pkg.lib()
    assert L.bark_hip_device_count() == 0
    h = ctypes.c_void_p()
    rc = L.bark_hip_create(0, 24, ctypes.byref(h))
    assert rc != 0 and not h.value
    assert L.bark_hip_last_error()
    with pytest.raises(pkg.HipError):
        pkg.HipEncoder(0)


def test_bad_arguments_return_codes(pkg):
    L = pkg.lib()
    h = ctypes.c_void_p()
    assert L.bark_hip_create(0, 0, ctypes.byref(h)) == -1  # n_layers out of range
    assert b"n_layers" in L.bark_hip_last_error()
    assert L.bark_hip_lowbit_linear(None, 0, None, None, None, 0, 1, 64, 128, None) == -1
    assert L.bark_hip_finalize(None) == -1
    L.bark_hip_destroy(None)  # a no-op
    zero = np.zeros(8, np.uint8)
    # shape checks happen before any device access
    rc = L.bark_hip_lowbit_linear(zero.ctypes.data, 0, zero.ctypes.data, zero.ctypes.data, zero.ctypes.data, 0, 1,
                                  100, 128, None)
    assert rc == -1 and b"multiple of 256" in L.bark_hip_last_error()
