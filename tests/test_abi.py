"""The C-ABI library: it loads, and exports exactly what the header declares.
No compute calls (these run without a GPU)."""

import ctypes
import os
import re
import subprocess
import sys

import pytest

from enilnets_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "enilnets_amd.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(enq_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_reports_abi_version():
    lib = _lib.load()
    declared = int(re.search(r"#define ENQ_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.enq_abi_version() == declared


def test_every_declared_function_is_exported_and_bound():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(_lib.SIGNATURES) == names


def test_no_undeclared_exports():
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = sorted({line.split()[-1] for line in out.splitlines()
                       if line.split()[-1].startswith("enq_")})
    assert exported == header_functions()


def test_calls_before_init_fail_with_no_device_status():
    # in a fresh process: nothing initialised, so no HIP call is made
    code = (
        "import ctypes, sys\n"
        f"lib = ctypes.CDLL({str(_lib.LIB_PATH)!r})\n"
        "lib.enq_last_error.restype = ctypes.c_char_p\n"
        "st = lib.enq_synchronize()\n"
        "print(st, lib.enq_last_error().decode())\n")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=60)
    status, _, msg = out.stdout.strip().partition(" ")
    assert int(status) == _lib.ERR_NO_DEVICE
    assert "enq_init" in msg


def test_status_mapping():
    assert _lib._EXC[_lib.ERR_INVALID] is ValueError
    assert _lib._EXC[_lib.ERR_RUNTIME] is RuntimeError
    assert _lib._EXC[_lib.ERR_NO_DEVICE] is RuntimeError
    assert _lib._EXC[_lib.ERR_UNSUPPORTED] is NotImplementedError


def test_activation_codes_match_header():
    text = open(HEADER).read()
    for name, code in _lib.ACTIVATIONS.items():
        m = re.search(rf"#define ENQ_ACT_{name.upper()} (\d+)", text)
        assert m and int(m.group(1)) == code
