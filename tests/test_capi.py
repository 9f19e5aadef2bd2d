"""CPU checks of the boundary: the C-ABI library loads and exports every symbol include/mechta_kv.h declares, and
the host-side code needs no GPU (rope_table, error reporting). No compute call is made here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import mechta_amd as mk
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mechta_kv.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mkv_[a-z_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = mk.lib()
    names = declared_symbols()
    assert len(names) >= 18
    for name in names:
        assert hasattr(lib, name), f"{name} missing from {mk.LIB_PATH}"
    assert sorted(mk.SYMBOLS) == names
    out = subprocess.run(["nm", "-D", "--defined-only", mk.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (mkv_\w+)", out))
    assert set(names) <= exported


def test_header_compiles_as_c():
    r = subprocess.run(["gcc", "-fsyntax-only", "-Wall", "-Werror", "-x", "c", HEADER], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("pos", [0, 1, 7, 4095, 65536, 262143])
def test_host_rope_table_matches_oracle(pos):
    """The library's host rope_table and the oracle's are the same f32 recurrence on the same libm: bit-equal."""
    got = np.array(mk.rope_table(pos), np.float32)
    assert np.array_equal(got, O.rope_table(pos))


def test_errors_without_gpu():
    lib = mk.lib()
    h = ctypes.c_void_p()
    assert lib.mkv_create(ctypes.byref(h), 1, 5000, mk.F16, None) == mk.E_CTX
    assert b"multiple of 1024" in lib.mkv_last_error()
    assert lib.mkv_create(ctypes.byref(h), 1, 4096, 7, None) == mk.E_ARG
    assert lib.mkv_create(None, 1, 4096, mk.F16, None) == mk.E_ARG
    assert lib.mkv_decode(None, 0, None, 1, 1, 0, 1.0, None, None) == mk.E_ARG
    assert lib.mkv_snapshot_bytes(None, 10) == 0
