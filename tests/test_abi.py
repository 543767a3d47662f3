"""The C-ABI library: builds, loads, exports what include/mlxq.h declares,
and reports errors through status + last-error (no GPU compute here)."""
import os
import re
import subprocess
import sys

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mlxq.h")


def declared_symbols():
    text = open(HEADER).read()
    return set(re.findall(r"^(?:int|const char\*)\s+(mlxq_\w+)\(", text, flags=re.M))


def test_header_declares_the_bound_symbols():
    from mlxq import _lib

    assert declared_symbols() == set(_lib.SYMBOLS)


def test_library_exports_every_declared_symbol():
    from mlxq import _lib

    L = _lib.lib()
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing
    assert L.mlxq_target_arch() == b"gfx950"
    assert L.mlxq_abi_version() == 1


def test_code_object_targets_gfx950():
    """The fat binary of our own build carries a gfx950 code object."""
    blob = open(os.path.join(ROOT, "mlx-bun_amd", "libmlxq.so"), "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


def test_calls_before_init_fail_with_state_error():
    """A fresh process that skips mlxq_init gets MLXQ_ERR_STATE and a message
    (the reference surfaces mlx-c failures as status + recorded message)."""
    code = (
        "import ctypes,sys; L=ctypes.CDLL(sys.argv[1]);"
        "L.mlxq_last_error.restype=ctypes.c_char_p;"
        "p=ctypes.c_void_p(); rc=L.mlxq_malloc(ctypes.byref(p), ctypes.c_uint64(64));"
        "print(rc, L.mlxq_last_error().decode())"
    )
    lib = os.path.join(ROOT, "mlx-bun_amd", "libmlxq.so")
    out = subprocess.run([sys.executable, "-c", code, lib], capture_output=True, text=True, timeout=120)
    rc, msg = out.stdout.strip().split(" ", 1)
    assert rc == "4" and "mlxq_init" in msg


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "mlx-bun_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", text, flags=re.M), f
                assert "liboracle" not in text, f
