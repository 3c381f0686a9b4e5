"""CPU-side checks of the C-ABI boundary: the built library loads and exports every function include/*.h declares,
the Python host mirror declares a signature for each, and the size rules hold. No GPU call is made."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(amv_[a-z0-9_]+)\s*\(", text, re.M):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    from ameva_compute_amd import _lib
    lib = _lib.lib()
    names = header_functions()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_sizes_match_ggml_nbytes():
    from ameva_compute_amd import _lib
    lib = _lib.lib()
    assert lib.amv_version() >= 100
    for t, be, bb in ((2, 32, 18), (8, 32, 34), (12, 256, 144), (14, 256, 210)):
        assert lib.amv_weight_bytes(t, 14336, 4096) == 14336 * 4096 // be * bb
        assert lib.amv_weight_bytes(t, 3, be) == 3 * bb
        assert lib.amv_weight_bytes(t, 1, be + 1) == -1
    assert lib.amv_act_bytes(8, 1, 4096) == 4096 + 128 * 8
    assert lib.amv_act_bytes(15, 2, 4096) == 2 * 4096 + 2 * 16 * 4 + 2 * 256 * 4


def test_argument_errors_fail_fast_without_gpu():
    """Invalid shapes are rejected on the host before any launch, with a message (the reference's FAIL-FAST)."""
    from ameva_compute_amd import _lib
    lib = _lib.lib()
    rc = lib.amv_mul_mat_vec(2, None, 16, 4096, None, 1, None, 16, None)
    assert rc == -1 and b"null" in lib.amv_last_error()
    rc = lib.amv_mul_mat_vec(3, ctypes.c_void_p(16), 16, 4096, ctypes.c_void_p(16), 1, ctypes.c_void_p(16), 16, None)
    assert rc == -2 and b"not supported" in lib.amv_last_error()
    rc = lib.amv_quantize_act(8, ctypes.c_void_p(16), 1, 33, 0, None, ctypes.c_void_p(16), None)
    assert rc == -1 and b"k % 32" in lib.amv_last_error()


def test_product_never_imports_the_oracle():
    for path in glob.glob(os.path.join(ROOT, "ameva_compute_amd", "**", "*.py"), recursive=True):
        src = open(path).read()
        assert "import oracle" not in src and "from oracle" not in src, path
    for path in glob.glob(os.path.join(ROOT, "ameva_compute_amd", "csrc", "*")):
        assert "orc_" not in open(path).read(), path
