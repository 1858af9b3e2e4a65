"""The C ABI: every function include/hy3x_moe.h declares is exported by
libhy3x.so; the header compiles as C and C++; argument errors are reported as
codes without touching a GPU. CPU only."""
import ctypes
import os
import re
import subprocess

import pytest

import hy3_amd as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hy3x_moe.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hy3x_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("hy3x_layer_create", "hy3x_layer_forward", "hy3x_layer_set_expert_q4k",
              "hy3x_layer_set_router", "hy3x_layer_destroy", "hy3x_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(H.lib_path)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.parametrize("lang,flags", [("c", ["-std=c99"]), ("c++", ["-std=c++11"])])
def test_header_compiles(lang, flags, tmp_path):
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text('#include "hy3x_moe.h"\nint main(void){return HY3X_OK;}\n')
    cc = "gcc" if lang == "c" else "g++"
    r = subprocess.run([cc, *flags, "-Wall", "-Werror", "-fsyntax-only",
                        "-I", os.path.dirname(HEADER), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_argument_errors_are_codes():
    lib = H.lib()
    assert lib.hy3x_layer_create(None, 4) == -1
    h = ctypes.c_void_p()
    assert lib.hy3x_layer_create(ctypes.byref(h), 0) == -1
    assert b"max_tokens" in lib.hy3x_last_error()
    assert lib.hy3x_layer_forward(None, None, 1, 8, 2.826, None) == -1
    assert lib.hy3x_layer_set_router(None, None, None, None) == -1
    assert lib.hy3x_layer_set_expert_q4k(None, 0, None, None, None, 0) == -1
    assert lib.hy3x_layer_destroy(None) == 0
    assert lib.hy3x_synth_quantize_q4k(None, None, 100, None) == -1


def test_python_binding_has_no_fallback(monkeypatch, tmp_path):
    monkeypatch.setattr(H, "lib_path", str(tmp_path / "missing.so"))
    monkeypatch.setattr(H, "_lib", None)
    with pytest.raises(H.HY3XError):
        H.lib()


def test_stage_index_is_a_permutation():
    # the pair-staged activation layout (hy3x_common.h) visits every slot once
    def stage_index(i):
        g, r = i >> 6, i & 63
        hi, l = r >> 5, r & 31
        j, e = l >> 2, l & 3
        return g * 64 + 2 * (4 * j + hi + ((e & 1) << 1)) + (e >> 1)
    idx = [stage_index(i) for i in range(4096)]
    assert sorted(idx) == list(range(4096))
