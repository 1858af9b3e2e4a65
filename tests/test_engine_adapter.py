"""The engine-side drop-in (include/hy3_gpu_moe.h, hy3_amd/engine/): hy3's own
GPU entry points hy3_gpu_init / hy3_gpu_free (hy3_gpu.cu:544,632) and the MoE
forward, compiled as C against the engine's hy3.h and driven by a C program
(tests/engine/adapter_check.c) exactly as the engine calls them. Both are
built by __graft_entry__.build() where the engine's headers are present."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADAPTER = os.path.join(ROOT, "hy3_amd", "engine", "_build", "libhy3gpu_moe.so")
CHECK = os.path.join(ROOT, "tests", "engine", "_build", "adapter_check")
HEADER = os.path.join(ROOT, "include", "hy3_gpu_moe.h")
needs_build = pytest.mark.skipif(
    not (os.path.exists(ADAPTER) and os.path.exists(CHECK)),
    reason="drop-in not built (build() compiles it where the engine's hy3.h is present)")


def run_check(mode, timeout):
    r = subprocess.run([CHECK, mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    print(r.stderr)
    return r


@needs_build
def test_adapter_exports_the_reference_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", ADAPTER], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (\w+)", out))
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    declared = set(re.findall(r"\b(hy3_gpu_\w+)\s*\(", src))
    assert {"hy3_gpu_init", "hy3_gpu_free"} <= declared
    assert declared <= exported, declared - exported


@needs_build
def test_adapter_refuses_malformed_models():
    r = run_check("validate", 60)
    assert r.returncode == 0 and "adapter_check validate: OK" in r.stdout


@pytest.mark.gpu
@needs_build
def test_adapter_forward_equals_library_forward():
    r = run_check("run", 240)
    assert r.returncode == 0 and "adapter_check run: OK" in r.stdout
