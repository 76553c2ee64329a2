"""The build targets gfx950 and nothing else (CPU only, no GPU needed).

The kernels rely on gfx950 specifics -- MFMA shapes, LDS size, the 8-XCD
workgroup mapping and the hardware ordering the cross-workgroup split-K
exchange depends on -- so the recipe must name that one target, every
compile must disable packed-fp32 VALU ops, and a device compile for any other
target must stop at the guard in nibble_common.h.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from nibblegemm_amd import build

HAVE_HIPCC = os.path.exists(build._hipcc()) or shutil.which("hipcc") is not None


def _arch_flags(flags):
    return [f for f in flags if f.startswith("--offload-arch") or f.startswith("--amdgpu-target")]


def test_recipe_names_gfx950_only():
    assert build.ARCH == "gfx950"
    assert _arch_flags(build.HIPCC_FLAGS) == ["--offload-arch=gfx950"]
    i = build.HIPCC_FLAGS.index("-packed-fp32-ops")
    assert build.HIPCC_FLAGS[i - 3:i] == ["-Xclang", "-target-feature", "-Xclang"]


def test_every_hip_source_is_built_and_includes_the_guard():
    on_disk = sorted(f for f in os.listdir(build.CSRC) if f.endswith(".hip"))
    assert sorted(build.HIP_SOURCES) == on_disk
    for src in on_disk:
        with open(os.path.join(build.CSRC, src)) as f:
            text = f.read()
        assert '#include "nibble_common.h"' in text, src


def _device_compile(tmp_path, arch):
    src = tmp_path / "guard.hip"
    src.write_text('#include "nibble_common.h"\n__global__ void k(int* p) { *p = 1; }\n')
    cmd = [build._hipcc(), "-std=c++17", f"--offload-arch={arch}", "--cuda-device-only", "-c",
           "-I", build.CSRC, "-I", build.INCLUDE, str(src), "-o", str(tmp_path / "guard.o")]
    return subprocess.run(cmd, capture_output=True, text=True, timeout=300)


@pytest.mark.skipif(not HAVE_HIPCC, reason="hipcc not installed")
def test_guard_rejects_another_target(tmp_path):
    r = _device_compile(tmp_path, "gfx942")
    assert r.returncode != 0
    assert "built for gfx950 only" in r.stderr


@pytest.mark.skipif(not HAVE_HIPCC, reason="hipcc not installed")
def test_guard_passes_gfx950(tmp_path):
    r = _device_compile(tmp_path, "gfx950")
    assert r.returncode == 0, r.stderr
