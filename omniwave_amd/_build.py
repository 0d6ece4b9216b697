"""Builds libomniwave_amd.so in-tree with hipcc for gfx950.

The library is a plain C-ABI shared object (include/omniwave_amd.h): host route tables
(route.cpp) and the HIP kernels + launchers (bigemm_fwd.hip).  It is written next to this
file so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libomniwave_amd.so"
SOURCES = ["route.cpp", "bigemm_fwd.hip", "bigemm_fwd_resident.hip", "bigemm_fwd_wave16.hip", "bigemm_fwd_persist.hip", "bigemm_fwd_f32.hip", "bigemm_bwd.hip", "bigemm_bwd_f32.hip", "stem.hip", "fwd_noalloc.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")
    return found


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        # Packed-FP32 VALU ops stay off: scalar float code only.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA accumulators in VGPRs: the SiLU and epilogue read them with VALU instructions.
        "-mllvm", "-amdgpu-mfma-vgpr-form=1",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def build(verbose: bool = False) -> Path:
    """Compile every source into LIB_PATH (always recompiles); returns the library path."""
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="ow_build_") as tmp:
        objs = [str(Path(tmp) / (Path(src).stem + ".o")) for src in SOURCES]
        cmds = [[cc, *compile_flags(), "-c", str(CSRC / src), "-o", obj] for src, obj in zip(SOURCES, objs)]
        if verbose:
            for cmd in cmds:
                print(" ".join(cmd), flush=True)
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
            for fut in [pool.submit(_run, cmd) for cmd in cmds]:
                fut.result()
        out_tmp = Path(tmp) / LIB_PATH.name
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(out_tmp)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        staged = LIB_PATH.with_suffix(".so.tmp")
        shutil.copyfile(out_tmp, staged)
        os.replace(staged, LIB_PATH)
    return LIB_PATH


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "is not a recognized feature for this target"
        stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
        raise RuntimeError(f"build failed ({proc.returncode}): {' '.join(cmd)}\n{stderr}")


if __name__ == "__main__":
    print(build(verbose=True))
