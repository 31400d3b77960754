"""Build and run mfma_clock.hip: the power-limited INT8 MFMA ceiling of the device.

Usage (on a gfx950 box): python -m lynnreal_omni_amd.probes.mfma_clock
Prints, per operand mode, TOPS, the shader clock and the MFMA busy fraction at that clock.
"""
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent


def main() -> int:
    src = HERE / "mfma_clock.hip"
    exe = HERE / "_build" / "mfma_clock"
    exe.parent.mkdir(exist_ok=True)
    if not exe.exists() or exe.stat().st_mtime < src.stat().st_mtime:
        hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
        subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-mllvm", "-amdgpu-mfma-vgpr-form",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)]).returncode


if __name__ == "__main__":
    sys.exit(main())
