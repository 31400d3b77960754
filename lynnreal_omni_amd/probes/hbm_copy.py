"""Build and run hbm_copy.hip: the practical HBM streaming ceiling of the device.

Usage (on a gfx950 box): python -m lynnreal_omni_amd.probes.hbm_copy
Prints, per copy variant, the median cold-cache time of a 512 MiB copy and its
read + write rate against the 8 TB/s peak.
"""
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent


def main() -> int:
    src = HERE / "hbm_copy.hip"
    exe = HERE / "_build" / "hbm_copy"
    exe.parent.mkdir(exist_ok=True)
    if not exe.exists() or exe.stat().st_mtime < src.stat().st_mtime:
        hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
        subprocess.run([hipcc, "--offload-arch=gfx950", "-O3",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)]).returncode


if __name__ == "__main__":
    sys.exit(main())
