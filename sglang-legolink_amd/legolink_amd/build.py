"""Build ``liblegolink_kv.so`` in-tree with hipcc for gfx950.

    python -m legolink_amd.build            (from sglang-legolink_amd/)

Flags that matter for parity:
  -ffp-contract=off      RoPE products and sums stay separate RNE ops (no FMA)
  -packed-fp32-ops off   no v_pk_*_f32 forms are generated
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE = PACKAGE_DIR.parent / "csrc" / "legolink_kv.hip"
# Translation units of liblegolink_kv.so: the link kernels and the repair attention.
SOURCES = (SOURCE, PACKAGE_DIR.parent / "csrc" / "repair_attention.hip")
INCLUDE_DIR = PACKAGE_DIR.parents[1] / "include"
OUTPUT = PACKAGE_DIR / "lib" / "liblegolink_kv.so"
# The row-access calibration kernels of bench.py's sweep (measurement only,
# not part of the link's C ABI): their own small library.
CALIBRATION_SOURCE = PACKAGE_DIR.parent / "csrc" / "row_calibration.hip"
CALIBRATION_OUTPUT = PACKAGE_DIR / "lib" / "liblegolink_calibration.so"
# The CPython module that converts a link plan's lists to int64 arrays
# (host code only, built with the C compiler against this interpreter).
HOST_SEQUENCES_SOURCE = PACKAGE_DIR.parent / "csrc" / "host_sequences.c"
HOST_SEQUENCES_OUTPUT = PACKAGE_DIR / f"_host_sequences{sysconfig.get_config_var('EXT_SUFFIX')}"
# The same library with its host code under AddressSanitizer and
# UndefinedBehaviorSanitizer (device code unchanged), for the CPU tests of the
# host entries; never loaded on a GPU.
SANITIZED_OUTPUT = PACKAGE_DIR / "lib" / "host_sanitized" / "liblegolink_kv.so"
SANITIZE_FLAGS = ["-g", "-fno-omit-frame-pointer", "-shared-libsan",
                  "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=all"]
OFFLOAD_ARCH = "gfx950"


def hipcc_path() -> str:
    candidate = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(candidate).exists():
        raise FileNotFoundError(f"hipcc not found (looked for {candidate})")
    return candidate


def _flags() -> list[str]:
    return [
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        "-Wall",
        f"-I{INCLUDE_DIR}",
    ]


def build_library(verbose: bool = False, *, sanitize_host: bool = False) -> Path:
    """Compile every translation unit in parallel, then link the library; the
    output is replaced atomically.  ``sanitize_host`` builds the host-sanitized
    copy (SANITIZED_OUTPUT) instead.  The unsanitized build also builds the
    calibration library (CALIBRATION_OUTPUT) and the host module
    (HOST_SEQUENCES_OUTPUT)."""

    output = SANITIZED_OUTPUT if sanitize_host else OUTPUT
    extra = SANITIZE_FLAGS if sanitize_host else []
    output.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(dir=output.parent, prefix=".build.") as scratch:
        objects = [Path(scratch) / f"{source.stem}.o" for source in SOURCES]
        jobs = [
            (subprocess.Popen([hipcc_path(), *_flags(), *extra, "-c", "-o", str(obj), str(source)],
                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), source)
            for source, obj in zip(SOURCES, objects)
        ]
        calibration = None
        if not sanitize_host:
            calibration_tmp = Path(scratch) / CALIBRATION_OUTPUT.name
            calibration = (subprocess.Popen([hipcc_path(), *_flags(), "-shared", "-o", str(calibration_tmp),
                                             str(CALIBRATION_SOURCE)],
                                            stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True),
                           CALIBRATION_SOURCE)
            jobs.append(calibration)
            host_sequences_tmp = Path(scratch) / HOST_SEQUENCES_OUTPUT.name
            compiler = os.environ.get("CC") or shutil.which("gcc") or "cc"
            jobs.append((subprocess.Popen([compiler, "-O2", "-shared", "-fPIC", "-Wall",
                                           f"-I{sysconfig.get_paths()['include']}", "-o", str(host_sequences_tmp),
                                           str(HOST_SEQUENCES_SOURCE)],
                                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True),
                         HOST_SEQUENCES_SOURCE))
        failures = []
        for job, source in jobs:
            printed, _ = job.communicate()
            messages = _messages(printed)
            if job.returncode != 0:
                failures.append(f"compiling {source.name} failed:\n" + "\n".join(messages))
            elif verbose and messages:
                print("\n".join(messages), file=sys.stderr)
        if failures:
            raise RuntimeError("\n".join(failures))
        temporary = Path(scratch) / output.name
        result = subprocess.run([hipcc_path(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *extra,
                                 "-o", str(temporary), *[str(obj) for obj in objects]],
                                capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError("hipcc link failed:\n" + "\n".join(_messages(result.stdout + result.stderr)))
        os.replace(temporary, output)
        if calibration is not None:
            os.replace(calibration_tmp, CALIBRATION_OUTPUT)
            os.replace(host_sequences_tmp, HOST_SEQUENCES_OUTPUT)
    return output


def sanitizer_runtime() -> Path:
    """The AddressSanitizer runtime of the compiler that builds the sanitized
    library (to preload into the process that loads it)."""

    clang = Path(hipcc_path()).resolve().parent.parent / "lib" / "llvm" / "bin" / "clang"
    if not clang.exists():
        clang = Path("/opt/rocm/lib/llvm/bin/clang")
    result = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"],
                            capture_output=True, text=True, check=True)
    runtime = Path(result.stdout.strip())
    if not runtime.is_file():
        raise FileNotFoundError(f"AddressSanitizer runtime not found ({runtime})")
    return runtime


def _messages(text: str) -> list[str]:
    # hipcc's host pass does not know the packed-fp32 target feature; that
    # warning is expected and harmless.
    return [line for line in text.splitlines() if "packed-fp32-ops" not in line and line.strip()]


if __name__ == "__main__":
    print(build_library(verbose=True))
