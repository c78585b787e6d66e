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
import tempfile
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE = PACKAGE_DIR.parent / "csrc" / "legolink_kv.hip"
# Translation units of liblegolink_kv.so: the link kernels and the repair attention.
SOURCES = (SOURCE, PACKAGE_DIR.parent / "csrc" / "repair_attention.hip")
INCLUDE_DIR = PACKAGE_DIR.parents[1] / "include"
OUTPUT = PACKAGE_DIR / "lib" / "liblegolink_kv.so"
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


def compile_command(output: Path, sources=SOURCES) -> list[str]:
    """One hipcc call that compiles and links ``sources`` into ``output``."""

    sources = [sources] if isinstance(sources, Path) else list(sources)
    return [hipcc_path(), *_flags(), "-shared", "-o", str(output), *[str(source) for source in sources]]


def build_library(verbose: bool = False) -> Path:
    """Compile every translation unit in parallel, then link the library; the
    output is replaced atomically."""

    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(dir=OUTPUT.parent, prefix=".build.") as scratch:
        objects = [Path(scratch) / f"{source.stem}.o" for source in SOURCES]
        jobs = [
            (subprocess.Popen([hipcc_path(), *_flags(), "-c", "-o", str(obj), str(source)],
                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), source)
            for source, obj in zip(SOURCES, objects)
        ]
        failures = []
        for job, source in jobs:
            output, _ = job.communicate()
            messages = _messages(output)
            if job.returncode != 0:
                failures.append(f"hipcc failed on {source.name}:\n" + "\n".join(messages))
            elif verbose and messages:
                print("\n".join(messages), file=sys.stderr)
        if failures:
            raise RuntimeError("\n".join(failures))
        temporary = Path(scratch) / OUTPUT.name
        result = subprocess.run([hipcc_path(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o",
                                 str(temporary), *[str(obj) for obj in objects]],
                                capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError("hipcc link failed:\n" + "\n".join(_messages(result.stdout + result.stderr)))
        os.replace(temporary, OUTPUT)
    return OUTPUT


def _messages(text: str) -> list[str]:
    # hipcc's host pass does not know the packed-fp32 target feature; that
    # warning is expected and harmless.
    return [line for line in text.splitlines() if "packed-fp32-ops" not in line and line.strip()]


if __name__ == "__main__":
    print(build_library(verbose=True))
