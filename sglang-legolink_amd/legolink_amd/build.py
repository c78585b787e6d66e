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


def compile_command(output: Path, sources=SOURCES) -> list[str]:
    sources = [sources] if isinstance(sources, Path) else list(sources)
    return [
        hipcc_path(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-ffp-contract=off",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        "-Wall",
        f"-I{INCLUDE_DIR}",
        "-o",
        str(output),
        *[str(source) for source in sources],
    ]


def build_library(verbose: bool = False) -> Path:
    """Compile the link library; the output is replaced atomically."""

    _compile(SOURCES, OUTPUT, verbose)
    return OUTPUT


def _compile(sources, output: Path, verbose: bool) -> None:
    output.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.NamedTemporaryFile(
        dir=output.parent, prefix=f".{output.stem}.", suffix=".so.tmp", delete=False
    ) as handle:
        temporary = Path(handle.name)
    command = compile_command(temporary, sources)
    try:
        result = subprocess.run(command, capture_output=True, text=True)
        # hipcc's host pass does not know the packed-fp32 target feature; that
        # warning is expected and harmless.
        messages = [
            line
            for line in (result.stdout + result.stderr).splitlines()
            if "packed-fp32-ops" not in line and line.strip()
        ]
        if result.returncode != 0:
            raise RuntimeError(
                "hipcc failed:\n" + " ".join(command) + "\n" + "\n".join(messages)
            )
        if verbose and messages:
            print("\n".join(messages), file=sys.stderr)
        os.replace(temporary, output)
    finally:
        if temporary.exists():
            temporary.unlink()


if __name__ == "__main__":
    print(build_library(verbose=True))
