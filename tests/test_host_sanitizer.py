"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

Builds the host-sanitized copy of liblegolink_kv.so (device code unchanged,
see ``legolink_amd.build.SANITIZE_FLAGS``), then runs the CPU tests of the
host entries against it in a child process that preloads the sanitizer
runtime: argument validation of the link, map-builder and attention entries,
the run planner, the repair attention planner, and the hostile and
undersized-capacity cases of test_host_hostile_inputs.py.  Any report aborts
the child (``-fno-sanitize-recover``), so a clean exit is the check.

The library is rebuilt only when a source or the public header is newer
than the sanitized build (about a minute of hipcc).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

from legolink_amd import build

REPO_ROOT = Path(__file__).resolve().parents[1]
SANITIZED_TESTS = ("tests/test_native_abi.py", "tests/test_link_maps.py", "tests/test_repair_attention.py",
                   "tests/test_host_hostile_inputs.py")


def _sanitized_library() -> Path:
    output = build.SANITIZED_OUTPUT
    inputs = [*build.SOURCES, build.INCLUDE_DIR / "legolink_kv.h", Path(build.__file__)]
    if not output.is_file() or output.stat().st_mtime < max(path.stat().st_mtime for path in inputs):
        build.build_library(sanitize_host=True)
    return output


# Reads two block records past a one-record array: the sanitized build must
# report it (the check that the run below is live), from the library itself.
_PLANTED_OVERREAD = '''
import ctypes, numpy as np
from legolink_amd import _native
lib = _native.load_library()
maps = open("/proc/self/maps").read()
assert "host_sanitized" in maps and "libclang_rt.asan" in maps, "sanitized build not loaded"
blocks = np.zeros((1, len(_native.BLOCK_FIELDS)), dtype=np.int64)
info = _native.LinkRunPlanInfo()
lib.ll_plan_link_runs(blocks.ctypes.data, 3, None, 0, 0, None, 0, None, None, 0, ctypes.byref(info))
print("not caught")
'''


def _sanitizer_env():
    try:
        runtime = build.sanitizer_runtime()
    except (FileNotFoundError, subprocess.CalledProcessError) as error:
        pytest.skip(f"no AddressSanitizer runtime for hipcc's clang: {error}")
    library = _sanitized_library()
    env = dict(os.environ)
    env.update(
        LEGOLINK_KV_LIBRARY=str(library),
        LD_PRELOAD=" ".join(filter(None, [str(runtime), env.get("LD_PRELOAD", "")])),
        # Python and torch keep allocations alive at exit by design; leaks are
        # not what this run looks for.
        ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:print_summary=1",
        UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
        PYTHONDONTWRITEBYTECODE="1",
        PYTHONPATH=os.pathsep.join([str(REPO_ROOT / "sglang-legolink_amd"), env.get("PYTHONPATH", "")]),
    )
    return env


@pytest.mark.timeout(900)
def test_sanitized_build_reports_an_overread():
    env = _sanitizer_env()
    result = subprocess.run([sys.executable, "-c", _PLANTED_OVERREAD], cwd=REPO_ROOT, env=env,
                            capture_output=True, text=True, timeout=300)
    assert "sanitized build not loaded" not in result.stderr, result.stderr[-3000:]
    assert result.returncode != 0 and "not caught" not in result.stdout
    assert "heap-buffer-overflow" in result.stderr and "ll_plan_link_runs" in result.stderr, result.stderr[-3000:]


@pytest.mark.timeout(900)
def test_host_entries_are_clean_under_asan_and_ubsan():
    env = _sanitizer_env()
    result = subprocess.run(
        [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
         *SANITIZED_TESTS],
        cwd=REPO_ROOT, env=env, capture_output=True, text=True, timeout=840)
    output = result.stdout + result.stderr
    assert "AddressSanitizer" not in output and "runtime error:" not in output, output[-6000:]
    assert result.returncode == 0, output[-6000:]
    assert " passed" in result.stdout, output[-3000:]
