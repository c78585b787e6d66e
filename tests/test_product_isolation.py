"""The product package stands alone: it never loads the oracle (test
infrastructure), and without its HIP library it fails loudly instead of
falling back to any CPU path."""

from __future__ import annotations

import ast
import os
import subprocess
import sys
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parents[1]
PACKAGE = REPO_ROOT / "sglang-legolink_amd" / "legolink_amd"


def test_no_product_source_imports_the_oracle():
    for path in sorted(PACKAGE.glob("*.py")):
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                names = [alias.name for alias in node.names]
            elif isinstance(node, ast.ImportFrom):
                names = [node.module or ""]
            else:
                continue
            assert not any(name == "oracle" or name.startswith("oracle.") for name in names), path.name


def _run(code: str, **env) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, "-c", code], cwd=REPO_ROOT, capture_output=True, text=True,
                          env={**os.environ, "PYTHONPATH": str(REPO_ROOT / "sglang-legolink_amd"), **env},
                          timeout=300)


def test_importing_every_product_module_loads_no_oracle_module():
    modules = [path.stem for path in sorted(PACKAGE.glob("*.py")) if path.stem != "__init__"]
    code = ("import sys, importlib\n"
            f"for name in {modules!r}:\n"
            "    importlib.import_module('legolink_amd.' + name)\n"
            "loaded = [m for m in sys.modules if m == 'oracle' or m.startswith('oracle.')]\n"
            "print('LOADED', loaded)\n")
    result = _run(code)
    assert result.returncode == 0, result.stderr[-2000:]
    assert "LOADED []" in result.stdout, result.stdout


def test_missing_library_fails_loudly():
    code = ("from legolink_amd import _native\n"
            "try:\n"
            "    _native.load_library()\n"
            "except _native.NativeLibraryUnavailable as error:\n"
            "    print('UNAVAILABLE', error)\n"
            "else:\n"
            "    print('LOADED')\n")
    result = _run(code, LEGOLINK_KV_LIBRARY=str(REPO_ROOT / "no-such-dir" / "liblegolink_kv.so"))
    assert result.returncode == 0, result.stderr[-2000:]
    assert "UNAVAILABLE" in result.stdout and "not built" in result.stdout, result.stdout
