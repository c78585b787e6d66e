"""The benchmark's ctypes mirror of the row-calibration library (CPU: the
library loads and reports its argument struct size without a GPU), and the
argument checks that run before any launch."""

from __future__ import annotations

import ctypes
import importlib.util
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", REPO / "bench.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_argument_struct_matches_the_library():
    bench = _bench()
    calibration = bench._RowCalibration(torch)  # raises if the sizes differ
    assert calibration.lib.llc_row_args_size() == ctypes.sizeof(calibration.Args)


@pytest.mark.parametrize("change, message", [
    (dict(buffers=4), b"buffers must be 0..3"),
    (dict(mode=1, buffers=1), b"read only moves both buffers"),
    (dict(mode=2, buffers=2), b"write only moves both buffers"),
    (dict(row_bytes=512), b"row_bytes must be a positive multiple of 1024"),
    (dict(layer_major=1, tokens_per_wave=3), b"tokens_per_wave must be even and divide num_tokens"),
])
def test_bad_arguments_are_refused_before_a_launch(change, message):
    bench = _bench()
    calibration = bench._RowCalibration(torch)
    layers = (ctypes.c_void_p * 2)(1, 2)
    fields = dict(struct_size=ctypes.sizeof(calibration.Args), num_layers=2, key_layers=ctypes.addressof(layers),
                  value_layers=ctypes.addressof(layers), num_slots=16, row_bytes=1024, num_tokens=4,
                  source_slots=8, destination_slots=8, mode=0, layer_major=0, layers_per_wave=2,
                  tokens_per_wave=0, lds_bytes=0, sink=8, buffers=3)
    fields.update(change)
    args = calibration.Args(**fields)
    assert calibration.lib.llc_rows(ctypes.byref(args), None) != 0
    assert message in calibration.lib.llc_last_error()
