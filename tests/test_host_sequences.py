"""The C conversions of a link plan's lists (CPU): the same values and the
same errors as the Python conversions they replace."""

from __future__ import annotations

from collections import OrderedDict

import numpy as np
import pytest

from legolink_amd import _host_sequences
from legolink_amd.link_runtime import _index_array, _range_bounds


def test_integers_of_a_list_or_tuple():
    rng = np.random.default_rng(4)
    values = rng.integers(-(1 << 62), 1 << 62, size=5000).tolist() + [0, -1, (1 << 63) - 1, -(1 << 63)]
    for sequence in (values, tuple(values)):
        out = np.full(len(values) + 3, 7, dtype=np.int64)
        assert _host_sequences.int64_from_sequence(sequence, out) == len(values)
        assert out[: len(values)].tolist() == values and out[len(values):].tolist() == [7, 7, 7]
    assert _index_array(values).tolist() == values
    assert _index_array([]).dtype == np.int64 and _index_array([]).size == 0


def test_integer_like_entries_and_fallbacks():
    # numpy integers and bools convert through __index__, as with array.array.
    mixed = [np.int32(5), np.int64(-3), True, 9]
    assert _index_array(mixed).tolist() == [5, -3, 1, 9]
    # Floats are not integers: the general conversion truncates them, as before.
    assert _index_array([1.0, 2.7]).tolist() == [1, 2]
    with pytest.raises(TypeError):
        _host_sequences.int64_from_sequence([1, 2.5], np.empty(2, dtype=np.int64))
    with pytest.raises(OverflowError):
        _index_array([1 << 63])
    # Arrays, tensors and generators take the general path.
    assert _index_array(np.array([3, 1], dtype=np.int32)).tolist() == [3, 1]
    assert _index_array(iter([4, 5])).tolist() == [4, 5]


def test_buffer_checks():
    with pytest.raises(ValueError):
        _host_sequences.int64_from_sequence([1, 2, 3], np.empty(2, dtype=np.int64))   # too short
    with pytest.raises(ValueError):
        _host_sequences.int64_from_sequence([1, 2], np.empty(2, dtype=np.int32))      # not int64
    with pytest.raises(ValueError):
        _host_sequences.int64_from_sequence([1, 2], np.empty(4, dtype=np.int64)[::2])  # not contiguous
    readonly = np.empty(2, dtype=np.int64)
    readonly.flags.writeable = False
    with pytest.raises((ValueError, BufferError)):
        _host_sequences.int64_from_sequence([1, 2], readonly)
    with pytest.raises(TypeError):
        _host_sequences.int64_from_sequence(5, np.empty(1, dtype=np.int64))


def test_range_fields_of_dicts_and_other_mappings():
    ranges = [{"start_token": 0, "end_token": 64, "cache_key": "a"},
              OrderedDict(start_token=64, end_token=96),
              {"end_token": 200, "start_token": 96}]
    assert _range_bounds(ranges).tolist() == [[0, 64], [64, 96], [96, 200]]
    # Fields that are not integers go through int(), as the reference's plan code does.
    assert _range_bounds([{"start_token": 1.0, "end_token": "5"}]).tolist() == [[1, 5]]
    with pytest.raises(KeyError):
        _range_bounds([{"start_token": 0}])
    with pytest.raises(KeyError):
        _range_bounds([OrderedDict(end_token=3)])
    assert _range_bounds([]).shape == (0, 2)
