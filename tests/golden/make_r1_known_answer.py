"""Expected output of the reference's eager (R1) remap known-answer test.

tests/pic/test_rope_remap.py:53-78 of the reference checks its
``_remap_key_positions`` bit for bit against a closed form it states in the
test: the fp32 delta from the fp32 cos/sin table (FakeRotary, theta 1e4,
rotary dim 8, tests/pic/support.py:49-71), cast to bf16, then bf16 products
and sums.  This script evaluates that closed form (torch on the CPU, the
reference is not imported) and prints the eight expected bf16 bit patterns;
they are stored as ``expected_bits`` of ``bf16_single_delta_rounding`` in
reference_known_answers.json.

    python tests/golden/make_r1_known_answer.py
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

GOLDEN = Path(__file__).resolve().parent / "reference_known_answers.json"


def fake_rotary_cache(max_position: int, rotary_dim: int, theta: float) -> torch.Tensor:
    inv_freq = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    positions = torch.arange(max_position, dtype=torch.float32)
    angles = torch.outer(positions, inv_freq)
    return torch.cat((angles.cos(), angles.sin()), dim=-1)


def expected_bits(case: dict) -> list[int]:
    cache = fake_rotary_cache(case["max_position"], case["rotary_dim"], case["theta"])
    key = torch.zeros(*case["key_shape"], dtype=torch.bfloat16)
    for index, value in case["key_nonzero"].items():
        key[0, 0, int(index)] = value
    local = torch.tensor([case["local"]])
    destination = torch.tensor([case["destination"]])
    local_cos, local_sin = cache[local].chunk(2, dim=-1)
    global_cos, global_sin = cache[destination].chunk(2, dim=-1)
    delta_cos = (global_cos * local_cos + global_sin * local_sin).to(torch.bfloat16)
    delta_sin = (global_sin * local_cos - global_cos * local_sin).to(torch.bfloat16)
    first, second = key.chunk(2, dim=-1)
    expected = torch.cat(
        (first * delta_cos.unsqueeze(1) - second * delta_sin.unsqueeze(1),
         second * delta_cos.unsqueeze(1) + first * delta_sin.unsqueeze(1)),
        dim=-1,
    ).to(torch.bfloat16)
    return [int(v) & 0xFFFF for v in expected.view(torch.int16).reshape(-1).tolist()]


if __name__ == "__main__":
    case = json.loads(GOLDEN.read_text())["bf16_single_delta_rounding"]
    print(json.dumps(expected_bits(case)))
