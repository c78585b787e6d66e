"""Seeded synthetic link workloads (Qwen2.5-7B / Qwen3-32B KV shapes).

Each workload is the input of one link step: which pool slots hold the
registered blocks, where the linked tokens go, the RoPE positions they carry
(compile-time ``local``) and need (request-global), the repair rows
(``imp_indices`` that fall inside blocks) and the identity prefix.

Placement follows the reference's plan derivation
(patched_sglang_files/python/sglang/srt/pic_runtime.py:3161-3250 and
:4911-5013): blocks land back to back in link order, block b covers request
positions [start_b, end_b), the repair rows are the first k tokens of every
block after the first ("k per seam", recompute_first_block off), and the
identity prefix is block 0 when its positions need no remap.

Position deltas.  The reference compiles every block at local positions
0..n-1, so a block's delta equals its start.  Workloads "c1", "c4" and "c5"
draw a per-block delta in [-R, R] instead (blocks compiled behind a different
prefix); delta_b is clipped to <= start_b so that local = global - delta >= 0.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field

import numpy as np

BASE_SEED = 20260824


@dataclass(frozen=True)
class KVShape:
    layers: int
    kv_heads: int
    head_dim: int
    dtype: str = "bfloat16"

    @property
    def row_bytes(self) -> int:
        """Bytes of one (slot, layer) K row (V rows are the same size)."""

        return self.kv_heads * self.head_dim * 2

    @property
    def bytes_per_token(self) -> int:
        """Read + write bytes of one linked token over all layers (K and V)."""

        return self.layers * 2 * self.row_bytes * 2


QWEN25_7B = KVShape(layers=28, kv_heads=4, head_dim=128)
QWEN3_32B = KVShape(layers=64, kv_heads=8, head_dim=128)


@dataclass
class LinkWorkload:
    name: str
    description: str
    shape: KVShape
    num_slots: int
    source_slots: np.ndarray       # int64 [T]
    destination_slots: np.ndarray  # int64 [T]
    local_positions: np.ndarray    # int64 [T]
    global_positions: np.ndarray   # int64 [T]
    repair_mask: np.ndarray        # uint8 [T]
    prefix_token_count: int
    block_lengths: list[int]
    requests: int = 1
    rotary_dim: int = 128
    theta: float = 1_000_000.0
    seed: int = BASE_SEED
    notes: dict = field(default_factory=dict)

    def rank_share(self, tp: int) -> "LinkWorkload":
        """The workload as one of ``tp`` tensor-parallel ranks sees it: kv_heads / tp
        heads of every layer (the ranks' shards of srt/models/qwen2.py:127-141),
        the same tokens, slots and positions."""

        if tp < 1 or self.shape.kv_heads % tp:
            raise ValueError(f"tp {tp} must divide the {self.shape.kv_heads} KV heads of {self.name}")
        if tp == 1:
            return self
        shape = dataclasses.replace(self.shape, kv_heads=self.shape.kv_heads // tp)
        return dataclasses.replace(self, shape=shape,
                                   description=f"{self.description}; TP rank share: {shape.kv_heads} "
                                               f"of {self.shape.kv_heads} KV heads")

    @property
    def tokens(self) -> int:
        return int(self.source_slots.shape[0])

    @property
    def repair_offsets(self) -> np.ndarray:
        return np.flatnonzero(self.repair_mask).astype(np.int64)

    @property
    def repair_rows(self) -> int:
        return int(self.repair_mask.sum())

    @property
    def repair_destination_slots(self) -> np.ndarray:
        return self.destination_slots[self.repair_offsets]

    @property
    def max_position(self) -> int:
        return int(max(self.local_positions.max(), self.global_positions.max()))

    def link_requests(self) -> tuple[dict[str, tuple[np.ndarray, np.ndarray]],
                                     list[tuple[np.ndarray, dict]]]:
        """The workload as the link executor's inputs.

        Returns the blocks to register (cache key -> (source slots, compile-time
        positions); a catalogue block shared by several requests is one entry)
        and, per request, its destination slots indexed by request position
        (positions before its first block hold 0 and are never read) and its
        link plan (``cache_keys``, ``block_ranges``, ``imp_indices``)."""

        blocks: dict[str, tuple[np.ndarray, np.ndarray]] = {}
        requests: list[tuple[np.ndarray, dict]] = []
        lengths = self.block_lengths
        per_request = len(lengths) // self.requests
        cursor = 0
        for request in range(self.requests):
            own = lengths[request * per_request : (request + 1) * per_request]
            span = slice(cursor, cursor + int(sum(own)))
            positions = self.global_positions[span]
            destination = np.zeros(int(positions.max()) + 1, dtype=np.int64)
            destination[positions] = self.destination_slots[span]
            keys, ranges = [], []
            for n in own:
                source = self.source_slots[cursor : cursor + n]
                local = self.local_positions[cursor : cursor + n]
                key = f"blk-{int(source[0])}-{n}-{int(local[0])}"
                blocks.setdefault(key, (source, local))
                start = int(self.global_positions[cursor])
                keys.append(key)
                ranges.append({"start_token": start, "end_token": start + int(n)})
                cursor += n
            imp = positions[self.repair_mask[span] == 1].tolist()
            requests.append((destination, {"cache_keys": keys, "block_ranges": ranges, "imp_indices": imp}))
        return blocks, requests

    def algorithmic_bytes(self) -> dict[str, int]:
        """Bytes the link step must move: copied tokens plus repaired rows,
        K and V of every layer, read once and written once."""

        per_token = self.shape.bytes_per_token
        copied = self.tokens - self.repair_rows
        link = copied * per_token
        scatter = self.repair_rows * per_token
        return {"link_bytes": link, "scatter_bytes": scatter, "total_bytes": link + scatter}


def _lengths_summing_to(rng: np.random.Generator, count: int, low: int, high: int, total: int) -> list[int]:
    """``count`` integers in [low, high] summing to ``total``: start from uniform
    draws and move the surplus/deficit one block at a time."""

    if not count * low <= total <= count * high:
        raise ValueError("infeasible block length constraints")
    lengths = rng.integers(low, high + 1, size=count).astype(np.int64)
    diff = int(total - lengths.sum())
    while diff != 0:
        index = int(rng.integers(0, count))
        if diff > 0:
            step = min(diff, high - int(lengths[index]))
            if step > 0:
                step = int(rng.integers(1, step + 1))
                lengths[index] += step
                diff -= step
        else:
            step = min(-diff, int(lengths[index]) - low)
            if step > 0:
                step = int(rng.integers(1, step + 1))
                lengths[index] -= step
                diff += step
    return [int(value) for value in lengths]


def _single_request(
    name: str,
    description: str,
    shape: KVShape,
    num_slots: int,
    block_lengths: list[int],
    imp_per_seam: int,
    delta_range: int | None,
    seed: int,
) -> LinkWorkload:
    rng = np.random.default_rng(seed)
    total = int(sum(block_lengths))
    perm = rng.permutation(num_slots).astype(np.int64)
    if 2 * total > num_slots:
        raise ValueError("pool too small for the sources and destinations")
    # Registration order: block i owns the i-th run of the permutation.
    starts = np.concatenate(([0], np.cumsum(block_lengths)[:-1]))
    block_slots = [perm[s : s + n] for s, n in zip(starts, block_lengths)]
    order = rng.permutation(len(block_lengths))
    src, local, glob, mask = [], [], [], []
    request_start = 0
    deltas = []
    for position, block in enumerate(order):
        n = block_lengths[block]
        if delta_range is None:
            delta = request_start
        else:
            delta = int(rng.integers(-delta_range, min(delta_range, request_start) + 1))
        deltas.append(delta)
        g = request_start + np.arange(n, dtype=np.int64)
        src.append(block_slots[block])
        glob.append(g)
        local.append(g - delta)
        m = np.zeros(n, dtype=np.uint8)
        if position > 0:
            m[: min(imp_per_seam, n)] = 1
        mask.append(m)
        request_start += n
    first_delta = deltas[0]
    prefix = block_lengths[order[0]] if first_delta == 0 else 0
    return LinkWorkload(
        name=name,
        description=description,
        shape=shape,
        num_slots=num_slots,
        source_slots=np.concatenate(src),
        destination_slots=perm[total : 2 * total].copy(),
        local_positions=np.concatenate(local),
        global_positions=np.concatenate(glob),
        repair_mask=np.concatenate(mask),
        prefix_token_count=int(prefix),
        block_lengths=[int(block_lengths[b]) for b in order],
        seed=seed,
        notes={"deltas": deltas, "imp_per_seam": imp_per_seam},
    )


def _batched_requests(seed: int, *, requests: int = 64, blocks_per_request: int = 8,
                      block_tokens: int = 1024, catalogue: int = 512, num_slots: int = 1 << 20,
                      imp_per_seam: int = 8, zipf_s: float = 1.1,
                      shape: KVShape = QWEN25_7B) -> LinkWorkload:
    rng = np.random.default_rng(seed)
    perm = rng.permutation(num_slots).astype(np.int64)
    catalogue_tokens = catalogue * block_tokens
    total = requests * blocks_per_request * block_tokens
    if catalogue_tokens + total > num_slots:
        raise ValueError("pool too small for the catalogue and destinations")
    weights = 1.0 / np.arange(1, catalogue + 1, dtype=np.float64) ** zipf_s
    weights /= weights.sum()
    src, local, glob, mask = [], [], [], []
    chosen_all = []
    for _ in range(requests):
        chosen = rng.choice(catalogue, size=blocks_per_request, replace=False, p=weights)
        chosen_all.append(chosen)
        # Every request sits behind its own prompt prefix, so every block is
        # remapped (no identity prefix inside the batch).
        request_start = int(rng.integers(1, 8192))
        for position, block in enumerate(chosen):
            base = int(block) * block_tokens
            src.append(perm[base : base + block_tokens])
            g = request_start + position * block_tokens + np.arange(block_tokens, dtype=np.int64)
            glob.append(g)
            local.append(np.arange(block_tokens, dtype=np.int64))
            m = np.zeros(block_tokens, dtype=np.uint8)
            if position > 0:
                m[:imp_per_seam] = 1
            mask.append(m)
    chosen_flat = np.concatenate(chosen_all)
    return LinkWorkload(
        name="c3",
        description=(
            f"{requests} batched links x {blocks_per_request} blocks of {block_tokens} tokens, "
            f"Zipf({zipf_s}) over a {catalogue}-block catalogue, pool {num_slots} slots"
        ),
        shape=shape,
        num_slots=num_slots,
        source_slots=np.concatenate(src),
        destination_slots=perm[catalogue_tokens : catalogue_tokens + total].copy(),
        local_positions=np.concatenate(local),
        global_positions=np.concatenate(glob),
        repair_mask=np.concatenate(mask),
        prefix_token_count=0,
        block_lengths=[block_tokens] * (requests * blocks_per_request),
        requests=requests,
        seed=seed,
        notes={
            "distinct_blocks": int(np.unique(chosen_flat).size),
            "imp_per_seam": imp_per_seam,
        },
    )


WORKLOAD_NAMES = ("c1", "c2", "c3", "c4", "c5")


def make_workload(name: str, seed: int = BASE_SEED) -> LinkWorkload:
    """The five link workloads at their full sizes."""

    if name == "c1":
        return _single_request(
            "c1",
            "Qwen2.5-7B KV, pool 65,536; 4 x 512-token blocks in permuted order; "
            "deltas U[-1536, 1536]; 8 imp_indices per seam",
            QWEN25_7B, 65_536, [512] * 4, 8, 1536, seed,
        )
    if name == "c2":
        rng = np.random.default_rng(seed + 2)
        lengths = _lengths_summing_to(rng, 16, 256, 4096, 32_768)
        return _single_request(
            "c2",
            "Qwen2.5-7B KV, pool 262,144 random-permuted slots; 16 blocks U[256, 4096] "
            "summing to 32,768 tokens in random order; 16 imp_indices per seam",
            QWEN25_7B, 262_144, lengths, 16, None, seed,
        )
    if name == "c3":
        return _batched_requests(seed)
    if name == "c4":
        rng = np.random.default_rng(seed + 4)
        lengths = _lengths_summing_to(rng, 12, 512, 2048, 16_384)
        return _single_request(
            "c4",
            "Qwen3-32B KV, pool 131,072; 12 blocks U[512, 2048] summing to 16,384; "
            "deltas up to +-14,000; 16 imp_indices per seam",
            QWEN3_32B, 131_072, lengths, 16, 14_000, seed,
        )
    if name == "c5":
        return _single_request(
            "c5",
            "Qwen2.5-7B KV, pool 262,144; 512 x 64-token blocks; deltas U[-32768, 32768]; "
            "32 imp_indices per seam",
            QWEN25_7B, 262_144, [64] * 512, 32, 32_768, seed,
        )
    raise KeyError(f"unknown workload {name!r}; expected one of {WORKLOAD_NAMES}")


def scaled_single_request(
    *,
    shape: KVShape,
    num_slots: int,
    block_lengths: list[int],
    imp_per_seam: int,
    delta_range: int | None,
    seed: int = BASE_SEED,
    name: str = "custom",
) -> LinkWorkload:
    """A single-request workload with explicit sizes (tests, CPU samples)."""

    return _single_request(
        name, f"custom single-request link of {sum(block_lengths)} tokens", shape,
        num_slots, block_lengths, imp_per_seam, delta_range, seed,
    )
