"""Benchmark of the LegoLink KV link step on one MI355X.

One step = one link of the workload: the fused gather -> RoPE re-rotation ->
scatter over every layer (repair rows left out) plus the repaired-row
write-back, with every input already resident in HBM.  The link runs through
the product's executor: the workload's blocks are registered, each request's
plan is prepared once (registry lookup, token maps built on the device,
launch arguments) and the prepared link and write-back are launched per step;
preparation is timed separately (``host_prepare_ms``).  Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--workload c2]

The default workload is the Qwen2.5-7B-shaped 32,768-token link (pool 262,144
fully fragmented slots, 16 blocks, 240 repair rows).  ``--cpu-baseline`` (on by
default) times the reference's eager torch link path on the host cores on a
bounded sample of the same workload.  ``--copy-calibration`` instead times a
plain device copy of known size, for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT / "sglang-legolink_amd"))

HBM_PEAK_GBPS = 8000.0
METRIC = "linked KV GB/s (rd+wr) and % of 8 TB/s HBM; tokens linked/s, Qwen2.5-7B"
PROFILES = REPO_ROOT / "profiles"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    parser.add_argument("--cpu-baseline", dest="cpu_baseline", action="store_true", default=True)
    parser.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    parser.add_argument("--cpu-attention-gflop", type=float, default=20.0,
                        help="flop budget of the repair attention CPU baseline sample")
    parser.add_argument("--cpu-sample-tokens", type=int, default=32768)
    parser.add_argument("--cpu-reps", type=int, default=25)
    parser.add_argument("--layers-per-wave", type=int, default=0)
    parser.add_argument("--waves-per-block", type=int, default=4)
    parser.add_argument("--layer-groups-per-block", type=int, default=0)
    parser.add_argument("--delta-staging", choices=["auto", "per_wave", "workgroup", "table"], default="auto",
                        help="where the link kernel computes its RoPE deltas (same result)")
    parser.add_argument("--visit-order", choices=["auto", "plan", "source", "destination"], default="auto",
                        help="order in which the link kernel visits the rotated rows (same result; auto: "
                             "the executor's choice)")
    parser.add_argument("--repair-rows", choices=["compact", "mask"], default="compact",
                        help="drop repair rows from the link maps (as the executor does) or pass a mask")
    parser.add_argument("--copy-calibration", type=int, default=0,
                        help="time a plain device copy of this many MiB instead of the link")
    parser.add_argument("--run-sweep", action="store_true",
                        help="time the link kernel on maps whose sources and destinations come in "
                             "contiguous runs of 1..64 slots, for several launch shapes")
    parser.add_argument("--calibration-only", action="store_true",
                        help="only the sweep's row calibration (calibration kernels and torch's index "
                             "kernels) on the workload's random, destination-sorted and contiguous maps: "
                             "a short run for hardware counters")
    parser.add_argument("--no-calibration", dest="calibration", action="store_false", default=True,
                        help="sweep: skip the row calibration (calibration kernels and torch index ops)")
    parser.add_argument("--sweep-detail-run", type=int, default=64,
                        help="run length that gets every launch-shape variant (besides 1)")
    parser.add_argument("--repair-attention", action="store_true",
                        help="time the sparse repair attention of the workload's repair spans "
                             "(one layer) instead of the link")
    parser.add_argument("--tp", type=int, default=1,
                        help="bench one tensor-parallel rank's share: kv_heads / tp heads of every layer "
                             "(the link has no exchange step; each rank links its own head shard)")
    parser.add_argument("--rounding", choices=["fused", "eager"], default="fused",
                        help="rounding of re-rotated K: the reference's fused kernel (default) or its "
                             "torch path")
    parser.add_argument("--storage", choices=["reference", "clone"], default="reference",
                        help="blocks read from pool slots (reference) or captured into a snapshot arena and "
                             "linked from it (clone); clone also times the capture and a group promotion")
    parser.add_argument("--split-tokens", type=int, default=0,
                        help="repair attention: KV tokens per work item (0: the planner's choice)")
    parser.add_argument("--head-dim", type=int, default=0, choices=[0, 64, 128, 256],
                        help="repair attention: head dim in place of the workload's (same spans and heads)")
    parser.add_argument("--heads", default="",
                        help="repair attention: query/KV heads in place of the model's, e.g. 8/8 (MHA), "
                             "32/8 (same spans)")
    return parser.parse_args()


def copy_calibration(args: argparse.Namespace) -> None:
    import torch

    device = torch.device("cuda", 0)
    nbytes = args.copy_calibration << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device=device).random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize(device)
    start = time.perf_counter()
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize(device)
    elapsed = (time.perf_counter() - start) / args.steps
    print(json.dumps({"copy_bytes": nbytes, "read_kib": nbytes / 1024, "write_kib": nbytes / 1024,
                      "ms_per_copy": elapsed * 1e3, "gbps_rd_wr": 2 * nbytes / elapsed / 1e9}), flush=True)


def cpu_baseline(workload, args) -> dict:
    """The reference's eager torch link path (index_select -> remap -> index_copy_,
    then the repair write-back) on the host cores, on a bounded sample."""

    import numpy as np
    import torch

    from legolink_amd.rope import build_cos_sin_cache
    from legolink_amd.workloads import scaled_single_request
    from oracle import r1_torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    lengths, total = [], 0
    for length in workload.block_lengths:
        if total >= args.cpu_sample_tokens:
            break
        lengths.append(length)
        total += length
    shape = workload.shape
    # The workload's own pool when the sample is the whole workload and the
    # pool fits in 40 GB of host memory (c2: 262,144 slots, 15 GB); else a
    # pool four times the sample.
    pool_bytes = workload.num_slots * shape.layers * 2 * shape.kv_heads * shape.head_dim * 2
    whole = len(lengths) == len(workload.block_lengths)
    slots = workload.num_slots if whole and pool_bytes <= 40e9 else 4 * total
    sample = scaled_single_request(shape=shape, num_slots=slots, block_lengths=lengths,
                                   imp_per_seam=int(workload.notes.get("imp_per_seam", 16)),
                                   delta_range=None, seed=workload.seed, name="cpu_sample")
    log(f"cpu baseline: {sample.tokens} tokens, pool {slots} slots, {shape.layers} layers, {cores} threads")
    generator = torch.Generator().manual_seed(1)
    tile = torch.randn(1 << 20, generator=generator).to(torch.bfloat16)
    row = shape.kv_heads * shape.head_dim

    def filled() -> torch.Tensor:
        flat = tile.repeat((slots * row + tile.numel() - 1) // tile.numel())[: slots * row]
        return flat.view(slots, shape.kv_heads, shape.head_dim).clone()

    keys = [filled() for _ in range(shape.layers)]
    values = [filled() for _ in range(shape.layers)]
    table = build_cos_sin_cache(sample.max_position + 1, sample.rotary_dim, theta=sample.theta)
    src = torch.from_numpy(sample.source_slots)
    dst = torch.from_numpy(sample.destination_slots)
    local = torch.from_numpy(sample.local_positions)
    glob = torch.from_numpy(sample.global_positions)
    repair_slots = torch.from_numpy(sample.repair_destination_slots)
    repaired = torch.randn(shape.layers, sample.repair_rows, shape.kv_heads, shape.head_dim,
                           generator=generator).to(torch.bfloat16)

    def step() -> None:
        r1_torch.link_batched_layers(keys, values, src, dst, local, glob, table,
                                     prefix_token_count=sample.prefix_token_count,
                                     rotary_dim=sample.rotary_dim, is_neox_style=True)
        r1_torch.scatter_rows(keys, values, repair_slots, repaired, repaired)

    step()
    times = []
    for _ in range(max(1, args.cpu_reps)):
        start = time.perf_counter()
        step()
        times.append(time.perf_counter() - start)
    seconds = float(np.median(times))
    total_bytes = sample.algorithmic_bytes()["total_bytes"]
    return {
        "value": total_bytes / seconds / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "tokens_linked_per_s": sample.tokens / seconds,
        "seconds_per_link": seconds,
        "sample": (
            f"eager torch link path of the reference (per layer index_select -> R1 RoPE remap -> "
            f"index_copy_, then repair-row index_copy_) on the first {len(lengths)} blocks of the "
            f"workload ({sample.tokens} tokens, {sample.repair_rows} repair rows) in a "
            f"{slots}-slot bf16 pool, {shape.layers} layers x {shape.kv_heads} KV heads x "
            f"{shape.head_dim}; 1 warm-up + {len(times)} timed reps, median"
        ),
    }


def _median_ms(torch, run, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    for start, end in events:
        start.record()
        run()
        end.record()
    torch.cuda.synchronize()
    return sorted(s.elapsed_time(e) for s, e in events)[steps // 2]


RUN_LENGTHS = (1, 2, 4, 8, 16, 64)


# Orders (at run length 1) on which the sweep also runs the row calibration.
CALIBRATION_ORDERS = ("random", "sorted_destination", "contiguous")


SWEEP_ORDERS = ("random", "sorted_source", "sorted_destination", "bucketed_destination", "sorted_both", "contiguous",
                "random_source_contiguous_destination", "contiguous_source_random_destination",
                "random_in_first_65536_slots", "random_in_first_131072_slots")


def ordered_maps(workload, run: int, order: str, seed: int):
    """``run_length_maps`` visited in ``order``: "random" (as drawn),
    "sorted_source" / "sorted_destination" (tokens reordered so that one map
    increases; positions move with their tokens), "bucketed_destination"
    (destination slots increasing by bucket of 2^shift slots, as the
    executor orders a single request's rows), "sorted_both" (each map
    sorted on its own: the same slots, both increasing), "contiguous" (sources
    [0, T), destinations [T, 2T)).  Returns src, dst, local, global."""

    import numpy as np

    local, glob = workload.local_positions, workload.global_positions
    tokens = np.arange(workload.tokens, dtype=np.int64)
    if order == "contiguous":
        return tokens, tokens + workload.tokens, local, glob
    if order.startswith("random_in_first_"):
        # Every row of a smaller slot range is read or written: random order,
        # smaller footprint per buffer.
        span = int(order.rsplit("_", 2)[1])
        perm = np.random.default_rng(seed).permutation(span).astype(np.int64)
        return perm[: workload.tokens], perm[workload.tokens : 2 * workload.tokens], local, glob
    if order in ("random_source_contiguous_destination", "contiguous_source_random_destination"):
        # One side is the last T slots in token order, the other random rows
        # of the slots before them.
        block = tokens + workload.num_slots - workload.tokens
        scattered = np.random.default_rng(seed).permutation(workload.num_slots - workload.tokens)
        scattered = scattered[: workload.tokens].astype(np.int64)
        if order == "random_source_contiguous_destination":
            return scattered, block, local, glob
        return block, scattered, local, glob
    src, dst = run_length_maps(workload, run, seed)
    if order == "sorted_source":
        index = np.argsort(src, kind="stable")
        return src[index], dst[index], local[index], glob[index]
    if order == "sorted_destination":
        index = np.argsort(dst, kind="stable")
        return src[index], dst[index], local[index], glob[index]
    if order == "bucketed_destination":
        # The executor's destination order: by bucket of 2^shift slots (16,384
        # buckets over the pool), in no fixed order within a bucket (here: as drawn).
        shift = 0
        while ((workload.num_slots - 1) >> shift) >= 16384:
            shift += 1
        index = np.argsort(dst >> shift, kind="stable")
        return src[index], dst[index], local[index], glob[index]
    if order == "sorted_both":
        return np.sort(src), np.sort(dst), local, glob
    return src, dst, local, glob


def run_length_maps(workload, run: int, seed: int):
    """Token maps of ``workload``'s tokens whose source and destination slots
    come in contiguous runs of ``run`` rows: the pool is cut into runs of
    ``run`` slots, distinct runs are drawn at random for the sources and for
    the destinations, and token t reads row t % run of its source run and
    writes row t % run of its destination run.  run = 1 is a fully fragmented
    pool (page size 1, random permutation), as the workload itself."""

    import numpy as np

    rng = np.random.default_rng(seed)
    tokens = workload.tokens
    runs_needed = -(-tokens // run)
    runs = rng.permutation(workload.num_slots // run)[: 2 * runs_needed].astype(np.int64)
    if runs.size < 2 * runs_needed:
        raise ValueError("pool too small for these runs")
    offsets = np.arange(tokens, dtype=np.int64)
    src = runs[offsets // run] * run + offsets % run
    dst = runs[runs_needed + offsets // run] * run + offsets % run
    return src, dst


class _RowCalibration:
    """ctypes binding of liblegolink_calibration.so (csrc/row_calibration.hip):
    the link's row traffic without the RoPE arithmetic, and its halves."""

    MODES = {"copy": 0, "read_only": 1, "write_only": 2}

    def __init__(self, torch) -> None:
        import ctypes

        self.ctypes = ctypes
        path = REPO_ROOT / "sglang-legolink_amd" / "legolink_amd" / "lib" / "liblegolink_calibration.so"
        if not path.is_file():
            raise SystemExit(f"{path} is not built (python -c 'import __graft_entry__ as g; g.build()')")
        self.lib = ctypes.CDLL(str(path))
        i64, ptr = ctypes.c_int64, ctypes.c_void_p

        class Args(ctypes.Structure):
            _fields_ = [("struct_size", i64), ("num_layers", i64), ("key_layers", ptr), ("value_layers", ptr),
                        ("num_slots", i64), ("row_bytes", i64), ("num_tokens", i64), ("source_slots", ptr),
                        ("destination_slots", ptr), ("mode", i64), ("layer_major", i64),
                        ("layers_per_wave", i64), ("tokens_per_wave", i64), ("lds_bytes", i64), ("sink", ptr),
                        ("buffers", i64)]

        self.Args = Args
        self.lib.llc_rows.argtypes = [ctypes.POINTER(Args), ptr]
        self.lib.llc_rows.restype = ctypes.c_int
        self.lib.llc_row_args_size.restype = i64
        self.lib.llc_last_error.restype = ctypes.c_char_p
        if self.lib.llc_row_args_size() != ctypes.sizeof(Args):
            raise SystemExit("liblegolink_calibration.so does not match bench.py's argument struct")
        self.torch = torch

    def prepare(self, keys, values, src, dst, *, mode: str, layer_major: bool, per_wave: int, lds_bytes: int,
                sink, buffers: int = 3):
        ctypes = self.ctypes
        key_table = (ctypes.c_void_p * len(keys))(*[k.data_ptr() for k in keys])
        value_table = (ctypes.c_void_p * len(values))(*[v.data_ptr() for v in values])
        args = self.Args(struct_size=ctypes.sizeof(self.Args), num_layers=len(keys),
                         key_layers=ctypes.addressof(key_table), value_layers=ctypes.addressof(value_table),
                         num_slots=int(keys[0].shape[0]), row_bytes=int(keys[0][0].numel()) * keys[0].element_size(),
                         num_tokens=int(src.numel()), source_slots=src.data_ptr(), destination_slots=dst.data_ptr(),
                         mode=self.MODES[mode], layer_major=1 if layer_major else 0,
                         layers_per_wave=0 if layer_major else per_wave, tokens_per_wave=per_wave if layer_major else 0,
                         lds_bytes=lds_bytes, sink=sink.data_ptr(), buffers=buffers)
        keep = (key_table, value_table, args, keys, values, src, dst, sink)
        torch = self.torch

        def run() -> None:
            status = self.lib.llc_rows(ctypes.byref(keep[2]), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if status != 0:
                raise RuntimeError(f"llc_rows: {self.lib.llc_last_error().decode()}")

        return run


# Occupancy limits of the calibration kernels: dynamic LDS per 256-thread
# workgroup (160 KiB of LDS per CU): none, 40 KiB (4 workgroups per CU), 64 KiB (2).
CALIBRATION_LDS = (0, 40960, 65536)


def calibrate_rows(torch, workload, keys, values, src_t, dst_t, order: str, args) -> list[dict]:
    """The link's row traffic on these maps, moved by code other than the link
    kernel: the calibration kernels (copy, read only, write only; token-major
    4 layers per wave and layer-major 2 tokens per wave; three occupancies)
    and in two layer-major passes (K rows, then V rows), and torch's own index
    kernels per layer (index_select + index_copy_ as the
    reference's eager path moves rows, and each half alone: the gather into a
    contiguous buffer, the scatter from one).  GB/s count the bytes each
    variant moves: the link's 2 x T x L x (K + V row) for a copy, half of it
    for a read-only or write-only pass, and the gather's and scatter's own
    read + write bytes for torch's halves."""

    calibration = _RowCalibration(torch)
    sink = torch.zeros(65536 * 4, dtype=torch.int32, device=keys[0].device)
    row = int(keys[0][0].numel()) * keys[0].element_size()
    one_way = workload.tokens * len(keys) * 2 * row
    rows = []
    for mode in ("copy", "read_only", "write_only"):
        for layer_major, per_wave in ((False, 4), (True, 2)):
            for lds in CALIBRATION_LDS:
                run = calibration.prepare(keys, values, src_t, dst_t, mode=mode, layer_major=layer_major,
                                          per_wave=per_wave, lds_bytes=lds, sink=sink)
                ms = _median_ms(torch, run, args.steps, args.warmup)
                moved = 2 * one_way if mode == "copy" else one_way
                shape = f"{'layer_major_2_tokens' if layer_major else 'token_major_4_layers'}_lds{lds // 1024}k"
                rows.append({"order": order, "source": "calibration", "mode": mode, "variant": shape,
                             "ms": round(ms, 5), "bytes": moved, "GBps": round(moved / ms / 1e6, 1)})
                log(f"calibration {order:18s} {mode:10s} {shape:34s} {ms:.4f} ms {moved / ms / 1e6:8.1f} GB/s")
    # The copy in two layer-major passes (all K rows, then all V rows), as the
    # delta-table link moves them.
    for per_wave in (2, 4):
        key_pass = calibration.prepare(keys, values, src_t, dst_t, mode="copy", layer_major=True,
                                       per_wave=per_wave, lds_bytes=0, sink=sink, buffers=1)
        value_pass = calibration.prepare(keys, values, src_t, dst_t, mode="copy", layer_major=True,
                                         per_wave=per_wave, lds_bytes=0, sink=sink, buffers=2)

        def two_passes(key_pass=key_pass, value_pass=value_pass) -> None:
            key_pass()
            value_pass()

        ms = _median_ms(torch, two_passes, args.steps, args.warmup)
        shape = f"layer_major_{per_wave}_tokens_two_passes"
        rows.append({"order": order, "source": "calibration", "mode": "copy", "variant": shape,
                     "ms": round(ms, 5), "bytes": 2 * one_way, "GBps": round(2 * one_way / ms / 1e6, 1)})
        log(f"calibration {order:18s} {'copy':10s} {shape:34s} {ms:.4f} ms {2 * one_way / ms / 1e6:8.1f} GB/s")
    staging_k = torch.empty((workload.tokens,) + tuple(keys[0].shape[1:]), dtype=keys[0].dtype, device=keys[0].device)
    staging_v = torch.empty_like(staging_k)

    def torch_copy() -> None:
        for key, value in zip(keys, values):
            key.index_copy_(0, dst_t, key.index_select(0, src_t))
            value.index_copy_(0, dst_t, value.index_select(0, src_t))

    def torch_gather() -> None:
        for key, value in zip(keys, values):
            torch.index_select(key, 0, src_t, out=staging_k)
            torch.index_select(value, 0, src_t, out=staging_v)

    def torch_scatter() -> None:
        for key, value in zip(keys, values):
            key.index_copy_(0, dst_t, staging_k)
            value.index_copy_(0, dst_t, staging_v)

    for mode, run in (("copy", torch_copy), ("gather_half", torch_gather), ("scatter_half", torch_scatter)):
        ms = _median_ms(torch, run, args.steps, args.warmup)
        moved = 2 * one_way
        rows.append({"order": order, "source": "torch", "mode": mode,
                     "variant": {"copy": "index_select + index_copy_ per layer",
                                 "gather_half": "index_select into a contiguous buffer per layer",
                                 "scatter_half": "index_copy_ from a contiguous buffer per layer"}[mode],
                     "ms": round(ms, 5), "bytes": moved, "GBps": round(moved / ms / 1e6, 1)})
        log(f"torch       {order:18s} {mode:12s} {ms:.4f} ms {moved / ms / 1e6:8.1f} GB/s")
    return rows


def sweep_ceiling(rows: list[dict], calibration: list[dict], link_bytes: int) -> dict:
    """The fastest valid way to move the workload's own rows (fully fragmented,
    in any visit order): the link kernel's variants, the calibration copies and
    torch's copy; and the bound the separately timed halves give when a copy's
    reads and writes do not slow each other down."""

    own = [r for r in rows if r["run"] == 1 and r["order"] in ("random", "sorted_destination", "sorted_source",
                                                                "sorted_both", "bucketed_destination")]
    best_link = max(own, key=lambda r: r["GBps"])
    fragmented = [c for c in calibration if c["order"] != "contiguous"]
    copies = [c for c in fragmented if c["mode"] == "copy"]
    best_copy = max(copies, key=lambda c: c["GBps"])
    reads = [c for c in fragmented if c["source"] == "calibration" and c["mode"] == "read_only"]
    writes = [c for c in fragmented if c["source"] == "calibration" and c["mode"] == "write_only"]
    best_read, best_write = min(reads, key=lambda c: c["ms"]), min(writes, key=lambda c: c["ms"])
    halves_ms = best_read["ms"] + best_write["ms"]
    return {
        "link_kernel_best": {"GBps": best_link["GBps"], "order": best_link["order"], "variant": best_link["variant"]},
        "independent_copy_best": {"GBps": best_copy["GBps"], "order": best_copy["order"],
                                  "source": best_copy["source"], "variant": best_copy["variant"]},
        "read_only_best": {"GBps": best_read["GBps"], "ms": best_read["ms"], "order": best_read["order"],
                           "variant": best_read["variant"]},
        "write_only_best": {"GBps": best_write["GBps"], "ms": best_write["ms"], "order": best_write["order"],
                            "variant": best_write["variant"]},
        "halves_bound": {"GBps": round(link_bytes / halves_ms / 1e6, 1), "ms": round(halves_ms, 5)},
    }


def run_sweep(args: argparse.Namespace) -> None:
    """The link kernel itself on maps of growing contiguity: how fast the
    kernel moves the workload's rows when sources and destinations come in
    runs of 1 (fully fragmented), 2, 4, ... 64 consecutive slots, for several
    launch shapes.  Every launch links all of the workload's tokens (repair
    rows included) with the workload's positions; GB/s counts each token's K
    and V rows of every layer read once and written once.  Prints one JSON line
    with a row per (run length, variant) and the order of their launches (for
    matching rocprofv3 dispatches)."""

    import numpy as np
    import torch

    from legolink_amd import kv_link
    from legolink_amd.rope import build_cos_sin_cache
    from legolink_amd.workloads import make_workload

    device = torch.device("cuda", 0)
    workload = make_workload(args.workload)
    shape = workload.shape
    generator = torch.Generator(device=device).manual_seed(20260824)
    keys = [torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, dtype=torch.bfloat16,
                        device=device, generator=generator) for _ in range(shape.layers)]
    values = [torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, dtype=torch.bfloat16,
                          device=device, generator=generator) for _ in range(shape.layers)]
    table = build_cos_sin_cache(workload.max_position + 1, workload.rotary_dim, theta=workload.theta).to(device)
    link_bytes = workload.tokens * shape.bytes_per_token
    # (name, launch keywords); the first is the executor's choice for a single request.
    default = {"num_warps": 4, "layers_per_wave": 0, "stream_source_rows": True}
    table_workspace = torch.empty(kv_link.delta_workspace_bytes(workload.tokens, workload.rotary_dim),
                                  dtype=torch.uint8, device=device)
    variants = [("default", {}), ("staged_deltas", {"delta_staging": "workgroup"}),
                ("delta_table", {"delta_staging": "table", "delta_workspace": table_workspace})]
    detailed = {1, int(args.sweep_detail_run)}
    extra = [
        ("cached_loads", {"stream_source_rows": False}),
        ("rotation_off", {"rotation_off": True}),
        ("layers_per_wave_1", {"layers_per_wave": 1}),
        ("layers_per_wave_2", {"layers_per_wave": 2}),
        ("layers_per_wave_7", {"layers_per_wave": 7}),
        ("layers_per_wave_28", {"layers_per_wave": 28}),
        ("waves_per_block_1", {"num_warps": 1}),
        ("waves_per_block_8", {"num_warps": 8}),
        ("staged_deltas", {"delta_staging": "workgroup"}),
        ("staged_deltas_layers_per_wave_2", {"delta_staging": "workgroup", "layers_per_wave": 2}),
        ("staged_deltas_layers_per_wave_7", {"delta_staging": "workgroup", "layers_per_wave": 7}),
    ]
    rows, schedule, dispatch, calibration, calibration_maps = [], [], 0, [], []
    cases = [(run, "random") for run in RUN_LENGTHS]
    cases += [(1, order) for order in SWEEP_ORDERS if order != "random"]
    # The runs again in the executor's visit order (destination buckets).
    cases += [(run, "bucketed_destination") for run in RUN_LENGTHS if run > 1]
    for run, order in cases:
        src, dst, local_np, global_np = ordered_maps(workload, run, order, seed=20260824 + run)
        src_t = torch.from_numpy(src).to(device)
        dst_t = torch.from_numpy(dst).to(device)
        local = torch.from_numpy(np.ascontiguousarray(local_np)).to(device)
        glob = torch.from_numpy(np.ascontiguousarray(global_np)).to(device)
        chosen = variants + ([v for v in extra if v[0] != "staged_deltas"]
                             if (run in detailed and order == "random") or order == "contiguous" else [])
        for name, changes in chosen:
            options = dict(default, **changes)
            rotation_off = options.pop("rotation_off", False)
            prepared = kv_link.PreparedKVLink(
                key_buffers=keys, value_buffers=values, source_slots=src_t, destination_slots=dst_t,
                local_positions=local, global_positions=glob, cos_sin_cache=table,
                prefix_token_count=workload.tokens if rotation_off else workload.prefix_token_count,
                rotary_dim=workload.rotary_dim, is_neox_style=True, **options)
            ms = _median_ms(torch, prepared, args.steps, args.warmup)
            launches = prepared.launch["launches"] * (args.steps + args.warmup)
            schedule.append({"run": run, "order": order, "variant": name, "first_dispatch": dispatch,
                             "dispatches": launches})
            dispatch += launches
            rows.append({"run": run, "order": order, "variant": name, "ms": round(ms, 5),
                         "GBps": round(link_bytes / ms / 1e6, 1),
                         "frac": round(link_bytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
                         "launch": prepared.launch})
            log(f"run {run:3d} {order:18s} {name:20s} {ms:.4f} ms  {link_bytes / ms / 1e6:8.1f} GB/s")
        if args.calibration and run == 1 and order in CALIBRATION_ORDERS:
            calibration_maps.append((order, src_t, dst_t))
    # After every link launch, so that the link's dispatches keep their
    # positions in a counter trace; the calibration's are matched by kernel name.
    for order, src_t, dst_t in calibration_maps:
        calibration += calibrate_rows(torch, workload, keys, values, src_t, dst_t, order, args)
    ceiling = sweep_ceiling(rows, calibration, link_bytes) if calibration else None
    print(json.dumps({"sweep": rows, "calibration": calibration, "ceiling": ceiling, "schedule": schedule,
                      "workload": workload.name, "tokens": workload.tokens, "bytes_per_launch": link_bytes,
                      "steps": args.steps, "warmup": args.warmup, "peak_GBps": HBM_PEAK_GBPS}), flush=True)


def same_maps_ceiling(torch, prepared, keys, values, link_bytes: int, args) -> dict | None:
    """The fastest independent copy of exactly the rows this link moves: the
    row-calibration kernels (copy, read only, write only) on the link's own
    device maps, timed in this process alternately with the link itself
    (three rounds, median of 20 launches each).  None where the calibration
    does not apply (several map sets, rows not a multiple of 1 KiB, or the
    calibration library not built)."""

    import numpy as np

    maps = prepared.kernel_maps
    row = int(keys[0][0].numel()) * keys[0].element_size()
    if len(maps) != 1 or row % 1024 or int(maps[0].shape[1]) % 2:
        return None
    try:
        calibration = _RowCalibration(torch)
    except SystemExit:
        return None
    src, dst = maps[0][0].contiguous(), maps[0][1].contiguous()
    sink = torch.zeros(65536 * 4, dtype=torch.int32, device=keys[0].device)
    shapes = {"layer_major_2_tokens": (True, 2), "token_major_4_layers": (False, 4)}
    runs = {"link": prepared.launch}
    moved = {"link": link_bytes}
    for mode in ("copy", "read_only", "write_only"):
        for shape, (layer_major, per_wave) in shapes.items():
            if not layer_major and len(keys) % per_wave:
                continue
            runs[f"{mode} {shape}"] = calibration.prepare(keys, values, src, dst, mode=mode, layer_major=layer_major,
                                                          per_wave=per_wave, lds_bytes=0, sink=sink)
            moved[f"{mode} {shape}"] = link_bytes if mode == "copy" else link_bytes // 2
    key_pass = calibration.prepare(keys, values, src, dst, mode="copy", layer_major=True, per_wave=2,
                                   lds_bytes=0, sink=sink, buffers=1)
    value_pass = calibration.prepare(keys, values, src, dst, mode="copy", layer_major=True, per_wave=2,
                                     lds_bytes=0, sink=sink, buffers=2)

    def two_passes() -> None:
        key_pass()
        value_pass()

    runs["copy layer_major_2_tokens_two_passes"] = two_passes
    moved["copy layer_major_2_tokens_two_passes"] = link_bytes
    times = {name: [] for name in runs}
    for _ in range(3):
        for name, run in runs.items():
            times[name].append(_median_ms(torch, run, 20, 3))
    gbps = {name: moved[name] / float(np.median(ms)) / 1e6 for name, ms in times.items()}
    copies = {name: value for name, value in gbps.items() if name.startswith("copy ")}
    best = max(copies, key=copies.get)
    reads = [float(np.median(times[n])) for n in times if n.startswith("read_only")]
    writes = [float(np.median(times[n])) for n in times if n.startswith("write_only")]
    halves = link_bytes / (min(reads) + min(writes)) / 1e6 if reads and writes else None
    log(f"same-maps ceiling: link {gbps['link']:.1f} GB/s, best copy {copies[best]:.1f} GB/s ({best}), "
        f"ratio {gbps['link'] / copies[best]:.4f}")
    return {"GBps": round(copies[best], 1), "frac": round(copies[best] / HBM_PEAK_GBPS, 4),
            "what": f"fastest independent copy of this link's own rows (the executor's maps of this run), "
                    f"calibration {best.split(' ', 1)[1]}, timed in this process alternately with the link",
            "halves_bound_GBps": None if halves is None else round(halves, 1),
            "link_in_same_run_GBps": round(gbps["link"], 1),
            "link_over_ceiling_in_same_run": round(gbps["link"] / copies[best], 4),
            "variants_GBps": {name: round(value, 1) for name, value in gbps.items() if name != "link"}}


def time_attention_plan(workload, requests, device) -> float | None:
    """Host time of the repair pass's attention plan for this link's repair
    spans (built once per batch, shared by every layer; Qwen's 7 query heads
    per KV head, Qwen3-32B's 8): median of 5 after a first, each computed
    afresh.  None when the link has no repair rows."""

    import numpy as np
    import torch

    from legolink_amd import _native
    from legolink_amd.link_plan import contiguous_ranges
    from legolink_amd.repair_attention import RepairAttentionPlan

    spans = [(slots, int(start), int(end)) for slots, plan in requests
             for start, end in contiguous_ranges(plan.get("imp_indices") or [])]
    if not spans:
        return None
    shape = workload.shape
    q_heads = (7 if shape.kv_heads == 4 else 8) * shape.kv_heads
    times = []
    for _ in range(6):
        _native.repair_attention_plan(np.array([[0, 0, 1, 0]], dtype=np.int64), q_heads, shape.kv_heads, 0)
        torch.cuda.synchronize(device)
        start = time.perf_counter()
        RepairAttentionPlan(spans, num_q_heads=q_heads, num_kv_heads=shape.kv_heads, head_dim=shape.head_dim,
                            pool_size=workload.num_slots)
        torch.cuda.synchronize(device)
        times.append((time.perf_counter() - start) * 1e3)
    return float(np.median(times[1:]))


def calibration_only(args: argparse.Namespace) -> None:
    """The sweep's calibration leg alone (no link launches): the same pool and
    maps, every calibration variant and torch's index kernels, in a fixed
    dispatch order that the JSON line lists (for matching counter rows)."""

    import torch

    from legolink_amd.workloads import make_workload

    device = torch.device("cuda", 0)
    workload = make_workload(args.workload)
    shape = workload.shape
    generator = torch.Generator(device=device).manual_seed(20260824)
    keys = [torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, dtype=torch.bfloat16,
                        device=device, generator=generator) for _ in range(shape.layers)]
    values = [torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, dtype=torch.bfloat16,
                          device=device, generator=generator) for _ in range(shape.layers)]
    rows = []
    for order in CALIBRATION_ORDERS:
        src, dst, _, _ = ordered_maps(workload, 1, order, seed=20260824 + 1)
        src_t = torch.from_numpy(src).to(device)
        dst_t = torch.from_numpy(dst).to(device)
        rows += calibrate_rows(torch, workload, keys, values, src_t, dst_t, order, args)
    print(json.dumps({"calibration": rows, "workload": workload.name, "tokens": workload.tokens,
                      "layers": shape.layers, "steps": args.steps, "warmup": args.warmup,
                      "dispatch_order": "per row: (warmup + steps) launches of its kernels; calibration "
                                        "rows one launch each, torch rows 4 launches per layer (copy: "
                                        "index_select + index_copy_ for K and V) or 2 (a half)"}), flush=True)


def load_traffic(workload_name: str, link_launch_bytes: int) -> float | None:
    """HBM bytes per link launch from the committed rocprofv3 counter summary of
    this workload; None when there is none, or when it was taken on a launch
    that moved a different number of algorithmic bytes (another repair-row mode)."""

    path = PROFILES / f"traffic_kv_link_{workload_name}.json"
    if not path.is_file():
        return None
    data = json.loads(path.read_text())
    try:
        if int(data["algorithmic_bytes_per_launch"]) != int(link_launch_bytes):
            return None
        return float(data["hbm_bytes_per_launch"])
    except (KeyError, TypeError, ValueError):
        return None


def load_pattern_ceiling(workload_name: str) -> dict | None:
    """The committed sweep's ceiling for this workload's access pattern: the
    fastest independent copy of the workload's own fragmented rows (the
    row-calibration kernels and torch's index kernels), the bound of its
    read-only and write-only halves, and the link as the executor launches
    it, all measured in one process; None when there is none."""

    path = PROFILES / f"pattern_ceiling_kv_link_{workload_name}.json"
    if not path.is_file():
        return None
    data = json.loads(path.read_text())
    try:
        best = data["independent_copy_best"]
        return {"GBps": best["GBps"], "frac": round(best["GBps"] / HBM_PEAK_GBPS, 4),
                "what": f"fastest independent copy of the same rows ({best['source']} {best['variant']}, "
                        f"{best['order']} order)",
                "halves_bound_GBps": data["halves_bound"]["GBps"],
                "link_in_same_run_GBps": data["link_as_run"]["GBps"],
                "link_over_ceiling_in_same_run": data["link_over_independent_copy"],
                "source": f"profiles/{path.name}: {data['command']}"}
    except (KeyError, TypeError):
        return None


def repair_attention_bench(args: argparse.Namespace) -> None:
    """The repair pass's attention for the workload's repair spans, one layer
    of the Qwen2.5-7B shape (28 query heads over 4 KV heads, head dim 128):
    each contiguous run of imp_indices attends over its request's tokens
    0..end-1 through the request's slots.  Prints one JSON line."""

    import math

    import numpy as np
    import torch

    from legolink_amd import _native
    from legolink_amd.link_plan import contiguous_ranges
    from legolink_amd.repair_attention import RepairAttentionPlan
    from legolink_amd.workloads import make_workload

    device = torch.device("cuda", 0)
    full = make_workload(args.workload)
    group = 7 if full.shape.kv_heads == 4 else 8  # Qwen2.5-7B: 28 / 4; Qwen3-32B: 64 / 8
    workload = tp_share(full, args.tp)
    shape = workload.shape
    if args.head_dim:
        shape = dataclasses.replace(shape, head_dim=args.head_dim)
    if args.heads:
        q_heads, kv_heads = (int(x) for x in args.heads.split("/"))
        if q_heads < 1 or kv_heads < 1 or q_heads % kv_heads:
            raise SystemExit("--heads takes Q/KV with Q a multiple of KV")
        shape = dataclasses.replace(shape, kv_heads=kv_heads)
        group = q_heads // kv_heads
    q_heads = group * shape.kv_heads
    generator = torch.Generator(device=device).manual_seed(20260824)
    key = torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, generator=generator,
                      device=device).to(torch.bfloat16)
    value = torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, generator=generator,
                        device=device).to(torch.bfloat16)
    spans = []
    for destination, plan in workload.link_requests()[1]:
        slots = torch.from_numpy(destination).to(device)
        for start, end in contiguous_ranges(plan["imp_indices"]):
            spans.append((slots, int(start), int(end)))
    plan_times = []
    for _ in range(4):  # the first plan pays torch's first-use costs: report the median of the rest
        # The planner keeps its last plan per thread; plan other rows first so
        # that every timed plan is computed, as for a new batch.
        _native.repair_attention_plan(np.array([[0, 0, 1, 0]], dtype=np.int64), q_heads, shape.kv_heads, 0)
        torch.cuda.synchronize(device)  # earlier device work is not the plan's
        plan_start = time.perf_counter()
        plan = RepairAttentionPlan(spans, num_q_heads=q_heads, num_kv_heads=shape.kv_heads,
                                   head_dim=shape.head_dim, pool_size=workload.num_slots,
                                   split_tokens=args.split_tokens)
        torch.cuda.synchronize(device)
        plan_times.append((time.perf_counter() - plan_start) * 1e3)
    plan_ms = float(np.median(plan_times[1:]))
    query = torch.randn(plan.num_queries, q_heads, shape.head_dim, generator=generator,
                        device=device).to(torch.bfloat16)
    output = torch.empty_like(query)
    for _ in range(args.warmup):
        plan.run(query, key, value, output=output)
    torch.cuda.synchronize(device)
    stream = torch.cuda.current_stream(device)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    for start_event, end_event in events:
        start_event.record(stream)
        plan.run(query, key, value, output=output)
        end_event.record(stream)
    torch.cuda.synchronize(device)
    ms = float(np.mean([s.elapsed_time(e) for s, e in events]))
    flops = plan.algorithmic_flops
    achieved = flops / (ms / 1e3) / 1e12
    kv_bytes = plan.kv_bytes_read
    log(f"repair attention {workload.name}: {len(spans)} spans, {plan.num_queries} queries, "
        f"plan {plan.info}, {ms:.4f} ms per layer")
    baseline = None
    if args.cpu_baseline:
        baseline = cpu_attention_baseline(spans, query, key, value, q_heads, shape.head_dim,
                                          args.cpu_attention_gflop)
    print(json.dumps({
        "metric": "sparse repair attention TFLOP/s (bf16 MFMA, one layer)",
        "value": round(achieved, 2),
        "unit": "TFLOP/s",
        "ms_per_layer": round(ms, 5),
        "steps": args.steps,
        "warmup": args.warmup,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) bf16 queries and KV pool",
        "config": {"workload": f"{workload.name}: repair spans of {workload.description}",
                   "spans": len(spans), "queries": plan.num_queries, "q_heads": q_heads,
                   "kv_heads": shape.kv_heads, "head_dim": shape.head_dim,
                   "algorithmic_flops": flops, "plan": plan.info, "host_plan_ms": round(plan_ms, 3)},
        "roofline": {"bound": "mfma", "kernel": f"repair_attention_m32_kernel<{shape.head_dim}>", "achieved": round(achieved, 2),
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": round(achieved / 2500.0, 4),
                     "kv_bytes_gathered": kv_bytes,
                     "kv_gather_GBps": round(kv_bytes / (ms / 1e3) / 1e9, 1)},
        "cpu_baseline": baseline,
    }), flush=True)


def tp_share(workload, tp: int):
    try:
        return workload.rank_share(tp)
    except ValueError as error:
        raise SystemExit(f"--tp: {error}")


def cpu_attention_baseline(spans, query, key, value, q_heads: int, head_dim: int, gflop_budget: float) -> dict:
    """The reference's restated repair attention (gqa_attention over the logical
    causal mask, tests/pic/reference/attention_reference.py:8-48) in fp32 torch
    on the host cores, over the first spans of the workload up to a flop budget."""

    import math

    import numpy as np
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    kv_heads = key.shape[1]
    group = q_heads // kv_heads
    scale = 1.0 / math.sqrt(head_dim)
    jobs, flops, cursor = [], 0, 0
    for slots, start, end in spans:
        n = end - start
        if flops and flops + 4 * head_dim * q_heads * n * (start + end + 1) // 2 > gflop_budget * 1e9:
            break
        rows = slots[:end]
        jobs.append((query[cursor : cursor + n].float().cpu(), key[rows].float().cpu(),
                     value[rows].float().cpu(), start, end))
        flops += 4 * head_dim * q_heads * n * (start + end + 1) // 2
        cursor += n

    def run() -> None:
        for q, k, v, start, end in jobs:
            positions = torch.arange(start, end)[:, None]
            visible = torch.arange(end)[None, :] <= positions                       # [n, end]
            kh = k.repeat_interleave(group, dim=1).permute(1, 2, 0).contiguous()    # [hq, d, end]
            vh = v.repeat_interleave(group, dim=1).permute(1, 0, 2).contiguous()    # [hq, end, d]
            scores = torch.bmm(q.permute(1, 0, 2).contiguous(), kh) * scale        # [hq, n, end]
            scores = scores.masked_fill(~visible[None], float("-inf"))
            torch.bmm(torch.softmax(scores, dim=-1), vh)

    run()
    times = []
    for _ in range(3):
        start = time.perf_counter()
        run()
        times.append(time.perf_counter() - start)
    seconds = float(np.median(times))
    return {"value": round(flops / seconds / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"first {len(jobs)} of {len(spans)} spans ({flops / 1e9:.1f} GFLOP): fp32 torch "
                      f"gather -> masked softmax attention per span, {cores} threads, median of 3 after a "
                      f"warm-up"}


def main() -> int:
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the link step on one GPU only; there is no multi-GPU "
              "configuration to run (the link shards by KV head / request with no exchange step).",
              file=sys.stderr)
        return 2
    if args.copy_calibration:
        copy_calibration(args)
        return 0
    if args.run_sweep:
        run_sweep(args)
        return 0
    if args.calibration_only:
        calibration_only(args)
        return 0
    if args.repair_attention:
        repair_attention_bench(args)
        return 0

    import numpy as np
    import torch

    from legolink_amd.link_runtime import KVLinkExecutor, KVPool
    from legolink_amd.registry import LegoLinkBlockRegistry
    from legolink_amd.rope import RotarySpec, build_cos_sin_cache
    from legolink_amd.workloads import make_workload

    device = torch.device("cuda", 0)
    host_start = time.perf_counter()
    workload = tp_share(make_workload(args.workload), args.tp)
    shape = workload.shape
    log(f"workload {workload.name}: {workload.description}")
    keys, values = [], []
    generator = torch.Generator(device=device).manual_seed(20260824)
    for _ in range(shape.layers):
        keys.append(torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, dtype=torch.bfloat16,
                                device=device, generator=generator))
        values.append(torch.randn(workload.num_slots, shape.kv_heads, shape.head_dim, dtype=torch.bfloat16,
                                  device=device, generator=generator))
    table = build_cos_sin_cache(workload.max_position + 1, workload.rotary_dim, theta=workload.theta).to(device)
    repaired_k = torch.randn(shape.layers, workload.repair_rows, shape.kv_heads, shape.head_dim,
                             dtype=torch.bfloat16, device=device, generator=generator)
    repaired_v = torch.randn_like(repaired_k)
    torch.cuda.synchronize(device)
    setup_s = time.perf_counter() - host_start

    # Host preparation of one link through the executor, as a serving loop runs
    # it: registry lookup -> plan -> token maps built on the device -> launch
    # arguments validated and built.  Timed separately (median of 5); not part
    # of the step.  Batched workloads (several requests) prepare one link.
    registry = LegoLinkBlockRegistry()
    blocks, requests = workload.link_requests()
    arena = None
    clone = args.storage == "clone"
    if clone:
        from legolink_amd.link_runtime import SnapshotArena
        arena = SnapshotArena.allocate(num_slots=sum(source.size for source, _ in blocks.values()),
                                       num_layers=shape.layers, num_heads=shape.kv_heads,
                                       head_dim=shape.head_dim, device=device)
    # The fused rounding (fp32 rotation, one rounding at the store) is what the
    # link is measured on; clone blocks take the reference's torch-path rounding
    # ("auto" falls back to it, as the reference does).  --rounding eager times
    # the torch path's rounding on the same kernel.
    fused_mode = "disabled" if args.rounding == "eager" else ("auto" if clone else "required")
    executor = KVLinkExecutor(registry, RotarySpec(table, rotary_dim=workload.rotary_dim),
                              end_layer=shape.layers, num_warps=args.waves_per_block,
                              layers_per_wave=args.layers_per_wave,
                              layer_groups_per_block=args.layer_groups_per_block, arena=arena,
                              fused_mode=fused_mode, delta_staging=args.delta_staging,
                              visit_order=None if args.visit_order == "auto" else args.visit_order)
    pool = KVPool(keys, values)
    row_bytes = 2 * shape.kv_heads * shape.head_dim * 2  # one token's K and V row, one layer
    storage = {"mode": args.storage}
    if clone:
        # Capture every block into the arena (a bit copy of all its layers,
        # capture_compile_blocks), then link from the arena.
        sources = {key: torch.from_numpy(source).to(device) for key, (source, _) in blocks.items()}

        entries = [{"cache_key": key, "token_ids": range(source.size), "slots": sources[key],
                    "storage_mode": "clone", "compile_local_positions": local}
                   for key, (source, local) in blocks.items()]

        def capture_all() -> float:
            torch.cuda.synchronize(device)
            start = time.perf_counter()
            executor.capture_blocks(pool, entries)
            torch.cuda.synchronize(device)
            return time.perf_counter() - start

        capture_all()  # the first pass also loads the kernels
        for key in blocks:
            executor.release_block(key)
        capture_s = capture_all()
        captured = int(arena.size)
        capture_bytes = captured * shape.layers * row_bytes * 2
        # The capture's device copy alone: the same one-launch row copy over
        # the same maps (it rewrites identical rows), 10 launches back to back
        # between two HIP events so that host work overlaps the kernels.
        handles = registry.lookup_legolink_blocks(list(blocks)).matched_handles
        copy_src = torch.cat([sources[handle.cache_key] for handle in handles])
        copy_dst = torch.cat([handle.kv_slots for handle in handles])
        zeros = torch.zeros_like(copy_src)

        def copy_once() -> None:
            executor._copy_rows(destination=arena, source=pool, source_slots=copy_src, destination_slots=copy_dst,
                                local=zeros, global_=zeros, prefix=captured)

        copy_once()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(10):
            copy_once()
        end.record()
        end.synchronize()
        copy = begin.elapsed_time(end) / 10
        storage.update({"captured_tokens": captured, "capture_ms": round(capture_s * 1e3, 3),
                        "capture_GBps": round(capture_bytes / capture_s / 1e9, 1),
                        "capture_copy_ms": round(copy, 4),
                        "capture_copy_GBps": round(capture_bytes / (copy / 1e3) / 1e9, 1)})
    else:
        for key, (source, local) in blocks.items():
            registry.register_legolink_block(key, range(source.size), torch.from_numpy(source).to(device),
                                             compile_local_positions=local.tolist())
    requests = [(torch.from_numpy(slots).to(device), plan) for slots, plan in requests]
    compact = args.repair_rows == "compact"
    prepare_ms = []
    for _ in range(11):
        torch.cuda.synchronize(device)
        prepare_start = time.perf_counter()
        if len(requests) == 1:
            prepared = executor.prepare_link(pool, requests[0][0], requests[0][1], boundary_repair_aware=True,
                                             compact_repair_rows=compact)
        else:
            prepared = executor.prepare_links(pool, requests, boundary_repair_aware=True,
                                              compact_repair_rows=compact)
        prepare_ms.append((time.perf_counter() - prepare_start) * 1e3)
    torch.cuda.synchronize(device)
    host_prepare_ms = float(np.median(prepare_ms[1:]))  # the first pays first-use costs
    attention_plan_ms = time_attention_plan(workload, requests, device)
    if (prepared.linked_token_count != workload.tokens - workload.repair_rows
            or int(prepared.repair_offsets.size) != workload.repair_rows):
        raise RuntimeError("prepared link does not match the workload's token and repair-row counts")
    link = prepared.launch
    scatter = prepared.prepare_write_repaired(repaired_k, repaired_v)
    launch = dict(prepared.launch_info[0], stream_source_rows=bool(prepared.stream_source_rows),
                  rounding=prepared.rounding, visit_order=prepared.visit_order)
    log(f"setup {setup_s:.1f}s; host prepare {host_prepare_ms:.2f} ms; link launch {launch}")

    for _ in range(args.warmup):
        link()
        scatter()
    torch.cuda.synchronize(device)
    log(f"warmup {args.warmup} steps done; timing {args.steps} steps")

    stream = torch.cuda.current_stream(device)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
               torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize(device)
    wall_start = time.perf_counter()
    for start, middle, end in events:
        start.record(stream)
        link()
        middle.record(stream)
        scatter()
        end.record(stream)
    torch.cuda.synchronize(device)
    wall_s = time.perf_counter() - wall_start
    link_ms = [s.elapsed_time(m) for s, m, _ in events]
    scatter_ms = [m.elapsed_time(e) for _, m, e in events]
    gpu_ms = events[0][0].elapsed_time(events[-1][2]) / args.steps
    ms_per_step = wall_s * 1e3 / args.steps
    log(f"timed: {ms_per_step:.4f} ms/step wall, {gpu_ms:.4f} ms/step events, "
        f"link {np.mean(link_ms):.4f} ms, scatter {np.mean(scatter_ms):.4f} ms")
    if clone:
        # Group promotion (_promote_reconstructed_group): the first request's
        # linked rows copied into free pool slots with K rotated back to local
        # positions, then registered as a block.  Median of 5.
        destination = requests[0][0]
        count = int(destination.numel())
        used = np.union1d(workload.source_slots, workload.destination_slots)
        free = torch.from_numpy(np.setdiff1d(np.arange(workload.num_slots), used)[:count]).to(device)
        promote_ms = []
        for index in range(6):
            torch.cuda.synchronize(device)
            promote_start = time.perf_counter()
            executor.promote_group(pool, destination, group_start=0, group_end=count, new_slots=free,
                                   cache_key=f"promoted-{index}", token_ids=range(count))
            torch.cuda.synchronize(device)
            promote_ms.append((time.perf_counter() - promote_start) * 1e3)
            registry.evict_legolink_block(f"promoted-{index}")
        promote = float(np.median(promote_ms[1:]))
        storage.update({"promoted_tokens": count, "promote_ms": round(promote, 3),
                        "promote_GBps": round(count * shape.layers * row_bytes * 2 / (promote / 1e3) / 1e9, 1)})

    # Per-link latency as a serving loop sees it: a fresh prepare (registry
    # lookup, run plan, device map build, launch arguments), the link and the
    # repaired-row write-back, synchronised, per repetition (median of 10).
    end_to_end_ms = []
    for _ in range(11):
        torch.cuda.synchronize(device)
        e2e_start = time.perf_counter()
        if len(requests) == 1:
            fresh = executor.prepare_link(pool, requests[0][0], requests[0][1], boundary_repair_aware=True,
                                          compact_repair_rows=compact)
        else:
            fresh = executor.prepare_links(pool, requests, boundary_repair_aware=True, compact_repair_rows=compact)
        fresh.launch()
        fresh.write_repaired(repaired_k, repaired_v)
        torch.cuda.synchronize(device)
        end_to_end_ms.append((time.perf_counter() - e2e_start) * 1e3)
    end_to_end_link_ms = float(np.median(end_to_end_ms[1:]))
    del fresh
    log(f"end to end per link (fresh prepare + link + write-back): {end_to_end_link_ms:.3f} ms")
    # Every link above counted the tokens its kernel skipped for a bad index:
    # the synthetic plans have none.
    executor.check_skipped_rows()

    bytes_info = workload.algorithmic_bytes()
    ceiling = None
    if args.tp == 1 and not clone:
        try:
            ceiling = same_maps_ceiling(torch, prepared, keys, values, bytes_info["link_bytes"], args)
        except RuntimeError as error:  # a calibration launch refused these maps: report without it
            log(f"same-maps ceiling not measured: {error}")
    if args.tp == 1:
        committed = load_pattern_ceiling(workload.name)
        if ceiling is None:
            ceiling = committed
        elif committed is not None:
            ceiling["synthetic_sweep"] = committed
    total_bytes = bytes_info["total_bytes"]
    value = total_bytes / (ms_per_step / 1e3) / 1e9
    link_avg_ms = float(np.mean(link_ms))
    achieved = bytes_info["link_bytes"] / (link_avg_ms / 1e3) / 1e9
    traffic = load_traffic(workload.name, bytes_info["link_bytes"]) if args.tp == 1 else None
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) bf16 K/V pool, seeded slot permutation and block layout",
        "config": {
            "workload": f"{workload.name}: {workload.description}",
            "layers": shape.layers,
            "kv_heads": shape.kv_heads,
            "head_dim": shape.head_dim,
            "pool_slots": workload.num_slots,
            "linked_tokens": workload.tokens,
            "repair_rows": workload.repair_rows,
            "blocks": len(workload.block_lengths),
            "requests": workload.requests,
            "prefix_token_count": workload.prefix_token_count,
            "algorithmic_bytes_per_step": total_bytes,
            "tp_share": f"1/{args.tp} of the KV heads (one rank's head shard)" if args.tp > 1 else None,
        },
        "tokens_linked_per_s": round(workload.tokens / (ms_per_step / 1e3), 1),
        "hbm_fraction": round(value / HBM_PEAK_GBPS, 4),
        "link_kernel_ms": round(link_avg_ms, 5),
        "scatter_kernel_ms": round(float(np.mean(scatter_ms)), 5),
        "event_ms_per_step": round(gpu_ms, 5),
        "host_prepare_ms": round(host_prepare_ms, 3),
        "host_attention_plan_ms": None if attention_plan_ms is None else round(attention_plan_ms, 3),
        "end_to_end_link_ms": round(end_to_end_link_ms, 3),
        "repair_rows_mode": args.repair_rows,
        "storage": storage,
        "launch": launch,
        "roofline": {
            "bound": "hbm",
            "kernel": "kv_link_vec_kernel" if launch["kernel"] == "vector" else "kv_link_generic_kernel",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic if not clone else None,
            "algorithmic_bytes_per_launch": bytes_info["link_bytes"],
            "pattern_ceiling": ceiling,
        },
        "cpu_baseline": None,
    }
    del keys, values, pool, prepared, link, scatter
    torch.cuda.empty_cache()
    if args.cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(workload, args)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
