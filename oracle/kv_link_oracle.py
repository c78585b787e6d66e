"""CPU oracle for the LegoLink KV link step.

TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg may import this module, and only to check results.  The product
path (legolink_amd) never calls it.

Two independent restatements of the per-token K arithmetic of the reference,
which the tests check against each other bit for bit:

* ``rerotate_rows_c``      plain C (ll_oracle.c), one element at a time;
* ``rerotate_rows_numpy``  numpy float32 ufuncs, one rounding per operation.

Both take ``rounding``: ``FUSED`` (the default) follows the reference's fused
link kernel (patched_sglang_files/python/sglang/srt/legolink_triton.py:
302-547); ``EAGER`` follows its torch path (pic_runtime.py:6039-6058 and
:1874-1885), whose rounding points differ.

plus the pool-level semantics around them:

* ``link_pool``    gather -> re-rotate (t >= prefix) -> scatter for every layer,
                   repair-masked tokens untouched; V and prefix K bit copies
                   (legolink_triton.py:332-347, :471-547;
                   pic_runtime.py:4881-5013 for the prefix and mask rules);
* ``scatter_rows`` repaired-row write-back (tests/pic/reference/repair_reference.py:14-25).

Arrays are numpy uint16 bit patterns of bf16/fp16 values: pools are
``[layers][slots, heads, dim]`` lists, rows ``[tokens, heads, dim]``.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
C_SOURCE = ORACLE_DIR / "ll_oracle.c"
C_LIBRARY = ORACLE_DIR / "libll_oracle.so"

F16, BF16, F32 = 1, 2, 3
FUSED, EAGER = 0, 1
_DTYPE_CODES = {"float16": F16, "bfloat16": BF16, "float32": F32}


def build_c_oracle() -> Path:
    """gcc -O2 -ffp-contract=off: scalar SSE float ops, each rounded to nearest even."""

    temporary = C_LIBRARY.with_suffix(".so.tmp")
    subprocess.run(
        [
            "gcc",
            "-O2",
            "-ffp-contract=off",
            "-fno-fast-math",
            "-std=c11",
            "-Wall",
            "-shared",
            "-fPIC",
            "-o",
            str(temporary),
            str(C_SOURCE),
        ],
        check=True,
    )
    temporary.replace(C_LIBRARY)
    return C_LIBRARY


_c_lib: ctypes.CDLL | None = None


def c_oracle() -> ctypes.CDLL:
    global _c_lib
    if _c_lib is None:
        if not C_LIBRARY.is_file() or (
            C_SOURCE.is_file() and C_SOURCE.stat().st_mtime > C_LIBRARY.stat().st_mtime
        ):
            build_c_oracle()
        lib = ctypes.CDLL(str(C_LIBRARY))
        ptr = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.llo_rerotate_rows.argtypes = [
            ptr, ptr, i64, i64, i64, ctypes.c_int, ptr, ctypes.c_int,
            i64, i64, i64, ptr, ptr, i64, ctypes.c_int, i64, ctypes.c_int,
        ]
        lib.llo_rerotate_rows.restype = ctypes.c_int
        lib.llo_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.llo_f32_to_bf16.restype = ctypes.c_uint16
        lib.llo_f32_to_f16.argtypes = [ctypes.c_float]
        lib.llo_f32_to_f16.restype = ctypes.c_uint16
        lib.llo_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.llo_f16_to_f32.restype = ctypes.c_float
        for name in ("llo_f32_to_bf16_array", "llo_f32_to_f16_array", "llo_f16_to_f32_array"):
            getattr(lib, name).argtypes = [ptr, ptr, i64]
            getattr(lib, name).restype = None
        _c_lib = lib
    return _c_lib


def c_f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    c_oracle().llo_f32_to_bf16_array(values.ctypes.data, out.ctypes.data, values.size)
    return out


def c_f32_to_f16_bits(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    c_oracle().llo_f32_to_f16_array(values.ctypes.data, out.ctypes.data, values.size)
    return out


def c_f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    c_oracle().llo_f16_to_f32_array(bits.ctypes.data, out.ctypes.data, bits.size)
    return out


# ---------------------------------------------------------------------------
# Element conversions (numpy).
# ---------------------------------------------------------------------------
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round to nearest even; NaN -> 0x7fc0."""

    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded[nan] = 0x7FC0
    return rounded


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def _to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    return bf16_bits_to_f32(bits) if dtype == BF16 else f16_bits_to_f32(bits)


def _from_f32(values: np.ndarray, dtype: int) -> np.ndarray:
    return f32_to_bf16_bits(values) if dtype == BF16 else f32_to_f16_bits(values)


def _round_bf16(values: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(values))


def _stored_as(values: np.ndarray, dtype: int) -> np.ndarray:
    """fp32 values stored in ``dtype`` and read back (F32: unchanged)."""

    if dtype == F32:
        return np.asarray(values, dtype=np.float32)
    return _to_f32(_from_f32(values, dtype), dtype)


def cache_to_f32(cache: np.ndarray, cache_dtype: int) -> np.ndarray:
    if cache_dtype == F32:
        return np.asarray(cache, dtype=np.float32)
    return _to_f32(cache, cache_dtype)


# ---------------------------------------------------------------------------
# Per-token K arithmetic.
# ---------------------------------------------------------------------------
def rerotate_rows_numpy(
    rows: np.ndarray,
    local: np.ndarray,
    global_: np.ndarray,
    cache: np.ndarray,
    *,
    key_dtype: int,
    cache_dtype: int,
    rotary_dim: int,
    neox: bool,
    prefix: int,
    rounding: int = FUSED,
) -> np.ndarray:
    """rows [T, H, D] uint16 -> re-rotated rows (t >= prefix), copies (t < prefix)."""

    out = np.array(rows, dtype=np.uint16, copy=True)
    tail = slice(int(prefix), rows.shape[0])
    if rows.shape[0] <= prefix:
        return out
    half = rotary_dim // 2
    table = cache_to_f32(cache, cache_dtype)
    lp = np.asarray(local, dtype=np.int64)[tail]
    gp = np.asarray(global_, dtype=np.int64)[tail]
    lc = table[lp, :half][:, None, :]
    ls = table[lp, half : 2 * half][:, None, :]
    gc = table[gp, :half][:, None, :]
    gs = table[gp, half : 2 * half][:, None, :]
    if neox:
        d1 = np.arange(half)
        d2 = d1 + half
    else:
        d1 = 2 * np.arange(half)
        d2 = d1 + 1
    x1 = _to_f32(rows[tail][:, :, d1], key_dtype)
    x2 = _to_f32(rows[tail][:, :, d2], key_dtype)
    if rounding == EAGER:
        # the delta as tensors of the cache's dtype, cast to the key dtype,
        # then the rotation as tensors of the key dtype
        dc = _stored_as(_stored_as(gc * lc, cache_dtype) + _stored_as(gs * ls, cache_dtype), cache_dtype)
        ds = _stored_as(_stored_as(gs * lc, cache_dtype) - _stored_as(gc * ls, cache_dtype), cache_dtype)
        dc = _stored_as(dc, key_dtype)
        ds = _stored_as(ds, key_dtype)
        o1 = _from_f32(_stored_as(x1 * dc, key_dtype) - _stored_as(x2 * ds, key_dtype), key_dtype)
        o2 = _from_f32(_stored_as(x2 * dc, key_dtype) + _stored_as(x1 * ds, key_dtype), key_dtype)
    elif key_dtype == BF16 and cache_dtype != F32:
        dc = _round_bf16(_round_bf16(gc * lc) + _round_bf16(gs * ls))
        ds = _round_bf16(_round_bf16(gs * lc) - _round_bf16(gc * ls))
        first_cos = _round_bf16(x1 * dc)
        second_sin = _round_bf16(x2 * ds)
        second_cos = _round_bf16(x2 * dc)
        first_sin = _round_bf16(x1 * ds)
        o1 = _from_f32(first_cos - second_sin, BF16)
        o2 = _from_f32(second_cos + first_sin, BF16)
    else:
        dc = gc * lc + gs * ls
        ds = gs * lc - gc * ls
        o1 = _from_f32(x1 * dc - x2 * ds, key_dtype)
        o2 = _from_f32(x2 * dc + x1 * ds, key_dtype)
    block = out[tail]
    block[:, :, d1] = o1
    block[:, :, d2] = o2
    out[tail] = block
    return out


def rerotate_rows_c(
    rows: np.ndarray,
    local: np.ndarray,
    global_: np.ndarray,
    cache: np.ndarray,
    *,
    key_dtype: int,
    cache_dtype: int,
    rotary_dim: int,
    neox: bool,
    prefix: int,
    rounding: int = FUSED,
) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.uint16)
    local = np.ascontiguousarray(local, dtype=np.int64)
    global_ = np.ascontiguousarray(global_, dtype=np.int64)
    cache = np.asarray(cache)
    itemsize = cache.itemsize
    out = np.empty_like(rows)
    tokens, heads, dim = rows.shape
    rc = c_oracle().llo_rerotate_rows(
        rows.ctypes.data,
        out.ctypes.data,
        tokens,
        heads,
        dim,
        key_dtype,
        cache.ctypes.data,
        cache_dtype,
        cache.shape[0],
        cache.strides[0] // itemsize,
        cache.strides[1] // itemsize,
        local.ctypes.data,
        global_.ctypes.data,
        rotary_dim,
        1 if neox else 0,
        int(prefix),
        int(rounding),
    )
    if rc != 0:
        raise IndexError("a remapped token's position is outside the cos/sin cache")
    return out


# ---------------------------------------------------------------------------
# Pool-level semantics.
# ---------------------------------------------------------------------------
def skipped_token_mask(
    src: np.ndarray,
    dst: np.ndarray,
    local: np.ndarray,
    global_: np.ndarray,
    *,
    source_slots: int,
    destination_slots: int,
    cache_rows: int,
    prefix: int,
    repair_mask: np.ndarray | None = None,
) -> np.ndarray:
    """Tokens the link skips for an out-of-range index: unmasked, and a slot
    outside its pool, or (remapped tokens, t >= prefix) a position outside
    the table.  The reference leaves such inputs undefined in its fused kernel
    (legolink_triton.py:336-339 load the slots and positions unchecked) and
    raises in its torch path (index_select, pic_runtime.py:5534-5599); the
    library skips them and counts them, and this is that contract."""

    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    local = np.asarray(local, dtype=np.int64)
    global_ = np.asarray(global_, dtype=np.int64)
    masked = np.zeros(src.shape[0], dtype=bool) if repair_mask is None else np.asarray(repair_mask) != 0
    bad = (src < 0) | (src >= source_slots) | (dst < 0) | (dst >= destination_slots)
    remap = np.arange(src.shape[0]) >= prefix
    bad_position = (local < 0) | (local >= cache_rows) | (global_ < 0) | (global_ >= cache_rows)
    return ~masked & (bad | (remap & bad_position))


def link_pool(
    key_layers: list[np.ndarray],
    value_layers: list[np.ndarray],
    src: np.ndarray,
    dst: np.ndarray,
    local: np.ndarray,
    global_: np.ndarray,
    cache: np.ndarray,
    *,
    key_dtype: int,
    cache_dtype: int,
    rotary_dim: int,
    neox: bool,
    prefix: int,
    repair_mask: np.ndarray | None = None,
    rerotate=rerotate_rows_c,
    source_key_layers: list[np.ndarray] | None = None,
    source_value_layers: list[np.ndarray] | None = None,
    rounding: int = FUSED,
) -> tuple[list[np.ndarray], list[np.ndarray]]:
    """Expected pool after the link; the inputs are not modified.  Source rows
    come from ``source_*_layers`` when given, else from the pool itself."""

    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    keep = np.ones(src.shape[0], dtype=bool)
    if repair_mask is not None:
        keep = np.asarray(repair_mask) == 0
    source_key_layers = key_layers if source_key_layers is None else source_key_layers
    source_value_layers = value_layers if source_value_layers is None else source_value_layers
    # Tokens with an out-of-range index are skipped (skipped_token_mask); the
    # rows of the others are computed with those indices replaced by 0.
    skipped = skipped_token_mask(src, dst, local, global_, source_slots=source_key_layers[0].shape[0],
                                 destination_slots=key_layers[0].shape[0], cache_rows=cache.shape[0],
                                 prefix=prefix, repair_mask=repair_mask)
    keep = keep & ~skipped
    # Masked and skipped tokens store nothing: read row 0 and position 0 for
    # any index of theirs that is out of range.
    local = np.asarray(local, dtype=np.int64)
    global_ = np.asarray(global_, dtype=np.int64)
    cache_rows = cache.shape[0]
    src = np.where((src >= 0) & (src < source_key_layers[0].shape[0]), src, 0)
    local = np.where((local >= 0) & (local < cache_rows), local, 0)
    global_ = np.where((global_ >= 0) & (global_ < cache_rows), global_, 0)
    if cache_rows == 0:  # every remapped token is skipped: nothing reads the table
        prefix = src.shape[0]
    out_k, out_v = [], []
    for key, value, source_key, source_value in zip(
        key_layers, value_layers, source_key_layers, source_value_layers
    ):
        rows = rerotate(
            source_key[src],
            local,
            global_,
            cache,
            key_dtype=key_dtype,
            cache_dtype=cache_dtype,
            rotary_dim=rotary_dim,
            neox=neox,
            prefix=prefix,
            rounding=rounding,
        )
        new_k = key.copy()
        new_v = value.copy()
        new_k[dst[keep]] = rows[keep]
        new_v[dst[keep]] = source_value[src[keep]]
        out_k.append(new_k)
        out_v.append(new_v)
    return out_k, out_v


def scatter_rows(
    key_layers: list[np.ndarray],
    value_layers: list[np.ndarray],
    dst: np.ndarray,
    repaired_keys: np.ndarray,
    repaired_values: np.ndarray,
) -> tuple[list[np.ndarray], list[np.ndarray]]:
    """K_l[dst[r]] = repaired_keys[l, r]; V likewise (rows written in order)."""

    dst = np.asarray(dst, dtype=np.int64)
    out_k, out_v = [], []
    for layer, (key, value) in enumerate(zip(key_layers, value_layers)):
        new_k = key.copy()
        new_v = value.copy()
        new_k[dst] = repaired_keys[layer]
        new_v[dst] = repaired_values[layer]
        out_k.append(new_k)
        out_v.append(new_v)
    return out_k, out_v
