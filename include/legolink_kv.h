/*
 * legolink_kv.h - C ABI of the MI355X (gfx950) LegoLink KV link library
 * (liblegolink_kv.so).
 *
 * The library moves registered KV blocks of a paged KV pool into a new
 * request's slots: it gathers source rows, re-rotates K from each token's
 * compile-time RoPE position to its request-global position, and scatters
 * the result into destination rows; V rows and non-rotated K rows are moved
 * bit-exactly.  A second entry writes repaired boundary rows (imp_indices)
 * into the pool.
 *
 * Pool layout (unchanged from the reference, patched_sglang_files/python/
 * sglang/srt/legolink_triton.py:184-193 and pic_runtime.py:6283-6289): every
 * layer owns one dense [num_slots, num_heads, key_head_dim] K buffer and one
 * dense [num_slots, num_heads, value_head_dim] V buffer, both fp16 or bf16.
 * Layers are separate allocations, so the entries take host arrays of
 * per-layer device pointers.
 *
 * Conventions
 *   - Every integer field is int64_t, so the structs have no padding and a
 *     ctypes / cgo / JNI mirror is a flat list of 8-byte fields.
 *   - Device pointers are plain addresses in the device's HIP address space.
 *     Host pointers are marked "host".
 *   - Work is enqueued on `stream` (a hipStream_t) and is asynchronous.  No
 *     entry allocates device memory, synchronises or keeps state between
 *     calls other than the thread-local error string and, in
 *     ll_repair_attention_plan, a thread-local copy of the last plan it
 *     computed (a cache that no result depends on).  Entries are reentrant.
 *   - A return value of 0 is success; a negative value is one of the LL_ERR_*
 *     codes below, and ll_last_error() then holds a message.
 *   - Rows whose slot index lies outside [0, num_slots) and remapped tokens
 *     whose positions lie outside [0, cos_sin_rows) are neither read nor
 *     written (the kernels bound-check every index they dereference).
 *   - Preconditions that are NOT checked: source rows and destination rows
 *     are disjoint, and destination slots are pairwise distinct.
 *     Overlapping or repeated destinations race, as in the reference.
 */
#ifndef LEGOLINK_KV_H
#define LEGOLINK_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LL_ABI_VERSION 17

/* hipStream_t, declared without pulling in the HIP headers. */
struct ihipStream_t;
typedef struct ihipStream_t *ll_stream_t;

/* Element type codes (the *_dtype fields). */
enum {
  LL_DTYPE_FLOAT16 = 1,
  LL_DTYPE_BFLOAT16 = 2,
  LL_DTYPE_FLOAT32 = 3,
  LL_DTYPE_INT32 = 4,
  LL_DTYPE_INT64 = 5,
  LL_DTYPE_UINT8 = 6 /* uint8 or bool repair mask */
};

/* Kernel selection (ll_kv_link_args.kernel). */
enum {
  LL_KERNEL_AUTO = 0,   /* vectorised kernel when the shape allows, else generic */
  LL_KERNEL_VECTOR = 1, /* 16-byte row-chunk kernel; LL_ERR_UNSUPPORTED_KERNEL if the shape does not fit */
  LL_KERNEL_GENERIC = 2 /* element-wise kernel for every eligible shape */
};

/*
 * Rounding of re-rotated K (ll_kv_link_args.rounding).  The reference computes
 * the link in two ways that round differently; both are available:
 *   LL_ROUNDING_FUSED  its fused kernel (legolink_triton.py:413-470), which its
 *                      link uses when the fused mode is on and every block is
 *                      read from pool slots;
 *   LL_ROUNDING_EAGER  its torch path (pic_runtime.py:6025-6058 with
 *                      _apply_rotary_emb, :1868-1885), which it uses by default
 *                      (fused mode off, :1307-1308), for every link that holds
 *                      a clone-mode block (:5034-5035) and for group promotion
 *                      (:5914-5919).
 */
enum {
  LL_ROUNDING_FUSED = 0,
  LL_ROUNDING_EAGER = 1
};

/*
 * Where the vector kernel computes each token's RoPE delta
 * (ll_kv_link_args.delta_staging).  The result is the same either way.
 *   LL_DELTA_PER_WAVE   every wave computes its lanes' pairs from the cos/sin
 *                       table itself (each layer group of a token reads the
 *                       token's two table rows again);
 *   LL_DELTA_WORKGROUP  one workgroup holds every layer group of its tokens
 *                       and computes each token's delta once into LDS (the
 *                       two table rows read once per token); neox links
 *                       with full rotary and an fp32 table only, else per
 *                       wave;
 *   LL_DELTA_TABLE      two layer-major launches (two tokens of one layer per
 *                       wave, the GPU working on one layer's buffers at a
 *                       time): the first moves the V rows and writes every
 *                       token's deltas to a table in delta_workspace, the
 *                       second moves the K rows, reading each token's deltas
 *                       from that table.  Neox links with full
 *                       rotary, an fp32 table and rows of a multiple of 1 KiB
 *                       (num_heads * key_head_dim a multiple of 512), and a
 *                       workspace of at least num_tokens * rotary_dim * 4
 *                       bytes, 16-byte aligned; else as LL_DELTA_AUTO;
 *   LL_DELTA_AUTO       workgroup where it fits, the source rows are streamed
 *                       (stream_source_rows) and layer_groups_per_block is 0
 *                       (waves_per_block then sizes per-wave blocks only),
 *                       else per wave.
 */
enum {
  LL_DELTA_AUTO = 0,
  LL_DELTA_PER_WAVE = 1,
  LL_DELTA_WORKGROUP = 2,
  LL_DELTA_TABLE = 3
};

/*
 * Status codes.  Each eligibility code corresponds 1:1 to a reason string of
 * check_fused_kv_link_eligibility (legolink_triton.py:159-247); ll_status_reason()
 * returns that string.
 */
enum {
  LL_OK = 0,
  LL_ERR_INVALID_ARGUMENT = -1,                /* "invalid_argument" (NULL pointer, bad struct_size, negative count) */
  LL_ERR_MHA_3D_KV_BUFFERS_REQUIRED = -2,      /* "mha_3d_kv_buffers_required" */
  LL_ERR_KV_HEAD_LAYOUT_MISMATCH = -3,         /* "kv_head_layout_mismatch" */
  LL_ERR_KV_DTYPE_MISMATCH = -4,               /* "kv_dtype_mismatch" */
  LL_ERR_FP16_OR_BF16_REQUIRED = -5,           /* "fp16_or_bf16_required" */
  LL_ERR_CONTIGUOUS_KV_BUFFERS_REQUIRED = -6,  /* "contiguous_kv_buffers_required" */
  LL_ERR_HEAD_DIMENSION_OUT_OF_RANGE = -7,     /* "head_dimension_out_of_range" */
  LL_ERR_EMPTY_LINK = -8,                      /* "empty_link" */
  LL_ERR_TOKEN_MAP_LENGTH_MISMATCH = -9,       /* "token_map_length_mismatch" */
  LL_ERR_REPAIR_MASK_LENGTH_MISMATCH = -10,    /* "repair_mask_length_mismatch" */
  LL_ERR_BOOLEAN_REPAIR_MASK_REQUIRED = -11,   /* "boolean_repair_mask_required" */
  LL_ERR_INTEGER_TOKEN_MAPS_REQUIRED = -12,    /* "integer_token_maps_required" */
  LL_ERR_EVEN_ROTARY_DIM_REQUIRED = -13,       /* "even_rotary_dim_required" */
  LL_ERR_ROTARY_DIM_EXCEEDS_HEAD_DIM = -14,    /* "rotary_dim_exceeds_head_dim" */
  LL_ERR_UNSUPPORTED_COS_SIN_CACHE = -15,      /* "unsupported_cos_sin_cache" */
  LL_ERR_UNSUPPORTED_COS_SIN_DTYPE = -16,      /* "unsupported_cos_sin_dtype" */
  LL_ERR_PREFIX_OUT_OF_RANGE = -17,            /* "prefix_token_count_out_of_range" (reference raises ValueError) */
  LL_ERR_LAUNCH_CONFIG = -18,                  /* "invalid_launch_config" (reference raises ValueError) */
  LL_ERR_UNSUPPORTED_KERNEL = -19,             /* "unsupported_kernel_for_shape" (LL_KERNEL_VECTOR forced on an unfit shape) */
  LL_ERR_HIP = -20                             /* "hip_error" (launch failed; message from the HIP runtime) */
};

/*
 * Link: for every token t in [0, num_tokens) and every layer l, with S_l the
 * source buffers (source_key_layers / source_value_layers, or the destination
 * pool's own buffers when those tables are NULL):
 *     if repair_mask != NULL and repair_mask[t] != 0: nothing is written;
 *     V_l[destination_slots[t]] = SV_l[source_slots[t]]                    (bit copy)
 *     K_l[destination_slots[t]] = SK_l[source_slots[t]]  if t <  prefix_token_count (bit copy)
 *     K_l[destination_slots[t]] = rerotate(SK_l[source_slots[t]],
 *                                          local_positions[t] -> global_positions[t])
 *                                                        if t >= prefix_token_count
 * rerotate applies, per rotary pair i of every head, the delta rotation
 *     dc = gc*lc + gs*ls,  ds = gs*lc - gc*ls
 *     first'  = first*dc - second*ds,  second' = second*dc + first*ds
 * with (lc, ls) = cos_sin_cache[local][i], cos_sin_cache[local][i + rotary_dim/2]
 * and  (gc, gs) the same at the global position; pairs are (i, i + rotary_dim/2)
 * for neox style and (2i, 2i + 1) otherwise.  Dims >= rotary_dim are copied.
 * Every multiply and add is a separate round-to-nearest-even op (no fused
 * multiply-add).  Rounding points:
 *   LL_ROUNDING_FUSED (legolink_triton.py:413-470): bf16 K with an fp32 cache
 *     computes the delta and the rotation in fp32 and rounds once to bf16 at
 *     the store; bf16 K with a bf16 or fp16 cache rounds every product and sum
 *     (delta and rotation) to bf16; fp16 K computes in fp32 and rounds once to
 *     fp16.
 *   LL_ROUNDING_EAGER (pic_runtime.py:6039-6058, :1874-1885): every product
 *     and sum of the delta is rounded to the cache's dtype (fp32 ops for an
 *     fp32 cache), dc and ds are then rounded to the key dtype, and every
 *     product and sum of the rotation is rounded to the key dtype.
 *
 * Replaces, with num_layers == 1, fused_kv_link_inplace
 * (patched_sglang_files/python/sglang/srt/legolink_triton.py:550-645), and with
 * num_layers == L the per-layer loop that calls it
 * (patched_sglang_files/python/sglang/srt/pic_runtime.py:5168-5208): one launch
 * covers up to 64 layers.  With a separate source pool it also replaces the
 * clone-mode snapshot copy (pic_runtime.py:3519-3527, prefix = all tokens), the
 * link from clone snapshots (pic_runtime.py:5553-5567) and, with the position
 * vectors swapped, the global -> local copy of group promotion
 * (pic_runtime.py:5901-5922).
 */
typedef struct ll_kv_link_args {
  int64_t struct_size;             /* sizeof(ll_kv_link_args) */
  int64_t num_layers;              /* >= 1 */
  void *const *key_layers;         /* host array [num_layers] of device pointers */
  void *const *value_layers;       /* host array [num_layers] of device pointers */
  int64_t num_slots;               /* rows of every layer buffer */
  int64_t num_heads;               /* KV heads per row (this rank's shard) */
  int64_t key_head_dim;            /* 1..256 */
  int64_t value_head_dim;          /* 1..256 */
  int64_t kv_dtype;                /* LL_DTYPE_BFLOAT16 or LL_DTYPE_FLOAT16 */
  int64_t num_tokens;              /* linked tokens, >= 1 */
  const void *source_slots;        /* device [num_tokens], int32 or int64 */
  int64_t source_slots_dtype;
  const void *destination_slots;   /* device [num_tokens], int32 or int64 */
  int64_t destination_slots_dtype;
  const void *local_positions;     /* device [num_tokens], int32 or int64: compile-time RoPE positions */
  int64_t local_positions_dtype;
  const void *global_positions;    /* device [num_tokens], int32 or int64: request-global positions */
  int64_t global_positions_dtype;
  const void *repair_mask;         /* device [num_tokens] uint8/bool, or NULL */
  int64_t repair_mask_dtype;
  const void *cos_sin_cache;       /* device [cos_sin_rows, cos_sin_cols]: cos in [0, r/2), sin in [r/2, r) */
  int64_t cos_sin_dtype;           /* LL_DTYPE_FLOAT32, LL_DTYPE_BFLOAT16 or LL_DTYPE_FLOAT16 */
  int64_t cos_sin_rows;
  int64_t cos_sin_cols;
  int64_t cos_sin_stride_row;      /* elements */
  int64_t cos_sin_stride_col;      /* elements */
  int64_t rotary_dim;              /* even, 2..key_head_dim */
  int64_t is_neox_style;           /* 1: pairs (i, i + r/2); 0: pairs (2i, 2i + 1) */
  int64_t prefix_token_count;      /* tokens [0, prefix) are copied unrotated; 0..num_tokens */
  int64_t kernel;                  /* LL_KERNEL_* */
  int64_t waves_per_block;         /* 0 = default; else 1, 2, 4 or 8 */
  int64_t layers_per_wave;         /* 0 = auto; else >= 1 */
  int64_t layer_groups_per_block;  /* 0 = auto; else divides waves_per_block: waves of one
                                      workgroup that take the same tokens' different layers */
  void *const *source_key_layers;  /* host array [num_layers] of device pointers, or NULL:
                                      read sources from key_layers */
  void *const *source_value_layers;/* host array [num_layers], or NULL (with source_key_layers) */
  int64_t source_num_slots;        /* rows of every source buffer (when the tables are set) */
  int64_t stream_source_rows;      /* 1: each source row is read once (no reuse within the launch)
                                      and the rows exceed the caches: the vector kernel's
                                      full-rotary fp32-table variants read them with non-temporal
                                      loads (+1-2 % on random rows); 0: rows may repeat (batched
                                      requests sharing blocks) or be cache-resident and stay
                                      cacheable.  The result is the same either way.  (ABI 8) */
  int64_t rounding;                /* LL_ROUNDING_FUSED or LL_ROUNDING_EAGER (ABI 9) */
  int64_t delta_staging;           /* LL_DELTA_*; with LL_DELTA_WORKGROUP, waves_per_block (0..16,
                                      0 = 16) caps the workgroup and layer_groups_per_block
                                      must be 0 (ABI 10) */
  uint64_t *skipped_rows;          /* device counter, or NULL (ABI 11): the link adds the number of
                                      unmasked tokens it skipped because a slot lies outside its
                                      pool or, for a remapped token, a position lies outside the
                                      cos/sin table; each such token once per call.  The caller
                                      zeroes it and reads it after the stream's work.  With a
                                      counter, a pool of no rows is rejected (nothing would run
                                      to count) */
  void *delta_workspace;           /* device scratch of LL_DELTA_TABLE, or NULL (ABI 15): the link
                                      writes each token's deltas there before it reads them back;
                                      links that share it must not overlap */
  int64_t delta_workspace_bytes;   /* its size */
} ll_kv_link_args;

/*
 * Repaired-row write-back: for every layer l and row r in [0, num_rows):
 *     K_l[destination_slots[r]] = repaired_key[l][r]    (bit copy, all heads)
 *     V_l[destination_slots[r]] = repaired_value[l][r]
 * repaired_key[l] is the dense [num_rows, num_heads, key_head_dim] block at
 * element offset l * repaired_key_layer_stride (likewise for V).
 *
 * Replaces the repair pass's KV write of the imp_indices rows
 * (patched_sglang_files/python/sglang/srt/flashinfer_sparse_repair.py:2235-2239,
 * whose semantics the reference restates as write_repaired_kv in
 * tests/pic/reference/repair_reference.py:14-25).
 */
typedef struct ll_kv_scatter_args {
  int64_t struct_size;             /* sizeof(ll_kv_scatter_args) */
  int64_t num_layers;
  void *const *key_layers;         /* host array [num_layers] of device pointers */
  void *const *value_layers;       /* host array [num_layers] of device pointers */
  int64_t num_slots;
  int64_t num_heads;
  int64_t key_head_dim;
  int64_t value_head_dim;
  int64_t kv_dtype;                /* LL_DTYPE_BFLOAT16 or LL_DTYPE_FLOAT16 */
  int64_t num_rows;                /* >= 0; 0 is a no-op */
  const void *destination_slots;   /* device [num_rows], int32 or int64 */
  int64_t destination_slots_dtype;
  const void *repaired_key;        /* device */
  int64_t repaired_key_layer_stride;   /* elements */
  const void *repaired_value;      /* device */
  int64_t repaired_value_layer_stride; /* elements */
  int64_t waves_per_block;         /* 0 = default; else 1, 2, 4 or 8 */
} ll_kv_scatter_args;

/*
 * Token maps of a link, built on the device from a plan's runs.
 *
 * A run is a stretch of consecutive request positions taken from one block:
 * token i of the run (0 <= i < token_count) sits at request position
 * p = start_token + i, is written to destination_slots[destination_start + i],
 * reads its rows from source slot source_slots[i] and carries compile-time
 * position local_positions[i] (or local_start + i when local_positions is
 * NULL).  For one request destination_start == start_token; runs of several
 * requests can share one call with their destination slots concatenated.
 * Tokens [repair_begin, repair_end) of the run are repair rows (imp_indices
 * inside the block).  For every token:
 *     d = destination_slots[destination_start + i]
 *     if it is a repair row and repair_offset >= 0:
 *         repair_destination_slots[repair_offset + i - repair_begin] = d
 *     unless it is a repair row of a set without a mask (compacted set):
 *         o = map_offset + i, minus (repair_end - repair_begin) past the
 *             repair rows of a compacted set
 *         maps[s][0][o] = source slot, maps[s][1][o] = d,
 *         maps[s][2][o] = local position, maps[s][3][o] = p  (s = map_set)
 *         repair_mask[s][o] = 1 for a repair row, else 0 (when the set has a mask)
 * maps[s] is an int64 [4, map_capacity[s]] array (row stride map_capacity[s]);
 * its rows are the source_slots, destination_slots, local_positions and
 * global_positions of an ll_kv_link call.  Two sets let a link whose blocks
 * live in two places (pool slots and a snapshot arena) build both launches'
 * maps in one call.
 *
 * Every run is validated on the host before any launch: destination indices
 * inside [0, num_destination_slots), map and repair indices inside their
 * capacities, map_set 0 or 1 with a map array.  The source and local
 * position arrays must hold token_count entries (not checkable).
 *
 * Replaces the per-block map construction of _copy_linked_kv_batched_blocks
 * (patched_sglang_files/python/sglang/srt/pic_runtime.py:4905-5003: slot
 * slices, arange positions, torch.cat of every map, the boundary repair mask
 * built on the host and copied over).
 */
typedef struct ll_link_segment {
  const int64_t *source_slots;     /* device [token_count] */
  const int64_t *local_positions;  /* device [token_count], or NULL: local_start + i */
  int64_t token_count;             /* >= 0 */
  int64_t start_token;             /* request position (global position) of token 0 */
  int64_t destination_start;       /* index of token 0's slot in destination_slots */
  int64_t local_start;
  int64_t repair_begin;            /* 0 <= repair_begin <= repair_end <= token_count */
  int64_t repair_end;
  int64_t map_set;                 /* 0 or 1 */
  int64_t map_offset;              /* map index of the run's first map entry */
  int64_t repair_offset;           /* index of the run's first repair row, or -1: not recorded */
} ll_link_segment;

/*
 * A link's blocks, in plan order, for the run planner.  Block b covers request
 * positions [start_token, start_token + token_count); its tokens' destination
 * indices start at start_token + destination_base (0 for one request; the
 * offset of the block's request when several requests' slots are
 * concatenated).
 */
typedef struct ll_link_block {
  const int64_t *source_slots;     /* device [token_count] */
  const int64_t *local_positions;  /* device [token_count], or NULL: local_start + i */
  int64_t token_count;             /* 0 .. 2^31 - 1 */
  int64_t start_token;             /* 0 .. 2^62 - 1 */
  int64_t destination_base;        /* 0 .. 2^62 - 1 */
  int64_t local_start;
  int64_t map_set;                 /* 0: pool slots, 1: snapshot arena */
  int64_t leading;                 /* 1: an identity block (no token needs a remap): its runs
                                      take the first map entries of its set */
} ll_link_block;

typedef struct ll_link_run_plan_info {
  int64_t num_segments;            /* runs written (or needed, when the outputs are NULL) */
  int64_t map_count[2];            /* map entries of set 0 and set 1 */
  int64_t set_repair_rows[2];      /* repair rows whose tokens belong to each set */
  int64_t set_prefix[2];           /* identity entries heading each set's maps */
  int64_t repair_count;            /* repair rows in blocks (write-back order: plan order) */
} ll_link_run_plan_info;

/*
 * Run planner (host only): cuts a link's blocks into the runs of
 * ll_kv_build_link_maps.  repair_positions are destination indices (request
 * positions for one request), in any order, duplicates allowed; only those
 * inside a block count.  A run is a stretch of one block holding at most one
 * contiguous stretch of repair rows; runs are in plan order.  With compact
 * the repair rows take no map entry (else they are flagged in the set's
 * mask).  Leading blocks' runs head their set's maps (the identity prefix);
 * the other runs follow in plan order.  Outputs: the runs (segments), the
 * block of every run (segment_blocks), and the concatenation offset of every
 * repair row in plan order (repair_offsets); any of them may be NULL, and
 * with all three NULL the call only fills info (sizing).  A run count of at
 * most num_blocks + num_repair_positions fits every plan.
 *
 * Replaces the host loops of _copy_linked_kv_batched_blocks that find the
 * repair rows inside blocks (patched_sglang_files/python/sglang/srt/
 * pic_runtime.py:4981-5003: offset + position - start for every imp_indices
 * entry inside a block).
 */
int ll_plan_link_runs(const ll_link_block *blocks, int64_t num_blocks, const int64_t *repair_positions,
                      int64_t num_repair_positions, int64_t compact, ll_link_segment *segments,
                      int64_t segment_capacity, int64_t *segment_blocks, int64_t *repair_offsets,
                      int64_t repair_offsets_capacity, ll_link_run_plan_info *info);

typedef struct ll_link_maps_args {
  int64_t struct_size;             /* sizeof(ll_link_maps_args) */
  int64_t num_segments;            /* >= 0 */
  const ll_link_segment *segments; /* host array [num_segments] */
  const void *destination_slots;   /* device [num_destination_slots], int32 or int64:
                                      the request's slots by request position (or
                                      several requests' slots, concatenated) */
  int64_t destination_slots_dtype;
  int64_t num_destination_slots;
  int64_t *maps[2];                /* device int64 [4, map_capacity[s]], or NULL for an unused set */
  int64_t map_capacity[2];
  uint8_t *repair_mask[2];         /* device uint8 [map_capacity[s]], or NULL: compacted set */
  int64_t *repair_destination_slots; /* device int64 [repair_capacity], or NULL */
  int64_t repair_capacity;
  const ll_link_segment *device_segments; /* device copy of segments[0, num_segments), or NULL (ABI 16):
                                      with it the builder is one launch that reads the runs
                                      there (each run re-checked on the device, a run that
                                      fails is left out); without it the runs travel in
                                      kernel arguments, 56 per launch.  `segments` is
                                      validated either way. */
} ll_link_maps_args;

/*
 * Visit order of a map set.  No counterpart in the reference, whose torch path
 * writes the rows in plan order: the kernel's result does not depend on the
 * order it visits the map entries in (every destination row is written once).
 * A single request's scattered row writes run faster in destination-slot
 * order; a batch whose requests share catalogue blocks reads repeated source
 * rows from cache in source-slot order.  This reorders the entries
 * [prefix, count) of a map set by the slots of map row key_row (0: source
 * slots, 1: destination slots) into out_maps (and the mask with them),
 * keeping entries [0, prefix) (the identity rows) first, in three launches: a
 * count of the entries per bucket of 2^shift consecutive slots (16,384
 * buckets over [0, num_slots), the key pool's rows; slots outside go to the
 * first or last bucket), one workgroup turning the counts into bucket
 * offsets, and a scatter.  Entries of one bucket are placed in no fixed order;
 * with num_slots <= 16,384 buckets hold one slot each.  out_maps is a
 * permutation of the entries for any input, duplicate or out-of-range slots
 * included.
 *
 * The workspace (LL_ORDER_WORKSPACE_BYTES, device, 16-byte aligned) must be
 * zero before its first use; every call leaves it so.  Calls that share a
 * workspace must not overlap (one stream).
 */
#define LL_ORDER_BUCKETS 16384
#define LL_ORDER_WORKSPACE_BYTES (8 * LL_ORDER_BUCKETS + 256)

typedef struct ll_order_maps_args {
  int64_t struct_size;             /* sizeof(ll_order_maps_args) */
  const int64_t *maps;             /* device int64 [4, capacity]: source slots, destination slots,
                                      local positions, global positions */
  const uint8_t *mask;             /* device uint8 [capacity], or NULL */
  int64_t capacity;                /* row stride of maps and out_maps; count <= capacity < 2^31 */
  int64_t count;                   /* entries */
  int64_t prefix;                  /* 0 <= prefix <= count: entries kept in place */
  int64_t num_slots;               /* rows of the pool the key slots index (>= 1) */
  int64_t *out_maps;               /* device int64 [4, capacity], not overlapping maps */
  uint8_t *out_mask;               /* device uint8 [capacity] (NULL iff mask is NULL) */
  void *workspace;
  int64_t workspace_bytes;
  int64_t key_row;                 /* 0: order by source slots, 1: by destination slots (ABI 17) */
} ll_order_maps_args;

int ll_order_link_maps(const ll_order_maps_args *args, ll_stream_t stream);
int64_t ll_order_maps_args_size(void);

/*
 * Sparse repair attention: the attention of the repair pass over the linked KV.
 *
 * A repair row is a contiguous span of query positions [query_start,
 * query_start + query_count) of one request.  Its keys and values are the
 * request's tokens at logical positions 0 .. query_start + query_count - 1,
 * found through the request's slot list: the slot of logical position j is
 * kv_slots[kv_offset + j].  Query i of the row (position p = query_start + i)
 * sees exactly the positions j <= p (the explicit causal rule of the
 * reference's physical-slot pattern); with G = num_q_heads / num_kv_heads,
 * query head h reads KV head h / G:
 *     out[query_index + i][h] = sum_j softmax_j(scale * q . K[slot_j][h / G]) V[slot_j][h / G]
 * The softmax is computed online in fp32 with exp2; scores and probabilities
 * come from bf16 (or fp16) MFMA products accumulated in fp32 (probabilities
 * are rounded to the KV dtype for the value product), and the output is
 * rounded once to the KV dtype.
 * Slots outside [0, num_slots) are invisible (never read).
 *
 * Two phases, like the reference's plan/run wrapper:
 *   ll_repair_attention_plan (host only) cuts the rows into 16-query tiles
 *   (consecutive rows of one request -- contiguous query_index, same
 *   kv_offset -- share a tile, so short repair spans fill it; rows must not
 *   overlap), writes every query's logical position into the positions
 *   table, cuts the (tile, query head) pairs of each run of consecutive tiles
 *   of one request (tile-major: G pairs per tile) into work items of 16
 *   consecutive pairs that share every staged K/V tile (a window may start
 *   or end inside a tile, so groups that do not divide 16 still fill every
 *   item), splits long KV ranges into chunks of
 *   split_tokens keys (a multiple of 64 below 2^31; 0 lets the plan choose
 *   from a model of the device's workgroup rounds, which may leave a range
 *   whole: no partials, no combine), and writes the item and
 *   combine tables; the caller copies them to the device once and reuses them
 *   for every layer.  Call it with NULL tables to size them.  num_q_heads is
 *   at most 65535.
 *   ll_repair_attention runs one layer; it takes tables made by this plan
 *   and num_slots < 2^31.  A workgroup reads its item's slots into LDS 7,680
 *   at a time, so items of any key length run in one workgroup.
 *
 * Replaces the FlashInfer block-sparse repair attention of
 * patched_sglang_files/python/sglang/srt/flashinfer_sparse_repair.py
 * (build_explicit_causal_masked_pattern :1241-1263, the plan/run of
 * _try_flashinfer_sparse_attention_single :2009-2272, and the row batching of
 * build_grouped_explicit_causal_masked_pattern :1266-1318), whose semantics the
 * reference restates as gqa_attention + logical_causal_mask in
 * tests/pic/reference/attention_reference.py.
 */
typedef struct ll_repair_row {
  int64_t query_index;             /* index of the row's first query in query / output */
  int64_t query_start;             /* logical position of the row's first query */
  int64_t query_count;             /* >= 1 */
  int64_t kv_offset;               /* index in kv_slots of logical position 0's slot */
} ll_repair_row;

typedef struct ll_repair_attention_plan_info {
  int64_t num_items;               /* int32 [num_items, 86] work items (ABI 13) */
  int64_t num_combine;             /* int32 [num_combine, 4] combine items */
  int64_t workspace_items;         /* partial results (see ll_repair_attention_args.workspace) */
  int64_t split_tokens;            /* KV tokens per work item (the plan's choice when 0 was asked) */
  int64_t num_queries;             /* entries of the positions table: max(query_index + query_count) */
} ll_repair_attention_plan_info;

typedef struct ll_repair_attention_args {
  int64_t struct_size;             /* sizeof(ll_repair_attention_args) */
  const void *query;               /* device kv_dtype [num_queries, num_q_heads, head_dim], dense */
  void *output;                    /* device kv_dtype [num_queries, num_q_heads, head_dim], dense */
  int64_t num_queries;
  const void *key_buffer;          /* device kv_dtype [num_slots, num_kv_heads, head_dim]: one layer */
  const void *value_buffer;        /* device kv_dtype [num_slots, num_kv_heads, head_dim] */
  int64_t num_slots;
  int64_t num_q_heads;
  int64_t num_kv_heads;            /* divides num_q_heads (any GQA ratio; MQA: 1); num_q_heads <= 65535 */
  int64_t head_dim;                /* 64, 128 or 256 */
  int64_t kv_dtype;                /* LL_DTYPE_BFLOAT16 or LL_DTYPE_FLOAT16: queries, K/V and output */
  double softmax_scale;
  const void *kv_slots;            /* device int32/int64 [kv_slots_len]: the requests' slot lists */
  int64_t kv_slots_dtype;
  int64_t kv_slots_len;
  const int32_t *items;            /* device copy of the plan's work items */
  int64_t num_items;
  const int32_t *combine;          /* device copy of the plan's combine items, or NULL */
  int64_t num_combine;
  const int32_t *query_positions;  /* device copy of the plan's positions table [num_queries] */
  float *workspace;                /* device, 16-byte aligned: workspace_items x num_q_heads blocks of
                                      8 * head_dim + 32 floats (16 queries' outputs in the KV dtype,
                                      then 16 fp32 (maximum, sum) pairs) (ABI 14) */
  int64_t workspace_items;
} ll_repair_attention_args;

int ll_repair_attention_plan(const ll_repair_row *rows, int64_t num_rows, int64_t num_q_heads,
                             int64_t num_kv_heads, int64_t split_tokens, int32_t *items,
                             int64_t items_capacity, int32_t *combine, int64_t combine_capacity,
                             int32_t *positions, int64_t positions_capacity,
                             ll_repair_attention_plan_info *info);
int ll_repair_attention(const ll_repair_attention_args *args, ll_stream_t stream);

/*
 * Allocation-free repair attention.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).
 *
 * Same arguments, semantics and output as ll_repair_attention, except that
 * args->workspace must be NULL: the split partial results go to a device array
 * of LL_REPAIR_SCRATCH_BYTES that the library holds on every GPU it runs on
 * (args->workspace_items still gives the plan's partial count).  The array
 * is part of the repair attention's code object: a process is charged
 * LL_REPAIR_SCRATCH_BYTES of device memory on a GPU from the first repair
 * attention launch there (through either entry) until it exits; with the
 * HIP runtime's deferred code-object loading (its default) a process that
 * only links is not charged.  A plan whose partials need more --
 * workspace_items * num_q_heads * (8 * head_dim + 32) * 4 bytes -- is
 * rejected with LL_ERR_INVALID_ARGUMENT before any launch.  Nothing needs
 * clearing: every partial the combine reads is written by the same call.
 * Calls that overlap on one GPU (two streams, or two threads) share that
 * GPU's array and race; serialise them.  The entry allocates nothing and
 * calls no allocating routine; the first call on a device looks up the
 * array's address there (hipGetSymbolAddress).
 */
#define LL_REPAIR_SCRATCH_BYTES (64LL << 20)
int ll_repair_attention_noalloc(const ll_repair_attention_args *args, ll_stream_t stream);
/* LL_REPAIR_SCRATCH_BYTES, as built into the library. */
int64_t ll_repair_scratch_bytes(void);

/* Which kernel and launch shape ll_kv_link would use (no GPU work). */
typedef struct ll_launch_info {
  int64_t kernel;                  /* LL_KERNEL_VECTOR or LL_KERNEL_GENERIC */
  int64_t launches;                /* kernel launches (one per group of <= 64 layers) */
  int64_t grid_x;                  /* of the first launch */
  int64_t grid_y;
  int64_t block_threads;
  int64_t layers_per_wave;
  int64_t layer_groups_per_block;
  int64_t delta_staging;           /* LL_DELTA_PER_WAVE, LL_DELTA_WORKGROUP or LL_DELTA_TABLE (vector kernels), else 0 */
} ll_launch_info;

int ll_kv_link(const ll_kv_link_args *args, ll_stream_t stream);
int ll_kv_link_describe(const ll_kv_link_args *args, ll_launch_info *info);
int ll_kv_scatter_rows(const ll_kv_scatter_args *args, ll_stream_t stream);
int ll_kv_build_link_maps(const ll_link_maps_args *args, ll_stream_t stream);

/* Reason string of a status code ("supported" for LL_OK). */
const char *ll_status_reason(int status);
/* Message of the last failing call on this thread ("" if none). */
const char *ll_last_error(void);
int ll_abi_version(void);
int64_t ll_kv_link_args_size(void);
int64_t ll_kv_scatter_args_size(void);
int64_t ll_link_maps_args_size(void);
int64_t ll_repair_attention_args_size(void);

#ifdef __cplusplus
}
#endif

#endif /* LEGOLINK_KV_H */
