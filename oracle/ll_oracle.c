/*
 * ll_oracle.c - CPU restatement of the LegoLink KV link arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  The HIP kernels are compared against this
 * restatement; only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg may load it.  It is never part of the product path.
 *
 * What it restates (reference = Nyannyan222/sglang-Legolink):
 *   llo_rerotate_rows  the per-token K arithmetic of the fused link kernel,
 *                      patched_sglang_files/python/sglang/srt/legolink_triton.py:
 *                        :332-347  token maps, prefix rule (remap = t >= prefix)
 *                        :349-362  neox / GPT-J pair indexing
 *                        :364-412  cos/sin reads: cos at column i, sin at i + r/2
 *                        :413-436  fp32 delta with separate RNE mul/add (no FMA);
 *                                  bf16 K + fp32 cache: fp32 rotation, one RNE
 *                                  to bf16 at the store
 *                        :437-468  bf16 K + bf16/fp16 cache: every product and
 *                                  sum rounded to bf16
 *                        :469-470  fp16 K: fp32 rotation, one RNE to fp16
 *                        :471-486  prefix tokens stored unrotated
 *                        :488-519  dims >= rotary_dim copied
 *                      and, with rounding = 1 ("eager"), the reference's torch
 *                      path instead, patched_sglang_files/python/sglang/srt/
 *                      pic_runtime.py:6039-6058 (_remap_key_positions: the
 *                      delta's products and sums in the cache's dtype) and
 *                      :1874-1885 (_apply_rotary_emb: delta cast to the key
 *                      dtype, every product and sum in the key dtype)
 *   llo_f32_to_bf16 / llo_f32_to_f16   round-to-nearest-even conversions.
 *
 * Compiled with gcc -O2 -ffp-contract=off: on x86-64 every float operation
 * is an SSE scalar op rounded to nearest even, and no FMA is formed.
 *
 * Data layout: rows[t][h][d], 16-bit elements, one layer.
 */
#include <stdint.h>
#include <string.h>

enum { LLO_F16 = 1, LLO_BF16 = 2, LLO_F32 = 3 };

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

float llo_bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

/* Round to nearest even; NaN -> 0x7fc0 (the quiet NaN torch also produces). */
uint16_t llo_f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float llo_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    if (man == 0) return bits_to_f32(sign);
    /* subnormal: man * 2^-24 is exact in fp32 */
    float v = (float)man * bits_to_f32(0x33800000u); /* 2^-24 */
    return sign ? -v : v;
  }
  if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* float -> fp16 bits, round to nearest even (IEEE 754 binary16). */
uint16_t llo_f32_to_f16(float f) {
  uint32_t u = f32_to_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t abs = u & 0x7fffffffu;
  if (abs > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((abs >> 13) & 0x3ffu));
  if (abs >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
  if (abs < 0x38800000u) {
    /* result is subnormal or zero: value / 2^-24 rounded to an integer */
    if (abs < 0x33000000u) return sign; /* < 2^-25: rounds to 0 (ties at 2^-25 go to even 0) */
    uint32_t exp = abs >> 23;
    uint32_t man = (abs & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - exp; /* 14..24 */
    uint32_t q = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
  }
  uint32_t q = abs >> 13;
  uint32_t rem = abs & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;
  return (uint16_t)(sign | (q - (112u << 10)));
}

void llo_f32_to_bf16_array(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = llo_f32_to_bf16(in[i]);
}

void llo_f32_to_f16_array(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = llo_f32_to_f16(in[i]);
}

void llo_f16_to_f32_array(const uint16_t *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = llo_f16_to_f32(in[i]);
}

static float round_bf16(float f) { return llo_bf16_to_f32(llo_f32_to_bf16(f)); }

/* An fp32 result stored in `dtype` and read back (fp32: unchanged). */
static float stored_as(float f, int dtype) {
  if (dtype == LLO_BF16) return round_bf16(f);
  if (dtype == LLO_F16) return llo_f16_to_f32(llo_f32_to_f16(f));
  return f;
}

static float key_to_f32(uint16_t bits, int key_dtype) {
  return key_dtype == LLO_BF16 ? llo_bf16_to_f32(bits) : llo_f16_to_f32(bits);
}

static uint16_t f32_to_key(float f, int key_dtype) {
  return key_dtype == LLO_BF16 ? llo_f32_to_bf16(f) : llo_f32_to_f16(f);
}

static float cache_at(const void *cache, int cache_dtype, int64_t offset) {
  if (cache_dtype == LLO_F32) return ((const float *)cache)[offset];
  uint16_t b = ((const uint16_t *)cache)[offset];
  return cache_dtype == LLO_BF16 ? llo_bf16_to_f32(b) : llo_f16_to_f32(b);
}

/*
 * out[t] = in[t] re-rotated from local[t] to global[t] (t >= prefix) or copied
 * (t < prefix); rounding 0 = the fused kernel's rounding points, 1 = the torch
 * path's.  Returns 0, or -1 if a remapped token's position is outside
 * [0, cache_rows).
 */
int llo_rerotate_rows(const uint16_t *in, uint16_t *out, int64_t num_tokens, int64_t num_heads,
                      int64_t head_dim, int key_dtype, const void *cache, int cache_dtype,
                      int64_t cache_rows, int64_t cs_stride_row, int64_t cs_stride_col,
                      const int64_t *local, const int64_t *global, int64_t rotary_dim, int neox,
                      int64_t prefix, int rounding) {
  const int64_t half = rotary_dim / 2;
  const int64_t row = num_heads * head_dim;
  for (int64_t t = 0; t < num_tokens; ++t) {
    const uint16_t *src = in + t * row;
    uint16_t *dst = out + t * row;
    memcpy(dst, src, (size_t)row * sizeof(uint16_t));
    if (t < prefix) continue;
    const int64_t lp = local[t], gp = global[t];
    if (lp < 0 || lp >= cache_rows || gp < 0 || gp >= cache_rows) return -1;
    for (int64_t i = 0; i < half; ++i) {
      const float lc = cache_at(cache, cache_dtype, lp * cs_stride_row + i * cs_stride_col);
      const float ls = cache_at(cache, cache_dtype, lp * cs_stride_row + (i + half) * cs_stride_col);
      const float gc = cache_at(cache, cache_dtype, gp * cs_stride_row + i * cs_stride_col);
      const float gs = cache_at(cache, cache_dtype, gp * cs_stride_row + (i + half) * cs_stride_col);
      const int64_t d1 = neox ? i : 2 * i;
      const int64_t d2 = neox ? i + half : 2 * i + 1;
      for (int64_t h = 0; h < num_heads; ++h) {
        const float x1 = key_to_f32(src[h * head_dim + d1], key_dtype);
        const float x2 = key_to_f32(src[h * head_dim + d2], key_dtype);
        uint16_t o1, o2;
        if (rounding == 1) {
          /* pic_runtime.py:6050-6051: torch tensors of the cache's dtype */
          const float cos_local = stored_as(gc * lc, cache_dtype);
          const float sin_local = stored_as(gs * ls, cache_dtype);
          const float dcc = stored_as(cos_local + sin_local, cache_dtype);
          const float sin_cos = stored_as(gs * lc, cache_dtype);
          const float cos_sin = stored_as(gc * ls, cache_dtype);
          const float dsc = stored_as(sin_cos - cos_sin, cache_dtype);
          /* pic_runtime.py:1874-1882: cos/sin cast to the key dtype, then
           * tensors of the key dtype */
          const float dck = stored_as(dcc, key_dtype);
          const float dsk = stored_as(dsc, key_dtype);
          const float first_cos = stored_as(x1 * dck, key_dtype);
          const float second_sin = stored_as(x2 * dsk, key_dtype);
          const float second_cos = stored_as(x2 * dck, key_dtype);
          const float first_sin = stored_as(x1 * dsk, key_dtype);
          o1 = f32_to_key(first_cos - second_sin, key_dtype);
          o2 = f32_to_key(second_cos + first_sin, key_dtype);
        } else if (key_dtype == LLO_BF16 && cache_dtype != LLO_F32) {
          /* legolink_triton.py:437-468 */
          const float p1 = round_bf16(gc * lc);
          const float p2 = round_bf16(gs * ls);
          const float dcb = round_bf16(p1 + p2);
          const float p3 = round_bf16(gs * lc);
          const float p4 = round_bf16(gc * ls);
          const float dsb = round_bf16(p3 - p4);
          const float first_cos = round_bf16(x1 * dcb);
          const float second_sin = round_bf16(x2 * dsb);
          const float second_cos = round_bf16(x2 * dcb);
          const float first_sin = round_bf16(x1 * dsb);
          o1 = llo_f32_to_bf16(first_cos - second_sin);
          o2 = llo_f32_to_bf16(second_cos + first_sin);
        } else {
          /* legolink_triton.py:413-436 (and :469-470 for fp16 K) */
          const float a = gc * lc;
          const float b = gs * ls;
          const float dc = a + b;
          const float c = gs * lc;
          const float d = gc * ls;
          const float ds = c - d;
          const float m1 = x1 * dc;
          const float m2 = x2 * ds;
          const float m3 = x2 * dc;
          const float m4 = x1 * ds;
          o1 = f32_to_key(m1 - m2, key_dtype);
          o2 = f32_to_key(m3 + m4, key_dtype);
        }
        dst[h * head_dim + d1] = o1;
        dst[h * head_dim + d2] = o2;
      }
    }
  }
  return 0;
}
