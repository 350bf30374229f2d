/* Oracle (test infrastructure only): plain-C restatement of the OSCAR INT2
 * store for pre-rotated fp32 input.
 *
 * Follows oscar_ascend/backend.py:129-147 (sort-based clip),
 * oscar_ascend/format.py:51-88 (scale/zero rounded to fp16, then
 * q = clamp(floor((x - zero) / scale + 0.5), 0, 3), 4 codes per byte) and
 * oscar_ascend/kernels/store_kernel.py:54-102 (split-slot byte placement,
 * negative slots skipped, pad bytes untouched).
 *
 * Built with -O2 -ffp-contract=off and no fast-math so every fp32 operation
 * rounds once, exactly like the reference's separate torch ops.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* fp32 -> fp16 bits, round to nearest even (IEEE 754 binary16). */
uint16_t oscar_oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t a = x & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* >= 65520 -> inf */
  if (a >= 0x38800000u) {                                            /* normal result */
    uint32_t h = ((((a >> 23) - 112u) << 10) | ((a & 0x7FFFFFu) >> 13));
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  /* subnormal (or zero) result: units of 2^-24 */
  const int e = (int)(a >> 23);
  const int shift = 126 - e;                 /* >= 14 */
  if (shift > 31) return (uint16_t)sign;
  const uint64_t m = (uint64_t)((a & 0x7FFFFFu) | (e ? 0x800000u : 0u));
  uint64_t k = m >> shift;
  const uint64_t rem = m & ((1ull << shift) - 1ull);
  const uint64_t halfway = 1ull << (shift - 1);
  if (rem > halfway || (rem == halfway && (k & 1ull))) ++k;
  return (uint16_t)(sign | (uint32_t)k);
}

float oscar_oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  float v;
  if (e == 0) {
    v = ldexpf((float)m, -24);
  } else if (e == 31) {
    v = m ? NAN : INFINITY;
  } else {
    v = ldexpf((float)(m | 0x400u), (int)e - 25);
  }
  uint32_t bits;
  memcpy(&bits, &v, 4);
  bits |= sign;
  memcpy(&v, &bits, 4);
  return v;
}

static int cmp_float(const void* a, const void* b) {
  const float x = *(const float*)a, y = *(const float*)b;
  return (x > y) - (x < y);
}

/* Quantize one rotated vector of length d (clip_idx < 0: no clip).
 * codes: d/4 bytes; meta: (scale fp16 bits, zero fp16 bits). */
static void quantize_vector(const float* x, int d, int clip_idx, uint8_t* codes, uint16_t* meta,
                            float* scratch) {
  float* xc = scratch;          /* clipped copy */
  float* tmp = scratch + d;     /* sorted |x| */
  for (int i = 0; i < d; ++i) xc[i] = x[i];
  if (clip_idx >= 0) {
    for (int i = 0; i < d; ++i) tmp[i] = fabsf(x[i]);
    qsort(tmp, (size_t)d, sizeof(float), cmp_float);
    const float thr = tmp[clip_idx];
    for (int i = 0; i < d; ++i) {
      float v = xc[i];
      if (v < -thr) v = -thr;     /* torch.clamp(x, -thr, thr) = min(max(x, -thr), thr) */
      if (v > thr) v = thr;
      xc[i] = v;
    }
  }
  float lo = xc[0], hi = xc[0];
  for (int i = 1; i < d; ++i) {
    if (xc[i] < lo) lo = xc[i];
    if (xc[i] > hi) hi = xc[i];
  }
  volatile float scale = (hi - lo) / 3.0f;
  float s = scale > 0x1p-14f ? scale : 0x1p-14f;
  const uint16_t s16 = oscar_oracle_f32_to_f16(s);
  const uint16_t z16 = oscar_oracle_f32_to_f16(lo);
  const float sf = oscar_oracle_f16_to_f32(s16);
  const float zf = oscar_oracle_f16_to_f32(z16);
  meta[0] = s16;
  meta[1] = z16;
  for (int b = 0; b < d / 4; ++b) {
    unsigned byte = 0;
    for (int k = 0; k < 4; ++k) {
      volatile float t = xc[4 * b + k] - zf;
      volatile float u = t / sf;
      volatile float w = u + 0.5f;
      float q = floorf(w);
      if (!(q >= 0.0f)) q = 0.0f;
      if (q > 3.0f) q = 3.0f;
      byte |= ((unsigned)q & 3u) << (2 * k);
    }
    codes[b] = (uint8_t)byte;
  }
}

/* Store n rotated tokens.  x_k/x_v: [n][hk][d] fp32 contiguous.  Caches are
 * byte arrays addressed with byte strides (page, token, head). */
int oscar_oracle_store(const float* x_k, const float* x_v, int64_t n, int hk, int d,
                       const int64_t* slots, uint8_t* k_cache, uint8_t* v_cache, int64_t bs,
                       int64_t k_page, int64_t k_tok, int64_t k_head, int64_t v_page,
                       int64_t v_tok, int64_t v_head, int clip_k, int clip_v) {
  if (d % 4 != 0 || d / 4 > 64 || bs <= 0) return -1;
  float* scratch = (float*)malloc(sizeof(float) * 2 * (size_t)d);
  uint8_t codes[64];
  uint16_t meta[2];
  if (!scratch) return -2;
  for (int64_t t = 0; t < n; ++t) {
    const int64_t s = slots[t];
    if (s < 0) continue;
    const int64_t page = s / bs, row = s % bs;
    for (int h = 0; h < hk; ++h) {
      uint8_t* ks = k_cache + page * k_page + row * k_tok + h * k_head;
      uint8_t* vs = v_cache + page * v_page + row * v_tok + h * v_head;
      quantize_vector(x_k + (t * hk + h) * d, d, clip_k, codes, meta, scratch);
      ks[0] = (uint8_t)(meta[0] & 0xFF); ks[1] = (uint8_t)(meta[0] >> 8);
      ks[2] = (uint8_t)(meta[1] & 0xFF); ks[3] = (uint8_t)(meta[1] >> 8);
      memcpy(ks + 32, codes, (size_t)d / 4);
      quantize_vector(x_v + (t * hk + h) * d, d, clip_v, codes, meta, scratch);
      ks[4] = (uint8_t)(meta[0] & 0xFF); ks[5] = (uint8_t)(meta[0] >> 8);
      ks[6] = (uint8_t)(meta[1] & 0xFF); ks[7] = (uint8_t)(meta[1] >> 8);
      memcpy(vs, codes, (size_t)d / 4);
    }
  }
  free(scratch);
  return 0;
}
