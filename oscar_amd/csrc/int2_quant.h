// Exact INT2 quantizer parameters shared by the write kernels (gfx950).
//
// Quantization is bit-exact with the reference's fp32 formula
// (oscar_ascend/format.py:51-88):
//   scale = max((vmax - vmin) / 3, 2^-14) rounded to fp16, zero = fp16(vmin),
//   q = clamp(floor((x - zero) / scale + 0.5), 0, 3)
// without a per-value divide: with t = fl(x - zero), q >= n holds exactly when
// t >= T_n, where T_n is the smallest float at or above scale * c_n (c_1 just
// below 0.5, c_2 just below 1.5, c_3 just below 2.5; the offsets encode the
// round-to-nearest-even ties of the divide and of the +0.5), computed once
// per vector in fp64 (exact: scale has 11 significant bits).  Clipping to
// [-thr, thr] folds into the thresholds, because x -> fl(x - zero) is
// monotone: a threshold outside [fl(-thr - zero), fl(thr - zero)] moves to
// -inf or +inf.
#pragma once

#include "oscar_common.h"

namespace oscar {

struct QParams {
  float zero;
  float t1, t2, t3;       // thresholds on t = fl(x - zero), clip folded in
  uint32_t meta;          // scale fp16 bits | zero fp16 bits << 16
};

// Smallest float >= d for a positive finite-or-infinite double d.
__device__ __forceinline__ float round_up_f32(double d) {
  float f = (float)d;
  if ((double)f < d) f = __uint_as_float(__float_as_uint(f) + 1u);
  return f;
}

// mn / mx: minimum and maximum of the unclipped vector; thr: clip threshold
// (ignored without clip).
__device__ inline QParams make_qparams(float mn, float mx, float thr, bool clip) {
  if (clip) {
    mx = fminf(fmaxf(mx, -thr), thr);
    mn = fminf(fmaxf(mn, -thr), thr);
  }
  float scale = (mx - mn) / 3.0f;                       // IEEE divide
  scale = (scale > kScaleFloor) ? scale : kScaleFloor;
  const uint16_t s16 = f32_to_f16_bits(scale);
  const uint16_t z16 = f32_to_f16_bits(mn);
  const float s = f16_bits_to_f32(s16);
  const float z = f16_bits_to_f32(z16);
  // q >= 1 <=> fl(t/s) >= 0.5 - 2^-25 <=> t/s >  0.5 - 3*2^-26
  // q >= 2 <=> fl(t/s) >= 1.5        <=> t/s >= 1.5 - 2^-24
  // q >= 3 <=> fl(t/s) >= 2.5        <=> t/s >= 2.5 - 2^-23
  // s * c1 is never a float (odd 25-bit mantissa times s), so ">" and ">="
  // both become t >= round_up(s * c1).
  const double sd = (double)s;
  float t1 = round_up_f32(sd * (0.5 - 3.0 * 0x1p-26));
  float t2 = round_up_f32(sd * (1.5 - 0x1p-24));
  float t3 = round_up_f32(sd * (2.5 - 0x1p-23));
  if (clip) {
    const float tlo = -thr - z;
    const float thi = thr - z;
    const float inf = __builtin_inff();
    t1 = (t1 <= tlo) ? -inf : ((t1 > thi) ? inf : t1);
    t2 = (t2 <= tlo) ? -inf : ((t2 > thi) ? inf : t2);
    t3 = (t3 <= tlo) ? -inf : ((t3 > thi) ? inf : t3);
  }
  QParams p;
  p.zero = z;
  p.t1 = t1;
  p.t2 = t2;
  p.t3 = t3;
  p.meta = (uint32_t)s16 | ((uint32_t)z16 << 16);
  return p;
}

// INT2 code of an unclipped value.
__device__ __forceinline__ uint32_t int2_code(float x, const QParams& p) {
  const float t = x - p.zero;
  const bool a = t >= p.t2;
  const bool b = t >= (a ? p.t3 : p.t1);
  return (a ? 2u : 0u) | (b ? 1u : 0u);
}

}  // namespace oscar
