// Shared definitions for the OSCAR INT2 KV-cache kernels (gfx950 / CDNA4).
//
// Slot layout (per token, per kv-head), byte offsets inside the engine's
// paged caches:
//   K slot  [0:2] K scale fp16 LE  [2:4] K zero  [4:6] V scale  [6:8] V zero
//           [8:32] pad (never written)           [32:96] K codes
//   V slot  [0:64] V codes
// Code k of byte b holds value 4b+k in bits [2k, 2k+2).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace oscar {

constexpr int kHeadDim = 256;          // the kernels are written for D = 256
constexpr int kCodeBytes = kHeadDim / 4;
constexpr int kKCodeOff = 32;
constexpr int kMetaBytes = 8;
constexpr float kScaleFloor = 6.103515625e-05f;   // 2^-14

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Status codes returned by every extern "C" entry point.
enum Status : int {
  kOk = 0,
  kErrInvalidArgument = -1,
  kErrUnsupportedHeadDim = -2,
  kErrWorkspaceTooSmall = -3,
  kErrLaunch = -4,
  kErrUnsupportedGeometry = -5,
};

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) once per (kernel, device):
// `done` holds one bit per device ordinal (ordinals >= 64 set it on every call).
inline int set_dynamic_lds(const void* kernel, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return kErrLaunch;
  const uint64_t bit = dev < 64 ? (1ull << dev) : 0ull;
  if (bit != 0ull && (done.load(std::memory_order_acquire) & bit) != 0ull) return kOk;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) return kErrLaunch;
  done.fetch_or(bit, std::memory_order_acq_rel);
  return kOk;
}

// Division of n in [0, 2^31) by a divisor d in [1, 2^31) fixed at launch, as
// a multiply-high, an add and a shift (Granlund and Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, theorem 4.2): with
// 2^(l-1) < d <= 2^l and M = floor(2^(32+l) / d) + 1 = 2^32 + m (m < 2^32),
// floor(n / d) = floor(M n / 2^(32+l)) = (n + mulhi(m, n)) >> l, and the sum
// stays below 2^32 because mulhi(m, n) < n < 2^31.
struct FastDiv {
  uint32_t d, m;
  int32_t l;
};

inline FastDiv make_fast_div(uint32_t d) {      // host side, d >= 1
  int32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint64_t m = ((((uint64_t)1 << l) - d) << 32) / d + 1;
  return FastDiv{d, (uint32_t)m, l};
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
  return (__umulhi(f.m, n) + n) >> f.l;
}

__device__ __forceinline__ uint32_t fast_mod(uint32_t n, const FastDiv& f) {
  return n - fast_div(n, f) * f.d;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  _Float16 h = (_Float16)x;            // v_cvt_f16_f32, round-to-nearest-even
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

__device__ __forceinline__ float shfl_xor_f32(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ uint32_t shfl_xor_u32(uint32_t v, int mask) {
  return (uint32_t)__shfl_xor((int)v, mask, 64);
}

}  // namespace oscar
