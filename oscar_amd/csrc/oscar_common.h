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
