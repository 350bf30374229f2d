// fp16 operand images of the FP32 window arena (written by the window-write
// kernels, read by the paged decode), per (arena row, 32-token tile, kv head):
//   K image [2 parts][16 k-steps m][64 lanes][8 slots]: lane t + 32g, slot
//     2i + b of step m = 2j + a holds feature 128g + 16j + 4a + i + 8b of
//     token t;
//   V image [4 q][2 b][2 s][64 lanes][2 parts][8 slots]: lane m + 32gs holds
//     feature 64q + 4(m >> 1) + 2b + (m & 1); slot u holds token 16s + 8gs +
//     {0, 2, 1, 3, 4, 6, 5, 7}[u] (a lane's two parts are adjacent, so that
//     loading the high parts brings the low parts' cache lines too).
// In both, part 0 is RNE fp16(x) and part 1 RNE fp16(x - part 0), so that the
// two parts carry the FP32 value to about 2^-22 of its magnitude.
// Both are exactly MFMA operand registers of the decode's wavefronts (K: the
// tile's owner, V: wavefront q's quarter of the features), which read them
// with one 16-byte load per lane and block.
#pragma once

#include "oscar_common.h"

namespace oscar {

constexpr int kImgHalfs = 16 * 64 * 8;     // one part of an operand image
constexpr int kKImgHalfs = 2 * kImgHalfs;  // K image: high part, then low part
constexpr int kVImgHalfs = 2 * kImgHalfs;  // V image: high and low part of each lane's 8 slots

// The two fp16 parts of a window value.
__device__ __forceinline__ void fp16_parts(float x, _Float16& hi, _Float16& lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// Offsets of feature f of token t (0..31 within its tile) in the two images.
__device__ __forceinline__ int kimg_offset(int f, int t) {
  const int g = f >> 7, rr = f & 127, jj = rr >> 4, r16 = rr & 15, b = r16 >> 3, r8 = r16 & 7;
  const int m = 2 * jj + (r8 >> 2), u = 2 * (r8 & 3) + b;
  return (m * 64 + t + 32 * g) * 8 + u;
}

// (V: the high part; the low part follows 8 halves later.)
__device__ __forceinline__ int vimg_offset(int f, int t) {
  const int q = f >> 6, b = (f >> 1) & 1, m = 2 * ((f >> 2) & 15) + (f & 1);
  const int s = t >> 4, gs = (t >> 3) & 1, r = t & 7;
  const int slot = r == 1 ? 2 : (r == 2 ? 1 : (r == 5 ? 6 : (r == 6 ? 5 : r)));   // self-inverse
  return ((((q * 2 + b) * 2 + s) * 64) + m + 32 * gs) * 16 + slot;
}
constexpr int kVPartHalfs = 8;             // low part of a V slot: 8 halves after the high part

// Index, in 8-half vectors, of part `part` of lane-block `lb` (block * 64 +
// lane) of a V image.
__device__ __forceinline__ int vimg_part(int lb, int part) { return 2 * lb + part; }

// Image of the 32-token tile holding arena seat row `prow` of arena row
// `arow`, kv head h.
__device__ __forceinline__ int64_t image_of(int64_t arow, int prow, int block_size, int h, int num_kv_heads) {
  return (arow * (block_size / 32) + prow / 32) * num_kv_heads + h;
}

// Seat winners of a bulk window write.  The buffer is int64
// [seats + 2]: one key per arena seat, then the epoch of the last call and an
// arrival counter (all zero when allocated; never reset).  A call's pass over
// its tokens stores max(key, (epoch + 1) << 32 | t) per seat (t: token index
// within the step), and its last workgroup to arrive advances the epoch, so
// that afterwards a seat's winner is the token t whose key equals
// epoch << 32 | t.  Keys of earlier calls carry smaller epochs and lose.
__device__ __forceinline__ int64_t winner_key(int64_t epoch, int64_t t) { return (epoch << 32) | t; }

// One thread per token of the pass (blockDim.x threads per workgroup).
__device__ __forceinline__ void seat_winner_pass(const int64_t* __restrict__ slots, int32_t n_tokens, int64_t* winner,
                                                 int64_t seats, int32_t block_size, int32_t rows, int64_t* epoch_lds) {
  if (threadIdx.x == 0)
    *epoch_lds = __hip_atomic_load(winner + seats, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
  __syncthreads();
  const int64_t e = *epoch_lds;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n_tokens) {
    const int64_t s = slots[t];
    if (s >= 0) {
      const int64_t page = s / block_size;
      const int64_t seat = (page % rows) * block_size + (s - page * block_size);
      __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(winner + seat),
                             (unsigned long long)winner_key(e, t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    // every thread of this workgroup has read the epoch; the last workgroup
    // to arrive publishes the call's epoch and clears the counter
    const unsigned long long done = __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(winner + seats + 1),
                                                           1ull, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1) {
      __hip_atomic_store(winner + seats, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(winner + seats + 1, (int64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// After the pass (a later launch): whether token t with slot s (>= 0) won
// its seat; seat returned.
__device__ __forceinline__ bool won_seat(const int64_t* winner, int64_t seats, int64_t s, int64_t t, int32_t block_size,
                                         int32_t rows, int64_t& seat, int64_t& page) {
  page = s / block_size;
  seat = (page % rows) * block_size + (s - page * block_size);
  return winner[seat] == winner_key(winner[seats], t);
}

}  // namespace oscar
