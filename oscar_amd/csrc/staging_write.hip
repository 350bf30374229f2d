// FP32 sink/recent window write into the owner-tagged staging arena (gfx950).
//
// Semantics (reference _staging_write): token t of the step (t < N, slot s >=
// 0) belongs to request i (qsl[i] <= t < qsl[i+1]) at absolute position
// pos = seq[i] - qsl[i+1] + t; it is kept when pos >= seq[i] - recent or
// pos < sink_eff.  Its seat is ((s / bs) % rows) * bs + s % bs.  Per seat the
// token with the largest index wins (the reference's stable sort + last);
// the winner sets owner[seat] = s / bs if kept, else -1, and a kept winner
// stores its unclipped rotated K/V (x @ R, fp32) in the seat.
//
// Kernel 1 records the winning token per seat with a 64-bit atomicMax of
// epoch-tagged keys into a persistent buffer that is never reset (see
// seat_winner_pass).  Kernel 2: one block per token; the winner updates
// owner / values.
//
// A kept winner also refreshes the fp16 operand images of window_images.h.
#include "window_images.h"
#include "../../include/oscar_amd.h"

namespace oscar {
namespace {

struct StageArgs {
  const uint16_t* key;      // [N][token_stride] bf16
  const uint16_t* value;
  int64_t token_stride;
  const int64_t* slots;     // [N]
  int32_t n_tokens;
  const int32_t* query_start;   // [B + 1]
  const int32_t* seq_lens;      // [B]
  int32_t num_requests;
  int32_t num_kv_heads;
  int32_t block_size;
  int32_t rows;
  int32_t sink_eff, recent;
  const float* rot_k;       // [D][D]
  const float* rot_v;
  float* stage_k;           // [rows][bs][Hk][D]
  float* stage_v;
  int64_t* owner;           // [rows][bs]
  int64_t* winner;          // [rows * bs] keys, then epoch and arrival counter
  _Float16* kimg;           // [rows][bs / 32][Hk][kKImgHalfs] or null
  _Float16* vimg;           // [rows][bs / 32][Hk][kVImgHalfs] or null
};

__global__ __launch_bounds__(256) void stage_winner_kernel(StageArgs a) {
  __shared__ int64_t epoch;
  seat_winner_pass(a.slots, a.n_tokens, a.winner, (int64_t)a.rows * a.block_size, a.block_size, a.rows, &epoch);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float((uint32_t)x << 16);
}

__global__ __launch_bounds__(256) void stage_update_kernel(StageArgs a) {
  __shared__ float xk[kHeadDim];
  __shared__ float xv[kHeadDim];
  const int t = blockIdx.x;
  const int64_t s = a.slots[t];
  if (s < 0) return;
  int64_t seat, page;
  if (!won_seat(a.winner, (int64_t)a.rows * a.block_size, s, t, a.block_size, a.rows, seat, page))
    return;                              // block-uniform
  // Request of token t: last i with query_start[i] <= t.
  int lo = 0, hi = a.num_requests - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.query_start[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int64_t seq = a.seq_lens[lo];
  const int64_t pos = seq - a.query_start[lo + 1] + t;
  const bool keep = pos >= seq - a.recent || pos < a.sink_eff;
  __syncthreads();
  if (threadIdx.x == 0) a.owner[seat] = keep ? page : -1;
  if (!keep) return;
  const int f = threadIdx.x;
  for (int h = 0; h < a.num_kv_heads; ++h) {
    __syncthreads();
    const int64_t src = (int64_t)t * a.token_stride + (int64_t)h * kHeadDim + f;
    xk[f] = bf16_to_f32(a.key[src]);
    xv[f] = bf16_to_f32(a.value[src]);
    __syncthreads();
    float yk = 0.f, yv = 0.f;
#pragma unroll 8
    for (int e = 0; e < kHeadDim; ++e) {
      yk = fmaf(xk[e], a.rot_k[e * kHeadDim + f], yk);
      yv = fmaf(xv[e], a.rot_v[e * kHeadDim + f], yv);
    }
    const int64_t dst = (seat * a.num_kv_heads + h) * kHeadDim + f;
    a.stage_k[dst] = yk;
    a.stage_v[dst] = yv;
    if (a.kimg != nullptr) {
      const int prow = (int)(seat % a.block_size);
      const int64_t img = ((seat / a.block_size) * (a.block_size / 32) + prow / 32) * a.num_kv_heads + h;
      _Float16* kd = a.kimg + img * kKImgHalfs + kimg_offset(f, prow & 31);
      fp16_parts(yk, kd[0], kd[kImgHalfs]);
      _Float16* vd = a.vimg + img * kVImgHalfs + vimg_offset(f, prow & 31);
      fp16_parts(yv, vd[0], vd[kVPartHalfs]);
    }
  }
}

}  // namespace
}  // namespace oscar

using namespace oscar;

extern "C" int oscar_staging_write(const void* key_bf16, const void* value_bf16, int64_t token_stride,
                                   const int64_t* slot_mapping, int32_t num_tokens,
                                   const int32_t* query_start_loc, const int32_t* seq_lens,
                                   int32_t num_requests, int32_t num_kv_heads, int32_t head_size,
                                   int32_t block_size, int32_t stage_rows, int32_t sink_eff,
                                   int32_t recent, const float* rot_k, const float* rot_v,
                                   float* stage_k, float* stage_v, int64_t* stage_owner,
                                   int64_t* seat_winner, void* stage_k_image, void* stage_v_image,
                                   hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_requests < 0 || num_kv_heads <= 0 || block_size <= 0 || stage_rows <= 0 ||
      sink_eff < 0 || recent < 0 || token_stride < (int64_t)num_kv_heads * kHeadDim)
    return kErrInvalidArgument;
  if (num_tokens == 0 || num_requests == 0) return kOk;
  if (!key_bf16 || !value_bf16 || !slot_mapping || !query_start_loc || !seq_lens || !rot_k || !rot_v ||
      !stage_k || !stage_v || !stage_owner || !seat_winner)
    return kErrInvalidArgument;
  if ((stage_k_image == nullptr) != (stage_v_image == nullptr)) return kErrInvalidArgument;
  if (stage_k_image != nullptr && block_size % 32 != 0) return kErrUnsupportedGeometry;
  StageArgs a{static_cast<const uint16_t*>(key_bf16), static_cast<const uint16_t*>(value_bf16),
              token_stride, slot_mapping, num_tokens, query_start_loc, seq_lens, num_requests,
              num_kv_heads, block_size, stage_rows, sink_eff, recent, rot_k, rot_v, stage_k, stage_v,
              stage_owner, seat_winner, static_cast<_Float16*>(stage_k_image),
              static_cast<_Float16*>(stage_v_image)};
  hipLaunchKernelGGL(stage_winner_kernel, dim3((num_tokens + 255) / 256), dim3(256), 0, stream, a);
  if (hipGetLastError() != hipSuccess) return kErrLaunch;
  hipLaunchKernelGGL(stage_update_kernel, dim3(num_tokens), dim3(kHeadDim), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
