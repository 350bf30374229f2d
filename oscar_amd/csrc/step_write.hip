// Fused write of a short step's new tokens (MTP decode steps) (gfx950).
//
// One launch does, for the step's N <= kMaxStepTokens new tokens, what the
// reference does around its paged read (oscar_ascend/backend.py:150-189,
// 261-269, 291-295, 439-481):
//   * q_rot = query @ R_k, k_rot = key @ R_k, v_rot = value @ R_v in fp32
//     (the read kernels' inputs, backend.py:291-295);
//   * the INT2 write of k_rot / v_rot: sort-clip to the idx-th smallest |x|,
//     quantize, pack, paged-slot write (backend.py:129-189);
//   * the FP32 window write (backend.py:439-481): per arena seat
//     ((slot / bs) % rows, slot % bs) the step's last token wins; the winner
//     sets owner = its page if the window keeps it (position >= seq - recent
//     or < sink_eff), else -1, and a kept winner stores its unclipped k_rot /
//     v_rot and their fp16 operand images (window_images.h).
//
// Work layout: a workgroup rotates up to four vectors that share a rotation
// (query heads, key heads or value heads of consecutive tokens).  Thread
// (wave w, lane l) accumulates rows 64w .. 64w + 63 of R against output
// columns 4l .. 4l + 3 (one 16-byte load of R per row feeds every vector),
// in fp32 FMAs in row order; the four waves' sums are added in wave order.
// Wave v then owns vector v, four features per lane (lane l: 4l .. 4l + 3,
// exactly the features of code byte l): it writes the fp32 result, and for
// keys and values finds the clip threshold by a bitwise radix select over the
// 256 |x| (ballots), quantizes with the exact thresholds of int2_quant.h,
// writes the slot and, when it is its seat's winner, the window.
#include "int2_quant.h"
#include "window_images.h"

namespace oscar {
namespace {

constexpr int kMaxStepTokens = 1024;
constexpr int kGroupVecs = 4;

struct StepArgs {
  const uint16_t* q;            // [N][q_stride] bf16
  const uint16_t* k;            // [N][kv_stride] bf16
  const uint16_t* v;
  int64_t q_stride, kv_stride;
  int32_t n_tokens, num_heads, num_kv_heads;
  const float* rot_k;           // [D][D]
  const float* rot_v;
  const int64_t* slots;         // [N], < 0 skipped
  uint8_t* k_cache;
  uint8_t* v_cache;
  int64_t k_page, k_tok, k_head, v_page, v_tok, v_head;   // byte strides
  int32_t block_size;
  int64_t num_slots;            // slots at or beyond are not written to the caches
  int32_t clip_k, clip_v;       // sorted-|x| index of the clip threshold, -1: none
  float* stage_k;               // [rows][bs][Hk][D] or null
  float* stage_v;
  int64_t* owner;               // [rows][bs]
  _Float16* kimg;               // [rows][bs / 32][Hk][kImgHalfs] or null
  _Float16* vimg;
  int32_t stage_rows;           // 0: no window
  float* q_rot;                 // [N][Hq][D]
  float* k_rot;                 // [N][Hk][D]
  float* v_rot;
  int32_t vecs_per_group;       // 1, 2 or 4
  int32_t kv_groups;            // workgroups per side (K, V)
  uint32_t keep[kMaxStepTokens / 32];   // bit t: the window keeps token t
};

__device__ __forceinline__ float bf16_to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// idx-th smallest |x| (ascending) of the 256 values one wave holds four per
// lane: bitwise radix select on the IEEE bits (for non-negative floats, bit
// order is value order).
__device__ float select_abs_rank_wave(const floatx4& y, int idx) {
  uint32_t u[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) u[j] = __float_as_uint(y[j]) & 0x7FFFFFFFu;
  uint32_t prefix = 0;
#pragma unroll 1
  for (int bit = 30; bit >= 0; --bit) {
    const uint32_t probe = prefix | (1u << bit);
    int below = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) below += __popcll(__ballot(u[j] < probe));
    if (idx >= below) prefix = probe;
  }
  return __uint_as_float(prefix);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, shfl_xor_f32(x, o));
  return x;
}
__device__ __forceinline__ float wave_min(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fminf(x, shfl_xor_f32(x, o));
  return x;
}

// Whether token t (slot s >= 0) is the last token of the step on its arena seat.
__device__ bool seat_winner(const StepArgs& a, int t, int64_t s, int lane) {
  const int64_t page = s / a.block_size;
  const int64_t row = page % a.stage_rows, col = s - page * a.block_size;
#pragma unroll 1
  for (int base = t + 1; base < a.n_tokens; base += 64) {
    const int u = base + lane;
    bool hit = false;
    if (u < a.n_tokens) {
      const int64_t s2 = a.slots[u];
      if (s2 >= 0) {
        const int64_t p2 = s2 / a.block_size;
        hit = p2 % a.stage_rows == row && s2 - p2 * a.block_size == col;
      }
    }
    if (__ballot(hit) != 0ull) return false;
  }
  return true;
}

// Quantize, pack and write one key (side 0) or value (side 1) vector, then
// the window; y: this lane's features 4l .. 4l + 3 (rotated, unclipped).
__device__ void write_vector(const StepArgs& a, const floatx4& y, int t, int h, int side, int lane) {
  const int clip = side == 0 ? a.clip_k : a.clip_v;
  float mx = wave_max(fmaxf(fmaxf(y[0], y[1]), fmaxf(y[2], y[3])));
  float mn = wave_min(fminf(fminf(y[0], y[1]), fminf(y[2], y[3])));
  const float thr = clip >= 0 ? select_abs_rank_wave(y, clip) : __builtin_inff();
  const QParams p = make_qparams(mn, mx, thr, clip >= 0);
  const uint32_t byte = int2_code(y[0], p) | (int2_code(y[1], p) << 2) | (int2_code(y[2], p) << 4) |
                        (int2_code(y[3], p) << 6);
  const uint32_t word = byte | ((uint32_t)__shfl((int)byte, lane + 1, 64) << 8) |
                        ((uint32_t)__shfl((int)byte, lane + 2, 64) << 16) |
                        ((uint32_t)__shfl((int)byte, lane + 3, 64) << 24);
  const int64_t s = a.slots[t];
  if (s < 0) return;
  const int64_t page = s / a.block_size;
  const int64_t prow = s - page * a.block_size;
  if (s < a.num_slots) {
    uint8_t* kslot = a.k_cache + page * a.k_page + prow * a.k_tok + (int64_t)h * a.k_head;
    uint8_t* codes = side == 0 ? kslot + kKCodeOff
                               : a.v_cache + page * a.v_page + prow * a.v_tok + (int64_t)h * a.v_head;
    if ((lane & 3) == 0) *reinterpret_cast<uint32_t*>(codes + lane) = word;
    if (lane == 0) *reinterpret_cast<uint32_t*>(kslot + 4 * side) = p.meta;
  }
  if (a.stage_rows <= 0 || !seat_winner(a, t, s, lane)) return;
  const bool keep = (a.keep[t >> 5] >> (t & 31)) & 1u;
  const int64_t arow = page % a.stage_rows;
  const int64_t seat = arow * a.block_size + prow;
  if (side == 0 && h == 0 && lane == 0) a.owner[seat] = keep ? page : -1;
  if (!keep) return;
  float* dst = (side == 0 ? a.stage_k : a.stage_v) + (seat * a.num_kv_heads + h) * kHeadDim;
  *reinterpret_cast<floatx4*>(dst + 4 * lane) = y;
  _Float16* img = side == 0 ? a.kimg : a.vimg;
  if (img != nullptr) {
    img += image_of(arow, (int)prow, a.block_size, h, a.num_kv_heads) * kImgHalfs;
    const int tt = (int)(prow & 31);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int f = 4 * lane + c;
      img[side == 0 ? kimg_offset(f, tt) : vimg_offset(f, tt)] = (_Float16)y[c];
    }
  }
}

__global__ __launch_bounds__(256) void step_write_kernel(StepArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kGroupVecs][kHeadDim];
  __shared__ __attribute__((aligned(16))) float part[4][kGroupVecs][kHeadDim];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int grp = blockIdx.x;
  int side = 0;                           // 0 keys, 1 values, 2 queries
  if (grp >= 2 * a.kv_groups) {
    side = 2;
    grp -= 2 * a.kv_groups;
  } else if (grp >= a.kv_groups) {
    side = 1;
    grp -= a.kv_groups;
  }
  const int heads = side == 2 ? a.num_heads : a.num_kv_heads;
  const int e0 = grp * a.vecs_per_group;
  const int nv = min(a.vecs_per_group, a.n_tokens * heads - e0);
  if (nv <= 0) return;
  const uint16_t* src = side == 0 ? a.k : (side == 1 ? a.v : a.q);
  const int64_t stride = side == 2 ? a.q_stride : a.kv_stride;
  const float* R = side == 1 ? a.rot_v : a.rot_k;

  for (int idx = tid; idx < nv * kHeadDim; idx += 256) {
    const int vv = idx >> 8, f = idx & 255;
    const int e = e0 + vv, t = e / heads, h = e - t * heads;
    xs[vv][f] = bf16_to_f32(src[(int64_t)t * stride + (int64_t)h * kHeadDim + f]);
  }
  __syncthreads();

  floatx4 acc[kGroupVecs];
#pragma unroll
  for (int vv = 0; vv < kGroupVecs; ++vv) acc[vv] = floatx4{0.f, 0.f, 0.f, 0.f};
  // Rows of R in chunks of eight, the next chunk's loads in flight while
  // the current one is used.
  const float* Rw = R + (int64_t)(64 * w) * kHeadDim + 4 * lane;
  floatx4 r[2][8];
  auto load_chunk = [&](int c, floatx4 (&dst)[8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = *reinterpret_cast<const floatx4*>(Rw + (int64_t)(8 * c + k) * kHeadDim);
  };
  load_chunk(0, r[0]);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if (c + 1 < 8) load_chunk(c + 1, r[(c + 1) & 1]);
#pragma unroll
    for (int vv = 0; vv < kGroupVecs; ++vv) {
      if (vv < nv) {
        const floatx4 x0 = *reinterpret_cast<const floatx4*>(&xs[vv][64 * w + 8 * c]);
        const floatx4 x1 = *reinterpret_cast<const floatx4*>(&xs[vv][64 * w + 8 * c + 4]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float xk = k < 4 ? x0[k] : x1[k - 4];
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) acc[vv][cc] = fmaf(xk, r[c & 1][k][cc], acc[vv][cc]);
        }
      }
    }
  }
#pragma unroll
  for (int vv = 0; vv < kGroupVecs; ++vv)
    if (vv < nv) *reinterpret_cast<floatx4*>(&part[w][vv][4 * lane]) = acc[vv];
  __syncthreads();
  if (w >= nv) return;
  floatx4 y = *reinterpret_cast<const floatx4*>(&part[0][w][4 * lane]);
#pragma unroll
  for (int ww = 1; ww < 4; ++ww) {
    const floatx4 z = *reinterpret_cast<const floatx4*>(&part[ww][w][4 * lane]);
#pragma unroll
    for (int c = 0; c < 4; ++c) y[c] += z[c];
  }
  const int e = e0 + w, t = e / heads, h = e - t * heads;
  float* out = side == 0 ? a.k_rot : (side == 1 ? a.v_rot : a.q_rot);
  *reinterpret_cast<floatx4*>(out + ((int64_t)t * heads + h) * kHeadDim + 4 * lane) = y;
  if (side < 2) write_vector(a, y, t, h, side, lane);
}

}  // namespace
}  // namespace oscar

using namespace oscar;

extern "C" int oscar_step_write(const void* query_bf16, int64_t query_token_stride, const void* key_bf16,
                                const void* value_bf16, int64_t kv_token_stride, int32_t num_tokens,
                                int32_t num_heads, int32_t num_kv_heads, int32_t head_size, const float* rot_k,
                                const float* rot_v, const int64_t* slot_mapping, const int32_t* query_start_loc,
                                const int32_t* seq_lens, int32_t num_requests, void* k_cache, void* v_cache,
                                int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                                int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                                int64_t v_stride_token, int64_t v_stride_head, int32_t clip_index_k,
                                int32_t clip_index_v, float* stage_k, float* stage_v, int64_t* stage_owner,
                                void* stage_k_image, void* stage_v_image, int32_t stage_rows, int32_t sink_eff,
                                int32_t recent, float* q_rot, float* k_rot, float* v_rot, hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_tokens > kMaxStepTokens || num_requests < 0 || num_heads <= 0 ||
      num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || block_size <= 0 || num_pages <= 0 ||
      stage_rows < 0 || sink_eff < 0 || recent < 0 || clip_index_k >= kHeadDim || clip_index_v >= kHeadDim)
    return kErrInvalidArgument;
  if (num_tokens == 0) return kOk;
  if (!query_bf16 || !key_bf16 || !value_bf16 || !rot_k || !rot_v || !slot_mapping || !k_cache || !v_cache ||
      !q_rot || !k_rot || !v_rot || (num_requests > 0 && (!query_start_loc || !seq_lens)))
    return kErrInvalidArgument;
  if (query_token_stride < (int64_t)num_heads * kHeadDim || kv_token_stride < (int64_t)num_kv_heads * kHeadDim)
    return kErrInvalidArgument;
  if (stage_rows > 0 && (!stage_k || !stage_v || !stage_owner)) return kErrInvalidArgument;
  if ((stage_k_image == nullptr) != (stage_v_image == nullptr)) return kErrInvalidArgument;
  if (stage_k_image != nullptr && block_size % 32 != 0) return kErrUnsupportedGeometry;
  if (k_stride_head < kKCodeOff + kCodeBytes || v_stride_head < kCodeBytes || (k_stride_page & 3) ||
      (k_stride_token & 3) || (k_stride_head & 3) || (v_stride_page & 3) || (v_stride_token & 3) ||
      (v_stride_head & 3) || (reinterpret_cast<uintptr_t>(k_cache) & 3) || (reinterpret_cast<uintptr_t>(v_cache) & 3))
    return kErrUnsupportedGeometry;
  if ((reinterpret_cast<uintptr_t>(q_rot) & 15) || (reinterpret_cast<uintptr_t>(k_rot) & 15) ||
      (reinterpret_cast<uintptr_t>(v_rot) & 15) || (reinterpret_cast<uintptr_t>(rot_k) & 15) ||
      (reinterpret_cast<uintptr_t>(rot_v) & 15) || (stage_k && (reinterpret_cast<uintptr_t>(stage_k) & 15)) ||
      (stage_v && (reinterpret_cast<uintptr_t>(stage_v) & 15)))
    return kErrInvalidArgument;
  StepArgs a{};
  a.q = static_cast<const uint16_t*>(query_bf16);
  a.k = static_cast<const uint16_t*>(key_bf16);
  a.v = static_cast<const uint16_t*>(value_bf16);
  a.q_stride = query_token_stride;
  a.kv_stride = kv_token_stride;
  a.n_tokens = num_tokens;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.rot_k = rot_k;
  a.rot_v = rot_v;
  a.slots = slot_mapping;
  a.k_cache = static_cast<uint8_t*>(k_cache);
  a.v_cache = static_cast<uint8_t*>(v_cache);
  a.k_page = k_stride_page;
  a.k_tok = k_stride_token;
  a.k_head = k_stride_head;
  a.v_page = v_stride_page;
  a.v_tok = v_stride_token;
  a.v_head = v_stride_head;
  a.block_size = block_size;
  a.num_slots = num_pages * (int64_t)block_size;
  a.clip_k = clip_index_k;
  a.clip_v = clip_index_v;
  a.stage_k = stage_k;
  a.stage_v = stage_v;
  a.owner = stage_owner;
  a.kimg = static_cast<_Float16*>(stage_k_image);
  a.vimg = static_cast<_Float16*>(stage_v_image);
  a.stage_rows = stage_rows;
  a.q_rot = q_rot;
  a.k_rot = k_rot;
  a.v_rot = v_rot;
  // Window keep rule per token (host lists, as the reference's): token t of
  // request i sits at seq[i] - qsl[i + 1] + t.
  for (int32_t i = 0; i < num_requests; ++i) {
    const int32_t lo = query_start_loc[i] < 0 ? 0 : query_start_loc[i];
    const int32_t hi = query_start_loc[i + 1] < num_tokens ? query_start_loc[i + 1] : num_tokens;
    for (int32_t t = lo; t < hi; ++t) {
      const int64_t pos = (int64_t)seq_lens[i] - query_start_loc[i + 1] + t;
      if (pos >= (int64_t)seq_lens[i] - recent || pos < sink_eff) a.keep[t >> 5] |= 1u << (t & 31);
    }
  }
  // Vectors per workgroup: one while the step has few vectors (every
  // workgroup streams R once; fewer vectors each finish sooner), up to four
  // for larger steps.
  const int64_t vectors = (int64_t)num_tokens * (num_heads + 2 * num_kv_heads);
  a.vecs_per_group = vectors <= 512 ? 1 : (vectors <= 2048 ? 2 : 4);
  a.kv_groups = (int32_t)(((int64_t)num_tokens * num_kv_heads + a.vecs_per_group - 1) / a.vecs_per_group);
  const int64_t q_groups = ((int64_t)num_tokens * num_heads + a.vecs_per_group - 1) / a.vecs_per_group;
  hipLaunchKernelGGL(step_write_kernel, dim3((unsigned)(2 * a.kv_groups + q_groups)), dim3(256), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
