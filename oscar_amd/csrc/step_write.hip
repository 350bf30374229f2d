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
// oscar_quant_write runs the same kernel without a query or window (num_heads
// = 0, no arena) for writes of at most 2048 key + value vectors.
//
// Work layout: a 1024-thread workgroup rotates up to four vectors that share a
// rotation (query heads, key heads or value heads of consecutive tokens).
// Thread (wave w, lane l) holds rows 16w .. 16w + 15 of R at output columns
// 4l .. 4l + 3 (sixteen 16-byte loads, all issued before any wait, feed every
// vector) and sums them in fp32 FMAs in row order; the sixteen waves' sums
// are added in wave order.
// Wave v then owns vector v, four features per lane (lane l: 4l .. 4l + 3,
// exactly the features of code byte l): it writes the fp32 result, and for
// keys and values finds the clip threshold by a bitwise radix select over the
// 256 |x| (ballots), quantizes with the exact thresholds of int2_quant.h,
// writes the slot and, when it is its seat's winner, the window.
#include "int2_quant.h"
#include "window_images.h"
#include "../../include/oscar_amd.h"

namespace oscar {
namespace {

constexpr int kMaxStepTokens = 1024;
constexpr int kGroupVecs = 4;
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kRowsPerWave = kHeadDim / kWaves;   // 16 rows of R per wavefront

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
  FastDiv bs_div;               // block_size
  FastDiv rows_div;             // stage_rows (1 without an arena)
  int64_t num_slots;            // slots at or beyond are not written to the caches
  int32_t clip_k, clip_v;       // sorted-|x| index of the clip threshold, -1: none
  float* stage_k;               // [rows][bs][Hk][D] or null
  float* stage_v;
  int64_t* owner;               // [rows][bs]
  _Float16* kimg;               // [rows][bs / 32][Hk][kKImgHalfs] or null
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

// The kernel arguments the key / value write path reads.
struct WriteCtx {
  const int64_t* slots;
  uint8_t* k_cache;
  uint8_t* v_cache;
  int64_t k_page, k_tok, k_head, v_page, v_tok, v_head;
  int64_t num_slots;
  float* stage;             // stage_k or stage_v (this workgroup's side)
  int64_t* owner;
  _Float16* img;            // kimg or vimg
  FastDiv bs_div, rows_div;
  int32_t block_size, stage_rows, num_kv_heads, n_tokens, clip;
};

// Every scalar kernel argument, loaded in one round before any of them is
// used: a kernel-argument read the compiler leaves next to its use (or behind
// a branch on another argument) costs a memory round trip of its own.
struct Scalars {
  WriteCtx w;
  float* stage_k;
  float* stage_v;
  _Float16* kimg;
  _Float16* vimg;
  int32_t clip_k, clip_v;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, kv_stride;
  const float* rot_k;
  const float* rot_v;
  float* q_rot;
  float* k_rot;
  float* v_rot;
  int32_t num_heads, kv_groups, vecs_per_group;
};

__device__ __forceinline__ Scalars load_scalars(const StepArgs& a) {
  Scalars c;
  c.w.slots = a.slots;
  c.w.k_cache = a.k_cache;
  c.w.v_cache = a.v_cache;
  c.w.k_page = a.k_page;
  c.w.k_tok = a.k_tok;
  c.w.k_head = a.k_head;
  c.w.v_page = a.v_page;
  c.w.v_tok = a.v_tok;
  c.w.v_head = a.v_head;
  c.w.num_slots = a.num_slots;
  c.w.owner = a.owner;
  c.w.bs_div = a.bs_div;
  c.w.rows_div = a.rows_div;
  c.w.block_size = a.block_size;
  c.w.stage_rows = a.stage_rows;
  c.w.num_kv_heads = a.num_kv_heads;
  c.w.n_tokens = a.n_tokens;
  c.stage_k = a.stage_k;
  c.stage_v = a.stage_v;
  c.kimg = a.kimg;
  c.vimg = a.vimg;
  c.clip_k = a.clip_k;
  c.clip_v = a.clip_v;
  c.q = a.q;
  c.k = a.k;
  c.v = a.v;
  c.q_stride = a.q_stride;
  c.kv_stride = a.kv_stride;
  c.rot_k = a.rot_k;
  c.rot_v = a.rot_v;
  c.q_rot = a.q_rot;
  c.k_rot = a.k_rot;
  c.v_rot = a.v_rot;
  c.num_heads = a.num_heads;
  c.kv_groups = a.kv_groups;
  c.vecs_per_group = a.vecs_per_group;
  asm volatile("" : "+s"(c.w.slots), "+s"(c.w.k_cache), "+s"(c.w.v_cache), "+s"(c.w.k_page), "+s"(c.w.k_tok),
               "+s"(c.w.k_head), "+s"(c.w.v_page), "+s"(c.w.v_tok), "+s"(c.w.v_head), "+s"(c.w.num_slots),
               "+s"(c.w.owner), "+s"(c.w.bs_div.d), "+s"(c.w.bs_div.m), "+s"(c.w.bs_div.l), "+s"(c.w.rows_div.d),
               "+s"(c.w.rows_div.m), "+s"(c.w.rows_div.l), "+s"(c.w.block_size), "+s"(c.w.stage_rows),
               "+s"(c.w.num_kv_heads), "+s"(c.w.n_tokens));
  asm volatile("" : "+s"(c.stage_k), "+s"(c.stage_v), "+s"(c.kimg), "+s"(c.vimg), "+s"(c.clip_k), "+s"(c.clip_v),
               "+s"(c.q), "+s"(c.k), "+s"(c.v), "+s"(c.q_stride), "+s"(c.kv_stride), "+s"(c.rot_k), "+s"(c.rot_v),
               "+s"(c.q_rot), "+s"(c.k_rot), "+s"(c.v_rot), "+s"(c.num_heads), "+s"(c.kv_groups),
               "+s"(c.vecs_per_group));
  return c;
}

// idx-th smallest |x| (ascending) of the 256 values one wave holds four per
// lane: radix select on the IEEE bits (for non-negative floats, bit order is
// value order), two bits per round: of the probes prefix | d << b (d = 1, 2,
// 3) the largest with at most idx values below it extends the prefix.
__device__ float select_abs_rank_wave(const floatx4& y, int idx) {
  uint32_t u[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) u[j] = __float_as_uint(y[j]) & 0x7FFFFFFFu;
  auto below = [&](uint32_t probe) {
    int n = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) n += __popcll(__ballot(u[j] < probe));
    return n;
  };
  uint32_t prefix = idx >= below(1u << 30) ? (1u << 30) : 0u;       // bit 30 alone
#pragma unroll 1
  for (int b = 28; b >= 0; b -= 2) {
    const uint32_t p1 = prefix | (1u << b), p2 = prefix | (2u << b), p3 = prefix | (3u << b);
    const int n1 = below(p1), n2 = below(p2), n3 = below(p3);
    prefix = idx >= n3 ? p3 : (idx >= n2 ? p2 : (idx >= n1 ? p1 : prefix));
  }
  return __uint_as_float(prefix);
}

// Wave-wide max / min through DPP row operations (result in every lane).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), kCtrl, kRowMask, 0xF, false));
}

template <bool kMax>
__device__ __forceinline__ float wave_reduce(float x) {
  auto op = [](float a, float b) { return kMax ? fmaxf(a, b) : fminf(a, b); };
  x = op(x, dpp_f32<0xB1, 0xF>(x));     // quad_perm [1, 0, 3, 2]
  x = op(x, dpp_f32<0x4E, 0xF>(x));     // quad_perm [2, 3, 0, 1]
  x = op(x, dpp_f32<0x141, 0xF>(x));    // row_half_mirror
  x = op(x, dpp_f32<0x140, 0xF>(x));    // row_mirror
  x = op(x, dpp_f32<0x142, 0xA>(x));    // row_bcast:15 into rows 1 and 3
  x = op(x, dpp_f32<0x143, 0xC>(x));    // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// (page, row) of a slot: the fixed-divisor path for slots below 2^31.
__device__ __forceinline__ void slot_page_row(const WriteCtx& a, int64_t s, int64_t& page, int64_t& row) {
  if (s < (int64_t(1) << 31)) {
    const uint32_t p = fast_div((uint32_t)s, a.bs_div);
    page = p;
    row = (int64_t)((uint32_t)s - p * a.bs_div.d);
  } else {
    page = s / a.block_size;
    row = s - page * a.block_size;
  }
}

__device__ __forceinline__ int64_t arena_row(const WriteCtx& a, int64_t page) {
  return page < (int64_t(1) << 31) ? (int64_t)fast_mod((uint32_t)page, a.rows_div) : page % a.stage_rows;
}

// Whether token t (slot s >= 0) is the last token of the step on its arena
// seat; later[l] = slot of token t + 1 + l (prefetched, -1 past the step).
__device__ bool seat_winner(const WriteCtx& a, int t, int64_t s, int64_t later, int lane) {
  int64_t page, col;
  slot_page_row(a, s, page, col);
  const int64_t row = arena_row(a, page);
  auto hit = [&](int64_t s2) {
    if (s2 < 0) return false;
    int64_t p2, c2;
    slot_page_row(a, s2, p2, c2);
    return c2 == col && arena_row(a, p2) == row;
  };
  if (__ballot(hit(later)) != 0ull) return false;
#pragma unroll 1
  for (int base = t + 65; base < a.n_tokens; base += 64) {
    const int u = base + lane;
    if (__ballot(hit(u < a.n_tokens ? a.slots[u] : -1)) != 0ull) return false;
  }
  return true;
}

// Quantize, pack and write one key (side 0) or value (side 1) vector, then
// the window; y: this lane's features 4l .. 4l + 3 (rotated, unclipped);
// s: the token's slot; later: prefetched slots of the next 64 tokens.
__device__ void write_vector(const WriteCtx& a, const floatx4& y, int t, int h, int side, int lane, int64_t s,
                             int64_t later, uint32_t keep_word) {
  const int clip = a.clip;
  const float mx = wave_reduce<true>(fmaxf(fmaxf(y[0], y[1]), fmaxf(y[2], y[3])));
  const float mn = wave_reduce<false>(fminf(fminf(y[0], y[1]), fminf(y[2], y[3])));
  const float thr = clip >= 0 ? select_abs_rank_wave(y, clip) : __builtin_inff();
  const QParams p = make_qparams(mn, mx, thr, clip >= 0);
  const uint32_t byte = int2_code(y[0], p) | (int2_code(y[1], p) << 2) | (int2_code(y[2], p) << 4) |
                        (int2_code(y[3], p) << 6);
  const uint32_t word = byte | ((uint32_t)__shfl((int)byte, lane + 1, 64) << 8) |
                        ((uint32_t)__shfl((int)byte, lane + 2, 64) << 16) |
                        ((uint32_t)__shfl((int)byte, lane + 3, 64) << 24);
  if (s < 0) return;
  int64_t page, prow;
  slot_page_row(a, s, page, prow);
  if (s < a.num_slots) {
    uint8_t* kslot = a.k_cache + page * a.k_page + prow * a.k_tok + (int64_t)h * a.k_head;
    uint8_t* codes = side == 0 ? kslot + kKCodeOff
                               : a.v_cache + page * a.v_page + prow * a.v_tok + (int64_t)h * a.v_head;
    if ((lane & 3) == 0) *reinterpret_cast<uint32_t*>(codes + lane) = word;
    if (lane == 0) *reinterpret_cast<uint32_t*>(kslot + 4 * side) = p.meta;
  }
  if (a.stage_rows <= 0 || !seat_winner(a, t, s, later, lane)) return;
  const bool keep = (keep_word >> (t & 31)) & 1u;
  const int64_t arow = arena_row(a, page);
  const int64_t seat = arow * a.block_size + prow;
  if (side == 0 && h == 0 && lane == 0) a.owner[seat] = keep ? page : -1;
  if (!keep) return;
  float* dst = a.stage + (seat * a.num_kv_heads + h) * kHeadDim;
  *reinterpret_cast<floatx4*>(dst + 4 * lane) = y;
  if (a.img != nullptr) {
    const int64_t tile = image_of(arow, (int)prow, a.block_size, h, a.num_kv_heads);
    const int tt = (int)(prow & 31);
    static_assert(kKImgHalfs == kVImgHalfs, "one image stride for both sides");
    _Float16* img = a.img + tile * kKImgHalfs;
    const int lo = side == 0 ? kImgHalfs : kVPartHalfs;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      _Float16* d = img + (side == 0 ? kimg_offset(4 * lane + c, tt) : vimg_offset(4 * lane + c, tt));
      fp16_parts(y[c], d[0], d[lo]);
    }
  }
}

__global__ __launch_bounds__(kThreads) void step_write_kernel(StepArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kGroupVecs][kHeadDim];
  __shared__ __attribute__((aligned(16))) float part[kWaves][kGroupVecs][kHeadDim];
  const Scalars c = load_scalars(a);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int grp = blockIdx.x;
  int side = 0;                           // 0 keys, 1 values, 2 queries
  if (grp >= 2 * c.kv_groups) {
    side = 2;
    grp -= 2 * c.kv_groups;
  } else if (grp >= c.kv_groups) {
    side = 1;
    grp -= c.kv_groups;
  }
  const int heads = side == 2 ? c.num_heads : c.w.num_kv_heads;
  const int e0 = grp * c.vecs_per_group;
  const int nv = min(c.vecs_per_group, c.w.n_tokens * heads - e0);
  if (nv <= 0) return;
  const uint16_t* src = side == 0 ? c.k : (side == 1 ? c.v : c.q);
  const int64_t stride = side == 2 ? c.q_stride : c.kv_stride;
  const float* R = side == 1 ? c.rot_v : c.rot_k;

  // This thread's 16 rows of R (columns 4l .. 4l + 3) are requested before
  // anything is waited for: one round of loads covers the whole matrix.
  floatx4 r[kRowsPerWave];
  const float* Rw = R + (int64_t)(kRowsPerWave * w) * kHeadDim + 4 * lane;
#pragma unroll
  for (int k = 0; k < kRowsPerWave; ++k) r[k] = *reinterpret_cast<const floatx4*>(Rw + (int64_t)k * kHeadDim);
  // Keys and values: the wave's token slot, the next 64 tokens' slots (seat
  // winner test) and its window keep bits go out with the same round.
  int64_t my_slot = -1, later = -1;
  uint32_t keep_word = 0;
  WriteCtx ctx = c.w;
  ctx.stage = side == 0 ? c.stage_k : c.stage_v;
  ctx.img = side == 0 ? c.kimg : c.vimg;
  ctx.clip = side == 0 ? c.clip_k : c.clip_v;
  if (side < 2 && w < nv) {
    const int t = (e0 + w) / heads;
    keep_word = a.keep[t >> 5];
    my_slot = ctx.slots[t];
    later = t + 1 + lane < ctx.n_tokens ? ctx.slots[t + 1 + lane] : -1;
  }
  for (int idx = tid; idx < nv * kHeadDim; idx += kThreads) {
    const int vv = idx >> 8, f = idx & 255;
    const int e = e0 + vv, t = e / heads, h = e - t * heads;
    xs[vv][f] = bf16_to_f32(src[(int64_t)t * stride + (int64_t)h * kHeadDim + f]);
  }
  __syncthreads();
#pragma unroll
  for (int vv = 0; vv < kGroupVecs; ++vv) {
    if (vv < nv) {
      floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k4 = 0; k4 < kRowsPerWave; k4 += 4) {
        const floatx4 x = *reinterpret_cast<const floatx4*>(&xs[vv][kRowsPerWave * w + k4]);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) acc[cc] = fmaf(x[k], r[k4 + k][cc], acc[cc]);
      }
      *reinterpret_cast<floatx4*>(&part[w][vv][4 * lane]) = acc;
    }
  }
  __syncthreads();
  if (w >= nv) return;
  floatx4 y = *reinterpret_cast<const floatx4*>(&part[0][w][4 * lane]);
#pragma unroll
  for (int ww = 1; ww < kWaves; ++ww) {
    const floatx4 z = *reinterpret_cast<const floatx4*>(&part[ww][w][4 * lane]);
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) y[cc] += z[cc];
  }
  const int e = e0 + w, t = e / heads, h = e - t * heads;
  float* out = side == 0 ? c.k_rot : (side == 1 ? c.v_rot : c.q_rot);
  if (out != nullptr) *reinterpret_cast<floatx4*>(out + ((int64_t)t * heads + h) * kHeadDim + 4 * lane) = y;
  if (side < 2) write_vector(ctx, y, t, h, side, lane, my_slot, later, keep_word);
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
  if (num_tokens < 0 || num_tokens > kMaxStepTokens || num_requests < 0 || num_heads < 0 ||
      num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || block_size <= 0 || num_pages <= 0 ||
      stage_rows < 0 || sink_eff < 0 || recent < 0 || clip_index_k >= kHeadDim || clip_index_v >= kHeadDim)
    return kErrInvalidArgument;
  if (num_tokens == 0) return kOk;
  if (!key_bf16 || !value_bf16 || !rot_k || !rot_v || !slot_mapping || !k_cache || !v_cache ||
      (num_heads > 0 && (!query_bf16 || !q_rot)) || (num_requests > 0 && (!query_start_loc || !seq_lens)))
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
  a.bs_div = make_fast_div((uint32_t)block_size);
  a.rows_div = make_fast_div(stage_rows > 0 ? (uint32_t)stage_rows : 1u);
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
  hipLaunchKernelGGL(step_write_kernel, dim3((unsigned)(2 * a.kv_groups + q_groups)), dim3(kThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
