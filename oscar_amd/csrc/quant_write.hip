// Fused rotate + sort-clip + INT2 quantize + 4-codes-per-byte pack + paged
// slot write (gfx950).
//
// Work layout: one wavefront owns 32 tokens of one (kv-head, K-or-V) side.
// Lane l holds token (l & 31), features 128*(l >> 5) .. +127 of that token in
// 128 fp32 registers, so every per-vector reduction is lane-local plus one
// exchange with lane l ^ 32.  That is exactly the fp32 accumulator layout of
// a 32x32 MFMA tile whose columns are tokens, which the fused entry point
// uses for the 256x256 rotation (bf16 hi + lo split of R, two passes; the
// operand streams through a 4-deep LDS ring filled by direct-to-LDS loads).
//
// Clip threshold (the idx-th smallest |x| of a vector, i.e. its kk-th largest
// with kk = 256 - idx) without sorting: a 64-bucket histogram of |x| keyed on
// the float bits (bucket = key(max|x|) - key(|x|), key = bits >> S, S = 18:
// 1/32 octave per bucket over two octaves) built with LDS atomics gives the
// bucket holding the answer and its rank j inside that bucket; the bucket's
// few values are gathered into small per-lane LDS lists and the j-th largest
// of them is taken exactly (ties counted).  Vectors whose answer lies outside
// the histogram's range or whose bucket overflows the lists use a bitwise
// radix select instead (exact, slow, rare).
//
// Quantization: the exact divide-free thresholds of int2_quant.h.
//
// With a window arena (oscar_quant_write_window) the fused kernel also does
// the window write of the step's bulk tokens from the same rotated values
// (see window_epilogue), after a seat-winner pass over the step's slots.
#include "int2_quant.h"
#include "window_images.h"
#include "../../include/oscar_amd.h"

namespace oscar {
namespace {

constexpr int kPerLane = kHeadDim / 2;      // 128 values of one vector per lane
constexpr int kTokPerWave = 32;

struct CacheArgs {
  uint8_t* k_cache;
  uint8_t* v_cache;
  int64_t k_page, k_tok, k_head;     // byte strides
  int64_t v_page, v_tok, v_head;
  int32_t block_size;
  int64_t num_slots;                 // pages * block_size (< 2^31); larger slots are skipped
  FastDiv bs_div;                    // block_size
};

// Exact value of ascending-sorted |x| at index `idx` over the 256 values held
// by this lane and its partner (l ^ 32).  Bitwise radix select on the IEEE
// bit pattern: for non-negative finite floats, float order equals bit order.
__device__ float select_abs_rank(const float (&v)[kPerLane], int idx) {
  uint32_t prefix = 0;
#pragma unroll 1
  for (int bit = 30; bit >= 0; --bit) {
    const uint32_t probe = prefix | (1u << bit);
    const float pf = __uint_as_float(probe);
    int below = 0;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) below += (fabsf(v[i]) < pf) ? 1 : 0;
    below += __shfl_xor(below, 32, 64);
    if (idx >= below) prefix = probe;
  }
  return __uint_as_float(prefix);
}

// Per-wave LDS of the threshold search: 32 token histograms (64 buckets + one
// bucket for everything below the range; stride 65 words keeps the tokens of
// one wave on different banks) and one candidate list per lane.
constexpr int kHistBuckets = 64;
constexpr int kHistStride = kHistBuckets + 1;
constexpr int kListCap = 8;
constexpr int kListStride = kListCap + 1;          // + one slot that absorbs non-candidates
struct SelLds {
  uint32_t hist[32 * kHistStride];
  uint32_t list[64 * kListStride];
};

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// kk-th largest |x| (kk = 256 - idx) of the 256 values held by this lane and
// its partner, as float bits; amax_bits = bits of max |x| over both lanes.
__device__ uint32_t select_clip_bits(const float (&v)[kPerLane], int idx, uint32_t amax_bits, SelLds& L,
                                     int lane) {
  const uint32_t kk = (uint32_t)(kHeadDim - idx);
  const int t = lane & 31, g = lane >> 5;
  const int S = kk <= 40 ? 18 : 20;          // 1/32 octave per bucket (2 octaves); coarser for deep ranks
  uint4* hz = reinterpret_cast<uint4*>(L.hist);
  for (int i = lane; i < 32 * kHistStride / 4; i += 64) hz[i] = uint4{0u, 0u, 0u, 0u};
  wave_sync_lds();
  // Row t: word 0 absorbs every key below the window, word 1 + j counts key
  // kl + j (kl = kh - 63), so bucket b from the top (key kh - b) is word 64 - b.
  // The byte address of key's word is 4 key + (row + 4 - 4 kl) on the 32-bit
  // LDS address, clamped from below to the absorbing word.
  typedef __attribute__((address_space(3))) uint32_t lds_u32;
  uint32_t* H = L.hist + t * kHistStride;
  const uint32_t kh = amax_bits >> S;
  const int32_t row = (int32_t)(uint32_t)(uintptr_t)(lds_u32*)H;
  const uint32_t base = (uint32_t)(row + 4 - 4 * ((int32_t)kh - (kHistBuckets - 1)));
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const uint32_t key = __builtin_amdgcn_ubfe(__float_as_uint(v[i]), S, 31 - S);
    const int32_t addr = max((int32_t)((key << 2) + base), row);
    __atomic_fetch_add((lds_u32*)(uintptr_t)(uint32_t)addr, 1u, __ATOMIC_RELAXED);
  }
  wave_sync_lds();

  // Bucket b* where the count from the top reaches kk; lane g scans buckets
  // 32g .. 32g + 31.
  uint32_t cnt[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) cnt[i] = H[kHistBuckets - 32 * g - i];
  uint32_t tot = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) tot += cnt[i];
  // (the exchange runs on every lane: a shuffle reads only active lanes)
  const uint32_t tot0 = (uint32_t)__shfl((int)tot, t, 64);
  uint32_t run = g ? tot0 : 0u;
  int bf = -1;
  uint32_t above = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    if (bf < 0 && run + cnt[i] >= kk) {
      bf = 32 * g + i;
      above = run;
    }
    run += cnt[i];
  }
  const int b0 = __shfl(bf, t, 64), b1 = __shfl(bf, t + 32, 64);
  const uint32_t a0 = (uint32_t)__shfl((int)above, t, 64), a1 = (uint32_t)__shfl((int)above, t + 32, 64);
  const int bstar = b0 >= 0 ? b0 : b1;
  const uint32_t ab = b0 >= 0 ? a0 : a1;
  const uint32_t keystar = kh - (uint32_t)bstar;
  bool fb = bstar < 0 || keystar == 0;

  // Gather bucket b*'s values: every value is written at the lane's next free
  // slot, which only advances on a match (capped at the absorbing slot).
  // The raw bits are stored (sign cleared on reading them back); the match
  // |x| >> S == keystar is tested on bits << 1, which drops the sign, as one
  // wrapping subtract and compare.
  uint32_t* mine = L.list + lane * kListStride;
  uint32_t n = 0;
  const uint32_t lo2 = keystar << (S + 1), w2 = 2u << S;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const uint32_t u = __float_as_uint(v[i]);
    mine[min(n, (uint32_t)kListCap)] = u;
    n += ((u << 1) - lo2 < w2) ? 1u : 0u;
  }
  wave_sync_lds();
  const uint32_t n0 = (uint32_t)__shfl((int)n, t, 64), n1 = (uint32_t)__shfl((int)n, t + 32, 64);
  fb = fb || n0 > kListCap || n1 > kListCap;
  uint32_t c[2 * kListCap];
  const uint32_t* l0 = L.list + t * kListStride;
  const uint32_t* l1 = L.list + (t + 32) * kListStride;
#pragma unroll
  for (int i = 0; i < kListCap; ++i) {
    c[i] = (uint32_t)i < n0 ? l0[i] & 0x7FFFFFFFu : 0u;
    c[kListCap + i] = (uint32_t)i < n1 ? l1[i] & 0x7FFFFFFFu : 0u;
  }
  // j-th largest of the candidates (j = kk - above >= 1), ties counted.
  uint32_t rem = kk - ab, prev = 0xFFFFFFFFu, res = 0u;
  if (fb) rem = 0;
#pragma unroll 1
  for (int it = 0; it <= 2 * kListCap && __ballot(rem > 0); ++it) {
    uint32_t m = 0u;
#pragma unroll
    for (int i = 0; i < 2 * kListCap; ++i) m = max(m, c[i] < prev ? c[i] : 0u);
    uint32_t ce = 0u;
#pragma unroll
    for (int i = 0; i < 2 * kListCap; ++i) ce += (c[i] == m) ? 1u : 0u;
    if (rem > 0) {
      if (m == 0u) {
        fb = true;
        rem = 0;
      } else if (ce >= rem) {
        res = m;
        rem = 0;
      } else {
        rem -= ce;
        prev = m;
      }
    }
  }
  if (__ballot(fb)) {
    const uint32_t r = __float_as_uint(select_abs_rank(v, idx));
    if (fb) res = r;
  }
  return res;
}

__device__ QParams vector_params(const float (&v)[kPerLane], int clip_idx, SelLds& L, int lane) {
  float mx = v[0], mn = v[0];
#pragma unroll
  for (int i = 1; i < kPerLane; ++i) {
    mx = fmaxf(mx, v[i]);
    mn = fminf(mn, v[i]);
  }
  mx = fmaxf(mx, shfl_xor_f32(mx, 32));
  mn = fminf(mn, shfl_xor_f32(mn, 32));
  float thr = __builtin_inff();
  if (clip_idx >= 0) {
    const uint32_t amax_bits = max(__float_as_uint(mx) & 0x7FFFFFFFu, __float_as_uint(mn) & 0x7FFFFFFFu);
    thr = __uint_as_float(select_clip_bits(v, clip_idx, amax_bits, L, lane));
  }
  return make_qparams(mn, mx, thr, clip_idx >= 0);
}

// Quantize, pack and store this lane's 128 codes (32 bytes) plus, on the
// lower half lane, the 4 meta bytes of this side.
__device__ void quantize_store(const float (&v)[kPerLane], const QParams& p, int64_t slot,
                               int head, int side, int half, const CacheArgs& c) {
  uint32_t words[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t acc = 0;
#pragma unroll
    for (int i = 15; i >= 0; --i) acc = (acc << 2) | int2_code(v[16 * w + i], p);
    words[w] = acc;
  }
  if (slot < 0 || slot >= c.num_slots) return;
  const int64_t page = fast_div((uint32_t)slot, c.bs_div);
  const int64_t row = slot - page * c.block_size;
  uint8_t* kslot = c.k_cache + page * c.k_page + row * c.k_tok + (int64_t)head * c.k_head;
  uint8_t* dst;
  if (side == 0) {
    dst = kslot + kKCodeOff + 32 * half;
  } else {
    dst = c.v_cache + page * c.v_page + row * c.v_tok + (int64_t)head * c.v_head + 32 * half;
  }
  u32x4* d4 = reinterpret_cast<u32x4*>(dst);
  d4[0] = u32x4{words[0], words[1], words[2], words[3]};
  d4[1] = u32x4{words[4], words[5], words[6], words[7]};
  if (half == 0) *reinterpret_cast<uint32_t*>(kslot + 4 * side) = p.meta;
}

// The window arena of a bulk write (rows = 0: none).
struct WindowArgs {
  const int32_t* query_start;   // [num_requests + 1] on the device
  const int32_t* seq_lens;      // [num_requests]
  int32_t num_requests;
  int32_t rows;
  int32_t sink_eff, recent;
  int32_t num_kv_heads;
  float* stage_k;               // [rows][bs][Hk][D] fp32
  float* stage_v;
  int64_t* owner;               // [rows][bs]
  int64_t* winner;              // seat winners (read after this call's pass)
  _Float16* kimg;               // operand images, or null
  _Float16* vimg;
};

// The window half of the bulk write (the reference's _staging_write,
// backend.py:439-481) for this lane's token (slot >= 0): if the token won
// its seat, it sets the seat's owner (the K side of head 0 does) to its page
// when it lies in the sink or recent window and to -1 otherwise; a kept token
// then stores this lane's 128 unclipped rotated values (features 128 half ..
// +127 of this side and head) and their fp16 image parts.  The lane's token
// half is exactly one lane of the K image (token row prow % 32, half g), so
// the K parts go out as 16-byte blocks; the V image holds tokens in slots, so
// each V value is two 2-byte stores.
__device__ void window_epilogue(const float (&v)[kPerLane], int64_t tok, int64_t slot, int head, int side, int half,
                                int block_size, const WindowArgs& w) {
  int64_t seat, page;
  if (!won_seat(w.winner, (int64_t)w.rows * block_size, slot, tok, block_size, w.rows, seat, page)) return;
  int lo = 0, hi = w.num_requests - 1;       // request of the token: last i with query_start[i] <= tok
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (w.query_start[mid] <= tok) lo = mid; else hi = mid - 1;
  }
  const int64_t seq = w.seq_lens[lo];
  const int64_t pos = seq - w.query_start[lo + 1] + tok;
  const bool keep = pos >= seq - w.recent || pos < w.sink_eff;
  if (side == 0 && head == 0 && half == 0) w.owner[seat] = keep ? page : -1;
  if (!keep) return;
  float* dst = (side == 0 ? w.stage_k : w.stage_v) + (seat * w.num_kv_heads + head) * kHeadDim + kPerLane * half;
#pragma unroll
  for (int k = 0; k < kPerLane / 4; ++k)
    reinterpret_cast<floatx4*>(dst)[k] = floatx4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
  if (w.kimg == nullptr) return;
  const int prow = (int)(slot - page * block_size);
  const int64_t tile = image_of(seat / block_size, prow, block_size, head, w.num_kv_heads);
  const int tt = prow & 31;
  if (side == 0) {
    // block m = 2j + a, slot u = 2i + b: local feature 16j + 4a + i + 8b
    _Float16* img = w.kimg + tile * kKImgHalfs + (tt + 32 * half) * 8;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      half8 h, l;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float x = v[16 * (m >> 1) + 4 * (m & 1) + (u >> 1) + 8 * (u & 1)];
        h[u] = (_Float16)x;
        l[u] = (_Float16)(x - (float)h[u]);
      }
      *reinterpret_cast<half8*>(img + m * 64 * 8) = h;
      *reinterpret_cast<half8*>(img + kImgHalfs + m * 64 * 8) = l;
    }
  } else {
    _Float16* img = w.vimg + tile * kVImgHalfs;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      _Float16* d = img + vimg_offset(kPerLane * half + k, tt);
      fp16_parts(v[k], d[0], d[kVPartHalfs]);
    }
  }
}

__global__ __launch_bounds__(256) void quant_window_winner_kernel(const int64_t* __restrict__ slots, int32_t n_tokens,
                                                                   int64_t* winner, int32_t block_size, int32_t rows) {
  __shared__ int64_t epoch;
  seat_winner_pass(slots, n_tokens, winner, (int64_t)rows * block_size, block_size, rows, &epoch);
}

// ---------------------------------------------------------------------------
// Pre-rotated entry: fp32 rotated input [N, Hk, D] (token stride in elements).
// grid = (ceil(N / 128), Hk * 2), block = 256 (4 waves x 32 tokens).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quant_write_prerotated_kernel(
    const float* __restrict__ k_rot, const float* __restrict__ v_rot, int64_t n_tokens,
    int64_t token_stride, const int64_t* __restrict__ slots, CacheArgs c, int clip_k,
    int clip_v) {
  __shared__ SelLds sel[4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int head = blockIdx.y >> 1;
  const int side = blockIdx.y & 1;
  const int half = lane >> 5;
  const int64_t tok = (int64_t)blockIdx.x * 128 + wave * kTokPerWave + (lane & 31);
  const bool live = tok < n_tokens;
  const float* src = (side == 0 ? k_rot : v_rot) + (live ? tok : 0) * token_stride +
                     (int64_t)head * kHeadDim + half * kPerLane;
  float v[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; i += 4) {
    floatx4 x = live ? *reinterpret_cast<const floatx4*>(src + i) : floatx4{0.f, 0.f, 0.f, 0.f};
    v[i] = x[0];
    v[i + 1] = x[1];
    v[i + 2] = x[2];
    v[i + 3] = x[3];
  }
  const QParams p = vector_params(v, side == 0 ? clip_k : clip_v, sel[wave], lane);
  quantize_store(v, p, live ? slots[tok] : -1, head, side, half, c);
}

// ---------------------------------------------------------------------------
// Fused entry: bf16 input, rotation on MFMA.
//
// Rotation operand (prepared once per layer by oscar_rotation_operand):
//   op[m][p][T][lane][u] (bf16), m = 16-row K step, p = 0 hi / 1 lo split,
//   T = 32-feature output tile.  Entry = R[e][f] with
//     e = 128*(lane >> 5) + 8*m + u                      (input feature)
//     f = 128*((r >> 2) & 1) + 16*T + 4*(r >> 3) + (r & 3), r = lane & 31
//   so that accumulator register i of tile T in lane l is feature
//   128*(l >> 5) + 16*T + i of token (l & 31) -- the per-lane layout above.
// grid = (ceil(N / 128), Hk * 2), block = 256 (4 waves x 32 tokens; two
// blocks per CU).  The 16 K-step chunks (16 KB each) stream through a 4-slot
// LDS ring filled with buffer_load_dwordx4 ... lds: chunk m + 3 is requested
// while chunk m is multiplied, into the slot chunk m - 1 left.  Each K step
// issues the 8 tiles' hi passes, then their lo passes, so no MFMA waits on the
// previous.
// ---------------------------------------------------------------------------
constexpr int kFusedWaves = 4;
constexpr int kChunkBytes = 2 * 8 * 64 * 16;   // one K step: 2 passes x 8 tiles x 64 lanes x 16 B
constexpr int kRing = 4;
constexpr int kSteps = 16;
// The rotation operand: the MFMA tiles (kSteps chunks, bf16 hi + lo), then R
// itself in fp32 (row-major), which short writes rotate with.
constexpr int kMfmaEntries = kSteps * kChunkBytes / 2;
constexpr size_t kMfmaOperandBytes = (size_t)kSteps * kChunkBytes;
constexpr size_t kOperandBytes = kMfmaOperandBytes + sizeof(float) * kHeadDim * kHeadDim;
constexpr int64_t kShortWriteVectors = 2048;   // at most 1024 tokens (the step write's limit)
constexpr int kDmaPerChunk = kChunkBytes / (kFusedWaves * 64 * 16);   // 2 per thread
constexpr size_t kFusedLds = kFusedWaves * sizeof(SelLds) > kRing * kChunkBytes
                                 ? kFusedWaves * sizeof(SelLds) : (size_t)kRing * kChunkBytes;

// Workgroup barrier without a memory fence: __syncthreads() would also wait
// for every outstanding global access (vmcnt(0)) and so drain the ring's
// prefetches.  The asm memory clobber keeps the compiler from moving LDS
// accesses across it; LDS visibility comes from the vmcnt waits above it
// (direct-to-LDS loads count as complete once their data is in LDS) and
// from the LDS reads' own completion before the next overwrite.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);                     // lgkmcnt(0): this wave's LDS reads done
  asm volatile("s_barrier" ::: "memory");
}

// s_waitcnt vmcnt(n) with expcnt / lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__global__ __launch_bounds__(256, 2) void quant_write_fused_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value, int64_t n_tokens,
    int64_t token_stride, const uint8_t* __restrict__ rot_k, const uint8_t* __restrict__ rot_v,
    const int64_t* __restrict__ slots, CacheArgs c, int clip_k, int clip_v, WindowArgs w) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];     // ring, then the selection buffers
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int head = blockIdx.y >> 1;
  const int side = blockIdx.y & 1;
  const int half = lane >> 5;
  const int64_t tok = (int64_t)blockIdx.x * (kFusedWaves * kTokPerWave) + wave * kTokPerWave + (lane & 31);
  const bool live = tok < n_tokens;
  const uint8_t* rop = side == 0 ? rot_k : rot_v;

  // B operand of K step m: this lane's token, input features 128*half + 8m .. +7.
  // Loaded in two halves, each one 128-byte line of the lane's half-row:
  // steps 0..7 up front, steps 8..15 during step 4, so the first step waits
  // for half the loads and each line is still fetched in one burst.
  const uint16_t* xsrc = (side == 0 ? key : value) + (live ? tok : 0) * token_stride +
                         (int64_t)head * kHeadDim + half * kPerLane;
  // A lane past the last token reads token 0: its MFMA column (and the
  // vector the selection then computes) is never stored.
  auto load_x = [&](int m) -> bf16x8 {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(xsrc + 8 * m));
  };
  bf16x8 xlo[8], xhi[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) xlo[m] = load_x(m);
  // Thread's share of a chunk: wave w copies 1 KB blocks 4w .. 4w + 3.  The
  // copies are buffer loads: unlike the flat-encoded global form, they count
  // only in vmcnt, so the operand reads from LDS below keep a partial
  // lgkmcnt wait each instead of draining every outstanding LDS read.
  typedef __attribute__((address_space(3))) void lds_void;
  const __amdgpu_buffer_rsrc_t rop_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)rop, (short)0, (int)(kSteps * kChunkBytes), 0x00020000);
  auto request = [&](int chunk) {
#pragma unroll
    for (int i = 0; i < kDmaPerChunk; ++i) {
      const int blk = kDmaPerChunk * wave + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rop_rsrc, (lds_void*)(uintptr_t)(uint32_t)(uintptr_t)(ring + (chunk % kRing) * kChunkBytes + blk * 1024),
          16, chunk * kChunkBytes + (blk * 64 + lane) * 16, 0, 0, 0);
    }
  };
  request(0);
  request(1);
  request(2);

  floatx16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx16{};

#pragma unroll
  for (int m = 0; m < kSteps; ++m) {
    // This thread's copies of chunk m (and x_m) have landed (later ones may
    // still be in flight); after the barrier every thread's have, and chunk
    // m - 1's slot is free for chunk m + 3.  Issue order: x_0..7, chunks
    // 0..2, then per step chunk m + 3, and x_8..15 after chunk 7 (step 4);
    // what was issued after chunk m is left outstanding.
    if (m >= 5 && m <= 7) wait_vmcnt<2 * kDmaPerChunk + 8>();
    else if (m + 2 < kSteps) wait_vmcnt<2 * kDmaPerChunk>();
    else if (m + 1 < kSteps) wait_vmcnt<kDmaPerChunk>();
    else wait_vmcnt<0>();
    lds_barrier();
    if (m + 3 < kSteps) request(m + 3);
    // The waits of steps 5-7 count x_8..15 after chunk 7's copies: keep the
    // scheduler from hoisting any of those loads above the request (one
    // hoisted load would leave chunk 7's last copy unwaited at step 7).
    __builtin_amdgcn_sched_barrier(0);
    if (m == 4) {
#pragma unroll
      for (int k = 0; k < 8; ++k) xhi[k] = load_x(8 + k);
    }
    const bf16x8 xm = m < 8 ? xlo[m] : xhi[m - 8];
    const u32x4* a_src = reinterpret_cast<const u32x4*>(ring + (m % kRing) * kChunkBytes);
    // Operand reads run kAhead MFMAs ahead of their use (register rotation);
    // the 8 tiles' hi passes come first, then their lo passes.
    constexpr int kAhead = 6;
    bf16x8 a[kAhead];
#pragma unroll
    for (int i = 0; i < kAhead; ++i) a[i] = __builtin_bit_cast(bf16x8, a_src[i * 64 + lane]);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const bf16x8 cur = a[i % kAhead];
      if (i + kAhead < 16) a[i % kAhead] = __builtin_bit_cast(bf16x8, a_src[(i + kAhead) * 64 + lane]);
      acc[i & 7] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur, xm, acc[i & 7], 0, 0, 0);
    }
    // Keep that pipeline in the schedule: kAhead LDS reads, then each MFMA
    // followed by the read kAhead positions ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + kAhead < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  }
  __syncthreads();      // the ring becomes the waves' selection buffers

  float v[kPerLane];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[16 * t + i] = acc[t][i];
  }
  SelLds& sel = reinterpret_cast<SelLds*>(ring)[wave];
  const QParams p = vector_params(v, side == 0 ? clip_k : clip_v, sel, lane);
  const int64_t slot = live ? slots[tok] : -1;
  quantize_store(v, p, slot, head, side, half, c);
  if (w.rows > 0 && slot >= 0) window_epilogue(v, tok, slot, head, side, half, c.block_size, w);
}

// ---------------------------------------------------------------------------
// Rows rotated on MFMA: out = in @ R for rows of D = 256 features (the
// prefill route's q / k / v rotations and its output's R_v^T,
// oscar_ascend/backend.py:392-413).  in: bf16 (an exact operand) or fp32
// (its bf16 high and low parts); R: the operand's bf16 high and low parts;
// fp32 accumulation (about 2^-16 of each product); out: fp32, or bf16
// rounded to nearest even.
// grid = ceil(rows / 128), block = 256 (4 waves x 32 rows): lane l takes row
// (l & 31) of its wave, input and output features 128 (l >> 5) .. +127, and
// the operand streams through the fused kernel's 4-slot LDS ring.  A bf16
// input's first half (K steps 0-7) is requested before the ring and its
// second half during step 4; an fp32 input (twice the registers) comes in
// quarters, the first before the ring and quarter q (steps 4q .. 4q + 3)
// during step 4q - 3.  kRotWait gives each step's wait: the loads issued
// after the last one the step needs (its chunk and its input).
// ---------------------------------------------------------------------------
template <bool kF32In>
struct RotSched {
  static constexpr int kParts = kF32In ? 4 : 2;                 // input parts (quarters / halves)
  static constexpr int kPartLoads = 2 * kSteps / kParts / (kF32In ? 1 : 2);   // 16-byte loads per part
  // step during which part p (> 0) is requested
  static __device__ constexpr int step_of(int p) { return kF32In ? 4 * p - 3 : 4; }
};
template <bool kF32In>
__device__ constexpr int kRotWait(int m) {
  return kF32In ? (m == 14 ? 4 : m == 15 ? 0 : ((m & 3) >= 2 ? 16 : 8))
                : ((m >= 5 && m <= 7) ? 16 : m == 14 ? 4 : m == 15 ? 0 : 8);
}

template <bool kF32In, bool kBf16Out>
__global__ __launch_bounds__(256, 2) void rotate_rows_kernel(const void* __restrict__ in, int64_t in_stride,
                                                            int64_t rows, const uint8_t* __restrict__ rop,
                                                            void* __restrict__ out, int64_t out_stride) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
  using Sched = RotSched<kF32In>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int half = lane >> 5;
  const int64_t row = (int64_t)blockIdx.x * (kFusedWaves * kTokPerWave) + wave * kTokPerWave + (lane & 31);
  const bool live = row < rows;
  const int64_t rr = live ? row : 0;        // a lane past the last row computes row 0 and stores nothing
  // input of K step m: features 128 half + 8m .. +7 (one 16-byte load, or two for fp32)
  u32x4 xr[Sched::kParts * Sched::kPartLoads];
  const uint8_t* xsrc = static_cast<const uint8_t*>(in) + (rr * in_stride + kPerLane * half) * (kF32In ? 4 : 2);
  auto load_part = [&](int p) {
#pragma unroll
    for (int i = 0; i < Sched::kPartLoads; ++i)
      xr[p * Sched::kPartLoads + i] = reinterpret_cast<const u32x4*>(xsrc)[p * Sched::kPartLoads + i];
  };
  load_part(0);
  typedef __attribute__((address_space(3))) void lds_void;
  const __amdgpu_buffer_rsrc_t rop_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)rop, (short)0, (int)(kSteps * kChunkBytes), 0x00020000);
  auto request = [&](int chunk) {
#pragma unroll
    for (int i = 0; i < kDmaPerChunk; ++i) {
      const int blk = kDmaPerChunk * wave + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rop_rsrc, (lds_void*)(uintptr_t)(uint32_t)(uintptr_t)(ring + (chunk % kRing) * kChunkBytes + blk * 1024),
          16, chunk * kChunkBytes + (blk * 64 + lane) * 16, 0, 0, 0);
    }
  };
  request(0);
  request(1);
  request(2);
  floatx16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx16{};
  constexpr int kPairs = kF32In ? 24 : 16;      // (fragment, operand) products per K step
#pragma unroll
  for (int m = 0; m < kSteps; ++m) {
    {
      // (m is a constant once the loop is unrolled: one wait remains)
      const int wn = kRotWait<kF32In>(m);
      if (wn == 24) wait_vmcnt<24>();
      else if (wn == 16) wait_vmcnt<16>();
      else if (wn == 8) wait_vmcnt<8>();
      else if (wn == 4) wait_vmcnt<4>();
      else wait_vmcnt<0>();
    }
    lds_barrier();
    if (m + 3 < kSteps) request(m + 3);
    // the wait counts above assume every input load of a part after this
    // step's chunk request: keep the scheduler from hoisting one
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 1; p < Sched::kParts; ++p)
      if (m == Sched::step_of(p)) load_part(p);
    bf16x8 xh, xl;
    if constexpr (kF32In) {
      const floatx4 f0 = __builtin_bit_cast(floatx4, xr[2 * m]), f1 = __builtin_bit_cast(floatx4, xr[2 * m + 1]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float v = u < 4 ? f0[u] : f1[u - 4];
        const __bf16 h = (__bf16)v;
        xh[u] = h;
        xl[u] = (__bf16)(v - (float)h);
      }
    } else {
      xh = __builtin_bit_cast(bf16x8, xr[m]);
      xl = xh;
    }
    // pair i < 16: fragment i (8 p + t) times the high part; i >= 16 (fp32
    // input): fragment i - 16 (R's high part) times the low part
    const u32x4* a_src = reinterpret_cast<const u32x4*>(ring + (m % kRing) * kChunkBytes);
    constexpr int kAhead = 6;
    bf16x8 a[kAhead];
#pragma unroll
    for (int i = 0; i < kAhead; ++i) a[i] = __builtin_bit_cast(bf16x8, a_src[(i & 15) * 64 + lane]);
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
      const bf16x8 cur = a[i % kAhead];
      if (i + kAhead < kPairs)
        a[i % kAhead] = __builtin_bit_cast(bf16x8, a_src[((i + kAhead) & 15) * 64 + lane]);
      acc[i & 7] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur, i < 16 ? xh : xl, acc[i & 7], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + kAhead < kPairs) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  }
  if (!live) return;
  // register i of tile t: output feature 128 half + 16 t + i
  if constexpr (kBf16Out) {
    __bf16* dst = static_cast<__bf16*>(out) + row * out_stride + kPerLane * half;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        bf16x8 o;
#pragma unroll
        for (int u = 0; u < 8; ++u) o[u] = (__bf16)acc[t][8 * q + u];
        *reinterpret_cast<bf16x8*>(dst + 16 * t + 8 * q) = o;
      }
  } else {
    float* dst = static_cast<float*>(out) + row * out_stride + kPerLane * half;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<floatx4*>(dst + 16 * t + 4 * q) =
            floatx4{acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
  }
}

// One thread per operand element (2 x 16 x 8 x 64 x 8 = 131072 entries), then
// one per element of the fp32 copy of R that follows them (65536 entries).
__global__ void rotation_operand_kernel(const float* __restrict__ R, __bf16* __restrict__ out) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= kMfmaEntries) {
    if (idx < kMfmaEntries + kHeadDim * kHeadDim)
      reinterpret_cast<float*>(out + kMfmaEntries)[idx - kMfmaEntries] = R[idx - kMfmaEntries];
    return;
  }
  const int u = idx & 7;
  const int lane = (idx >> 3) & 63;
  const int t = (idx >> 9) & 7;
  const int p = (idx >> 12) & 1;
  const int m = idx >> 13;
  const int r = lane & 31;
  const int e = 128 * (lane >> 5) + 8 * m + u;
  const int f = 128 * ((r >> 2) & 1) + 16 * t + 4 * (r >> 3) + (r & 3);
  const float x = R[e * kHeadDim + f];
  const __bf16 hi = (__bf16)x;
  out[idx] = p == 0 ? hi : (__bf16)(x - (float)hi);
}

int check_cache_args(CacheArgs& c) {
  if (c.block_size <= 0 || c.num_slots <= 0 || c.k_cache == nullptr || c.v_cache == nullptr)
    return kErrInvalidArgument;
  if (c.num_slots >= ((int64_t)1 << 31)) return kErrUnsupportedGeometry;
  if (c.k_head < kKCodeOff + kCodeBytes || c.v_head < kCodeBytes) return kErrUnsupportedGeometry;
  const int64_t strides[6] = {c.k_page, c.k_tok, c.k_head, c.v_page, c.v_tok, c.v_head};
  for (int64_t s : strides)
    if (s <= 0 || (s & 15) != 0) return kErrUnsupportedGeometry;
  c.bs_div = make_fast_div((uint32_t)c.block_size);
  if ((reinterpret_cast<uintptr_t>(c.k_cache) & 15) || (reinterpret_cast<uintptr_t>(c.v_cache) & 15))
    return kErrUnsupportedGeometry;
  return kOk;
}

std::atomic<uint64_t> g_lds_set{0};   // dynamic-LDS attribute set, one bit per device
std::atomic<uint64_t> g_rot_lds_set[4] = {{0}, {0}, {0}, {0}};   // the same for the rotate_rows instances

}  // namespace
}  // namespace oscar

using namespace oscar;

extern "C" {

size_t oscar_rotation_operand_bytes(int32_t head_size) {
  return head_size == kHeadDim ? kOperandBytes : 0;
}

int oscar_rotation_operand(const float* rotation, void* operand, int32_t head_size,
                           hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (rotation == nullptr || operand == nullptr) return kErrInvalidArgument;
  const int total = kMfmaEntries + kHeadDim * kHeadDim;
  hipLaunchKernelGGL(rotation_operand_kernel, dim3((total + 255) / 256), dim3(256), 0, stream,
                     rotation, static_cast<__bf16*>(operand));
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int oscar_rotate_rows(const void* in, int32_t in_f32, int64_t in_row_stride, int64_t rows, int32_t head_size,
                      const void* rot_operand, void* out, int32_t out_bf16, int64_t out_row_stride,
                      hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (rows < 0 || (in_f32 != 0 && in_f32 != 1) || (out_bf16 != 0 && out_bf16 != 1)) return kErrInvalidArgument;
  if (rows == 0) return kOk;
  if (!in || !rot_operand || !out || in_row_stride < kHeadDim || out_row_stride < kHeadDim)
    return kErrInvalidArgument;
  // 16-byte vector accesses: every row start 16-byte aligned
  const int64_t in_bytes = in_f32 ? 4 : 2, out_bytes = out_bf16 ? 2 : 4;
  if (((in_row_stride * in_bytes) & 15) || ((out_row_stride * out_bytes) & 15) ||
      (reinterpret_cast<uintptr_t>(in) & 15) || (reinterpret_cast<uintptr_t>(out) & 15) ||
      (reinterpret_cast<uintptr_t>(rot_operand) & 15))
    return kErrInvalidArgument;
  const int64_t per_block = kFusedWaves * kTokPerWave;
  const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
  const uint8_t* rop = static_cast<const uint8_t*>(rot_operand);
  const void* k[4] = {reinterpret_cast<const void*>(rotate_rows_kernel<false, false>),
                      reinterpret_cast<const void*>(rotate_rows_kernel<false, true>),
                      reinterpret_cast<const void*>(rotate_rows_kernel<true, false>),
                      reinterpret_cast<const void*>(rotate_rows_kernel<true, true>)};
  const int which = 2 * in_f32 + out_bf16;
  constexpr int kRingLds = kRing * kChunkBytes;
  if (set_dynamic_lds(k[which], kRingLds, g_rot_lds_set[which]) != kOk) return kErrLaunch;
  if (in_f32 && out_bf16)
    hipLaunchKernelGGL((rotate_rows_kernel<true, true>), grid, dim3(256), kRingLds, stream, in, in_row_stride, rows,
                       rop, out, out_row_stride);
  else if (in_f32)
    hipLaunchKernelGGL((rotate_rows_kernel<true, false>), grid, dim3(256), kRingLds, stream, in, in_row_stride, rows,
                       rop, out, out_row_stride);
  else if (out_bf16)
    hipLaunchKernelGGL((rotate_rows_kernel<false, true>), grid, dim3(256), kRingLds, stream, in, in_row_stride, rows,
                       rop, out, out_row_stride);
  else
    hipLaunchKernelGGL((rotate_rows_kernel<false, false>), grid, dim3(256), kRingLds, stream, in, in_row_stride, rows,
                       rop, out, out_row_stride);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int oscar_quant_write_prerotated(const float* k_rot, const float* v_rot, int64_t num_tokens,
                                 int32_t num_kv_heads, int32_t head_size, int64_t token_stride,
                                 const int64_t* slot_mapping, void* k_cache, void* v_cache,
                                 int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                                 int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                                 int64_t v_stride_token, int64_t v_stride_head,
                                 int32_t clip_index_k, int32_t clip_index_v, hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_kv_heads <= 0 || clip_index_k >= kHeadDim || clip_index_v >= kHeadDim)
    return kErrInvalidArgument;
  if (num_tokens == 0) return kOk;
  if (k_rot == nullptr || v_rot == nullptr || slot_mapping == nullptr) return kErrInvalidArgument;
  if (token_stride < (int64_t)num_kv_heads * kHeadDim || (token_stride & 3) ||
      (reinterpret_cast<uintptr_t>(k_rot) & 15) || (reinterpret_cast<uintptr_t>(v_rot) & 15))
    return kErrInvalidArgument;
  CacheArgs c{static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache), k_stride_page,
              k_stride_token, k_stride_head, v_stride_page, v_stride_token, v_stride_head,
              block_size, num_pages * (int64_t)block_size, FastDiv{}};
  int st = check_cache_args(c);
  if (st != kOk) return st;
  dim3 grid((unsigned)((num_tokens + 127) / 128), (unsigned)(num_kv_heads * 2));
  hipLaunchKernelGGL(quant_write_prerotated_kernel, grid, dim3(256), 0, stream, k_rot, v_rot,
                     num_tokens, token_stride, slot_mapping, c, (int)clip_index_k,
                     (int)clip_index_v);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"

namespace {

// oscar_quant_write with an optional window arena (w.rows > 0).
int quant_write_impl(const void* key_bf16, const void* value_bf16, int64_t num_tokens, int32_t num_kv_heads,
                     int32_t head_size, int64_t token_stride, const void* rot_k_operand, const void* rot_v_operand,
                     const int64_t* slot_mapping, void* k_cache, void* v_cache, int32_t block_size,
                     int64_t num_pages, int64_t k_stride_page, int64_t k_stride_token, int64_t k_stride_head,
                     int64_t v_stride_page, int64_t v_stride_token, int64_t v_stride_head, int32_t clip_index_k,
                     int32_t clip_index_v, const WindowArgs& w, hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_kv_heads <= 0 || clip_index_k >= kHeadDim || clip_index_v >= kHeadDim)
    return kErrInvalidArgument;
  if (num_tokens == 0) return kOk;
  if (key_bf16 == nullptr || value_bf16 == nullptr || slot_mapping == nullptr ||
      rot_k_operand == nullptr || rot_v_operand == nullptr)
    return kErrInvalidArgument;
  if (token_stride < (int64_t)num_kv_heads * kHeadDim || (token_stride & 7) ||
      (reinterpret_cast<uintptr_t>(key_bf16) & 15) || (reinterpret_cast<uintptr_t>(value_bf16) & 15) ||
      (reinterpret_cast<uintptr_t>(rot_k_operand) & 15) ||
      (reinterpret_cast<uintptr_t>(rot_v_operand) & 15))
    return kErrInvalidArgument;
  CacheArgs c{static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache), k_stride_page,
              k_stride_token, k_stride_head, v_stride_page, v_stride_token, v_stride_head,
              block_size, num_pages * (int64_t)block_size, FastDiv{}};
  int st = check_cache_args(c);
  if (st != kOk) return st;
  // Short writes (at most kShortWriteVectors key + value vectors): the fp32
  // rotation of the short-step write (1024-thread workgroups of one to four
  // vectors, R read from the operand's fp32 copy), instead of a 128-token
  // MFMA tile that streams the whole operand through one CU's LDS for a few
  // tokens (4 tokens: 19.4 -> 6.2 us).
  if (2 * num_tokens * num_kv_heads <= kShortWriteVectors) {
    const uint8_t* ok = static_cast<const uint8_t*>(rot_k_operand) + kMfmaOperandBytes;
    const uint8_t* ov = static_cast<const uint8_t*>(rot_v_operand) + kMfmaOperandBytes;
    const bool win = w.rows > 0;
    return oscar_step_write(nullptr, 0, key_bf16, value_bf16, token_stride, (int32_t)num_tokens, 0, num_kv_heads,
                            head_size, reinterpret_cast<const float*>(ok), reinterpret_cast<const float*>(ov),
                            slot_mapping, win ? w.query_start : nullptr, win ? w.seq_lens : nullptr,
                            win ? w.num_requests : 0, k_cache, v_cache, block_size, num_pages, k_stride_page,
                            k_stride_token, k_stride_head, v_stride_page, v_stride_token, v_stride_head,
                            clip_index_k, clip_index_v, w.stage_k, w.stage_v, w.owner, w.kimg, w.vimg, w.rows,
                            w.sink_eff, w.recent, nullptr, nullptr, nullptr, stream);
  }
  if (set_dynamic_lds(reinterpret_cast<const void*>(quant_write_fused_kernel), (int)kFusedLds, g_lds_set) != kOk) return kErrLaunch;
  const int64_t per_block = kFusedWaves * kTokPerWave;
  dim3 grid((unsigned)((num_tokens + per_block - 1) / per_block), (unsigned)(num_kv_heads * 2));
  if (w.rows > 0) {
    hipLaunchKernelGGL(quant_window_winner_kernel, dim3((unsigned)((num_tokens + 255) / 256)), dim3(256), 0, stream,
                       slot_mapping, (int32_t)num_tokens, w.winner, block_size, w.rows);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  hipLaunchKernelGGL(quant_write_fused_kernel, grid, dim3(kFusedWaves * 64), kFusedLds, stream,
                     static_cast<const uint16_t*>(key_bf16), static_cast<const uint16_t*>(value_bf16),
                     num_tokens, token_stride, static_cast<const uint8_t*>(rot_k_operand),
                     static_cast<const uint8_t*>(rot_v_operand), slot_mapping, c,
                     (int)clip_index_k, (int)clip_index_v, w);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace

extern "C" {

int oscar_quant_write(const void* key_bf16, const void* value_bf16, int64_t num_tokens,
                      int32_t num_kv_heads, int32_t head_size, int64_t token_stride,
                      const void* rot_k_operand, const void* rot_v_operand,
                      const int64_t* slot_mapping, void* k_cache, void* v_cache,
                      int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                      int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                      int64_t v_stride_token, int64_t v_stride_head, int32_t clip_index_k,
                      int32_t clip_index_v, hipStream_t stream) {
  return quant_write_impl(key_bf16, value_bf16, num_tokens, num_kv_heads, head_size, token_stride, rot_k_operand,
                          rot_v_operand, slot_mapping, k_cache, v_cache, block_size, num_pages, k_stride_page,
                          k_stride_token, k_stride_head, v_stride_page, v_stride_token, v_stride_head,
                          clip_index_k, clip_index_v, WindowArgs{}, stream);
}

int oscar_quant_write_window(const void* key_bf16, const void* value_bf16, int64_t num_tokens,
                             int32_t num_kv_heads, int32_t head_size, int64_t token_stride,
                             const void* rot_k_operand, const void* rot_v_operand,
                             const int64_t* slot_mapping, void* k_cache, void* v_cache,
                             int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                             int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                             int64_t v_stride_token, int64_t v_stride_head, int32_t clip_index_k,
                             int32_t clip_index_v, const int32_t* query_start_loc, const int32_t* seq_lens,
                             int32_t num_requests, int32_t stage_rows, int32_t sink_eff, int32_t recent,
                             float* stage_k, float* stage_v, int64_t* stage_owner, int64_t* seat_winner,
                             void* stage_k_image, void* stage_v_image, hipStream_t stream) {
  if (num_requests < 0 || stage_rows <= 0 || sink_eff < 0 || recent < 0 || num_tokens > INT32_MAX)
    return kErrInvalidArgument;
  if (num_tokens > 0 && num_requests == 0) return kErrInvalidArgument;
  if (!query_start_loc || !seq_lens || !stage_k || !stage_v || !stage_owner || !seat_winner)
    return kErrInvalidArgument;
  if ((stage_k_image == nullptr) != (stage_v_image == nullptr)) return kErrInvalidArgument;
  if (stage_k_image != nullptr && block_size % 32 != 0) return kErrUnsupportedGeometry;
  if ((reinterpret_cast<uintptr_t>(stage_k) & 15) || (reinterpret_cast<uintptr_t>(stage_v) & 15) ||
      (reinterpret_cast<uintptr_t>(stage_k_image) & 15) || (reinterpret_cast<uintptr_t>(stage_v_image) & 15))
    return kErrInvalidArgument;
  WindowArgs w{query_start_loc, seq_lens, num_requests, stage_rows, sink_eff, recent, num_kv_heads, stage_k, stage_v,
               stage_owner, seat_winner, static_cast<_Float16*>(stage_k_image),
               static_cast<_Float16*>(stage_v_image)};
  return quant_write_impl(key_bf16, value_bf16, num_tokens, num_kv_heads, head_size, token_stride, rot_k_operand,
                          rot_v_operand, slot_mapping, k_cache, v_cache, block_size, num_pages, k_stride_page,
                          k_stride_token, k_stride_head, v_stride_page, v_stride_token, v_stride_head,
                          clip_index_k, clip_index_v, w, stream);
}

}  // extern "C"
