// Prefill continuation: causal attention of N new tokens over C cached INT2
// tokens plus themselves (gfx950, 16-bit MFMA).
//
// Semantics (reference dense path): keys 0 .. C-1 are the dequantized history
// (owner-matched FP32 staging values override INT2), keys C .. C+N-1 are the
// new tokens; new token j (absolute position C + j) sees keys 0 .. C + j.
// MFMA operands are rounded to fp16: the same MFMA rate as bf16 (the
// reference runs this attention in the model's bf16 dtype) with 3 more
// mantissa bits, which keeps softmax-weight rounding below the bf16 output
// tolerance even on x8 outlier channels.  Accumulation and softmax are fp32.
// Rotated domain in, rotated-V domain out (fp32).
//
// One workgroup per 128 consecutive rows of one kv-head, a row being (new
// token j, head-in-group); workgroups of later rows (more keys) are
// dispatched first.  Keys are walked in 32-key blocks through two LDS tile
// buffers, history blocks first, then new-token blocks.  Waves 4-7 produce:
// the raw loads of block i + 2 (codes, meta, owner tags, or the new tokens'
// fp32 values) are in flight while block i + 1's become fp16 K (token-major)
// and V (feature-major) tiles.  Waves 0-3 consume, 32 rows each: S^T = K Q^T
// (16 MFMA 32x32x16, two accumulator chains, Q^T from LDS) and O^T += V^T
// P^T (16 MFMA) with base-2 online softmax and a lazily raised running max.
// One barrier per block hands a buffer from producers to consumers; a
// producer wave and a consumer wave share each SIMD, so dequantization
// overlaps the MFMAs.
#include "oscar_common.h"
#include "../../include/oscar_amd.h"

namespace oscar {
namespace {

constexpr int kBlk = 32;
constexpr int kRowsPerWave = 32;
constexpr int kWaves = 4;
constexpr int kKs = kHeadDim + 8;     // halfs per K row in LDS
constexpr int kVs = kBlk + 4;         // halfs per V feature row in LDS (72 B: 8-byte reads conflict-free)
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.f;          // log2 headroom before a running max is raised
constexpr float kVsMax = 240.f;       // p vs stays below 2^kLazy * 240 < 65504 (fp16) under the lazy max

struct PrefillArgs {
  const float* q;        // [N][Hq][D]
  const float* k_new;    // [N][Hk][D]
  const float* v_new;
  int32_t n_new;
  int32_t num_heads, num_kv_heads, group;
  const uint8_t* k_cache;
  const uint8_t* v_cache;
  int64_t k_page, k_tok, k_head, v_page, v_tok, v_head;
  int32_t block_size;
  FastDiv bs_div;        // block_size
  FastDiv rows_div;      // stage_rows (1 without an arena)
  int64_t num_pages;
  const int32_t* bt;     // one request's block-table row
  int32_t bt_cols;
  int64_t cached;        // C
  const float* stage_k;
  const float* stage_v;
  const int64_t* owner;
  int32_t stage_rows;
  float scale_log2;
  float* out;
};

// Two key blocks of fp16 tiles: block k is computed from one while block
// k + 1 is written into the other.
struct PrefillLds {
  _Float16 kh[2][kBlk * kKs];           // K operand, token-major (features permuted, see below)
  _Float16 vt[2][kHeadDim * kVs];       // V operand, feature-major
  float kpar[2][2][kBlk];               // per key: score = ta * (K'.q) + tb * sum(q)   [ta | tb]
  float vpar[2][2][kBlk];               // per key: v = vs * V' + vz                    [vs | vz]
  uint32_t big[2][4];                   // a key of the block has vs above kVsMax
  _Float16 q[kWaves][16 * 2 * kRowsPerWave * 8];   // Q^T operands [wave][m][g][row][8]
};
constexpr size_t kPrefillLds = sizeof(PrefillLds);
static_assert(kPrefillLds <= 160 * 1024, "LDS of one workgroup");

__device__ __forceinline__ _Float16 to_h(float x) { return (_Float16)x; }

// s_barrier without __syncthreads' memory fence (which would also wait for
// the producers' outstanding global loads); LDS writes are complete at
// lgkmcnt(0).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0); vmcnt and expcnt left at their maxima
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The key blocks a workgroup walks: first the history blocks (keys < C, in
// 32-key blocks from 0), then the new-token blocks (from the block holding
// key C).  A block that straddles C is walked twice, each time with the
// other side's keys masked out.
struct BlockPlan {
  int64_t n_hist;     // history blocks
  int64_t n_new;      // new-token blocks
  int64_t new0;       // first key of the first new-token block
};

__device__ __forceinline__ BlockPlan block_plan(int64_t C, int64_t keys) {
  BlockPlan b;
  b.n_hist = (C + kBlk - 1) / kBlk;
  b.new0 = (C / kBlk) * kBlk;
  b.n_new = keys > C ? (keys - b.new0 + kBlk - 1) / kBlk : 0;
  return b;
}

// Raw loads of one history block for one producer thread: K role (token ktt,
// features 32 kfg .. +31) k = {codes lo, codes hi, meta, owner}; V role
// (tokens 8 vtg + w, features 4 vfg .. +3) v[w] = {code byte, V meta, owner}.
// Every thread issues all 27 loads whatever the block holds (tokens past C
// and invalid pages read an in-bounds slot, masked later), so a wait counts
// exactly one block's loads.
struct HistLoad {
  u32x4 k;
  uint32_t vb[8], vm[8], vo[8];
};

// Raw loads of one new-token block: K role k[i] = fp32 values 32 kfg + 4i ..,
// V role v[w] = fp32 values 4 vfg .. +3 of token 8 vtg + w (16 loads, indices
// clamped into range, masked later).
struct NewLoad {
  floatx4 k[8];
  floatx4 v[8];
};

// Page of the block at key k0 (uniform).  Read through the scalar cache, so
// that waiting for it never waits for the vector loads in flight.
__device__ __forceinline__ int32_t block_page(const PrefillArgs& a, int64_t k0) {
  if (k0 >= a.cached) return -1;
  const uint32_t pidx = fast_div((uint32_t)k0, a.bs_div);       // key positions stay below 2^31
  if ((int64_t)pidx >= a.bt_cols) return -1;
  typedef __attribute__((address_space(4))) const int32_t const_i32;
  return ((const const_i32*)a.bt)[__builtin_amdgcn_readfirstlane(pidx)];
}

__device__ __forceinline__ HistLoad load_hist(const PrefillArgs& a, int64_t k0, int32_t page, int kvh, int ktt,
                                              int kfg, int vtg, int vfg) {
  HistLoad L;
  const bool page_ok = page >= 0 && page < a.num_pages;
  const int64_t pg = page_ok ? page : 0;
  const uint8_t* kpage = a.k_cache + pg * a.k_page + (int64_t)kvh * a.k_head;
  const uint8_t* vpage = a.v_cache + pg * a.v_page + (int64_t)kvh * a.v_head;
  // Owner tags are pages (< 2^31) or -1: the low word of the little-endian
  // int64 identifies them.  Without an arena the K slot's meta stands in.
  const int32_t* opage = a.stage_rows > 0 ? reinterpret_cast<const int32_t*>(
                                                a.owner + (int64_t)fast_mod((uint32_t)pg, a.rows_div) *
                                                              a.block_size)
                                          : reinterpret_cast<const int32_t*>(kpage);
  const int ostride = a.stage_rows > 0 ? 2 : 0;
  const int prow0 = (int)fast_mod((uint32_t)k0, a.bs_div);
  const uint32_t ktok = (uint32_t)a.k_tok, vtok = (uint32_t)a.v_tok;
  {
    const int row = prow0 + ktt;
    const uint8_t* ks = kpage + (uint32_t)row * ktok;
    const u32x2 cw = *reinterpret_cast<const u32x2*>(ks + kKCodeOff + 8 * kfg);
    L.k[0] = cw[0];
    L.k[1] = cw[1];
    L.k[2] = *reinterpret_cast<const uint32_t*>(ks);
    L.k[3] = (uint32_t)opage[ostride * row];
  }
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const int row = prow0 + 8 * vtg + w;
    L.vb[w] = vpage[(uint32_t)row * vtok + vfg];
    L.vm[w] = *reinterpret_cast<const uint32_t*>(kpage + (uint32_t)row * ktok + 4);
    L.vo[w] = (uint32_t)opage[ostride * row];
  }
  return L;
}

__device__ __forceinline__ NewLoad load_new(const PrefillArgs& a, int64_t k0, int kvh, int ktt, int kfg, int vtg,
                                            int vfg) {
  NewLoad L;
  const int64_t C = a.cached, N = a.n_new;
  const int64_t hs = (int64_t)a.num_kv_heads * kHeadDim;
  {
    const int64_t j = min(max(k0 + ktt - C, (int64_t)0), N - 1);
    const floatx4* src = reinterpret_cast<const floatx4*>(a.k_new + j * hs + kvh * kHeadDim + 32 * kfg);
#pragma unroll
    for (int i = 0; i < 8; ++i) L.k[i] = src[i];
  }
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const int64_t j = min(max(k0 + 8 * vtg + w - C, (int64_t)0), N - 1);
    L.v[w] = *reinterpret_cast<const floatx4*>(a.v_new + j * hs + kvh * kHeadDim + 4 * vfg);
  }
  return L;
}

// fp16 pair (1 + c/4) of the codes at bits [sh, sh + 2) and [sh + 16, sh + 18)
// of w (exact: 1, 1.25, 1.5, 1.75).
__device__ __forceinline__ uint32_t magic_pair(uint32_t w, int sh) {
  const uint32_t x = sh < 8 ? (w << (8 - sh)) : (w >> (sh - 8));
  return (x & 0x03000300u) | 0x3C003C00u;
}

// K tile rows hold each 16-feature group in the order 0, 8, 1, 9, .., 7, 15
// (position p is feature (p >> 1) + 8 (p & 1)), so that one shift and mask of
// a code dword yields a pair; the Q^T operand uses the same order.
__device__ __forceinline__ int k_feature(int p) { return (p >> 1) + 8 * (p & 1); }

// 16-byte chunk q8 (0..3) of feature group kfg sits at position
// (q8 + kfg / 2) mod 4 of the group's 64 bytes: the eight threads that write
// one row store chunk q8 into eight different bank groups at once (unrotated,
// the eight stores fell into two bank groups; measured C4 2.18 -> 2.08 ms).
__device__ __forceinline__ int k_chunk_slot(int q8, int kfg) { return (q8 + (kfg >> 1)) & 3; }

// A thread's 32 K values (features 32 kfg .. +31, natural order) into its
// token's row in the permuted order.
__device__ __forceinline__ void store_k_values(const float (&kv)[32], int ktt, int kfg, _Float16* kh) {
  half8* dst = reinterpret_cast<half8*>(kh + ktt * kKs + 32 * kfg);
#pragma unroll
  for (int q8 = 0; q8 < 4; ++q8) {
    half8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = to_h(kv[16 * (q8 >> 1) + k_feature(8 * (q8 & 1) + e)]);
    dst[k_chunk_slot(q8, kfg)] = x;
  }
}

// A thread's V values vv[u][w] (feature 4 vfg + u, token 8 vtg + w).
__device__ __forceinline__ void store_v_values(const float (&vv)[4][8], int vtg, int vfg, _Float16* vt) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    half4 lo, hi;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      lo[w] = to_h(vv[u][w]);
      hi[w] = to_h(vv[u][4 + w]);
    }
    half4* d = reinterpret_cast<half4*>(vt + (4 * vfg + u) * kVs + 8 * vtg);
    d[0] = lo;
    d[1] = hi;
  }
}

// History tiles as code operands: K' = V' = 1 + c/4 (exact in fp16) with the
// token's scale and zero moved into per-key parameters: k = 4s K' + (z - 4s),
// so a score is ta (K'.q) + tb sum(q) with ta = 4 s_k, tb = z_k - 4 s_k (times
// the softmax scale), and v = vs V' + vz with vs = 4 s_v, vz = z_v - 4 s_v.
// Tokens the staging arena owns (rare: the sink / recent window) keep their
// FP32 values (rounded to fp16) with ta = scale, tb = 0, vs = 1, vz = 0.  Keys
// past C or on an unmapped page get all-zero parameters (an unmapped page
// reads as zeros; keys past C are masked by the consumer).
__device__ __forceinline__ void store_hist(const PrefillArgs& a, const HistLoad& L, int64_t k0, int32_t page,
                                           int kvh, int ktt, int kfg, int vtg, int vfg, _Float16* kh,
                                           _Float16* vt, float (&kpar)[2][kBlk], float (&vpar)[2][kBlk],
                                           uint32_t* big) {
  const bool page_ok = page >= 0 && page < a.num_pages;
  const bool arena = a.stage_rows > 0 && page_ok;
  const int64_t seat0 = arena ? (int64_t)fast_mod((uint32_t)page, a.rows_div) * a.block_size : 0;
  const int prow0 = (int)fast_mod((uint32_t)k0, a.bs_div);
  const int64_t C = a.cached;
  {
    const bool live = page_ok && k0 + ktt < C;
    const bool win = arena && live && (int32_t)L.k[3] == page;
    if (!win) {
      half8* dst = reinterpret_cast<half8*>(kh + ktt * kKs + 32 * kfg);
#pragma unroll
      for (int q8 = 0; q8 < 4; ++q8) {
        const uint32_t w = L.k[q8 >> 1];
        const int j0 = 4 * (q8 & 1);
        dst[k_chunk_slot(q8, kfg)] = __builtin_bit_cast(
            half8, u32x4{magic_pair(w, 2 * j0), magic_pair(w, 2 * j0 + 2), magic_pair(w, 2 * j0 + 4),
                         magic_pair(w, 2 * j0 + 6)});
      }
    } else {
      const floatx4* src = reinterpret_cast<const floatx4*>(
          a.stage_k + ((seat0 + prow0 + ktt) * a.num_kv_heads + kvh) * kHeadDim + 32 * kfg);
      float kv[32];
#pragma unroll
      for (int q4 = 0; q4 < 8; ++q4) {
        const floatx4 x = src[q4];
#pragma unroll
        for (int e = 0; e < 4; ++e) kv[4 * q4 + e] = x[e];
      }
      store_k_values(kv, ktt, kfg, kh);
    }
    if (kfg == 0) {
      const float sc = f16_bits_to_f32(L.k[2]), zr = f16_bits_to_f32(L.k[2] >> 16);
      kpar[0][ktt] = win ? a.scale_log2 : (live ? 4.f * sc * a.scale_log2 : 0.f);
      kpar[1][ktt] = (win || !live) ? 0.f : (zr - 4.f * sc) * a.scale_log2;
    }
  }
  {
    uint32_t winmask = 0u, livemask = 0u;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const bool live = page_ok && k0 + 8 * vtg + w < C;
      livemask |= live ? 1u << w : 0u;
      winmask |= (arena && live && (int32_t)L.vo[w] == page) ? 1u << w : 0u;
    }
    if (winmask == 0u) {
      // Code bytes of tokens 8 vtg + 0..3 and + 4..7; per feature u the codes
      // at bits 2u of each byte become fp16 pairs (1 + c/4) of two tokens.
      const uint32_t b0 = L.vb[0] | (L.vb[1] << 8) | (L.vb[2] << 16) | (L.vb[3] << 24);
      const uint32_t b1 = L.vb[4] | (L.vb[5] << 8) | (L.vb[6] << 16) | (L.vb[7] << 24);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t y0 = ((b0 >> (2 * u)) & 0x03030303u) | 0x3C3C3C3Cu;
        const uint32_t y1 = ((b1 >> (2 * u)) & 0x03030303u) | 0x3C3C3C3Cu;
        // bytes {0, y.b0, 0, y.b1} and {0, y.b2, 0, y.b3}
        const u32x2 lo{__builtin_amdgcn_perm(0u, y0, 0x010C000Cu), __builtin_amdgcn_perm(0u, y0, 0x030C020Cu)};
        const u32x2 hi{__builtin_amdgcn_perm(0u, y1, 0x010C000Cu), __builtin_amdgcn_perm(0u, y1, 0x030C020Cu)};
        u32x2* d = reinterpret_cast<u32x2*>(vt + (4 * vfg + u) * kVs + 8 * vtg);
        d[0] = lo;
        d[1] = hi;
      }
    } else {
      float vv[4][8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
#pragma unroll
        for (int u = 0; u < 4; ++u) vv[u][w] = 1.f + 0.25f * (float)((L.vb[w] >> (2 * u)) & 3u);
        if ((winmask >> w) & 1u) {
          const floatx4 y = *reinterpret_cast<const floatx4*>(
              a.stage_v + ((seat0 + prow0 + 8 * vtg + w) * a.num_kv_heads + kvh) * kHeadDim + 4 * vfg);
#pragma unroll
          for (int u = 0; u < 4; ++u) vv[u][w] = y[u];
        }
      }
      store_v_values(vv, vtg, vfg, vt);
    }
    if (vfg == 0) {
      bool bg = false;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const float sc = f16_bits_to_f32(L.vm[w]), zr = f16_bits_to_f32(L.vm[w] >> 16);
        const bool live = (livemask >> w) & 1u, win = (winmask >> w) & 1u;
        vpar[0][8 * vtg + w] = win ? 1.f : (live ? 4.f * sc : 0.f);
        vpar[1][8 * vtg + w] = (win || !live) ? 0.f : zr - 4.f * sc;
        bg = bg || (live && !win && 4.f * sc > kVsMax);
      }
      big[vtg] = bg ? 1u : 0u;
    }
  }
}

// New-token tiles: the fp32 values rounded to fp16, ta = scale, tb = 0,
// vs = 1, vz = 0.
__device__ __forceinline__ void store_new(const PrefillArgs& a, const NewLoad& L, int ktt, int kfg, int vtg, int vfg,
                                          _Float16* kh, _Float16* vt, float (&kpar)[2][kBlk],
                                          float (&vpar)[2][kBlk], uint32_t* big) {
  float kv[32];
  float vv[4][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) kv[4 * i + e] = L.k[i][e];
#pragma unroll
  for (int w = 0; w < 8; ++w)
#pragma unroll
    for (int u = 0; u < 4; ++u) vv[u][w] = L.v[w][u];
  store_k_values(kv, ktt, kfg, kh);
  store_v_values(vv, vtg, vfg, vt);
  if (kfg == 0) {
    kpar[0][ktt] = a.scale_log2;
    kpar[1][ktt] = 0.f;
  }
  if (vfg == 0) {
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      vpar[0][8 * vtg + w] = 1.f;
      vpar[1][8 * vtg + w] = 0.f;
    }
    big[vtg] = 0u;
  }
}

// 8 wavefronts: waves 0-3 compute (32 rows each), waves 4-7 produce the
// fp16 tiles of the next key block, two blocks of loads ahead.
__global__ __launch_bounds__(512, 1) void prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  PrefillLds& S = *reinterpret_cast<PrefillLds*>(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool producer = wave >= kWaves;
  const int g = lane >> 5;
  const int col = lane & 31;
  const int kvh = blockIdx.y;
  const int64_t rows_total = (int64_t)a.n_new * a.group;
  // Blocks of later rows see more keys: they are dispatched first.
  const int64_t row0 = (int64_t)(gridDim.x - 1 - blockIdx.x) * (kWaves * kRowsPerWave);
  const int64_t C = a.cached;
  const int64_t last_row = min(row0 + kWaves * kRowsPerWave, rows_total) - 1;
  const int64_t keys_blk = C + last_row / a.group + 1;
  const BlockPlan plan = block_plan(C, keys_blk);
  const int64_t nblk = plan.n_hist + plan.n_new;
  auto block_k0 = [&](int64_t i) { return i < plan.n_hist ? i * kBlk : plan.new0 + (i - plan.n_hist) * kBlk; };

  if (producer) {
    const int ptid = tid - kWaves * 64;
    const int ktt = ptid >> 3, kfg = ptid & 7;       // K: token ktt, features 32*kfg .. +31
    const int vtg = ptid >> 6, vfg = ptid & 63;      // V: tokens 8*vtg .. +7, features 4*vfg .. +3
    // History pass: loads of block i + 2 out while block i + 1's are turned
    // into tiles; then the same for the new-token pass.  The loop is unrolled
    // twice so that the two load sets alternate in place: a load never lands
    // in registers that still have to be copied, and each wait counts one
    // block's loads.
    const int64_t nh = plan.n_hist;
    int64_t i = 0;
    if (nh > 0) {
      int32_t pg_a = block_page(a, 0), pg_b = block_page(a, kBlk);
      HistLoad La = load_hist(a, 0, pg_a, kvh, ktt, kfg, vtg, vfg);
      HistLoad Lb = load_hist(a, kBlk, pg_b, kvh, ktt, kfg, vtg, vfg);
      int32_t pg_c = block_page(a, 2 * kBlk);
      // top of the loop: La holds block i (page pg_a), Lb block i + 1 (pg_b),
      // pg_c is block i + 2's page
#pragma unroll 1
      for (;;) {
        store_hist(a, La, i * kBlk, pg_a, kvh, ktt, kfg, vtg, vfg, S.kh[i & 1], S.vt[i & 1], S.kpar[i & 1],
                   S.vpar[i & 1], S.big[i & 1]);
        const int32_t pg_d = block_page(a, (i + 3) * kBlk);
        La = load_hist(a, (i + 2) * kBlk, pg_c, kvh, ktt, kfg, vtg, vfg);
        pg_a = pg_c;
        lds_barrier();        // tiles of block i ready / block i - 1 consumed
        if (++i == nh) break;
        store_hist(a, Lb, i * kBlk, pg_b, kvh, ktt, kfg, vtg, vfg, S.kh[i & 1], S.vt[i & 1], S.kpar[i & 1],
                   S.vpar[i & 1], S.big[i & 1]);
        pg_c = block_page(a, (i + 3) * kBlk);
        Lb = load_hist(a, (i + 2) * kBlk, pg_d, kvh, ktt, kfg, vtg, vfg);
        pg_b = pg_d;
        lds_barrier();
        if (++i == nh) break;
      }
    }
    if (plan.n_new > 0) {
      NewLoad La = load_new(a, plan.new0, kvh, ktt, kfg, vtg, vfg);
      NewLoad Lb = load_new(a, plan.new0 + kBlk, kvh, ktt, kfg, vtg, vfg);
#pragma unroll 1
      for (;;) {
        store_new(a, La, ktt, kfg, vtg, vfg, S.kh[i & 1], S.vt[i & 1], S.kpar[i & 1], S.vpar[i & 1],
                  S.big[i & 1]);
        La = load_new(a, block_k0(i) + 2 * kBlk, kvh, ktt, kfg, vtg, vfg);
        lds_barrier();
        if (++i == nblk) break;
        store_new(a, Lb, ktt, kfg, vtg, vfg, S.kh[i & 1], S.vt[i & 1], S.kpar[i & 1], S.vpar[i & 1],
                  S.big[i & 1]);
        Lb = load_new(a, block_k0(i) + 2 * kBlk, kvh, ktt, kfg, vtg, vfg);
        lds_barrier();
        if (++i == nblk) break;
      }
    }
    lds_barrier();            // the consumers' last block
    return;
  }

  // ---- consumers: 32 rows per wave ----
  const int64_t wrow0 = row0 + wave * kRowsPerWave;
  const int64_t row = wrow0 + col;
  const bool row_ok = row < rows_total;
  const int64_t wave_last = min(wrow0 + kRowsPerWave, rows_total) - 1;
  const int64_t keys_wave = wrow0 < rows_total ? C + wave_last / a.group + 1 : 0;
  const int64_t my_limit = row_ok ? C + row / a.group : -1;   // last visible key
  // Keys every row of the wave sees (all rows in range): history keys
  // 0 .. C - 1 in the history pass, C .. C + wrow0 / group in the new pass.
  const bool wave_full = wrow0 + kRowsPerWave <= rows_total;
  const int32_t full_hi_new = (int32_t)(C + wrow0 / a.group);
  auto lo_wave = [&](bool hist) { return hist ? 0 : (int32_t)C; };
  auto hi_wave = [&](bool hist) {
    return wave_full ? (hist ? (int32_t)C - 1 : full_hi_new) : (int32_t)-1;
  };
  // Offsets (halves) of a K operand chunk for this lane's g: + 8g, or - 24g
  // where the rotated slot wraps from 3 to 0.
  const int kstep = 8 * g, kwrap = -24 * g;
  float qsum;
  {
    // Q^T operands of the wave's rows in the K tiles' feature order: lane
    // (row col, half g) holds positions 8g .. 8g + 7 of k-step m, i.e.
    // features 16m + 4g + {0, 8, 1, 9, 2, 10, 3, 11}.  qsum: the row's sum of
    // the fp16 values.
    const int64_t j = row_ok ? row / a.group : 0;
    const int h = kvh * a.group + (row_ok ? (int)(row % a.group) : 0);
    const float* qp = a.q + (j * a.num_heads + h) * kHeadDim + 4 * g;
    _Float16* qdst = S.q[wave] + (g * kRowsPerWave + col) * 8;
    float qs = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const floatx4 x0 = row_ok ? *reinterpret_cast<const floatx4*>(qp + 16 * m) : floatx4{};
      const floatx4 x1 = row_ok ? *reinterpret_cast<const floatx4*>(qp + 16 * m + 8) : floatx4{};
      const half8 v = half8{to_h(x0[0]), to_h(x1[0]), to_h(x0[1]), to_h(x1[1]),
                            to_h(x0[2]), to_h(x1[2]), to_h(x0[3]), to_h(x1[3])};
#pragma unroll
      for (int e = 0; e < 8; ++e) qs += (float)v[e];
      *reinterpret_cast<half8*>(qdst + m * 2 * kRowsPerWave * 8) = v;
    }
    qsum = qs + shfl_xor_f32(qs, 32);
  }
  wave_sync_lds();

  floatx16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx16{};
  float m_run = -__builtin_inff();
  float l_run = 0.f, z_run = 0.f;     // this lane's keys' sums of p and p vz

#pragma unroll 1
  for (int64_t i = 0; i < nblk; ++i) {
    lds_barrier();            // tiles of block i ready
    const int64_t k0 = block_k0(i);
    const bool hist = i < plan.n_hist;
    if (k0 < keys_wave) {
      const _Float16* kh = S.kh[i & 1];
      const _Float16* vt = S.vt[i & 1];
      const _Float16* krow = kh + col * kKs;
      const half8* qsrc = reinterpret_cast<const half8*>(S.q[wave] + (g * kRowsPerWave + col) * 8);
      // K operand of k-step m: chunk 2m + g of the row (feature group m / 2,
      // chunk 2 (m % 2) + g), at its rotated slot; the lane's g enters as one
      // of two per-lane offsets (with or without the wrap of the slot).
      auto kchunk = [&](int m) {
        const int c0 = (2 * (m & 1) + (m >> 2)) & 3;          // slot for g = 0
        return *reinterpret_cast<const half8*>(krow + 8 * (4 * (m >> 1) + c0) + (c0 == 3 ? kwrap : kstep));
      };
      floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
      for (int m = 0; m < 16; m += 2) {
        const half8 ka = kchunk(m);
        const half8 kb2 = kchunk(m + 1);
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qsrc[m * 2 * kRowsPerWave], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb2, qsrc[(m + 1) * 2 * kRowsPerWave], s1, 0, 0, 0);
      }
      floatx16 s = s0 + s1;
      // Visible keys of this pass: history keys < C in the history pass, new
      // keys >= C in the new-token pass, causal for both.  A block every row
      // of the wave sees whole skips the per-key test.
      const int32_t lo = hist ? 0 : (int32_t)C;
      const int32_t hi = hist ? (int32_t)min(C - 1, my_limit) : (int32_t)my_limit;
      const bool whole = (int32_t)k0 >= lo_wave(hist) && (int32_t)k0 + kBlk - 1 <= hi_wave(hist);
      // key 8 jj + 4g + i of the block is register 4 jj + i
      const float* kpar0 = S.kpar[i & 1][0] + 4 * g;
      const float* kpar1 = S.kpar[i & 1][1] + 4 * g;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const floatx4 ta = *reinterpret_cast<const floatx4*>(kpar0 + 8 * jj);
        const floatx4 tb = *reinterpret_cast<const floatx4*>(kpar1 + 8 * jj);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * jj + e] = fmaf(ta[e], s[4 * jj + e], tb[e] * qsum);
      }
      float mb = -__builtin_inff();
      if (whole) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mb = fmaxf(mb, s[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int32_t kp = (int32_t)k0 + 8 * (r >> 2) + 4 * g + (r & 3);
          const float x = (kp >= lo && kp <= hi) ? s[r] : -__builtin_inff();
          s[r] = x;
          mb = fmaxf(mb, x);
        }
      }
      mb = fmaxf(mb, shfl_xor_f32(mb, 32));
      // Lazy running max: raised only when a block exceeds it by more than
      // 2^kLazy (p vs stays in fp16 range), or by any amount when a key of the
      // block has vs above kVsMax; the first raise of a row needs no rescale.
      const uint4 bg4 = *reinterpret_cast<const uint4*>(S.big[i & 1]);
      const bool eager = (bg4[0] | bg4[1] | bg4[2] | bg4[3]) != 0u;
      const bool need = mb > m_run + (eager ? 0.f : kLazy);
      const bool resc = need && m_run != -__builtin_inff();
      if (__ballot(resc)) {
        const float alpha = resc ? __builtin_amdgcn_exp2f(m_run - mb) : 1.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] *= alpha;
        l_run *= alpha;
        z_run *= alpha;
      }
      if (need) m_run = mb;
      // exp2(-inf - m) = 0 needs a finite m: rows that have seen no key yet use 0.
      const float m_use = m_run == -__builtin_inff() ? 0.f : m_run;
      float psum = 0.f, zsum = 0.f;
      half8 pb[2];
      const float* vpar0 = S.vpar[i & 1][0] + 4 * g;
      const float* vpar1 = S.vpar[i & 1][1] + 4 * g;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const floatx4 vs = *reinterpret_cast<const floatx4*>(vpar0 + 8 * jj);
        const floatx4 vz = *reinterpret_cast<const floatx4*>(vpar1 + 8 * jj);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * jj + e;
          const float p = __builtin_amdgcn_exp2f(s[r] - m_use);
          psum += p;
          zsum = fmaf(p, vz[e], zsum);
          pb[r >> 3][r & 7] = to_h(p * vs[e]);
        }
      }
      l_run += psum;
      z_run += zsum;
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const _Float16* vrow = vt + (32 * t + col) * kVs + 16 * mm + 4 * g;
          const u32x2 lo2 = *reinterpret_cast<const u32x2*>(vrow);
          const u32x2 hi2 = *reinterpret_cast<const u32x2*>(vrow + 8);
          const half8 va = __builtin_bit_cast(half8, u32x4{lo2[0], lo2[1], hi2[0], hi2[1]});
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[mm], acc[t], 0, 0, 0);
        }
      }
    }
  }
  lds_barrier();              // pairs with the producers' last barrier

  const float l_tot = l_run + shfl_xor_f32(l_run, 32);
  const float z_tot = z_run + shfl_xor_f32(z_run, 32);
  if (!row_ok) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const int64_t j = row / a.group;
  const int h = kvh * a.group + (int)(row % a.group);
  float* op = a.out + (j * a.num_heads + h) * kHeadDim;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) op[32 * t + 8 * (r >> 2) + 4 * g + (r & 3)] = (acc[t][r] + z_tot) * inv;
  }
}

std::atomic<uint64_t> g_lds_set{0};   // dynamic-LDS attribute set, one bit per device

}  // namespace
}  // namespace oscar

using namespace oscar;

extern "C" int oscar_prefill_continuation(
    const float* q_rot, const float* k_new, const float* v_new, int32_t num_new, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_size, const void* k_cache, const void* v_cache,
    int32_t block_size, int64_t num_pages, int64_t k_stride_page, int64_t k_stride_token,
    int64_t k_stride_head, int64_t v_stride_page, int64_t v_stride_token, int64_t v_stride_head,
    const int32_t* block_table_row, int32_t block_table_cols, int64_t cached_len,
    const float* stage_k, const float* stage_v, const int64_t* stage_owner, int32_t stage_rows,
    float scale, float* out, hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_new < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads ||
      block_size <= 0 || num_pages <= 0 || cached_len < 0 || stage_rows < 0 || block_table_cols < 0)
    return kErrInvalidArgument;
  if (num_new == 0) return kOk;
  // key positions and rows are handled in 32 bits inside the kernel
  if (cached_len + num_new >= ((int64_t)1 << 31) || (int64_t)num_new * num_heads >= ((int64_t)1 << 31))
    return kErrInvalidArgument;
  if (!q_rot || !k_new || !v_new || !k_cache || !v_cache || !out) return kErrInvalidArgument;
  if (cached_len > 0 && (!block_table_row || (cached_len + block_size - 1) / block_size > block_table_cols))
    return kErrInvalidArgument;
  if (stage_rows > 0 && (!stage_k || !stage_v || !stage_owner)) return kErrInvalidArgument;
  if (k_stride_head < kKCodeOff + kCodeBytes || v_stride_head < kCodeBytes || (k_stride_head & 7) ||
      (k_stride_token & 7) || (k_stride_page & 7) || block_size % kBlk != 0)
    return kErrUnsupportedGeometry;
  PrefillArgs a{};
  a.q = q_rot;
  a.k_new = k_new;
  a.v_new = v_new;
  a.n_new = num_new;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_heads / num_kv_heads;
  a.k_cache = static_cast<const uint8_t*>(k_cache);
  a.v_cache = static_cast<const uint8_t*>(v_cache);
  a.k_page = k_stride_page;
  a.k_tok = k_stride_token;
  a.k_head = k_stride_head;
  a.v_page = v_stride_page;
  a.v_tok = v_stride_token;
  a.v_head = v_stride_head;
  a.block_size = block_size;
  a.bs_div = make_fast_div((uint32_t)block_size);
  a.rows_div = make_fast_div(stage_rows > 0 ? (uint32_t)stage_rows : 1u);
  a.num_pages = num_pages;
  a.bt = block_table_row;
  a.bt_cols = block_table_cols;
  a.cached = cached_len;
  a.stage_k = stage_k;
  a.stage_v = stage_v;
  a.owner = stage_owner;
  a.stage_rows = stage_rows;
  a.scale_log2 = scale * kLog2e;
  a.out = out;
  const int64_t rows = (int64_t)num_new * a.group;
  dim3 grid((unsigned)((rows + kWaves * kRowsPerWave - 1) / (kWaves * kRowsPerWave)), (unsigned)num_kv_heads);
  if (set_dynamic_lds(reinterpret_cast<const void*>(prefill_kernel), (int)kPrefillLds, g_lds_set) != kOk) return kErrLaunch;
  hipLaunchKernelGGL(prefill_kernel, grid, dim3(2 * kWaves * 64), kPrefillLds, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
