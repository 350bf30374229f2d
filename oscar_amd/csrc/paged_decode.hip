// Paged MTP decode attention over INT2 history + FP32 window (gfx950).
//
// Semantics (per request i with query rows [a, b), n = b - a, prefix =
// seq_i - n): query token j attends to history positions 0 .. prefix-1 and to
// the request's own new tokens 0 .. j.  History position p lives in page
// bt[i][p / bs], row p % bs; it is read from the staging arena when the arena
// seat (page % rows, row) is owned by that page, otherwise it is dequantized
// from the INT2 slot.  All inputs are in the rotated domain; the output is in
// the rotated-V domain.
//
// Rows are (query token, head-in-group) pairs of one kv-head's GQA group, 32
// per tile, so each INT2 token is read and unpacked once for all of them.
//
// split kernel: one workgroup (4 wavefronts) per (request, kv-head, split,
//   row tile).  With S splits, split s takes the history's 32-token tiles
//   s, s + S, s + 2S, ... and wave w of it every fourth of those, so the
//   window's tiles (the history's first and last pages) spread over many
//   splits.  Per tile (one page, as block_size % 32 == 0):
//   * S^T = K Q^T on 32x32x16 f16 MFMA.  K operands are the exact fp16 values
//     1 + c/4 built from the code bits (one shift and one and-or per pair);
//     the token's scale s and zero z act on the score tile:
//       q.k = s * sum q c + z * sum q = 4s * (q.k') + (z - 4s) * sum q.
//     The K dimension is permuted (feature 128g + 16j + 4a + i + 8b sits in
//     k-step 2j + a, slot 2i + b) so that pairs come straight out of a code
//     dword; Q^T (fp16, in LDS) uses the same permutation.
//   * O^T += V^T P'^T on 16 more MFMAs with V operands 1 + c/4 from byte-
//     transposed codes in LDS and P' = p * vs (fp16).  Then
//       sum_t p (c vs + vz) = 4 * acc - 4 * sum_t P' + sum_t p vz,
//     where sum_t P' is taken over the same fp16 values (v_dot2).
//   * Tokens owned by the staging arena use its fp16 operand images (K in
//     the MFMA A-operand lane order, V^T likewise), copied into LDS with
//     global_load_lds_dwordx4 only for tiles that hold such tokens; their
//     probabilities enter the PV pass as p / 4.
//   Base-2 online softmax in fp32; a row's running max is only raised when a
//   tile's max exceeds it by more than 2^4 (so P' <= 16 * vs stays finite in
//   fp16; a tile with a V scale above 4094 rescales eagerly).  The 4
//   wavefronts merge in LDS and the workgroup writes (m, l, unnormalised
//   O[row][256]) for its valid rows.
// merge kernel: one 256-thread block per (output row, feature quarter):
//   LSE-combines the split partials with the fresh-token scores (fp32,
//   causal) and writes that slice of the row.
#include "oscar_common.h"

namespace oscar {
namespace {

constexpr int kTile = 32;
constexpr int kWaves = 4;
constexpr int kRows = 32;
constexpr int kMaxFresh = 16;
constexpr int kVtStride = 9;            // dwords per V code byte-row (32 tokens + pad)
constexpr int kImgHalfs = 16 * 64 * 8;  // one staged operand image: 16 blocks x 64 lanes x 8
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 4.f;            // log2 headroom before a running max is raised
constexpr float kLazyVsMax = 4094.f;    // 16 * 4094 < 65504 (fp16 max)

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Requests of one launch travel inside the kernel arguments (no device round
// trip for the metadata); larger batches are launched in chunks.
constexpr int kMaxInlineReqs = 128;

struct ReqInfo {
  int32_t qa;        // first query row (token) of the request
  int32_t nq;        // query rows
  int32_t prefix;    // history length
  int32_t pad;
};

struct DecodeArgs {
  const float* q;          // [n, Hq, D]
  const float* k_new;      // [n, Hk, D]
  const float* v_new;
  const uint8_t* k_cache;
  const uint8_t* v_cache;
  int64_t k_page, k_tok, k_head, v_page, v_tok, v_head;
  int32_t block_size;
  int64_t num_pages;
  const int32_t* block_table;
  int64_t bt_stride;
  int32_t bt_cols;
  int32_t num_tokens;
  int32_t num_heads, num_kv_heads, group;
  const int64_t* owner;         // [rows, bs] or null
  const _Float16* kimg;         // [rows][bs / 32][Hk][kImgHalfs]
  const _Float16* vimg;
  int32_t stage_rows;
  float scale_log2;             // attention scale * log2(e)
  float* out;                   // [n, Hq, D]
  float* ws;                    // partials
  int32_t max_splits, row_tiles;
  ReqInfo reqs[kMaxInlineReqs];
};

struct LdsLayout {
  float scratch[kWaves * kImgHalfs / 2 + 64];     // per-wave staged image / combine buffers
  _Float16 q[16 * 2 * kRows * 8];                 // Q^T operand [m][g][row][8]
  float qsum[kRows];                              // sum of each row's fp16 q
  uint32_t vt[kWaves][64 * kVtStride];            // V codes [byte][token/4]
  float ta[kWaves][kTile];                        // score = ta * (q.k') + tb * qsum
  float tb[kWaves][kTile];
  float tvs[kWaves][kTile];                       // V scale (0: staged / invalid)
  float tvz[kWaves][kTile];                       // V zero
  float mrow[kWaves][kRows];
  float lrow[kWaves][kRows];
};

constexpr size_t kPartialFloats = kRows * kHeadDim + 2 * kRows;

__device__ __forceinline__ int64_t item_index(const DecodeArgs& a, int req, int kvh, int split, int rt) {
  return (((int64_t)req * a.num_kv_heads + kvh) * a.max_splits + split) * a.row_tiles + rt;
}

// fp16 pair (1.0, 1.0) held in a VGPR: gfx950's three-operand and-or takes at
// most one literal/SGPR operand, so the mask goes to an SGPR and this stays a
// register (the opaque move keeps the compiler from folding it back).
__device__ __forceinline__ uint32_t magic_ones() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, 0x3c003c00" : "=v"(m));
  return m;
}

// Codes at bits [sh, sh+2) and [sh+16, sh+18) of w -> fp16 pair (1 + c/4), exact.
__device__ __forceinline__ uint32_t magic_pair(uint32_t w, int sh, uint32_t ones) {
  const uint32_t x = sh < 8 ? (w << (8 - sh)) : (w >> (sh - 8));
  return (x & 0x03000300u) | ones;
}

__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ half8 as_half8(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3) {
  return __builtin_bit_cast(half8, u32x4{d0, d1, d2, d3});
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Copy one staged operand image (16 KB) into this wave's LDS buffer.
__device__ __forceinline__ void image_to_lds(const _Float16* src, _Float16* dst, int lane) {
#pragma unroll
  for (int i = 0; i < 16; ++i)
    __builtin_amdgcn_global_load_lds(src + (i * 64 + lane) * 8, dst + i * 64 * 8, 16, 0, 0);
}

struct TileLoad {
  u32x4 kc0, kc1;     // this lane's 32 K code bytes
  u32x2 meta;         // K scale, K zero, V scale, V zero (fp16 pairs)
  u32x2 vc[4];        // V code bytes 8*bg .. +7 of tokens 4*tq .. +3
  int64_t own;        // owner tag of this lane's token seat (-2: no arena)
  int32_t page;       // -1: tile invalid
  int32_t prow0;
};

// Page of history tile `tile` (-1 when past the block table or out of range).
__device__ __forceinline__ int tile_page(const DecodeArgs& a, const int32_t* bt_row, int tile) {
  const int pidx = tile * kTile / a.block_size;
  if (pidx >= a.bt_cols) return -1;
  const int page = bt_row[pidx];
  return (page < 0 || page >= a.num_pages) ? -1 : page;
}

// Loads of one tile whose page is already known (wave-uniform).
__device__ __forceinline__ TileLoad load_tile(const DecodeArgs& a, int page, int p0, int prefix, int kvh,
                                              int lane) {
  TileLoad L;
  L.page = -1;
  L.prow0 = 0;
  L.own = -2;
  L.kc0 = L.kc1 = u32x4{0u, 0u, 0u, 0u};
  L.meta = u32x2{0u, 0u};
#pragma unroll
  for (int k = 0; k < 4; ++k) L.vc[k] = u32x2{0u, 0u};
  if (p0 >= prefix || page < 0) return L;
  L.page = page;
  L.prow0 = p0 - (p0 / a.block_size) * a.block_size;
  const int t = lane & 31, g = lane >> 5;
  const int tq = lane & 7, bg = lane >> 3;
  const uint8_t* kbase = a.k_cache + (int64_t)page * a.k_page + (int64_t)kvh * a.k_head;
  const uint8_t* vbase = a.v_cache + (int64_t)page * a.v_page + (int64_t)kvh * a.v_head;
  if (p0 + t < prefix) {
    const uint8_t* ks = kbase + (int64_t)(L.prow0 + t) * a.k_tok;
    L.meta = *reinterpret_cast<const u32x2*>(ks);
    L.kc0 = *reinterpret_cast<const u32x4*>(ks + kKCodeOff + 32 * g);
    L.kc1 = *reinterpret_cast<const u32x4*>(ks + kKCodeOff + 32 * g + 16);
    if (a.stage_rows > 0)
      L.own = a.owner[(int64_t)(page % a.stage_rows) * a.block_size + L.prow0 + t];
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int tk = 4 * tq + k;
    if (p0 + tk < prefix)
      L.vc[k] = *reinterpret_cast<const u32x2*>(vbase + (int64_t)(L.prow0 + tk) * a.v_tok + 8 * bg);
  }
  return L;
}

// 4x4 byte transpose: out[b] = {d0.byte b, d1.byte b, d2.byte b, d3.byte b}.
__device__ __forceinline__ void transpose4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3, uint32_t (&o)[4]) {
  const uint32_t lo01 = __builtin_amdgcn_perm(d1, d0, 0x05010400u);
  const uint32_t hi01 = __builtin_amdgcn_perm(d1, d0, 0x07030602u);
  const uint32_t lo23 = __builtin_amdgcn_perm(d3, d2, 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(d3, d2, 0x07030602u);
  o[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// K operands of k-steps m = 2j, 2j + 1 from code dword w (this lane's token).
__device__ __forceinline__ void k_operands(uint32_t w, uint32_t ones, half8 (&ka)[2]) {
#pragma unroll
  for (int aa = 0; aa < 2; ++aa)
    ka[aa] = as_half8(magic_pair(w, 8 * aa, ones), magic_pair(w, 8 * aa + 2, ones),
                      magic_pair(w, 8 * aa + 4, ones), magic_pair(w, 8 * aa + 6, ones));
}

__global__ __launch_bounds__(256) void paged_decode_split_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  LdsLayout& S = *reinterpret_cast<LdsLayout*>(smem_raw);

  const int split = blockIdx.x;
  const int nsplit = gridDim.x;
  const int req = blockIdx.y / a.num_kv_heads;
  const int kvh = blockIdx.y - req * a.num_kv_heads;
  const int rt = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;

  const ReqInfo ri = a.reqs[req];
  const int qa = ri.qa, nq = ri.nq, prefix = ri.prefix;
  if (nq <= 0) return;
  const int tiles = prefix > 0 ? (prefix + kTile - 1) / kTile : 0;
  if (split >= tiles) return;
  const int rows = nq * a.group;
  if (rt * kRows >= rows) return;
  const int32_t* bt_row = a.block_table + (int64_t)req * a.bt_stride;

  // Wave w takes tiles split + nsplit * (w + 4k), k < ntw; lane k holds the
  // page of its k-th tile (one block-table load for all of them).
  const int tstep = nsplit * kWaves;
  const int first = split + nsplit * w;
  const int ntw = first < tiles ? (tiles - 1 - first) / tstep + 1 : 0;
  const int my_page = lane < ntw ? tile_page(a, bt_row, first + tstep * lane) : -1;

  // ---- Q^T operand into LDS (permuted K dimension, fp16) and row sums ----
  // Thread: row tid >> 3, features 32 * (tid & 7) .. +31.  The Q loads, the
  // page loads and then the first tile's loads are all in flight together.
  TileLoad cur;
  {
    const int r = tid >> 3, c = tid & 7;
    const int row = rt * kRows + r;
    floatx4 x[8];
    if (row < rows) {
      const int j = row / a.group, h = kvh * a.group + row % a.group;
      const floatx4* src = reinterpret_cast<const floatx4*>(
          a.q + ((int64_t)(qa + j) * a.num_heads + h) * kHeadDim + 32 * c);
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = src[k];
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = floatx4{};
    }
    cur = load_tile(a, ntw > 0 ? __builtin_amdgcn_readfirstlane(my_page) : -1, first * kTile, prefix, kvh,
                    lane);
    // The thread's 32 features (128gg + 32(c & 3) + k) are exactly the four
    // operand vectors (m = 2jj + a, gg) with jj = 2(c & 3) + jl: slot 2i + b of
    // vector (jl, a) is local feature 16jl + 4a + i + 8b.
    float qs = 0.f;
    const int gg = c >> 2;
#pragma unroll
    for (int jl = 0; jl < 2; ++jl) {
#pragma unroll
      for (int aa = 0; aa < 2; ++aa) {
        half8 v;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int k = 16 * jl + 4 * aa + (u >> 1) + 8 * (u & 1);
          v[u] = (_Float16)x[k >> 2][k & 3];
          qs += (float)v[u];
        }
        const int m = 2 * (2 * (c & 3) + jl) + aa;
        *reinterpret_cast<half8*>(&S.q[((m * 2 + gg) * kRows + r) * 8]) = v;
      }
    }
    qs += shfl_xor_f32(qs, 1);
    qs += shfl_xor_f32(qs, 2);
    qs += shfl_xor_f32(qs, 4);
    if (c == 0) S.qsum[r] = qs;
  }
  __syncthreads();

  floatx16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx16{};
  float m_run = -__builtin_inff(), l_run = 0.f, z_run = 0.f, ps_run = 0.f;
  const float qsum = S.qsum[col];
  const int tq = lane & 7, bg = lane >> 3;
  _Float16* ibuf = reinterpret_cast<_Float16*>(S.scratch) + w * kImgHalfs;
  const int tiles_per_page = a.block_size / kTile;
  const half2v ones{(_Float16)1.f, (_Float16)1.f};
  const uint32_t ones16 = magic_ones();

#pragma unroll 1
  for (int k = 0; k < ntw; ++k) {
    const int ti = first + tstep * k;
    const int p0 = ti * kTile;
    const TileLoad L = cur;
    if (k + 1 < ntw)
      cur = load_tile(a, __builtin_amdgcn_readlane(my_page, k + 1), (ti + tstep) * kTile, prefix, kvh, lane);

    const int nvalid = L.page >= 0 ? min(kTile, prefix - p0) : 0;
    const bool tok_ok = col < nvalid;
    const bool staged = tok_ok && L.own == (int64_t)L.page;
    const uint32_t smask = (uint32_t)__ballot(staged && g == 0);
    const _Float16* kimg_src = nullptr;
    const _Float16* vimg_src = nullptr;
    if (smask) {
      const int64_t img = ((int64_t)(L.page % a.stage_rows) * tiles_per_page + L.prow0 / kTile) *
                          a.num_kv_heads + kvh;
      kimg_src = a.kimg + img * kImgHalfs;
      vimg_src = a.vimg + img * kImgHalfs;
      image_to_lds(kimg_src, ibuf, lane);
    }

    // ---- V codes -> LDS [byte][token], per-token score/V parameters ----
    float vsc = 0.f;
    {
      uint32_t o0[4], o1[4];
      transpose4(L.vc[0][0], L.vc[1][0], L.vc[2][0], L.vc[3][0], o0);
      transpose4(L.vc[0][1], L.vc[1][1], L.vc[2][1], L.vc[3][1], o1);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        S.vt[w][(8 * bg + k) * kVtStride + tq] = o0[k];
        S.vt[w][(8 * bg + 4 + k) * kVtStride + tq] = o1[k];
      }
      if (g == 0) {
        float av = 0.f, bv = 0.f, vzv = 0.f;
        if (staged) {
          av = a.scale_log2;
        } else if (tok_ok) {
          const float ks = f16_bits_to_f32(L.meta[0]);
          const float kz = f16_bits_to_f32(L.meta[0] >> 16);
          av = 4.f * ks * a.scale_log2;
          bv = (kz - 4.f * ks) * a.scale_log2;
          vsc = f16_bits_to_f32(L.meta[1]);
          vzv = f16_bits_to_f32(L.meta[1] >> 16);
        }
        S.ta[w][col] = av;
        S.tb[w][col] = bv;
        S.tvs[w][col] = vsc;
        S.tvz[w][col] = vzv;
      }
    }
    const bool vs_big = __ballot(vsc > kLazyVsMax) != 0;
    if (smask) wait_vmem();
    wave_sync_lds();

    // ---- S^T = K' Q^T ----
    const uint32_t kw[8] = {L.kc0[0], L.kc0[1], L.kc0[2], L.kc0[3], L.kc1[0], L.kc1[1], L.kc1[2], L.kc1[3]};
    floatx16 s = floatx16{};
    if (!smask) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        half8 ka[2];
        k_operands(kw[j], ones16, ka);
#pragma unroll
        for (int aa = 0; aa < 2; ++aa) {
          const int m = 2 * j + aa;
          const half8 qb = *reinterpret_cast<const half8*>(&S.q[((m * 2 + g) * kRows + col) * 8]);
          s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[aa], qb, s, 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        half8 ka[2];
        k_operands(kw[j], ones16, ka);
        if (staged) {
#pragma unroll
          for (int aa = 0; aa < 2; ++aa)
            ka[aa] = *reinterpret_cast<const half8*>(ibuf + ((2 * j + aa) * 64 + lane) * 8);
        }
#pragma unroll
        for (int aa = 0; aa < 2; ++aa) {
          const int m = 2 * j + aa;
          const half8 qb = *reinterpret_cast<const half8*>(&S.q[((m * 2 + g) * kRows + col) * 8]);
          s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[aa], qb, s, 0, 0, 0);
        }
      }
      // The K image has been read; bring in the V image while the softmax runs.
      wave_sync_lds();
      image_to_lds(vimg_src, ibuf, lane);
    }

    // ---- scores and lazy online softmax (lane: row `col`, tokens 8*(r/4) + 4*g + r%4) ----
    float mb = -__builtin_inff();
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const floatx4 av = *reinterpret_cast<const floatx4*>(&S.ta[w][8 * jj + 4 * g]);
      const floatx4 bv = *reinterpret_cast<const floatx4*>(&S.tb[w][8 * jj + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[4 * jj + i] = fmaf(av[i], s[4 * jj + i], bv[i] * qsum);
    }
    if (nvalid < kTile) {          // partial tile (uniform): mask tokens past the history
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + 4 * g + (r & 3) >= nvalid) s[r] = -__builtin_inff();
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) mb = fmaxf(mb, s[r]);
    mb = fmaxf(mb, shfl_xor_f32(mb, 32));
    const bool need = mb > m_run + (vs_big ? 0.f : kLazy);
    if (__ballot(need)) {
      const float alpha = !need ? 1.f : (m_run == -__builtin_inff() ? 0.f : exp2_raw(m_run - mb));
      if (need) m_run = mb;
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] *= alpha;
      l_run *= alpha;
      z_run *= alpha;
      ps_run *= alpha;
    }
    float pv[16];
    half8 pb[2];
    float psum = 0.f, zsum = 0.f;
    // exp2(-inf - m) = 0 needs a finite m: rows that have seen no key yet use 0.
    const float m_use = m_run == -__builtin_inff() ? 0.f : m_run;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const floatx4 vsv = *reinterpret_cast<const floatx4*>(&S.tvs[w][8 * jj + 4 * g]);
      const floatx4 vze = *reinterpret_cast<const floatx4*>(&S.tvz[w][8 * jj + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * jj + i;
        const float p = exp2_raw(s[r] - m_use);
        psum += p;
        zsum = fmaf(p, vze[i], zsum);
        pv[r] = p;
        s[r] = p * vsv[i];          // P' (scale folded)
      }
    }
    // slot u <-> tokens (t0, t2, t1, t3, t4, t6, t5, t7) of each 8-token group
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int r0 = 8 * mm;
      pb[mm] = half8{(_Float16)s[r0 + 0], (_Float16)s[r0 + 2], (_Float16)s[r0 + 1], (_Float16)s[r0 + 3],
                     (_Float16)s[r0 + 4], (_Float16)s[r0 + 6], (_Float16)s[r0 + 5], (_Float16)s[r0 + 7]};
      float pss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pss = __builtin_amdgcn_fdot2(half2v{pb[mm][2 * e], pb[mm][2 * e + 1]}, ones, pss, false);
      ps_run += pss;
    }
    l_run += psum;
    z_run += zsum;

    // ---- O^T += V'^T P'^T ----
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t* vrow = &S.vt[w][(32 * h + col) * kVtStride];
        const uint32_t d0 = vrow[4 * mm + g];
        const uint32_t d1 = vrow[4 * mm + 2 + g];
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
          const half8 va = as_half8(magic_pair(d0, 2 * sp, ones16), magic_pair(d0, 2 * sp + 8, ones16),
                                    magic_pair(d1, 2 * sp, ones16), magic_pair(d1, 2 * sp + 8, ones16));
          acc[4 * h + sp] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[mm], acc[4 * h + sp], 0, 0, 0);
        }
      }
    }
    if (smask) {
      // Window-owned tokens: O^T += Vimg^T (P / 4)^T.
      wait_vmem();
      wave_sync_lds();
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        float q4[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * mm + e;
          const int tok = 8 * (r >> 2) + 4 * g + (r & 3);
          q4[e] = ((smask >> tok) & 1u) ? 0.25f * pv[r] : 0.f;
        }
        const half8 ps = half8{(_Float16)q4[0], (_Float16)q4[2], (_Float16)q4[1], (_Float16)q4[3],
                               (_Float16)q4[4], (_Float16)q4[6], (_Float16)q4[5], (_Float16)q4[7]};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int sp = 0; sp < 4; ++sp) {
            const half8 va = *reinterpret_cast<const half8*>(ibuf + ((((h * 4 + sp) * 2 + mm) * 64) + lane) * 8);
            acc[4 * h + sp] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ps, acc[4 * h + sp], 0, 0, 0);
          }
        }
      }
    }
    wave_sync_lds();
  }

  // ---- combine the 4 wavefronts: common max, then a 2-round tree in LDS ----
  const float l_tot = l_run + shfl_xor_f32(l_run, 32);
  const float z_tot = z_run + shfl_xor_f32(z_run, 32);
  const float ps_tot = ps_run + shfl_xor_f32(ps_run, 32);
  if (g == 0) {
    S.mrow[w][col] = m_run;
    S.lrow[w][col] = l_tot;
  }
  __syncthreads();
  float mx = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < kWaves; ++k) mx = fmaxf(mx, S.mrow[k][col]);
  const float fw = (m_run == -__builtin_inff()) ? 0.f : exp2f(m_run - mx);
  const float f4 = 4.f * fw;
  const float off = (z_tot - 4.f * ps_tot) * fw;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = fmaf(acc[t][r], f4, off);
  }
  // Fragment buffers: [8 tiles][16 regs][64 lanes] fp32, lane-contiguous.
  float* frag0 = S.scratch;
  float* frag1 = frag0 + 8 * 16 * 64;
  if (w >= 2) {
    float* dst = (w == 2 ? frag0 : frag1) + lane;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[(t * 16 + r) * 64] = acc[t][r];
    }
  }
  __syncthreads();
  if (w < 2) {
    const float* src = (w == 0 ? frag0 : frag1) + lane;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][r] += src[(t * 16 + r) * 64];
    }
  }
  __syncthreads();
  if (w == 1) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) frag0[(t * 16 + r) * 64 + lane] = acc[t][r];
    }
  }
  __syncthreads();
  // Wave 0 adds the last fragment and writes [row][256] (row stride 257: no bank conflicts).
  constexpr int kOStride = kHeadDim + 1;
  float* obuf = frag1;
  if (w == 0) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = acc[t][r] + frag0[(t * 16 + r) * 64 + lane];
        const int h = t >> 2, sp = t & 3;
        const int f = 4 * (32 * h + 8 * (r >> 2) + 4 * g + (r & 3)) + sp;
        obuf[col * kOStride + f] = x;
      }
    }
  }
  __syncthreads();
  const int nrow = min(kRows, rows - rt * kRows);
  const int64_t item = item_index(a, req, kvh, split, rt);
  float* part = a.ws + item * kPartialFloats;
  for (int i = 4 * tid; i < nrow * kHeadDim; i += 1024) {
    const float* src = &obuf[(i >> 8) * kOStride + (i & 255)];
    *reinterpret_cast<floatx4*>(part + i) = floatx4{src[0], src[1], src[2], src[3]};
  }
  if (tid < nrow) {
    float lsum = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      const float mk = S.mrow[k][tid];
      if (mk != -__builtin_inff()) lsum += S.lrow[k][tid] * exp2f(mk - mx);
    }
    part[kRows * kHeadDim + tid] = mx;
    part[kRows * kHeadDim + kRows + tid] = lsum;
  }
}

// One 256-thread block per (output row, quarter of the features).  Every load
// the block needs goes out in one round: the splits' (m, l) (thread per
// split), the query row and the fresh keys (thread per feature), the block's
// 64-feature slice of every partial row (thread: split group t / 16, features
// 4 * (t % 16) .. +3 of the quarter) and the fresh values of that slice.
// Spreading a row over four blocks keeps each block's reads to a quarter of
// the partials, which the per-CU limit on outstanding misses rewards.
constexpr int kMaxSplits = 1024;
constexpr int kMergeGroups = 16;                 // split groups per block
constexpr int kMergeBatch = 8;                   // partial loads per thread per round

__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a) {
  __shared__ float red[kMaxFresh][4];
  __shared__ float fresh[kMaxFresh];
  __shared__ float wsplit[kMaxSplits];
  __shared__ float lsplit[kMaxSplits];
  __shared__ float wmax[4];
  __shared__ floatx4 osum[kMergeGroups][16];
  __shared__ float lsum_g[kMergeGroups];
  const int gidx = blockIdx.x;
  const int qd = gidx & 3;
  const int r = (gidx >> 2) % kRows;
  const int rest = (gidx >> 2) / kRows;
  const int rt = rest % a.row_tiles;
  const int rk = rest / a.row_tiles;
  const int req = rk / a.num_kv_heads;
  const int kvh = rk - req * a.num_kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int sg = tid >> 4, fl = tid & 15;
  const int f0 = 64 * qd + 4 * fl;

  const ReqInfo ri = a.reqs[req];
  const int qa = ri.qa, nq = ri.nq, prefix = ri.prefix;
  if (nq <= 0) return;
  const int row = rt * kRows + r;
  if (row >= nq * a.group) return;
  const int j = row / a.group;
  const int h = kvh * a.group + row % a.group;
  const int tiles = prefix > 0 ? (prefix + kTile - 1) / kTile : 0;
  const int splits = min(a.max_splits, tiles);     // split s holds tiles s, s + S, ...

  // ---- issue every load ----
  const float qf = a.q[((int64_t)(qa + j) * a.num_heads + h) * kHeadDim + tid];
  float kx[kMaxFresh];
#pragma unroll
  for (int i = 0; i < kMaxFresh; ++i)
    kx[i] = i <= j ? a.k_new[((int64_t)(qa + i) * a.num_kv_heads + kvh) * kHeadDim + tid] : 0.f;
  float mreg[kMaxSplits / 256], lreg[kMaxSplits / 256];
#pragma unroll
  for (int k = 0; k < kMaxSplits / 256; ++k) {
    const int sp = tid + 256 * k;
    mreg[k] = -__builtin_inff();
    lreg[k] = 0.f;
    if (sp < splits) {
      const float* part = a.ws + item_index(a, req, kvh, sp, rt) * kPartialFloats;
      mreg[k] = part[kRows * kHeadDim + r];
      lreg[k] = part[kRows * kHeadDim + kRows + r];
    }
  }
  const float* base = a.ws + item_index(a, req, kvh, 0, rt) * kPartialFloats + r * kHeadDim + f0;
  const int64_t pstride = (int64_t)a.row_tiles * kPartialFloats;
  floatx4 x[kMergeBatch];
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const int sp = sg + kMergeGroups * k;
    x[k] = sp < splits ? *reinterpret_cast<const floatx4*>(base + sp * pstride) : floatx4{};
  }
  floatx4 vf[kMaxFresh];
  if (sg == 0) {
#pragma unroll
    for (int i = 0; i < kMaxFresh; ++i)
      vf[i] = i <= j ? *reinterpret_cast<const floatx4*>(
                           a.v_new + ((int64_t)(qa + i) * a.num_kv_heads + kvh) * kHeadDim + f0)
                     : floatx4{};
  }

  // ---- fresh-token scores and the row max ----
  float mloc = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < kMaxSplits / 256; ++k) {
    const int sp = tid + 256 * k;
    if (sp < splits) {
      wsplit[sp] = mreg[k];
      lsplit[sp] = lreg[k];
      mloc = fmaxf(mloc, mreg[k]);
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxFresh; ++i) {
    if (i <= j) {
      float d = qf * kx[i];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) d += __shfl_xor(d, o, 64);
      if (lane == 0) red[i][w] = d;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
  if (lane == 0) wmax[w] = mloc;
  __syncthreads();
  if (tid <= j) fresh[tid] = (red[tid][0] + red[tid][1] + red[tid][2] + red[tid][3]) * a.scale_log2;
  __syncthreads();
  float mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  for (int i = 0; i <= j; ++i) mx = fmaxf(mx, fresh[i]);
  for (int sp = tid; sp < splits; sp += 256) {
    const float mc = wsplit[sp];
    wsplit[sp] = (mc == -__builtin_inff()) ? 0.f : exp2f(mc - mx);
  }
  __syncthreads();

  // ---- weighted sum of the partial slices ----
  floatx4 acc = floatx4{};
  float ls = 0.f;
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const int sp = sg + kMergeGroups * k;
    if (sp < splits) {
      acc += wsplit[sp] * x[k];
      ls = fmaf(wsplit[sp], lsplit[sp], ls);
    }
  }
  for (int s0 = sg + kMergeGroups * kMergeBatch; s0 < splits; s0 += kMergeGroups * kMergeBatch) {
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int sp = s0 + kMergeGroups * k;
      x[k] = sp < splits ? *reinterpret_cast<const floatx4*>(base + sp * pstride) : floatx4{};
    }
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int sp = s0 + kMergeGroups * k;
      if (sp < splits) {
        acc += wsplit[sp] * x[k];
        ls = fmaf(wsplit[sp], lsplit[sp], ls);
      }
    }
  }
  osum[sg][fl] = acc;
  if (fl == 0) lsum_g[sg] = ls;
  __syncthreads();
  if (sg == 0) {
    floatx4 o = floatx4{};
    float l = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < kMergeGroups; ++g2) {
      o += osum[g2][fl];
      l += lsum_g[g2];
    }
#pragma unroll
    for (int i = 0; i < kMaxFresh; ++i) {
      if (i <= j) {
        const float wgt = exp2f(fresh[i] - mx);
        l += wgt;
        o += wgt * vf[i];
      }
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    *reinterpret_cast<floatx4*>(a.out + ((int64_t)(qa + j) * a.num_heads + h) * kHeadDim + f0) = o * inv;
  }
}

int64_t splits_for(int64_t max_history, int tiles_per_split) {
  const int64_t tiles = max_history > 0 ? (max_history + kTile - 1) / kTile : 0;
  return (tiles + tiles_per_split - 1) / tiles_per_split;
}

int default_tiles_per_split(int32_t num_requests, int32_t num_kv_heads, int64_t max_history) {
  // Enough workgroups to cover the GPU for one long request, few enough that
  // the partials stay a fraction of the INT2 bytes read.
  const int64_t tiles = max_history > 0 ? (max_history + kTile - 1) / kTile : 0;
  const int64_t work = tiles * num_requests * num_kv_heads;
  int tps = 8;
  while (tps < 64 && work / tps > 1024) tps *= 2;
  return tps;
}

size_t workspace_floats(int32_t num_requests, int32_t num_kv_heads, int32_t num_heads,
                        int32_t max_query_len, int64_t max_history, int tiles_per_split) {
  const int64_t group = num_heads / num_kv_heads;
  const int64_t tiles_r = (max_query_len * group + kRows - 1) / kRows;
  const int64_t reqs = num_requests < kMaxInlineReqs ? num_requests : kMaxInlineReqs;   // one launch chunk
  return (size_t)reqs * num_kv_heads * splits_for(max_history, tiles_per_split) * tiles_r * kPartialFloats;
}

}  // namespace
}  // namespace oscar

using namespace oscar;

extern "C" {

size_t oscar_paged_decode_workspace_bytes(int32_t num_requests, int32_t num_kv_heads,
                                          int32_t num_heads, int32_t max_query_len,
                                          int64_t max_history, int32_t tiles_per_split) {
  if (num_requests <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads ||
      max_query_len <= 0 || max_history < 0 || tiles_per_split < 0 || tiles_per_split > 256)
    return 0;
  const int tps = tiles_per_split > 0 ? tiles_per_split
                                      : default_tiles_per_split(num_requests, num_kv_heads, max_history);
  return workspace_floats(num_requests, num_kv_heads, num_heads, max_query_len, max_history, tps) * sizeof(float);
}

int oscar_paged_decode(const float* q_rot, const float* k_new, const float* v_new,
                       int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                       int32_t head_size, const void* k_cache, const void* v_cache,
                       int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                       int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                       int64_t v_stride_token, int64_t v_stride_head, const int32_t* block_table,
                       int64_t block_table_stride, int32_t block_table_cols,
                       const int32_t* query_start_loc, const int32_t* seq_lens,
                       int32_t num_requests, int32_t max_query_len, int64_t max_history,
                       const int64_t* stage_owner, const void* stage_k_image,
                       const void* stage_v_image, int32_t stage_rows, float scale,
                       int32_t tiles_per_split, float* out, void* workspace,
                       size_t workspace_size, hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_requests < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || max_query_len < 0 || max_query_len > kMaxFresh ||
      max_history < 0 || block_size <= 0 || num_pages <= 0 || block_table_cols < 0 ||
      stage_rows < 0 || tiles_per_split < 0 || tiles_per_split > 256)
    return kErrInvalidArgument;
  if (num_tokens == 0 || num_requests == 0 || max_query_len == 0) return kOk;
  if (!q_rot || !k_new || !v_new || !k_cache || !v_cache || !query_start_loc || !seq_lens || !out)
    return kErrInvalidArgument;
  // Host-side request layout (the reference's query_layout checks).
  if (query_start_loc[0] < 0 || query_start_loc[num_requests] > num_tokens) return kErrInvalidArgument;
  for (int32_t i = 0; i < num_requests; ++i) {
    const int32_t nq = query_start_loc[i + 1] - query_start_loc[i];
    if (nq < 0 || nq > max_query_len || seq_lens[i] < nq || (int64_t)(seq_lens[i] - nq) > max_history)
      return kErrInvalidArgument;
  }
  if (max_history > 0 && !block_table) return kErrInvalidArgument;
  if (stage_rows > 0 && (!stage_owner || !stage_k_image || !stage_v_image)) return kErrInvalidArgument;
  if (stage_rows > 0 && ((reinterpret_cast<uintptr_t>(stage_k_image) & 15) ||
                         (reinterpret_cast<uintptr_t>(stage_v_image) & 15)))
    return kErrInvalidArgument;
  if (block_size % kTile != 0 || k_stride_head < kKCodeOff + kCodeBytes || v_stride_head < kCodeBytes ||
      (k_stride_head & 15) || (k_stride_token & 15) || (k_stride_page & 15) || (v_stride_head & 7) ||
      (v_stride_token & 7) || (v_stride_page & 7) || (reinterpret_cast<uintptr_t>(k_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(v_cache) & 7))
    return kErrUnsupportedGeometry;
  const int tps = tiles_per_split > 0 ? tiles_per_split
                                      : default_tiles_per_split(num_requests, num_kv_heads, max_history);
  const size_t need = workspace_floats(num_requests, num_kv_heads, num_heads, max_query_len, max_history, tps) *
                      sizeof(float);
  if (need > 0 && (workspace == nullptr || workspace_size < need)) return kErrWorkspaceTooSmall;

  DecodeArgs a{};
  a.q = q_rot;
  a.k_new = k_new;
  a.v_new = v_new;
  a.k_cache = static_cast<const uint8_t*>(k_cache);
  a.v_cache = static_cast<const uint8_t*>(v_cache);
  a.k_page = k_stride_page;
  a.k_tok = k_stride_token;
  a.k_head = k_stride_head;
  a.v_page = v_stride_page;
  a.v_tok = v_stride_token;
  a.v_head = v_stride_head;
  a.block_size = block_size;
  a.num_pages = num_pages;
  a.bt_stride = block_table_stride;
  a.bt_cols = block_table_cols;
  a.num_tokens = num_tokens;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_heads / num_kv_heads;
  a.owner = stage_owner;
  a.kimg = static_cast<const _Float16*>(stage_k_image);
  a.vimg = static_cast<const _Float16*>(stage_v_image);
  a.stage_rows = stage_rows;
  a.scale_log2 = scale * kLog2e;
  a.out = out;
  a.ws = static_cast<float*>(workspace);
  a.max_splits = (int32_t)splits_for(max_history, tps);
  if (a.max_splits > kMaxSplits) return kErrInvalidArgument;
  a.row_tiles = (max_query_len * a.group + kRows - 1) / kRows;

  static bool lds_attr_set = false;
  if (!lds_attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(paged_decode_split_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(LdsLayout)) != hipSuccess)
      return kErrLaunch;
    lds_attr_set = true;
  }
  // Chunks of kMaxInlineReqs requests; each chunk's partials reuse the same
  // workspace (the merge of one chunk precedes the next split in stream order).
  for (int32_t c0 = 0; c0 < num_requests; c0 += kMaxInlineReqs) {
    const int32_t nreq = num_requests - c0 < kMaxInlineReqs ? num_requests - c0 : kMaxInlineReqs;
    for (int32_t i = 0; i < nreq; ++i) {
      const int32_t qa = query_start_loc[c0 + i];
      const int32_t nq = query_start_loc[c0 + i + 1] - qa;
      a.reqs[i] = ReqInfo{qa, nq, seq_lens[c0 + i] - nq, 0};
    }
    a.block_table = block_table ? block_table + (int64_t)c0 * block_table_stride : nullptr;
    if (a.max_splits > 0) {
      dim3 grid((unsigned)a.max_splits, (unsigned)(nreq * num_kv_heads), (unsigned)a.row_tiles);
      hipLaunchKernelGGL(paged_decode_split_kernel, grid, dim3(256), sizeof(LdsLayout), stream, a);
      if (hipGetLastError() != hipSuccess) return kErrLaunch;
    }
    dim3 mgrid((unsigned)(nreq * num_kv_heads * a.row_tiles * kRows * 4));
    hipLaunchKernelGGL(paged_decode_merge_kernel, mgrid, dim3(256), 0, stream, a);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  return kOk;
}

}  // extern "C"
