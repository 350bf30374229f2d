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
// per row tile, so each INT2 token is read and unpacked once for all of them.
// A work item is (request, kv head, row tile).
//
// split kernel, grid (S + 1, items, row tiles), 4 wavefronts per workgroup:
//  * workgroup s < S: history split s.  Wave w takes the 32-token tiles
//    s + S (w + 4k) of the history, so the window's tiles (first and last
//    pages) spread over many waves.  The query rows and the wave's pages are
//    requested before anything is waited for, then the first two tiles' codes,
//    meta and owner tags; tiles are double-buffered after that.
//    Per tile (one page, as block_size % 32 == 0):
//    * S^T = K Q^T on 32x32x16 f16 MFMA.  K operands are the exact fp16 values
//      1 + c/4 built from the code bits (one shift and one and-or per pair);
//      the token's scale s and zero z act on the score tile:
//        q.k = s * sum q c + z * sum q = 4s * (q.k') + (z - 4s) * sum q.
//      The K dimension is permuted (feature 128g + 16j + 4a + i + 8b sits in
//      k-step 2j + a, slot 2i + b) so that pairs come straight out of a code
//      dword; Q^T (fp16, in LDS) uses the same permutation.
//    * O^T += V^T P'^T on 16 more MFMAs with V operands 1 + c/4 from byte-
//      transposed codes in LDS and P' = p * vs (fp16).  Then
//        sum_t p (c vs + vz) = 4 * acc - 4 * sum_t P' + sum_t p vz,
//      where sum_t P' is taken over the same fp16 values (v_dot2).
//    * Tokens owned by the staging arena are masked out of that pass.  The
//      first tile of a wave that holds any has its fp16 operand images (K in
//      the MFMA A-operand lane order, V^T likewise) copied to LDS with
//      global_load_lds_dwordx4 as soon as its owner tags arrive, and is run
//      again from the images after the INT2 tiles, for its window tokens only
//      (probabilities enter the PV pass as p / 4).  Further such tiles of the
//      same wave (common only when the window holds long-decoded history) are
//      run from their images one by one afterwards.
//    Base-2 online softmax in fp32; a row's running max is only raised when a
//    tile's max exceeds it by more than 2^4 (so P' <= 16 * vs stays finite in
//    fp16; a tile with a V scale above 4094 raises it eagerly), and the first
//    raise of a row needs no rescale.  The 4 wavefronts agree on a common max
//    in LDS and reduce-scatter their O^T fragments in two LDS rounds: wave w
//    ends with features 64w .. 64w + 63 of every row, transposes them through
//    LDS and writes whole row segments of the split's partial [32 rows][256]
//    + m[32] + l[32] (fp32, row-major).
//  * workgroup S: the step's own new tokens in exact fp32 (row (token j,
//    head) against new tokens 0 .. j), written as one more partial.
// merge kernel: one 256-thread block per (output row, feature quarter) of an
//   item; LSE-combines the item's partials and writes that slice of the row.
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
constexpr int kMaxTilesPerSplit = 256;
constexpr int kMaxWaveTiles = kMaxTilesPerSplit / kWaves;
constexpr int kMaxSplits = 1023;        // history splits; the fresh partial makes 1024

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Work items of one launch travel inside the kernel arguments (no device
// round trip for the metadata); larger batches are launched in chunks.
constexpr int kMaxInlineItems = 128;

struct ItemInfo {
  int32_t qa;        // first query row (token) of the request
  int32_t nq;        // query tokens of the request
  int32_t prefix;    // history length
  int16_t req;       // block-table row (request index within the launch chunk)
  int16_t kvh;       // kv head
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
  int32_t num_heads, num_kv_heads, group;
  const int64_t* owner;         // [rows, bs] or null
  const _Float16* kimg;         // [rows][bs / 32][Hk][kImgHalfs]
  const _Float16* vimg;
  int32_t stage_rows;
  float scale_log2;             // attention scale * log2(e)
  float* out;                   // [n, Hq, D]
  float* ws;                    // partials
  int32_t max_splits, row_tiles;
  ItemInfo items[kMaxInlineItems];
};

struct MainLds {
  _Float16 img[kWaves][2][kImgHalfs];             // staged K / V operand images (combine buffers alias)
  _Float16 q[16 * 2 * kRows * 8];                 // Q^T operand [m][g][row][8]
  float qsum[kRows];                              // sum of each row's fp16 q
  uint32_t vt[kWaves][64 * kVtStride];            // V codes [byte][token/4]
  float ta[kWaves][kTile];                        // score = ta * (q.k') + tb * qsum (+ tm)
  float tb[kWaves][kTile];
  float tm[kWaves][kTile];                        // 0, or -inf for a token left out of the INT2 pass
  float tvs[kWaves][kTile];                       // V scale (0: left out)
  float tvz[kWaves][kTile];                       // V zero
  float mrow[kWaves][kRows];
  float lrow[kWaves][kRows];
  uint32_t defmask[kWaves][kMaxWaveTiles];        // window-token masks of deferred tiles
};

struct FreshLds {
  float kf[kMaxFresh][kHeadDim];
  float vf[kMaxFresh][kHeadDim];
};

constexpr size_t kLdsBytes = sizeof(MainLds) > sizeof(FreshLds) ? sizeof(MainLds) : sizeof(FreshLds);
static_assert(kLdsBytes <= 160 * 1024, "one workgroup's LDS must fit the CU's 160 KiB");

constexpr int kPartO = kRows * kHeadDim;          // row-major O partial
constexpr size_t kPartialFloats = kPartO + 2 * kRows;

__device__ __forceinline__ int64_t item_index(const DecodeArgs& a, int item, int split, int rt) {
  return ((int64_t)item * (a.max_splits + 1) + split) * a.row_tiles + rt;
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

// Copy one staged operand image (16 KB) into a wave-owned LDS buffer.
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

// Loads of one tile whose page is already known (wave-uniform).  Every lane
// issues the same loads whatever the tile holds (tokens past the history read
// an in-bounds row of the page, an invalid tile reads page 0, no arena reads
// the slot's own bytes), so the compiler can wait for exactly one tile's loads
// while the next tile's are in flight; results that must not count are
// neutralised afterwards.
__device__ __forceinline__ TileLoad load_tile(const DecodeArgs& a, int page, int p0, int prefix, int kvh,
                                              int lane) {
  TileLoad L;
  const bool tile_ok = p0 < prefix && page >= 0;
  const int pg = tile_ok ? page : 0;
  L.page = tile_ok ? page : -1;
  L.prow0 = p0 - (p0 / a.block_size) * a.block_size;
  const int t = lane & 31, g = lane >> 5;
  const int tq = lane & 7, bg = lane >> 3;
  const uint8_t* kbase = a.k_cache + (int64_t)pg * a.k_page + (int64_t)kvh * a.k_head;
  const uint8_t* vbase = a.v_cache + (int64_t)pg * a.v_page + (int64_t)kvh * a.v_head;
  const bool tok_ok = tile_ok && p0 + t < prefix;
  const int trow = tok_ok ? L.prow0 + t : 0;
  const uint8_t* ks = kbase + (int64_t)trow * a.k_tok;
  L.meta = *reinterpret_cast<const u32x2*>(ks);
  L.kc0 = *reinterpret_cast<const u32x4*>(ks + kKCodeOff + 32 * g);
  L.kc1 = *reinterpret_cast<const u32x4*>(ks + kKCodeOff + 32 * g + 16);
  const bool arena = a.stage_rows > 0;
  const int64_t* op = arena ? a.owner + (int64_t)(pg % a.stage_rows) * a.block_size + trow
                            : reinterpret_cast<const int64_t*>(ks);
  const int64_t own = *op;
  L.own = arena ? own : -2;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int tk = 4 * tq + k;
    const int vrow = (tile_ok && p0 + tk < prefix) ? L.prow0 + tk : 0;
    L.vc[k] = *reinterpret_cast<const u32x2*>(vbase + (int64_t)vrow * a.v_tok + 8 * bg);
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

// Online-softmax state of one wavefront: O^T fragments (8 tiles of 32
// features x 32 rows) and per-row running max / sums.
struct WaveState {
  floatx16 acc[8];
  float m_run, l_run, z_run, ps_run;
};

// Raise the running max where a tile needs it (rescaling the state only for
// rows that already hold mass) and return the max the tile's exponents use.
__device__ __forceinline__ float lazy_max(const floatx16& s, bool eager, WaveState& st) {
  float mb = -__builtin_inff();
#pragma unroll
  for (int r = 0; r < 16; ++r) mb = fmaxf(mb, s[r]);
  mb = fmaxf(mb, shfl_xor_f32(mb, 32));
  const bool need = mb > st.m_run + (eager ? 0.f : kLazy);
  const bool resc = need && st.m_run != -__builtin_inff();
  if (__ballot(resc)) {
    const float alpha = resc ? exp2_raw(st.m_run - mb) : 1.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) st.acc[t] *= alpha;
    st.l_run *= alpha;
    st.z_run *= alpha;
    st.ps_run *= alpha;
  }
  if (need) st.m_run = mb;
  // exp2(-inf - m) = 0 needs a finite m: rows that have seen no key yet use 0.
  return st.m_run == -__builtin_inff() ? 0.f : st.m_run;
}

// Bit mask (token t of the tile -> bit t) of the tile's tokens that the
// staging arena owns.
__device__ __forceinline__ uint32_t window_mask(const TileLoad& L, int p0, int prefix, int lane) {
  const int col = lane & 31;
  const bool staged = L.page >= 0 && p0 + col < prefix && L.own == (int64_t)L.page;
  return (uint32_t)__ballot(staged && lane < 32);
}

__device__ __forceinline__ void issue_images(const DecodeArgs& a, MainLds& S, int page, int prow0, int kvh,
                                             int w, int lane) {
  const int64_t img = ((int64_t)(page % a.stage_rows) * (a.block_size / kTile) + prow0 / kTile) *
                      a.num_kv_heads + kvh;
  image_to_lds(a.kimg + img * kImgHalfs, S.img[w][0], lane);
  image_to_lds(a.vimg + img * kImgHalfs, S.img[w][1], lane);
}

// One history tile from its INT2 codes; tokens in `wmask` (window-owned) and
// tokens past the history are left out.
__device__ __forceinline__ void int2_tile(const DecodeArgs& a, MainLds& S, WaveState& st, const TileLoad& L,
                                          int p0, int prefix, uint32_t wmask, int w, int lane, float qsum,
                                          uint32_t ones16) {
  const int g = lane >> 5, col = lane & 31;
  const int tq = lane & 7, bg = lane >> 3;
  const int nvalid = L.page >= 0 ? min(kTile, prefix - p0) : 0;
  const bool used = col < nvalid && !((wmask >> col) & 1u);
  const bool masked = wmask != 0 || nvalid < kTile;      // wave-uniform

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
      float av = 0.f, bv = 0.f, vzv = 0.f, tmv = -__builtin_inff();
      if (used) {
        const float ks = f16_bits_to_f32(L.meta[0]);
        const float kz = f16_bits_to_f32(L.meta[0] >> 16);
        av = 4.f * ks * a.scale_log2;
        bv = (kz - 4.f * ks) * a.scale_log2;
        vsc = f16_bits_to_f32(L.meta[1]);
        vzv = f16_bits_to_f32(L.meta[1] >> 16);
        tmv = 0.f;
      }
      S.ta[w][col] = av;
      S.tb[w][col] = bv;
      S.tm[w][col] = tmv;
      S.tvs[w][col] = vsc;
      S.tvz[w][col] = vzv;
    }
  }
  const bool vs_big = __ballot(vsc > kLazyVsMax) != 0;
  wave_sync_lds();

  // ---- S^T = K' Q^T (all Q^T operand reads in flight together; two
  // accumulator chains) ----
  half8 qb[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) qb[m] = *reinterpret_cast<const half8*>(&S.q[((m * 2 + g) * kRows + col) * 8]);
  const uint32_t kw[8] = {L.kc0[0], L.kc0[1], L.kc0[2], L.kc0[3], L.kc1[0], L.kc1[1], L.kc1[2], L.kc1[3]};
  floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    half8 ka[2];
    k_operands(kw[j], ones16, ka);
    if (j & 1) {
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[0], qb[2 * j], s1, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[1], qb[2 * j + 1], s1, 0, 0, 0);
    } else {
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[0], qb[2 * j], s0, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[1], qb[2 * j + 1], s0, 0, 0, 0);
    }
  }
  floatx16 s = s0 + s1;

  // ---- scores and lazy online softmax (lane: row `col`, tokens 8*(r/4) + 4*g + r%4) ----
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const floatx4 av = *reinterpret_cast<const floatx4*>(&S.ta[w][8 * jj + 4 * g]);
    const floatx4 bv = *reinterpret_cast<const floatx4*>(&S.tb[w][8 * jj + 4 * g]);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[4 * jj + i] = fmaf(av[i], s[4 * jj + i], bv[i] * qsum);
  }
  if (masked) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const floatx4 tmv = *reinterpret_cast<const floatx4*>(&S.tm[w][8 * jj + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[4 * jj + i] += tmv[i];
    }
  }
  const float m_use = lazy_max(s, vs_big, st);
  half8 pb[2];
  float psum = 0.f, zsum = 0.f;
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
      s[r] = p * vsv[i];          // P' (scale folded)
    }
  }
  const half2v ones{(_Float16)1.f, (_Float16)1.f};
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
    st.ps_run += pss;
  }
  st.l_run += psum;
  st.z_run += zsum;

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
        st.acc[4 * h + sp] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[mm], st.acc[4 * h + sp], 0, 0, 0);
      }
    }
  }
  wave_sync_lds();
}

// The window-owned tokens `wmask` of a tile whose operand images are in the
// wave's LDS buffers: exact fp16 K / V values, probabilities into the PV pass
// as p / 4 (the state's O^T is scaled by 4 at the end).
__device__ __forceinline__ void window_tile(const DecodeArgs& a, MainLds& S, WaveState& st, uint32_t wmask,
                                            int w, int lane) {
  const int g = lane >> 5, col = lane & 31;
  const _Float16* kb = S.img[w][0];
  const _Float16* vb = S.img[w][1];
  floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
  for (int m0 = 0; m0 < 16; m0 += 8) {
    half8 ka[8], qb[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      ka[m] = *reinterpret_cast<const half8*>(kb + ((m0 + m) * 64 + lane) * 8);
      qb[m] = *reinterpret_cast<const half8*>(&S.q[(((m0 + m) * 2 + g) * kRows + col) * 8]);
    }
#pragma unroll
    for (int m = 0; m < 8; m += 2) {
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[m], qb[m], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[m + 1], qb[m + 1], s1, 0, 0, 0);
    }
  }
  floatx16 s = s0 + s1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int tok = 8 * (r >> 2) + 4 * g + (r & 3);
    s[r] = ((wmask >> tok) & 1u) ? s[r] * a.scale_log2 : -__builtin_inff();
  }
  const float m_use = lazy_max(s, false, st);
  float q4[16];
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float p = exp2_raw(s[r] - m_use);
    psum += p;
    q4[r] = 0.25f * p;
  }
  st.l_run += psum;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
    const float* e = q4 + 8 * mm;
    const half8 ps = half8{(_Float16)e[0], (_Float16)e[2], (_Float16)e[1], (_Float16)e[3],
                           (_Float16)e[4], (_Float16)e[6], (_Float16)e[5], (_Float16)e[7]};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int sp = 0; sp < 4; ++sp) {
        const half8 va = *reinterpret_cast<const half8*>(vb + ((((h * 4 + sp) * 2 + mm) * 64) + lane) * 8);
        st.acc[4 * h + sp] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ps, st.acc[4 * h + sp], 0, 0, 0);
      }
    }
  }
}

// ---- cross-wave reduce-scatter of the O^T fragments ----
// Round 1 pairs waves w and w ^ 2: wave w keeps tiles 4H .. 4H + 3 (H = w / 2)
// and sends the other four.  Round 2 pairs w and w ^ 1: wave w keeps the
// fragment registers 8J .. 8J + 7 (J = w % 2) of its tiles and sends the rest.
constexpr int kR1Floats = 4 * 4 * 64 * 4;   // per wave: 4 tiles x 4 register quads x 64 lanes x 4
constexpr int kR2Floats = 4 * 2 * 64 * 4;

// Fragments enter the exchange already finished: x -> x * f4 + off (the
// wave's share of the common max, the 1 + c/4 code offset and the V zeros).
template <int W>
__device__ __forceinline__ void rs_send1(const floatx16 (&acc)[8], float f4, float off, float* cb, int lane) {
  constexpr int Hs = 1 - (W >> 1);
  float* dst = cb + W * kR1Floats;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const floatx16& x = acc[4 * Hs + tt];
      *reinterpret_cast<floatx4*>(dst + ((tt * 4 + jq) * 64 + lane) * 4) =
          floatx4{fmaf(x[4 * jq], f4, off), fmaf(x[4 * jq + 1], f4, off), fmaf(x[4 * jq + 2], f4, off),
                  fmaf(x[4 * jq + 3], f4, off)};
    }
}

template <int W>
__device__ __forceinline__ void rs_recv1_send2(floatx16 (&acc)[8], float f4, float off, float* cb, int lane) {
  constexpr int H = W >> 1, J = W & 1, Js = 1 - J;
  const float* src = cb + (W ^ 2) * kR1Floats;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(src + ((tt * 4 + jq) * 64 + lane) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[4 * H + tt][4 * jq + i] = fmaf(acc[4 * H + tt][4 * jq + i], f4, off) + v[i];
    }
  float* dst = cb + 4 * kR1Floats + W * kR2Floats;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int r0 = 4 * (2 * Js + jj);
      *reinterpret_cast<floatx4*>(dst + ((tt * 2 + jj) * 64 + lane) * 4) =
          floatx4{acc[4 * H + tt][r0], acc[4 * H + tt][r0 + 1], acc[4 * H + tt][r0 + 2], acc[4 * H + tt][r0 + 3]};
    }
}

// Final round: add the partner's copy of the kept registers and stage this
// wave's 64 features of every row, [row][64 + 4 pad] fp32, in LDS (register
// 4jq + i of tile 4H + sp is local feature 32(jq - 2J) + 16g + 4i + sp).
constexpr int kTRow = 68;
constexpr int kTFloats = kRows * kTRow;

template <int W>
__device__ __forceinline__ void rs_recv2_stage(floatx16 (&acc)[8], const float* cb, float* tb, int lane) {
  constexpr int H = W >> 1, J = W & 1;
  const float* src = cb + 4 * kR1Floats + (W ^ 1) * kR2Floats;
  const int g = lane >> 5, col = lane & 31;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(src + ((tt * 2 + jj) * 64 + lane) * 4);
      const int r0 = 4 * (2 * J + jj);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[4 * H + tt][r0 + i] += v[i];
    }
  float* row = tb + W * kTFloats + col * kTRow + 16 * g;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * (2 * J + jj) + i;
      *reinterpret_cast<floatx4*>(row + 32 * jj + 4 * i) =
          floatx4{acc[4 * H][r], acc[4 * H + 1][r], acc[4 * H + 2][r], acc[4 * H + 3][r]};
    }
  }
}

// The step's own new tokens of one item, exact fp32: row (token j, head h)
// against new keys 0 .. j, written as a partial like a history split's.
__device__ void fresh_partial(const DecodeArgs& a, const ItemInfo& it, int item, int rt, FreshLds& F) {
  const int tid = threadIdx.x;
  const int nq = it.nq, kvh = it.kvh;
  const int rows = nq * a.group;
  const int r = tid >> 3, c = tid & 7;
  const int qrow = rt * kRows + r;
  const bool valid = qrow < rows;
  const int row = valid ? qrow : rows - 1;
  const int j = row / a.group;
  const int h = kvh * a.group + (row - j * a.group);
  floatx4 x[8];
  {
    // Thread (r, c) owns features 32k + 4c .. +3: each load and store
    // instruction covers whole 128-byte row segments.
    const floatx4* src = reinterpret_cast<const floatx4*>(a.q + ((int64_t)(it.qa + j) * a.num_heads + h) *
                                                          kHeadDim + 4 * c);
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = src[8 * k];
  }
  // New keys and values of the request: [nq][2][64 float4], 8 per thread at most.
  floatx4 kv[kMaxFresh * 128 / 256];
#pragma unroll
  for (int u = 0; u < kMaxFresh * 128 / 256; ++u) {
    const int idx = tid + 256 * u;
    const int i = idx >> 7, which = (idx >> 6) & 1, f4 = idx & 63;
    kv[u] = floatx4{};
    if (i < nq)
      kv[u] = *reinterpret_cast<const floatx4*>((which ? a.v_new : a.k_new) +
                                                ((int64_t)(it.qa + i) * a.num_kv_heads + kvh) * kHeadDim + 4 * f4);
  }
#pragma unroll
  for (int u = 0; u < kMaxFresh * 128 / 256; ++u) {
    const int idx = tid + 256 * u;
    const int i = idx >> 7, which = (idx >> 6) & 1, f4 = idx & 63;
    if (i < nq) *reinterpret_cast<floatx4*>((which ? F.vf[i] : F.kf[i]) + 4 * f4) = kv[u];
  }
  __syncthreads();
  float sc[kMaxFresh];
  float mx = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kMaxFresh; ++i) {
    sc[i] = -__builtin_inff();
    if (i < nq) {
      const floatx4* kr = reinterpret_cast<const floatx4*>(&F.kf[i][4 * c]);
      float d = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const floatx4 kk = kr[8 * k];
        d = fmaf(x[k][0], kk[0], d);
        d = fmaf(x[k][1], kk[1], d);
        d = fmaf(x[k][2], kk[2], d);
        d = fmaf(x[k][3], kk[3], d);
      }
      d += shfl_xor_f32(d, 1);
      d += shfl_xor_f32(d, 2);
      d += shfl_xor_f32(d, 4);
      if (i <= j) {
        sc[i] = d * a.scale_log2;
        mx = fmaxf(mx, sc[i]);
      }
    }
  }
  float l = 0.f;
  floatx4 o[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = floatx4{};
#pragma unroll
  for (int i = 0; i < kMaxFresh; ++i) {
    if (i < nq) {
      const float p = (i <= j) ? exp2f(sc[i] - mx) : 0.f;
      l += p;
      const floatx4* vr = reinterpret_cast<const floatx4*>(&F.vf[i][4 * c]);
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] += p * vr[8 * k];
    }
  }
  if (valid) {
    float* part = a.ws + item_index(a, item, a.max_splits, rt) * kPartialFloats;
    float* dst = part + r * kHeadDim + 4 * c;
#pragma unroll
    for (int k = 0; k < 8; ++k) reinterpret_cast<floatx4*>(dst)[8 * k] = o[k];
    if (c == 0) {
      part[kPartO + r] = mx;
      part[kPartO + kRows + r] = l;
    }
  }
}

__global__ __launch_bounds__(256) void paged_decode_split_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  const int split = blockIdx.x;
  const int item = blockIdx.y;
  const int rt = blockIdx.z;
  const ItemInfo it = a.items[item];
  const int rows = it.nq * a.group;
  if (it.nq <= 0 || rt * kRows >= rows) return;
  if (split == a.max_splits) {
    fresh_partial(a, it, item, rt, *reinterpret_cast<FreshLds*>(smem_raw));
    return;
  }
  const int prefix = it.prefix;
  const int tiles = (prefix + kTile - 1) / kTile;
  if (split >= tiles) return;
  MainLds& S = *reinterpret_cast<MainLds*>(smem_raw);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;
  const int kvh = it.kvh;
  const int nsplit = a.max_splits;
  const int tstep = nsplit * kWaves;
  const int first = split + nsplit * w;
  const int ntw = first < tiles ? (tiles - 1 - first) / tstep + 1 : 0;

  // ---- requests before any wait: this thread's query features and the
  // wave's pages (lane k: page of the wave's k-th tile), then the first two
  // tiles' loads, which are in flight while Q is converted ----
  const int r8 = tid >> 3, c8 = tid & 7;
  floatx4 x[8];
  {
    const int qrow = rt * kRows + r8;
    const int row = qrow < rows ? qrow : rows - 1;
    const int j = row / a.group, h = kvh * a.group + (row - j * a.group);
    const floatx4* src = reinterpret_cast<const floatx4*>(a.q + ((int64_t)(it.qa + j) * a.num_heads + h) *
                                                          kHeadDim + 32 * c8);
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = src[k];
  }
  int my_page = -1;
  if (lane < ntw) {
    const int pidx = (first + tstep * lane) * kTile / a.block_size;
    if (pidx < a.bt_cols) my_page = a.block_table[(int64_t)it.req * a.bt_stride + pidx];
  }
  if (my_page >= a.num_pages) my_page = -1;
  // @probe:1
  TileLoad A = load_tile(a, ntw > 0 ? __builtin_amdgcn_readlane(my_page, 0) : -1, first * kTile, prefix, kvh,
                         lane);
  TileLoad B = load_tile(a, ntw > 1 ? __builtin_amdgcn_readlane(my_page, 1) : -1, (first + tstep) * kTile,
                         prefix, kvh, lane);

  // ---- Q^T operand into LDS (permuted K dimension, fp16) and row sums ----
  // Thread: row r8, features 32 * c8 .. +31, which are exactly the four
  // operand vectors (m = 2jj + aa, gg) with jj = 2(c8 & 3) + jl: slot 2i + b of
  // vector (jl, aa) is local feature 16jl + 4aa + i + 8b.
  {
    float qs = 0.f;
    const int gg = c8 >> 2;
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
        const int m = 2 * (2 * (c8 & 3) + jl) + aa;
        *reinterpret_cast<half8*>(&S.q[((m * 2 + gg) * kRows + r8) * 8]) = v;
      }
    }
    qs += shfl_xor_f32(qs, 1);
    qs += shfl_xor_f32(qs, 2);
    qs += shfl_xor_f32(qs, 4);
    if (c8 == 0) S.qsum[r8] = (rt * kRows + r8 < rows) ? qs : 0.f;
  }
  __syncthreads();
  // @probe:2

  WaveState st;
#pragma unroll
  for (int t = 0; t < 8; ++t) st.acc[t] = floatx16{};
  st.m_run = -__builtin_inff();
  st.l_run = st.z_run = st.ps_run = 0.f;
  const float qsum = S.qsum[col];
  const uint32_t ones16 = magic_ones();
  int pend = -1;                 // first tile with window tokens (images in flight)
  uint32_t pend_mask = 0;
  uint64_t defer = 0;            // later tiles with window tokens

  // Window tokens of a tile: the first such tile's images are requested at
  // once, later ones are deferred.  Both prologue tiles are checked before
  // any compute so that their images are in flight early.
  auto note_window = [&](const TileLoad& L, int k, uint32_t wm) {
    if (wm == 0) return;
    if (pend < 0) {
      pend = k;
      pend_mask = wm;
      issue_images(a, S, L.page, L.prow0, kvh, w, lane);
    } else {
      defer |= 1ull << k;
      if (lane == 0) S.defmask[w][k] = wm;
    }
  };
  // A tile whose every history token is window-owned skips the INT2 pass.
  auto all_window = [&](int p0, uint32_t wm) {
    const int nvalid = min(kTile, prefix - p0);
    return wm != 0 && wm == (nvalid >= kTile ? 0xFFFFFFFFu : ((1u << nvalid) - 1u));
  };
  uint32_t wmA = ntw > 0 ? window_mask(A, first * kTile, prefix, lane) : 0u;
  uint32_t wmB = ntw > 1 ? window_mask(B, (first + tstep) * kTile, prefix, lane) : 0u;
  note_window(A, 0, wmA);
  note_window(B, 1, wmB);
#pragma unroll 1
  for (int k = 0; k < ntw; k += 2) {
    {
      const int p0 = (first + tstep * k) * kTile;
      if (k > 0) {
        wmA = window_mask(A, p0, prefix, lane);
        note_window(A, k, wmA);
      }
      if (!all_window(p0, wmA)) int2_tile(a, S, st, A, p0, prefix, wmA, w, lane, qsum, ones16);
      if (k + 2 < ntw)
        A = load_tile(a, __builtin_amdgcn_readlane(my_page, k + 2), p0 + 2 * tstep * kTile, prefix, kvh, lane);
    }
    if (k + 1 < ntw) {
      const int p0 = (first + tstep * (k + 1)) * kTile;
      if (k > 0) {
        wmB = window_mask(B, p0, prefix, lane);
        note_window(B, k + 1, wmB);
      }
      if (!all_window(p0, wmB)) int2_tile(a, S, st, B, p0, prefix, wmB, w, lane, qsum, ones16);
      if (k + 3 < ntw)
        B = load_tile(a, __builtin_amdgcn_readlane(my_page, k + 3), p0 + 2 * tstep * kTile, prefix, kvh, lane);
    }
  }
  // @probe:3

  // ---- window tokens from their operand images ----
  if (pend >= 0) {
    wait_vmem();
    wave_sync_lds();
    window_tile(a, S, st, pend_mask, w, lane);
#pragma unroll 1
    while (defer) {
      const int k = __builtin_ctzll(defer);
      defer &= defer - 1;
      const int p0 = (first + tstep * k) * kTile;
      wave_sync_lds();
      issue_images(a, S, __builtin_amdgcn_readlane(my_page, k), p0 % a.block_size, kvh, w, lane);
      wait_vmem();
      wave_sync_lds();
      window_tile(a, S, st, S.defmask[w][k], w, lane);
    }
  }
  // @probe:4

  // ---- combine the 4 wavefronts: common max, then reduce-scatter in LDS ----
  const float l_tot = st.l_run + shfl_xor_f32(st.l_run, 32);
  const float z_tot = st.z_run + shfl_xor_f32(st.z_run, 32);
  const float ps_tot = st.ps_run + shfl_xor_f32(st.ps_run, 32);
  if (g == 0) {
    S.mrow[w][col] = st.m_run;
    S.lrow[w][col] = l_tot;
  }
  __syncthreads();
  float mx = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < kWaves; ++k) mx = fmaxf(mx, S.mrow[k][col]);
  const float fw = (st.m_run == -__builtin_inff()) ? 0.f : exp2f(st.m_run - mx);
  const float f4 = 4.f * fw;
  const float off = (z_tot - 4.f * ps_tot) * fw;
  float* cb = reinterpret_cast<float*>(&S.img[0][0][0]);
  switch (w) {
    case 0: rs_send1<0>(st.acc, f4, off, cb, lane); break;
    case 1: rs_send1<1>(st.acc, f4, off, cb, lane); break;
    case 2: rs_send1<2>(st.acc, f4, off, cb, lane); break;
    default: rs_send1<3>(st.acc, f4, off, cb, lane); break;
  }
  __syncthreads();
  switch (w) {
    case 0: rs_recv1_send2<0>(st.acc, f4, off, cb, lane); break;
    case 1: rs_recv1_send2<1>(st.acc, f4, off, cb, lane); break;
    case 2: rs_recv1_send2<2>(st.acc, f4, off, cb, lane); break;
    default: rs_recv1_send2<3>(st.acc, f4, off, cb, lane); break;
  }
  __syncthreads();
  // Round 1's buffers are free now: each wave stages its [32][64] block
  // there and writes whole 256-byte row segments (16 lanes per row).
  float* tb = cb;
  switch (w) {
    case 0: rs_recv2_stage<0>(st.acc, cb, tb, lane); break;
    case 1: rs_recv2_stage<1>(st.acc, cb, tb, lane); break;
    case 2: rs_recv2_stage<2>(st.acc, cb, tb, lane); break;
    default: rs_recv2_stage<3>(st.acc, cb, tb, lane); break;
  }
  wave_sync_lds();
  const int nrow = min(kRows, rows - rt * kRows);
  float* part = a.ws + item_index(a, item, split, rt) * kPartialFloats;
#pragma unroll
  for (int s4 = 0; s4 < kRows / 4; ++s4) {
    const int row = 4 * s4 + (lane >> 4);
    if (row < nrow)
      *reinterpret_cast<floatx4*>(part + row * kHeadDim + 64 * w + 4 * (lane & 15)) =
          *reinterpret_cast<const floatx4*>(tb + w * kTFloats + row * kTRow + 4 * (lane & 15));
  }
  if (w == 0 && lane < nrow) {
    float lsum = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      const float mk = S.mrow[k][lane];
      if (mk != -__builtin_inff()) lsum += S.lrow[k][lane] * exp2f(mk - mx);
    }
    part[kPartO + lane] = mx;
    part[kPartO + kRows + lane] = lsum;
  }
  // @probe:5
}

// One 256-thread block per (output row, quarter of the features) of an item.
// Every load the block needs goes out in one round: the partials' (m, l)
// (thread per partial) and the block's 64-feature slice of every partial row
// (thread: partial group t / 16, features 4 * (t % 16) .. +3 of the quarter).
constexpr int kMergeGroups = 16;                 // partial groups per block
constexpr int kMergeBatch = 16;                  // partial loads per thread per round
constexpr int kMaxPartials = kMaxSplits + 1;

__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a) {
  __shared__ float wpart[kMaxPartials];
  __shared__ float lpart[kMaxPartials];
  __shared__ float wmax[4];
  __shared__ floatx4 osum[kMergeGroups][16];
  __shared__ float lsum_g[kMergeGroups];
  const int qd = blockIdx.x & 3;
  const int r = blockIdx.x >> 2;
  const int item = blockIdx.y;
  const int rt = blockIdx.z;
  const ItemInfo it = a.items[item];
  const int rows = it.nq * a.group;
  const int row = rt * kRows + r;
  if (it.nq <= 0 || row >= rows) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int sg = tid >> 4, fl = tid & 15;
  const int tiles = (it.prefix + kTile - 1) / kTile;
  const int hs = min(a.max_splits, tiles);        // history partials 0 .. hs - 1
  const int P = hs + 1;                           // partial hs is the fresh one (split max_splits)
  const float* base = a.ws + item_index(a, item, 0, rt) * kPartialFloats;
  const int64_t pstride = (int64_t)a.row_tiles * kPartialFloats;
  const int f0 = 64 * qd + 4 * fl;

  // ---- issue every load ----
  float mreg[kMaxPartials / 256], lreg[kMaxPartials / 256];
#pragma unroll
  for (int k = 0; k < kMaxPartials / 256; ++k) {
    const int p = tid + 256 * k;
    mreg[k] = -__builtin_inff();
    lreg[k] = 0.f;
    if (p < P) {
      const float* pp = base + (p < hs ? p : a.max_splits) * pstride;
      mreg[k] = pp[kPartO + r];
      lreg[k] = pp[kPartO + kRows + r];
    }
  }
  floatx4 x[kMergeBatch];
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const int p = sg + kMergeGroups * k;
    x[k] = p < P ? *reinterpret_cast<const floatx4*>(base + (p < hs ? p : a.max_splits) * pstride +
                                                     r * kHeadDim + f0)
                 : floatx4{};
  }

  // ---- common max and partial weights ----
  float mloc = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < kMaxPartials / 256; ++k) mloc = fmaxf(mloc, mreg[k]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
  if (lane == 0) wmax[w] = mloc;
  __syncthreads();
  const float mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
#pragma unroll
  for (int k = 0; k < kMaxPartials / 256; ++k) {
    const int p = tid + 256 * k;
    if (p < P) {
      wpart[p] = (mreg[k] == -__builtin_inff()) ? 0.f : exp2f(mreg[k] - mx);
      lpart[p] = lreg[k];
    }
  }
  __syncthreads();

  // ---- weighted sum of the partial slices ----
  floatx4 acc = floatx4{};
  float ls = 0.f;
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const int p = sg + kMergeGroups * k;
    if (p < P) {
      acc += wpart[p] * x[k];
      ls = fmaf(wpart[p], lpart[p], ls);
    }
  }
  for (int s0 = sg + kMergeGroups * kMergeBatch; s0 < P; s0 += kMergeGroups * kMergeBatch) {
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int p = s0 + kMergeGroups * k;
      x[k] = p < P ? *reinterpret_cast<const floatx4*>(base + (p < hs ? p : a.max_splits) * pstride +
                                                       r * kHeadDim + f0)
                   : floatx4{};
    }
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int p = s0 + kMergeGroups * k;
      if (p < P) {
        acc += wpart[p] * x[k];
        ls = fmaf(wpart[p], lpart[p], ls);
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
    const int j = row / a.group;
    const int h = it.kvh * a.group + (row - j * a.group);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    *reinterpret_cast<floatx4*>(a.out + ((int64_t)(it.qa + j) * a.num_heads + h) * kHeadDim + f0) = o * inv;
  }
}

int64_t splits_for(int64_t max_history, int tiles_per_split) {
  const int64_t tiles = max_history > 0 ? (max_history + kTile - 1) / kTile : 0;
  return (tiles + tiles_per_split - 1) / tiles_per_split;
}

int default_tiles_per_split(int32_t num_requests, int32_t num_kv_heads, int64_t max_history) {
  // Enough workgroups to cover the GPU for one long request, few enough that
  // the partials stay a fraction of the INT2 bytes read, and never more
  // splits than the merge takes.
  const int64_t tiles = max_history > 0 ? (max_history + kTile - 1) / kTile : 0;
  const int64_t work = tiles * num_requests * num_kv_heads;
  int tps = 4;
  while (tps < 64 && work / tps > 1024) tps *= 2;
  while (tps < kMaxTilesPerSplit && (tiles + tps - 1) / tps > kMaxSplits) tps *= 2;
  return tps;
}

int32_t requests_per_launch(int32_t num_kv_heads) {
  const int32_t r = kMaxInlineItems / num_kv_heads;
  return r > 0 ? r : 0;
}

size_t workspace_floats(int32_t num_requests, int32_t num_kv_heads, int32_t num_heads,
                        int32_t max_query_len, int64_t max_history, int tiles_per_split) {
  const int64_t group = num_heads / num_kv_heads;
  const int64_t tiles_r = (max_query_len * group + kRows - 1) / kRows;
  const int64_t per = requests_per_launch(num_kv_heads);
  const int64_t reqs = num_requests < per ? num_requests : per;     // one launch chunk
  return (size_t)reqs * num_kv_heads * (splits_for(max_history, tiles_per_split) + 1) * tiles_r *
         kPartialFloats;
}

}  // namespace
}  // namespace oscar

using namespace oscar;

extern "C" {

size_t oscar_paged_decode_workspace_bytes(int32_t num_requests, int32_t num_kv_heads,
                                          int32_t num_heads, int32_t max_query_len,
                                          int64_t max_history, int32_t tiles_per_split) {
  if (num_requests <= 0 || num_kv_heads <= 0 || num_kv_heads > kMaxInlineItems || num_heads <= 0 ||
      num_heads % num_kv_heads || max_query_len <= 0 || max_history < 0 || tiles_per_split < 0 ||
      tiles_per_split > kMaxTilesPerSplit)
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
      num_kv_heads > kMaxInlineItems || num_heads % num_kv_heads != 0 || max_query_len < 0 ||
      max_query_len > kMaxFresh || max_history < 0 || block_size <= 0 || num_pages <= 0 ||
      block_table_cols < 0 || stage_rows < 0 || tiles_per_split < 0 || tiles_per_split > kMaxTilesPerSplit)
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
  const int64_t splits = splits_for(max_history, tps);
  if (splits > kMaxSplits) return kErrInvalidArgument;
  const size_t need = workspace_floats(num_requests, num_kv_heads, num_heads, max_query_len, max_history, tps) *
                      sizeof(float);
  if (workspace == nullptr || workspace_size < need) return kErrWorkspaceTooSmall;

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
  a.max_splits = (int32_t)splits;
  a.row_tiles = (max_query_len * a.group + kRows - 1) / kRows;

  static bool lds_attr_set = false;
  if (!lds_attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(paged_decode_split_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes) != hipSuccess)
      return kErrLaunch;
    lds_attr_set = true;
  }
  // Chunks of whole requests (at most kMaxInlineItems items); each chunk's
  // partials reuse the same workspace (the merge of one chunk precedes the
  // next split in stream order).
  const int32_t per = requests_per_launch(num_kv_heads);
  for (int32_t c0 = 0; c0 < num_requests; c0 += per) {
    const int32_t nreq = num_requests - c0 < per ? num_requests - c0 : per;
    for (int32_t i = 0; i < nreq; ++i) {
      const int32_t qa = query_start_loc[c0 + i];
      const int32_t nq = query_start_loc[c0 + i + 1] - qa;
      for (int32_t h = 0; h < num_kv_heads; ++h)
        a.items[i * num_kv_heads + h] = ItemInfo{qa, nq, seq_lens[c0 + i] - nq, (int16_t)i, (int16_t)h};
    }
    a.block_table = block_table ? block_table + (int64_t)c0 * block_table_stride : nullptr;
    const unsigned nitems = (unsigned)(nreq * num_kv_heads);
    dim3 grid((unsigned)(a.max_splits + 1), nitems, (unsigned)a.row_tiles);
    hipLaunchKernelGGL(paged_decode_split_kernel, grid, dim3(256), kLdsBytes, stream, a);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
    dim3 mgrid((unsigned)(kRows * 4), nitems, (unsigned)a.row_tiles);
    hipLaunchKernelGGL(paged_decode_merge_kernel, mgrid, dim3(256), 0, stream, a);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  return kOk;
}

}  // extern "C"
