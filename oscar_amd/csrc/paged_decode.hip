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
// History splits: an item's history is cut into 128-token steps (one 32-token
// tile per wavefront); split s of an item with S splits takes steps s,
// s + S, s + 2S, ..., so the window's first and last steps land in different
// workgroups.  The host plans S per item (a common number of steps per split,
// the smallest that keeps the launch's splits within one round of resident
// workgroups).  The grid's x dimension runs over the launch chunk's
// workgroups: each item's splits (split 0 first, then S - 1, S - 2, ..., 1,
// so that the window steps start first), then the item's fresh-token
// workgroup when it has one; a workgroup finds its item by a binary search
// of the items' first workgroups.  The z dimension is the row tile.
//
// split kernels (4 wavefronts, two workgroups per CU), one fp32 partial
// [32 rows][256] + m[32] + l[32] per (item, split, row tile):
//  * paged_decode_split_kernel (items of more than 8 rows): the wavefronts
//    take a step together.  Wave w scores tile w of the step for every row:
//    S^T = K Q^T on 32x32x16 f16 MFMA.  K operands are the exact fp16 values
//    1 + c/4 built from the code bits (one shift and one and-or per pair);
//    the token's scale s and zero z act on the score tile:
//      q.k = s * sum q c + z * sum q = 4s * (q.k') + (z - 4s) * sum q.
//    The K dimension is permuted (feature 128g + 16j + 4a + i + 8b sits in
//    k-step 2j + a, slot 2i + b) so that pairs come straight out of a code
//    dword; Q^T sits in LDS as an fp16 high part and low part (q - high),
//    and each K operand meets both.  The waves agree on the step's row maxima
//    in LDS and write P' = p * vs (fp16) of their tiles there; wave w then
//    accumulates features 64w .. 64w + 63 of every row over the step's four
//    tiles, O^T += V^T P'^T with V operands 1 + c/4 from byte-transposed
//    codes, and
//      sum_t p (c vs + vz) = 4 * acc - 4 * sum_t P' + sum_t p vz.
//    Window-owned tokens (arena owner tag = the token's page) take their K
//    operand from the tile's fp16 image (high part, then the low part against
//    q's high part) and their V from the V image's high and low parts, with
//    weight p / 4.
//  * paged_decode_split_small_kernel (items of at most 8 rows): each
//    wavefront walks its own tiles on 16x16x32 MFMA tiles (its own comment
//    below).
//  Base-2 online softmax in fp32; a row's running max is raised only when a
//  tile or step exceeds it by more than 2^kLazy (so P' = p * vs stays finite
//  in fp16; a V scale above kLazyVsMax raises it eagerly), and the first
//  raise of a row needs no rescale.  Every row sum is taken over the weights
//  as their fp16 rounding left them, so the output stays a convex
//  combination of the values.
//  * the fresh-token workgroup of an item (or, when the item has none of its
//    own, the history split with the least work): the step's own new tokens
//    in exact fp32 (row (token j, head) against new tokens 0 .. j), written
//    as one more partial.
// merge kernels: the item's partials LSE-combined per output row (one block
//   per row and feature quarter, or one thread per four features when every
//   item has at most 32 partials); the rotated variant also multiplies by
//   R_v^T and casts to the output dtype.
//
// DecodeOnly read (no fresh K/V; one query token per request, history
// [0, seq)): the same kernels without the fresh-token workgroup, and a
// staged value replaces the INT2 one only at positions p < head or p >= cut
// of the request: head is the sink length when every seat of the sink pages
// holds its page, else 0; cut starts the run of staged positions that ends
// at seq - 1 inside [max(seq - recent, head), seq).  The small-row kernel's
// kFold instance finds (head, cut) in its prologue (at most 256 sink and
// recent positions: one of each per thread); other launches run a bounds
// kernel first.
#include <type_traits>

#include "oscar_common.h"
#include "window_images.h"
#include "../../include/oscar_amd.h"

namespace oscar {
namespace {

constexpr int kTile = 32;
constexpr int kWaves = 4;
constexpr int kRows = 32;
constexpr int kStepTok = kWaves * kTile;  // history tokens per step: one tile per wavefront
constexpr int kMaxFresh = 16;
constexpr int kPRow = 40;               // halves per P' row: 32 token slots + pad (16-byte rows)
constexpr int kVtRow = 10;              // dwords per V code byte row: 8 groups of 4 tokens + pad
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 4.f;            // log2 headroom before a running max is raised
constexpr float kLazyVsMax = 4094.f;    // 16 * 4094 < 65504 (fp16 max)
constexpr int kMaxTilesPerSplit = 256;  // 64 steps: one page-register lane per step
constexpr int kMaxSplits = 1023;        // history splits; the fresh partial makes 1024

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));

// Work items of one launch travel inside the kernel arguments (no device
// round trip for the metadata); larger batches are launched in chunks.
constexpr int kMaxInlineItems = 128;

struct ItemInfo {
  int32_t qa;        // first query row (token) of the request
  int32_t prefix;    // history length
  int32_t pbase;     // first partial slot of the item: history splits 0 .. nsplit - 1, then the fresh one
  int16_t nq;        // query tokens of the request
  int16_t req;       // block-table row (request index within the launch chunk)
  int16_t kvh;       // kv head
  int16_t nsplit;    // history splits of the item: split s takes steps s, s + nsplit, s + 2 nsplit, ...
};

struct DecodeArgs {
  const float* q;          // [n, Hq, D]
  const float* k_new;      // [n, Hk, D]
  const float* v_new;
  const uint8_t* k_cache;
  const uint8_t* v_cache;
  int64_t k_page, k_tok, k_head, v_page, v_tok, v_head;
  int32_t block_size;
  FastDiv bs_div;               // block_size
  FastDiv rows_div;             // stage_rows (1 without an arena)
  int64_t num_pages;
  const int32_t* block_table;
  int64_t bt_stride;
  int32_t bt_cols;
  int32_t num_heads, num_kv_heads, group;
  const int64_t* owner;         // [rows, bs] or null
  const _Float16* kimg;         // [rows][bs / 32][Hk][kKImgHalfs]
  const _Float16* vimg;
  int32_t stage_rows;
  float scale_log2;             // attention scale * log2(e)
  float* out;                   // [n, Hq, D]
  float* ws;                    // partials
  const int32_t* win;           // DecodeOnly: (head, cut) per chunk request; null: every position
  int32_t fresh;                // 1: the fresh-token partial exists (MTP read); 0: DecodeOnly
  int32_t fresh_block;          // 1: a workgroup of its own computes it (x = the item's nsplit); 0: a history split does
  int32_t max_splits, row_tiles;  // the largest nsplit of the launch; row tiles per item
  int32_t nitems;               // items of the launch chunk
  ItemInfo items[kMaxInlineItems];
  int32_t win_fold;             // DecodeOnly through the small-row kernel: it finds (head, cut) itself
  int32_t win_sink, win_recent; // ... from sink_eff and recent (each at most 256: one position per thread)
};

// One step is 128 history tokens, one 32-token tile per wavefront.  Only the
// V code transpose is written before a step's first barrier, while a slower
// wave may still run the previous step's PV pass on it, so it alone is
// double-buffered; everything else a step exchanges is written after that
// barrier and read before the next step's.
struct StepLds {
  uint32_t vt[kWaves][64 * kVtRow];        // V code bytes, [byte][group of 4 tokens]
};

struct MainLds {
  _Float16 q[16 * 2 * kRows * 8];          // Q^T operand [m][g][row][8], fp16 high part
  _Float16 qlo[16 * 2 * kRows * 8];        // the low part, fp16(q - high): q = high + low to 2^-22
  float qsum[kRows];                       // sum of each row's q
  float ta[kWaves][kTile];                 // score = ta * acc + tb * qsum + tm (own tile)
  float tb[kWaves][kTile];
  float tm[kWaves][kTile];                 // 0, or -inf for a token left out
  float tvs[kWaves][kTile];                // V scale of an INT2 token (else 0)
  float trv[kWaves][kTile];                // 1 / V scale of an INT2 token (else 0)
  float tvz[kWaves][kTile];                // V zero / V scale of an INT2 token (else 0)
  _Float16 p[kWaves][kRows * kPRow];       // P' = p * vs of each tile's INT2 tokens, [row][slot]
  _Float16 pw[kWaves][kRows * kPRow];      // p / 4 of each tile's window tokens, [row][slot]
  float mx[kWaves][kRows];                 // each tile's row maxima
  uint32_t big[kWaves];                    // the tile holds a V scale above kLazyVsMax
  StepLds buf[2];
};

struct FreshLds {
  float kf[kMaxFresh][kHeadDim];
  float vf[kMaxFresh][kHeadDim];
};

constexpr size_t kLdsBytes = sizeof(MainLds) > sizeof(FreshLds) ? sizeof(MainLds) : sizeof(FreshLds);
static_assert(kLdsBytes <= 80 * 1024, "two workgroups' LDS must fit the CU's 160 KiB");

constexpr int kPartO = kRows * kHeadDim;          // row-major O partial
constexpr size_t kPartialFloats = kPartO + 2 * kRows;

// The item of split-kernel workgroup b (the split grid is one dimension of
// exactly the launch's workgroups, item by item: each item's history splits,
// then its fresh-token workgroup when it has one), b's index within it, and
// the item's fields.  Item i's workgroups start at pbase(i) - i * (fresh -
// fresh_block), a non-decreasing sequence: the item is the last one whose
// start is <= b, i.e. the number of starts <= b, less one.  Every lane reads
// items `lane` and `lane + 64` (all inline items) in one round of independent
// loads, a ballot counts the starts, and the chosen item's fields come from
// its lane: one memory round trip, where a search would take a dependent
// round trip per halving.  Called by every lane of the wavefront.
static_assert(kMaxInlineItems <= 128, "two items per lane");
__device__ __forceinline__ ItemInfo find_item(const DecodeArgs& a, int b, int& item, int& local) {
  const int skip = a.fresh - a.fresh_block;     // fresh slots without a workgroup of their own
  const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  // (unconditional loads, lanes past the last item reading item 0, so that
  // all ten go out before one wait)
  const int n = a.nitems;
  const int* f0 = reinterpret_cast<const int*>(&a.items[lane < n ? lane : 0]);
  const int* f1 = reinterpret_cast<const int*>(&a.items[lane + 64 < n ? lane + 64 : 0]);
  int w0[5], w1[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    w0[k] = f0[k];
    w1[k] = f1[k];
  }
  static_assert(offsetof(ItemInfo, pbase) == 2 * sizeof(int), "pbase is the third word");
  const int s0 = lane < n ? w0[2] - lane * skip : 0x7fffffff;
  const int s1 = lane + 64 < n ? w1[2] - (lane + 64) * skip : 0x7fffffff;
  item = __popcll(__ballot(s0 <= b)) + __popcll(__ballot(s1 <= b)) - 1;
  item = __builtin_amdgcn_readfirstlane(item);
  int fld[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    const int v0 = __builtin_amdgcn_readlane(w0[k], item & 63), v1 = __builtin_amdgcn_readlane(w1[k], item & 63);
    fld[k] = item < 64 ? v0 : v1;
  }
  static_assert(sizeof(ItemInfo) == 5 * sizeof(int), "ItemInfo is five words");
  ItemInfo it;
  __builtin_memcpy(&it, fld, sizeof(it));
  local = b - (it.pbase - item * skip);
  return it;
}

__device__ __forceinline__ int64_t partial_index(const DecodeArgs& a, const ItemInfo& it, int split, int rt) {
  return ((int64_t)it.pbase + split) * a.row_tiles + rt;
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

// Bits of a tile's valid tokens (the first n of its 32).
__device__ __forceinline__ uint32_t tile_valid(int n) { return n >= 32 ? ~0u : (n <= 0 ? 0u : (1u << n) - 1u); }

__device__ __forceinline__ half8 as_half8(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3) {
  return __builtin_bit_cast(half8, u32x4{d0, d1, d2, d3});
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s_barrier without the memory fence __syncthreads carries: the fence would
// wait for every outstanding global load, including the next step's, which
// are meant to stay in flight.  LDS writes are complete at lgkmcnt(0).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0); vmcnt and expcnt left at their maxima
  asm volatile("s_barrier" ::: "memory");
}

// One step's loads of one wavefront: its own tile's K codes, meta and V codes,
// and the owner tags of all 128 tokens of the step (lane l: tokens l, 64 + l).
struct StepLoad {
  u32x4 kc0, kc1;     // this lane's 32 K code bytes (token col, half g)
  u32x2 meta;         // K scale, K zero, V scale, V zero (fp16 pairs)
  u32x2 vc[4];        // V code bytes 8*bg .. +7 of tokens 4*tq .. +3
  int32_t own0, own1; // owner tags, low 32 bits (meaningful only with an arena)
};

// Every lane issues the same loads whatever the step holds (tokens past the
// history read an in-bounds row, an invalid tile reads page 0, no arena reads
// slot bytes), so the compiler can wait for exactly one step's loads while the
// next step's are in flight; results that must not count are neutralised
// where they are used.
__device__ __forceinline__ StepLoad load_step(const DecodeArgs& a, const int (&pg)[kWaves], const int (&tb)[kWaves],
                                              int prefix, int kvh, int w, int lane) {
  StepLoad L;
  const int t = lane & 31, g = lane >> 5;
  const int tq = lane & 7, bg = lane >> 3;
  const int p0 = w == 0 ? tb[0] : (w == 1 ? tb[1] : (w == 2 ? tb[2] : tb[3]));
  const int page = pg[w];
  const bool tile_ok = p0 < prefix && page >= 0;
  const int pgc = tile_ok ? page : 0;
  const int prow0 = (int)fast_mod((uint32_t)p0, a.bs_div);
  const uint8_t* kbase = a.k_cache + (int64_t)pgc * a.k_page + (int64_t)kvh * a.k_head;
  const uint8_t* vbase = a.v_cache + (int64_t)pgc * a.v_page + (int64_t)kvh * a.v_head;
  const int trow = (tile_ok && p0 + t < prefix) ? prow0 + t : 0;
  const uint8_t* ks = kbase + (int64_t)trow * a.k_tok;
  L.meta = *reinterpret_cast<const u32x2*>(ks);
  L.kc0 = *reinterpret_cast<const u32x4*>(ks + kKCodeOff + 32 * g);
  L.kc1 = *reinterpret_cast<const u32x4*>(ks + kKCodeOff + 32 * g + 16);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int tk = 4 * tq + k;
    const int vrow = (tile_ok && p0 + tk < prefix) ? prow0 + tk : 0;
    L.vc[k] = *reinterpret_cast<const u32x2*>(vbase + (int64_t)vrow * a.v_tok + 8 * bg);
  }
  // Owner tags.  The pointers are made opaque so that the loads are always
  // issued (without an arena the compiler would reuse the meta load instead,
  // which makes the step's load count path-dependent).
  typedef __attribute__((address_space(1))) const int32_t global_i32;
  const bool arena = a.stage_rows > 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tk = 64 * h + lane;
    const int j = tk >> 5;
    const int pj = j == 0 ? pg[0] : (j == 1 ? pg[1] : (j == 2 ? pg[2] : pg[3]));
    const int pos = (j == 0 ? tb[0] : (j == 1 ? tb[1] : (j == 2 ? tb[2] : tb[3]))) + (tk & (kTile - 1));
    const bool ok = arena && pj >= 0 && pos < prefix;
    const int64_t* op = ok ? a.owner + (int64_t)fast_mod((uint32_t)pj, a.rows_div) * a.block_size +
                                 fast_mod((uint32_t)pos, a.bs_div)
                           : reinterpret_cast<const int64_t*>(ks);
    // Owner tags are pages (< 2^31) or -1: the low word identifies them
    // (little-endian int64).
    global_i32* gop = (global_i32*)op;
    asm volatile("" : "+v"(gop));
    (h == 0 ? L.own0 : L.own1) = *gop;
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

// Index of the staged operand image of the tile whose first row is prow0 on
// `page` (the arena seat row is page % rows).
__device__ __forceinline__ int64_t image_index(const DecodeArgs& a, int page, int prow0, int kvh) {
  return ((int64_t)fast_mod((uint32_t)page, a.rows_div) * (a.block_size / kTile) + prow0 / kTile) * a.num_kv_heads +
         kvh;
}
// The step's own new tokens of one item, exact fp32: row (token j, head h)
// against new keys 0 .. j, written as a partial like a history split's.
__device__ void fresh_partial(const DecodeArgs& a, const ItemInfo& it, int item, int rt, FreshLds& F, int tid) {
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
    float* part = a.ws + partial_index(a, it, it.nsplit, rt) * kPartialFloats;
    float* dst = part + r * kHeadDim + 4 * c;
#pragma unroll
    for (int k = 0; k < 8; ++k) reinterpret_cast<floatx4*>(dst)[8 * k] = o[k];
    if (c == 0) {
      part[kPartO + r] = mx;
      part[kPartO + kRows + r] = l;
    }
  }
}

__device__ __forceinline__ uint32_t pair_lo(uint32_t d, uint32_t ls, uint32_t ones) {
  return ((d << ls) & 0x03000300u) | ones;     // code of bytes 0 and 2 -> fp16 pair 1 + c/4
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t d, uint32_t rs, uint32_t ones) {
  return ((d >> rs) & 0x03000300u) | ones;     // code of bytes 1 and 3
}

template <typename T>
__device__ __forceinline__ T pick4(T v0, T v1, T v2, T v3, int i) {
  return i == 0 ? v0 : (i == 1 ? v1 : (i == 2 ? v2 : v3));
}

template <int kCtrl>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}

// Max / sum over the 32 lanes of this lane's half wave, in every lane: quad
// xor 1 and 2, half-row and row mirrors, then the other 16 lanes.
template <bool kMax>
__device__ __forceinline__ float half_wave_reduce(float x) {
  auto op = [](float u, float v) { return kMax ? fmaxf(u, v) : u + v; };
  x = op(x, dpp_move<0xB1>(x));
  x = op(x, dpp_move<0x4E>(x));
  x = op(x, dpp_move<0x141>(x));
  x = op(x, dpp_move<0x140>(x));
  return op(x, shfl_xor_f32(x, 16));
}

// kMidIssue selects where the step loop requests the next step's loads: at
// the top of the step (false), or after the step's score pass (true), where
// every image load of the step has been issued before them.  Loads complete
// in issue order and the compiler cannot tell which of a step's conditional
// image loads a path really issued, so at the top it makes the window-free
// path wait for the next step's loads before its score pass; after the score
// pass they are newer than every image load.  The single-step workgroups
// (long-history MTP reads such as 1 x 4 tokens over 24K) run the first
// instance, whose allocation was tuned for their window tiles; multi-step
// launches run the second (C3 55.1 -> 54.1 us; C5 unchanged within noise).
template <bool kMidIssue>
__global__ __launch_bounds__(256, 2) void paged_decode_split_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  // History splits are dispatched as 0, S - 1, S - 2, ..., 1: the first and
  // last steps hold the window tokens, whose extra passes make them the
  // longest workgroups, so they start first (measured: C5 decode 37.6 ->
  // 34 us, C2 unchanged).
  int bx, item;
  const ItemInfo it = find_item(a, (int)blockIdx.x, item, bx);
  const int rt = blockIdx.z;
  const int rows = it.nq * a.group;
  if (it.nq <= 0 || rt * kRows >= rows) return;
  if (bx >= it.nsplit) {                  // the fresh-token workgroup, or none for this item
    if (a.fresh_block && bx == it.nsplit)
      fresh_partial(a, it, item, rt, *reinterpret_cast<FreshLds*>(smem_raw), (int)threadIdx.x);
    return;
  }
  const int split = bx == 0 ? 0 : it.nsplit - bx;
  const int prefix = it.prefix;
  const int steps = (prefix + kStepTok - 1) / kStepTok;
  // Without a workgroup of its own (when one more per item would not find a
  // resident slot), the step's own new tokens (the fresh partial, partial
  // slot S) go to a split with the least history work that holds no window
  // step (sink and recent tokens lie in the first and last steps): an idle
  // split when the history has fewer steps than there are splits; else the
  // last split when the steps do not divide evenly (it has one step fewer
  // than the splits that hold the last steps); else the middle one.
  const int rem = steps % it.nsplit;
  const int fresh_split = steps < it.nsplit ? steps : (rem != 0 ? it.nsplit - 1 : it.nsplit / 2);
  const bool fresh_here = a.fresh && !a.fresh_block && split == fresh_split;
  if (split >= steps) {
    if (fresh_here) fresh_partial(a, it, item, rt, *reinterpret_cast<FreshLds*>(smem_raw), (int)threadIdx.x);
    return;
  }
  MainLds& S = *reinterpret_cast<MainLds*>(smem_raw);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int col = lane & 31;
  const int kvh = it.kvh;
  const int nsplit = it.nsplit;
  const int nst = (steps - 1 - split) / nsplit + 1;     // steps split + nsplit k, k < nst (<= 64)
  // Single-step launches with one split per step: wave j takes tile j of
  // step (split + j * spread) mod nsplit, so that the four tiles of a step
  // (the window steps, first and last, among them) go to four workgroups,
  // whose waves then each hold at most one window tile's images.
  const int spread = (!kMidIssue && nsplit == steps && nsplit >= 8) ? nsplit / 4 : 0;
  auto step_of = [&](int k, int j) {
    const int sj = split + j * spread;
    return (sj >= nsplit ? sj - nsplit : sj) + nsplit * k;
  };
  // first token of tile j of the k-th step this workgroup takes
  auto tile_bases = [&](int k, int (&tb)[kWaves]) {
#pragma unroll
    for (int j = 0; j < kWaves; ++j) tb[j] = step_of(k, j) * kStepTok + kTile * j;
  };
  const bool arena = a.stage_rows > 0;
  // Positions whose staged value may replace the INT2 one: p < win_head or
  // p >= win_tail (every position for the MTP read).  Scalar loads, waited
  // for with the LDS barrier below.
  int win_head = 0, win_tail = 0;
  if (a.win) {
    typedef __attribute__((address_space(4))) const int32_t const_i32;
    const const_i32* wb = (const const_i32*)a.win;
    win_head = wb[2 * it.req];
    win_tail = wb[2 * it.req + 1];
  }

  // ---- requests before any wait: the query features, then the pages of the
  // workgroup's tiles (lane k of pgv[j]: tile j of step k), then the first
  // step.  The page reads are unconditional (an unused lane reads column 0)
  // so that the query and page loads issue back to back. ----
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
  __builtin_amdgcn_sched_barrier(0);      // the query loads go out first
  int pgv[kWaves];
  const int32_t* bt_row = a.block_table + (int64_t)it.req * a.bt_stride;
#pragma unroll
  for (int j = 0; j < kWaves; ++j) {
    // token offsets stay below 2^31: (split + nsplit * lane) * 128 < 1024 * 64 * 128
    const uint32_t tok0 = (uint32_t)step_of(lane, j) * kStepTok + kTile * j;
    const uint32_t pidx = fast_div(tok0, a.bs_div);
    const bool ok = lane < nst && (int)tok0 < prefix && (int)pidx < a.bt_cols;
    const int p = bt_row[ok ? pidx : 0];
    pgv[j] = ok ? p : -1;
  }
  auto step_pages = [&](int k, int (&pg)[kWaves]) {
#pragma unroll
    for (int j = 0; j < kWaves; ++j) {
      const int p = __builtin_amdgcn_readlane(pgv[j], k);
      pg[j] = (p >= 0 && p < a.num_pages) ? p : -1;
    }
  };
  int pg[kWaves];
  step_pages(0, pg);
  // Touch the pages of this wave's later tiles in both caches (lane k: step
  // k), so that their address translations overlap the first step instead of
  // each step's own loads.  The words are consumed (below) where the first
  // step's loads, issued after them, are needed anyway.
  uint32_t touched;
  {
    const int pk = pick4(pgv[0], pgv[1], pgv[2], pgv[3], w);
    const int64_t pgk = (lane < nst && pk >= 0 && pk < a.num_pages) ? pk : 0;
    touched = *reinterpret_cast<const uint32_t*>(a.k_cache + pgk * a.k_page) ^
              *reinterpret_cast<const uint32_t*>(a.v_cache + pgk * a.v_page);
  }
  int tb0[kWaves];
  tile_bases(0, tb0);
  StepLoad cur = load_step(a, pg, tb0, prefix, kvh, w, lane);

  // ---- Q^T operand into LDS (permuted K dimension, fp16 high + low parts) and row sums ----
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
        half8 v, vl;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int k = 16 * jl + 4 * aa + (u >> 1) + 8 * (u & 1);
          const float xq = x[k >> 2][k & 3];
          v[u] = (_Float16)xq;
          vl[u] = (_Float16)(xq - (float)v[u]);
          qs += xq;
        }
        const int m = 2 * (2 * (c8 & 3) + jl) + aa;
        *reinterpret_cast<half8*>(&S.q[((m * 2 + gg) * kRows + r8) * 8]) = v;
        *reinterpret_cast<half8*>(&S.qlo[((m * 2 + gg) * kRows + r8) * 8]) = vl;
      }
    }
    qs += shfl_xor_f32(qs, 1);
    qs += shfl_xor_f32(qs, 2);
    qs += shfl_xor_f32(qs, 4);
    if (c8 == 0) S.qsum[r8] = (rt * kRows + r8 < rows) ? qs : 0.f;
  }
  lds_barrier();
  asm volatile("" ::"v"(touched));

  floatx16 acc[2] = {floatx16{}, floatx16{}};   // O^T of features 64w .. 64w + 63 (2 blocks of 32)
  float m_run = -__builtin_inff();
  float l_run = 0.f, z_run = 0.f, ps_run = 0.f;  // this lane's share of its row's sums (own tiles)
  const float qsum = S.qsum[col];
  const uint32_t ones16 = magic_ones();
  // PV operand lane constants: block b, row m = col is code sp = 2b + (m & 1)
  // of V code byte 16w + (m >> 1).
  const int vrow = 16 * w + (col >> 1);
  const uint32_t e2 = 2u * (uint32_t)(col & 1);
  const uint32_t ls0 = 8u - e2, rs0 = e2, ls1 = 4u - e2, rs1 = 4u + e2;

  auto run_step = [&](const StepLoad& L, int k, const int (&pgs)[kWaves], auto&& issue_next) {
    int tb[kWaves];
    tile_bases(k, tb);
    StepLds& B = S.buf[k & 1];
    // window-owned tokens of the step's four tiles (bit t of wmj: token t of tile j)
    uint32_t wm0 = 0u, wm1 = 0u, wm2 = 0u, wm3 = 0u;
    if (arena) {
      const int pa = g == 0 ? pgs[0] : pgs[1];
      const int pb = g == 0 ? pgs[2] : pgs[3];
      const int q0 = (g == 0 ? tb[0] : tb[1]) + col, q1 = (g == 0 ? tb[2] : tb[3]) + col;
      const bool s0 = pa >= 0 && q0 < prefix && (q0 < win_head || q0 >= win_tail) && L.own0 == pa;
      const bool s1 = pb >= 0 && q1 < prefix && (q1 < win_head || q1 >= win_tail) && L.own1 == pb;
      const uint64_t b0 = __ballot(s0), b1 = __ballot(s1);
      wm0 = (uint32_t)b0;
      wm1 = (uint32_t)(b0 >> 32);
      wm2 = (uint32_t)b1;
      wm3 = (uint32_t)(b1 >> 32);
    }
    const uint32_t wmw = pick4(wm0, wm1, wm2, wm3, w);
    const int pgw = pick4(pgs[0], pgs[1], pgs[2], pgs[3], w);
    const int p0 = pick4(tb[0], tb[1], tb[2], tb[3], w);
    const int nvalid = pgw >= 0 ? min(kTile, max(prefix - p0, 0)) : 0;
    // A tile with window tokens reads the high part of their K operand image
    // now, a phase before the score pass uses it (the low part reuses these
    // registers inside that pass).
    const u32x4* img = reinterpret_cast<const u32x4*>(
        a.kimg + image_index(a, wmw != 0u ? pgw : 0, (int)fast_mod((uint32_t)p0, a.bs_div), kvh) * kKImgHalfs);
    u32x4 im[16];
    if (wmw != 0u) {
#pragma unroll
      for (int m = 0; m < 16; ++m) im[m] = img[m * 64 + lane];
    }

    // ---- own tile: token parameters and byte-transposed V codes ----
    bool big;
    {
      const bool win = (wmw >> col) & 1u;
      const bool used = col < nvalid && !win;
      const float ksc = f16_bits_to_f32(L.meta[0]);
      const float kz = f16_bits_to_f32(L.meta[0] >> 16);
      const float vsc = f16_bits_to_f32(L.meta[1]);
      const float vz = f16_bits_to_f32(L.meta[1] >> 16);
      if (g == 0) {
        S.ta[w][col] = used ? 4.f * ksc * a.scale_log2 : (win ? a.scale_log2 : 0.f);
        S.tb[w][col] = used ? (kz - 4.f * ksc) * a.scale_log2 : 0.f;
        S.tm[w][col] = (used || win) ? 0.f : -__builtin_inff();
        const float rvs = used ? 1.f / vsc : 0.f;
        S.tvs[w][col] = used ? vsc : 0.f;
        S.trv[w][col] = rvs;
        S.tvz[w][col] = used ? vz * rvs : 0.f;
      }
      big = __ballot(used && vsc > kLazyVsMax) != 0;
      const int tq = lane & 7, bg = lane >> 3;
      uint32_t o0[4], o1[4];
      transpose4(L.vc[0][0], L.vc[1][0], L.vc[2][0], L.vc[3][0], o0);
      transpose4(L.vc[0][1], L.vc[1][1], L.vc[2][1], L.vc[3][1], o1);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        B.vt[w][(8 * bg + kk) * kVtRow + tq] = o0[kk];
        B.vt[w][(8 * bg + 4 + kk) * kVtRow + tq] = o1[kk];
      }
    }
    wave_sync_lds();

    // ---- S^T = K Q^T of the own tile (window tokens from their image) ----
    floatx16 s;
    {
      // Q^T operands (high and low parts, so the products see q to 2^-22;
      // the code operands 1 + c/4 are exact) are read from LDS one k-step
      // pair ahead of their use.
      const half8* qsrc = reinterpret_cast<const half8*>(&S.q[(g * kRows + col) * 8]);   // + m * 2 * kRows
      const half8* qlsrc = reinterpret_cast<const half8*>(&S.qlo[(g * kRows + col) * 8]);
      const uint32_t kw[8] = {L.kc0[0], L.kc0[1], L.kc0[2], L.kc0[3], L.kc1[0], L.kc1[1], L.kc1[2], L.kc1[3]};
      // One accumulator chain: the other workgroup on the SIMD covers the
      // MFMA latency.
      s = floatx16{};
      // S^T = K Q^T (lane: row col, 16 tokens)
      auto score_mfma = [&](const half8& kop, const half8& qop) {
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qop, s, 0, 0, 0);
      };
      half8 qa = qsrc[0], qb = qsrc[2 * kRows], qal = qlsrc[0], qbl = qlsrc[2 * kRows];
      auto qk_pair = [&](int j, const half8& k0, const half8& k1) {
        half8 na = qa, nb = qb, nal = qal, nbl = qbl;
        if (j < 7) {
          na = qsrc[(2 * j + 2) * 2 * kRows];
          nb = qsrc[(2 * j + 3) * 2 * kRows];
          nal = qlsrc[(2 * j + 2) * 2 * kRows];
          nbl = qlsrc[(2 * j + 3) * 2 * kRows];
        }
        score_mfma(k0, qa);
        score_mfma(k1, qb);
        score_mfma(k0, qal);
        score_mfma(k1, qbl);
        qa = na;
        qb = nb;
        qal = nal;
        qbl = nbl;
      };
      if (wmw == 0u) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          half8 ka[2];
          k_operands(kw[j], ones16, ka);
          qk_pair(j, ka[0], ka[1]);
        }
      } else {
        const bool wl = (wmw >> col) & 1u;
        const u32x4* img_lo = img + 16 * 64;
        // a tile whose valid tokens are all window-owned needs no code operands
        const bool all_win = (tile_valid(nvalid) & ~wmw) == 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          half8 ka[2];
          if (all_win) {
            ka[0] = __builtin_bit_cast(half8, im[2 * j]);
            ka[1] = __builtin_bit_cast(half8, im[2 * j + 1]);
          } else {
            k_operands(kw[j], ones16, ka);
#pragma unroll
            for (int aa = 0; aa < 2; ++aa)
              ka[aa] = wl ? __builtin_bit_cast(half8, im[2 * j + aa]) : ka[aa];
          }
          qk_pair(j, ka[0], ka[1]);
          // As soon as a k-step pair of the high part is used, its registers
          // take the same pair of the low part, zero for lanes of tokens
          // outside the window, so the first low loads have the rest of the
          // high pass to arrive (the barriers keep the loads from moving up,
          // where they would need registers of their own).
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int m = 2 * j; m < 2 * j + 2; ++m) im[m] = wl ? img_lo[m * 64 + lane] : u32x4{};
          __builtin_amdgcn_sched_barrier(0);
        }
        // window tokens (the other lanes hold zeros): low part of k against
        // the high part of q (the low-low product is below 2^-22 of the
        // score's terms)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const half8 la = __builtin_bit_cast(half8, im[2 * j]);
          const half8 lb = __builtin_bit_cast(half8, im[2 * j + 1]);
          score_mfma(la, qsrc[(2 * j) * 2 * kRows]);
          score_mfma(lb, qsrc[(2 * j + 1) * 2 * kRows]);
        }
      }
    }
    // The window tiles' V image blocks of this wave's features (high parts)
    // are requested here, a phase before the PV pass uses them.  The low
    // parts share their cache lines and replace them in the PV pass.
    const bool anywin = (wm0 | wm1 | wm2 | wm3) != 0u;
    auto vimg_of = [&](int j) {
      return reinterpret_cast<const half8*>(
          a.vimg + image_index(a, pgs[j], (int)fast_mod((uint32_t)tb[j], a.bs_div), kvh) *
                       kVImgHalfs);
    };
    half8 vim[kWaves][2][2];
    if (anywin) {
#pragma unroll
      for (int j = 0; j < kWaves; ++j) {
        const uint32_t wmj = j == 0 ? wm0 : (j == 1 ? wm1 : (j == 2 ? wm2 : wm3));
        if (wmj != 0u) {
          const half8* vimg = vimg_of(j);
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) vim[j][b][s2] = vimg[vimg_part(((w * 2 + b) * 2 + s2) * 64 + lane, 0)];
        }
      }
    }
    issue_next();
    // scores (lane: row col, tokens 8 (r / 4) + 4g + r % 4) and the tile's row max
    float mb = -__builtin_inff();
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const floatx4 av = *reinterpret_cast<const floatx4*>(&S.ta[w][8 * jj + 4 * g]);
      const floatx4 bv = *reinterpret_cast<const floatx4*>(&S.tb[w][8 * jj + 4 * g]);
      const floatx4 tmv = *reinterpret_cast<const floatx4*>(&S.tm[w][8 * jj + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[4 * jj + i] = fmaf(av[i], s[4 * jj + i], bv[i] * qsum) + tmv[i];
        mb = fmaxf(mb, s[4 * jj + i]);
      }
    }
    mb = fmaxf(mb, shfl_xor_f32(mb, 32));
    if (g == 0) S.mx[w][col] = mb;
    if (lane == 0) S.big[w] = big ? 1u : 0u;
    lds_barrier();

    // ---- common max of the step (same decision in every wave), P' of the own tile ----
    const bool eager = (S.big[0] | S.big[1] | S.big[2] | S.big[3]) != 0u;
    {
      const float M = fmaxf(fmaxf(S.mx[0][col], S.mx[1][col]), fmaxf(S.mx[2][col], S.mx[3][col]));
      const bool need = M > m_run + (eager ? 0.f : kLazy);
      const bool resc = need && m_run != -__builtin_inff();
      if (__ballot(resc)) {
        const float alpha = resc ? exp2_raw(m_run - M) : 1.f;
        acc[0] *= alpha;
        acc[1] *= alpha;
        l_run *= alpha;
        z_run *= alpha;
        ps_run *= alpha;
      }
      if (need) m_run = M;
    }
    // exp2(-inf - m) = 0 needs a finite m: rows that have seen no key yet use 0.
    const float m_use = m_run == -__builtin_inff() ? 0.f : m_run;
    float psum = 0.f, zsum = 0.f, pss = 0.f;
    const half2v ones{(_Float16)1.f, (_Float16)1.f};
    _Float16* prow = &S.p[w][col * kPRow + 4 * g];
    _Float16* pwrow = &S.pw[w][col * kPRow + 4 * g];
#pragma unroll
    // The row sums take each token's weight as the PV pass sees it (after
    // its fp16 rounding: P' / vs of an INT2 token, 4 * (p / 4) of a window
    // token), so that the output is a convex combination of the values
    // whatever that rounding did.
    for (int jj = 0; jj < 4; ++jj) {
      const floatx4 vsv = *reinterpret_cast<const floatx4*>(&S.tvs[w][8 * jj + 4 * g]);
      const floatx4 rvv = *reinterpret_cast<const floatx4*>(&S.trv[w][8 * jj + 4 * g]);
      const floatx4 zrv = *reinterpret_cast<const floatx4*>(&S.tvz[w][8 * jj + 4 * g]);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = exp2_raw(s[4 * jj + i] - m_use);
      // slots 8jj + 4g + {0, 1, 2, 3} hold tokens 8jj + 4g + {0, 2, 1, 3}
      const half4 h = half4{(_Float16)(p[0] * vsv[0]), (_Float16)(p[2] * vsv[2]), (_Float16)(p[1] * vsv[1]),
                            (_Float16)(p[3] * vsv[3])};
      *reinterpret_cast<half4*>(prow + 8 * jj) = h;
      pss = __builtin_amdgcn_fdot2(half2v{h[0], h[1]}, ones, pss, false);
      pss = __builtin_amdgcn_fdot2(half2v{h[2], h[3]}, ones, pss, false);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float wi = (float)h[i == 1 ? 2 : (i == 2 ? 1 : i)];
        psum = fmaf(wi, rvv[i], psum);
        zsum = fmaf(wi, zrv[i], zsum);
      }
      if (wmw != 0u) {
        const uint32_t wb = wmw >> (8 * jj + 4 * g);
        const half4 hw = half4{(wb & 1u) ? (_Float16)(0.25f * p[0]) : (_Float16)0.f,
                               (wb & 4u) ? (_Float16)(0.25f * p[2]) : (_Float16)0.f,
                               (wb & 2u) ? (_Float16)(0.25f * p[1]) : (_Float16)0.f,
                               (wb & 8u) ? (_Float16)(0.25f * p[3]) : (_Float16)0.f};
        *reinterpret_cast<half4*>(pwrow + 8 * jj) = hw;
        float ws = __builtin_amdgcn_fdot2(half2v{hw[0], hw[1]}, ones, 0.f, false);
        ws = __builtin_amdgcn_fdot2(half2v{hw[2], hw[3]}, ones, ws, false);
        psum = fmaf(4.f, ws, psum);
      }
    }
    l_run += psum;
    z_run += zsum;
    ps_run += pss;
    lds_barrier();

    // ---- O^T (features 64w .. 64w + 63) += V^T P'^T over the step's tiles ----
#pragma unroll
    for (int j = 0; j < kWaves; ++j) {
      if (pgs[j] < 0 || tb[j] >= prefix) continue;
      const uint32_t wmj = j == 0 ? wm0 : (j == 1 ? wm1 : (j == 2 ? wm2 : wm3));
      // a tile without INT2 tokens has all its P' zero: only its window part
      const bool int2 = (tile_valid(min(kTile, prefix - tb[j])) & ~wmj) != 0u;
      if (int2) {
        const uint32_t* vr = &B.vt[j][vrow * kVtRow];
        const _Float16* pr = &S.p[j][col * kPRow + 8 * g];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const uint32_t d0 = vr[4 * s2 + 2 * g], d1 = vr[4 * s2 + 2 * g + 1];
          const half8 pop = *reinterpret_cast<const half8*>(pr + 16 * s2);
          const half8 v0 = as_half8(pair_lo(d0, ls0, ones16), pair_hi(d0, rs0, ones16), pair_lo(d1, ls0, ones16),
                                    pair_hi(d1, rs0, ones16));
          const half8 v1 = as_half8(pair_lo(d0, ls1, ones16), pair_hi(d0, rs1, ones16), pair_lo(d1, ls1, ones16),
                                    pair_hi(d1, rs1, ones16));
          acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v0, pop, acc[0], 0, 0, 0);
          acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v1, pop, acc[1], 0, 0, 0);
        }
      }
      if (wmj != 0u) {
        const _Float16* pwr = &S.pw[j][col * kPRow + 8 * g];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const half8 pwop = *reinterpret_cast<const half8*>(pwr + 16 * s2);
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vim[j][b][s2], pwop, acc[b], 0, 0, 0);
        }
        // the low parts into the same registers (cache lines the high parts
        // brought in), multiplied in after the last tile
        const half8* vimg = vimg_of(j);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) vim[j][b][s2] = vimg[vimg_part(((w * 2 + b) * 2 + s2) * 64 + lane, 1)];
      }
    }
    if (anywin) {
#pragma unroll
      for (int j = 0; j < kWaves; ++j) {
        const uint32_t wmj = j == 0 ? wm0 : (j == 1 ? wm1 : (j == 2 ? wm2 : wm3));
        if (wmj != 0u) {
          const _Float16* pwr = &S.pw[j][col * kPRow + 8 * g];
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const half8 pwop = *reinterpret_cast<const half8*>(pwr + 16 * s2);
#pragma unroll
            for (int b = 0; b < 2; ++b)
              acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vim[j][b][s2], pwop, acc[b], 0, 0, 0);
          }
        }
      }
    }
  };

  // Steady state: the next step's loads are issued before this step's are
  // used (at the top of the step or after its score pass), unconditionally,
  // so each wait counts exactly one step's loads.
  int k = 0;
#pragma unroll 1
  for (; k + 1 < nst; ++k) {
    int pgn[kWaves];
    StepLoad nxt;
    auto issue = [&] {
      step_pages(k + 1, pgn);
      int tbn[kWaves];
      tile_bases(k + 1, tbn);
      nxt = load_step(a, pgn, tbn, prefix, kvh, w, lane);
    };
    if constexpr (kMidIssue) {
      run_step(cur, k, pg, issue);
    } else {
      issue();
      run_step(cur, k, pg, [] {});
    }
    cur = nxt;
#pragma unroll
    for (int j = 0; j < kWaves; ++j) pg[j] = pgn[j];
  }
  run_step(cur, k, pg, [] {});

  // ---- row sums over both lane halves and the four waves, then the partial ----
  // The sums go through the Q^T area, which no wave reads after the last
  // step's scores (every wave has passed that step's barriers by now).
  float* red = reinterpret_cast<float*>(S.q);
  static_assert(sizeof(S.q) >= kWaves * 3 * kRows * sizeof(float), "row sums fit the Q^T area");
  l_run += shfl_xor_f32(l_run, 32);
  z_run += shfl_xor_f32(z_run, 32);
  ps_run += shfl_xor_f32(ps_run, 32);
  if (g == 0) {
    red[(w * 3 + 0) * kRows + col] = l_run;
    red[(w * 3 + 1) * kRows + col] = z_run;
    red[(w * 3 + 2) * kRows + col] = ps_run;
  }
  lds_barrier();
  float lt = 0.f, zt = 0.f, pt = 0.f;
#pragma unroll
  for (int ww = 0; ww < kWaves; ++ww) {
    lt += red[(ww * 3 + 0) * kRows + col];
    zt += red[(ww * 3 + 1) * kRows + col];
    pt += red[(ww * 3 + 2) * kRows + col];
  }
  // sum_t p (c vs + vz) = 4 * acc - 4 * sum_t P' + sum_t p vz
  const float off = zt - 4.f * pt;
  // Registers 4jq + 2h, 4jq + 2h + 1 of blocks 0 and 1 are local features
  // 16jq + 8g + 4h + 0 .. 3 of row col: stored straight from the registers.
  const int nrow = min(kRows, rows - rt * kRows);
  float* part = a.ws + partial_index(a, it, split, rt) * kPartialFloats;
  if (col < nrow) {
    float* dst = part + col * kHeadDim + 64 * w + 8 * g;
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *reinterpret_cast<floatx4*>(dst + 16 * jq + 4 * h) =
            floatx4{fmaf(4.f, acc[0][4 * jq + 2 * h], off), fmaf(4.f, acc[0][4 * jq + 2 * h + 1], off),
                    fmaf(4.f, acc[1][4 * jq + 2 * h], off), fmaf(4.f, acc[1][4 * jq + 2 * h + 1], off)};
    }
  }
  if (w == 0 && lane < nrow) {
    part[kPartO + lane] = m_run;
    part[kPartO + kRows + lane] = lt;
  }
  if (fresh_here) {
    __syncthreads();               // the history's LDS is no longer read
    // the thread index rebuilt from the wave index and the lane count, so
    // that no register holds it through the steps
    const int ftid = 64 * w + (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    fresh_partial(a, it, item, rt, *reinterpret_cast<FreshLds*>(smem_raw), ftid);
  }
}

// ---------------------------------------------------------------- small-row split kernel
// Launches whose items all have at most 8 rows (single-token requests of a
// GQA group of up to 8: long-context decode, the DecodeOnly read).  Same work
// split, partials and window semantics as paged_decode_split_kernel, but each
// wavefront walks its own 32-token tiles (tile w of each of the workgroup's
// steps) on its own: running maxima and sums per wavefront, no barrier
// between the wavefronts until the workgroup combines their four partial
// rows at the end.  A tile's bytes (K codes, meta, V codes, owner tags) are
// copied straight into a 3-slot LDS ring of the wavefront by buffer loads to
// LDS, two tiles ahead of the one being computed, so that the history
// streams without holding registers for the loads in flight.  Window-owned
// tokens are left out of a tile and added by a window pass from the fp16
// images; a wavefront takes its last tile first (the recent window's, when
// it holds any) and runs that tile's window pass at once, while the next two
// tiles arrive, and the other window tiles' passes after its last tile.
//
// Lane l = (c, G), c = l % 16, G = l / 16, on v_mfma_f32_16x16x32_f16:
//  * S^T = K Q^T for each half h of the tile: A = K (16 tokens x 32
//    features): lane (t, G) holds token 8 (t / 4) + 4h + t % 4; B = Q^T:
//    column c < 8 is the fp16 high part of row c, column 8 + r the low part
//    of row r, so one pass gives both products and a row-rotation by 8 lanes
//    adds them.  The result registers r of lane (c, G) are then the scores of
//    tokens 8G + 4h + r for row c % 8: lane group G holds tokens 8G .. 8G + 7.
//    K-step s of lane group G covers the features of window-image block
//    m = 8 (G >> 1) + s, half g = G & 1 (one 16-byte code chunk per half).
//  * O^T += V^T P'^T over 16 feature tiles n = (q, b, mh): A = V^T: lane
//    (c, G) holds feature 64q + 32mh + 4 (c >> 1) + 2b + (c & 1) of tokens
//    8G + {0, 2, 1, 3, 4, 6, 5, 7} (exactly a window V-image chunk), B = P'^T
//    in the same token order, built from the lane's own scores.  Output lane
//    (c, G): features 64q + 32mh + 8G + {0, 1, 4, 5} + 2b of row c.
constexpr int kSmRows = 8;
constexpr int kSmVtRow = 10;     // dwords per V code byte row: 8 groups of 4 tokens + pad
constexpr int kSmRing = 3;       // tiles resident per wavefront: the one computed and two in flight

// One tile's bytes as the buffer loads leave them (lane order of each load).
struct SmallSlot {
  u32x4 kc[2][64];               // K code chunk of lane l for half h (see load_small_tile)
  uint8_t vc[kTile][kCodeBytes]; // V code bytes, token-major
  u32x2 meta[kTile];             // K scale, K zero, V scale, V zero
  u32x2 own[kTile];              // owner tag (int64) of the token's arena seat
};

struct SmallTileLds {
  uint32_t vt[64 * kSmVtRow];    // vt[b * kSmVtRow + t / 4]: byte b of tokens t .. t + 3
  float prm[6][kTile];           // per token: ta, tb, tm, vs, 1 / vs, vz / vs
};

struct SmallLds {
  half8 qt[8][64];               // Q^T operand of k-step s, lane l (shared by the wavefronts)
  float qs[kWaves][kSmRows];     // the wavefronts' shares of each row's q sum
  SmallTileLds tile[kWaves];
  uint32_t wbits[kWaves][kMaxTilesPerSplit / kWaves];   // window-token bits of each of the wavefront's tiles
  SmallSlot ring[kWaves][kSmRing];
  int32_t wbound[kWaves][2];     // folded DecodeOnly bounds: a sink position not staged, highest recent one
};

struct SmallCombineLds {
  float o[kWaves][kSmRows][kHeadDim];
  float m[kWaves][kSmRows];
  float l[kWaves][kSmRows];
};

constexpr size_t kSmallLdsBytes = sizeof(SmallCombineLds) > sizeof(SmallLds)
                                      ? (sizeof(SmallCombineLds) > sizeof(FreshLds) ? sizeof(SmallCombineLds)
                                                                                    : sizeof(FreshLds))
                                      : (sizeof(SmallLds) > sizeof(FreshLds) ? sizeof(SmallLds) : sizeof(FreshLds));
static_assert(kSmallLdsBytes <= 80 * 1024, "two workgroups' LDS must fit the CU's 160 KiB");

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(n), expcnt and lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

constexpr int kSmallLoadsPerTile = 6;

// Copy one tile's bytes into a ring slot with six buffer loads to LDS per
// lane (each lane's 16 or 4 bytes land at slot offset + lane * size).  Every
// lane issues them whatever the tile holds (an invalid tile reads page 0,
// positions past the history read the tile's first row; without an arena the
// owner loads read nothing and leave zeros), so each wait counts exactly
// whole tiles.  Buffer loads count only in vmcnt.
__device__ __forceinline__ void load_small_tile(const DecodeArgs& a, SmallSlot& slot, int page, int p0, int prefix,
                                                int kvh, int lane) {
  const int c = lane & 15, G = lane >> 4;
  const bool tile_ok = p0 < prefix && page >= 0;
  const int pgc = tile_ok ? page : 0;
  const int prow0 = (int)fast_mod((uint32_t)p0, a.bs_div);
  const int nrow = tile_ok ? min(kTile, prefix - p0) : 0;       // rows of the tile inside the history
  auto row_of = [&](int t) { return t < nrow ? prow0 + t : 0; };
  // Records end at the last code byte of the page's last row of this kv head.
  const uint32_t krec = (uint32_t)((int64_t)(a.block_size - 1) * a.k_tok + kKCodeOff + kCodeBytes);
  const uint32_t vrec = (uint32_t)((int64_t)(a.block_size - 1) * a.v_tok + kCodeBytes);
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.k_cache + (int64_t)pgc * a.k_page + (int64_t)kvh * a.k_head), (short)0, krec, 0x00020000);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.v_cache + (int64_t)pgc * a.v_page + (int64_t)kvh * a.v_head), (short)0, vrec, 0x00020000);
  const int kofs = kKCodeOff + 32 * (G & 1) + 16 * (G >> 1);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tk = 8 * (c >> 2) + 4 * h + (c & 3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void*)&slot.kc[h][0], 16, row_of(tk) * (int)a.k_tok + kofs,
                                             0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int tk = 16 * i + (lane >> 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_void*)&slot.vc[16 * i][0], 16,
                                             row_of(tk) * (int)a.v_tok + 16 * (lane & 3), 0, 0, 0);
  }
  __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void*)&slot.meta[0], 4,
                                           row_of(lane >> 1) * (int)a.k_tok + 4 * (lane & 1), 0, 0, 0);
  // owner tags of the tile's seats (page % rows, prow0 .. prow0 + 31); no arena: zero records
  const bool arena = a.stage_rows > 0;
  const int64_t seat0 = arena ? (int64_t)fast_mod((uint32_t)pgc, a.rows_div) * a.block_size + prow0 : 0;
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc(
      arena ? (void*)(a.owner + seat0) : (void*)a.k_cache, (short)0, arena ? (uint32_t)(kTile * 8) : 0u,
      0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(orr, (lds_void*)&slot.own[0], 4, 4 * lane, 0, 0, 0);
}

// x op x^16 and x op x^32 in every lane (gfx950 permlane swaps).
template <bool kMax>
__device__ __forceinline__ float across_groups(float x) {
  auto op = [](float u, float v) { return kMax ? fmaxf(u, v) : u + v; };
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  x = op(__int_as_float(s16[0]), __int_as_float(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return op(__int_as_float(s32[0]), __int_as_float(s32[1]));
}

__device__ __forceinline__ float ror8_add(float x) {
  return x + dpp_move<0x128>(x);          // row_ror:8: lane c takes lane (c + 8) % 16 of its row
}

// kFold: the DecodeOnly read whose window bounds the kernel finds itself
// (a.win_fold); the other instance runs every other small-row launch.
template <bool kFold>
__global__ __launch_bounds__(256, 2) void paged_decode_split_small_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  int bx, item;
  const ItemInfo it = find_item(a, (int)blockIdx.x, item, bx);
  const int rows = it.nq * a.group;
  if (it.nq <= 0 || blockIdx.z != 0) return;
  if (bx >= it.nsplit) {                  // the fresh-token workgroup, or none for this item
    if (a.fresh_block && bx == it.nsplit)
      fresh_partial(a, it, item, 0, *reinterpret_cast<FreshLds*>(smem_raw), (int)threadIdx.x);
    return;
  }
  // history splits dispatched as 0, S - 1, S - 2, ..., 1 (the window steps first)
  const int split = bx == 0 ? 0 : it.nsplit - bx;
  const int prefix = it.prefix;
  const int steps = (prefix + kStepTok - 1) / kStepTok;
  const int rem = steps % it.nsplit;
  const int fresh_split = steps < it.nsplit ? steps : (rem != 0 ? it.nsplit - 1 : it.nsplit / 2);
  const bool fresh_here = a.fresh && !a.fresh_block && split == fresh_split;
  if (split >= steps) {
    if (fresh_here) fresh_partial(a, it, item, 0, *reinterpret_cast<FreshLds*>(smem_raw), (int)threadIdx.x);
    return;
  }
  SmallLds& S = *reinterpret_cast<SmallLds*>(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, G = lane >> 4, t32 = lane & 31;
  const int kvh = it.kvh;
  const int nsplit = it.nsplit;
  // Wave w walks the steps of split (split + w * nsplit / 4) mod nsplit (for
  // items of at least 8 splits, none of them empty), so that the tiles of
  // one step (a window step's among them) go to four workgroups and no CU
  // loads more than one window tile's images per step; the waves are
  // independent, so their tile counts may differ by one.
  const int sw0 = split + ((nsplit >= 8 && nsplit <= steps) ? w * (nsplit / 4) : 0);
  const int sw = sw0 >= nsplit ? sw0 - nsplit : sw0;
  const int nst = (steps - 1 - sw) / nsplit + 1;
  const bool arena = a.stage_rows > 0;
  int win_head = 0, win_tail = 0;
  if (a.win) {
    typedef __attribute__((address_space(4))) const int32_t const_i32;
    const const_i32* wb = (const const_i32*)a.win;
    win_head = wb[2 * it.req];
    win_tail = wb[2 * it.req + 1];
  }

  // ---- requests before any wait: the query features of this wavefront's
  // two k-steps and the wavefront's page of each step (lane k: step k) ----
  const int r = c & (kSmRows - 1);
  const bool row_ok = r < rows;
  floatx4 x[4];
  {
    // k-steps 2w, 2w + 1 of lane group G: features 128 (G & 1) + 64 (G >> 1) + 16w .. + 15
    const int row = row_ok ? r : 0;
    const int j = row / a.group, h = kvh * a.group + (row - j * a.group);
    const floatx4* src = reinterpret_cast<const floatx4*>(
        a.q + ((int64_t)(it.qa + j) * a.num_heads + h) * kHeadDim + 128 * (G & 1) + 64 * (G >> 1) + 16 * w);
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = src[k];
  }
  __builtin_amdgcn_sched_barrier(0);
  int pgv;
  {
    const int32_t* bt_row = a.block_table + (int64_t)it.req * a.bt_stride;
    const uint32_t tok0 = (uint32_t)(sw + nsplit * lane) * kStepTok + kTile * w;
    const uint32_t pidx = fast_div(tok0, a.bs_div);
    const bool ok = lane < nst && (int)tok0 < prefix && (int)pidx < a.bt_cols;
    const int p = bt_row[ok ? pidx : 0];
    pgv = ok ? p : -1;
  }
  auto tile_page = [&](int k) {
    const int p = __builtin_amdgcn_readlane(pgv, k);
    return (p >= 0 && p < a.num_pages) ? p : -1;
  };
  auto tile_pos = [&](int k) { return (sw + nsplit * k) * kStepTok + kTile * w; };
  // Processing order: the wavefront's last tile first (the one that holds the
  // recent window when any does, so its window pass can run while the next
  // tiles are in flight), then tiles 0, 1, ...; ring slot i % kSmRing holds the
  // i-th tile processed.
  auto tile_of = [&](int i) { return nst > 1 ? (i == 0 ? nst - 1 : i - 1) : i; };
  // Folded DecodeOnly bounds (the bounds kernel's rule, one sink and one
  // recent position per thread): the owner tags are requested here, before
  // the tiles, and compared after the tile requests, so their round trip
  // overlaps the Q^T set-up and the first tiles' flight.
  const bool fold = kFold;
  const bool sink_len = fold && a.win_sink > 0 && prefix > a.win_sink;
  const int rlo = max(prefix - a.win_recent, 0);
  const int ps = tid, pr = prefix - 1 - tid;
  bool chk_s = false, chk_r = false;
  int pg_s = -1, pg_r = -1;
  int64_t own_s = -1, own_r = -1;
  uint32_t pis = 0, pir = 0;
  if (fold) {
    const int32_t* bt_row = a.block_table + (int64_t)it.req * a.bt_stride;
    chk_s = sink_len && ps < a.win_sink;
    chk_r = pr >= rlo;
    pis = fast_div((uint32_t)(chk_s ? ps : 0), a.bs_div);
    pir = fast_div((uint32_t)(chk_r ? pr : 0), a.bs_div);
    if (chk_s && (int)pis < a.bt_cols) pg_s = bt_row[pis];
    if (chk_r && (int)pir < a.bt_cols) pg_r = bt_row[pir];
  }
  // The pages of the first two tiles, read (after the page loads above) into
  // scalar registers before the owner tags are requested, so that the tile
  // requests below never wait for those.
  int page_i0 = -1, page_i1 = -1;
  if (fold) {
    page_i0 = tile_page(tile_of(0));
    page_i1 = nst > 1 ? tile_page(tile_of(1)) : -1;
  }
  __builtin_amdgcn_sched_barrier(0);
  if (fold) {
    auto seat = [&](int page, int pos, uint32_t pi) {
      return (int64_t)fast_mod((uint32_t)page, a.rows_div) * a.block_size + (pos - (int)pi * a.block_size);
    };
    if (pg_s >= 0 && pg_s < a.num_pages) own_s = a.owner[seat(pg_s, ps, pis)];
    if (pg_r >= 0 && pg_r < a.num_pages) own_r = a.owner[seat(pg_r, pr, pir)];
  }
  auto issue = [&](int i) {
    const int k = tile_of(i);
    const int page = (fold && i < 2) ? (i == 0 ? page_i0 : page_i1) : tile_page(k);
    load_small_tile(a, S.ring[w][i % kSmRing], page, tile_pos(k), prefix, kvh, lane);
  };

  // ---- Q^T operands (column c: high part of row c, or low part of row c - 8)
  // of k-steps 2w and 2w + 1 into LDS, and the wavefront's share of the q sums ----
  {
    const bool lo = c >= kSmRows;
#pragma unroll
    for (int aa = 0; aa < 2; ++aa) {
      half8 v;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int f = 4 * aa + (u >> 1) + 8 * (u & 1);
        const float xq = x[f >> 2][f & 3];
        const _Float16 hi = (_Float16)xq;
        const _Float16 lw = (_Float16)(xq - (float)hi);
        v[u] = row_ok ? (lo ? lw : hi) : (_Float16)0.f;
      }
      S.qt[2 * w + aa][lane] = v;
    }
    float qs = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) qs += (x[k][0] + x[k][1]) + (x[k][2] + x[k][3]);
    qs = across_groups<false>(qs);
    if (lane < kSmRows) S.qs[w][lane] = row_ok ? qs : 0.f;
  }
  // the first two tiles (the page reads above are complete by now)
  issue(0);
  if (nst > 1) issue(1);
  if (fold) {
    // a position checked is staged when its page is in range and owns the seat
    const bool bad_s = chk_s && !(pg_s >= 0 && pg_s < a.num_pages && own_s == (int64_t)pg_s);
    const bool bad_r = chk_r && !(pg_r >= 0 && pg_r < a.num_pages && own_r == (int64_t)pg_r);
    int h = bad_r ? pr : -1;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) h = max(h, __shfl_xor(h, o, 64));
    const bool any_s = __ballot(bad_s) != 0ull;
    if (lane == 0) {
      S.wbound[w][0] = any_s ? 1 : 0;
      S.wbound[w][1] = h;
    }
  }
  lds_barrier();
  const float qsum = (S.qs[0][r] + S.qs[1][r]) + (S.qs[2][r] + S.qs[3][r]);
  if (fold) {
    int sb = 0, hb = -1;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      sb |= S.wbound[k][0];
      hb = max(hb, S.wbound[k][1]);
    }
    win_head = (sink_len && sb == 0) ? a.win_sink : 0;
    const int t0 = max(prefix - a.win_recent, win_head);
    win_tail = hb >= t0 ? hb + 1 : t0;
  }

  floatx4 acc[16];                 // O^T tile n = 4q + 2mh + b
#pragma unroll
  for (int n = 0; n < 16; ++n) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff();
  float l_run = 0.f, z_run = 0.f, ps_run = 0.f;     // this lane's share (its 8 tokens) of row r's sums
  const uint32_t ones16 = magic_ones();
  const uint32_t e2 = 2u * (uint32_t)(c & 1);
  const uint32_t ls0 = 8u - e2, rs0 = e2, ls1 = 4u - e2, rs1 = 4u + e2;
  SmallTileLds& T = S.tile[w];
  constexpr int kSlotTok[8] = {0, 2, 1, 3, 4, 6, 5, 7};   // PV k-slot u holds token 8G + kSlotTok[u]

  // The tile's row maximum mb (this lane's row) against the running maximum:
  // raised lazily (only when it grows by more than 2^kLazy, or at once when
  // `eager`), rescaling the accumulators and sums; returns the exponent base.
  auto raise_max = [&](float mb, bool eager) {
    mb = across_groups<true>(mb);
    const bool need = mb > m_run + (eager ? 0.f : kLazy);
    const bool resc = need && m_run != -__builtin_inff();
    if (__ballot(resc)) {
      const float alpha = resc ? exp2_raw(m_run - mb) : 1.f;
#pragma unroll
      for (int n = 0; n < 16; ++n) acc[n] *= alpha;
      l_run *= alpha;
      z_run *= alpha;
      ps_run *= alpha;
    }
    if (need) m_run = mb;
    return m_run == -__builtin_inff() ? 0.f : m_run;
  };

  // One tile of INT2 tokens.  Window-owned tokens (bits of wm) are left out
  // here (score -inf, no weight) and added by the window pass after the loop.
  auto tile_body = [&](const SmallSlot& L, int i, int nvalid, uint32_t wm) {
    // The tile processed i + 2-th goes into the slot the one before this left
    // (its LDS reads are complete: lgkmcnt(0)).
    if (i + 2 < nst) {
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("" ::: "memory");
      issue(i + 2);
    }
    // A tile without INT2 tokens (every valid token window-owned, or none
    // valid) adds nothing here: all its scores would be masked out.
    if ((tile_valid(nvalid) & ~wm) == 0u) return;
    // ---- token parameters (lane t32 < 32) and the byte-transposed V codes ----
    bool big;
    {
      const bool used = t32 < nvalid && !((wm >> t32) & 1u);
      const u32x2 meta = L.meta[t32];
      const float ksc = f16_bits_to_f32(meta[0]);
      const float kz = f16_bits_to_f32(meta[0] >> 16);
      const float vsc = f16_bits_to_f32(meta[1]);
      const float vz = f16_bits_to_f32(meta[1] >> 16);
      if (lane < kTile) {
        const float rvs = used ? 1.f / vsc : 0.f;
        T.prm[0][t32] = used ? 4.f * ksc * a.scale_log2 : 0.f;
        T.prm[1][t32] = used ? (kz - 4.f * ksc) * a.scale_log2 : 0.f;
        T.prm[2][t32] = used ? 0.f : -__builtin_inff();
        T.prm[3][t32] = used ? vsc : 0.f;
        T.prm[4][t32] = rvs;
        T.prm[5][t32] = used ? vz * rvs : 0.f;
      }
      big = __ballot(used && vsc > kLazyVsMax) != 0;
      const int tq = lane & 7, bg = lane >> 3;
      u32x2 vc[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) vc[kk] = *reinterpret_cast<const u32x2*>(&L.vc[4 * tq + kk][8 * bg]);
      uint32_t o0[4], o1[4];
      transpose4(vc[0][0], vc[1][0], vc[2][0], vc[3][0], o0);
      transpose4(vc[0][1], vc[1][1], vc[2][1], vc[3][1], o1);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        T.vt[(8 * bg + kk) * kSmVtRow + tq] = o0[kk];
        T.vt[(8 * bg + 4 + kk) * kSmVtRow + tq] = o1[kk];
      }
    }

    // ---- S^T = K Q^T, both halves ----
    floatx4 sc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
    const u32x4 kc0 = L.kc[0][lane], kc1 = L.kc[1][lane];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const half8 qa0 = S.qt[2 * jj][lane], qa1 = S.qt[2 * jj + 1][lane];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        half8 ka[2];
        k_operands(h == 0 ? kc0[jj] : kc1[jj], ones16, ka);
        sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[0], qa0, sc[h], 0, 0, 0);
        sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[1], qa1, sc[h], 0, 0, 0);
      }
    }
    wave_sync_lds();

    // ---- scores of tokens 8G + 4h + i for row r, the tile's row maximum ----
    float sv[8];
    float mb = -__builtin_inff();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const floatx4 av = *reinterpret_cast<const floatx4*>(&T.prm[0][8 * G + 4 * h]);
      const floatx4 bv = *reinterpret_cast<const floatx4*>(&T.prm[1][8 * G + 4 * h]);
      const floatx4 tmv = *reinterpret_cast<const floatx4*>(&T.prm[2][8 * G + 4 * h]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = ror8_add(sc[h][i]);
        sv[4 * h + i] = fmaf(av[i], v, bv[i] * qsum) + tmv[i];
        mb = fmaxf(mb, sv[4 * h + i]);
      }
    }
    const float m_use = raise_max(mb, big);

    // ---- P' = p * vs in the PV token order ----
    half8 pop;
    {
      const floatx4 vs0 = *reinterpret_cast<const floatx4*>(&T.prm[3][8 * G]);
      const floatx4 vs1 = *reinterpret_cast<const floatx4*>(&T.prm[3][8 * G + 4]);
      const floatx4 rv0 = *reinterpret_cast<const floatx4*>(&T.prm[4][8 * G]);
      const floatx4 rv1 = *reinterpret_cast<const floatx4*>(&T.prm[4][8 * G + 4]);
      const floatx4 zv0 = *reinterpret_cast<const floatx4*>(&T.prm[5][8 * G]);
      const floatx4 zv1 = *reinterpret_cast<const floatx4*>(&T.prm[5][8 * G + 4]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int t = kSlotTok[u];
        const float p = exp2_raw(sv[t] - m_use);
        const float vs = t < 4 ? vs0[t] : vs1[t - 4];
        const float rv = t < 4 ? rv0[t] : rv1[t - 4];
        const float zv = t < 4 ? zv0[t] : zv1[t - 4];
        const _Float16 hp = (_Float16)(p * vs);
        pop[u] = hp;
        const float wh = (float)hp;
        ps_run += wh;
        l_run = fmaf(wh, rv, l_run);
        z_run = fmaf(wh, zv, z_run);
      }
    }

    // ---- O^T += V^T P'^T over the 16 feature tiles ----
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        const int brow = 16 * q + 8 * mh + (c >> 1);
        const u32x2 d = *reinterpret_cast<const u32x2*>(&T.vt[brow * kSmVtRow + 2 * G]);
        const half8 v0 = as_half8(pair_lo(d[0], ls0, ones16), pair_hi(d[0], rs0, ones16),
                                  pair_lo(d[1], ls0, ones16), pair_hi(d[1], rs0, ones16));
        const half8 v1 = as_half8(pair_lo(d[0], ls1, ones16), pair_hi(d[0], rs1, ones16),
                                  pair_lo(d[1], ls1, ones16), pair_hi(d[1], rs1, ones16));
        acc[4 * q + 2 * mh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v0, pop, acc[4 * q + 2 * mh], 0, 0, 0);
        acc[4 * q + 2 * mh + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v1, pop, acc[4 * q + 2 * mh + 1], 0, 0, 0);
      }
    }
  };

  // window-owned tokens of tile k, from its owner tags (bit t: token t)
  auto window_bits = [&](int k, int own) -> uint32_t {
    if (!arena) return 0u;
    const int page = tile_page(k);
    const int pos = tile_pos(k) + t32;
    const bool st = page >= 0 && pos < prefix && (pos < win_head || pos >= win_tail) && own == page;
    return (uint32_t)__ballot(st);
  };

  // The window tokens of tile k: K from the fp16 image (high and low parts),
  // V from the V image (high and low parts), probabilities p / 4 into the
  // same accumulators.
  auto window_tile = [&](int k) {
    const int page = tile_page(k);
    const int prow0 = (int)fast_mod((uint32_t)tile_pos(k), a.bs_div);
    const uint32_t wm = __builtin_amdgcn_readfirstlane(S.wbits[w][k]);
    const int64_t img = image_index(a, page, prow0, kvh);
    const u32x4* kimg = reinterpret_cast<const u32x4*>(a.kimg + img * kKImgHalfs);
    const int il = 8 * (c >> 2) + (c & 3) + 32 * (G & 1);      // image lane of half 0's token
    // Both parts of both halves at once, zero for tokens outside the window.
    u32x4 khi[2][8], klo[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool wl = (wm >> (8 * (c >> 2) + 4 * h + (c & 3))) & 1u;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        khi[h][s] = wl ? kimg[(8 * (G >> 1) + s) * 64 + il + 4 * h] : u32x4{};
        klo[h][s] = wl ? kimg[kImgHalfs / 8 + (8 * (G >> 1) + s) * 64 + il + 4 * h] : u32x4{};
      }
    }
    floatx4 sc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const half8 qa = S.qt[s][lane];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, khi[h][s]), qa, sc[h], 0, 0, 0);
    }
    // the V image's high part (feature tile n = 4q + 2mh + b: chunk (q, b,
    // G >> 1), lane 16 mh + c + 32 (G & 1)) requested as soon as K's high
    // parts are used, into their registers, and its low part likewise after
    // K's low parts (the barriers keep the loads below those MFMAs)
    __builtin_amdgcn_sched_barrier(0);
    const half8* vimg = reinterpret_cast<const half8*>(a.vimg + img * kVImgHalfs);
    auto vimg_index = [&](int n) {
      return (((n >> 2) * 2 + (n & 1)) * 2 + (G >> 1)) * 64 + 16 * ((n >> 1) & 1) + c + 32 * (G & 1);
    };
    half8 vv[16], vl[16];
#pragma unroll
    for (int n = 0; n < 16; ++n) vv[n] = vimg[vimg_part(vimg_index(n), 0)];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const half8 qa = S.qt[s][lane];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, klo[h][s]), qa, sc[h], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int n = 0; n < 16; ++n) vl[n] = vimg[vimg_part(vimg_index(n), 1)];
    float sv[8];
    float mb = -__builtin_inff();
    const uint32_t wb = wm >> (8 * G);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = ror8_add(sc[h][i]) * a.scale_log2;
        sv[4 * h + i] = ((wb >> (4 * h + i)) & 1u) ? v : -__builtin_inff();
        mb = fmaxf(mb, sv[4 * h + i]);
      }
    const float m_use = raise_max(mb, false);
    half8 pwop;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const _Float16 hw = (_Float16)(0.25f * exp2_raw(sv[kSlotTok[u]] - m_use));
      pwop[u] = hw;
      l_run = fmaf(4.f, (float)hw, l_run);
    }
#pragma unroll
    for (int n = 0; n < 16; ++n) acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv[n], pwop, acc[n], 0, 0, 0);
#pragma unroll
    for (int n = 0; n < 16; ++n) acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl[n], pwop, acc[n], 0, 0, 0);
    };

  uint64_t wtiles = 0;             // tiles k of this wavefront that hold window tokens
  // One tile: wait for its loads, leaving the next one's in flight (the one
  // after is requested in the tile body); returns its window bits.
  auto step_tile = [&](int i) -> uint32_t {
    if (i + 1 < nst)
      wait_vmcnt<kSmallLoadsPerTile>();
    else
      wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    const SmallSlot& L = S.ring[w][i % kSmRing];
    const int k = tile_of(i);
    const int page = tile_page(k);
    const int nvalid = page >= 0 ? min(kTile, max(prefix - tile_pos(k), 0)) : 0;
    const uint32_t wm = window_bits(k, (int)L.own[t32][0]);
    if (wm != 0u) {
      wtiles |= 1ull << k;
      S.wbits[w][k] = wm;
    }
    tile_body(L, i, nvalid, wm);
    return wm;
  };
  int i0 = 0;
  if (nst > 1) {
    // The first tile processed (the wavefront's last) and, at once, its
    // window tokens, while the next two tiles arrive; peeled off the loop so
    // that the window pass's registers stay out of it.
    if (step_tile(0) != 0u) {
      wtiles &= ~(1ull << (nst - 1));
      window_tile(nst - 1);
    }
    i0 = 1;
  }
#pragma unroll 1
  for (int i = i0; i < nst; ++i) step_tile(i);

  // ---- the window tiles not done yet ----
#pragma unroll 1
  while (wtiles != 0ull) {
    const int k = __builtin_ctzll(wtiles);
    wtiles &= wtiles - 1;
    window_tile(k);
  }

  // ---- the four wavefronts' rows combined into the split's partial ----
  l_run = across_groups<false>(l_run);
  z_run = across_groups<false>(z_run);
  ps_run = across_groups<false>(ps_run);
  lds_barrier();                                   // every wavefront is past its last tile
  SmallCombineLds& C = *reinterpret_cast<SmallCombineLds*>(smem_raw);
  if (lane < kSmRows) C.m[w][lane] = m_run;
  lds_barrier();
  float M = C.m[0][r];
#pragma unroll
  for (int ww = 1; ww < kWaves; ++ww) M = fmaxf(M, C.m[ww][r]);
  const float alpha = m_run == -__builtin_inff() ? 0.f : exp2_raw(m_run - M);
  // sum_t p (c vs + vz) = 4 * acc - 4 * sum_t P' + sum_t p vz, scaled to the common maximum
  const float off = alpha * (z_run - 4.f * ps_run);
  const float a4 = 4.f * alpha;
  if (c < kSmRows) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        const floatx4 b0 = acc[4 * q + 2 * mh], b1 = acc[4 * q + 2 * mh + 1];
        float* dst = &C.o[w][c][64 * q + 32 * mh + 8 * G];
        *reinterpret_cast<floatx4*>(dst) =
            floatx4{fmaf(a4, b0[0], off), fmaf(a4, b0[1], off), fmaf(a4, b1[0], off), fmaf(a4, b1[1], off)};
        *reinterpret_cast<floatx4*>(dst + 4) =
            floatx4{fmaf(a4, b0[2], off), fmaf(a4, b0[3], off), fmaf(a4, b1[2], off), fmaf(a4, b1[3], off)};
      }
    }
    if (G == 0) C.l[w][c] = alpha * l_run;
  }
  lds_barrier();
  // wavefront w: features 64w .. 64w + 63 of every row; lane: row lane / 8, 8 features
  const int nrow = min(kSmRows, rows);
  float* part = a.ws + partial_index(a, it, split, 0) * kPartialFloats;
  {
    const int row = lane >> 3, f = 64 * w + 8 * (lane & 7);
    if (row < nrow) {
      floatx4 s0 = *reinterpret_cast<const floatx4*>(&C.o[0][row][f]);
      floatx4 s1 = *reinterpret_cast<const floatx4*>(&C.o[0][row][f + 4]);
#pragma unroll
      for (int ww = 1; ww < kWaves; ++ww) {
        s0 += *reinterpret_cast<const floatx4*>(&C.o[ww][row][f]);
        s1 += *reinterpret_cast<const floatx4*>(&C.o[ww][row][f + 4]);
      }
      *reinterpret_cast<floatx4*>(part + row * kHeadDim + f) = s0;
      *reinterpret_cast<floatx4*>(part + row * kHeadDim + f + 4) = s1;
    }
    if (w == 0 && lane < nrow) {
      part[kPartO + lane] = M;
      part[kPartO + kRows + lane] = (C.l[0][lane] + C.l[1][lane]) + (C.l[2][lane] + C.l[3][lane]);
    }
  }
  if (fresh_here) {
    __syncthreads();
    const int ftid = 64 * w + (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    fresh_partial(a, it, item, 0, *reinterpret_cast<FreshLds*>(smem_raw), ftid);
  }
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
  const int steps = (it.prefix + kStepTok - 1) / kStepTok;
  const int hs = min((int)it.nsplit, steps);      // history partials 0 .. hs - 1
  const int P = hs + a.fresh;                     // partial hs is the fresh one (slot nsplit)
  const float* base = a.ws + partial_index(a, it, 0, rt) * kPartialFloats;
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
      const float* pp = base + (p < hs ? p : it.nsplit) * pstride;
      mreg[k] = pp[kPartO + r];
      lreg[k] = pp[kPartO + kRows + r];
    }
  }
  floatx4 x[kMergeBatch];
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const int p = sg + kMergeGroups * k;
    x[k] = p < P ? *reinterpret_cast<const floatx4*>(base + (p < hs ? p : it.nsplit) * pstride +
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
      x[k] = p < P ? *reinterpret_cast<const floatx4*>(base + (p < hs ? p : it.nsplit) * pstride +
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

// Merge for launches with few partials per item (at most kSmallP, e.g. many
// requests with a handful of splits each): one thread per four features of a
// row loads every partial's slice and (m, l) itself, so the combine needs no
// LDS round.  256 threads = 16 row-quarters x 16 threads.
constexpr int kSmallP = 32;

__global__ __launch_bounds__(256) void paged_decode_merge_small_kernel(DecodeArgs a) {
  const int tid = threadIdx.x;
  const int rq = blockIdx.x * 16 + (tid >> 4);
  const int r = rq >> 2, qd = rq & 3;
  const int item = blockIdx.y;
  const int rt = blockIdx.z;
  const ItemInfo it = a.items[item];
  const int rows = it.nq * a.group;
  const int row = rt * kRows + r;
  if (it.nq <= 0 || r >= kRows || row >= rows) return;
  const int steps = (it.prefix + kStepTok - 1) / kStepTok;
  const int hs = min((int)it.nsplit, steps);
  const int P = hs + a.fresh;
  const float* base = a.ws + partial_index(a, it, 0, rt) * kPartialFloats;
  const int64_t pstride = (int64_t)a.row_tiles * kPartialFloats;
  const int f0 = 64 * qd + 4 * (tid & 15);
  float m[kSmallP], l[kSmallP];
  floatx4 x[kSmallP];
#pragma unroll
  for (int p = 0; p < kSmallP; ++p) {
    m[p] = -__builtin_inff();
    l[p] = 0.f;
    x[p] = floatx4{};
    if (p < P) {
      const float* pp = base + (p < hs ? p : it.nsplit) * pstride;
      m[p] = pp[kPartO + r];
      l[p] = pp[kPartO + kRows + r];
      x[p] = *reinterpret_cast<const floatx4*>(pp + r * kHeadDim + f0);
    }
  }
  float mx = -__builtin_inff();
#pragma unroll
  for (int p = 0; p < kSmallP; ++p) mx = fmaxf(mx, m[p]);
  floatx4 acc = floatx4{};
  float ls = 0.f;
#pragma unroll
  for (int p = 0; p < kSmallP; ++p) {
    const float wgt = (m[p] == -__builtin_inff()) ? 0.f : exp2f(m[p] - mx);
    acc += wgt * x[p];
    ls = fmaf(wgt, l[p], ls);
  }
  const int j = row / a.group;
  const int h = it.kvh * a.group + (row - j * a.group);
  const float inv = ls > 0.f ? 1.f / ls : 0.f;
  *reinterpret_cast<floatx4*>(a.out + ((int64_t)(it.qa + j) * a.num_heads + h) * kHeadDim + f0) = acc * inv;
}

// Merge with the output rotation (the reference's `out @ R_v^T`,
// backend.py:293-295) and the cast to the model dtype fused in: one
// 1024-thread block per (output row, quarter of the output features) of an
// item.  Every load goes out before any wait: the block's 64 columns of R_v^T
// (wave w: rotated features 16w .. 16w + 15, lane: one output feature), every
// partial's (m, l) (thread per partial) and the partial rows (wave w: partials
// w, w + 16, ..., lane: four rotated features).  The block LSE-combines the
// row over all 256 rotated features, normalises it, multiplies it by its
// columns of R_v^T (the sixteen waves' sums added in wave order) and writes
// fp32 or bf16 (RNE).
constexpr int kRotThreads = 1024;
constexpr int kRotWaves = kRotThreads / 64;
constexpr int kRotBatch = 16;                    // partial rows per thread per round

__global__ __launch_bounds__(kRotThreads) void paged_decode_merge_rotate_kernel(
    DecodeArgs a, const float* __restrict__ rot_t, void* __restrict__ out, int64_t out_stride, int out_bf16) {
  __shared__ float wpart[kMaxPartials];
  __shared__ float red[2][kRotWaves];
  __shared__ floatx4 osum[kRotWaves][64];
  __shared__ __attribute__((aligned(16))) float orow[kHeadDim];
  __shared__ float csum[kRotWaves][64];
  static_assert(kMaxPartials <= kRotThreads, "one partial per thread");
  // blockIdx.x = (r & 7) + 8 qd + 32 (r >> 3): workgroups are dealt to the 8
  // XCDs by linear id mod 8, so the four quarter blocks of row r, which all
  // read the row's every partial, share one XCD and its L2.
  const int qd = (blockIdx.x >> 3) & 3;
  const int r = (blockIdx.x & 7) + 8 * (blockIdx.x >> 5);
  const int item = blockIdx.y;
  const int rt = blockIdx.z;
  const ItemInfo it = a.items[item];
  const int rows = it.nq * a.group;
  const int row = rt * kRows + r;
  if (it.nq <= 0 || row >= rows) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int steps = (it.prefix + kStepTok - 1) / kStepTok;
  const int hs = min((int)it.nsplit, steps);
  const int P = hs + a.fresh;
  const float* base = a.ws + partial_index(a, it, 0, rt) * kPartialFloats;
  const int64_t pstride = (int64_t)a.row_tiles * kPartialFloats;
  auto partial = [&](int p) { return base + (p < hs ? p : it.nsplit) * pstride; };

  // ---- every load of the first round ----
  float rv[kHeadDim / kRotWaves];
  const float* rcol = rot_t + (int64_t)(16 * w) * kHeadDim + 64 * qd + lane;
#pragma unroll
  for (int k = 0; k < kHeadDim / kRotWaves; ++k) rv[k] = rcol[(int64_t)k * kHeadDim];
  float mp = -__builtin_inff(), lp = 0.f;
  if (tid < P) {
    mp = partial(tid)[kPartO + r];
    lp = partial(tid)[kPartO + kRows + r];
  }
  floatx4 x[kRotBatch];
#pragma unroll
  for (int k = 0; k < kRotBatch; ++k) {
    const int p = w + kRotWaves * k;
    x[k] = p < P ? *reinterpret_cast<const floatx4*>(partial(p) + r * kHeadDim + 4 * lane) : floatx4{};
  }

  // ---- partial weights ----
  float mloc = mp;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
  if (lane == 0) red[0][w] = mloc;
  __syncthreads();
  float mx = red[0][0];
#pragma unroll
  for (int ww = 1; ww < kRotWaves; ++ww) mx = fmaxf(mx, red[0][ww]);
  const float wgt = (mp == -__builtin_inff()) ? 0.f : exp2f(mp - mx);
  if (tid < P) wpart[tid] = wgt;
  float lsum = wgt * lp;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lsum += __shfl_xor(lsum, o, 64);
  if (lane == 0) red[1][w] = lsum;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int ww = 0; ww < kRotWaves; ++ww) L += red[1][ww];

  // ---- the row in the rotated domain ----
  floatx4 acc = floatx4{};
#pragma unroll
  for (int k = 0; k < kRotBatch; ++k) {
    const int p = w + kRotWaves * k;
    if (p < P) acc += wpart[p] * x[k];
  }
  for (int p0 = w + kRotWaves * kRotBatch; p0 < P; p0 += kRotWaves * kRotBatch) {
#pragma unroll
    for (int k = 0; k < kRotBatch; ++k) {
      const int p = p0 + kRotWaves * k;
      x[k] = p < P ? *reinterpret_cast<const floatx4*>(partial(p) + r * kHeadDim + 4 * lane) : floatx4{};
    }
#pragma unroll
    for (int k = 0; k < kRotBatch; ++k) {
      const int p = p0 + kRotWaves * k;
      if (p < P) acc += wpart[p] * x[k];
    }
  }
  osum[w][lane] = acc;
  __syncthreads();
  if (w == 0) {
    floatx4 o = osum[0][lane];
#pragma unroll
    for (int ww = 1; ww < kRotWaves; ++ww) o += osum[ww][lane];
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *reinterpret_cast<floatx4*>(&orow[4 * lane]) = o * inv;
  }
  __syncthreads();

  // ---- out[64 qd + lane] = sum_f orow[f] * R_v^T[f][64 qd + lane] ----
  float y = 0.f;
#pragma unroll
  for (int k = 0; k < kHeadDim / kRotWaves; ++k) y = fmaf(orow[16 * w + k], rv[k], y);
  csum[w][lane] = y;
  __syncthreads();
  if (w == 0) {
    float o = csum[0][lane];
#pragma unroll
    for (int ww = 1; ww < kRotWaves; ++ww) o += csum[ww][lane];
    const int j = row / a.group;
    const int h = it.kvh * a.group + (row - j * a.group);
    const int64_t idx = (int64_t)(it.qa + j) * out_stride + (int64_t)h * kHeadDim + 64 * qd + lane;
    if (out_bf16)
      reinterpret_cast<__bf16*>(out)[idx] = (__bf16)o;
    else
      reinterpret_cast<float*>(out)[idx] = o;
  }
}

// DecodeOnly window bounds of the launch chunk's requests (backend.py:514-551):
// win[2r] = head (sink_eff when the request is longer than the sink and every
// seat of its sink pages holds that page, else 0), win[2r + 1] = cut (start of
// the run of staged positions ending at seq - 1 inside [t0, seq), t0 =
// max(seq - recent, head); seq when position seq - 1 is not staged).  With h
// the highest position in [max(seq - recent, 0), seq) that is not staged,
// cut = h + 1 if h >= t0, else t0.  One 256-thread block per request; every
// position is checked by its own thread (block-table entries outside
// [0, num_pages) count as not staged).
constexpr int kBoundsThreads = 256;

__global__ __launch_bounds__(kBoundsThreads) void decode_only_bounds_kernel(DecodeArgs a, int32_t* __restrict__ win,
                                                                            int32_t sink_eff, int32_t recent) {
  __shared__ int32_t sink_bad[kBoundsThreads / 64];
  __shared__ int32_t top_bad[kBoundsThreads / 64];
  const int r = blockIdx.x;
  const ItemInfo it = a.items[r * a.num_kv_heads];
  const int seq = it.prefix;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int32_t* bt_row = a.block_table + (int64_t)it.req * a.bt_stride;
  auto staged = [&](int pos) -> bool {
    const uint32_t pi = fast_div((uint32_t)pos, a.bs_div);
    if ((int)pi >= a.bt_cols) return false;
    const int page = bt_row[pi];
    if (page < 0 || page >= a.num_pages) return false;
    const int64_t seat = (int64_t)fast_mod((uint32_t)page, a.rows_div) * a.block_size +
                         (pos - (int)pi * a.block_size);
    return a.owner[seat] == (int64_t)page;
  };
  const bool sink_len = sink_eff > 0 && seq > sink_eff;
  bool bad_sink = false;
  if (sink_len)
    for (int p = tid; p < sink_eff; p += kBoundsThreads) bad_sink = bad_sink || !staged(p);
  const int lo = max(seq - recent, 0);
  int h = -1;                                   // highest unstaged position of this thread
  for (int p = seq - 1 - tid; p >= lo; p -= kBoundsThreads)
    if (!staged(p)) {
      h = p;
      break;
    }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) h = max(h, __shfl_xor(h, o, 64));
  const bool any_bad = __ballot(bad_sink) != 0ull;
  if (lane == 0) {
    sink_bad[w] = any_bad;
    top_bad[w] = h;
  }
  __syncthreads();
  if (tid == 0) {
    bool sb = false;
    int hb = -1;
#pragma unroll
    for (int k = 0; k < kBoundsThreads / 64; ++k) {
      sb = sb || sink_bad[k];
      hb = max(hb, top_bad[k]);
    }
    const int head = (sink_len && !sb) ? sink_eff : 0;
    const int t0 = max(seq - recent, head);
    win[2 * r] = head;
    win[2 * r + 1] = hb >= t0 ? hb + 1 : t0;
  }
}

int64_t splits_for(int64_t max_history, int tiles_per_split) {
  const int64_t tiles = max_history > 0 ? (max_history + kTile - 1) / kTile : 0;
  return (tiles + tiles_per_split - 1) / tiles_per_split;
}

int32_t requests_per_launch(int32_t num_kv_heads);

// Split workgroups resident at once: two per CU on MI355X's 256 CUs.
constexpr int64_t kResidentSplitWgs = 512;
constexpr int64_t kMaxStepsPerSplit = kMaxTilesPerSplit / kWaves;   // 64: one page-register lane per step

int32_t requests_per_launch(int32_t num_kv_heads) {
  const int32_t r = kMaxInlineItems / num_kv_heads;
  return r > 0 ? r : 0;
}

// Partial slots of one launch chunk (items = requests x kv heads of the
// chunk, one fresh-token slot each).  Explicit tiles per split: every item
// takes the same ceil(tiles / tps) splits.  Automatic (tps = 0): per-item
// split counts from plan_splits, at most one round of resident workgroups
// (or one split per 64 steps of each item, when that is more) and never
// more than the items' steps.
int64_t partial_slots(int64_t items, int64_t max_history, int tiles_per_split) {
  if (tiles_per_split > 0) return items * (splits_for(max_history, tiles_per_split) + 1);
  const int64_t steps = max_history > 0 ? (max_history + kStepTok - 1) / kStepTok : 0;
  const int64_t per64 = items * ((steps + kMaxStepsPerSplit - 1) / kMaxStepsPerSplit);
  const int64_t bound = per64 > kResidentSplitWgs ? per64 : kResidentSplitWgs;
  const int64_t all = items * steps;
  return (all < bound ? all : bound) + items;
}

size_t workspace_floats(int32_t num_requests, int32_t num_kv_heads, int32_t num_heads,
                        int32_t max_query_len, int64_t max_history, int tiles_per_split) {
  const int64_t group = num_heads / num_kv_heads;
  const int64_t tiles_r = (max_query_len * group + kRows - 1) / kRows;
  const int64_t per = requests_per_launch(num_kv_heads);
  const int64_t reqs = num_requests < per ? num_requests : per;     // one launch chunk
  return (size_t)partial_slots(reqs * num_kv_heads, max_history, tiles_per_split) * tiles_r * kPartialFloats;
}

// History splits of each item of a launch chunk (items[0 .. nitems) hold
// qa / nq / prefix / req / kvh), their partial slots (pbase), the launch's
// largest split count and whether each fresh partial gets a workgroup of its
// own.  Explicit tiles per split: S = ceil(tiles / tps) for every item (at
// most its steps).  Automatic: a common number of 128-token steps per split
// T, the smallest that keeps the chunk's history splits within one round of
// resident workgroups (T <= 64, one page-register lane per step), and
// ceil(steps / T) splits per item, so that items of different lengths end
// together.  Returns false when some item needs more than kMaxSplits splits.
bool plan_splits(DecodeArgs& a, unsigned nitems, int64_t max_history, int tiles_per_split, int fresh) {
  int64_t steps[kMaxInlineItems];
  int64_t total = 0, max_steps = 0;
  for (unsigned i = 0; i < nitems; ++i) {
    steps[i] = a.items[i].nq > 0 ? ((int64_t)a.items[i].prefix + kStepTok - 1) / kStepTok : 0;
    total += steps[i];
    max_steps = steps[i] > max_steps ? steps[i] : max_steps;
  }
  // Automatic: the common number T of steps per split, the smallest that
  // keeps the history splits within one round of resident workgroups.  An
  // item whose last step holds at most one tile's tokens may leave that step
  // out of the count when that lowers T (its split then takes T steps and
  // the short one): 8 DecodeOnly reads of 32769 positions (257 steps) take
  // 4 steps per split over 512 workgroups instead of 5 over 416.
  int64_t counted[kMaxInlineItems];
  int64_t total_cut = 0;
  for (unsigned i = 0; i < nitems; ++i) {
    const int64_t r = (int64_t)a.items[i].prefix % kStepTok;
    counted[i] = steps[i] - ((steps[i] > 1 && r != 0 && r <= kTile) ? 1 : 0);
    total_cut += counted[i];
  }
  auto least_t = [&](const int64_t* cnt, int64_t sum) {
    int64_t t = (sum + kResidentSplitWgs - 1) / kResidentSplitWgs;
    for (t = t < 1 ? 1 : t;; ++t) {
      int64_t n = 0;
      for (unsigned i = 0; i < nitems; ++i) n += (cnt[i] + t - 1) / t;
      if (n <= kResidentSplitWgs || t >= kMaxStepsPerSplit) return t;
    }
  };
  int64_t T = 0, S = 0;
  const int64_t* cnt = steps;
  if (tiles_per_split > 0) {
    S = splits_for(max_history, tiles_per_split);
  } else {
    T = least_t(steps, total);
    const int64_t Tc = least_t(counted, total_cut);
    if (Tc < T) {
      T = Tc;
      cnt = counted;
    }
  }
  int64_t slots = 0, max_split = 0;
  bool empty = false;
  for (unsigned i = 0; i < nitems; ++i) {
    int64_t n = tiles_per_split > 0 ? S : (cnt[i] + T - 1) / T;
    if (tiles_per_split == 0) {
      const int64_t lo = (steps[i] + kMaxStepsPerSplit - 1) / kMaxStepsPerSplit;   // one page lane per step
      n = n > lo ? n : lo;
    }
    n = n < steps[i] ? n : steps[i];
    empty = empty || (n == 0 && a.items[i].nq > 0);
    if (n > kMaxSplits) return false;
    a.items[i].nsplit = (int16_t)n;
    a.items[i].pbase = (int32_t)slots;
    slots += n + fresh;
    max_split = n > max_split ? n : max_split;
  }
  a.max_splits = (int32_t)max_split;
  // (a request without history has no split to carry its fresh partial)
  a.fresh_block = fresh && (slots <= kResidentSplitWgs || empty) ? 1 : 0;
  a.nitems = (int32_t)nitems;
  return true;
}

// Cache, block-table and arena checks shared by both entries, then the
// common kernel arguments.  Returns kOk or the error code.
int fill_common(DecodeArgs& a, const float* q_rot, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                const void* k_cache, const void* v_cache, int32_t block_size, int64_t num_pages,
                int64_t k_stride_page, int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                int64_t v_stride_token, int64_t v_stride_head, const int32_t* block_table,
                int64_t block_table_stride, int32_t block_table_cols, int64_t max_history,
                const int64_t* stage_owner, const void* stage_k_image, const void* stage_v_image,
                int32_t stage_rows, float scale, float* out, void* workspace) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_heads <= 0 || num_kv_heads <= 0 || num_kv_heads > kMaxInlineItems || num_heads % num_kv_heads != 0 ||
      max_history < 0 || block_size <= 0 || num_pages <= 0 || block_table_cols < 0 || stage_rows < 0)
    return kErrInvalidArgument;
  if (!q_rot || !k_cache || !v_cache || !out) return kErrInvalidArgument;
  if (max_history > 0 && (!block_table || block_table_cols <= 0)) return kErrInvalidArgument;
  if (stage_rows > 0 && (!stage_owner || !stage_k_image || !stage_v_image)) return kErrInvalidArgument;
  if (stage_rows > 0 && ((reinterpret_cast<uintptr_t>(stage_k_image) & 15) ||
                         (reinterpret_cast<uintptr_t>(stage_v_image) & 15)))
    return kErrInvalidArgument;
  if (block_size % kTile != 0 || k_stride_head < kKCodeOff + kCodeBytes || v_stride_head < kCodeBytes ||
      (k_stride_head & 15) || (k_stride_token & 15) || (k_stride_page & 15) || (v_stride_head & 7) ||
      (v_stride_token & 7) || (v_stride_page & 7) || (reinterpret_cast<uintptr_t>(k_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(v_cache) & 7))
    return kErrUnsupportedGeometry;
  a.q = q_rot;
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
  return kOk;
}

std::atomic<uint64_t> g_split_lds_set[4] = {{0}, {0}, {0}, {0}};

int set_split_lds() {
  const void* k[4] = {reinterpret_cast<const void*>(paged_decode_split_kernel<false>),
                      reinterpret_cast<const void*>(paged_decode_split_kernel<true>),
                      reinterpret_cast<const void*>(paged_decode_split_small_kernel<false>),
                      reinterpret_cast<const void*>(paged_decode_split_small_kernel<true>)};
  const size_t bytes[4] = {kLdsBytes, kLdsBytes, kSmallLdsBytes, kSmallLdsBytes};
  for (int i = 0; i < 4; ++i) {
    const int rc = set_dynamic_lds(k[i], (int)bytes[i], g_split_lds_set[i]);
    if (rc != kOk) return rc;
  }
  return kOk;
}

// Workgroups of the launch's split grid (one per history split of each
// item, plus one per item for the fresh partial when it has its own).
unsigned split_workgroups(const DecodeArgs& a) {
  int64_t n = 0;
  for (int i = 0; i < a.nitems; ++i) n += a.items[i].nsplit + a.fresh_block;
  return (unsigned)n;
}

// Split kernel of a launch chunk: the small-row kernel when no item has more
// than 8 rows; else the cooperative kernel, with the mid-step load issue when
// some item has more 128-token steps than it has splits.
void launch_split(const DecodeArgs& a, unsigned nitems, dim3 grid, hipStream_t stream) {
  bool multi = false;
  int64_t max_rows = 0;
  for (unsigned i = 0; i < nitems; ++i) {
    if (a.items[i].nq <= 0) continue;
    const int64_t steps = ((int64_t)a.items[i].prefix + kStepTok - 1) / kStepTok;
    if (steps > a.items[i].nsplit) multi = true;
    const int64_t r = (int64_t)a.items[i].nq * a.group;
    max_rows = r > max_rows ? r : max_rows;
  }
  // (a folded DecodeOnly launch has at most 8 rows per item: oscar_decode_only
  // folds only then)
  if (max_rows <= kSmRows) {
    if (a.win_fold)
      hipLaunchKernelGGL(paged_decode_split_small_kernel<true>, grid, dim3(256), kSmallLdsBytes, stream, a);
    else
      hipLaunchKernelGGL(paged_decode_split_small_kernel<false>, grid, dim3(256), kSmallLdsBytes, stream, a);
  } else if (multi)
    hipLaunchKernelGGL((paged_decode_split_kernel<true>), grid, dim3(256), kLdsBytes, stream, a);
  else
    hipLaunchKernelGGL((paged_decode_split_kernel<false>), grid, dim3(256), kLdsBytes, stream, a);
}

// Merge blocks per feature quarter: one per row of a row tile that can hold
// rows (a launch's longest request fills at most this many).
int merge_rows(int64_t rows) { return (int)(rows < kRows ? rows : kRows); }

// The merge of one launch chunk: the per-thread combine when every item has
// at most kSmallP partials, else one block per (row, feature quarter).
struct OutRotation {
  const float* rot_t;     // R_v^T [D][D], or null: rotated-V-domain fp32 output in a.out
  void* out;              // [tokens][out_stride] fp32 or bf16
  int64_t out_stride;     // elements per token
  int32_t out_bf16;
};

int launch_merge(const DecodeArgs& a, int64_t max_rows, unsigned nitems, const OutRotation& orot,
                 hipStream_t stream) {
  const int mr = merge_rows(max_rows);
  if (orot.rot_t != nullptr) {
    dim3 grid((unsigned)(32 * ((mr + 7) / 8)), nitems, (unsigned)a.row_tiles);
    hipLaunchKernelGGL(paged_decode_merge_rotate_kernel, grid, dim3(kRotThreads), 0, stream, a, orot.rot_t, orot.out,
                       orot.out_stride, (int)orot.out_bf16);
  } else if (a.max_splits + a.fresh <= kSmallP) {
    dim3 grid((unsigned)((mr * 4 + 15) / 16), nitems, (unsigned)a.row_tiles);
    hipLaunchKernelGGL(paged_decode_merge_small_kernel, grid, dim3(256), 0, stream, a);
  } else {
    dim3 grid((unsigned)(mr * 4), nitems, (unsigned)a.row_tiles);
    hipLaunchKernelGGL(paged_decode_merge_kernel, grid, dim3(256), 0, stream, a);
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Bytes of the DecodeOnly bounds array after the partials (256-byte aligned).
size_t bounds_offset(size_t partial_bytes) { return (partial_bytes + 255) & ~(size_t)255; }

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
  return workspace_floats(num_requests, num_kv_heads, num_heads, max_query_len, max_history, tiles_per_split) *
         sizeof(float);
}

}  // extern "C"

namespace oscar {
namespace {

// A checked decode: the kernel arguments and the host request layout of one
// oscar_paged_decode call, ready to enqueue (empty: nothing to launch).
struct DecodeLaunch {
  DecodeArgs a;
  OutRotation orot;
  const int32_t* qsl;
  const int32_t* seqs;
  const int32_t* block_table;
  int64_t bt_stride;
  int32_t num_requests;
  int32_t max_query_len;
  int32_t num_kv_heads;
  int64_t max_history;
  int32_t tiles_per_split;
  bool empty;
};

int prepare_decode(DecodeLaunch& L, const float* q_rot, const float* k_new, const float* v_new, int32_t num_tokens,
                   int32_t num_heads, int32_t num_kv_heads, int32_t head_size, const void* k_cache,
                   const void* v_cache, int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                   int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page, int64_t v_stride_token,
                   int64_t v_stride_head, const int32_t* block_table, int64_t block_table_stride,
                   int32_t block_table_cols, const int32_t* query_start_loc, const int32_t* seq_lens,
                   int32_t num_requests, int32_t max_query_len, int64_t max_history, const int64_t* stage_owner,
                   const void* stage_k_image, const void* stage_v_image, int32_t stage_rows, float scale,
                   int32_t tiles_per_split, float* out, const OutRotation& orot, void* workspace,
                   size_t workspace_size) {
  L.empty = true;
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_requests < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_kv_heads > kMaxInlineItems || num_heads % num_kv_heads != 0 || max_query_len < 0 ||
      max_query_len > kMaxFresh || max_history < 0 || block_size <= 0 || num_pages <= 0 ||
      block_table_cols < 0 || stage_rows < 0 || tiles_per_split < 0 || tiles_per_split > kMaxTilesPerSplit)
    return kErrInvalidArgument;
  if (num_tokens == 0 || num_requests == 0 || max_query_len == 0) return kOk;
  DecodeArgs& a = L.a;
  a = DecodeArgs{};
  int rc = fill_common(a, q_rot, num_heads, num_kv_heads, head_size, k_cache, v_cache, block_size, num_pages,
                       k_stride_page, k_stride_token, k_stride_head, v_stride_page, v_stride_token, v_stride_head,
                       block_table, block_table_stride, block_table_cols, max_history, stage_owner, stage_k_image,
                       stage_v_image, stage_rows, scale, out, workspace);
  if (rc != kOk) return rc;
  if (!k_new || !v_new || !query_start_loc || !seq_lens) return kErrInvalidArgument;
  // Host-side request layout (the reference's query_layout checks).
  if (query_start_loc[0] < 0 || query_start_loc[num_requests] > num_tokens) return kErrInvalidArgument;
  for (int32_t i = 0; i < num_requests; ++i) {
    const int32_t nq = query_start_loc[i + 1] - query_start_loc[i];
    if (nq < 0 || nq > max_query_len || seq_lens[i] < nq || (int64_t)(seq_lens[i] - nq) > max_history)
      return kErrInvalidArgument;
  }
  if (tiles_per_split > 0 && splits_for(max_history, tiles_per_split) > kMaxSplits) return kErrInvalidArgument;
  if (tiles_per_split == 0 && (max_history + kStepTok - 1) / kStepTok > kMaxSplits * kMaxStepsPerSplit)
    return kErrInvalidArgument;
  const size_t need = workspace_floats(num_requests, num_kv_heads, num_heads, max_query_len, max_history,
                                       tiles_per_split) * sizeof(float);
  if (workspace == nullptr || workspace_size < need) return kErrWorkspaceTooSmall;
  a.k_new = k_new;
  a.v_new = v_new;
  a.win = nullptr;
  a.fresh = 1;
  L.max_history = max_history;
  L.tiles_per_split = tiles_per_split;
  a.row_tiles = (max_query_len * a.group + kRows - 1) / kRows;
  if ((rc = set_split_lds()) != kOk) return rc;
  L.orot = orot;
  L.qsl = query_start_loc;
  L.seqs = seq_lens;
  L.block_table = block_table;
  L.bt_stride = block_table_stride;
  L.num_requests = num_requests;
  L.max_query_len = max_query_len;
  L.num_kv_heads = num_kv_heads;
  L.empty = false;
  return kOk;
}

int launch_decode(DecodeLaunch& L, hipStream_t stream) {
  if (L.empty) return kOk;
  DecodeArgs& a = L.a;
  // Chunks of whole requests (at most kMaxInlineItems items); each chunk's
  // partials reuse the same workspace (the merge of one chunk precedes the
  // next split in stream order).
  const int32_t per = requests_per_launch(L.num_kv_heads);
  for (int32_t c0 = 0; c0 < L.num_requests; c0 += per) {
    const int32_t nreq = L.num_requests - c0 < per ? L.num_requests - c0 : per;
    for (int32_t i = 0; i < nreq; ++i) {
      const int32_t qa = L.qsl[c0 + i];
      const int32_t nq = L.qsl[c0 + i + 1] - qa;
      for (int32_t h = 0; h < L.num_kv_heads; ++h)
        a.items[i * L.num_kv_heads + h] = ItemInfo{qa, L.seqs[c0 + i] - nq, 0, (int16_t)nq, (int16_t)i, (int16_t)h, 0};
    }
    a.block_table = L.block_table ? L.block_table + (int64_t)c0 * L.bt_stride : nullptr;
    const unsigned nitems = (unsigned)(nreq * L.num_kv_heads);
    // Per-item splits; the fresh partial gets a workgroup of its own when one
    // more per item still fits the resident budget, else it rides on a
    // history split.
    if (!plan_splits(a, nitems, L.max_history, L.tiles_per_split, 1)) return kErrInvalidArgument;
    const unsigned gx = split_workgroups(a);
    if (gx > 0) launch_split(a, nitems, dim3(gx, 1, (unsigned)a.row_tiles), stream);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
    const int rc = launch_merge(a, (int64_t)L.max_query_len * a.group, nitems, L.orot, stream);
    if (rc != kOk) return rc;
  }
  return kOk;
}

int paged_decode(const float* q_rot, const float* k_new, const float* v_new, int32_t num_tokens, int32_t num_heads,
                 int32_t num_kv_heads, int32_t head_size, const void* k_cache, const void* v_cache,
                 int32_t block_size, int64_t num_pages, int64_t k_stride_page, int64_t k_stride_token,
                 int64_t k_stride_head, int64_t v_stride_page, int64_t v_stride_token, int64_t v_stride_head,
                 const int32_t* block_table, int64_t block_table_stride, int32_t block_table_cols,
                 const int32_t* query_start_loc, const int32_t* seq_lens, int32_t num_requests,
                 int32_t max_query_len, int64_t max_history, const int64_t* stage_owner,
                 const void* stage_k_image, const void* stage_v_image, int32_t stage_rows, float scale,
                 int32_t tiles_per_split, float* out, const OutRotation& orot, void* workspace,
                 size_t workspace_size, hipStream_t stream) {
  DecodeLaunch L;
  const int rc = prepare_decode(L, q_rot, k_new, v_new, num_tokens, num_heads, num_kv_heads, head_size, k_cache,
                                v_cache, block_size, num_pages, k_stride_page, k_stride_token, k_stride_head,
                                v_stride_page, v_stride_token, v_stride_head, block_table, block_table_stride,
                                block_table_cols, query_start_loc, seq_lens, num_requests, max_query_len,
                                max_history, stage_owner, stage_k_image, stage_v_image, stage_rows, scale,
                                tiles_per_split, out, orot, workspace, workspace_size);
  return rc != kOk ? rc : launch_decode(L, stream);
}

// Device scratch of the no-allocation entry (oscar_paged_decode_noalloc):
// the split partials of one launch, at most kScratchBytes.  Every GPU the
// library runs on holds its own copy until the process ends.
constexpr size_t kScratchBytes = OSCAR_DECODE_NOALLOC_SCRATCH_BYTES;

}  // namespace
}  // namespace oscar

static __device__ __align__(256) uint8_t scratch[oscar::kScratchBytes];

namespace oscar {
namespace {

// Device address of this GPU's `scratch`, looked up once per device with
// that device current (the array's name is a host-side stand-in, never a
// device address).
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kErrLaunch;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return kErrLaunch;
    g_scratch_addr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return kOk;
}

}  // namespace
}  // namespace oscar

extern "C" {

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
  if (!out) return kErrInvalidArgument;
  return paged_decode(q_rot, k_new, v_new, num_tokens, num_heads, num_kv_heads, head_size, k_cache, v_cache,
                      block_size, num_pages, k_stride_page, k_stride_token, k_stride_head, v_stride_page,
                      v_stride_token, v_stride_head, block_table, block_table_stride, block_table_cols,
                      query_start_loc, seq_lens, num_requests, max_query_len, max_history, stage_owner,
                      stage_k_image, stage_v_image, stage_rows, scale, tiles_per_split, out,
                      OutRotation{nullptr, nullptr, 0, 0}, workspace, workspace_size, stream);
}

int oscar_paged_decode_rotated(const float* q_rot, const float* k_new, const float* v_new,
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
                               int32_t tiles_per_split, const float* rot_v_t, void* out,
                               int64_t out_token_stride, int32_t out_bf16, void* workspace,
                               size_t workspace_size, hipStream_t stream) {
  if (!rot_v_t || !out || out_token_stride < (int64_t)num_heads * kHeadDim || out_bf16 < 0 || out_bf16 > 1)
    return kErrInvalidArgument;
  // The merge blocks write their outputs through this pointer only; the
  // fp32 rotated-domain output pointer of the split kernels is unused.
  return paged_decode(q_rot, k_new, v_new, num_tokens, num_heads, num_kv_heads, head_size, k_cache, v_cache,
                      block_size, num_pages, k_stride_page, k_stride_token, k_stride_head, v_stride_page,
                      v_stride_token, v_stride_head, block_table, block_table_stride, block_table_cols,
                      query_start_loc, seq_lens, num_requests, max_query_len, max_history, stage_owner,
                      stage_k_image, stage_v_image, stage_rows, scale, tiles_per_split,
                      reinterpret_cast<float*>(out), OutRotation{rot_v_t, out, out_token_stride, out_bf16},
                      workspace, workspace_size, stream);
}

int oscar_paged_decode_noalloc(const float* q_rot, const float* k_new, const float* v_new,
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
                               int32_t tiles_per_split, float* out, hipStream_t stream) {
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != kOk) return rc;
  // oscar_paged_decode rejects a launch whose partials exceed the scratch
  // (kErrWorkspaceTooSmall) before anything is enqueued.
  return oscar_paged_decode(q_rot, k_new, v_new, num_tokens, num_heads, num_kv_heads, head_size, k_cache, v_cache,
                            block_size, num_pages, k_stride_page, k_stride_token, k_stride_head, v_stride_page,
                            v_stride_token, v_stride_head, block_table, block_table_stride, block_table_cols,
                            query_start_loc, seq_lens, num_requests, max_query_len, max_history, stage_owner,
                            stage_k_image, stage_v_image, stage_rows, scale, tiles_per_split, out, ws, kScratchBytes,
                            stream);
}

size_t oscar_decode_only_workspace_bytes(int32_t num_requests, int32_t num_kv_heads, int32_t num_heads,
                                         int64_t max_history, int32_t tiles_per_split) {
  const size_t partials = oscar_paged_decode_workspace_bytes(num_requests, num_kv_heads, num_heads, 1,
                                                             max_history, tiles_per_split);
  if (partials == 0) return 0;
  const int64_t per = requests_per_launch(num_kv_heads);
  const int64_t reqs = num_requests < per ? num_requests : per;
  return bounds_offset(partials) + (size_t)reqs * 2 * sizeof(int32_t);
}

int oscar_decode_only(const float* q_rot, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                      const void* k_cache, const void* v_cache, int32_t block_size, int64_t num_pages,
                      int64_t k_stride_page, int64_t k_stride_token, int64_t k_stride_head,
                      int64_t v_stride_page, int64_t v_stride_token, int64_t v_stride_head,
                      const int32_t* block_table, int64_t block_table_stride, int32_t block_table_cols,
                      const int32_t* seq_lens, int32_t num_requests, int64_t max_history,
                      const int64_t* stage_owner, const void* stage_k_image, const void* stage_v_image,
                      int32_t stage_rows, int32_t sink_tokens, int32_t recent_tokens, float scale,
                      int32_t tiles_per_split, float* out, void* workspace, size_t workspace_size,
                      hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_requests < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_kv_heads > kMaxInlineItems ||
      num_heads % num_kv_heads != 0 || max_history < 0 ||
      block_size <= 0 || num_pages <= 0 || block_table_cols < 0 || stage_rows < 0 || sink_tokens < 0 ||
      recent_tokens < 0 || tiles_per_split < 0 || tiles_per_split > kMaxTilesPerSplit)
    return kErrInvalidArgument;
  if (num_requests == 0) return kOk;
  DecodeArgs a{};
  int rc = fill_common(a, q_rot, num_heads, num_kv_heads, head_size, k_cache, v_cache, block_size, num_pages,
                       k_stride_page, k_stride_token, k_stride_head, v_stride_page, v_stride_token, v_stride_head,
                       block_table, block_table_stride, block_table_cols, max_history, stage_owner, stage_k_image,
                       stage_v_image, stage_rows, scale, out, workspace);
  if (rc != kOk) return rc;
  if (!seq_lens) return kErrInvalidArgument;
  for (int32_t i = 0; i < num_requests; ++i)
    if (seq_lens[i] < 0 || seq_lens[i] > max_history) return kErrInvalidArgument;
  if (tiles_per_split > 0 && splits_for(max_history, tiles_per_split) > kMaxSplits) return kErrInvalidArgument;
  if (tiles_per_split == 0 && (max_history + kStepTok - 1) / kStepTok > kMaxSplits * kMaxStepsPerSplit)
    return kErrInvalidArgument;
  const size_t partials = workspace_floats(num_requests, num_kv_heads, num_heads, 1, max_history,
                                           tiles_per_split) * sizeof(float);
  const int32_t per = requests_per_launch(num_kv_heads);
  const size_t need = bounds_offset(partials) +
                      (size_t)(num_requests < per ? num_requests : per) * 2 * sizeof(int32_t);
  if (workspace == nullptr || workspace_size < need) return kErrWorkspaceTooSmall;
  const bool window = stage_rows > 0;
  int32_t* bounds = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + bounds_offset(partials));
  const int32_t sink_eff = window ? (sink_tokens / block_size) * block_size : 0;
  a.k_new = nullptr;
  a.v_new = nullptr;
  // One query per request: the small-row kernel reads when the group has at
  // most 8 heads, and then finds the bounds itself when each of the sink and
  // recent spans fits one position per thread; else the bounds kernel runs.
  const bool fold = window && a.group <= kSmRows && sink_eff <= 256 && recent_tokens <= 256;
  a.win = window && !fold ? bounds : nullptr;
  a.win_fold = fold ? 1 : 0;
  a.win_sink = sink_eff;
  a.win_recent = recent_tokens;
  a.fresh = 0;
  a.row_tiles = (a.group + kRows - 1) / kRows;
  if ((rc = set_split_lds()) != kOk) return rc;
  for (int32_t c0 = 0; c0 < num_requests; c0 += per) {
    const int32_t nreq = num_requests - c0 < per ? num_requests - c0 : per;
    for (int32_t i = 0; i < nreq; ++i)
      for (int32_t h = 0; h < num_kv_heads; ++h)
        a.items[i * num_kv_heads + h] = ItemInfo{c0 + i, seq_lens[c0 + i], 0, 1, (int16_t)i, (int16_t)h, 0};
    a.block_table = block_table ? block_table + (int64_t)c0 * block_table_stride : nullptr;
    const unsigned nitems = (unsigned)(nreq * num_kv_heads);
    if (!plan_splits(a, nitems, max_history, tiles_per_split, 0)) return kErrInvalidArgument;
    if (window && !fold) {
      hipLaunchKernelGGL(decode_only_bounds_kernel, dim3((unsigned)nreq), dim3(kBoundsThreads), 0, stream, a, bounds,
                         sink_eff, recent_tokens);
      if (hipGetLastError() != hipSuccess) return kErrLaunch;
    }
    const unsigned gx = split_workgroups(a);
    if (gx > 0) {
      launch_split(a, nitems, dim3(gx, 1, (unsigned)a.row_tiles), stream);
      if (hipGetLastError() != hipSuccess) return kErrLaunch;
    }
    if ((rc = launch_merge(a, a.group, nitems, OutRotation{nullptr, nullptr, 0, 0}, stream)) != kOk) return rc;
  }
  return kOk;
}

// The short-step forward of one layer: every argument of the decode is
// checked before the step write is enqueued, so an error enqueues nothing.
int oscar_mtp_forward(const oscar_mtp_layer* layer, const oscar_mtp_step* step, const void* query_bf16,
                      int64_t query_token_stride, const void* key_bf16, const void* value_bf16,
                      int64_t kv_token_stride, void* out, int64_t out_token_stride, int32_t out_bf16,
                      hipStream_t stream) {
  if (!layer || !step || layer->num_heads != step->num_heads || layer->num_kv_heads != step->num_kv_heads)
    return kErrInvalidArgument;
  const oscar_mtp_layer& L = *layer;
  const oscar_mtp_step& S = *step;
  if (!L.rot_v_t || !out || out_token_stride < (int64_t)L.num_heads * kHeadDim || out_bf16 < 0 || out_bf16 > 1)
    return kErrInvalidArgument;
  const int32_t rows = L.stage_rows;
  DecodeLaunch D;
  int rc = prepare_decode(D, S.q_rot, S.k_rot, S.v_rot, S.num_tokens, L.num_heads, L.num_kv_heads, L.head_size,
                          L.k_cache, L.v_cache, L.block_size, L.num_pages, L.k_stride_page, L.k_stride_token,
                          L.k_stride_head, L.v_stride_page, L.v_stride_token, L.v_stride_head, S.block_table,
                          S.block_table_stride, S.block_table_cols, S.query_start_loc, S.seq_lens, S.num_requests,
                          S.max_query_len, S.max_history, rows > 0 ? L.stage_owner : nullptr,
                          rows > 0 ? L.stage_k_image : nullptr, rows > 0 ? L.stage_v_image : nullptr, rows, L.scale,
                          S.tiles_per_split, reinterpret_cast<float*>(out),
                          OutRotation{L.rot_v_t, out, out_token_stride, out_bf16}, S.workspace, S.workspace_size);
  if (rc != kOk) return rc;
  rc = oscar_step_write(query_bf16, query_token_stride, key_bf16, value_bf16, kv_token_stride, S.num_tokens,
                        L.num_heads, L.num_kv_heads, L.head_size, L.rot_k, L.rot_v, S.slot_mapping,
                        S.query_start_loc, S.seq_lens, S.num_requests, L.k_cache, L.v_cache, L.block_size,
                        L.num_pages, L.k_stride_page, L.k_stride_token, L.k_stride_head, L.v_stride_page,
                        L.v_stride_token, L.v_stride_head, L.clip_index_k, L.clip_index_v,
                        rows > 0 ? L.stage_k : nullptr, rows > 0 ? L.stage_v : nullptr,
                        rows > 0 ? L.stage_owner : nullptr, rows > 0 ? L.stage_k_image : nullptr,
                        rows > 0 ? L.stage_v_image : nullptr, rows, L.sink_eff, L.recent, S.q_rot, S.k_rot, S.v_rot,
                        stream);
  if (rc != kOk) return rc;
  return launch_decode(D, stream);
}

}  // extern "C"
