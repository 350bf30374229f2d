// Paged MTP decode attention over INT2 history + FP32 window (gfx950).
//
// Semantics (per request i with query rows [a, b), n = b - a, prefix =
// seq_i - n): query token j attends to history positions 0 .. prefix-1 and to
// the request's own new tokens 0 .. j.  History position p lives in page
// bt[i][p / bs], row p % bs; it is read from the FP32 staging arena when the
// arena seat (page % rows, row) is owned by that page, otherwise it is
// dequantized from the INT2 slot.  All inputs are in the rotated domain; the
// output is in the rotated-V domain.
//
// Rows are (query token, head-in-group) pairs of one kv-head's GQA group, 32
// per tile, so each INT2 token is read and unpacked once for all of them.
//
// split kernel: one workgroup (4 wavefronts) per (request, kv-head, split of
//   `tiles_per_split` 32-token tiles, row tile); wave w takes tiles w, w+4, ...
//   Per tile (one page, since block_size % 32 == 0):
//   * S^T = K Q^T on 32x32x16 f16 MFMA.  Lane (token t, half g) turns its own
//     32 code bytes into fp16 K operands in registers: codes -> fp16 via the
//     1024 exponent trick, then one packed fma with its token's scale/zero.
//     The K dimension is permuted (feature 128g + 16j + 4a + i + 8b sits in
//     k-step 2j + a, slot 2i + b) so that pairs come straight out of a code
//     dword; Q^T (in LDS) uses the same permutation.
//   * O^T += V^T P'^T on 16 more MFMAs.  V codes are byte-transposed through
//     LDS ([byte][token]); one code dword of 4 tokens feeds the four features
//     of that byte, so output tile (h, s) holds features 4 * (32h + M) + s.
//     The V scale is folded into P' = p * vs_t and the V zero into a per-row
//     term sum_t p_t * vz_t added to every feature at the end.
//   * Tokens owned by the staging arena use their fp32 values: K operands
//     from the staged row, V through a second 16-MFMA pass over an fp16
//     V^T tile in LDS (only tiles that contain staged tokens).
//   Base-2 online softmax in fp32; the 4 wavefronts merge in LDS and the
//   workgroup writes (m, l, unnormalised O[row][256]).
// merge kernel: one 256-thread block per output row: LSE-combines the split
//   partials with the fresh-token scores (fp32, causal) and writes the row.
#include "oscar_common.h"

namespace oscar {
namespace {

constexpr int kTile = 32;
constexpr int kWaves = 4;
constexpr int kRows = 32;
constexpr int kMaxFresh = 16;
constexpr int kVtStride = 9;            // dwords per V code byte-row (32 tokens + pad)
constexpr int kVsStride = kTile + 8;    // halfs per staged V feature row
constexpr float kLog2e = 1.4426950408889634f;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

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
  const int32_t* query_start;   // [B + 1]
  const int32_t* seq_lens;      // [B]
  int32_t num_tokens;
  int32_t num_heads, num_kv_heads, group;
  const float* stage_k;         // [rows, bs, Hk, D] or null
  const float* stage_v;
  const int64_t* owner;         // [rows, bs]
  int32_t stage_rows;
  float scale_log2;             // attention scale * log2(e)
  float* out;                   // [n, Hq, D]
  float* ws;                    // partials
  int32_t max_splits, row_tiles, tiles_per_split;
};

struct LdsLayout {
  _Float16 q[16 * 2 * kRows * 8];                 // Q^T operand [m][g][row][8]
  uint32_t vt[kWaves][64 * kVtStride];            // V codes [byte][token/4]
  float vs[kWaves][kTile];                        // V scale per token (0: staged/invalid)
  float vz[kWaves][kTile];                        // V zero per token
  _Float16 vst[kWaves][kHeadDim * kVsStride];     // staged V^T tile
  float mrow[kWaves][kRows];
  float lrow[kWaves][kRows];
};

constexpr size_t kPartialFloats = kRows * kHeadDim + 2 * kRows;

__device__ __forceinline__ int64_t item_index(const DecodeArgs& a, int req, int kvh, int split, int rt) {
  return (((int64_t)req * a.num_kv_heads + kvh) * a.max_splits + split) * a.row_tiles + rt;
}

__device__ __forceinline__ half8 make_half8(half2v x0, half2v x1, half2v x2, half2v x3) {
  return half8{x0[0], x0[1], x1[0], x1[1], x2[0], x2[1], x3[0], x3[1]};
}

// 2 codes at bits [sh, sh+2) and [sh+16, sh+18) of w -> fp16 pair (exact 0..3).
__device__ __forceinline__ half2v code_pair(uint32_t w, int sh) {
  const uint32_t bits = ((w >> sh) & 0x00030003u) | 0x64006400u;   // fp16 1024 + code
  return __builtin_bit_cast(half2v, bits) - half2v{(_Float16)1024.f, (_Float16)1024.f};
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct TileLoad {
  u32x4 kc0, kc1;     // this lane's 32 K code bytes
  u32x2 meta;         // K scale, K zero, V scale, V zero (fp16 pairs)
  u32x2 vc[4];        // V code bytes 8*bg .. +7 of tokens 4*tq .. +3
  int64_t own;        // owner tag of this lane's token seat (-2: no arena)
  int32_t page;       // -1: tile invalid
  int32_t prow0;
};

__device__ __forceinline__ TileLoad load_tile(const DecodeArgs& a, const int32_t* bt_row, int p0,
                                              int prefix, int kvh, int lane) {
  TileLoad L;
  L.page = -1;
  L.prow0 = 0;
  L.own = -2;
  L.kc0 = L.kc1 = u32x4{0u, 0u, 0u, 0u};
  L.meta = u32x2{0u, 0u};
#pragma unroll
  for (int k = 0; k < 4; ++k) L.vc[k] = u32x2{0u, 0u};
  const int pidx = p0 / a.block_size;
  if (p0 >= prefix || pidx >= a.bt_cols) return L;
  const int page = bt_row[pidx];
  if (page < 0 || page >= a.num_pages) return L;
  L.page = page;
  L.prow0 = p0 - pidx * a.block_size;
  const int t = lane & 31, g = lane >> 5;
  const int tq = lane & 7, bg = lane >> 3;
  const uint8_t* kbase = a.k_cache + (int64_t)page * a.k_page + (int64_t)kvh * a.k_head;
  const uint8_t* vbase = a.v_cache + (int64_t)page * a.v_page + (int64_t)kvh * a.v_head;
  const bool tok_ok = p0 + t < prefix;
  if (tok_ok) {
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

__global__ __launch_bounds__(256) void paged_decode_split_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  LdsLayout& S = *reinterpret_cast<LdsLayout*>(smem_raw);

  const int split = blockIdx.x;
  const int req = blockIdx.y / a.num_kv_heads;
  const int kvh = blockIdx.y - req * a.num_kv_heads;
  const int rt = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;

  const int qa = a.query_start[req];
  const int qb = a.query_start[req + 1];
  const int nq = qb - qa;
  if (nq <= 0 || qa < 0 || qb > a.num_tokens) return;
  const int prefix = a.seq_lens[req] - nq;
  const int tiles = prefix > 0 ? (prefix + kTile - 1) / kTile : 0;
  const int t_begin = split * a.tiles_per_split;
  if (t_begin >= tiles) return;
  const int t_end = min(tiles, t_begin + a.tiles_per_split);
  const int rows = nq * a.group;
  if (rt * kRows >= rows) return;

  // ---- Q^T operand into LDS (permuted K dimension, fp16) ----
  // Thread: row tid >> 3, features 32 * (tid & 7) .. +31; all loads issued
  // before any store so the fill costs one memory latency.
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
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const int e = 32 * c + k;
      const int gg = e >> 7, rr = e & 127, jj = rr >> 4, r16 = rr & 15, b = r16 >> 3, r8 = r16 & 7;
      const int m = 2 * jj + (r8 >> 2), u = 2 * (r8 & 3) + b;
      S.q[((m * 2 + gg) * kRows + r) * 8 + u] = (_Float16)x[k >> 2][k & 3];
    }
  }
  __syncthreads();

  floatx16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx16{};
  float m_run = -__builtin_inff(), l_run = 0.f, z_run = 0.f;
  const int32_t* bt_row = a.block_table + (int64_t)req * a.bt_stride;
  const int tq = lane & 7, bg = lane >> 3;

  int ti = t_begin + w;
  TileLoad cur = load_tile(a, bt_row, ti * kTile, prefix, kvh, lane);
#pragma unroll 1
  for (; ti < t_end; ti += kWaves) {
    const int p0 = ti * kTile;
    const TileLoad L = cur;
    if (ti + kWaves < t_end) cur = load_tile(a, bt_row, (ti + kWaves) * kTile, prefix, kvh, lane);

    const bool tok_ok = L.page >= 0 && p0 + col < prefix;
    const bool staged = tok_ok && L.own == (int64_t)L.page;
    const uint64_t sball = __ballot(staged && g == 0);
    const uint32_t smask = (uint32_t)sball;

    // ---- V codes -> LDS [byte][token], V meta -> LDS ----
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
        const bool use = tok_ok && !staged;
        S.vs[w][col] = use ? f16_bits_to_f32(L.meta[1]) : 0.f;
        S.vz[w][col] = use ? f16_bits_to_f32(L.meta[1] >> 16) : 0.f;
      }
    }
    if (smask) {
      // Staged V^T tile (fp16), zero for tokens not owned by the arena.
      const float* sv = nullptr;
      if (staged) {
        const int64_t seat = (int64_t)(L.page % a.stage_rows) * a.block_size + L.prow0 + col;
        sv = a.stage_v + (seat * a.num_kv_heads + kvh) * kHeadDim + 128 * g;
      }
#pragma unroll 4
      for (int f4 = 0; f4 < 32; ++f4) {
        floatx4 x = staged ? *reinterpret_cast<const floatx4*>(sv + 4 * f4) : floatx4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) S.vst[w][(128 * g + 4 * f4 + e) * kVsStride + col] = (_Float16)x[e];
      }
    }

    // ---- S^T = K Q^T (K dequantized in registers) ----
    const uint32_t kw[8] = {L.kc0[0], L.kc0[1], L.kc0[2], L.kc0[3], L.kc1[0], L.kc1[1], L.kc1[2], L.kc1[3]};
    const _Float16 ksc = (_Float16)(tok_ok ? f16_bits_to_f32(L.meta[0]) : 0.f);
    const _Float16 kzr = (_Float16)(tok_ok ? f16_bits_to_f32(L.meta[0] >> 16) : 0.f);
    const half2v s2{ksc, ksc}, z2{kzr, kzr};
    const float* sk = nullptr;
    if (staged) {
      const int64_t seat = (int64_t)(L.page % a.stage_rows) * a.block_size + L.prow0 + col;
      sk = a.stage_k + (seat * a.num_kv_heads + kvh) * kHeadDim + 128 * g;
    }
    wave_sync_lds();
    floatx16 s = floatx16{};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half8 ka[2];
      if (!staged) {
#pragma unroll
        for (int aa = 0; aa < 2; ++aa) {
          half2v p[4];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) p[ii] = code_pair(kw[j], 2 * (4 * aa + ii)) * s2 + z2;
          ka[aa] = make_half8(p[0], p[1], p[2], p[3]);
        }
      } else {
        const floatx4 x0 = *reinterpret_cast<const floatx4*>(sk + 16 * j);
        const floatx4 x1 = *reinterpret_cast<const floatx4*>(sk + 16 * j + 4);
        const floatx4 x2 = *reinterpret_cast<const floatx4*>(sk + 16 * j + 8);
        const floatx4 x3 = *reinterpret_cast<const floatx4*>(sk + 16 * j + 12);
        // slot 2i + b <-> feature 16j + 4a + i + 8b
        ka[0] = half8{(_Float16)x0[0], (_Float16)x2[0], (_Float16)x0[1], (_Float16)x2[1],
                      (_Float16)x0[2], (_Float16)x2[2], (_Float16)x0[3], (_Float16)x2[3]};
        ka[1] = half8{(_Float16)x1[0], (_Float16)x3[0], (_Float16)x1[1], (_Float16)x3[1],
                      (_Float16)x1[2], (_Float16)x3[2], (_Float16)x1[3], (_Float16)x3[3]};
      }
#pragma unroll
      for (int aa = 0; aa < 2; ++aa) {
        const int m = 2 * j + aa;
        const half8 qb = *reinterpret_cast<const half8*>(&S.q[((m * 2 + g) * kRows + col) * 8]);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[aa], qb, s, 0, 0, 0);
      }
    }

    // ---- online softmax (lane: row `col`, tokens 8*(r/4) + 4*g + r%4) ----
    float mb = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tok = 8 * (r >> 2) + 4 * g + (r & 3);
      const float x = (L.page >= 0 && p0 + tok < prefix) ? s[r] * a.scale_log2 : -__builtin_inff();
      s[r] = x;
      mb = fmaxf(mb, x);
    }
    mb = fmaxf(mb, shfl_xor_f32(mb, 32));
    const float m_new = fmaxf(m_run, mb);
    const bool grow = m_new > m_run && m_run != -__builtin_inff();
    const float alpha = grow ? exp2f(m_run - m_new) : 1.f;
    if (__ballot(grow)) {
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] *= alpha;
      l_run *= alpha;
      z_run *= alpha;
    }
    m_run = m_new;
    float pv[16];
    float psum = 0.f, zsum = 0.f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const floatx4 vsc = *reinterpret_cast<const floatx4*>(&S.vs[w][8 * jj + 4 * g]);
      const floatx4 vze = *reinterpret_cast<const floatx4*>(&S.vz[w][8 * jj + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * jj + i;
        const float p = (s[r] == -__builtin_inff()) ? 0.f : exp2f(s[r] - m_new);
        psum += p;
        zsum = fmaf(p, vze[i], zsum);
        pv[r] = p;
        s[r] = p * vsc[i];          // P' (scale folded)
      }
    }
    l_run += psum;
    z_run += zsum;

    // ---- O^T += V^T P'^T : slot u <-> tokens (t0,t2,t1,t3,t4,t6,t5,t7) ----
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int r0 = 8 * mm;
      const half8 pb = half8{(_Float16)s[r0 + 0], (_Float16)s[r0 + 2], (_Float16)s[r0 + 1], (_Float16)s[r0 + 3],
                             (_Float16)s[r0 + 4], (_Float16)s[r0 + 6], (_Float16)s[r0 + 5], (_Float16)s[r0 + 7]};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t* vrow = &S.vt[w][(32 * h + col) * kVtStride];
        const uint32_t d0 = vrow[4 * mm + g];
        const uint32_t d1 = vrow[4 * mm + 2 + g];
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
          const half8 va = make_half8(code_pair(d0, 2 * sp), code_pair(d0, 2 * sp + 8),
                                      code_pair(d1, 2 * sp), code_pair(d1, 2 * sp + 8));
          acc[4 * h + sp] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, acc[4 * h + sp], 0, 0, 0);
        }
      }
    }
    if (smask) {
      // Staged tokens: O^T += Vst^T P^T with the unscaled probabilities.
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        const int r0 = 8 * mm;
        const half8 pb = half8{(_Float16)pv[r0 + 0], (_Float16)pv[r0 + 2], (_Float16)pv[r0 + 1], (_Float16)pv[r0 + 3],
                               (_Float16)pv[r0 + 4], (_Float16)pv[r0 + 6], (_Float16)pv[r0 + 5], (_Float16)pv[r0 + 7]};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int sp = 0; sp < 4; ++sp) {
            const _Float16* vr = &S.vst[w][(4 * (32 * h + col) + sp) * kVsStride];
            const _Float16* x0 = vr + 16 * mm + 4 * g;
            const _Float16* x1 = vr + 16 * mm + 8 + 4 * g;
            const half8 va = half8{x0[0], x0[2], x0[1], x0[3], x1[0], x1[2], x1[1], x1[3]};
            acc[4 * h + sp] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, acc[4 * h + sp], 0, 0, 0);
          }
        }
      }
    }
    wave_sync_lds();
  }

  // ---- combine the 4 wavefronts: common max, then a 2-round tree in LDS ----
  const float l_tot = l_run + shfl_xor_f32(l_run, 32);
  const float z_tot = z_run + shfl_xor_f32(z_run, 32);
  if (g == 0) {
    S.mrow[w][col] = m_run;
    S.lrow[w][col] = l_tot;
  }
  __syncthreads();
  float mx = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < kWaves; ++k) mx = fmaxf(mx, S.mrow[k][col]);
  const float fw = (m_run == -__builtin_inff()) ? 0.f : exp2f(m_run - mx);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = (acc[t][r] + z_tot) * fw;
  }
  // Fragment buffers: [8 tiles][16 regs][64 lanes] fp32, lane-contiguous.
  float* frag0 = reinterpret_cast<float*>(&S.vst[0][0]);
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
  const int64_t item = item_index(a, req, kvh, split, rt);
  float* part = a.ws + item * kPartialFloats;
  for (int i = tid; i < kRows * kHeadDim; i += 256) part[i] = obuf[(i >> 8) * kOStride + (i & 255)];
  if (tid < kRows) {
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

// One 256-thread block per output row (request, kv-head, row).  Wave w sums
// splits w, w+4, ... with lane holding features 4*lane .. +3 (16-byte loads,
// eight splits in flight per batch); the four waves combine in LDS.
constexpr int kMaxSplits = 1024;
constexpr int kBatch = 16;

__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a) {
  __shared__ float red[kMaxFresh][4];
  __shared__ float fresh[kMaxFresh];
  __shared__ float wsplit[kMaxSplits];
  __shared__ float lsplit[kMaxSplits];
  __shared__ float wmax[4];
  __shared__ floatx4 osum[4][64];
  __shared__ float lsum_w[4];
  const int gidx = blockIdx.x;
  const int r = gidx % kRows;
  const int rest = gidx / kRows;
  const int rt = rest % a.row_tiles;
  const int rk = rest / a.row_tiles;
  const int req = rk / a.num_kv_heads;
  const int kvh = rk - req * a.num_kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;

  const int qa = a.query_start[req];
  const int qb = a.query_start[req + 1];
  const int nq = qb - qa;
  if (nq <= 0 || nq > kMaxFresh || qa < 0 || qb > a.num_tokens) return;
  const int row = rt * kRows + r;
  if (row >= nq * a.group) return;
  const int prefix = a.seq_lens[req] - nq;
  const int j = row / a.group;
  const int h = kvh * a.group + row % a.group;
  const int tiles = prefix > 0 ? (prefix + kTile - 1) / kTile : 0;
  const int splits = (tiles + a.tiles_per_split - 1) / a.tiles_per_split;
  if (splits > kMaxSplits) return;

  // Fresh-token scores q . k_new for keys 0 .. j: thread tid = feature.
  const float qf = a.q[((int64_t)(qa + j) * a.num_heads + h) * kHeadDim + tid];
  float kx[kMaxFresh];
#pragma unroll
  for (int i = 0; i < kMaxFresh; ++i)
    kx[i] = i <= j ? a.k_new[((int64_t)(qa + i) * a.num_kv_heads + kvh) * kHeadDim + tid] : 0.f;
  float mloc = -__builtin_inff();
  for (int sp = tid; sp < splits; sp += 256) {
    const float* part = a.ws + item_index(a, req, kvh, sp, rt) * kPartialFloats;
    const float mc = part[kRows * kHeadDim + r];
    wsplit[sp] = mc;
    lsplit[sp] = part[kRows * kHeadDim + kRows + r];
    mloc = fmaxf(mloc, mc);
  }
#pragma unroll
  for (int i = 0; i < kMaxFresh; ++i) {
    if (i > j) break;
    float d = qf * kx[i];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) d += __shfl_xor(d, o, 64);
    if (lane == 0) red[i][w] = d;
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

  floatx4 acc = floatx4{};
  float ls = 0.f;
  const floatx4* base = reinterpret_cast<const floatx4*>(
      a.ws + item_index(a, req, kvh, 0, rt) * kPartialFloats + r * kHeadDim) + lane;
  const int64_t stride4 = (int64_t)a.row_tiles * kPartialFloats / 4;
  for (int s0 = w; s0 < splits; s0 += 4 * kBatch) {
    floatx4 x[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int sp = s0 + 4 * k;
      x[k] = sp < splits ? base[sp * stride4] : floatx4{};
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int sp = s0 + 4 * k;
      if (sp < splits) {
        acc += wsplit[sp] * x[k];
        ls = fmaf(wsplit[sp], lsplit[sp], ls);
      }
    }
  }
  osum[w][lane] = acc;
  if (lane == 0) lsum_w[w] = ls;
  __syncthreads();
  if (w == 0) {
    floatx4 o = osum[0][lane] + osum[1][lane] + osum[2][lane] + osum[3][lane];
    float l = lsum_w[0] + lsum_w[1] + lsum_w[2] + lsum_w[3];
    for (int i = 0; i <= j; ++i) {
      const float wgt = exp2f(fresh[i] - mx);
      l += wgt;
      const floatx4 v = *reinterpret_cast<const floatx4*>(
          a.v_new + ((int64_t)(qa + i) * a.num_kv_heads + kvh) * kHeadDim + 4 * lane);
      o += wgt * v;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    *reinterpret_cast<floatx4*>(a.out + ((int64_t)(qa + j) * a.num_heads + h) * kHeadDim + 4 * lane) = o * inv;
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
  return (size_t)num_requests * num_kv_heads * splits_for(max_history, tiles_per_split) * tiles_r *
         kPartialFloats;
}

}  // namespace
}  // namespace oscar

using namespace oscar;

extern "C" {

size_t oscar_paged_decode_workspace_bytes(int32_t num_requests, int32_t num_kv_heads,
                                          int32_t num_heads, int32_t max_query_len,
                                          int64_t max_history, int32_t tiles_per_split) {
  if (num_requests <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads ||
      max_query_len <= 0 || max_history < 0 || tiles_per_split < 0)
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
                       const float* stage_k, const float* stage_v, const int64_t* stage_owner,
                       int32_t stage_rows, float scale, int32_t tiles_per_split, float* out,
                       void* workspace, size_t workspace_size, hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_requests < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || max_query_len < 0 || max_query_len > kMaxFresh ||
      max_history < 0 || block_size <= 0 || num_pages <= 0 || block_table_cols < 0 ||
      stage_rows < 0 || tiles_per_split < 0)
    return kErrInvalidArgument;
  if (num_tokens == 0 || num_requests == 0 || max_query_len == 0) return kOk;
  if (!q_rot || !k_new || !v_new || !k_cache || !v_cache || !query_start_loc || !seq_lens || !out)
    return kErrInvalidArgument;
  if (max_history > 0 && !block_table) return kErrInvalidArgument;
  if (stage_rows > 0 && (!stage_k || !stage_v || !stage_owner)) return kErrInvalidArgument;
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
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.bt_cols = block_table_cols;
  a.query_start = query_start_loc;
  a.seq_lens = seq_lens;
  a.num_tokens = num_tokens;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_heads / num_kv_heads;
  a.stage_k = stage_k;
  a.stage_v = stage_v;
  a.owner = stage_owner;
  a.stage_rows = stage_rows;
  a.scale_log2 = scale * kLog2e;
  a.out = out;
  a.ws = static_cast<float*>(workspace);
  a.tiles_per_split = tps;
  a.max_splits = (int32_t)splits_for(max_history, tps);
  if (a.max_splits > kMaxSplits) return kErrInvalidArgument;
  a.row_tiles = (max_query_len * a.group + kRows - 1) / kRows;

  if (a.max_splits > 0) {
    static bool lds_attr_set = false;
    if (!lds_attr_set) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(paged_decode_split_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(LdsLayout)) != hipSuccess)
        return kErrLaunch;
      lds_attr_set = true;
    }
    dim3 grid((unsigned)a.max_splits, (unsigned)(num_requests * num_kv_heads), (unsigned)a.row_tiles);
    hipLaunchKernelGGL(paged_decode_split_kernel, grid, dim3(256), sizeof(LdsLayout), stream, a);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  dim3 mgrid((unsigned)(num_requests * num_kv_heads * a.row_tiles * kRows));
  hipLaunchKernelGGL(paged_decode_merge_kernel, mgrid, dim3(256), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
