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
// Two kernels:
//   split: one wavefront per (request, kv-head, 128-position chunk, 32-row
//          tile).  Rows are (query token, head-in-group) pairs of the GQA
//          group, so K/V are dequantized once for all of them.  Each 32-token
//          block is dequantized (or taken from staging) into LDS as fp16:
//          K token-major, V feature-major.  S^T = K Q^T and O^T += V^T P^T run
//          on 32x32x16 f16 MFMA with fp32 accumulation; online softmax in
//          base 2.  Emits (m, l, unnormalised O) per row.
//   merge: one block per (request, kv-head, row tile): LSE-combines the chunk
//          partials with the causal fresh-token scores computed in fp32.
#include "oscar_common.h"

namespace oscar {
namespace {

constexpr int kChunk = 128;            // history positions per split wavefront
constexpr int kBlock = 32;             // tokens per MFMA block
constexpr int kRowsPerTile = 32;
constexpr int kKhStride = kHeadDim + 8;   // halfs per K row in LDS
constexpr int kVtStride = kBlock + 8;     // halfs per V feature row in LDS
constexpr float kLog2e = 1.4426950408889634f;

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
  float* ws_o;                  // [items][D][32]
  float* ws_ml;                 // [items][2][32]
  int32_t max_chunks, row_tiles;
};

__device__ __forceinline__ int64_t item_index(const DecodeArgs& a, int req, int kvh, int chunk, int rt) {
  return (((int64_t)req * a.num_kv_heads + kvh) * a.max_chunks + chunk) * a.row_tiles + rt;
}

__global__ __launch_bounds__(64) void paged_decode_split_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 kh[kBlock * kKhStride];
  __shared__ __attribute__((aligned(16))) _Float16 vt[kHeadDim * kVtStride];

  const int chunk = blockIdx.x;
  const int req = blockIdx.y / a.num_kv_heads;
  const int kvh = blockIdx.y - req * a.num_kv_heads;
  const int rt = blockIdx.z;
  const int lane = threadIdx.x;
  const int g = lane >> 5;
  const int col = lane & 31;

  const int qa = a.query_start[req];
  const int qb = a.query_start[req + 1];
  const int nq = qb - qa;
  if (nq <= 0 || qa < 0 || qb > a.num_tokens) return;
  const int prefix = a.seq_lens[req] - nq;
  const int p_begin = chunk * kChunk;
  if (p_begin >= prefix) return;
  const int rows = nq * a.group;
  if (rt * kRowsPerTile >= rows) return;

  // Q^T operand: lane (row col, k-group g) holds q[row][16m + 8g .. +7].
  const int row = rt * kRowsPerTile + col;
  const bool row_ok = row < rows;
  half8 qb_op[16];
  {
    const int j = row_ok ? row / a.group : 0;
    const int h = kvh * a.group + (row_ok ? row % a.group : 0);
    const float* qp = a.q + ((int64_t)(qa + j) * a.num_heads + h) * kHeadDim + 8 * g;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      floatx4 x0 = row_ok ? *reinterpret_cast<const floatx4*>(qp + 16 * m) : floatx4{};
      floatx4 x1 = row_ok ? *reinterpret_cast<const floatx4*>(qp + 16 * m + 4) : floatx4{};
      qb_op[m] = half8{(_Float16)x0[0], (_Float16)x0[1], (_Float16)x0[2], (_Float16)x0[3],
                       (_Float16)x1[0], (_Float16)x1[1], (_Float16)x1[2], (_Float16)x1[3]};
    }
  }

  floatx16 acc_o[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc_o[t] = floatx16{};
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  const int tg = lane >> 4;     // producer: tokens 8*tg .. +7
  const int fg = lane & 15;     // producer: features 16*fg .. +15
  const int32_t* bt_row = a.block_table + (int64_t)req * a.bt_stride;
  const int p_end = min(prefix, p_begin + kChunk);

#pragma unroll 1
  for (int p0 = p_begin; p0 < p_end; p0 += kBlock) {
    // ---- produce fp16 K (token-major) and V (feature-major) into LDS ----
    // Pass 1: INT2 slots (zeros for positions past the prefix or staged).
    uint32_t kcw[8], vcw[8];
    float ksc[8], kzr[8], vsc[8], vzr[8];
    uint32_t staged_mask = 0;
    int64_t seat_of[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      const int pos = p0 + 8 * tg + tt;
      kcw[tt] = vcw[tt] = 0u;
      ksc[tt] = kzr[tt] = vsc[tt] = vzr[tt] = 0.f;
      seat_of[tt] = 0;
      int page = -1;
      const int pidx = pos / a.block_size;
      if (pos < prefix && pidx < a.bt_cols) page = bt_row[pidx];
      if (page < 0 || page >= a.num_pages) continue;
      const int prow = pos - pidx * a.block_size;
      if (a.stage_rows > 0) {
        const int64_t seat = (int64_t)(page % a.stage_rows) * a.block_size + prow;
        if (a.owner[seat] == (int64_t)page) {
          staged_mask |= 1u << tt;
          seat_of[tt] = seat;
          continue;
        }
      }
      const uint8_t* ks = a.k_cache + page * a.k_page + prow * a.k_tok + kvh * a.k_head;
      const uint8_t* vs = a.v_cache + page * a.v_page + prow * a.v_tok + kvh * a.v_head;
      const u32x2 meta = *reinterpret_cast<const u32x2*>(ks);
      kcw[tt] = *reinterpret_cast<const uint32_t*>(ks + kKCodeOff + 4 * fg);
      vcw[tt] = *reinterpret_cast<const uint32_t*>(vs + 4 * fg);
      ksc[tt] = f16_bits_to_f32(meta[0]);
      kzr[tt] = f16_bits_to_f32(meta[0] >> 16);
      vsc[tt] = f16_bits_to_f32(meta[1]);
      vzr[tt] = f16_bits_to_f32(meta[1] >> 16);
    }
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      half8 k0, k1;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        k0[u] = (_Float16)((float)((kcw[tt] >> (2 * u)) & 3u) * ksc[tt] + kzr[tt]);
        k1[u] = (_Float16)((float)((kcw[tt] >> (2 * u + 16)) & 3u) * ksc[tt] + kzr[tt]);
      }
      half8* kdst = reinterpret_cast<half8*>(kh + (8 * tg + tt) * kKhStride + 16 * fg);
      kdst[0] = k0;
      kdst[1] = k1;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      half8 x;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt)
        x[tt] = (_Float16)((float)((vcw[tt] >> (2 * u)) & 3u) * vsc[tt] + vzr[tt]);
      *reinterpret_cast<half8*>(vt + (16 * fg + u) * kVtStride + 8 * tg) = x;
    }
    // Pass 2 (rare): tokens owned by the FP32 staging arena overwrite their
    // entries with the unquantized rotated values.
    if (staged_mask) {
#pragma unroll 1
      for (int tt = 0; tt < 8; ++tt) {
        if (!((staged_mask >> tt) & 1u)) continue;
        const int64_t base = (seat_of[tt] * a.num_kv_heads + kvh) * kHeadDim + 16 * fg;
        const floatx4* sk = reinterpret_cast<const floatx4*>(a.stage_k + base);
        const floatx4* sv = reinterpret_cast<const floatx4*>(a.stage_v + base);
        _Float16* krow = kh + (8 * tg + tt) * kKhStride + 16 * fg;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const floatx4 x = sk[q4], y = sv[q4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            krow[4 * q4 + e] = (_Float16)x[e];
            vt[(16 * fg + 4 * q4 + e) * kVtStride + 8 * tg + tt] = (_Float16)y[e];
          }
        }
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T : lane holds row `col`, tokens 8*(r/4) + 4*g + r%4 ----
    floatx16 s = floatx16{};
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const half8 ka = *reinterpret_cast<const half8*>(kh + col * kKhStride + 16 * m + 8 * g);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb_op[m], s, 0, 0, 0);
    }
    float mb = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tok = 8 * (r >> 2) + 4 * g + (r & 3);
      const float x = (p0 + tok < prefix) ? s[r] * a.scale_log2 : -__builtin_inff();
      s[r] = x;
      mb = fmaxf(mb, x);
    }
    mb = fmaxf(mb, shfl_xor_f32(mb, 32));
    const float m_new = fmaxf(m_run, mb);
    const float alpha = (m_run == -__builtin_inff()) ? 0.f : exp2f(m_run - m_new);
    float psum = 0.f;
    half8 pb[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = (s[r] == -__builtin_inff()) ? 0.f : exp2f(s[r] - m_new);
      psum += p;
      pb[r >> 3][r & 7] = (_Float16)p;
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc_o[t] *= alpha;

    // ---- O^T += V^T P^T : K-slot 8g+u <-> token 16*mm + 8*(u/4) + 4*g + u%4 ----
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const _Float16* vrow = vt + (32 * t + col) * kVtStride + 16 * mm + 4 * g;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
        const half8 va = __builtin_bit_cast(half8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        acc_o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[mm], acc_o[t], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // ---- partial: O^T[f][row] (f = 32t + 8*(r/4) + 4*g + r%4), m, l ----
  const int64_t item = item_index(a, req, kvh, chunk, rt);
  float* wo = a.ws_o + item * (kHeadDim * kRowsPerTile);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int f = 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
      wo[f * kRowsPerTile + col] = acc_o[t][r];
    }
  }
  const float l_tot = l_run + shfl_xor_f32(l_run, 32);
  if (g == 0) {
    a.ws_ml[item * 2 * kRowsPerTile + col] = m_run;
    a.ws_ml[item * 2 * kRowsPerTile + kRowsPerTile + col] = l_tot;
  }
}

// One block of 256 threads per (request, kv-head, row tile).  Thread
// (row = tid & 31, fgrp = tid >> 5) owns features fgrp + 8k, k = 0..31.
constexpr int kMaxFresh = 16;

__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a) {
  __shared__ float part[8][kMaxFresh][kRowsPerTile];
  __shared__ float fresh[kMaxFresh][kRowsPerTile];

  const int req = blockIdx.x / a.num_kv_heads;
  const int kvh = blockIdx.x - req * a.num_kv_heads;
  const int rt = blockIdx.y;
  const int tid = threadIdx.x;
  const int rl = tid & 31;
  const int fgrp = tid >> 5;

  const int qa = a.query_start[req];
  const int qb = a.query_start[req + 1];
  const int nq = qb - qa;
  if (nq <= 0 || nq > kMaxFresh || qa < 0 || qb > a.num_tokens) return;
  const int prefix = a.seq_lens[req] - nq;
  const int rows = nq * a.group;
  if (rt * kRowsPerTile >= rows) return;
  const int row = rt * kRowsPerTile + rl;
  const bool row_ok = row < rows;
  const int j = row_ok ? row / a.group : 0;
  const int h = kvh * a.group + (row_ok ? row % a.group : 0);

  // Fresh-token scores (fp32), keys 0 .. j of this request's new tokens.
  const float* qp = a.q + ((int64_t)(qa + j) * a.num_heads + h) * kHeadDim;
  for (int i = 0; i < nq; ++i) {
    const float* kp = a.k_new + ((int64_t)(qa + i) * a.num_kv_heads + kvh) * kHeadDim;
    float d = 0.f;
#pragma unroll 8
    for (int k = 0; k < 32; ++k) d = fmaf(qp[fgrp + 8 * k], kp[fgrp + 8 * k], d);
    part[fgrp][i][rl] = d;
  }
  __syncthreads();
  if (fgrp == 0) {
    for (int i = 0; i < nq; ++i) {
      float d = 0.f;
#pragma unroll
      for (int q8 = 0; q8 < 8; ++q8) d += part[q8][i][rl];
      fresh[i][rl] = (i <= j) ? d * a.scale_log2 : -__builtin_inff();
    }
  }
  __syncthreads();

  const int chunks = prefix > 0 ? (prefix + kChunk - 1) / kChunk : 0;
  float mx = -__builtin_inff();
  for (int c = 0; c < chunks; ++c) {
    const int64_t item = item_index(a, req, kvh, c, rt);
    mx = fmaxf(mx, a.ws_ml[item * 2 * kRowsPerTile + rl]);
  }
  for (int i = 0; i < nq; ++i) mx = fmaxf(mx, fresh[i][rl]);

  float acc[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) acc[k] = 0.f;
  float lsum = 0.f;
  for (int c = 0; c < chunks; ++c) {
    const int64_t item = item_index(a, req, kvh, c, rt);
    const float mc = a.ws_ml[item * 2 * kRowsPerTile + rl];
    const float lc = a.ws_ml[item * 2 * kRowsPerTile + kRowsPerTile + rl];
    const float w = (mc == -__builtin_inff()) ? 0.f : exp2f(mc - mx);
    lsum += w * lc;
    const float* wo = a.ws_o + item * (kHeadDim * kRowsPerTile);
#pragma unroll
    for (int k = 0; k < 32; ++k) acc[k] = fmaf(w, wo[(fgrp + 8 * k) * kRowsPerTile + rl], acc[k]);
  }
  for (int i = 0; i < nq; ++i) {
    const float si = fresh[i][rl];
    const float w = (si == -__builtin_inff()) ? 0.f : exp2f(si - mx);
    lsum += w;
    const float* vp = a.v_new + ((int64_t)(qa + i) * a.num_kv_heads + kvh) * kHeadDim;
#pragma unroll
    for (int k = 0; k < 32; ++k) acc[k] = fmaf(w, vp[fgrp + 8 * k], acc[k]);
  }
  if (!row_ok) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  float* op = a.out + ((int64_t)(qa + j) * a.num_heads + h) * kHeadDim;
#pragma unroll
  for (int k = 0; k < 32; ++k) op[fgrp + 8 * k] = acc[k] * inv;
}

}  // namespace
}  // namespace oscar

using namespace oscar;

namespace {

int64_t max_chunks_for(int64_t max_history) {
  return max_history > 0 ? (max_history + kChunk - 1) / kChunk : 0;
}

size_t workspace_bytes(int32_t num_requests, int32_t num_kv_heads, int32_t num_heads,
                       int32_t max_query_len, int64_t max_history) {
  const int64_t group = num_kv_heads > 0 ? num_heads / num_kv_heads : 0;
  const int64_t tiles = (max_query_len * group + kRowsPerTile - 1) / kRowsPerTile;
  const int64_t items = (int64_t)num_requests * num_kv_heads * max_chunks_for(max_history) * tiles;
  return (size_t)(items * (kHeadDim * kRowsPerTile + 2 * kRowsPerTile) * sizeof(float));
}

}  // namespace

extern "C" {

size_t oscar_paged_decode_workspace_bytes(int32_t num_requests, int32_t num_kv_heads,
                                          int32_t num_heads, int32_t max_query_len,
                                          int64_t max_history) {
  if (num_requests <= 0 || num_kv_heads <= 0 || num_heads <= 0 || max_query_len <= 0 ||
      max_history < 0)
    return 0;
  return workspace_bytes(num_requests, num_kv_heads, num_heads, max_query_len, max_history);
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
                       int32_t stage_rows, float scale, float* out, void* workspace,
                       size_t workspace_size, hipStream_t stream) {
  if (head_size != kHeadDim) return kErrUnsupportedHeadDim;
  if (num_tokens < 0 || num_requests < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || max_query_len < 0 || max_query_len > kMaxFresh ||
      max_history < 0 || block_size <= 0 || num_pages <= 0 || block_table_cols < 0 ||
      stage_rows < 0)
    return kErrInvalidArgument;
  if (num_tokens == 0 || num_requests == 0 || max_query_len == 0) return kOk;
  if (!q_rot || !k_new || !v_new || !k_cache || !v_cache || !query_start_loc || !seq_lens || !out)
    return kErrInvalidArgument;
  if (max_history > 0 && !block_table) return kErrInvalidArgument;
  if (stage_rows > 0 && (!stage_k || !stage_v || !stage_owner)) return kErrInvalidArgument;
  if (k_stride_head < kKCodeOff + kCodeBytes || v_stride_head < kCodeBytes ||
      (k_stride_head & 7) || (k_stride_token & 7) || (k_stride_page & 7) || (v_stride_head & 3) ||
      (v_stride_token & 3) || (v_stride_page & 3))
    return kErrUnsupportedGeometry;
  const size_t need = workspace_bytes(num_requests, num_kv_heads, num_heads, max_query_len, max_history);
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
  a.ws_o = static_cast<float*>(workspace);
  const int64_t chunks = max_chunks_for(max_history);
  a.max_chunks = (int32_t)chunks;
  a.row_tiles = (max_query_len * a.group + kRowsPerTile - 1) / kRowsPerTile;
  const int64_t items = (int64_t)num_requests * num_kv_heads * chunks * a.row_tiles;
  a.ws_ml = a.ws_o + items * (kHeadDim * kRowsPerTile);

  if (chunks > 0) {
    dim3 grid((unsigned)chunks, (unsigned)(num_requests * num_kv_heads), (unsigned)a.row_tiles);
    hipLaunchKernelGGL(paged_decode_split_kernel, grid, dim3(64), 0, stream, a);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  dim3 mgrid((unsigned)(num_requests * num_kv_heads), (unsigned)a.row_tiles);
  hipLaunchKernelGGL(paged_decode_merge_kernel, mgrid, dim3(256), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
