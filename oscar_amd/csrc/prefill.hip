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
// One block of 4 wavefronts per 128 consecutive rows of one kv-head, a row
// being (new token j, head-in-group).  For every 32-key block the 256 threads
// produce K (token-major) and V (feature-major) fp16 tiles in LDS; each wave
// then runs S^T = K Q^T (16 MFMA 32x32x16) and O^T += V^T P^T (16 MFMA) on
// its 32 rows with base-2 online softmax.
#include "oscar_common.h"

namespace oscar {
namespace {

constexpr int kBlk = 32;
constexpr int kRowsPerWave = 32;
constexpr int kWaves = 4;
constexpr int kKs = kHeadDim + 8;     // halfs per K row in LDS
constexpr int kVs = kBlk + 8;         // halfs per V feature row in LDS
constexpr float kLog2e = 1.4426950408889634f;

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

__device__ __forceinline__ _Float16 to_h(float x) { return (_Float16)x; }

// Resolve history position p (< C): page, row in page, staging seat (or -1).
struct HistLoc {
  int64_t page;
  int32_t prow;
  int64_t seat;   // >= 0: read FP32 staging
  bool ok;
};

__device__ __forceinline__ HistLoc locate(const PrefillArgs& a, int64_t p) {
  HistLoc h{0, 0, -1, false};
  const int64_t pidx = p / a.block_size;
  if (pidx >= a.bt_cols) return h;
  const int64_t page = a.bt[pidx];
  if (page < 0 || page >= a.num_pages) return h;
  h.page = page;
  h.prow = (int32_t)(p - pidx * a.block_size);
  h.ok = true;
  if (a.stage_rows > 0) {
    const int64_t seat = (page % a.stage_rows) * a.block_size + h.prow;
    if (a.owner[seat] == page) h.seat = seat;
  }
  return h;
}

__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 kh[kBlk * kKs];
  __shared__ __attribute__((aligned(16))) _Float16 vt[kHeadDim * kVs];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;
  const int kvh = blockIdx.y;
  const int64_t rows_total = (int64_t)a.n_new * a.group;
  const int64_t row0 = (int64_t)blockIdx.x * (kWaves * kRowsPerWave);
  const int64_t wrow0 = row0 + wave * kRowsPerWave;
  const int64_t row = wrow0 + col;
  const bool row_ok = row < rows_total;
  const int64_t C = a.cached;

  // Key range of the block: up to the last row's causal limit.
  const int64_t last_row = min(row0 + kWaves * kRowsPerWave, rows_total) - 1;
  const int64_t keys_blk = C + last_row / a.group + 1;
  const int64_t wave_last = min(wrow0 + kRowsPerWave, rows_total) - 1;
  const int64_t keys_wave = wrow0 < rows_total ? C + wave_last / a.group + 1 : 0;
  const int64_t my_limit = row_ok ? C + row / a.group : -1;   // last visible key

  half8 qop[16];
  {
    const int64_t j = row_ok ? row / a.group : 0;
    const int h = kvh * a.group + (row_ok ? (int)(row % a.group) : 0);
    const float* qp = a.q + (j * a.num_heads + h) * kHeadDim + 8 * g;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      floatx4 x0 = row_ok ? *reinterpret_cast<const floatx4*>(qp + 16 * m) : floatx4{};
      floatx4 x1 = row_ok ? *reinterpret_cast<const floatx4*>(qp + 16 * m + 4) : floatx4{};
      qop[m] = half8{to_h(x0[0]), to_h(x0[1]), to_h(x0[2]), to_h(x0[3]),
                      to_h(x1[0]), to_h(x1[1]), to_h(x1[2]), to_h(x1[3])};
    }
  }

  floatx16 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = floatx16{};
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  // Producer roles.
  const int ktt = tid >> 3, kfg = tid & 7;       // K: token ktt, features 32*kfg .. +31
  const int vtg = tid >> 6, vfg = tid & 63;      // V: tokens 8*vtg .. +7, features 4*vfg .. +3

#pragma unroll 1
  for (int64_t k0 = 0; k0 < keys_blk; k0 += kBlk) {
    // ---------------- K tile ----------------
    {
      const int64_t p = k0 + ktt;
      float kv[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) kv[u] = 0.f;
      if (p < C) {
        const HistLoc h = locate(a, p);
        if (h.ok && h.seat >= 0) {
          const floatx4* src = reinterpret_cast<const floatx4*>(
              a.stage_k + (h.seat * a.num_kv_heads + kvh) * kHeadDim + 32 * kfg);
#pragma unroll
          for (int q4 = 0; q4 < 8; ++q4) {
            const floatx4 x = src[q4];
#pragma unroll
            for (int e = 0; e < 4; ++e) kv[4 * q4 + e] = x[e];
          }
        } else if (h.ok) {
          const uint8_t* ks = a.k_cache + h.page * a.k_page + h.prow * a.k_tok + kvh * a.k_head;
          const uint32_t meta = *reinterpret_cast<const uint32_t*>(ks);
          const u32x2 cw = *reinterpret_cast<const u32x2*>(ks + kKCodeOff + 8 * kfg);
          const float sc = f16_bits_to_f32(meta), zr = f16_bits_to_f32(meta >> 16);
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            kv[u] = (float)((cw[0] >> (2 * u)) & 3u) * sc + zr;
            kv[16 + u] = (float)((cw[1] >> (2 * u)) & 3u) * sc + zr;
          }
        }
      } else if (p < C + a.n_new) {
        const floatx4* src = reinterpret_cast<const floatx4*>(
            a.k_new + ((p - C) * a.num_kv_heads + kvh) * kHeadDim + 32 * kfg);
#pragma unroll
        for (int q4 = 0; q4 < 8; ++q4) {
          const floatx4 x = src[q4];
#pragma unroll
          for (int e = 0; e < 4; ++e) kv[4 * q4 + e] = x[e];
        }
      }
      half8* dst = reinterpret_cast<half8*>(kh + ktt * kKs + 32 * kfg);
#pragma unroll
      for (int q8 = 0; q8 < 4; ++q8) {
        half8 x;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = to_h(kv[8 * q8 + e]);
        dst[q8] = x;
      }
    }
    // ---------------- V tile (feature-major) ----------------
    {
      float vv[4][8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
#pragma unroll
        for (int u = 0; u < 4; ++u) vv[u][w] = 0.f;
        const int64_t p = k0 + 8 * vtg + w;
        if (p < C) {
          const HistLoc h = locate(a, p);
          if (h.ok && h.seat >= 0) {
            const floatx4 x = *reinterpret_cast<const floatx4*>(
                a.stage_v + (h.seat * a.num_kv_heads + kvh) * kHeadDim + 4 * vfg);
#pragma unroll
            for (int u = 0; u < 4; ++u) vv[u][w] = x[u];
          } else if (h.ok) {
            const uint8_t* ks = a.k_cache + h.page * a.k_page + h.prow * a.k_tok + kvh * a.k_head;
            const uint8_t* vs = a.v_cache + h.page * a.v_page + h.prow * a.v_tok + kvh * a.v_head;
            const uint32_t meta = *reinterpret_cast<const uint32_t*>(ks + 4);
            const uint32_t cb = vs[vfg];
            const float sc = f16_bits_to_f32(meta), zr = f16_bits_to_f32(meta >> 16);
#pragma unroll
            for (int u = 0; u < 4; ++u) vv[u][w] = (float)((cb >> (2 * u)) & 3u) * sc + zr;
          }
        } else if (p < C + a.n_new) {
          const floatx4 x = *reinterpret_cast<const floatx4*>(
              a.v_new + ((p - C) * a.num_kv_heads + kvh) * kHeadDim + 4 * vfg);
#pragma unroll
          for (int u = 0; u < 4; ++u) vv[u][w] = x[u];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        half8 x;
#pragma unroll
        for (int w = 0; w < 8; ++w) x[w] = to_h(vv[u][w]);
        *reinterpret_cast<half8*>(vt + (4 * vfg + u) * kVs + 8 * vtg) = x;
      }
    }
    __syncthreads();

    if (k0 < keys_wave) {
      floatx16 s = floatx16{};
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const half8 ka = *reinterpret_cast<const half8*>(kh + col * kKs + 16 * m + 8 * g);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qop[m], s, 0, 0, 0);
      }
      float mb = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t kp = k0 + 8 * (r >> 2) + 4 * g + (r & 3);
        const float x = (kp <= my_limit) ? s[r] * a.scale_log2 : -__builtin_inff();
        s[r] = x;
        mb = fmaxf(mb, x);
      }
      mb = fmaxf(mb, shfl_xor_f32(mb, 32));
      const float m_new = fmaxf(m_run, mb);
      float alpha = 1.f;
      if (m_new != -__builtin_inff()) alpha = (m_run == -__builtin_inff()) ? 0.f : exp2f(m_run - m_new);
      float psum = 0.f;
      half8 pb[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = (s[r] == -__builtin_inff()) ? 0.f : exp2f(s[r] - m_new);
        psum += p;
        pb[r >> 3][r & 7] = to_h(p);
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] *= alpha;
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const _Float16* vrow = vt + (32 * t + col) * kVs + 16 * mm + 4 * g;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
          const half8 va = __builtin_bit_cast(half8, u32x4{lo[0], lo[1], hi[0], hi[1]});
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[mm], acc[t], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }

  if (!row_ok) return;
  const float l_tot = l_run + shfl_xor_f32(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const int64_t j = row / a.group;
  const int h = kvh * a.group + (int)(row % a.group);
  float* op = a.out + (j * a.num_heads + h) * kHeadDim;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) op[32 * t + 8 * (r >> 2) + 4 * g + (r & 3)] = acc[t][r] * inv;
  }
}

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
  if (!q_rot || !k_new || !v_new || !k_cache || !v_cache || !out) return kErrInvalidArgument;
  if (cached_len > 0 && (!block_table_row || (cached_len + block_size - 1) / block_size > block_table_cols))
    return kErrInvalidArgument;
  if (stage_rows > 0 && (!stage_k || !stage_v || !stage_owner)) return kErrInvalidArgument;
  if (k_stride_head < kKCodeOff + kCodeBytes || v_stride_head < kCodeBytes || (k_stride_head & 7) ||
      (k_stride_token & 7) || (k_stride_page & 7))
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
  hipLaunchKernelGGL(prefill_kernel, grid, dim3(kWaves * 64), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
