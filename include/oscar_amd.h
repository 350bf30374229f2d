/* oscar_amd.h — C ABI of the MI355X (gfx950) OSCAR INT2 KV-cache kernels.
 *
 * Library: oscar_amd/_oscar_hip.so (built by oscar_amd/csrc/build.py).
 *
 * Conventions for every entry point:
 *   - all tensor arguments are raw device pointers; sizes are element counts,
 *     strides of the paged caches are in BYTES (the reference addresses the
 *     caches through their uint8 view);
 *   - work is enqueued on `stream` and never synchronised; the return value
 *     is an oscar_status (0 = success, negative = error, nothing enqueued);
 *   - head_size must be 256 (kernels are written for D = 256);
 *   - caches are the engine's paged tensors (pages, block_size, Hk, W) with a
 *     per-head slot width W >= 96 bytes; the K slot holds 8 meta bytes at
 *     +0, pad at +8..31 (never written) and the K codes at +32; the V slot
 *     holds the V codes at +0.
 */
#ifndef OSCAR_AMD_H
#define OSCAR_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* oscar_stream_t; /* == hipStream_t */

enum oscar_status {
  OSCAR_OK = 0,
  OSCAR_ERR_INVALID_ARGUMENT = -1,
  OSCAR_ERR_UNSUPPORTED_HEAD_DIM = -2,
  OSCAR_ERR_WORKSPACE_TOO_SMALL = -3,
  OSCAR_ERR_LAUNCH = -4,
  OSCAR_ERR_UNSUPPORTED_GEOMETRY = -5,
};

/* ---------------------------------------------------------------- rotation
 * Prepare the MFMA operand of one orthogonal rotation R [D][D] fp32
 * (x_rot = x @ R).  Replaces the reference's per-call fp32 matmul operand
 * (oscar_ascend/backend.py:130 `torch.matmul(x.float(), R)`, rotations cached
 * per layer at backend.py:228-236).  `operand` must hold
 * oscar_rotation_operand_bytes(D) bytes: the MFMA tiles (bf16 hi + lo split,
 * permuted, 256 KiB), then R itself in fp32 (256 KiB) for short writes.
 */
size_t oscar_rotation_operand_bytes(int32_t head_size);
int oscar_rotation_operand(const float* rotation, void* operand, int32_t head_size,
                           oscar_stream_t stream);

/* Rows rotated on MFMA: out[r] = in[r] @ R for rows of head_size features.
 * Replaces the prefill route's fp32 rotations (oscar_ascend/backend.py:392-413:
 * q / k / v `x.float() @ rk` / `@ rv` before the attention, `out.float() @
 * rv.t()` after it).
 *   in:          [rows][in_row_stride] bf16 (in_f32 = 0) or fp32 (in_f32 = 1);
 *   rot_operand: oscar_rotation_operand of R (of R_v^T for the output);
 *   out:         [rows][out_row_stride] fp32 (out_bf16 = 0) or bf16 (out_bf16 = 1,
 *                rounded to nearest even).
 * fp32 input enters as bf16 high + low parts, R as the operand's parts, with
 * fp32 accumulation: about 2^-16 of each product.  Row starts must be 16-byte
 * aligned.
 */
int oscar_rotate_rows(const void* in, int32_t in_f32, int64_t in_row_stride, int64_t rows, int32_t head_size,
                      const void* rot_operand, void* out, int32_t out_bf16, int64_t out_row_stride,
                      oscar_stream_t stream);

/* ---------------------------------------------------------------- quantize-write
 * Fused rotate + clip + INT2 quantize + pack + paged-slot write.
 * Replaces do_kv_cache_update's _rotate_clip + oscar_store_triton
 * (oscar_ascend/backend.py:150-189, oscar_ascend/kernels/store_kernel.py:247-279).
 *   key_bf16, value_bf16: [num_tokens][token_stride] bf16, the Hk*D features of
 *                         each token first (token_stride in elements);
 *   rot_*_operand:        from oscar_rotation_operand;
 *   slot_mapping:         [num_tokens] int64, slot < 0 skipped (as are slots
 *                         at or beyond num_pages * block_size);
 *   clip_index_*:         sorted-|x| index of the clip threshold
 *                         (min(int(ratio * D), D - 1)), or -1 for no clip.
 * Writes of at most 2048 vectors (2 * num_tokens * num_kv_heads) rotate in
 * fp32 through oscar_step_write's kernel; larger ones on MFMA.
 */
int oscar_quant_write(const void* key_bf16, const void* value_bf16, int64_t num_tokens,
                      int32_t num_kv_heads, int32_t head_size, int64_t token_stride,
                      const void* rot_k_operand, const void* rot_v_operand,
                      const int64_t* slot_mapping, void* k_cache, void* v_cache,
                      int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                      int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                      int64_t v_stride_token, int64_t v_stride_head, int32_t clip_index_k,
                      int32_t clip_index_v, oscar_stream_t stream);

/* Same as oscar_quant_write for input that is already rotated (fp32,
 * [num_tokens][token_stride]); bytes are bit-exact with the reference store
 * given identical rotated input.  Replaces the clip half of _rotate_clip plus
 * oscar_store_ref / oscar_store_triton (backend.py:131-147,
 * store_kernel.py:54-102, 247-279).
 */
int oscar_quant_write_prerotated(const float* k_rot, const float* v_rot, int64_t num_tokens,
                                 int32_t num_kv_heads, int32_t head_size, int64_t token_stride,
                                 const int64_t* slot_mapping, void* k_cache, void* v_cache,
                                 int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                                 int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                                 int64_t v_stride_token, int64_t v_stride_head,
                                 int32_t clip_index_k, int32_t clip_index_v, oscar_stream_t stream);

/* ---------------------------------------------------------------- paged MTP decode
 * Causal multi-token attention of short requests (<= 16 query tokens each)
 * over their INT2 history plus the FP32 staging window, rotated domain.
 * Replaces oscar_paged_attention_triton / _oscar_paged_stage1 +
 * _oscar_decode_stage2 (oscar_ascend/kernels/paged_attention.py:272-360,
 * decode_kernel.py:250-293) with the semantics of oscar_paged_attention_ref
 * (paged_attention.py:41-64).
 *   q_rot [num_tokens][Hq][D], k_new / v_new [num_tokens][Hk][D]: fp32 rotated;
 *   block_table [num_requests][block_table_stride] int32 (block_table_cols used);
 *   query_start_loc [num_requests + 1], seq_lens [num_requests] int32 in HOST
 *     memory (the reference passes them as host lists; they are copied into
 *     the kernel arguments, up to 128 requests per launch, larger batches are
 *     launched in chunks); request i owns query rows [qsl[i], qsl[i+1]) and
 *     history positions 0 .. seq_lens[i] - n_i - 1;
 *   max_query_len / max_history: host upper bounds used to size the grid;
 *   stage_owner [stage_rows][block_size] int64 and the window's fp16 operand
 *     images stage_k_image / stage_v_image, each
 *     [stage_rows][block_size / 32][Hk][16384] (16-byte aligned, written by
 *     the window writes; stage_rows = 0: no window);
 *   tiles_per_split: 32-token tiles per split workgroup (0: automatic, at most 256);
 *   out [num_tokens][Hq][D] fp32 (rotated-V domain);
 *   workspace: >= oscar_paged_decode_workspace_bytes(...) bytes (same
 *     tiles_per_split); sized for one chunk of at most 128 requests.
 *     block_size must be a multiple of 32.
 */
size_t oscar_paged_decode_workspace_bytes(int32_t num_requests, int32_t num_kv_heads,
                                          int32_t num_heads, int32_t max_query_len,
                                          int64_t max_history, int32_t tiles_per_split);
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
                       size_t workspace_size, oscar_stream_t stream);

/* Same decode with the reference's output rotation and cast fused into the
 * merge: out = (attention in the rotated-V domain) @ R_v^T, written as fp32
 * (out_bf16 = 0) or bf16 round-to-nearest-even (out_bf16 = 1) at
 * out[token * out_token_stride + head * D + feature].  Replaces the
 * `.float() @ R_vT` and `.to(query.dtype)` after oscar_paged_attention_triton
 * (oscar_ascend/backend.py:291-295, 313-317).  rot_v_t: R_v^T fp32 [D][D]
 * row-major; other arguments and the workspace as oscar_paged_decode.
 */
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
                               size_t workspace_size, oscar_stream_t stream);

/* The same decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  This entry has no counterpart in the
 * reference.  The split partials live in a file-scope device array of the
 * library, 32 MiB per GPU (held until the process ends); a launch whose
 * partials need more (oscar_paged_decode_workspace_bytes with the same
 * arguments) returns OSCAR_ERR_WORKSPACE_TOO_SMALL and enqueues nothing.  The
 * entry allocates nothing and needs no zeroed memory.  Calls that overlap on
 * one GPU (several streams) share the array and race; the array keeps the
 * last call's partials.  Arguments as oscar_paged_decode.
 * Under graph capture: query_start_loc and seq_lens are read from host
 * memory when the call is made and placed in the kernel arguments, so a
 * captured launch replays the captured step's request layout on every
 * replay; only steps of a fixed layout (same query starts and lengths)
 * replay correctly.
 */
#define OSCAR_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20) /* the device array's size, per GPU */
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
                               int32_t tiles_per_split, float* out, oscar_stream_t stream);

/* ---------------------------------------------------------------- DecodeOnly decode
 * One query token per request over its whole history [0, seq_lens[i]) when
 * the step brings no fresh K/V (key = None).  Replaces
 * AscendOscarAttentionBackendImpl._decode_attention and
 * _decode_attention_windowed (oscar_ascend/backend.py:321-358, 500-611:
 * oscar_decode_triton over the INT2 middle, FP32 sink + staged tail, LSE
 * merge; kernels/decode_kernel.py:41-67, 250-293).
 *   q_rot [num_requests][Hq][D] fp32 rotated; out [num_requests][Hq][D] fp32
 *   rotated-V; seq_lens [num_requests] int32 in HOST memory; caches, block
 *   table and staging as in oscar_paged_decode.  With an arena
 *   (stage_rows > 0) the staged value of position p is used only where the
 *   reference's windowed decode uses it: p < sink_eff when the request is
 *   longer than sink_eff = (sink_tokens / block_size) * block_size and every
 *   seat of its sink pages holds its page, and p >= cut, where [cut, seq)
 *   is the run of staged positions ending at seq - 1 inside
 *   [max(seq - recent_tokens, sink end), seq).  Elsewhere the INT2 value.
 *   workspace: >= oscar_decode_only_workspace_bytes(...) bytes (same
 *   tiles_per_split).
 */
size_t oscar_decode_only_workspace_bytes(int32_t num_requests, int32_t num_kv_heads, int32_t num_heads,
                                         int64_t max_history, int32_t tiles_per_split);
int oscar_decode_only(const float* q_rot, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                      const void* k_cache, const void* v_cache, int32_t block_size, int64_t num_pages,
                      int64_t k_stride_page, int64_t k_stride_token, int64_t k_stride_head,
                      int64_t v_stride_page, int64_t v_stride_token, int64_t v_stride_head,
                      const int32_t* block_table, int64_t block_table_stride, int32_t block_table_cols,
                      const int32_t* seq_lens, int32_t num_requests, int64_t max_history,
                      const int64_t* stage_owner, const void* stage_k_image, const void* stage_v_image,
                      int32_t stage_rows, int32_t sink_tokens, int32_t recent_tokens, float scale,
                      int32_t tiles_per_split, float* out, void* workspace, size_t workspace_size,
                      oscar_stream_t stream);

/* ---------------------------------------------------------------- prefill continuation
 * Causal attention of one request's num_new new tokens over its cached_len
 * INT2 history tokens plus themselves (new token j sees keys 0 .. cached_len
 * + j), f16 MFMA on dequantized tiles, fp32 softmax.  Replaces the dense
 * read path of oscar_ascend/backend.py:361-415 (oscar_full_dequant +
 * _stage_splice + oscar_prefill, kernels/dequant_kernel.py:105-116,
 * kernels/prefill.py:69-72) for one request.
 *   q_rot [num_new][Hq][D], k_new / v_new [num_new][Hk][D]: fp32 rotated;
 *   block_table_row [block_table_cols] int32: the request's pages;
 *   staging as in oscar_paged_decode; out [num_new][Hq][D] fp32 rotated-V.
 */
int oscar_prefill_continuation(const float* q_rot, const float* k_new, const float* v_new,
                               int32_t num_new, int32_t num_heads, int32_t num_kv_heads,
                               int32_t head_size, const void* k_cache, const void* v_cache,
                               int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                               int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                               int64_t v_stride_token, int64_t v_stride_head,
                               const int32_t* block_table_row, int32_t block_table_cols,
                               int64_t cached_len, const float* stage_k, const float* stage_v,
                               const int64_t* stage_owner, int32_t stage_rows, float scale,
                               float* out, oscar_stream_t stream);

/* ---------------------------------------------------------------- step write
 * Everything a short step (num_tokens <= 1024 new tokens, e.g. MTP decode)
 * writes, in one launch: q_rot = query @ R_k, k_rot = key @ R_k, v_rot =
 * value @ R_v (fp32, the read kernels' inputs), the INT2 write of k_rot /
 * v_rot (clip, quantize, pack, slot write; bytes as oscar_quant_write) and,
 * with an arena (stage_rows > 0), the window write of oscar_staging_write
 * (same seat, winner and keep rules; the arena's fp16 operand images are
 * refreshed when given).  Replaces do_kv_cache_update + _staging_write + the
 * q/k/v rotations of the paged read (oscar_ascend/backend.py:150-189,
 * 261-269, 291-295, 439-481) for such steps.
 *   query_bf16 [num_tokens][query_token_stride], key_bf16 / value_bf16
 *     [num_tokens][kv_token_stride] (the Hk * D features of each token first);
 *   rot_k / rot_v fp32 [D][D] (x_rot = x @ R);
 *   query_start_loc [num_requests + 1], seq_lens [num_requests] in HOST memory
 *     (token t of request i sits at seq_lens[i] - query_start_loc[i + 1] + t);
 *   q_rot [num_tokens][Hq][D], k_rot / v_rot [num_tokens][Hk][D] fp32 outputs.
 * num_heads = 0 writes keys and values only (query_bf16 and q_rot unused);
 * a null k_rot / v_rot skips that output.
 */
int oscar_step_write(const void* query_bf16, int64_t query_token_stride, const void* key_bf16,
                     const void* value_bf16, int64_t kv_token_stride, int32_t num_tokens,
                     int32_t num_heads, int32_t num_kv_heads, int32_t head_size, const float* rot_k,
                     const float* rot_v, const int64_t* slot_mapping, const int32_t* query_start_loc,
                     const int32_t* seq_lens, int32_t num_requests, void* k_cache, void* v_cache,
                     int32_t block_size, int64_t num_pages, int64_t k_stride_page,
                     int64_t k_stride_token, int64_t k_stride_head, int64_t v_stride_page,
                     int64_t v_stride_token, int64_t v_stride_head, int32_t clip_index_k,
                     int32_t clip_index_v, float* stage_k, float* stage_v, int64_t* stage_owner,
                     void* stage_k_image, void* stage_v_image, int32_t stage_rows, int32_t sink_eff,
                     int32_t recent, float* q_rot, float* k_rot, float* v_rot, oscar_stream_t stream);

/* ---------------------------------------------------------------- MTP forward
 * The whole forward of one layer for a short step (every request has
 * 1 .. 16 query tokens, at most 1024 tokens in all): oscar_step_write, then
 * oscar_paged_decode_rotated over its q_rot / k_rot / v_rot, on one stream.
 * Replaces the short-step route of the reference's forward
 * (oscar_ascend/backend.py:239-319: the writes at 150-189 and 439-481, the
 * paged read at 273-303 with the rotations and @ R_v^T at 291-295).
 * Arguments and bytes written are those of the two entries; they come in
 * two parts that a caller builds once and reuses:
 *   oscar_mtp_layer: the layer's rotations, caches and window arena (fixed
 *     while the layer lives; stage_rows = 0: no window, the arena pointers
 *     are then ignored);
 *   oscar_mtp_step: the step's request layout (host arrays), slot mapping,
 *     block table and scratch, shared by every layer of the step; q_rot /
 *     k_rot / v_rot are fp32 scratch of num_tokens x num_heads (num_kv_heads)
 *     x D floats, workspace >= oscar_paged_decode_workspace_bytes(num_requests,
 *     num_kv_heads, num_heads, max_query_len, max_history, tiles_per_split).
 * Only the activations and the output pass per call: query_bf16
 * [num_tokens][query_token_stride], key_bf16 / value_bf16
 * [num_tokens][kv_token_stride], out [num_tokens][out_token_stride] bf16
 * (out_bf16 = 1) or fp32 in the model domain.  The layer and the step must
 * agree on num_heads and num_kv_heads.  Every argument is checked before
 * anything is enqueued.
 */
typedef struct oscar_mtp_layer {
  const float* rot_k;            /* [D][D] fp32, x_rot = x @ R_k */
  const float* rot_v;            /* [D][D] fp32 */
  const float* rot_v_t;          /* R_v^T [D][D] fp32, applied to the output */
  void* k_cache;
  void* v_cache;
  int64_t num_pages;
  int64_t k_stride_page, k_stride_token, k_stride_head;   /* bytes */
  int64_t v_stride_page, v_stride_token, v_stride_head;   /* bytes */
  int32_t block_size;
  int32_t num_heads, num_kv_heads, head_size;
  int32_t clip_index_k, clip_index_v;
  float scale;
  int32_t stage_rows;
  float* stage_k;
  float* stage_v;
  int64_t* stage_owner;
  void* stage_k_image;
  void* stage_v_image;
  int32_t sink_eff, recent;
} oscar_mtp_layer;

typedef struct oscar_mtp_step {
  int32_t num_tokens, num_requests, max_query_len;
  int64_t max_history;
  const int32_t* query_start_loc;  /* HOST [num_requests + 1] */
  const int32_t* seq_lens;         /* HOST [num_requests] */
  const int64_t* slot_mapping;     /* [num_tokens] */
  const int32_t* block_table;      /* [num_requests][block_table_stride] */
  int64_t block_table_stride;
  int32_t block_table_cols;
  int32_t num_heads, num_kv_heads;
  int32_t tiles_per_split;         /* 0: automatic */
  float* q_rot;
  float* k_rot;
  float* v_rot;
  void* workspace;
  size_t workspace_size;
} oscar_mtp_step;

int oscar_mtp_forward(const oscar_mtp_layer* layer, const oscar_mtp_step* step, const void* query_bf16,
                      int64_t query_token_stride, const void* key_bf16, const void* value_bf16,
                      int64_t kv_token_stride, void* out, int64_t out_token_stride, int32_t out_bf16,
                      oscar_stream_t stream);

/* ---------------------------------------------------------------- window write
 * Record the step's tokens in the FP32 sink/recent staging arena.
 * Replaces the torch body of _staging_write (oscar_ascend/backend.py:439-481)
 * without host synchronisation.  Token t (< num_tokens, slot >= 0) of request
 * i (query_start_loc[i] <= t < query_start_loc[i+1]) sits at absolute
 * position seq_lens[i] - query_start_loc[i+1] + t and is kept when that is
 * >= seq_lens[i] - recent or < sink_eff.  Per seat ((slot / block_size) %
 * stage_rows, slot % block_size) the highest token index wins: owner = page
 * (kept) or -1, and a kept winner stores key @ rot_k / value @ rot_v (fp32,
 * unclipped).  key/value: bf16 [num_tokens][token_stride]; rot_*: fp32 [D][D];
 * seat_winner: int64 [stage_rows * block_size + 2], zero when allocated and
 * kept by the caller across calls (never reset: a call tags its keys with an
 * epoch it advances in the buffer's last two words).  stage_k_image /
 * stage_v_image (both or neither, block_size % 32 == 0): fp16
 * [stage_rows][block_size / 32][Hk][16384] each (the fp16 rounding of each
 * value and the fp16 rounding of what it left: K as two 8192-half images, V
 * as the two parts of each lane's 8 slots); a kept winner also writes its
 * values there in the decode kernel's MFMA operand order.
 */
int oscar_staging_write(const void* key_bf16, const void* value_bf16, int64_t token_stride,
                        const int64_t* slot_mapping, int32_t num_tokens,
                        const int32_t* query_start_loc, const int32_t* seq_lens,
                        int32_t num_requests, int32_t num_kv_heads, int32_t head_size,
                        int32_t block_size, int32_t stage_rows, int32_t sink_eff, int32_t recent,
                        const float* rot_k, const float* rot_v, float* stage_k, float* stage_v,
                        int64_t* stage_owner, int64_t* seat_winner, void* stage_k_image,
                        void* stage_v_image, oscar_stream_t stream);

/* A prefill-sized step's whole write: oscar_quant_write and the window write
 * of oscar_staging_write from the same rotated values, in two launches (a
 * seat-winner pass over the step's slots, then the fused quantize-write
 * kernel, whose epilogue writes the owner tags, the staged values and their
 * images).  Replaces do_kv_cache_update followed by _staging_write
 * (oscar_ascend/backend.py:150-189, 439-481).  Arguments: those of
 * oscar_quant_write, then the step's request layout and the arena as for
 * oscar_staging_write (stage_rows > 0).  The staged values are the fused
 * kernel's MFMA rotation (the bf16 high + low split of R), which differs from
 * an fp32 x @ R by about 2^-17 of the values' scale.  Writes of at most 2048
 * vectors take oscar_step_write's kernel, window write included, in one
 * launch.
 */
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
                             void* stage_k_image, void* stage_v_image, oscar_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OSCAR_AMD_H */
