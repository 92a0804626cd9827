/*
 * starkv_hip.h -- C ABI of the MI355X (gfx950) STAR-KV paged decode library.
 *
 * Everything crosses this boundary as plain pointers, element/byte strides and
 * ints; no framework types. Device pointers are HIP device memory on the current
 * device, `stream` is a hipStream_t (NULL = the null stream). Every call only
 * enqueues work: no host synchronisation, no host reads of device data, and the
 * launch grid depends only on host ints, so the calls can be captured in a HIP
 * graph. Each function returns 0 on success and a nonzero STARKV_ERR_* code on a
 * bad argument or a HIP error; starkv_last_error() then holds the message (per
 * host thread).
 *
 * Dtype codes: STARKV_F32, STARKV_F16, STARKV_BF16.
 */
#ifndef STARKV_HIP_H
#define STARKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STARKV_F32 0
#define STARKV_F16 1
#define STARKV_BF16 2

/* Cache kinds of starkv_decode_workspace_bytes / starkv_decode_two_pass: STARKV_BF16 or
 * STARKV_F16 low-rank codes, or the 3.2-bit QuantRow cache. */
#define STARKV_CACHE_Q3_2 16

#define STARKV_OK 0
#define STARKV_ERR_ARG 1
#define STARKV_ERR_HIP 2
#define STARKV_ERR_UNSUPPORTED 3

/* Library ABI version (bumped on any signature change). */
int starkv_abi_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char *starkv_last_error(void);

/*
 * bf16/fp16 cache write: cache[slot // block_size, slot % block_size, :] =
 * cat(k_codes[i], v_codes[i]) cast to the cache dtype; slot < 0 -> slot 0 (the
 * null block). Replaces the inline index_put of the bf16 write branch in
 * StarKVAttentionImpl.forward, starkv_serve/attention.py:180-184.
 *   k_codes  [n, k_width], row stride k_s0 elements, last dim contiguous
 *   v_codes  [n, v_rank],  row stride v_s0 elements, last dim contiguous
 *   cache    [num_blocks, block_size, k_width + v_rank] with element strides c_s0, c_s1
 *   slot_mapping [n] int32 (slot_bits = 32) or int64 (slot_bits = 64); slots at or past
 *   num_blocks * block_size are skipped (the reference would write past the cache)
 */
int starkv_write_codes(void *stream, const void *k_codes, int64_t k_s0, const void *v_codes,
                       int64_t v_s0, int in_dtype, void *cache, int64_t c_s0, int64_t c_s1,
                       int cache_dtype, int block_size, int64_t num_blocks, const void *slot_mapping,
                       int slot_bits, int n, int k_width, int v_rank);

/*
 * Fused cache write of one layer step: codes = hidden @ kv_down^T (fp32 accumulate,
 * rounded to the model dtype with round-to-nearest-even, as F.linear returns them),
 * then either the bf16/fp16 scatter (row_bytes == 0) or the 3.2-bit quantize + scatter
 * (row_bytes == QuantRow.nbytes). Up to 256 tokens: split-K partial products, then a
 * store launch; one token (hidden_size a multiple of 512, at most 4096) or two (hidden_size
 * 4096): one launch whose workgroups own whole codes and store them (bf16/fp16 rows, the
 * 3.2-bit K blocks), then for a 3.2-bit row one launch that packs the V latent. Replaces
 * the code GEMM of
 * StarKVLlamaAttention.forward, starkv_serve/model.py:71 (kv = F.linear(hidden,
 * kv_down), kv_down = cat(k_down, v_down) from attention.py:161), followed by the cache
 * write of StarKVAttentionImpl.forward, starkv_serve/attention.py:179-188 (cat +
 * index_put, or pack_kv = paged_quant.py:205-216; the 3.2-bit rows are bit for bit
 * pack_kv of the rounded codes).
 *   hidden    [n, hidden_size], row stride h_s0 elements, bf16 or fp16 (w_dtype)
 *   kv_down   [k_width + v_rank, hidden_size], row stride w_s0, same dtype; rows 16-byte
 *             aligned, hidden_size a multiple of 64
 *   cache     row_bytes == 0: [num_blocks, block_size, >= k_width + v_rank] of the model
 *             dtype (cache_dtype == w_dtype), element strides c_s0, c_s1;
 *             row_bytes > 0: uint8 [num_blocks, block_size, row_bytes], byte strides
 *   slot_mapping [n] int32 / int64 (slot_bits); slot < 0 -> slot 0 (the null block);
 *             slots at or past num_blocks * block_size are skipped
 *   k_ranks / k_offsets / k_nouts [num_kv_heads] int32 device arrays (3.2-bit only)
 *   codes_out [n, k_width + v_rank] of the model dtype, row stride co_s0, or NULL: the
 *             rounded codes (what F.linear returns)
 *   workspace >= starkv_write_kv_workspace_bytes(n, k_width + v_rank, hidden_size) bytes,
 *             16-byte aligned (fp32 split-K partials, or the direct form's rounded codes
 *             and V maxima)
 */
size_t starkv_write_kv_workspace_bytes(int n, int width, int hidden_size);
int starkv_write_kv(void *stream, const void *hidden, int64_t h_s0, const void *kv_down, int64_t w_s0,
                    int w_dtype, int n, int hidden_size, int k_width, int v_rank, void *cache, int64_t c_s0,
                    int64_t c_s1, int cache_dtype, int block_size, int64_t num_blocks,
                    const void *slot_mapping, int slot_bits, int num_kv_heads, const int32_t *k_ranks,
                    const int32_t *k_offsets, const int32_t *k_nouts, int row_bytes, void *codes_out,
                    int64_t co_s0, void *workspace, size_t workspace_bytes);

/*
 * starkv_write_kv with its launches deferred to the calling thread's next decode call on
 * the same stream (starkv_lowrank_decode, starkv_quant_decode and their group and
 * no-alloc forms): that call runs the write's code GEMM inside its own first launch (the
 * page plan and query fold, which do not depend on the write), then the write's store,
 * then its decode kernels, so a decode step's write and decode take one launch fewer. A
 * write of the direct form (one or two tokens, above) has no store launch: its 3.2-bit V
 * latent is packed by the decode's logits pass when the decode is two-pass (P @ V, a later
 * launch, is the first reader of V), else by its own launch; the write and decode of one
 * token then take two launches fewer.
 * Same arguments, checks and results as starkv_write_kv; the reference has no
 * counterpart (its write and decode are separate framework calls, attention.py:179-217).
 * Until the write is launched, hidden, kv_down, the slot mapping, the head arrays and the
 * workspace must stay valid and unchanged. A pending write is also launched, on its own
 * stream and in its own launches, by the thread's next write call (deferred or not), by
 * a decode call on another stream or one that fails its checks, and by
 * starkv_flush_write. One write per thread can be pending.
 */
int starkv_write_kv_deferred(void *stream, const void *hidden, int64_t h_s0, const void *kv_down, int64_t w_s0,
                             int w_dtype, int n, int hidden_size, int k_width, int v_rank, void *cache,
                             int64_t c_s0, int64_t c_s1, int cache_dtype, int block_size, int64_t num_blocks,
                             const void *slot_mapping, int slot_bits, int num_kv_heads, const int32_t *k_ranks,
                             const int32_t *k_offsets, const int32_t *k_nouts, int row_bytes, void *codes_out,
                             int64_t co_s0, void *workspace, size_t workspace_bytes);

/* Launches the calling thread's deferred write, if one is pending (no counterpart in the
 * reference: the pair of starkv_write_kv_deferred). */
int starkv_flush_write(void);

/*
 * 3.2-bit write path: quantize one row per token (per-KV-head 4-bit outlier /
 * 3-bit inlier K blocks with bf16 scales, then the head-shared V latent) and
 * scatter it into its slot, bit for bit kv_quant._q (IEEE fp32 division,
 * round-half-even). Replaces starkv_serve/kernels/paged_quant.py:205-216
 * (pack_kv -> _pack_k 146-172, _pack_v 175-202). The row layout is QuantRow
 * (paged_quant.py:71-111) for (k_width, num_kv_heads, v_rank); row_bytes must
 * equal QuantRow.nbytes. Bytes [vq_off + v_bytes, row_bytes) are written as 0.
 *   k_codes [n, k_width], v_codes [n, v_rank] (dtype code_dtype, rows strided)
 *   cache   uint8 [num_blocks, block_size, row_bytes], byte strides c_s0, c_s1
 *   k_ranks / k_offsets / k_nouts  [num_kv_heads] int32 device arrays
 *   slots at or past num_blocks * block_size are skipped
 */
int starkv_pack_kv(void *stream, const void *k_codes, int64_t k_s0, const void *v_codes, int64_t v_s0,
                   int code_dtype, uint8_t *cache, int64_t c_s0, int64_t c_s1, int block_size,
                   int64_t num_blocks, const void *slot_mapping, int slot_bits, int n, int num_kv_heads,
                   const int32_t *k_ranks, const int32_t *k_offsets, const int32_t *k_nouts,
                   int k_width, int v_rank, int row_bytes);

/*
 * Fold the query into U: AB[b, r, i] = (q_i U[r,i] + q_{i+64} U[r,i+64]) * scale and
 * AB[b, r, 64 + i] = (q_{i+64} U[r,i] - q_i U[r,i+64]) * scale, i < 64, q of head
 * head_of_lane[r], stored fp16 [n, k_width, 128] contiguous. Replaces
 * starkv_serve/kernels/paged_quant.py:241-255 (fold_q). The decode entry points
 * below fold internally and do not need this; it is kept for the reference API.
 */
int starkv_fold_q(void *stream, const void *q, int64_t q_s0, int64_t q_s1, int q_dtype, const void *k_up,
                  int64_t ku_s0, int ku_dtype, const int32_t *head_of_lane, int n, int k_width,
                  float scale, void *ab);

/*
 * Grid (workgroups) the decode calls below use on the current device for n
 * requests bounded by max_seq_len: min(CUs, max(n, ceil(n * max_seq_len / 256))).
 * A pure function of (device, n, max_seq_len).
 */
int starkv_decode_grid(int n, int max_seq_len);

/*
 * The grid for one layer's calls: starkv_decode_grid's rule with 64 tokens per
 * workgroup. For a layer that decodes in two passes (V ranks too wide for one pass; see
 * starkv_decode_two_pass) this is the logits pass's grid; the P @ V pass takes ranges of
 * R of its ranges (R from the cache kind, n, max_seq_len and the grid, 1 to 4). A pure
 * function of its arguments and the device.
 * This build's Python wrappers take their grid from it (no counterpart in the
 * reference, whose Triton launches size their own grids, paged_decode.py:192-219).
 */
int starkv_decode_grid_for(int cache_kind, int n, int num_heads, int num_kv_heads, int k_width, int v_rank,
                           int max_seq_len);

/*
 * Workspace bytes a decode call needs: the page prefix sums, the page records (16 bytes
 * per request and page of max_seq_len), the wave plan, the q-folded bases (4 KiB per request and 16-lane rank tile), the split-K partials
 * ((grid + n) x num_heads x (v_rank + 2) fp32) and, for the two-pass form, the logits
 * (n x num_heads x max_seq_len rounded up to 16, fp32). cache_kind: STARKV_BF16,
 * STARKV_F16 or STARKV_CACHE_Q3_2 (num_kv_heads = num_heads). 0 for invalid sizes.
 */
size_t starkv_decode_workspace_bytes(int cache_kind, int n, int num_heads, int num_kv_heads, int k_width,
                                     int v_rank, int max_seq_len, int grid);

/*
 * 1 if a decode of this layer shape runs in two passes, else 0 (num_kv_heads = num_heads
 * for the 3.2-bit cache). The one-pass decode keeps P @ V in the decode kernel and takes
 * v_rank <= 256 (bf16/fp16) or up to five 64-lane blocks of outlier (padded to 4) plus
 * inlier columns (3.2-bit), where a kernel instantiation holds the layer's rank tiles per
 * wave (all but one of them at least) without scratch spills. Other V ranks (up to 4096)
 * run a logits pass and a P @ V pass, as the reference's paged_decode.py:199-219 /
 * paged_quant.py:390-407 split their V pass. Both forms give the same results to within
 * rounding.
 */
int starkv_decode_two_pass(int cache_kind, int num_heads, int num_kv_heads, int k_width, int v_rank);

/*
 * 1 if one decode call takes a layer of this shape, else 0 (host function, no device
 * access; call it at load time). k_ranks: host array of the num_kv_heads K ranks. One
 * call is refused when it has more than 32 query heads, more than 96 16-lane rank tiles
 * over its query heads ((num_heads / num_kv_heads) x k_width / 16), a wave of the decode
 * kernel's 8 that would hold more than 16 tiles after the wave plan balances whole heads,
 * v_rank above 4096, or (3.2-bit) num_kv_heads != num_heads. A decode call over a shape
 * refused here returns NaN rows; starkv_decode_layer_groups splits such a layer into
 * calls that fit. No counterpart in the reference, whose Triton kernels take any head
 * count.
 */
int starkv_decode_layer_fits(int cache_kind, int num_heads, int num_kv_heads, const int32_t *k_ranks, int v_rank);

/*
 * How a layer is decoded: as `count` calls over consecutive KV-head ranges, written to
 * groups[2 i], groups[2 i + 1] = [first, end) for i < count (host function, no device
 * access; call it at load time). Returns count >= 1 (1: the whole layer in one call),
 * 0 if some single KV head does not fit one call (or more than max_groups ranges are
 * needed), -1 for invalid arguments. Ranges are greedy: each as long as one call takes
 * (starkv_decode_layer_fits' limits on that range). bf16/fp16 calls over a range get
 * the cache pointer advanced to its first K lane and its V codes through v_col
 * (starkv_lowrank_decode); 3.2-bit calls go through starkv_quant_decode_group. No
 * counterpart in the reference, whose Triton kernels take any head count
 * (paged_quant.py:357-411 sizes its V block by next_pow2(H), :407).
 */
int starkv_decode_layer_groups(int cache_kind, int num_heads, int num_kv_heads, const int32_t *k_ranks, int v_rank,
                               int32_t *groups, int max_groups);

/*
 * Forces the decode form for the calls that follow (process-wide, not thread-safe; for
 * tests and benchmarks that compare the two): 0 = automatic (default), 1 = one-pass
 * only (shapes it cannot take are refused), 2 = two-pass always. Returns the previous
 * mode, or -1 for an invalid mode. No counterpart in the reference.
 */
int starkv_decode_set_path(int mode);

/*
 * bf16/fp16 low-rank paged decode. Replaces
 * starkv_serve/kernels/paged_decode.py:150-226 (paged_starkv_decode).
 * Per request b, query head h and token l < min(seq_lens[b], max_seq_len):
 *   logit = scale * q[b,h] . RoPE_l(U_kv^T x_l),  x_l = the first k_ranks[kv] codes of
 *   KV head kv = h / (H_q / H_kv) at lane k_head_offsets[kv] of the token's cache row,
 *   out[b,h] = (softmax(logit) @ V_codes) @ v_up_by_q[h].
 *   query       [n, H_q, 128] (element strides q_s0, q_s1; last dim contiguous)
 *   kv_cache    [num_blocks, block_size, >= v_col + v_rank], element strides c_s0, c_s1,
 *               last dim contiguous; code_dtype bf16 or fp16; block_size 16 * 2^s. From
 *               the pointer, a row holds the K lanes the call reads (k_width of them, at
 *               k_head_offsets) and the V codes at lane v_col: v_col = k_width for a
 *               [K | V] row; a caller that splits a layer's KV heads over calls (more than
 *               32 query heads or 96 rank tiles) advances the pointer to a group's first
 *               K lane and passes the distance from there to V (v_col >= k_width,
 *               a multiple of 8)
 *   block_table [n, max_blocks] int32 (strides bt_s0, bt_s1); seq_lens [n] int32
 *   k_up        [k_width, 128] (row stride ku_s0, dtype w_dtype), k_ranks /
 *               k_head_offsets [H_kv] int32
 *   v_up_by_q   [H_q, v_rank, 128] (strides vu_s0, vu_s1, dtype vu_dtype; v_rank <= 4096)
 *   cos_sin     [>= max_seq_len, 128] = cat(cos, sin) (row stride cs_s0), fp16
 *   out         [n, H_q, 128] (strides o_s0, o_s1), dtype out_dtype
 *   workspace   >= starkv_decode_workspace_bytes(code_dtype, n, H_q, H_kv, k_width, v_rank,
 *               max_seq_len, grid) bytes, 256-byte aligned; grid from
 *               starkv_decode_grid_for(...) (or any grid >= 1)
 * A request with no tokens (seq_lens <= 0) gets NaN rows, as the reference's softmax
 * over an empty row does.
 */
int starkv_lowrank_decode(void *stream, const void *query, int64_t q_s0, int64_t q_s1, int q_dtype,
                          const void *kv_cache, int64_t c_s0, int64_t c_s1, int code_dtype, int block_size,
                          const int32_t *block_table, int64_t bt_s0, int64_t bt_s1, const int32_t *seq_lens,
                          int n, int num_heads, int num_kv_heads, int max_seq_len, const void *k_up,
                          int64_t ku_s0, int w_dtype, const int32_t *k_ranks, const int32_t *k_head_offsets,
                          int k_width, int v_col, const void *v_up_by_q, int64_t vu_s0, int64_t vu_s1,
                          int vu_dtype, int v_rank, const void *cos_sin, int64_t cs_s0, int cs_dtype, float scale,
                          void *out, int64_t o_s0, int64_t o_s1, int out_dtype, void *workspace,
                          size_t workspace_bytes, int grid);

/*
 * starkv_lowrank_decode with no workspace argument and no allocation: the call's
 * workspace is a fixed 64 MiB array of device memory inside the library (one per
 * device, held until the process ends), so callers that cannot allocate (code under
 * HIP graph capture, serving loops that forbid allocation) can decode. A call whose
 * starkv_decode_workspace_bytes exceeds 64 MiB is refused with an error (for example
 * 64 requests x 8192 tokens fit in one-pass form, k_width 1280 / v_rank 64: ~23 MiB).
 * Every call on one device shares that array: calls that overlap on one device (other
 * streams, other host threads) race, so serialize them. Nothing in it needs clearing
 * between calls. No counterpart in the reference; it exists for callers that cannot
 * allocate. Arguments as starkv_lowrank_decode.
 */
int starkv_lowrank_decode_noalloc(void *stream, const void *query, int64_t q_s0, int64_t q_s1, int q_dtype,
                                  const void *kv_cache, int64_t c_s0, int64_t c_s1, int code_dtype,
                                  int block_size, const int32_t *block_table, int64_t bt_s0, int64_t bt_s1,
                                  const int32_t *seq_lens, int n, int num_heads, int num_kv_heads,
                                  int max_seq_len, const void *k_up, int64_t ku_s0, int w_dtype,
                                  const int32_t *k_ranks, const int32_t *k_head_offsets, int k_width, int v_col,
                                  const void *v_up_by_q, int64_t vu_s0, int64_t vu_s1, int vu_dtype, int v_rank,
                                  const void *cos_sin, int64_t cs_s0, int cs_dtype, float scale, void *out,
                                  int64_t o_s0, int64_t o_s1, int out_dtype, int grid);

/*
 * 3.2-bit paged decode over the QuantRow cache. Replaces
 * starkv_serve/kernels/paged_quant.py:357-411 (paged_quant_decode: fold_q,
 * _paged_abx_z, softmax, _paged_pv_fold, lift). MHA, head_dim 128.
 *   kv_cache    uint8 [num_blocks, block_size, row_bytes], byte strides c_s0, c_s1
 *   tile_head / tile_nout / tile_last  [k_width / 16] int32 (k_tables' per-16-lane tiles)
 *   workspace   >= starkv_decode_workspace_bytes(STARKV_CACHE_Q3_2, n, H, H, k_width, v_rank,
 *               max_seq_len, grid) bytes
 *   other arguments as starkv_lowrank_decode.
 */
int starkv_quant_decode(void *stream, const void *query, int64_t q_s0, int64_t q_s1, int q_dtype,
                        const uint8_t *kv_cache, int64_t c_s0, int64_t c_s1, int block_size,
                        const int32_t *block_table, int64_t bt_s0, int64_t bt_s1, const int32_t *seq_lens,
                        int n, int num_heads, int max_seq_len, int k_width, int v_rank, int row_bytes,
                        const void *k_up, int64_t ku_s0, int w_dtype, const int32_t *tile_head,
                        const int32_t *tile_nout, const int32_t *tile_last, const void *v_up_by_q,
                        int64_t vu_s0, int64_t vu_s1, int vu_dtype, const void *cos_sin, int64_t cs_s0,
                        int cs_dtype, float scale, void *out, int64_t o_s0, int64_t o_s1, int out_dtype,
                        void *workspace, size_t workspace_bytes, int grid);

/*
 * starkv_quant_decode over query heads [head0, head0 + num_heads) of a layer whose rows
 * are QuantRow(row_k_width, row_num_heads, v_rank) (row_bytes its nbytes): the heads' K
 * nibbles start at K lane k_lane0 (a multiple of 16) and span k_width lanes. kv_cache
 * points at the rows (as for the whole layer); query, k_up (the group's k_width rows),
 * tile_head / tile_nout / tile_last (from the group's first tile: tile_head values are
 * the layer's head indices), v_up_by_q and out cover the group's heads only. The call
 * reads its heads' K nibbles and K scales and the whole V block. The whole-layer call
 * is row_k_width = k_width, row_num_heads = num_heads, head0 = k_lane0 = 0.
 *   workspace   >= starkv_quant_group_workspace_bytes(...) bytes
 * Layers beyond one call's limits (more than 32 heads or 96 rank tiles) run as such
 * groups (starkv_decode_layer_groups); the reference's Triton path takes them in one
 * launch (paged_quant.py:357-411).
 */
int starkv_quant_decode_group(void *stream, const void *query, int64_t q_s0, int64_t q_s1, int q_dtype,
                              const uint8_t *kv_cache, int64_t c_s0, int64_t c_s1, int block_size,
                              const int32_t *block_table, int64_t bt_s0, int64_t bt_s1, const int32_t *seq_lens,
                              int n, int num_heads, int max_seq_len, int k_width, int v_rank, int row_bytes,
                              const void *k_up, int64_t ku_s0, int w_dtype, const int32_t *tile_head,
                              const int32_t *tile_nout, const int32_t *tile_last, const void *v_up_by_q,
                              int64_t vu_s0, int64_t vu_s1, int vu_dtype, const void *cos_sin, int64_t cs_s0,
                              int cs_dtype, float scale, void *out, int64_t o_s0, int64_t o_s1, int out_dtype,
                              void *workspace, size_t workspace_bytes, int grid, int row_k_width,
                              int row_num_heads, int head0, int k_lane0);

/* Workspace bytes of starkv_quant_decode_group (0 for invalid sizes). */
size_t starkv_quant_group_workspace_bytes(int n, int row_k_width, int row_num_heads, int v_rank, int head0,
                                          int num_heads, int k_lane0, int k_width, int max_seq_len, int grid);

/* 1 if starkv_quant_decode_group over this group runs in two passes, else 0. */
int starkv_quant_group_two_pass(int row_k_width, int row_num_heads, int v_rank, int head0, int num_heads,
                                int k_lane0, int k_width);

/*
 * The step's K and V of uncompressed layers into vLLM's paged caches
 * [num_blocks, block_size, H_kv, 128] (what vLLM's reshape_and_cache does before its
 * paged attention, the reference's stock layers: starkv_serve/model.py:77-81):
 *   key, value    [n, H_kv, 128] bf16/fp16 (element strides k_s0, k_s1 / v_s0, v_s1;
 *                 head dim contiguous), dtype as the caches'
 *   k_cache, v_cache  element strides c_s0 (block), c_s1 (slot), c_s2 (head)
 *   slot_mapping  [n] int32 or int64 (slot_bits 32 / 64); slot -1 writes nothing
 * One launch for both caches.
 */
int starkv_stock_write(void *stream, const void *key, int64_t k_s0, int64_t k_s1, const void *value, int64_t v_s0,
                       int64_t v_s1, int dtype, void *k_cache, void *v_cache, int64_t c_s0, int64_t c_s1,
                       int64_t c_s2, int block_size, int64_t num_blocks, const void *slot_mapping, int slot_bits,
                       int n, int num_kv_heads);

/*
 * Uncompressed paged decode attention over bf16/fp16 K and V caches
 * [num_blocks, block_size, num_kv_heads, 128] (element strides c_s0, c_s1, c_s2, last
 * dimension contiguous): out[b, h] = softmax(scale q[b, h] . K[b, :L]) V[b, :L], L =
 * min(seq_lens[b], max_seq_len) (NaN rows for L = 0). It stands in for the stock
 * attention backend the reference runs its uncompressed layers on
 * (starkv_serve/model.py:77-81 builds vLLM's LlamaAttention for them; the reference has
 * no code of its own for it), and is the stock bf16 comparator of the benchmarks.
 * num_heads / num_kv_heads in {1, 2, 4, 8}; block_size 16 * 2^s; workspace >=
 * starkv_stock_decode_workspace_bytes(n, num_heads, num_kv_heads, max_seq_len) bytes.
 */
size_t starkv_stock_decode_workspace_bytes(int n, int num_heads, int num_kv_heads, int max_seq_len);
int starkv_stock_decode(void *stream, const void *query, int64_t q_s0, int64_t q_s1, int q_dtype,
                        const void *k_cache, const void *v_cache, int64_t c_s0, int64_t c_s1, int64_t c_s2,
                        int cache_dtype, int block_size, const int32_t *block_table, int64_t bt_s0,
                        int64_t bt_s1, const int32_t *seq_lens, int n, int num_heads, int num_kv_heads,
                        int max_seq_len, float scale, void *out, int64_t o_s0, int64_t o_s1, int out_dtype,
                        void *workspace, size_t workspace_bytes);

/*
 * Dense causal prefill attention of a STAR-KV layer: the attention half of the reference's
 * _dense_prefill (starkv_serve/attention.py:219-251, its flash_attn_varlen_func call with
 * causal=True, attention.py:243-249), over K and V already lifted from the step's codes.
 * Every prompt attends to itself only (no cached context): for token t of the prompt that
 * starts at s, out[t, h] = softmax(scale q[t, h] . K[s .. t, h / G]) V[s .. t, h / G] with
 * G = num_heads / num_kv_heads. query [T, num_heads, 128] (bf16, fp16 or fp32, element
 * strides q_s0, q_s1); key and value [T, num_kv_heads, 128] fp16 sharing element strides
 * (kv_s0, kv_s1); cu_seqlens [num_prompts + 1] int32 on the device (the prompts' first
 * tokens, then T); out [T, num_heads, 128] (element strides o_s0, o_s1). head_size 128.
 * blocks: num_blocks (prompt, 128-row query block) pairs on the device, as
 * starkv_prefill_block_list writes them on the host from a host copy of cu_seqlens
 * (it returns the count and writes at most `capacity` pairs; -1 for a bad prefix).
 */
int starkv_prefill_block_list(const int32_t *cu_seqlens, int num_prompts, int32_t *blocks, int capacity);
int starkv_prefill_attention(void *stream, const void *query, int64_t q_s0, int64_t q_s1, int q_dtype,
                             const void *key, const void *value, int64_t kv_s0, int64_t kv_s1, int kv_dtype,
                             const int32_t *cu_seqlens, const int32_t *blocks, int num_blocks, int num_heads,
                             int num_kv_heads, int head_size, float scale, void *out, int64_t o_s0, int64_t o_s1,
                             int out_dtype);

/*
 * Timing for benchmarks (no counterpart in the reference, whose benchmark reads profiler
 * traces instead, bench_serving.py:71-115). starkv_profile_begin arms up to max_calls
 * event pairs; each following decode call records one pair on its stream, around its
 * decode kernels (mode 0: the one-pass kernel, or the logits and P @ V passes) or around
 * the whole call (mode 1: from the prep launch to the merge). The events are created
 * without the system-scope fence. starkv_profile_end synchronizes them, returns the
 * summed milliseconds and the number of timed calls, and disarms; starkv_profile_times
 * then copies up to max per-call milliseconds and returns how many. Not for use under
 * graph capture.
 */
int starkv_profile_begin(int max_calls, int mode);
int starkv_profile_end(double *decode_ms_sum, int *calls);
int starkv_profile_times(double *ms, int max);

#ifdef __cplusplus
}
#endif

#endif /* STARKV_HIP_H */
