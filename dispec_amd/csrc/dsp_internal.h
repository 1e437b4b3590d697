// Entry points shared between the library's translation units (not part of the C ABI).
#pragma once

#include "dsp_common.h"

namespace dsp_detail {

// Compute units of the current device (256 if the query fails).
int device_cus();

// Block-table decode on the multi-query MFMA kernel (paged_mq.hip) with q_len 1 per
// sequence.  The caller (dsp_paged_decode) has validated the arguments; the kernel writes
// partial results as ws_acc[(b * Hq + h) * num_parts + part][D] and ws_ml[...][2] (row max,
// row sum) and the caller's combine kernel merges them.  P must be a multiple of 32.
int mq_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
              const uint16_t* v_cache, int64_t num_slots, int64_t kv_stride_slot,
              int64_t kv_stride_head, const int32_t* block_table, int64_t bt_stride,
              int32_t log2_bs, const int32_t* ctx_lens, int32_t B, int32_t KVH, int32_t G,
              int32_t D, float scale_log2, int32_t max_ctx, int32_t P, int32_t num_parts,
              float* ws_acc, float* ws_ml, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
              bool f16, int32_t* err_count, hipStream_t s);

// Balanced split-K attention on block tables (decode_balanced.hip): every wave of the
// launch takes an equal share of the (sequence, KV head, 16-key unit) work.  Decode:
// cu_q null, max_q_len 1, q/out rows indexed by sequence.  Multi-query (verify): cu_q as
// for dsp_paged_mq_attention, max_q_len * G <= 16 query rows per KV head, q/out rows
// indexed by token.  `applies` says whether the shape is one it serves; the workspace is
// balanced_workspace_bytes(..., max_q_len * G, ...) long.
bool balanced_decode_applies(int32_t B, int32_t KVH, int32_t D, int32_t max_ctx,
                             int32_t block_size);
int32_t balanced_workers(int32_t B, int32_t KVH, int32_t max_ctx);
int balanced_head_group(int32_t KVH);
size_t balanced_workspace_bytes(int32_t B, int32_t KVH, int32_t rows_per_head, int32_t D,
                                int32_t max_ctx);
int balanced_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                    const uint16_t* k_cache, const uint16_t* v_cache, int64_t num_slots,
                    int64_t kv_stride_slot, int64_t kv_stride_head, const int32_t* block_table,
                    int64_t bt_stride, int32_t log2_bs, const int32_t* ctx_lens,
                    const int32_t* cu_q, int32_t max_q_len, int32_t B, int32_t KVH, int32_t G,
                    int32_t D, float scale_log2, int32_t max_ctx, float* workspace,
                    uint16_t* out, int64_t o_stride_b, int64_t o_stride_h, bool f16,
                    int32_t* err_count, hipStream_t s);

// Long query blocks (chunked prefill) on the 128-row FlashAttention-style tile
// (paged_prefill.hip): the semantics, arguments and workspace layout of
// dsp_paged_mq_attention, whose entry point has validated them and routes here when
// `prefill_applies`; partial results go to the 16-row-tile layout its merge kernel reads
// (tiles16_max 16-row tiles per (sequence, KV head)).  P must be a multiple of 64.
bool prefill_applies(int32_t D, int32_t block_size, int64_t max_rows, int64_t num_slots,
                     int64_t kv_stride_slot);
int64_t prefill_tiles(int32_t max_q_len, int32_t G);
int prefill_attention(const uint16_t* q, int64_t q_stride_t, int64_t q_stride_h,
                      const uint16_t* k_cache, const uint16_t* v_cache, int64_t num_slots,
                      int64_t kv_stride_slot, int64_t kv_stride_head, const int32_t* block_table,
                      int64_t bt_stride, int32_t log2_bs, const int32_t* cu_q,
                      const int32_t* ctx_lens, int32_t B, int32_t KVH, int32_t G, int32_t D,
                      float scale_log2, int32_t max_q_len, int32_t max_ctx, int32_t P,
                      int32_t num_parts, int32_t tiles16_max, float* ws_acc, float* ws_ml,
                      uint16_t* out, int64_t o_stride_t, int64_t o_stride_h, bool f16,
                      int32_t* err_count, hipStream_t s);

// dsp_paged_mq_attention_shared_prefix in one launch: prefix tiles (every query row of the
// batch, token-major via cu_q, against the first prefix_tokens keys of block-table row 0,
// in prefix_tokens / P partitions) beside suffix tiles (each sequence's rows over its keys
// from prefix_tokens on, causal, in partitions of P numbered on from the prefix's); partial
// results in the merge layout, ceil(max_ctx / P) partitions per 16-row tile.  A sequence with
// bad lengths or ctx - q_len < prefix_tokens is counted and zeroed.  `applies` says
// whether the shape is served; `grid` is the launch's workgroups per KV head.
bool shared_prefix_applies(int32_t D, int32_t block_size, int32_t B, int64_t num_slots,
                           int64_t kv_stride_slot);
int64_t shared_prefix_grid(int32_t B, int32_t G, int32_t max_q_len, int32_t max_ctx, int32_t P,
                           int32_t prefix_tokens);
int prefill_shared_prefix(const uint16_t* q, int64_t q_stride_t, int64_t q_stride_h,
                          const uint16_t* k_cache, const uint16_t* v_cache, int64_t num_slots,
                          int64_t kv_stride_slot, int64_t kv_stride_head,
                          const int32_t* block_table, int64_t bt_stride, int32_t log2_bs,
                          const int32_t* cu_q, const int32_t* ctx_lens, int32_t B, int32_t KVH,
                          int32_t G, int32_t D, float scale_log2, int32_t max_q_len,
                          int32_t max_ctx, int32_t P, int32_t tiles16_max,
                          int32_t prefix_tokens, float* ws_acc, float* ws_ml, uint16_t* out,
                          int64_t o_stride_t, int64_t o_stride_h, bool f16, int32_t* err_count,
                          hipStream_t s);

// Attention for shapes outside the tuned kernels (generic_attn.hip): fp32 caches, head
// dims 8..256 (powers of two), any GQA group.  Decode: cu_q null, max_q_len 1, one row per
// sequence with its context clamped to [0, max_ctx]; multi-query: the semantics of
// dsp_paged_mq_attention.  log2_bs < 0 reads `table` as a per-token slot table.  Partial
// results need generic_workspace_bytes(B, Hq, D, max_q_len, max_ctx, P) bytes of `workspace`
// (none for a single partition).  Grid limits: B * max_q_len <= 2^26, ceil(max_ctx / P) <=
// 65535 (else DSP_EUNSUPPORTED).
bool generic_head_dim(int32_t D);
size_t generic_workspace_bytes(int32_t B, int32_t Hq, int32_t D, int32_t max_q_len,
                               int32_t max_ctx, int32_t P);
int generic_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                      const void* v_cache, int64_t num_slots, int64_t kv_stride_slot,
                      int64_t kv_stride_head, const int32_t* table, int64_t table_stride,
                      int32_t log2_bs, const int32_t* cu_q, const int32_t* ctx_lens, int32_t B,
                      int32_t Hq, int32_t KVH, int32_t D, float scale, int32_t max_q_len,
                      int32_t max_ctx, int32_t P, void* workspace, void* out,
                      int64_t o_stride_t, int64_t o_stride_h, int32_t dtype, int32_t* err_count,
                      hipStream_t s);

}  // namespace dsp_detail
