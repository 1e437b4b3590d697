/*
 * dispec_hip.h -- C ABI of the MI355X (gfx950) KV-cache data path.
 *
 * One shared library, libdispec_hip.so, exports these entry points. They are the
 * device side of DiSpec's KV path: append into the paged pool, block copy for
 * copy-on-write and prefix-cache eviction, paged decode attention (split-K with a
 * log-sum-exp combine), multi-query paged attention for speculative verify and
 * chunked prefill, and the transport gather / cross-model map / import scatter.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HBM) unless noted.  Strides are in ELEMENTS of
 *     the named dtype unless the name ends in `_bytes`.
 *   - The pool layout is the reference's: per layer, K and V are each
 *     [num_blocks * block_size, num_kv_heads, head_dim]; slot s of a layer is one
 *     row of num_kv_heads*head_dim contiguous elements (paged_cache.py:3-7, :39).
 *   - Nothing here allocates device memory or synchronises the host: outputs and the
 *     split-K workspace are passed in by the caller, and all work is enqueued on
 *     `stream`.  Device-side global state is limited to (a) two write-only 4 KiB sink
 *     regions (the append and the attention prologue send the stores of a skipped row
 *     there instead of branching around them; nothing ever reads them, so concurrent
 *     calls stay independent) and (b) the 32 MiB scratch array of
 *     dsp_paged_decode_noalloc, shared by every call of that one entry point on a
 *     device (overlapping calls of it race; every other entry point is reentrant
 *     across streams).  Host-side, the library caches two per-device values read once
 *     from the runtime: that array's address and the device's compute-unit count.
 *   - Return value: 0 on success, a negative DSP_E* code for an invalid argument
 *     (nothing was launched), or a positive hipError_t from the launch.
 *   - `err_count` (optional, may be NULL) is a device int32 that the kernels
 *     atomically increment once per out-of-range slot / block id they meet.  Such
 *     rows are skipped, never read or written out of bounds.
 */
#ifndef DISPEC_HIP_H
#define DISPEC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is passed as an opaque pointer so that this header needs no HIP headers. */
typedef void* dsp_stream_t;

enum dsp_dtype { DSP_BF16 = 0, DSP_F16 = 1, DSP_F32 = 2 };

enum dsp_status {
  DSP_OK = 0,
  DSP_EINVAL = -1,        /* null pointer, negative size, inconsistent shape */
  DSP_EALIGN = -2,        /* a stride or pointer breaks the alignment a kernel needs */
  DSP_EUNSUPPORTED = -3,  /* dtype / head_dim / group size with no compiled kernel */
  DSP_EWORKSPACE = -4,    /* workspace smaller than dsp_*_workspace_bytes() */
  DSP_ESCRATCH = -5       /* a no-allocation call needs more than its fixed scratch */
};

/* partition_tokens value of dsp_paged_mq_attention (and its workspace size) that asks for
 * the balanced split-K kernel instead of fixed key partitions. */
enum dsp_split { DSP_SPLIT_BALANCED = -1 };

/* Human-readable text for a status code (static storage; never NULL). */
const char* dsp_error_string(int status);

/* Library version, for the Python loader's sanity check. */
int dsp_version(void);

/* ------------------------------------------------------------------------------ J1
 * Slot-mapped append of one layer's new K/V rows into the pool.
 * Replaces PagedKVCache.write (dispec/kv/paged_cache.py:61-68):
 *     key[layer].index_copy_(0, slots, k); value[layer].index_copy_(0, slots, v)
 * and the graph-decoder copy at dispec/engine/cuda_graph.py:70-71.
 *   k_pool, v_pool : layer base of the pool, num_slots rows of row_bytes at
 *                    pool_slot_stride_bytes.
 *   k, v           : num_tokens source rows of row_bytes at src_token_stride_bytes.
 *   slots          : int64[num_tokens], unique (as index_copy_ requires).
 * Bit-exact (a byte copy).  K and V go in one launch. */
int dsp_kv_append(void* k_pool, void* v_pool, int64_t num_slots,
                  int64_t pool_slot_stride_bytes,
                  const void* k, const void* v, int64_t src_token_stride_bytes,
                  const int64_t* slots, int64_t num_tokens, int64_t row_bytes,
                  int32_t* err_count, dsp_stream_t stream);

/* Slot-list row gather of one layer: k_out[i] = k_pool[slots[i]], same for V.
 * Replaces PagedKVCache.gather (dispec/kv/paged_cache.py:70-72):
 *     return key[layer][slots], value[layer][slots]
 * Out-of-range slots are counted in err_count and their output rows left untouched. */
int dsp_kv_gather_slots(const void* k_pool, const void* v_pool, int64_t num_slots,
                        int64_t pool_slot_stride_bytes, const int64_t* slots,
                        int64_t num_tokens, int64_t row_bytes, void* k_out, void* v_out,
                        int64_t out_token_stride_bytes, int32_t* err_count,
                        dsp_stream_t stream);

/* ------------------------------------------------------------------------------ J2
 * Whole-block copy over every layer, for copy-on-write fork, prefix-cache block copy
 * and evict-by-copy into a second pool.  The reference shares blocks by refcount only
 * (dispec/kv/block_manager.py:119-126, dispec/kv/prefix_cache.py:64-70); this is the
 * data move those metadata operations imply:
 *     for l, i: dst[l, d_i*bs:(d_i+1)*bs] = src[l, s_i*bs:(s_i+1)*bs]   (K and V)
 * Source and destination pools may be the same pool.
 *   block_bytes       : block_size * num_kv_heads * head_dim * elem_size (same in both).
 *   *_layer_stride_bytes : num_blocks * block_bytes for a contiguous pool.
 *   src_blocks, dst_blocks : int32[num_pairs] device arrays.  Within one call no block
 *                    may be both read and written (the copies run concurrently). */
int dsp_kv_copy_blocks(const void* src_k_pool, const void* src_v_pool,
                       int64_t src_layer_stride_bytes, int64_t src_num_blocks,
                       void* dst_k_pool, void* dst_v_pool, int64_t dst_layer_stride_bytes,
                       int64_t dst_num_blocks, int64_t num_layers, int64_t block_bytes,
                       const int32_t* src_blocks, const int32_t* dst_blocks,
                       int64_t num_pairs, int32_t* err_count, dsp_stream_t stream);

/* J2 for one source block copied into many: the copy-on-write fork of one partial block
 * into every child of a prompt (block_manager.py:119-126, one cow_fork per child).  Same
 * result as dsp_kv_copy_blocks with every src_blocks[i] == src_block; the source is read
 * once per 8 copies instead of once per copy.
 *   src_block  : host value, must lie in [0, src_num_blocks) (else DSP_EINVAL).
 *   dst_blocks : int32[num_dst] device array; an id outside [0, dst_num_blocks) is skipped
 *                and counted in *err_count.  No destination may equal the source when the
 *                pools are the same. */
int dsp_kv_copy_block_fanout(const void* src_k_pool, const void* src_v_pool,
                             int64_t src_layer_stride_bytes, int64_t src_num_blocks,
                             void* dst_k_pool, void* dst_v_pool, int64_t dst_layer_stride_bytes,
                             int64_t dst_num_blocks, int64_t num_layers, int64_t block_bytes,
                             int32_t src_block, const int32_t* dst_blocks, int64_t num_dst,
                             int32_t* err_count, dsp_stream_t stream);

/* ------------------------------------------------------------------------ J5a / J5c
 * Block-table gather of whole sequences over every layer into contiguous transport
 * buffers, and the inverse scatter.
 * Replaces PagedKVCache.export_contiguous (paged_cache.py:87-90):
 *     k_out = key[:, context_slots(block_ids, seq_len)].contiguous()
 * and PagedKVCache.import_contiguous (paged_cache.py:92-96):
 *     key[:, context_slots(block_ids, T)] = k
 * batched over num_seqs sequences.  Sequence b's buffer is the (num_layers, T_b,
 * num_kv_heads, head_dim) KVPayload layout (dispec/transport/base.py:24-44) and
 * starts at row num_layers * cu_seqlens[b] of k_buf / v_buf.
 *   block_tables : int32 [num_seqs, bt_stride] physical block ids.
 *   cu_seqlens   : int64 [num_seqs + 1] device array of token offsets:
 *                  T_b = cu_seqlens[b+1] - cu_seqlens[b].
 *   The pool rows must be contiguous (slot stride == row_bytes), as the reference's
 *   pool is, so that one block of one layer is a single row_bytes*block_size span.
 *   max_seqlen   : an upper bound on every T_b (sizes the grid).
 *   block_size   : tokens per block, a power of two. */
int dsp_kv_gather(const void* k_pool, const void* v_pool, int64_t num_layers,
                  int64_t pool_layer_stride_bytes, int64_t num_blocks,
                  int64_t row_bytes, int32_t block_size,
                  const int32_t* block_tables, int64_t bt_stride,
                  const int64_t* cu_seqlens, int32_t num_seqs, int64_t max_seqlen,
                  void* k_buf, void* v_buf, int32_t* err_count, dsp_stream_t stream);

int dsp_kv_scatter(void* k_pool, void* v_pool, int64_t num_layers,
                   int64_t pool_layer_stride_bytes, int64_t num_blocks,
                   int64_t row_bytes, int32_t block_size,
                   const int32_t* block_tables, int64_t bt_stride,
                   const int64_t* cu_seqlens, int32_t num_seqs, int64_t max_seqlen,
                   const void* k_buf, const void* v_buf, int32_t* err_count,
                   dsp_stream_t stream);

/* dsp_kv_scatter with its copies visited in destination-block order: the same rows land
 * in the same slots (PagedKVCache.import_contiguous, paged_cache.py:92-96, batched), but
 * the pool is written through each layer in address order and the transport buffer is
 * read in block-sized runs out of order, which moves the bytes faster when the tables
 * name many of the pool's blocks.  With fewer than num_blocks / 2 table entries
 * (num_seqs * ceil(max_seqlen / block_size)) it runs dsp_kv_scatter itself.
 *   block_owner : device int32 [num_blocks] workspace, overwritten (which table entry
 *                 names each block); calls that overlap on one workspace race.
 * A block named by more than one table entry (an import into sequences' own blocks never
 * does this) is written from the last of them alone, in sequence order then block order:
 * its rows past a partial last entry keep what the pool held.  dsp_kv_scatter writes
 * every entry, in no defined order.  Other arguments and errors as for dsp_kv_scatter
 * (an out-of-range block id is counted once per table entry). */
int dsp_kv_scatter_ordered(void* k_pool, void* v_pool, int64_t num_layers,
                           int64_t pool_layer_stride_bytes, int64_t num_blocks,
                           int64_t row_bytes, int32_t block_size,
                           const int32_t* block_tables, int64_t bt_stride,
                           const int64_t* cu_seqlens, int32_t num_seqs, int64_t max_seqlen,
                           const void* k_buf, const void* v_buf, int32_t* block_owner,
                           int32_t* err_count, dsp_stream_t stream);

/* ------------------------------------------------------------------------------ J3
 * Paged decode attention, one query token per sequence, GQA-packed and split-K.
 * Replaces batched_paged_decode_attention (dispec/engine/triton_attn.py:98-116,
 * kernel :59-95) and paged_decode_attention (:119-139):
 *     o[b, h] = softmax_j(scale * q[b, h] . K[slot_j, h / G]) . V[slot_j, h / G]
 * over the ctx_lens[b] context tokens, accumulated in fp32, written in the cache
 * dtype.  Keys are addressed either by a per-token slot table (the reference's
 * signature, slot_table[b, j], block_table == NULL) or by a block table
 * (block_table[b, j / block_size] * block_size + j % block_size, slot_table == NULL).
 *   q, out       : [B, Hq, D] with strides (q_stride_b, q_stride_h), D contiguous.
 *   k/v_cache    : one layer, [num_slots, KVH, D] with strides (kv_stride_slot,
 *                  kv_stride_head), D contiguous; same strides for K and V.
 *   ctx_lens     : int32 [B], each in [0, max_ctx].  ctx_len 0 writes zeros.
 *   partition_tokens : 0 (automatic), DSP_SPLIT_BALANCED, or a split-K partition length.
 *                  0 with a block table, D in {32, 64, 128}: max_ctx <= 512 with at most
 *                  two (sequence, KV head) pairs per CU runs unsplit (one launch, no
 *                  combine: such decodes are launch-bound); otherwise, for B <= 512, a
 *                  balanced split -- the launch's (sequence, KV head, 16-key unit) work is
 *                  cut into equal contiguous shares, one per wave, computed on the device
 *                  from ctx_lens -- and a log-sum-exp combine kernel.  DSP_SPLIT_BALANCED
 *                  asks for the balanced split whatever the size (block tables, D in {32,
 *                  64, 128}, G <= 8, B <= 512; else DSP_EUNSUPPORTED).  Otherwise (or with
 *                  a slot table) fixed partitions of partition_tokens keys (0: chosen by
 *                  dsp_paged_decode_partition_tokens) per (sequence, KV head), merged by
 *                  the combine kernel when a sequence spans more than one.  `workspace`
 *                  must hold dsp_paged_decode_workspace_bytes(..., partition_tokens)
 *                  bytes (16-byte aligned) for the same arguments, on the same device.
 * dtype: DSP_BF16, DSP_F16 or DSP_F32 (caches, q and out all of it).  The tuned kernels
 * serve bf16 / fp16 with D in {16, 32, 64, 128} and G = Hq / KVH in 1..8; every other
 * shape with D a power of two from 8 to 256 (fp32, D 8 or 256, G above 8) runs on a
 * generic kernel -- one wave per (sequence, query head, partition), fp32 accumulation,
 * element-aligned pointers -- whose automatic partition is dsp_paged_decode_partition_tokens
 * and whose workspace is covered by dsp_paged_decode_workspace_bytes.  Other D:
 * DSP_EUNSUPPORTED.
 * err_count (optional) is incremented for a context length outside [0, max_ctx]
 * (clamped) and, on block tables and the generic kernel, once per wave that met a block id
 * whose slots lie outside the cache (those keys are skipped). */
size_t dsp_paged_decode_workspace_bytes(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                        int32_t max_ctx, int32_t partition_tokens);
int dsp_paged_decode_partition_tokens(int32_t B, int32_t KVH, int32_t D, int32_t max_ctx);

int dsp_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache, int64_t num_slots,
                     int64_t kv_stride_slot, int64_t kv_stride_head,
                     const int32_t* block_table, int64_t bt_stride, int32_t block_size,
                     const int32_t* slot_table, int64_t st_stride,
                     const int32_t* ctx_lens, int32_t B, int32_t Hq, int32_t KVH,
                     int32_t D, float scale, int32_t max_ctx, int32_t partition_tokens,
                     void* workspace, size_t workspace_bytes,
                     void* out, int64_t o_stride_b, int64_t o_stride_h,
                     int32_t dtype, int32_t* err_count, dsp_stream_t stream);

/* J3 without a workspace argument.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The same arguments and results as dsp_paged_decode
 * (same kernels and split), with the split-K workspace taken from a fixed device array of
 * DSP_NOALLOC_SCRATCH_BYTES held by the library on each GPU it runs on until the process
 * ends; the call itself allocates nothing.  A launch whose workspace
 * (dsp_paged_decode_workspace_bytes) exceeds it returns DSP_ESCRATCH with nothing
 * launched (config 3's 16 x 32k batch needs 6.7 MB on the automatic split, 17 MB on
 * 512-token partitions).  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race and must be ordered by the
 * caller.  The array's device address is fetched on the first call on each device (with
 * that device current). */
#define DSP_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int dsp_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* k_cache, const void* v_cache, int64_t num_slots,
                             int64_t kv_stride_slot, int64_t kv_stride_head,
                             const int32_t* block_table, int64_t bt_stride, int32_t block_size,
                             const int32_t* slot_table, int64_t st_stride,
                             const int32_t* ctx_lens, int32_t B, int32_t Hq, int32_t KVH,
                             int32_t D, float scale, int32_t max_ctx, int32_t partition_tokens,
                             void* out, int64_t o_stride_b, int64_t o_stride_h, int32_t dtype,
                             int32_t* err_count, dsp_stream_t stream);

/* ------------------------------------------------------------------------------ J4
 * Multi-query paged attention for speculative verify and chunked prefill.
 * Replaces the native branch of ModelRunner._attention (dispec/engine/model_runner.py:
 * 160-185): per sequence b, the last q_len_b = cu_q[b+1] - cu_q[b] context tokens are
 * queries, and
 *     out = SDPA(q, K, V, attn_mask=causal_lower_right(q_len_b, ctx_lens[b]),
 *                enable_gqa=True, scale=scale)
 * i.e. query i sees keys j <= ctx_lens[b] - q_len_b + i.  The new tokens' K/V must
 * already be in the cache (the reference writes before attending, :148).
 *   q, out     : packed [sum q_len, Hq, D], strides (q_stride_t, q_stride_h).
 *   block_table: int32 [B, bt_stride] (power-of-two block_size).
 *   cu_q       : int32 [B+1] device offsets; ctx_lens: int32 [B], q_len_b <= ctx <= max_ctx.
 *   max_q_len  : upper bound of q_len_b (sizes the grid and the workspace).  A larger
 *                q_len_b is a caller error that never leads to an out-of-bounds access:
 *                the balanced split counts it in err_count and writes the sequence's first
 *                max_q_len query rows as zeros; the tiled kernels compute its first
 *                max_q_len query rows (rows past them are computed or left untouched,
 *                depending on the split).
 *   partition_tokens : split-K key partition (multiple of 128, at most 64 partitions of
 *                max_ctx); 0 picks one from the shape.  More than one partition needs
 *                `workspace` (dsp_paged_mq_workspace_bytes with the same partition_tokens,
 *                0 included) and a merge kernel.
 *                DSP_SPLIT_BALANCED: the balanced split-K kernel of dsp_paged_decode --
 *                every wave of the launch takes an equal share of the (sequence, KV head,
 *                16-key unit) work, so one long context among short ones does not leave a
 *                tail of its partitions on an idle GPU (1 x 32k + 15 x 512 contexts, Qwen3
 *                heads, 5 queries: 44 against 93 us); contexts of similar length run 0-5 %
 *                faster on fixed partitions.  Needs max_q_len * G <= 16, blocks of >= 16
 *                tokens, B <= 512, D in {32, 64, 128} (else DSP_EUNSUPPORTED) and always
 *                `workspace` (dsp_paged_mq_workspace_bytes with DSP_SPLIT_BALANCED).
 * dtype DSP_BF16 / DSP_F16 with D in {32, 64, 128} on the tuned kernels; DSP_F32, or D 8,
 * 16 or 256, on a generic kernel (one wave per query row, head and key partition; fixed
 * partitions only -- DSP_SPLIT_BALANCED and the shared-prefix entry return
 * DSP_EUNSUPPORTED for them); any G = Hq / KVH.  A sequence with q_len > ctx or
 * ctx > max_ctx is counted in err_count and its rows written as zeros.  A block id whose
 * slots lie outside the cache is never dereferenced: it is counted once per wave that met
 * it, and its keys are masked out on the 16-row tiles and the balanced split, read from
 * slots 0..15 on the 128-row tile (that sequence's result is then unspecified).
 * Batches with max_q_len * G >= 128 (D 64 or 128, blocks of >= 16 tokens) run on a
 * 128-row tile built for chunked prefill; shorter ones (verify) on 16-row tiles.  The
 * automatic partition is sized for whichever runs. */
int dsp_paged_mq_partition_tokens(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                  int32_t max_q_len, int32_t max_ctx);
size_t dsp_paged_mq_workspace_bytes(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                    int32_t max_q_len, int32_t max_ctx, int32_t partition_tokens);
int dsp_paged_mq_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                           const void* k_cache, const void* v_cache, int64_t num_slots,
                           int64_t kv_stride_slot, int64_t kv_stride_head,
                           const int32_t* block_table, int64_t bt_stride, int32_t block_size,
                           const int32_t* cu_q, const int32_t* ctx_lens, int32_t B,
                           int32_t Hq, int32_t KVH, int32_t D, float scale, int32_t max_q_len,
                           int32_t max_ctx, int32_t partition_tokens, void* workspace,
                           size_t workspace_bytes, void* out, int64_t o_stride_t,
                           int64_t o_stride_h, int32_t dtype, int32_t* err_count,
                           dsp_stream_t stream);

/* J4, shared prefix (cascade).  The same attention when the first prefix_tokens context
 * tokens of every sequence are the same physical blocks -- copy-on-write forks of one
 * prompt (BlockManager.fork, dispec/kv/block_manager.py:119-126) or prefix-cache hits
 * (PrefixCache.match, dispec/kv/prefix_cache.py:39-50) -- and every query sees all of
 * them (prefix_tokens <= ctx_b - q_len_b; a sequence breaking this is counted in
 * err_count and zeroed).  The prefix keys are read once for every query row of the batch
 * (block-table row 0 supplies them) instead of once per sequence; the suffixes run per
 * sequence; one merge folds both.  No reference counterpart: the reference attends each
 * sequence over its whole context (model_runner.py:160-185); the result is the same
 * function.  prefix_tokens: a multiple of 128 and of partition_tokens, < max_ctx;
 * partition_tokens 0 = dsp_paged_mq_shared_prefix_partition_tokens.  D 64 or 128, blocks
 * of >= 16 tokens, B <= 1024 (else DSP_EUNSUPPORTED).  The workspace is
 * dsp_paged_mq_workspace_bytes at the partition used (always needed). */
int dsp_paged_mq_shared_prefix_partition_tokens(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                                int32_t max_q_len, int32_t max_ctx,
                                                int32_t prefix_tokens);
int dsp_paged_mq_attention_shared_prefix(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
    const void* v_cache, int64_t num_slots, int64_t kv_stride_slot, int64_t kv_stride_head,
    const int32_t* block_table, int64_t bt_stride, int32_t block_size, const int32_t* cu_q,
    const int32_t* ctx_lens, int32_t B, int32_t Hq, int32_t KVH, int32_t D, float scale,
    int32_t max_q_len, int32_t max_ctx, int32_t prefix_tokens, int32_t partition_tokens,
    void* workspace, size_t workspace_bytes, void* out, int64_t o_stride_t, int64_t o_stride_h,
    int32_t dtype, int32_t* err_count, dsp_stream_t stream);

/* ------------------------------------------------------------------------------ J5b
 * The cross-model map GEMM: C[M, N] = epilogue(A[M, K] . Bt[N, K]^T), bf16 operands,
 * fp32 accumulation (MFMA).  Replaces the matmuls of LayerMap.apply
 * (dispec/kv/transfer.py:104-112) on the design rows of CrossModelKVMap._apply (:249):
 *   A          : design rows read in place.  Column k of row m is
 *                a[a_segment_offsets[k / segment_len] + m*lda + k % segment_len]: the
 *                k-th segment is one source layer's KVH*D row (feature order layer ->
 *                head -> dim).  a_segment_offsets is a HOST array of num_segments
 *                (1..8) element offsets; num_segments * segment_len == K.
 *   Bt         : N x K row-major (K contiguous), leading dimension ldb: W^T for
 *                x @ W, or an F.linear weight as stored.
 *   C          : M x N row-major, leading dimension ldc.
 *   batch      : independent problems sharing Bt and the bias (grid z, <= 65535); problem
 *                z reads A at a + z*a_batch_stride and writes C at c + z*c_batch_stride
 *                (elements) -- e.g. several requests' transport buffers at once.
 *   bias_mode  : 0 none, 1 bf16(bf16(acc) + b) (x @ W + b as two bf16 ops),
 *                2 bf16(acc + b) (F.linear / addmm).  bias is bf16 [N].
 *   activation : 0 none, 1 gelu (erf form) applied to the rounded value and rounded.
 *   accumulate : 1 adds the result to the existing C in bf16 (residual add).
 * dtype: DSP_BF16. */
int dsp_kv_map_gemm(const void* a, const int64_t* a_segment_offsets, int32_t num_segments,
                    int64_t segment_len, int64_t lda, const void* bt, int64_t ldb, void* c,
                    int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t batch,
                    int64_t a_batch_stride, int64_t c_batch_stride, const void* bias,
                    int32_t bias_mode, int32_t activation, int32_t accumulate, int32_t dtype,
                    dsp_stream_t stream);

/* J5b + J5c fused: the map GEMM writing its rows straight into a target pool layer.
 * Replaces the tail of CrossModelKVMap._apply for one target layer -- y = x @ W + b
 * (transfer.py:250, LayerMap.apply :104-112), keys re-rotated with the target tables in
 * fp32 (:251-253) -- followed by PagedKVCache.import_contiguous of that layer
 * (paged_cache.py:92-96), without the (T, KVH*D) intermediate: row m of problem z lands in
 * pool slot block_tables[z * bt_stride + m / block_size] * block_size + m % block_size.
 * Same A / Bt / segment / batch arguments and the same rounding as dsp_kv_map_gemm with
 * bias_mode 1 (bias may be NULL: bf16(acc)); no activation or accumulate.
 *   pool, pool_row_stride, num_slots : one layer of the target pool (rows of KVH*D
 *                  elements, pool_row_stride apart); a row whose block id puts it outside
 *                  [0, num_slots) is skipped and counted in err_count (>= 1 per such row).
 *   rope_cos, rope_sin : fp32 [M][head_dim] tables (row m = the position of row m, shared
 *                  by the batch) or both NULL (values: no rotation).  head_dim 64 or 128.
 * Needs what the large-tile GEMM needs (16-byte aligned operands and rows, K and
 * segment_len multiples of 64, N a multiple of 8 and of head_dim, 32-bit element offsets),
 * else DSP_EUNSUPPORTED (the caller then runs dsp_kv_map_gemm + dsp_kv_rope +
 * dsp_kv_scatter).  The result is bit-identical to that three-launch sequence. */
int dsp_kv_map_gemm_to_pool(const void* a, const int64_t* a_segment_offsets,
                            int32_t num_segments, int64_t segment_len, int64_t lda,
                            const void* bt, int64_t ldb, void* pool, int64_t pool_row_stride,
                            int64_t num_slots, const int32_t* block_tables, int64_t bt_stride,
                            int32_t block_size, int64_t M, int64_t N, int64_t K, int32_t batch,
                            int64_t a_batch_stride, const void* bias, const float* rope_cos,
                            const float* rope_sin, int32_t head_dim, int32_t dtype,
                            int32_t* err_count, dsp_stream_t stream);

/* RoPE strip (direction -1) or apply (+1) on (L, T, H, D) rows in fp32:
 *     y = x * cos + direction * rotate_half(x) * sin,   rotate_half(x) = cat(-x2, x1)
 * Replaces strip_rope / apply_rope (dispec/kv/transfer.py:66-80).  cos/sin are fp32
 * (T, D) tables (rope_tables, :50-58).  x, y: layer strides in elements, rows
 * contiguous; in_dtype / out_dtype DSP_BF16 or DSP_F32 (bf16 output is rounded to
 * nearest even, as the reference's store into a bf16 buffer is).  y may alias x. */
int dsp_kv_rope(const void* x, int64_t x_layer_stride, void* y, int64_t y_layer_stride,
                int64_t L, int64_t T, int64_t H, int64_t D, const float* cos_table,
                const float* sin_table, int32_t direction, int32_t in_dtype, int32_t out_dtype,
                dsp_stream_t stream);

/* ------------------------------------------------------------------------------ J1+
 * The attention prologue of one layer in one launch: per-head RMSNorm of q and k
 * (optional), RoPE on q and k, and the append of k and v into the paged pool.
 * Replaces ModelRunner._attention's op sequence (dispec/engine/model_runner.py:142-148):
 *     q = q_norm(q); k = k_norm(k)          Qwen3RMSNorm: var = mean(x^2) in fp32,
 *                                          y = w * dtype(x * rsqrt(var + eps))
 *     q = q * cos + rotate_half(q) * sin   (:49-50 there), each product and the sum
 *     k = k * cos + rotate_half(k) * sin    rounded to the dtype, as torch does
 *     cache.write(layer, slots, k, v)      (paged_cache.py:61-68)
 *   q, k, v      : [T, Hq | KVH, D] with (token, head) strides; D contiguous.
 *   q/k_norm_weight : [D] RMSNorm weights, both or neither (NULL: no norm, Qwen2).
 *   cos/sin_table: [T, D] in the model dtype (the model's rotary tables), row stride.
 *   slots        : int64 [T] pool slots of the new tokens (out of range: counted in
 *                  err_count, that token's k/v not written).
 *   q_out        : [T, Hq, D] rotated q (may alias q when the strides match).
 *   k/v_pool     : one layer, [num_slots, KVH, D] with (slot, head) strides.
 * dtype DSP_BF16 / DSP_F16 / DSP_F32 (every tensor of that dtype; fp32 rounds nowhere but
 * in its own arithmetic, as torch's fp32 ops do); D in {32, 64, 128, 256}; all strides
 * multiples of 16 bytes and all pointers 16-byte aligned. */
int dsp_qk_norm_rope_append(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                            const void* k, int64_t k_stride_t, int64_t k_stride_h,
                            const void* v, int64_t v_stride_t, int64_t v_stride_h,
                            const void* q_norm_weight, const void* k_norm_weight, float eps,
                            const void* cos_table, const void* sin_table,
                            int64_t rope_stride_t, const int64_t* slots, int64_t T,
                            int32_t Hq, int32_t KVH, int32_t D, void* q_out,
                            int64_t q_out_stride_t, int64_t q_out_stride_h, void* k_pool,
                            void* v_pool, int64_t num_slots, int64_t pool_stride_slot,
                            int64_t pool_stride_head, int32_t dtype, int32_t* err_count,
                            dsp_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DISPEC_HIP_H */
