/*
 * dsp_probe.h -- measurement-only kernels of libdispec_probe.so (not part of the C ABI of
 * libdispec_hip.so; nothing in the KV path calls them).  bench.py uses them to calibrate
 * what this GPU's HBM delivers to the access patterns of the path's kernels.
 */
#ifndef DISPEC_PROBE_H
#define DISPEC_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#include "../include/dispec_hip.h" /* dsp_stream_t, DSP_E* */

/* Probes with no counterpart in the reference.  Each returns 0, a negative DSP_E* status
 * of dispec_hip.h for an invalid argument (nothing launched), or a positive hipError_t.
 *   dsp_probe_stream_read: `workgroups` workgroups stream `bytes` of `buf` (16-byte
 *     aligned) once.
 *   dsp_probe_slice_read: the paged decode's access pattern without its arithmetic --
 *     for each (sequence, KV head) `waves_per_seq_head` waves read that head's 128-dim
 *     bf16 row of K and V for all `ctx` keys through `block_table`, the waves of 4 heads
 *     of the same keys side by side in one workgroup when KVH % 4 == 0 (as the balanced
 *     decode kernel groups them), K with cached loads and V non-temporal (as the decode
 *     kernels load them); caches are [num_slots, KVH, 128] contiguous; ctx a multiple of
 *     32 * waves_per_seq_head.
 * Both store one word to `sink` only if what they read hashes to a sentinel. */
int dsp_probe_stream_read(const void* buf, int64_t bytes, int32_t workgroups, uint32_t* sink,
                          dsp_stream_t stream);
/*   dsp_probe_stream_copy: `workgroups` workgroups copy `bytes` from src to dst (both
 *     16-byte aligned, not overlapping) once: the ceiling of the byte-moving kernels. */
int dsp_probe_stream_copy(const void* src, void* dst, int64_t bytes, int32_t workgroups,
                          dsp_stream_t stream);
int dsp_probe_slice_read(const void* k_cache, const void* v_cache, int64_t num_slots,
                         const int32_t* block_table, int64_t bt_stride, int32_t block_size,
                         int32_t B, int32_t KVH, int32_t ctx, int32_t waves_per_seq_head,
                         uint32_t* sink, dsp_stream_t stream);
/*   dsp_probe_gemm_fill: the loads of one map_gemm_big_kernel launch (C = A . Bt^T, batch
 *     problems of M x N x K, A rows lda apart, problem z's A at a + z * a_batch_stride) into
 *     LDS stages, with no MFMA and no epilogue: the floor of that launch's time. */
int dsp_probe_gemm_fill(const void* a, int64_t lda, int64_t M, int64_t a_batch_stride,
                        const void* bt, int64_t ldb, int64_t N, int64_t K, int32_t batch,
                        uint32_t* sink, dsp_stream_t stream);
/*   dsp_probe_piece_scatter: copy `bytes` of src to dst in pieces of piece_bytes (a multiple
 *     of 16 dividing bytes), piece i landing at dst + dst_index[i] * piece_bytes (the caller
 *     gives a permutation, so every destination is written once): the ceiling of writes to
 *     random 32 KiB blocks (scatter, block copy) or 2 KiB rows (append). */
int dsp_probe_piece_scatter(const void* src, void* dst, int64_t bytes, int64_t piece_bytes,
                            const int32_t* dst_index, dsp_stream_t stream);
/*   dsp_probe_piece_gather: the opposite direction -- piece i of dst (contiguous) read from
 *     src + src_index[i] * piece_bytes (piece_bytes a multiple of 4096 dividing bytes): the
 *     ceiling of reads from random 32 KiB blocks written in order (the transport gather). */
int dsp_probe_piece_gather(const void* src, void* dst, int64_t bytes, int64_t piece_bytes,
                           const int32_t* src_index, dsp_stream_t stream);
/*   dsp_probe_batch_read: the K/V read of a decode batch (head_dim 128, KVH <= 8) with no
 *     arithmetic and equal work per workgroup: workgroup w reads keys [k0, min(k0 + 256,
 *     ctx_lens[b])) of sequence b for all KV heads, (b, k0) = work[2w], work[2w + 1], K
 *     cached and V non-temporal; the floor of a decode's time on those contexts. */
int dsp_probe_batch_read(const void* k_cache, const void* v_cache, int64_t num_slots,
                         const int32_t* block_table, int64_t bt_stride, int32_t block_size,
                         const int32_t* ctx_lens, const int32_t* work, int32_t num_work,
                         int32_t KVH, uint32_t* sink, dsp_stream_t stream);
/*   dsp_probe_piece_fill: stores only -- fill `bytes` of dst (pieces of piece_bytes, a
 *     multiple of 4096 dividing bytes) with a constant, piece i at dst + dst_index[i] *
 *     piece_bytes: HBM write bandwidth in order (identity) or to random 32 KiB blocks. */
int dsp_probe_piece_fill(void* dst, int64_t bytes, int64_t piece_bytes, const int32_t* dst_index,
                         dsp_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DISPEC_PROBE_H */
