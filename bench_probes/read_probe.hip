// Bandwidth probes for the roofline: what this GPU's HBM delivers to (1) a plain streaming
// read, (2) a read with the paged decode's access pattern, with no compute, (3) a plain
// streaming copy (the ceiling of the append / gather / scatter / block-copy kernels), and
// (4) the map GEMM's operand stages into LDS with no MFMA and no epilogue.
// They calibrate the decode kernel's measured GB/s: the datasheet peak (8 TB/s) is not
// reachable by any read, and the slot-major pool layout (one KV head's 256-byte slice of
// every 2 KiB slot row) caps what the decode can fetch below a streaming read.  Both probes
// reduce what they read to one word that is stored only if it matches a sentinel, so the
// loads cannot be removed.
#include "../dispec_amd/csrc/dsp_common.h"
#include "dsp_probe.h"

namespace {

// Each workgroup streams a contiguous span, 16 bytes per lane per load, 8 loads in flight.
__global__ __launch_bounds__(256) void stream_read_kernel(const dsp_u32x4* __restrict__ p,
                                                          int64_t n16, int64_t per_wg,
                                                          uint32_t* __restrict__ sink) {
  const int64_t base = int64_t(blockIdx.x) * per_wg;
  const int64_t end = base + per_wg < n16 ? base + per_wg : n16;
  dsp_u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t i = base + threadIdx.x; i < end; i += 256 * 8) {
    dsp_u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t j = i + u * 256;
      v[u] = j < end ? dsp_ld_stream(p + j) : dsp_u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u];
  }
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) sink[0] = r;
}

// One workgroup of HG waves per (sequence, group of HG KV heads, share of its keys), wave
// i reading head HG*group + i, as the balanced decode kernel groups its waves: per 32 keys
// a wave reads its head's row of K and of V for every key (16 bytes per lane, 4 rows per
// load), addressed through the block table exactly as the decode kernels address the pool,
// with their cache policy: K cached, V non-temporal.
template <int HG>
__global__ __launch_bounds__(64 * HG) void slice_read_kernel(const uint16_t* __restrict__ kc,
                                                             const uint16_t* __restrict__ vc,
                                                             int64_t num_slots,
                                                             const int32_t* __restrict__ bt,
                                                             int64_t bt_stride, int32_t log2_bs,
                                                             int32_t KVH, int32_t keys_per_wave,
                                                             int32_t waves_per_seg,
                                                             uint32_t* __restrict__ sink) {
  constexpr int D = 128;
  const int w = blockIdx.x;
  const int NG = KVH / HG;
  const int seg = w / waves_per_seg, part = w % waves_per_seg;
  const int b = seg / NG, h = (seg % NG) * HG + int(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bmask = (1 << log2_bs) - 1;
  dsp_u32x4 acc = {0u, 0u, 0u, 0u};
  const int k0 = part * keys_per_wave;
  for (int t = k0; t < k0 + keys_per_wave; t += 32) {
    dsp_u32x4 kv[8], vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = t + i * 4 + lane / 16;
      int64_t slot = int64_t(bt[int64_t(b) * bt_stride + (key >> log2_bs)]) * (bmask + 1) +
                     (key & bmask);
      slot = (slot >= 0 && slot < num_slots) ? slot : 0;  // a bad block id reads row 0
      const int64_t e = slot * (int64_t(KVH) * D) + int64_t(h) * D + (lane % 16) * 8;
      kv[i] = *reinterpret_cast<const dsp_u32x4*>(kc + e);
      vv[i] = dsp_ld_stream(reinterpret_cast<const dsp_u32x4*>(vc + e));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc ^= kv[i] ^ vv[i];
  }
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) sink[0] = r;
}

// Streaming copy: each workgroup copies a contiguous span, 4 loads of 16 bytes per lane in
// flight, then their stores (non-temporal both ways).
__global__ __launch_bounds__(256) void stream_copy_kernel(const dsp_u32x4* __restrict__ src,
                                                          dsp_u32x4* __restrict__ dst,
                                                          int64_t n16, int64_t per_wg) {
  const int64_t base = int64_t(blockIdx.x) * per_wg;
  const int64_t end = base + per_wg < n16 ? base + per_wg : n16;
  for (int64_t i = base + threadIdx.x; i < end; i += 256 * 4) {
    dsp_u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = i + u * 256;
      if (j < end) v[u] = dsp_ld_stream(src + j);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = i + u * 256;
      if (j < end) dsp_st_stream(v[u], dst + j);
    }
  }
}

// A copy whose destinations follow a permutation: contiguous source pieces of piece_bytes
// (a multiple of 16) go to dst + dst_index[i] * piece_bytes -- the write pattern of the
// scatter (32 KiB blocks) and of the append (2 KiB rows) with no table or slot logic.  One
// one-shot workgroup per 4 KiB of the source, one 16-byte vector per lane, non-temporal;
// pieces of 4 KiB or more take one index per workgroup (a scalar load, as the transport
// kernels read their block ids), smaller ones one per lane.  With the identity permutation
// it is the same kernel writing in order, the control of the pattern's cost.
__global__ __launch_bounds__(256) void piece_scatter_kernel(const dsp_u32x4* __restrict__ src,
                                                            dsp_u32x4* __restrict__ dst,
                                                            int64_t piece16, int64_t n16,
                                                            const int32_t* __restrict__ dst_index) {
  const int64_t base = int64_t(blockIdx.x) * 256;
  const int64_t f = base + threadIdx.x;
  if (piece16 >= 256) {
    const int64_t i = base / piece16;          // uniform: the workgroup lies in one piece
    const int64_t d = int64_t(dst_index[i]) * piece16 + (f - i * piece16);
    if (f < n16) dsp_st_stream(dsp_ld_stream(src + f), dst + d);
    return;
  }
  if (f >= n16) return;
  const int64_t i = f / piece16;
  dsp_st_stream(dsp_ld_stream(src + f), dst + int64_t(dst_index[i]) * piece16 + (f - i * piece16));
}

// The gather direction of the copy above: piece i of dst (contiguous) is read from
// src + src_index[i] * piece_bytes -- random source blocks, contiguous writes, the access
// pattern of the transport gather with no table logic.  Pieces of 4 KiB or more (one index
// per workgroup).
__global__ __launch_bounds__(256) void piece_gather_kernel(const dsp_u32x4* __restrict__ src,
                                                           dsp_u32x4* __restrict__ dst,
                                                           int64_t piece16, int64_t n16,
                                                           const int32_t* __restrict__ src_index) {
  const int64_t base = int64_t(blockIdx.x) * 256;
  const int64_t f = base + threadIdx.x;
  const int64_t i = base / piece16;  // uniform: the workgroup lies in one piece
  const int64_t s = int64_t(src_index[i]) * piece16 + (f - i * piece16);
  if (f < n16) dsp_st_stream(dsp_ld_stream(src + s), dst + f);
}

// The read of a decode batch with no arithmetic and no imbalance: workgroup w (KVH waves,
// wave h reading KV head h) reads keys [k0, min(k0 + kKeys, ctx_b)) of sequence b, where
// (b, k0) = work[w]; every key of every sequence once, the head slices of each slot row
// side by side (as the balanced decode kernel reads them when its head group is the whole
// row), K and V (K cached, V non-temporal, as the decode kernel loads them), addressed
// through the block table.  The host cuts every sequence into kKeys-key pieces, so all
// workgroups but a sequence's last read the same bytes.
constexpr int kSegKeys = 256;
__global__ __launch_bounds__(512) void batch_read_kernel(const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc,
                                                         int64_t num_slots,
                                                         const int32_t* __restrict__ bt,
                                                         int64_t bt_stride, int32_t log2_bs,
                                                         const int32_t* __restrict__ ctx_lens,
                                                         const int32_t* __restrict__ work,
                                                         int32_t KVH, uint32_t* __restrict__ sink) {
  constexpr int D = 128;
  const int b = work[2 * blockIdx.x], k0 = work[2 * blockIdx.x + 1];
  const int ctx = ctx_lens[b];
  const int h = int(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int bmask = (1 << log2_bs) - 1;
  const int k1 = min(k0 + kSegKeys, ctx);
  dsp_u32x4 acc = {0u, 0u, 0u, 0u};
  for (int t = k0; t < k1; t += 32) {
    dsp_u32x4 kv[8], vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = min(t + i * 4 + lane / 16, k1 - 1);
      int64_t slot = int64_t(bt[int64_t(b) * bt_stride + (key >> log2_bs)]) * (bmask + 1) +
                     (key & bmask);
      slot = (slot >= 0 && slot < num_slots) ? slot : 0;  // a bad block id reads row 0
      const int64_t e = slot * (int64_t(KVH) * D) + int64_t(h) * D + (lane % 16) * 8;
      kv[i] = *reinterpret_cast<const dsp_u32x4*>(kc + e);
      vv[i] = dsp_ld_stream(reinterpret_cast<const dsp_u32x4*>(vc + e));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc ^= kv[i] ^ vv[i];
  }
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) sink[0] = r;
}

// Stores only: piece i of dst (piece_bytes, a multiple of 4096) filled with a constant at
// dst + dst_index[i] * piece_bytes -- the write half of the copies above, alone (the
// copy-on-write fork's 32 copies of one block read it from L2 and write HBM only).  One
// one-shot workgroup per 4 KiB, one 16-byte non-temporal store per lane.
__global__ __launch_bounds__(256) void piece_fill_kernel(dsp_u32x4* __restrict__ dst,
                                                         int64_t piece16, int64_t n16,
                                                         const int32_t* __restrict__ dst_index,
                                                         uint32_t value) {
  const int64_t base = int64_t(blockIdx.x) * 256;
  const int64_t f = base + threadIdx.x;
  const int64_t i = base / piece16;  // uniform: the workgroup lies in one piece
  const int64_t d = int64_t(dst_index[i]) * piece16 + (f - i * piece16);
  if (f < n16) dsp_st_stream(dsp_u32x4{value, value, value, value}, dst + d);
}

// The map GEMM's loads without its arithmetic: the same 256 x 256 tiles in the same
// XCD-aware order, each 64-wide K stage of 256 A rows and 256 Bt rows (128 bytes each)
// going straight into LDS with global_load_lds_dwordx4, two stages resident, one barrier
// per stage -- what one launch of map_gemm_big_kernel needs just to fill its stages.
__global__ __launch_bounds__(512) void gemm_fill_kernel(const uint16_t* __restrict__ a, int64_t lda,
                                                        int64_t M, int64_t a_batch_stride,
                                                        const uint16_t* __restrict__ bt, int64_t ldb,
                                                        int64_t N, int64_t K,
                                                        uint32_t* __restrict__ sink) {
  constexpr int kBM = 256, kBN = 256, kBK = 64, kCPR = 8, kRowB = 128, kLPW = 8;
  constexpr int kStageB = (kBM + kBN) * kRowB;
  __shared__ __attribute__((aligned(1024))) char lds[2 * kStageB];
  const int tn = int((N + kBN - 1) / kBN), tm = int((M + kBM - 1) / kBM);
  int t = int(blockIdx.x);
  const int full = int(gridDim.x) & ~7;
  if (t < full) t = (t & 7) * (full >> 3) + (t >> 3);
  const int bx = t % tn, by = (t / tn) % tm, bz = t / (tn * tm);
  a += int64_t(bz) * a_batch_stride;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t m0 = int64_t(by) * kBM, n0 = int64_t(bx) * kBN;
  const bool loads_a = wave * kLPW * 64 < kBM * kCPR;
  uint32_t off[kLPW];
#pragma unroll
  for (int j = 0; j < kLPW; ++j) {
    const int r = (wave * kLPW + j) * (64 / kCPR) + lane / kCPR;
    const int chunk = (lane % kCPR) ^ (r & 7);
    const int64_t row = loads_a ? min<int64_t>(m0 + r, M - 1) : min<int64_t>(n0 + r - kBM, N - 1);
    off[j] = uint32_t(row * (loads_a ? lda : ldb) + chunk * 8);
  }
  auto issue = [&](int buf, int64_t k0) {
    const uint16_t* src = (loads_a ? a : bt) + k0;
    char* dst = lds + buf * kStageB + wave * kLPW * 1024;
#pragma unroll
    for (int j = 0; j < kLPW; ++j)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + off[j]),
                                       (__attribute__((address_space(3))) void*)(dst + j * 1024),
                                       16, 0, 0);
  };
  const int nk = int(K / kBK);
  issue(0, 0);
  uint32_t h = 0;
  for (int kt = 0; kt < nk; ++kt) {
    __syncthreads();  // stage kt landed; every wave is past its read of stage kt - 1
    h ^= *reinterpret_cast<const uint32_t*>(lds + (kt & 1) * kStageB + threadIdx.x * 4);
    if (kt + 1 < nk) issue((kt + 1) & 1, int64_t(kt + 1) * kBK);
  }
  if (h == 0x9e3779b9u) sink[0] = h;
}

}  // namespace

extern "C" int dsp_probe_stream_copy(const void* src, void* dst, int64_t bytes,
                                     int32_t workgroups, dsp_stream_t stream) {
  DSP_HOST_CHECK(src && dst && bytes >= 16 && workgroups > 0, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(src, 16) && dsp_aligned(dst, 16), DSP_EALIGN);
  const int64_t n16 = bytes / 16;
  const int64_t per = (n16 + workgroups - 1) / workgroups;
  stream_copy_kernel<<<dim3(static_cast<unsigned>(workgroups)), 256, 0,
                       static_cast<hipStream_t>(stream)>>>(
      static_cast<const dsp_u32x4*>(src), static_cast<dsp_u32x4*>(dst), n16, per);
  return dsp_launch_status();
}

extern "C" int dsp_probe_stream_read(const void* buf, int64_t bytes, int32_t workgroups,
                                     uint32_t* sink, dsp_stream_t stream) {
  DSP_HOST_CHECK(buf && sink && bytes >= 16 && workgroups > 0, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(buf, 16), DSP_EALIGN);
  const int64_t n16 = bytes / 16;
  const int64_t per = (n16 + workgroups - 1) / workgroups;
  stream_read_kernel<<<dim3(static_cast<unsigned>(workgroups)), 256, 0,
                       static_cast<hipStream_t>(stream)>>>(
      static_cast<const dsp_u32x4*>(buf), n16, per, sink);
  return dsp_launch_status();
}

extern "C" int dsp_probe_slice_read(const void* k_cache, const void* v_cache, int64_t num_slots,
                                    const int32_t* block_table, int64_t bt_stride,
                                    int32_t block_size, int32_t B, int32_t KVH, int32_t ctx,
                                    int32_t waves_per_seq_head, uint32_t* sink,
                                    dsp_stream_t stream) {
  DSP_HOST_CHECK(k_cache && v_cache && block_table && sink, DSP_EINVAL);
  DSP_HOST_CHECK(B > 0 && KVH > 0 && ctx > 0 && waves_per_seq_head > 0, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_is_pow2(block_size), DSP_EINVAL);
  DSP_HOST_CHECK(ctx % (32 * waves_per_seq_head) == 0, DSP_EINVAL);
  DSP_HOST_CHECK(bt_stride * block_size >= ctx, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(k_cache, 16) && dsp_aligned(v_cache, 16), DSP_EALIGN);
  DSP_HOST_CHECK(num_slots > 0, DSP_EINVAL);
  const int HG = KVH % 4 == 0 ? 4 : 1;  // heads read side by side, as the decode kernel does
  const int64_t grid = int64_t(B) * (KVH / HG) * waves_per_seq_head;
  DSP_HOST_CHECK(grid < (int64_t(1) << 31), DSP_EINVAL);
  const auto* kh = static_cast<const uint16_t*>(k_cache);
  const auto* vh = static_cast<const uint16_t*>(v_cache);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (HG == 4)
    slice_read_kernel<4><<<dim3(static_cast<unsigned>(grid)), 256, 0, st>>>(
        kh, vh, num_slots, block_table, bt_stride, dsp_log2i(block_size), KVH,
        ctx / waves_per_seq_head, waves_per_seq_head, sink);
  else
    slice_read_kernel<1><<<dim3(static_cast<unsigned>(grid)), 64, 0, st>>>(
        kh, vh, num_slots, block_table, bt_stride, dsp_log2i(block_size), KVH,
        ctx / waves_per_seq_head, waves_per_seq_head, sink);
  return dsp_launch_status();
}

extern "C" int dsp_probe_gemm_fill(const void* a, int64_t lda, int64_t M, int64_t a_batch_stride,
                                   const void* bt, int64_t ldb, int64_t N, int64_t K,
                                   int32_t batch, uint32_t* sink, dsp_stream_t stream) {
  DSP_HOST_CHECK(a && bt && sink && M > 0 && N > 0 && batch > 0, DSP_EINVAL);
  DSP_HOST_CHECK(K > 0 && K % 64 == 0 && lda >= K && ldb >= K && lda % 8 == 0 && ldb % 8 == 0 &&
                     a_batch_stride % 8 == 0,
                 DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(a, 16) && dsp_aligned(bt, 16), DSP_EALIGN);
  DSP_HOST_CHECK((M - 1) * lda + K <= int64_t(UINT32_MAX) && (N - 1) * ldb + K <= int64_t(UINT32_MAX),
                 DSP_EINVAL);
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256) * batch;
  DSP_HOST_CHECK(tiles < (int64_t(1) << 31), DSP_EINVAL);
  gemm_fill_kernel<<<dim3(static_cast<unsigned>(tiles)), 512, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(a), lda, M, a_batch_stride, static_cast<const uint16_t*>(bt), ldb,
      N, K, sink);
  return dsp_launch_status();
}

extern "C" int dsp_probe_piece_scatter(const void* src, void* dst, int64_t bytes,
                                       int64_t piece_bytes, const int32_t* dst_index,
                                       dsp_stream_t stream) {
  DSP_HOST_CHECK(src && dst && dst_index && bytes >= 16 && piece_bytes >= 16, DSP_EINVAL);
  DSP_HOST_CHECK(piece_bytes % 16 == 0 && bytes % piece_bytes == 0, DSP_EINVAL);
  // a piece of 4 KiB or more must hold whole workgroups (4 KiB each)
  DSP_HOST_CHECK(piece_bytes < 4096 || piece_bytes % 4096 == 0, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(src, 16) && dsp_aligned(dst, 16), DSP_EALIGN);
  const int64_t n16 = bytes / 16;
  const int64_t grid = (n16 + 255) / 256;
  DSP_HOST_CHECK(grid < (int64_t(1) << 31), DSP_EINVAL);
  piece_scatter_kernel<<<dim3(static_cast<unsigned>(grid)), 256, 0,
                         static_cast<hipStream_t>(stream)>>>(
      static_cast<const dsp_u32x4*>(src), static_cast<dsp_u32x4*>(dst), piece_bytes / 16, n16,
      dst_index);
  return dsp_launch_status();
}

extern "C" int dsp_probe_piece_fill(void* dst, int64_t bytes, int64_t piece_bytes,
                                    const int32_t* dst_index, dsp_stream_t stream) {
  DSP_HOST_CHECK(dst && dst_index && bytes >= 4096 && piece_bytes >= 4096, DSP_EINVAL);
  DSP_HOST_CHECK(piece_bytes % 4096 == 0 && bytes % piece_bytes == 0, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(dst, 16), DSP_EALIGN);
  const int64_t n16 = bytes / 16;
  const int64_t grid = n16 / 256;
  DSP_HOST_CHECK(grid < (int64_t(1) << 31), DSP_EINVAL);
  piece_fill_kernel<<<dim3(static_cast<unsigned>(grid)), 256, 0,
                      static_cast<hipStream_t>(stream)>>>(static_cast<dsp_u32x4*>(dst),
                                                          piece_bytes / 16, n16, dst_index,
                                                          0x3f803f80u);
  return dsp_launch_status();
}

extern "C" int dsp_probe_piece_gather(const void* src, void* dst, int64_t bytes,
                                      int64_t piece_bytes, const int32_t* src_index,
                                      dsp_stream_t stream) {
  DSP_HOST_CHECK(src && dst && src_index && bytes >= 16 && piece_bytes >= 4096, DSP_EINVAL);
  DSP_HOST_CHECK(piece_bytes % 4096 == 0 && bytes % piece_bytes == 0, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(src, 16) && dsp_aligned(dst, 16), DSP_EALIGN);
  const int64_t n16 = bytes / 16;
  DSP_HOST_CHECK(n16 / 256 < (int64_t(1) << 31), DSP_EINVAL);
  piece_gather_kernel<<<dim3(static_cast<unsigned>((n16 + 255) / 256)), 256, 0,
                        static_cast<hipStream_t>(stream)>>>(
      static_cast<const dsp_u32x4*>(src), static_cast<dsp_u32x4*>(dst), piece_bytes / 16, n16,
      src_index);
  return dsp_launch_status();
}

extern "C" int dsp_probe_batch_read(const void* k_cache, const void* v_cache, int64_t num_slots,
                                    const int32_t* block_table, int64_t bt_stride,
                                    int32_t block_size, const int32_t* ctx_lens,
                                    const int32_t* work, int32_t num_work, int32_t KVH,
                                    uint32_t* sink, dsp_stream_t stream) {
  DSP_HOST_CHECK(k_cache && v_cache && block_table && ctx_lens && work && sink, DSP_EINVAL);
  DSP_HOST_CHECK(num_work > 0 && KVH > 0 && KVH <= 8 && num_slots > 0, DSP_EINVAL);
  DSP_HOST_CHECK(dsp_is_pow2(block_size), DSP_EINVAL);
  DSP_HOST_CHECK(dsp_aligned(k_cache, 16) && dsp_aligned(v_cache, 16), DSP_EALIGN);
  batch_read_kernel<<<dim3(static_cast<unsigned>(num_work)), 64 * KVH, 0,
                      static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(k_cache), static_cast<const uint16_t*>(v_cache), num_slots,
      block_table, bt_stride, dsp_log2i(block_size), ctx_lens, work, KVH, sink);
  return dsp_launch_status();
}
