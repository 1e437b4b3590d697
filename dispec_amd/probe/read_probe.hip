// Bandwidth probes for the roofline: what this GPU's HBM delivers to (1) a plain streaming
// read, (2) a read with the paged decode's access pattern, with no compute, and (3) a plain
// streaming copy (the ceiling of the append / gather / scatter / block-copy kernels).
// They calibrate the decode kernel's measured GB/s: the datasheet peak (8 TB/s) is not
// reachable by any read, and the slot-major pool layout (one KV head's 256-byte slice of
// every 2 KiB slot row) caps what the decode can fetch below a streaming read.  Both probes
// reduce what they read to one word that is stored only if it matches a sentinel, so the
// loads cannot be removed.
#include "../csrc/dsp_common.h"
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
// load), addressed through the block table exactly as the decode kernels address the pool.
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
      vv[i] = *reinterpret_cast<const dsp_u32x4*>(vc + e);
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
