// The attention prologue of a decoder layer in one launch: per-head RMSNorm of q and k
// (Qwen3's q_norm / k_norm), RoPE on q and k, and the append of k and v into the paged
// pool.  Replaces the op sequence of ModelRunner._attention (dispec/engine/model_runner.py:
// 142-148):
//     q = q_norm(q); k = k_norm(k)              (Qwen3RMSNorm: fp32 variance, rsqrt, round
//                                                to the model dtype, times the weight)
//     q = q * cos + rotate_half(q) * sin        (_apply_rope, :49-50 there: every product
//     k = k * cos + rotate_half(k) * sin         and the sum rounded to the model dtype)
//     cache.write(layer, slots, k, v)           (index_copy_, paged_cache.py:61-68)
// which torch runs as ~25 elementwise and reduction kernels, each a round trip of q/k
// through HBM.  Rounding points are the reference's, so apart from the variance's
// summation order (fp32, different tree) the results are bit-identical.
//
// Layout on gfx950: a row (one head of one token, D elements) is held by D/8 lanes, 16
// bytes each; the sum of squares is a butterfly over those lanes, and rotate_half's
// partner element (d +- D/2) sits D/16 lanes away, one cross-lane exchange.  One launch
// covers the T*(Hq + KVH) rows of the step; a k row also moves its v row.
#include "dsp_common.h"

namespace {

// Where the prologue's stores with nowhere to go land (their values are never read): 16
// bytes per thread of a 256-thread workgroup, one region per device shared by every launch.
__device__ __attribute__((aligned(16))) uint16_t g_prologue_drop[256 * 8];

struct Bf16Tag {};
struct F16Tag {};

template <typename Tag>
__device__ __forceinline__ float lo(uint32_t u) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value) return dsp_bf16lo(u);
  else return dsp_f16lo(u);
}
template <typename Tag>
__device__ __forceinline__ float hi(uint32_t u) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value) return dsp_bf16hi(u);
  else return dsp_f16hi(u);
}
template <typename Tag>
__device__ __forceinline__ uint16_t rnd(float f) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value) return dsp_f32_to_bf16(f);
  else return dsp_f32_to_f16(f);
}
// Round to the model dtype and back: the value a torch op on that dtype produces.
template <typename Tag>
__device__ __forceinline__ float r(float f) {
  const uint16_t b = rnd<Tag>(f);
  return lo<Tag>(uint32_t(b));
}

__device__ __forceinline__ uint32_t shfl_xor_u32(uint32_t x, int mask) {
  const int lane = __lane_id();
  return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, static_cast<int>(x)));
}

template <typename Tag, int D>
__global__ __launch_bounds__(256) void qk_prologue_kernel(
    const uint16_t* __restrict__ q, int64_t qst, int64_t qsh, const uint16_t* __restrict__ k,
    int64_t kst, int64_t ksh, const uint16_t* __restrict__ v, int64_t vst, int64_t vsh,
    const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw, float eps,
    const uint16_t* __restrict__ cosp, const uint16_t* __restrict__ sinp, int64_t rst,
    const int64_t* __restrict__ slots, int64_t T, int32_t Hq, int32_t KVH,
    uint16_t* __restrict__ qo, int64_t qost, int64_t qosh, uint16_t* __restrict__ kpool,
    uint16_t* __restrict__ vpool, int64_t num_slots, int64_t pss, int64_t psh,
    int32_t* __restrict__ err_count) {
  constexpr int LPR = D / 8;       // lanes per row
  constexpr int RPW = 64 / LPR;    // rows per wave
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPR;      // 8-element chunk of the row this lane holds
  const int64_t row = (int64_t(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64) * RPW +
                      lane / LPR;
  const int heads = Hq + KVH;
  const bool live = row < T * heads;
  const int64_t t = live ? row / heads : 0;
  const int j = live ? static_cast<int>(row % heads) : 0;
  const bool is_q = j < Hq;
  const int kh = j - Hq;

  // Every load of the lane is issued here, together: the row, the norm weight, the RoPE
  // cos/sin, the token's slot and the v row a k lane stores (a lane past the rows reads
  // token 0's; q lanes read KV head 0's v row, lines the k lanes read anyway), so the lane
  // waits for one memory round trip instead of one per dependent step.
  const uint16_t* src = is_q ? q + t * qst + int64_t(j) * qsh : k + t * kst + int64_t(kh) * ksh;
  const uint16_t* w = is_q ? qw : kw;
  const dsp_u32x4 x = *reinterpret_cast<const dsp_u32x4*>(src + 8 * sub);
  const dsp_u32x4 wv = *reinterpret_cast<const dsp_u32x4*>((w != nullptr ? w : src) + 8 * sub);
  const dsp_u32x4 cv = *reinterpret_cast<const dsp_u32x4*>(cosp + t * rst + 8 * sub);
  const dsp_u32x4 sv = *reinterpret_cast<const dsp_u32x4*>(sinp + t * rst + 8 * sub);
  const int64_t slot = slots[t];
  const dsp_u32x4 vrow = *reinterpret_cast<const dsp_u32x4*>(
      v + t * vst + int64_t(is_q ? 0 : kh) * vsh + 8 * sub);
  // a compiler-only fence (no instruction): the loads above are not moved below it
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_sched_barrier(0);
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = lo<Tag>(x[i]);
    f[2 * i + 1] = hi<Tag>(x[i]);
  }

  // RMSNorm over the row: var = mean(x^2) in fp32, x * rsqrt(var + eps) rounded to the
  // dtype, times the weight (rounded).  Computed whatever w is and selected after, so that
  // the weight load has a use outside any branch (the compiler sinks a load into the branch
  // that uses it, behind the wait for x).
  {
    const bool norm = w != nullptr;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) ss += __int_as_float(static_cast<int>(shfl_xor_u32(__float_as_uint(ss), m)));
    const float inv = rsqrtf(ss / float(D) + eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = r<Tag>(lo<Tag>(wv[i]) * r<Tag>(f[2 * i] * inv));
      const float b = r<Tag>(hi<Tag>(wv[i]) * r<Tag>(f[2 * i + 1] * inv));
      f[2 * i] = norm ? a : f[2 * i];
      f[2 * i + 1] = norm ? b : f[2 * i + 1];
    }
  }

  // RoPE: out[d] = (x[d] * cos[d]) + (rot[d] * sin[d]), each product and the sum rounded;
  // rot[d] = -x[d + D/2] for d < D/2, x[d - D/2] otherwise -- the partner chunk is LPR/2
  // lanes away.
  uint32_t packed[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) packed[i] = uint32_t(rnd<Tag>(f[2 * i])) | (uint32_t(rnd<Tag>(f[2 * i + 1])) << 16);
  float pr[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = shfl_xor_u32(packed[i], LPR / 2);
    pr[2 * i] = lo<Tag>(o);
    pr[2 * i + 1] = hi<Tag>(o);
  }
  const bool first_half = sub < LPR / 2;
  dsp_u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float o2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float c = e ? hi<Tag>(cv[i]) : lo<Tag>(cv[i]);
      const float s = e ? hi<Tag>(sv[i]) : lo<Tag>(sv[i]);
      const float rot = first_half ? -pr[2 * i + e] : pr[2 * i + e];
      o2[e] = r<Tag>(r<Tag>(f[2 * i + e] * c) + r<Tag>(rot * s));
    }
    out[i] = uint32_t(rnd<Tag>(o2[0])) | (uint32_t(rnd<Tag>(o2[1])) << 16);
  }

  // Two stores per lane, neither under a branch (else the compiler sinks the loads that only
  // they use behind the waits of the steps above): a q row to q_out, a k row and its v row
  // to the token's pool slot; a lane past the rows, a k row whose slot is out of range and
  // a q lane's v store write into g_prologue_drop instead.  Bad slots are counted after.
  const bool slot_ok = slot >= 0 && slot < num_slots;
  uint16_t* const drop = g_prologue_drop + 8 * threadIdx.x;
  const int64_t pe = (slot_ok ? slot : 0) * pss + int64_t(is_q ? 0 : kh) * psh + 8 * sub;
  uint16_t* const o_dst = !live  ? drop
                          : is_q ? qo + t * qost + int64_t(j) * qosh + 8 * sub
                          : slot_ok ? kpool + pe
                                    : drop;
  *reinterpret_cast<dsp_u32x4*>(o_dst) = out;
  *reinterpret_cast<dsp_u32x4*>(live && !is_q && slot_ok ? vpool + pe : drop) = vrow;
  if (live && !is_q && !slot_ok && sub == 0 && err_count) atomicAdd(err_count, 1);
}

// fp32 models: the same prologue with 4 elements per 16-byte lane (D/4 lanes per row) and
// no rounding between the steps (every torch op on fp32 tensors rounds to fp32, which the
// fp32 arithmetic here does as it goes).
template <int D>
__global__ __launch_bounds__(256) void qk_prologue_f32_kernel(
    const float* __restrict__ q, int64_t qst, int64_t qsh, const float* __restrict__ k,
    int64_t kst, int64_t ksh, const float* __restrict__ v, int64_t vst, int64_t vsh,
    const float* __restrict__ qw, const float* __restrict__ kw, float eps,
    const float* __restrict__ cosp, const float* __restrict__ sinp, int64_t rst,
    const int64_t* __restrict__ slots, int64_t T, int32_t Hq, int32_t KVH,
    float* __restrict__ qo, int64_t qost, int64_t qosh, float* __restrict__ kpool,
    float* __restrict__ vpool, int64_t num_slots, int64_t pss, int64_t psh,
    int32_t* __restrict__ err_count) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int LPR = D / 4;       // lanes per row
  constexpr int RPW = 64 / LPR;    // rows per wave
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPR;      // 4-element chunk of the row this lane holds
  const int64_t row = (int64_t(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64) * RPW +
                      lane / LPR;
  const int heads = Hq + KVH;
  const bool live = row < T * heads;
  const int64_t t = live ? row / heads : 0;
  const int j = live ? static_cast<int>(row % heads) : 0;
  const bool is_q = j < Hq;
  const int kh = j - Hq;
  const float* src = is_q ? q + t * qst + int64_t(j) * qsh : k + t * kst + int64_t(kh) * ksh;
  f4 x = live ? *reinterpret_cast<const f4*>(src + 4 * sub) : f4{0.f, 0.f, 0.f, 0.f};
  const float* w = is_q ? qw : kw;
  if (w != nullptr) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss = fmaf(x[i], x[i], ss);
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) ss += __int_as_float(static_cast<int>(shfl_xor_u32(__float_as_uint(ss), m)));
    const float inv = rsqrtf(ss / float(D) + eps);
    const f4 wv = *reinterpret_cast<const f4*>(w + 4 * sub);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = wv[i] * (x[i] * inv);
  }
  f4 pr;
#pragma unroll
  for (int i = 0; i < 4; ++i) pr[i] = __uint_as_float(shfl_xor_u32(__float_as_uint(x[i]), LPR / 2));
  const bool first_half = sub < LPR / 2;
  const f4 cv = *reinterpret_cast<const f4*>(cosp + t * rst + 4 * sub);
  const f4 sv = *reinterpret_cast<const f4*>(sinp + t * rst + 4 * sub);
  f4 out;
  {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float rot = first_half ? -pr[i] : pr[i];
      out[i] = x[i] * cv[i] + rot * sv[i];
    }
  }
  if (!live) return;
  if (is_q) {
    *reinterpret_cast<f4*>(qo + t * qost + int64_t(j) * qosh + 4 * sub) = out;
    return;
  }
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) {
    if (sub == 0 && err_count) atomicAdd(err_count, 1);
    return;
  }
  const int64_t pe = slot * pss + int64_t(kh) * psh + 4 * sub;
  *reinterpret_cast<f4*>(kpool + pe) = out;
  *reinterpret_cast<f4*>(vpool + pe) = *reinterpret_cast<const f4*>(v + t * vst + int64_t(kh) * vsh + 4 * sub);
}

template <typename... A>
int launch_f32(int D, unsigned grid, hipStream_t s, A... args) {
  switch (D) {
    case 32: qk_prologue_f32_kernel<32><<<grid, 256, 0, s>>>(args...); break;
    case 64: qk_prologue_f32_kernel<64><<<grid, 256, 0, s>>>(args...); break;
    case 128: qk_prologue_f32_kernel<128><<<grid, 256, 0, s>>>(args...); break;
    case 256: qk_prologue_f32_kernel<256><<<grid, 256, 0, s>>>(args...); break;
    default: return DSP_EUNSUPPORTED;
  }
  return dsp_launch_status();
}

template <typename Tag, typename... A>
int launch(int D, unsigned grid, hipStream_t s, A... args) {
  switch (D) {
    case 32: qk_prologue_kernel<Tag, 32><<<grid, 256, 0, s>>>(args...); break;
    case 64: qk_prologue_kernel<Tag, 64><<<grid, 256, 0, s>>>(args...); break;
    case 128: qk_prologue_kernel<Tag, 128><<<grid, 256, 0, s>>>(args...); break;
    case 256: qk_prologue_kernel<Tag, 256><<<grid, 256, 0, s>>>(args...); break;
    default: return DSP_EUNSUPPORTED;
  }
  return dsp_launch_status();
}

}  // namespace

extern "C" int dsp_qk_norm_rope_append(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t,
    int64_t k_stride_h, const void* v, int64_t v_stride_t, int64_t v_stride_h,
    const void* q_norm_weight, const void* k_norm_weight, float eps, const void* cos_table,
    const void* sin_table, int64_t rope_stride_t, const int64_t* slots, int64_t T, int32_t Hq,
    int32_t KVH, int32_t D, void* q_out, int64_t q_out_stride_t, int64_t q_out_stride_h,
    void* k_pool, void* v_pool, int64_t num_slots, int64_t pool_stride_slot,
    int64_t pool_stride_head, int32_t dtype, int32_t* err_count, dsp_stream_t stream) {
  DSP_HOST_CHECK(T >= 0 && Hq > 0 && KVH > 0 && num_slots >= 0, DSP_EINVAL);
  DSP_HOST_CHECK((q_norm_weight == nullptr) == (k_norm_weight == nullptr), DSP_EINVAL);
  DSP_HOST_CHECK(dtype == DSP_BF16 || dtype == DSP_F16 || dtype == DSP_F32, DSP_EUNSUPPORTED);
  DSP_HOST_CHECK(D == 32 || D == 64 || D == 128 || D == 256, DSP_EUNSUPPORTED);
  if (T == 0) return DSP_OK;
  DSP_HOST_CHECK(q && k && v && cos_table && sin_table && slots && q_out && k_pool && v_pool,
                 DSP_EINVAL);
  DSP_HOST_CHECK(q_stride_t >= 0 && q_stride_h >= 0 && k_stride_t >= 0 && k_stride_h >= 0 &&
                     v_stride_t >= 0 && v_stride_h >= 0 && rope_stride_t >= 0 &&
                     pool_stride_slot >= 0 && pool_stride_head >= 0,
                 DSP_EINVAL);
  // 16-byte vectors: every row start and every stride a multiple of 16 bytes
  const int64_t ve = dtype == DSP_F32 ? 4 : 8;  // elements per 16 bytes
  DSP_HOST_CHECK(q_stride_t % ve == 0 && q_stride_h % ve == 0 && k_stride_t % ve == 0 &&
                     k_stride_h % ve == 0 && v_stride_t % ve == 0 && v_stride_h % ve == 0 &&
                     rope_stride_t % ve == 0 && q_out_stride_t % ve == 0 &&
                     q_out_stride_h % ve == 0 && pool_stride_slot % ve == 0 &&
                     pool_stride_head % ve == 0,
                 DSP_EALIGN);
  DSP_HOST_CHECK(dsp_aligned(q, 16) && dsp_aligned(k, 16) && dsp_aligned(v, 16) &&
                     dsp_aligned(cos_table, 16) && dsp_aligned(sin_table, 16) &&
                     dsp_aligned(q_out, 16) && dsp_aligned(k_pool, 16) &&
                     dsp_aligned(v_pool, 16) &&
                     (q_norm_weight == nullptr ||
                      (dsp_aligned(q_norm_weight, 16) && dsp_aligned(k_norm_weight, 16))),
                 DSP_EALIGN);
  const int rows_per_block = 4 * (64 / (D / int(ve)));
  const int64_t rows = T * int64_t(Hq + KVH);
  const int64_t grid = (rows + rows_per_block - 1) / rows_per_block;
  DSP_HOST_CHECK(grid < (int64_t(1) << 31), DSP_EINVAL);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == DSP_F32)
    return launch_f32(D, static_cast<unsigned>(grid), s, static_cast<const float*>(q),
                      q_stride_t, q_stride_h, static_cast<const float*>(k), k_stride_t,
                      k_stride_h, static_cast<const float*>(v), v_stride_t, v_stride_h,
                      static_cast<const float*>(q_norm_weight),
                      static_cast<const float*>(k_norm_weight), eps,
                      static_cast<const float*>(cos_table), static_cast<const float*>(sin_table),
                      rope_stride_t, slots, T, Hq, KVH, static_cast<float*>(q_out),
                      q_out_stride_t, q_out_stride_h, static_cast<float*>(k_pool),
                      static_cast<float*>(v_pool), num_slots, pool_stride_slot,
                      pool_stride_head, err_count);
  auto qh = static_cast<const uint16_t*>(q);
  auto kh = static_cast<const uint16_t*>(k);
  auto vh = static_cast<const uint16_t*>(v);
  auto qw = static_cast<const uint16_t*>(q_norm_weight);
  auto kw = static_cast<const uint16_t*>(k_norm_weight);
  auto ch = static_cast<const uint16_t*>(cos_table);
  auto sh = static_cast<const uint16_t*>(sin_table);
  auto qo = static_cast<uint16_t*>(q_out);
  auto kp = static_cast<uint16_t*>(k_pool);
  auto vp = static_cast<uint16_t*>(v_pool);
  if (dtype == DSP_BF16)
    return launch<Bf16Tag>(D, static_cast<unsigned>(grid), s, qh, q_stride_t, q_stride_h, kh,
                           k_stride_t, k_stride_h, vh, v_stride_t, v_stride_h, qw, kw, eps, ch, sh,
                           rope_stride_t, slots, T, Hq, KVH, qo, q_out_stride_t, q_out_stride_h,
                           kp, vp, num_slots, pool_stride_slot, pool_stride_head, err_count);
  return launch<F16Tag>(D, static_cast<unsigned>(grid), s, qh, q_stride_t, q_stride_h, kh,
                        k_stride_t, k_stride_h, vh, v_stride_t, v_stride_h, qw, kw, eps, ch, sh,
                        rope_stride_t, slots, T, Hq, KVH, qo, q_out_stride_t, q_out_stride_h, kp,
                        vp, num_slots, pool_stride_slot, pool_stride_head, err_count);
}
