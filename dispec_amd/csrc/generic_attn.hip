// J3 / J4 for the shapes the tuned attention kernels leave out: fp32 caches, head_dim 8 or
// 256 (any power of two from 8 to 256), GQA groups above 8 on decode.  The reference's
// Triton kernel takes any power-of-two HEAD_DIM and loads keys and values as fp32
// (dispec/engine/triton_attn.py:60-95, tl.arange(0, HEAD_DIM) at :71); its native path
// attends in whatever dtype the model runs (dispec/engine/model_runner.py:160-185).  These
// two kernels give dsp_paged_decode and dsp_paged_mq_attention the same reach -- correct
// and coalesced, without the tuned kernels' MFMA tiles:
//
//  * one wave per (query row, query head, key partition of P keys); lane d holds dims d,
//    d + 64, ..., so every K or V row is read by one coalesced load per 64 dims;
//  * eight keys per step: eight partial dot products reduced across the wave side by side
//    (DPP within rows of 16 lanes, then two lane permutes), an online softmax in base 2,
//    fp32 accumulation;
//  * query row i of sequence b's block sees keys j <= ctx_b - q_len_b + i (causal,
//    lower-right); decode is one row per sequence over its whole context;
//  * a row with more than one partition is merged by the second kernel (16 partitions'
//    partials in flight per lane).
//
// Grid x runs over B * max_q_len row slots z (b = z / max_q_len, i = z % max_q_len), as the
// tiled kernels' grids do: a sequence's rows beyond max_q_len are not computed.  Partial
// results go to ws row (z * Hq + h) * num_parts + part (B * max_q_len * Hq rows of
// num_parts partitions, then their (max, sum) pairs).
#include <float.h>

#include <type_traits>

#include "dsp_common.h"
#include "dsp_internal.h"

namespace {

struct GBf16 { using store = uint16_t; };
struct GF16 { using store = uint16_t; };
struct GF32 { using store = float; };

template <typename Tag>
__device__ __forceinline__ float ld1(const typename Tag::store* p) {
  if constexpr (std::is_same<Tag, GBf16>::value)
    return dsp_bf16lo(*p);
  else if constexpr (std::is_same<Tag, GF16>::value)
    return dsp_f16lo(*p);
  else
    return *p;
}

template <typename Tag>
__device__ __forceinline__ typename Tag::store st1(float f) {
  if constexpr (std::is_same<Tag, GBf16>::value)
    return dsp_f32_to_bf16(f);
  else if constexpr (std::is_same<Tag, GF16>::value)
    return dsp_f32_to_f16(f);
  else
    return f;
}

constexpr int kKeysPerStep = 8;
constexpr int kMergeBatch = 16;

// Where row slot z sits and how many keys it sees.
struct RowInfo {
  int b;         // sequence
  int64_t tok;   // packed row of q / out
  int vis;       // visible keys; 0 writes zeros
  bool live;     // false: slot beyond the sequence's q_len (nothing to write)
  bool counted;  // this slot reports the sequence's bad lengths (one slot per sequence)
};

__device__ __forceinline__ RowInfo row_info(const int32_t* __restrict__ cu_q,
                                            const int32_t* __restrict__ ctx_lens,
                                            int max_q_len, int max_ctx, int z) {
  RowInfo r;
  r.b = z / max_q_len;
  const int i = z - r.b * max_q_len;
  const int ctx = ctx_lens[r.b];
  if (cu_q == nullptr) {  // decode: one row per sequence, context clamped to [0, max_ctx]
    r.tok = r.b;
    r.live = true;
    r.vis = ctx < 0 ? 0 : (ctx > max_ctx ? max_ctx : ctx);
    r.counted = ctx < 0 || ctx > max_ctx;
    return r;
  }
  const int c0 = cu_q[r.b];
  const int qlen = cu_q[r.b + 1] - c0;
  r.tok = int64_t(c0) + i;
  r.live = i < qlen;
  const bool bad = qlen < 0 || ctx < qlen || ctx > max_ctx;
  r.vis = bad ? 0 : ctx - qlen + i + 1;
  r.counted = bad && i == 0;
  return r;
}

// Sum over all 64 lanes of the wave, every lane ending with the total.
__device__ __forceinline__ float wave_sum(float v) {
  v = dsp_group_sum<16>(v);
  v += dsp_shfl_xor(v, 16);
  return v + dsp_shfl_xor(v, 32);
}

template <typename Tag, int D>
__global__ __launch_bounds__(64) void generic_attn_kernel(
    const typename Tag::store* __restrict__ q, int64_t qst, int64_t qsh,
    const typename Tag::store* __restrict__ kc, const typename Tag::store* __restrict__ vc,
    int64_t num_slots, int64_t kvs_slot, int64_t kvs_head, const int32_t* __restrict__ table,
    int64_t table_stride, int32_t log2_bs, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ ctx_lens, int32_t G, int32_t max_ctx, int32_t max_q_len,
    float scale_log2, int32_t P, int32_t num_parts, float* __restrict__ ws_acc,
    float* __restrict__ ws_ml, typename Tag::store* __restrict__ out, int64_t ost, int64_t osh,
    int32_t* __restrict__ err_count) {
  constexpr int NV = D > 64 ? D / 64 : 1;  // dims per lane
  const int z = blockIdx.x, h = blockIdx.y, part = blockIdx.z, Hq = gridDim.y;
  const int lane = threadIdx.x;
  const bool act = lane < D;
  const RowInfo r = row_info(cu_q, ctx_lens, max_q_len, max_ctx, z);
  if (!r.live) return;
  if (r.counted && part == 0 && h == 0 && lane == 0 && err_count) atomicAdd(err_count, 1);
  const int vis = r.vis;
  const int nparts = vis > 0 ? (vis + P - 1) / P : 1;
  typename Tag::store* o = out + r.tok * ost + int64_t(h) * osh;
  if (vis <= 0) {  // no keys (an empty context or bad lengths): zeros
    if (part == 0 && act) {
#pragma unroll
      for (int j = 0; j < NV; ++j) o[lane + 64 * j] = st1<Tag>(0.f);
    }
    return;
  }
  if (part >= nparts) return;
  const int kbeg = part * P, kend = min(kbeg + P, vis);
  float qf[NV], acc[NV];
  const typename Tag::store* qrow = q + r.tok * qst + int64_t(h) * qsh;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    qf[j] = act ? ld1<Tag>(qrow + lane + 64 * j) * scale_log2 : 0.f;
    acc[j] = 0.f;
  }
  const int64_t head_off = int64_t(h / G) * kvs_head + (act ? lane : 0);
  const int32_t* trow = table + int64_t(r.b) * table_stride;
  float m = -INFINITY, l = 0.f;
  bool bad_slot = false;
  for (int k0 = kbeg; k0 < kend; k0 += kKeysPerStep) {
    float kv[kKeysPerStep][NV], vv[kKeysPerStep][NV], s[kKeysPerStep];
    bool ok[kKeysPerStep];
#pragma unroll
    for (int u = 0; u < kKeysPerStep; ++u) {
      const int key = k0 + u;
      int64_t sl = 0;
      if (key < kend) {
        sl = log2_bs >= 0 ? (int64_t(trow[key >> log2_bs]) << log2_bs) +
                                (key & ((1 << log2_bs) - 1))
                          : int64_t(trow[key]);
      }
      ok[u] = key < kend && sl >= 0 && sl < num_slots;
      bad_slot |= key < kend && !ok[u];
      const int64_t e = (ok[u] ? sl : 0) * kvs_slot + head_off;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        kv[u][j] = act && ok[u] ? ld1<Tag>(kc + e + 64 * j) : 0.f;
        vv[u][j] = act && ok[u] ? ld1<Tag>(vc + e + 64 * j) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kKeysPerStep; ++u) {
      float p = 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j) p = fmaf(qf[j], kv[u][j], p);
      s[u] = wave_sum(p);
    }
    float mx = m;
#pragma unroll
    for (int u = 0; u < kKeysPerStep; ++u) {
      s[u] = ok[u] ? s[u] : -INFINITY;
      mx = fmaxf(mx, s[u]);
    }
    const float mu = mx == -INFINITY ? 0.f : mx;
    const float alpha = dsp_exp2(m - mu);
    l *= alpha;
#pragma unroll
    for (int j = 0; j < NV; ++j) acc[j] *= alpha;
#pragma unroll
    for (int u = 0; u < kKeysPerStep; ++u) {
      const float p = dsp_exp2(s[u] - mu);
      l += p;
#pragma unroll
      for (int j = 0; j < NV; ++j) acc[j] = fmaf(p, vv[u][j], acc[j]);
    }
    m = mx;
  }
  if (bad_slot && lane == 0 && err_count) atomicAdd(err_count, 1);
  if (nparts == 1) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (act) {
#pragma unroll
      for (int j = 0; j < NV; ++j) o[lane + 64 * j] = st1<Tag>(acc[j] * inv);
    }
    return;
  }
  const int64_t row = (int64_t(z) * Hq + h) * num_parts + part;
  if (act) {
#pragma unroll
    for (int j = 0; j < NV; ++j) ws_acc[row * D + lane + 64 * j] = acc[j];
  }
  if (lane == 0) {
    ws_ml[2 * row] = m;
    ws_ml[2 * row + 1] = l;
  }
}

// Merge of a row's partitions: one wave per (row slot, head); lane d folds dims d, d+64, ...
template <typename Tag, int D>
__global__ __launch_bounds__(64) void generic_merge_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ ctx_lens, int32_t max_ctx,
    int32_t max_q_len, int32_t P, int32_t num_parts, typename Tag::store* __restrict__ out,
    int64_t ost, int64_t osh) {
  constexpr int NV = D > 64 ? D / 64 : 1;
  const int z = blockIdx.x, h = blockIdx.y, Hq = gridDim.y;
  const int lane = threadIdx.x;
  const RowInfo r = row_info(cu_q, ctx_lens, max_q_len, max_ctx, z);
  if (!r.live || r.vis <= P) return;  // one partition at most: written by the attention kernel
  const int nparts = (r.vis + P - 1) / P;
  const int64_t row0 = (int64_t(z) * Hq + h) * num_parts;
  const bool act = lane < D;
  float M = -INFINITY, L = 0.f, A[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) A[j] = 0.f;
  for (int p0 = 0; p0 < nparts; p0 += kMergeBatch) {
    const int n = min(nparts - p0, kMergeBatch);
    float vm[kMergeBatch], vl[kMergeBatch], va[kMergeBatch][NV];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const int64_t rr = row0 + p0 + (u < n ? u : 0);
      vm[u] = u < n ? ws_ml[2 * rr] : -INFINITY;
      vl[u] = u < n ? ws_ml[2 * rr + 1] : 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j)
        va[u][j] = (u < n && act) ? ws_acc[rr * D + lane + 64 * j] : 0.f;
    }
    float bm = M;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) bm = fmaxf(bm, vm[u]);
    const float bmu = bm == -INFINITY ? 0.f : bm;
    const float keep = dsp_exp2(M - bmu);
    L *= keep;
#pragma unroll
    for (int j = 0; j < NV; ++j) A[j] *= keep;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const float w = dsp_exp2(vm[u] - bmu);
      L = fmaf(vl[u], w, L);
#pragma unroll
      for (int j = 0; j < NV; ++j) A[j] = fmaf(va[u][j], w, A[j]);
    }
    M = bm;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (act) {
    typename Tag::store* o = out + r.tok * ost + int64_t(h) * osh;
#pragma unroll
    for (int j = 0; j < NV; ++j) o[lane + 64 * j] = st1<Tag>(A[j] * inv);
  }
}

struct GenericArgs {
  const void* q;
  int64_t qst, qsh;
  const void* kc;
  const void* vc;
  int64_t num_slots, kvs_slot, kvs_head;
  const int32_t* table;
  int64_t table_stride;
  int32_t log2_bs;
  const int32_t* cu_q;
  const int32_t* ctx_lens;
  int32_t G, max_ctx, max_q_len;
  float scale_log2;
  int32_t P, num_parts;
  float* ws_acc;
  float* ws_ml;
  void* out;
  int64_t ost, osh;
  int32_t* err_count;
};

template <typename Tag, int D>
int launch_generic_d(const GenericArgs& a, dim3 grid, dim3 mgrid, hipStream_t s) {
  using S = typename Tag::store;
  generic_attn_kernel<Tag, D><<<grid, 64, 0, s>>>(
      static_cast<const S*>(a.q), a.qst, a.qsh, static_cast<const S*>(a.kc),
      static_cast<const S*>(a.vc), a.num_slots, a.kvs_slot, a.kvs_head, a.table, a.table_stride,
      a.log2_bs, a.cu_q, a.ctx_lens, a.G, a.max_ctx, a.max_q_len, a.scale_log2, a.P,
      a.num_parts, a.ws_acc, a.ws_ml, static_cast<S*>(a.out), a.ost, a.osh, a.err_count);
  const int st = dsp_launch_status();
  if (st != DSP_OK || a.num_parts <= 1) return st;
  generic_merge_kernel<Tag, D><<<mgrid, 64, 0, s>>>(a.ws_acc, a.ws_ml, a.cu_q, a.ctx_lens,
                                                    a.max_ctx, a.max_q_len, a.P, a.num_parts,
                                                    static_cast<S*>(a.out), a.ost, a.osh);
  return dsp_launch_status();
}

template <typename Tag>
int launch_generic(int D, const GenericArgs& a, dim3 grid, dim3 mgrid, hipStream_t s) {
  switch (D) {
    case 8: return launch_generic_d<Tag, 8>(a, grid, mgrid, s);
    case 16: return launch_generic_d<Tag, 16>(a, grid, mgrid, s);
    case 32: return launch_generic_d<Tag, 32>(a, grid, mgrid, s);
    case 64: return launch_generic_d<Tag, 64>(a, grid, mgrid, s);
    case 128: return launch_generic_d<Tag, 128>(a, grid, mgrid, s);
    case 256: return launch_generic_d<Tag, 256>(a, grid, mgrid, s);
    default: return DSP_EUNSUPPORTED;
  }
}

}  // namespace

namespace dsp_detail {

bool generic_head_dim(int32_t D) {
  return D == 8 || D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

size_t generic_workspace_bytes(int32_t B, int32_t Hq, int32_t D, int32_t max_q_len,
                               int32_t max_ctx, int32_t P) {
  if (B <= 0 || Hq <= 0 || max_q_len <= 0 || max_ctx <= 0 || P <= 0) return 0;
  const int64_t np = (int64_t(max_ctx) + P - 1) / P;
  if (np <= 1) return 0;
  return size_t(B) * max_q_len * Hq * np * (size_t(D) + 2) * sizeof(float);
}

int generic_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                      const void* v_cache, int64_t num_slots, int64_t kv_stride_slot,
                      int64_t kv_stride_head, const int32_t* table, int64_t table_stride,
                      int32_t log2_bs, const int32_t* cu_q, const int32_t* ctx_lens, int32_t B,
                      int32_t Hq, int32_t KVH, int32_t D, float scale, int32_t max_q_len,
                      int32_t max_ctx, int32_t P, void* workspace, void* out,
                      int64_t o_stride_t, int64_t o_stride_h, int32_t dtype, int32_t* err_count,
                      hipStream_t s) {
  if (B == 0 || max_q_len == 0) return DSP_OK;
  const int32_t num_parts = max_ctx > 0 ? (max_ctx + P - 1) / P : 1;
  const int64_t rows = int64_t(B) * max_q_len;
  // grid: x row slots (a sequence's rows side by side: they read the same keys), y query
  // heads, z partitions
  if (rows > (int64_t(1) << 26) || Hq > 65535 || num_parts > 65535) return DSP_EUNSUPPORTED;
  float* ws_acc = static_cast<float*>(workspace);
  GenericArgs a{q, q_stride_t, q_stride_h, k_cache, v_cache, num_slots, kv_stride_slot,
                kv_stride_head, table, table_stride, log2_bs, cu_q, ctx_lens, Hq / KVH,
                max_ctx, max_q_len, scale * 1.4426950408889634f, P, num_parts, ws_acc,
                num_parts > 1 ? ws_acc + rows * Hq * num_parts * D : nullptr, out, o_stride_t,
                o_stride_h, err_count};
  dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(Hq),
            static_cast<unsigned>(num_parts));
  dim3 mgrid(static_cast<unsigned>(rows), static_cast<unsigned>(Hq));
  switch (dtype) {
    case DSP_BF16: return launch_generic<GBf16>(D, a, grid, mgrid, s);
    case DSP_F16: return launch_generic<GF16>(D, a, grid, mgrid, s);
    case DSP_F32: return launch_generic<GF32>(D, a, grid, mgrid, s);
    default: return DSP_EUNSUPPORTED;
  }
}

}  // namespace dsp_detail
