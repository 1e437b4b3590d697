// J3: paged decode attention for gfx950 -- GQA-packed, split-K, online softmax.
//
// Semantics follow the reference Triton kernel (dispec/engine/triton_attn.py:59-95):
// one query token per sequence, query head h reads KV head h / G (:70), fp32
// accumulation with an online softmax (:86-92), masked tail (:80-85), and the output
// cast to the cache dtype (:94-95).  The structure is MI355X-specific:
//
//  * One workgroup per (partition of `P` tokens, KV head, sequence).  All G query heads
//    of the KV head are served by the same workgroup, so each K/V row is read from HBM
//    once rather than G times.
//  * A row (one token of one KV head, D elements) is loaded by D/8 consecutive lanes,
//    16 bytes each (global_load_dwordx4), so a wave moves 1 KiB per load instruction.
//    The slot of every token of the partition is resolved once into LDS first.
//  * q.k uses v_dot2_f32_{bf16,f16} on packed pairs; the D/8-lane partial sums are
//    combined with DPP adds inside a 16-lane row (no LDS round trip), which leaves every
//    lane of the row holding the full scores of the tokens it loaded -- exactly the
//    weights it needs for its slice of p.V.
//  * Softmax is tracked in base 2 (log2(e) folded into the scale, v_exp_f32).  Each
//    row group keeps its own running max; row groups, then waves, are merged with the
//    usual rescale at the end of the partition.
//  * Partitions are merged by a second small kernel (log-sum-exp combine) only when a
//    sequence spans more than one partition.
//
// dsp_paged_decode sends block-table calls with head_dim >= 32 to the multi-query MFMA
// kernel of paged_mq.hip in its decode mode (measured faster on every decode shape, most
// for GQA groups of 6+); this VALU kernel serves per-token slot tables and head_dim 16.
#include <float.h>

#include <atomic>
#include <mutex>

#include "dsp_common.h"
#include "dsp_internal.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxPartition = 1024;
constexpr int kOneRoundCtx = 512;  // automatic block-table decode: unsplit up to this context

struct Bf16Tag {};
struct F16Tag {};

template <typename Tag>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc);
template <>
__device__ __forceinline__ float dot2<Bf16Tag>(uint32_t a, uint32_t b, float acc) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b),
                                         acc, false);
}
template <>
__device__ __forceinline__ float dot2<F16Tag>(uint32_t a, uint32_t b, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), acc, false);
}

template <typename Tag>
__device__ __forceinline__ void widen2(uint32_t u, float& lo, float& hi) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value) {
    lo = dsp_bf16lo(u);
    hi = dsp_bf16hi(u);
  } else {
    lo = dsp_f16lo(u);
    hi = dsp_f16hi(u);
  }
}

template <typename Tag>
__device__ __forceinline__ uint16_t narrow(float f) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value)
    return dsp_f32_to_bf16(f);
  else
    return dsp_f32_to_f16(f);
}

// Geometry of one wave's step over the context for head_dim D.
template <int D>
struct Geo {
  static constexpr int kRowLanes = D / 8;                 // lanes per token row
  static constexpr int kRowsPerLoad = 64 / kRowLanes;     // rows one load instruction covers
  static constexpr int kTpl = kRowsPerLoad >= 16 ? 1 : 16 / kRowsPerLoad;  // rows per lane
  static constexpr int kStep = kRowsPerLoad * kTpl;       // tokens per wave step
  static constexpr int kWgStep = kStep * kWaves;          // tokens per workgroup step
};

template <typename Tag, int D, int G, bool kBlockTable>
__global__ __launch_bounds__(kThreads) void paged_decode_kernel(
    const uint16_t* __restrict__ q, int64_t qsb, int64_t qsh, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t num_slots, int64_t kvs_slot, int64_t kvs_head,
    const int32_t* __restrict__ table, int64_t table_stride, int32_t log2_bs,
    const int32_t* __restrict__ ctx_lens, int32_t max_ctx, float scale_log2, int32_t P,
    int32_t num_parts, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    uint16_t* __restrict__ out, int64_t osb, int64_t osh, int32_t* __restrict__ err_count) {
  using Gm = Geo<D>;
  constexpr int RL = Gm::kRowLanes;
  constexpr int TPL = Gm::kTpl;
  constexpr int RPL = Gm::kRowsPerLoad;
  constexpr int Hq_per = G;

  __shared__ int32_t s_slot[kMaxPartition];
  __shared__ float s_acc[kWaves][G][D];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];

  const int part = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int Hq = gridDim.y * Hq_per;
  int ctx = ctx_lens[b];
  if (ctx > max_ctx || ctx < 0) {
    if (threadIdx.x == 0 && part == 0 && kvh == 0 && err_count) atomicAdd(err_count, 1);
    ctx = ctx < 0 ? 0 : max_ctx;
  }
  const int nparts = ctx > 0 ? (ctx + P - 1) / P : 1;
  if (part >= nparts) return;
  const int start = part * P;
  const int n = min(P, ctx - start);  // tokens of this partition (<= 0 only when ctx == 0)

  // Resolve the slot of every token of the partition once.
  for (int i = threadIdx.x; i < P; i += kThreads) {
    int32_t slot = -1;
    if (i < n) {
      const int t = start + i;
      int64_t s;
      if constexpr (kBlockTable) {
        const int64_t blk = table[int64_t(b) * table_stride + (t >> log2_bs)];
        s = blk * (int64_t(1) << log2_bs) + (t & ((1 << log2_bs) - 1));
      } else {
        s = table[int64_t(b) * table_stride + t];
      }
      if (s >= 0 && s < num_slots) {
        slot = static_cast<int32_t>(s);
      } else if (err_count) {
        atomicAdd(err_count, 1);
      }
    }
    s_slot[i] = slot;
  }

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rg = lane / RL;  // row group: which row of a load this lane reads
  const int c = lane % RL;   // 16-byte chunk of the row: dims [8c, 8c+8)

  dsp_u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qv[g] = *reinterpret_cast<const dsp_u32x4*>(q + int64_t(b) * qsb + int64_t(kvh * G + g) * qsh + 8 * c);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.f;
  }
  __syncthreads();

  const int64_t head_off = int64_t(kvh) * kvs_head + 8 * c;
  for (int base = wave * Gm::kStep; base < n; base += Gm::kWgStep) {
    dsp_u32x4 kr[TPL], vr[TPL];
    bool valid[TPL];
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      const int slot = s_slot[base + i * RPL + rg];
      valid[i] = slot >= 0;
      const int64_t off = int64_t(valid[i] ? slot : 0) * kvs_slot + head_off;
      if (valid[i]) {
        kr[i] = *reinterpret_cast<const dsp_u32x4*>(kc + off);
        vr[i] = *reinterpret_cast<const dsp_u32x4*>(vc + off);
      } else {
        kr[i] = dsp_u32x4{0u, 0u, 0u, 0u};
        vr[i] = dsp_u32x4{0u, 0u, 0u, 0u};
      }
    }
    float s[TPL][G];
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float p = dot2<Tag>(qv[g].x, kr[i].x, 0.f);
        p = dot2<Tag>(qv[g].y, kr[i].y, p);
        p = dot2<Tag>(qv[g].z, kr[i].z, p);
        p = dot2<Tag>(qv[g].w, kr[i].w, p);
        p = dsp_group_sum<RL>(p);
        s[i][g] = valid[i] ? p * scale_log2 : -INFINITY;
      }
    }
    float vf[TPL][8];
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      widen2<Tag>(vr[i].x, vf[i][0], vf[i][1]);
      widen2<Tag>(vr[i].y, vf[i][2], vf[i][3]);
      widen2<Tag>(vr[i].z, vf[i][4], vf[i][5]);
      widen2<Tag>(vr[i].w, vf[i][6], vf[i][7]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = s[0][g];
#pragma unroll
      for (int i = 1; i < TPL; ++i) mx = fmaxf(mx, s[i][g]);
      const float m_new = fmaxf(m[g], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = dsp_exp2(m[g] - m_use);
      float lsum = 0.f;
      float pv[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) pv[d] = acc[g][d] * alpha;
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        const float p = dsp_exp2(s[i][g] - m_use);
        lsum += p;
#pragma unroll
        for (int d = 0; d < 8; ++d) pv[d] = fmaf(p, vf[i][d], pv[d]);
      }
      l[g] = l[g] * alpha + lsum;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[g][d] = pv[d];
      m[g] = m_new;
    }
  }

  // Merge the row groups of this wave (lanes that differ in the bits above log2(RL)).
#pragma unroll
  for (int mask = RL; mask < 64; mask <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = dsp_shfl_xor(m[g], mask);
      const float lo = dsp_shfl_xor(l[g], mask);
      const float M = fmaxf(m[g], mo);
      const float Mu = M == -INFINITY ? 0.f : M;
      const float a = dsp_exp2(m[g] - Mu), bb = dsp_exp2(mo - Mu);
      l[g] = l[g] * a + lo * bb;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const float ao = dsp_shfl_xor(acc[g][d], mask);
        acc[g][d] = acc[g][d] * a + ao * bb;
      }
      m[g] = M;
    }
  }
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int d = 0; d < 8; ++d) s_acc[wave][g][8 * c + d] = acc[g][d];
      if (c == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  const bool single = nparts == 1;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int g = idx / D, d = idx % D;
    float M = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][g]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = dsp_exp2(s_m[w][g] - Mu);
      L = fmaf(s_l[w][g], e, L);
      A = fmaf(s_acc[w][g][d], e, A);
    }
    const int h = kvh * G + g;
    if (single) {
      out[int64_t(b) * osb + int64_t(h) * osh + d] = narrow<Tag>(L > 0.f ? A / L : 0.f);
    } else {
      const int64_t row = (int64_t(b) * Hq + h) * num_parts + part;
      ws_acc[row * D + d] = A;
      if (d == 0) {
        ws_ml[2 * row] = M;
        ws_ml[2 * row + 1] = L;
      }
    }
  }
}

// Log-sum-exp merge of the partitions of each (sequence, query head).
// One wave per (sequence, head), four heads per workgroup: grid = (ceil(Hq/4), B).  A lane
// holds 4 dims of the output row (D/4 lanes per row), so the wave's 64/(D/4) lane groups
// take interleaved partitions; each lane loads the (max, sum) pairs and accumulator
// elements of 16 partitions before folding them in with a running maximum -- the first 16
// together with the sequence's length, before it is known how many partitions there are
// (all lie inside the workspace; those past the count are discarded by a select) -- and
// the lane groups' results are merged by shuffles at the end.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename Tag, int D>
__global__ __launch_bounds__(256) void decode_combine_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ ctx_lens, int32_t max_ctx, int32_t P, int32_t num_parts,
    int32_t Hq, uint16_t* __restrict__ out, int64_t osb, int64_t osh) {
  constexpr int TPR = D / 4;        // lanes per output row
  constexpr int S = 64 / TPR;       // lane groups: partitions folded side by side
  constexpr int kBatch = 16;        // partitions in flight per lane
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = blockIdx.x * 4 + wave, b = blockIdx.y;
  if (h >= Hq) return;
  const int grp = lane / TPR, d = 4 * (lane % TPR);
  const int64_t row0 = (int64_t(b) * Hq + h) * num_parts;
  const float* src = ws_acc + row0 * D + d;
  const float* mlp = ws_ml + 2 * row0;
  f32x4 va[kBatch];
  float vm[kBatch], vl[kBatch];
  auto load = [&](int p0, int n) {  // partitions p0 + grp + S*u, u < kBatch, below n
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int p = p0 + grp + S * u;
      if (p < n) {
        va[u] = *reinterpret_cast<const f32x4*>(src + int64_t(p) * D);
        vm[u] = mlp[2 * p];
        vl[u] = mlp[2 * p + 1];
      }
    }
  };
  load(0, min(num_parts, S * kBatch));
  int ctx = ctx_lens[b];
  ctx = ctx < 0 ? 0 : (ctx > max_ctx ? max_ctx : ctx);
  const int nparts = ctx > 0 ? (ctx + P - 1) / P : 1;
  if (nparts <= 1) return;  // written directly by the partition kernel
  float M = -INFINITY, L = 0.f;
  f32x4 A = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int p0 = 0; p0 < nparts; p0 += S * kBatch) {
    if (p0 > 0) load(p0, nparts);
    float bm = M;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) bm = p0 + grp + S * u < nparts ? fmaxf(bm, vm[u]) : bm;
    const float Mu = bm == -INFINITY ? 0.f : bm;
    const float keep = dsp_exp2(M - Mu);  // 0 while nothing has been folded (M = -inf)
    L *= keep;
    A *= keep;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const bool in = p0 + grp + S * u < nparts;
      const float w = in ? dsp_exp2(vm[u] - Mu) : 0.f;
      L = fmaf(in ? vl[u] : 0.f, w, L);
#pragma unroll
      for (int e = 0; e < 4; ++e) A[e] = fmaf(in ? va[u][e] : 0.f, w, A[e]);
    }
    M = bm;
  }
  // merge the lane groups: group g's lane i meets group g ^ m's lane i
#pragma unroll
  for (int m = TPR; m < 64; m <<= 1) {
    const float Mo = dsp_shfl_xor(M, m), Lo = dsp_shfl_xor(L, m);
    const float Mn = fmaxf(M, Mo);
    const float Mu = Mn == -INFINITY ? 0.f : Mn;
    const float ws = dsp_exp2(M - Mu), wo = dsp_exp2(Mo - Mu);
    L = fmaf(L, ws, Lo * wo);
#pragma unroll
    for (int e = 0; e < 4; ++e) A[e] = fmaf(A[e], ws, dsp_shfl_xor(A[e], m) * wo);
    M = Mn;
  }
  if (grp == 0) {
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint16_t* o = out + int64_t(b) * osb + int64_t(h) * osh + d;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = narrow<Tag>(A[e] * inv);
  }
}

template <typename Tag>
void launch_combine(int D, dim3 grid, hipStream_t s, const float* ws_acc, const float* ws_ml,
                    const int32_t* ctx_lens, int32_t max_ctx, int32_t P, int32_t num_parts,
                    int32_t Hq, uint16_t* out, int64_t osb, int64_t osh) {
  switch (D) {
    case 16: decode_combine_kernel<Tag, 16><<<grid, 256, 0, s>>>(ws_acc, ws_ml, ctx_lens, max_ctx, P, num_parts, Hq, out, osb, osh); break;
    case 32: decode_combine_kernel<Tag, 32><<<grid, 256, 0, s>>>(ws_acc, ws_ml, ctx_lens, max_ctx, P, num_parts, Hq, out, osb, osh); break;
    case 64: decode_combine_kernel<Tag, 64><<<grid, 256, 0, s>>>(ws_acc, ws_ml, ctx_lens, max_ctx, P, num_parts, Hq, out, osb, osh); break;
    default: decode_combine_kernel<Tag, 128><<<grid, 256, 0, s>>>(ws_acc, ws_ml, ctx_lens, max_ctx, P, num_parts, Hq, out, osb, osh); break;
  }
}

int wg_step_for(int D) {
  switch (D) {
    case 16: return Geo<16>::kWgStep;
    case 32: return Geo<32>::kWgStep;
    case 64: return Geo<64>::kWgStep;
    case 128: return Geo<128>::kWgStep;
    default: return 0;
  }
}

template <typename Tag, int D, int G>
int launch_decode_dg(bool block_mode, dim3 grid, hipStream_t s, const uint16_t* q, int64_t qsb,
                     int64_t qsh, const uint16_t* kc, const uint16_t* vc, int64_t num_slots,
                     int64_t kvs_slot, int64_t kvs_head, const int32_t* table,
                     int64_t table_stride, int32_t log2_bs, const int32_t* ctx_lens,
                     int32_t max_ctx, float scale_log2, int32_t P, int32_t num_parts,
                     float* ws_acc, float* ws_ml, uint16_t* out, int64_t osb, int64_t osh,
                     int32_t* err) {
  if (block_mode)
    paged_decode_kernel<Tag, D, G, true><<<grid, kThreads, 0, s>>>(
        q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head, table, table_stride, log2_bs,
        ctx_lens, max_ctx, scale_log2, P, num_parts, ws_acc, ws_ml, out, osb, osh, err);
  else
    paged_decode_kernel<Tag, D, G, false><<<grid, kThreads, 0, s>>>(
        q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head, table, table_stride, log2_bs,
        ctx_lens, max_ctx, scale_log2, P, num_parts, ws_acc, ws_ml, out, osb, osh, err);
  return dsp_launch_status();
}

template <typename Tag, int D, typename... A>
int launch_decode_d(int G, A... args) {
  switch (G) {
    case 1: return launch_decode_dg<Tag, D, 1>(args...);
    case 2: return launch_decode_dg<Tag, D, 2>(args...);
    case 3: return launch_decode_dg<Tag, D, 3>(args...);
    case 4: return launch_decode_dg<Tag, D, 4>(args...);
    case 5: return launch_decode_dg<Tag, D, 5>(args...);
    case 6: return launch_decode_dg<Tag, D, 6>(args...);
    case 7: return launch_decode_dg<Tag, D, 7>(args...);
    case 8: return launch_decode_dg<Tag, D, 8>(args...);
    default: return DSP_EUNSUPPORTED;
  }
}

template <typename Tag, typename... A>
int launch_decode(int D, int G, A... args) {
  switch (D) {
    case 16: return launch_decode_d<Tag, 16>(G, args...);
    case 32: return launch_decode_d<Tag, 32>(G, args...);
    case 64: return launch_decode_d<Tag, 64>(G, args...);
    case 128: return launch_decode_d<Tag, 128>(G, args...);
    default: return DSP_EUNSUPPORTED;
  }
}

}  // namespace

extern "C" int dsp_paged_decode_partition_tokens(int32_t B, int32_t KVH, int32_t D,
                                                 int32_t max_ctx) {
  const int step = wg_step_for(D);
  if (step == 0) {
    if (!dsp_detail::generic_head_dim(D)) return 0;
    // generic kernel (head dims 8 and 256): one wave per (sequence, query head, partition);
    // 1024 keys, halved while the launch would have fewer than ~1024 x G waves
    if (B <= 0 || KVH <= 0 || max_ctx <= 0) return 64;
    int P = 1024;
    while (P > 64 && int64_t(B) * KVH * ((max_ctx + P - 1) / P) < 1024) P /= 2;
    return P;
  }
  if (B <= 0 || KVH <= 0 || max_ctx <= 0) return step;
  if (D == 16) {
    // VALU kernel: largest power-of-two multiple of the workgroup step, at most 512,
    // that still gives the launch enough workgroups to fill 256 CUs several times over.
    int P = step;
    while (P * 2 <= 512) P *= 2;
    while (P > step && int64_t(B) * KVH * ((max_ctx + P - 1) / P) < 2048) P /= 2;
    return P;
  }
  // MFMA kernel (block tables, D >= 32): long partitions -- 1024 keys, halved only while
  // the launch has fewer than 512 workgroups (measured best on 16 x 32k and 64 x 0.5-4k
  // contexts; the slot-table kernel accepts the same sizes).
  int P = 1024;
  while (P > 128 && int64_t(B) * KVH * ((max_ctx + P - 1) / P) < 512) P /= 2;
  return P;
}

namespace {

size_t fixed_workspace_bytes(int32_t B, int32_t Hq, int32_t D, int32_t max_ctx, int32_t P) {
  if (P <= 0) return 0;  // no kernel for this head dim: the launch is rejected anyway
  const int64_t np = (int64_t(max_ctx) + P - 1) / P;
  if (np <= 1) return 0;
  return size_t(B) * Hq * np * (size_t(D) + 2) * sizeof(float);
}

}  // namespace

extern "C" size_t dsp_paged_decode_workspace_bytes(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                                   int32_t max_ctx, int32_t partition_tokens) {
  if (B <= 0 || Hq <= 0 || KVH <= 0 || Hq % KVH != 0 || D <= 0 || max_ctx <= 0 ||
      (partition_tokens < 0 && partition_tokens != DSP_SPLIT_BALANCED))
    return 0;
  if (partition_tokens == DSP_SPLIT_BALANCED)
    return dsp_detail::balanced_decode_applies(B, KVH, D, max_ctx, 16)
               ? dsp_detail::balanced_workspace_bytes(B, KVH, Hq / KVH, D, max_ctx)
               : 0;
  if (partition_tokens > 0) return fixed_workspace_bytes(B, Hq, D, max_ctx, partition_tokens);
  // automatic: enough for whichever split the launch picks (balanced on block tables,
  // fixed partitions on slot tables)
  size_t need = fixed_workspace_bytes(B, Hq, D, max_ctx,
                                      dsp_paged_decode_partition_tokens(B, KVH, D, max_ctx));
  // (block size unknown here: size for the balanced split whenever it could apply)
  if (dsp_detail::balanced_decode_applies(B, KVH, D, max_ctx, 16)) {
    const size_t bal = dsp_detail::balanced_workspace_bytes(B, KVH, Hq / KVH, D, max_ctx);
    if (bal > need) need = bal;
  }
  return need;
}

extern "C" int dsp_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_cache, const void* v_cache, int64_t num_slots,
                                int64_t kv_stride_slot, int64_t kv_stride_head,
                                const int32_t* block_table, int64_t bt_stride,
                                int32_t block_size, const int32_t* slot_table,
                                int64_t st_stride, const int32_t* ctx_lens, int32_t B,
                                int32_t Hq, int32_t KVH, int32_t D, float scale,
                                int32_t max_ctx, int32_t partition_tokens, void* workspace,
                                size_t workspace_bytes, void* out, int64_t o_stride_b,
                                int64_t o_stride_h, int32_t dtype, int32_t* err_count,
                                dsp_stream_t stream) {
  DSP_HOST_CHECK(q && k_cache && v_cache && ctx_lens && out, DSP_EINVAL);
  DSP_HOST_CHECK((block_table != nullptr) != (slot_table != nullptr), DSP_EINVAL);
  DSP_HOST_CHECK(B >= 0 && Hq > 0 && KVH > 0 && Hq % KVH == 0 && max_ctx >= 0 && num_slots >= 0,
                 DSP_EINVAL);
  DSP_HOST_CHECK(B <= 65535 && KVH <= 65535 && num_slots < (int64_t(1) << 31), DSP_EINVAL);
  // a key whose block id is out of range reads row 0 instead: the cache must have one
  DSP_HOST_CHECK(num_slots > 0 || B == 0 || max_ctx == 0, DSP_EINVAL);
  DSP_HOST_CHECK(kv_stride_slot >= 0 && kv_stride_head >= 0, DSP_EINVAL);
  DSP_HOST_CHECK(dtype == DSP_BF16 || dtype == DSP_F16 || dtype == DSP_F32, DSP_EUNSUPPORTED);
  DSP_HOST_CHECK(partition_tokens >= 0 || partition_tokens == DSP_SPLIT_BALANCED, DSP_EINVAL);
  const int G = Hq / KVH;
  const int step = wg_step_for(D);
  if (dtype == DSP_F32 || step == 0 || G > 8) {
    DSP_HOST_CHECK(partition_tokens != DSP_SPLIT_BALANCED, DSP_EUNSUPPORTED);
    // fp32 caches, head dims outside {16, 32, 64, 128}, groups above 8: the generic kernel
    DSP_HOST_CHECK(dsp_detail::generic_head_dim(D), DSP_EUNSUPPORTED);
    if (B == 0) return DSP_OK;
    const int64_t es = dtype == DSP_F32 ? 4 : 2;
    DSP_HOST_CHECK(dsp_aligned(q, es) && dsp_aligned(k_cache, es) && dsp_aligned(v_cache, es) &&
                       dsp_aligned(out, es),
                   DSP_EALIGN);
    const int32_t* tbl = block_table ? block_table : slot_table;
    int32_t lbs = -1;
    if (block_table) {
      DSP_HOST_CHECK(dsp_is_pow2(block_size), DSP_EINVAL);
      DSP_HOST_CHECK(bt_stride * block_size >= max_ctx, DSP_EINVAL);
      lbs = dsp_log2i(block_size);
    } else {
      DSP_HOST_CHECK(st_stride >= max_ctx, DSP_EINVAL);
    }
    const int P = partition_tokens > 0 ? partition_tokens
                                       : dsp_paged_decode_partition_tokens(B, KVH, D, max_ctx);
    const size_t need = dsp_detail::generic_workspace_bytes(B, Hq, D, 1, max_ctx, P);
    DSP_HOST_CHECK(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                   DSP_EWORKSPACE);
    DSP_HOST_CHECK(need == 0 || dsp_aligned(workspace, 16), DSP_EALIGN);
    return dsp_detail::generic_attention(
        q, q_stride_b, q_stride_h, k_cache, v_cache, num_slots, kv_stride_slot, kv_stride_head,
        tbl, block_table ? bt_stride : st_stride, lbs, nullptr, ctx_lens, B, Hq, KVH, D, scale,
        1, max_ctx, P, workspace, out, o_stride_b, o_stride_h, dtype, err_count,
        static_cast<hipStream_t>(stream));
  }
  if (B == 0) return DSP_OK;
  // 16-byte vector loads of q and K/V rows.
  DSP_HOST_CHECK(q_stride_b % 8 == 0 && q_stride_h % 8 == 0 && kv_stride_slot % 8 == 0 &&
                     kv_stride_head % 8 == 0 && dsp_aligned(q, 16) && dsp_aligned(k_cache, 16) &&
                     dsp_aligned(v_cache, 16),
                 DSP_EALIGN);
  int32_t log2_bs = 0;
  const int32_t* table = block_table ? block_table : slot_table;
  int64_t table_stride = block_table ? bt_stride : st_stride;
  if (block_table) {
    DSP_HOST_CHECK(dsp_is_pow2(block_size), DSP_EINVAL);
    log2_bs = dsp_log2i(block_size);
    DSP_HOST_CHECK(bt_stride * block_size >= max_ctx, DSP_EINVAL);
  } else {
    DSP_HOST_CHECK(st_stride >= max_ctx, DSP_EINVAL);
  }
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* qh = static_cast<const uint16_t*>(q);
  const uint16_t* kh = static_cast<const uint16_t*>(k_cache);
  const uint16_t* vh = static_cast<const uint16_t*>(v_cache);
  uint16_t* oh = static_cast<uint16_t*>(out);
  const bool bm = block_table != nullptr;
  // Automatic split on block tables.  A small launch -- contexts of at most kOneRoundCtx
  // keys and one MFMA workgroup per (sequence, KV head) for at most two per CU -- runs
  // unsplit on the multi-query kernel: one launch, no combine (config 1, a draft model's
  // decode: 7.8 against 11.9 us on the balanced split and its combine, graph-captured).
  // Otherwise the balanced split where it applies.
  const bool one_round = bm && partition_tokens == 0 && D >= 32 && max_ctx > 0 &&
                         max_ctx <= kOneRoundCtx &&
                         int64_t(B) * KVH <= 2 * int64_t(dsp_detail::device_cus());
  if (partition_tokens == DSP_SPLIT_BALANCED) {
    DSP_HOST_CHECK(bm && dsp_detail::balanced_decode_applies(B, KVH, D, max_ctx, block_size),
                   DSP_EUNSUPPORTED);
  }
  if (bm && (partition_tokens == DSP_SPLIT_BALANCED || (partition_tokens == 0 && !one_round)) &&
      dsp_detail::balanced_decode_applies(B, KVH, D, max_ctx, block_size)) {
    // block tables, automatic split: every wave takes an equal share of the keys
    const size_t need = dsp_detail::balanced_workspace_bytes(B, KVH, G, D, max_ctx);
    DSP_HOST_CHECK(workspace_bytes >= need && workspace != nullptr, DSP_EWORKSPACE);
    DSP_HOST_CHECK(dsp_aligned(workspace, 16), DSP_EALIGN);
    return dsp_detail::balanced_decode(qh, q_stride_b, q_stride_h, kh, vh, num_slots,
                                       kv_stride_slot, kv_stride_head, table, table_stride,
                                       log2_bs, ctx_lens, nullptr, 1, B, KVH, G, D,
                                       scale_log2, max_ctx, static_cast<float*>(workspace), oh,
                                       o_stride_b,
                                       o_stride_h, dtype == DSP_F16, err_count, s);
  }
  int P = partition_tokens > 0 ? partition_tokens
          : one_round          ? (max_ctx + 127) / 128 * 128
                               : dsp_paged_decode_partition_tokens(B, KVH, D, max_ctx);
  DSP_HOST_CHECK(P % step == 0 && P <= kMaxPartition, DSP_EINVAL);
  const int num_parts = max_ctx > 0 ? (max_ctx + P - 1) / P : 1;
  const size_t need = fixed_workspace_bytes(B, Hq, D, max_ctx, P);
  DSP_HOST_CHECK(workspace_bytes >= need && (need == 0 || workspace != nullptr), DSP_EWORKSPACE);
  DSP_HOST_CHECK(need == 0 || dsp_aligned(workspace, 16), DSP_EALIGN);
  float* ws_acc = static_cast<float*>(workspace);
  float* ws_ml = need ? ws_acc + int64_t(B) * Hq * num_parts * D : nullptr;
  dim3 grid(static_cast<unsigned>(num_parts), static_cast<unsigned>(KVH), static_cast<unsigned>(B));
  int st;
  if (bm && D >= 32) {
    // block tables: the MFMA kernel (its decode mode writes this function's workspace layout)
    st = dsp_detail::mq_decode(qh, q_stride_b, q_stride_h, kh, vh, num_slots, kv_stride_slot,
                               kv_stride_head, table, table_stride, log2_bs, ctx_lens, B, KVH, G,
                               D, scale_log2, max_ctx, P, num_parts, ws_acc, ws_ml, oh, o_stride_b,
                               o_stride_h, dtype == DSP_F16, err_count, s);
  } else if (dtype == DSP_BF16)
    st = launch_decode<Bf16Tag>(D, G, bm, grid, s, qh, q_stride_b, q_stride_h, kh, vh, num_slots,
                                kv_stride_slot, kv_stride_head, table, table_stride, log2_bs,
                                ctx_lens, max_ctx, scale_log2, P, num_parts, ws_acc, ws_ml, oh,
                                o_stride_b, o_stride_h, err_count);
  else
    st = launch_decode<F16Tag>(D, G, bm, grid, s, qh, q_stride_b, q_stride_h, kh, vh, num_slots,
                               kv_stride_slot, kv_stride_head, table, table_stride, log2_bs,
                               ctx_lens, max_ctx, scale_log2, P, num_parts, ws_acc, ws_ml, oh,
                               o_stride_b, o_stride_h, err_count);
  if (st != DSP_OK || num_parts <= 1) return st;
  dim3 cgrid(static_cast<unsigned>((Hq + 3) / 4), static_cast<unsigned>(B));
  if (dtype == DSP_BF16)
    launch_combine<Bf16Tag>(D, cgrid, s, ws_acc, ws_ml, ctx_lens, max_ctx, P, num_parts, Hq, oh,
                            o_stride_b, o_stride_h);
  else
    launch_combine<F16Tag>(D, cgrid, s, ws_acc, ws_ml, ctx_lens, max_ctx, P, num_parts, Hq, oh,
                           o_stride_b, o_stride_h);
  return dsp_launch_status();
}

// ------------------------------------------------------------------ no-allocation variant
// dsp_paged_decode with its split-K workspace in a file-scope device array instead of a
// caller buffer, for callers that cannot allocate (graph capture, serving loops).  In host
// code `scratch` names a host-side stand-in, not device memory: its device address is
// fetched once per device with hipGetSymbolAddress (with that device current) and only
// that address is ever passed to a kernel.  The decode kernels write every workspace word
// they later read, so nothing has to be cleared between calls.
namespace {

__device__ __align__(256) unsigned char scratch[DSP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];

// The current device's copy of `scratch` (status 0).  The address is looked up on the
// first call per device and kept only once the lookup succeeds, so a failed lookup (a
// transient runtime error) is tried again on the next call instead of being returned for
// the life of the process.
int scratch_for_current_device(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return DSP_EUNSUPPORTED;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (r != hipSuccess) return static_cast<int>(r);
      if (p == nullptr) return DSP_EINVAL;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return DSP_OK;
}

}  // namespace

extern "C" int dsp_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                        const void* k_cache, const void* v_cache,
                                        int64_t num_slots, int64_t kv_stride_slot,
                                        int64_t kv_stride_head, const int32_t* block_table,
                                        int64_t bt_stride, int32_t block_size,
                                        const int32_t* slot_table, int64_t st_stride,
                                        const int32_t* ctx_lens, int32_t B, int32_t Hq,
                                        int32_t KVH, int32_t D, float scale, int32_t max_ctx,
                                        int32_t partition_tokens, void* out, int64_t o_stride_b,
                                        int64_t o_stride_h, int32_t dtype, int32_t* err_count,
                                        dsp_stream_t stream) {
  // the launch's workspace must fit the fixed scratch; checked before any device work
  const size_t need = dsp_paged_decode_workspace_bytes(B, Hq, KVH, D, max_ctx, partition_tokens);
  DSP_HOST_CHECK(need <= DSP_NOALLOC_SCRATCH_BYTES, DSP_ESCRATCH);
  void* ws = nullptr;
  const int st = scratch_for_current_device(&ws);
  if (st != DSP_OK) return st;
  return dsp_paged_decode(q, q_stride_b, q_stride_h, k_cache, v_cache, num_slots,
                          kv_stride_slot, kv_stride_head, block_table, bt_stride, block_size,
                          slot_table, st_stride, ctx_lens, B, Hq, KVH, D, scale, max_ctx,
                          partition_tokens, ws, DSP_NOALLOC_SCRATCH_BYTES, out, o_stride_b,
                          o_stride_h, dtype, err_count, stream);
}
