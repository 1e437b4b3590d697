// J4: multi-query paged attention (speculative verify, chunked prefill) on MFMA.
//
// Semantics: ModelRunner._attention's native branch (dispec/engine/model_runner.py:
// 160-185) -- for each sequence, SDPA over its paged context with
// causal_lower_right(q_len, ctx_len) and GQA: query i of a sequence sits at position
// ctx - q_len + i and sees keys j <= ctx - q_len + i; query head h reads KV head h / G.
//
// Layout on gfx950 (64-wide waves, v_mfma_f32_16x16x32_{bf16,f16}):
//  * A workgroup owns one tile of 16 "packed rows" of one (sequence, KV head); packed
//    row r is query r / G of query head kvh*G + r % G, so all G heads that share the KV
//    head ride in the same MFMA tile and every K/V row is loaded once for all of them.
//  * The 4 waves split the causal key range in 32-key chunks; their softmax states are
//    merged through LDS at the end.
//  * Scores are formed transposed, S^T = K . Q^T (keys on M, packed rows on N).  K goes
//    straight from HBM into the A operand (lane l: key l%16, 8 dims); Q^T is loaded once.
//    In the 16x16 output layout lane l holds keys 4*(l/16)+j of row l%16, which is
//    exactly the B operand of O^T = V^T . P^T for a 32-key step -- P never leaves
//    registers.  Only V needs a transpose: each wave stages its 32-key V chunk in LDS
//    (row pitch padded by 16 bytes so the transposed 2-byte reads are conflict-free).
//  * Softmax is online per packed row in base 2; the row max is combined across the 4
//    lane groups with two cross-lane exchanges.
#include <float.h>
#include <stdint.h>

#include "dsp_common.h"
#include "dsp_internal.h"
#include "dsp_mfma.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxParts = 64;  // key partitions per tile the merge kernel accepts
constexpr int kWinKeys = 1024; // keys per block-table window staged in LDS (8 rounds)

using namespace dsp_mfma;

// kDecode: one query per sequence (row b of q), no cu_q; the decode entry point's
// semantics for bad lengths (a context past max_ctx is clamped and counted, an empty one
// gives zeros) and its workspace layout ws[(b * Hq + h) * num_parts + part], which its
// combine kernel merges.
template <typename Tag, int D, bool kDecode>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void paged_mq_kernel(
    const uint16_t* __restrict__ q, int64_t qst, int64_t qsh, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t num_slots, int64_t kvs_slot, int64_t kvs_head,
    const int32_t* __restrict__ bt, int64_t bt_stride, int32_t log2_bs,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ ctx_lens, int32_t max_ctx,
    int32_t G, float scale_log2, int32_t P, int32_t num_parts, int32_t tiles_max,
    float* __restrict__ ws_acc, float* __restrict__ ws_ml, uint16_t* __restrict__ out,
    int64_t ost, int64_t osh, int32_t* __restrict__ err_count) {
  constexpr int NKK = D / 32;        // 32-dim K steps of the score MFMA
  constexpr int NT = D / 16;         // 16-dim output tiles
  constexpr int CPR = D / 8;         // 16-byte chunks per K/V row
  constexpr int ROWB = 2 * D;         // bytes of one K/V row
  constexpr int SLAB = 32 * ROWB;      // one wave's staged V chunk (32 rows)
  constexpr int VINS = SLAB / 1024;    // 1-KiB DMA loads per V chunk
  constexpr int RPI = 1024 / ROWB;     // V rows per DMA load

  // The V slabs are dead once the key loop ends; the cross-wave merge reuses their bytes.
  constexpr int kSlabBytes = kWaves * SLAB, kAccBytes = kWaves * 16 * (D + 1) * 4;
  __shared__ __attribute__((aligned(1024))) char s_raw[kSlabBytes > kAccBytes ? kSlabBytes : kAccBytes];
  __shared__ float s_m[kWaves][16];
  __shared__ float s_l[kWaves][16];
  __shared__ int32_t s_blk[kWinKeys + 1];  // block ids of the current key window
  auto s_acc = reinterpret_cast<float (*)[16][D + 1]>(s_raw);
  char* const slab_base = s_raw;

  const int part = blockIdx.x % num_parts, tile = blockIdx.x / num_parts;
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int KVH = gridDim.y;
  const int q0 = kDecode ? b : cu_q[b];
  const int qlen = kDecode ? 1 : cu_q[b + 1] - q0;
  int ctx = ctx_lens[b];
  const int rows = qlen * G;
  const int r0 = tile * 16;
  if (qlen <= 0 || r0 >= rows) return;
  bool bad = false;
  if (kDecode) {
    if (ctx > max_ctx || ctx < 0) {
      if (threadIdx.x == 0 && part == 0 && kvh == 0 && err_count) atomicAdd(err_count, 1);
      ctx = ctx < 0 ? 0 : max_ctx;
    }
  } else if (ctx > max_ctx || ctx < qlen) {
    bad = true;
    if (threadIdx.x == 0 && tile == 0 && part == 0 && kvh == 0 && err_count) atomicAdd(err_count, 1);
    ctx = 0;  // no keys: rows are written as zeros
  }

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15;   // packed row within the tile (N index)
  const int grp = lane >> 4; // lane group: K sub-range of the MFMA operands
  const int r = r0 + n;
  const bool row_ok = r < rows && !bad;
  const int qi = row_ok ? r / G : 0;
  const int h = kvh * G + (row_ok ? r % G : 0);
  const int pos_q = ctx - qlen + qi;  // keys 0..pos_q are visible to this row
  const int r_last = min(r0 + 15, rows - 1);
  const int kend = bad ? 0 : ctx - qlen + r_last / G + 1;  // keys any row of the tile sees
  // Split-K: this workgroup covers keys [kbeg, kfin) of the tile's causal range.
  const int nparts = kend > 0 ? (kend + P - 1) / P : 1;
  if (part >= nparts) return;
  const int kbeg = part * P;
  const int kfin = min(kbeg + P, kend);
  const int64_t bt_row = int64_t(b) * bt_stride;
  const int64_t head_off = int64_t(kvh) * kvs_head;

  dsp_u32x4 qop[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    qop[kk] = row_ok ? *reinterpret_cast<const dsp_u32x4*>(q + int64_t(q0 + qi) * qst + int64_t(h) * qsh +
                                                       32 * kk + 8 * grp)
                     : dsp_u32x4{0u, 0u, 0u, 0u};
  }

  float m = -INFINITY, lpart = 0.f;
  f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Rounds of 128 keys (32 per wave).  The block ids of each 1024-key window are staged
  // in LDS first, so a key's slot costs an LDS read rather than a dependent global load.
  const int bmask = (1 << log2_bs) - 1;
  int win_blk = 0;  // first block of the staged window
  bool any_bad = false;  // a visible key's block id put it outside the cache (skipped)
  auto slot_of = [&](int key) -> int64_t {
    const int64_t sl = int64_t(s_blk[(key >> log2_bs) - win_blk]) * (bmask + 1) + (key & bmask);
    return (sl >= 0 && sl < num_slots) ? sl : -1;
  };
  // K operands of the two 16-key halves of a 32-key chunk (lane: key t0 + 16*st + n, dims
  // 8*grp + 32*kk), zeros past kfin.  The chunk's V rows go straight into the wave's LDS
  // slab (global_load_lds_dwordx4, no registers); their 16-byte chunks are XOR-swizzled by
  // row -- chunk c of row r at slot c ^ 2*((r >> 2) & 3) -- so that the transposed 2-byte
  // reads of the 4 lane groups (rows 4 apart) hit different banks.  V rows past kfin
  // repeat the last key's row: finite data whose probabilities are exactly 0.  The V DMA is
  // non-temporal (aux 2): each (sequence, KV head, partition) reads its V rows once, and
  // caching them only evicts what other workgroups reuse (config-3 fixed-512 decode
  // 389.5 -> 357.6 us per layer on one box; nt K loads as well lose 4 % of that).
  dsp_u32x4 kop[2][NKK];
  char* const slab = slab_base + wave * SLAB;
  auto swz = [](int r, int c) { return c ^ ((2 * ((r >> 2) & 3)) & (CPR - 1)); };
  auto load_k = [&](int t0) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int key = t0 + 16 * st + n;
      const int64_t s = key < kfin ? slot_of(key) : -1;
      any_bad |= key < kfin && s < 0;
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk)
        kop[st][kk] = s >= 0 ? *reinterpret_cast<const dsp_u32x4*>(kc + s * kvs_slot + head_off +
                                                                32 * kk + 8 * grp)
                             : dsp_u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto load_v = [&](int t0) {
#pragma unroll
    for (int i = 0; i < VINS; ++i) {
      const int row = i * RPI + lane / CPR, slot = lane % CPR;
      const int64_t s = slot_of(min(t0 + row, kfin - 1));
      const uint16_t* src = vc + (s >= 0 ? s : 0) * kvs_slot + head_off + 8 * swz(row, slot);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                       (__attribute__((address_space(3))) void*)(slab + i * 1024),
                                       16, 0, 2);
    }
  };
  // Software pipeline: once a chunk's K has fed the score MFMAs and its V sits in LDS, the
  // same registers take the loads of this wave's chunk of the next round, which then
  // overlap the softmax and P.V of the current one.  (Not across a window boundary: the
  // next window's block ids are not staged yet.)
  bool pending = false;
  for (int base = kbeg; base < kfin; base += 32 * kWaves) {
    if ((base - kbeg) % kWinKeys == 0) {
      const int wend = min(base + kWinKeys, kfin);
      win_blk = base >> log2_bs;
      const int nblk = ((wend - 1) >> log2_bs) - win_blk + 1;
      __syncthreads();  // every wave is done with the previous window
      for (int i = threadIdx.x; i < nblk; i += kThreads) s_blk[i] = bt[bt_row + win_blk + i];
      __syncthreads();
    }
    const int t0 = base + wave * 32;
    if (t0 >= kfin) continue;
    const int tn = t0 + 32 * kWaves;
    const bool prefetch = tn < kfin && (base + 32 * kWaves - kbeg) % kWinKeys != 0;
    if (!pending) {
      load_v(t0);
      load_k(t0);
    }
    f32x4 sc[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      sc[st] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) sc[st] = mfma32<Tag>(kop[st][kk], qop[kk], sc[st]);
    }
    if (prefetch) load_k(tn);
    // Scale and causal mask; lane holds keys t0 + 16*st + 4*grp + j of packed row n.
    float s[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = t0 + 16 * st + 4 * grp + j;
        const bool ok = row_ok && key <= pos_q;
        s[st][j] = ok ? sc[st][j] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[st][j]);
      }
    }
    mx = fmaxf(mx, dsp_shfl_xor(mx, 16));
    mx = fmaxf(mx, dsp_shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = dsp_exp2(m - m_use);
    m = m_new;
    float psum = 0.f;
    uint16_t pb[8];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p = dsp_exp2(s[st][j] - m_use);
        psum += p;
        pb[4 * st + j] = narrow<Tag>(p);
      }
    }
    lpart = lpart * alpha + psum;
    const dsp_u32x4 pop = dsp_u32x4{pack2(pb[0], pb[1]), pack2(pb[2], pb[3]), pack2(pb[4], pb[5]),
                                 pack2(pb[6], pb[7])};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] *= alpha;

    // This chunk's V has landed in the slab: every VMEM op issued after it is the next
    // chunk's K (2 * NKK loads, when prefetching).
    if (prefetch)
      __builtin_amdgcn_s_waitcnt(dsp_waitcnt_vm<2 * NKK>());
    else
      __builtin_amdgcn_s_waitcnt(dsp_waitcnt_vm<0>());
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // V^T operand: lane needs dim 16*nt + n of keys {4*grp+u} (u<4) and {16+4*grp+u-4}.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int d = 16 * nt + n;
      uint16_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int kl = u < 4 ? 4 * grp + u : 16 + 4 * grp + (u - 4);
        v[u] = *reinterpret_cast<const uint16_t*>(slab + kl * ROWB + 16 * swz(kl, d >> 3) +
                                                  2 * (d & 7));
      }
      const dsp_u32x4 vop = dsp_u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]),
                                   pack2(v[6], v[7])};
      acc[nt] = mfma32<Tag>(vop, pop, acc[nt]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the slab's reads are done (their values fed the MFMAs): the next chunk's V may land
    if (prefetch) load_v(tn);
    pending = prefetch;
  }

  // counted once per wave that met an out-of-range block id
  if (err_count && __ballot(any_bad) && lane == 0) atomicAdd(err_count, 1);
  // Row sums: this lane's keys only so far; add the other three lane groups.
  lpart += dsp_shfl_xor(lpart, 16);
  lpart += dsp_shfl_xor(lpart, 32);
  __syncthreads();  // all waves are done with the V slabs that s_acc overlays
  if (grp == 0) {
    s_m[wave][n] = m;
    s_l[wave][n] = lpart;
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int j = 0; j < 4; ++j) s_acc[wave][n][16 * nt + 4 * grp + j] = acc[nt][j];
  __syncthreads();

  for (int idx = threadIdx.x; idx < 16 * D; idx += kThreads) {
    const int rr = idx / D, d = idx % D;
    const int row = r0 + rr;
    if (row >= rows) continue;
    float M = s_m[0][rr];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][rr]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = dsp_exp2(s_m[w][rr] - Mu);
      L = fmaf(s_l[w][rr], e, L);
      A = fmaf(s_acc[w][rr][d], e, A);
    }
    if (nparts == 1) {
      const int qrow = q0 + row / G, hh = kvh * G + row % G;
      out[int64_t(qrow) * ost + int64_t(hh) * osh + d] = narrow<Tag>(L > 0.f ? A / L : 0.f);
    } else if (kDecode) {
      const int64_t wrow = (int64_t(b) * KVH * G + kvh * G + row) * num_parts + part;
      ws_acc[wrow * D + d] = A;
      if (d == 0) {
        ws_ml[2 * wrow] = M;
        ws_ml[2 * wrow + 1] = L;
      }
    } else {
      const int64_t slot = ((int64_t(b) * KVH + kvh) * tiles_max + tile) * num_parts + part;
      ws_acc[(slot * 16 + rr) * D + d] = A;
      if (d == 0) {
        ws_ml[2 * (slot * 16 + rr)] = M;
        ws_ml[2 * (slot * 16 + rr) + 1] = L;
      }
    }
  }
}

// Merge the key partitions of one (tile, KV head, sequence).  Grid = (ceil(rows_max / R),
// KVH, B), R = mq_combine_rows(D) rows per workgroup (workgroup x takes packed rows x*R ..
// x*R + R - 1 of the sequence's 16-row tiles): one thread per (row, 4 dims) output, its
// accumulator elements one 16-byte load per partition.  rows_max = max_q_len * G bounds the
// rows any valid sequence has, so threads of rows at or past it load nothing: a tile's
// rows past it (6 of 16 for 5 queries of 2 heads, 14 for one query)
// would otherwise fetch partitions that no valid row reads (FETCH_SIZE per merge, config
// 4: verify 10.9 -> 7.0 MB, fork decode 21.7 -> 3.0 MB; fork decode step 21.0 -> 19.8 us
// per layer on one box, verify unchanged).  Every thread folds its row's
// partitions itself, 16 at a time with a running maximum, so the merge waits on one memory
// round trip: the first 16 partitions' (max, sum) pairs and its accumulator elements are
// loaded together with the sequence's lengths, before it is known how many of them the
// row has (all lie inside the workspace; those past the row's count, possibly never
// written, are discarded by a select, not weighted).
constexpr int mq_combine_rows(int D) { return 1024 / D < 16 ? 1024 / D : 16; }

template <typename Tag, int D>
__global__ __launch_bounds__(256) void mq_combine_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ ctx_lens, int32_t max_ctx,
    int32_t G, int32_t P, int32_t num_parts, int32_t tiles_max, int32_t prefix_tokens,
    int32_t rows_max, uint16_t* __restrict__ out, int64_t ost, int64_t osh) {
  constexpr int TPR = D / 4;                // threads per row
  constexpr int R = mq_combine_rows(D);     // rows per workgroup
  constexpr int kBatch = 16;                // partitions in flight per thread
  if (threadIdx.x >= R * TPR) return;       // D 32: 128 of the 256 threads
  const int tile = blockIdx.x / (16 / R), rsub = blockIdx.x % (16 / R);
  const int kvh = blockIdx.y, b = blockIdx.z, KVH = gridDim.y;
  const int rl = threadIdx.x / TPR, d = 4 * (threadIdx.x % TPR);
  const int rr = rsub * R + rl;
  // no valid sequence has a row at or past rows_max: such a thread loads nothing (a select
  // of the load count, not an early return, which would put a scalar round trip for
  // rows_max ahead of the other kernel arguments' loads)
  const bool live = tile * 16 + rr < rows_max;
  const int64_t slot0 = ((int64_t(b) * KVH + kvh) * tiles_max + tile) * num_parts;
  const float* src = ws_acc + (slot0 * 16 + rr) * D + d;
  const float* mlp = ws_ml + 2 * (slot0 * 16 + rr);
  constexpr int64_t kAccStride = int64_t(16) * D, kMlStride = 32;  // floats per partition
  f32x4 va[kBatch];
  float vm[kBatch], vl[kBatch];
  auto load = [&](int p0, int n) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (u < n) {
        va[u] = *reinterpret_cast<const f32x4*>(src + (p0 + u) * kAccStride);
        vm[u] = mlp[(p0 + u) * kMlStride];
        vl[u] = mlp[(p0 + u) * kMlStride + 1];
      }
  };
  load(0, live ? min(num_parts, kBatch) : 0);
  const int q0 = cu_q[b];
  const int qlen = cu_q[b + 1] - q0;
  const int ctx = ctx_lens[b];
  const int rows = qlen * G;
  const int r0 = tile * 16;
  if (qlen <= 0 || r0 >= rows || ctx > max_ctx || ctx < qlen || ctx - qlen < prefix_tokens)
    return;
  const int r_last = min(r0 + 15, rows - 1);
  const int kend = ctx - qlen + r_last / G + 1;
  // partitions of P keys up to the tile's last visible key (a shared-prefix launch numbers
  // its prefix and suffix partitions the same way)
  const int nparts = kend > 0 ? (kend + P - 1) / P : 1;
  const int row = r0 + rr;
  if (!live || nparts <= 1 || row >= rows) return;  // nparts 1: written by the attention kernel
  float M = -INFINITY, L = 0.f;
  f32x4 A = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int p0 = 0; p0 < nparts; p0 += kBatch) {
    const int n = min(nparts - p0, kBatch);
    if (p0 > 0) load(p0, n);
    float bm = -INFINITY;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) bm = u < n ? fmaxf(bm, vm[u]) : bm;
    const float Mn = fmaxf(M, bm);
    const float Mu = Mn == -INFINITY ? 0.f : Mn;
    const float keep = dsp_exp2(M - Mu);   // 0 while nothing has been folded (M = -inf)
    L *= keep;
    A *= keep;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float w = u < n ? dsp_exp2(vm[u] - Mu) : 0.f;
      L = fmaf(u < n ? vl[u] : 0.f, w, L);
#pragma unroll
      for (int e = 0; e < 4; ++e) A[e] = fmaf(u < n ? va[u][e] : 0.f, w, A[e]);
    }
    M = Mn;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const int qrow = q0 + row / G, hh = kvh * G + row % G;
  uint16_t* o = out + int64_t(qrow) * ost + int64_t(hh) * osh + d;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = narrow<Tag>(A[e] * inv);
}

template <typename Tag, bool kDecode = false, typename... A>
int launch_mq(int D, dim3 grid, hipStream_t s, A... args) {
  switch (D) {
    case 32: paged_mq_kernel<Tag, 32, kDecode><<<grid, kThreads, 0, s>>>(args...); break;
    case 64: paged_mq_kernel<Tag, 64, kDecode><<<grid, kThreads, 0, s>>>(args...); break;
    case 128: paged_mq_kernel<Tag, 128, kDecode><<<grid, kThreads, 0, s>>>(args...); break;
    default: return DSP_EUNSUPPORTED;
  }
  return dsp_launch_status();
}

template <typename Tag, typename... A>
int launch_mq_combine(int D, dim3 grid, hipStream_t s, A... args) {
  switch (D) {
    case 32: mq_combine_kernel<Tag, 32><<<grid, 256, 0, s>>>(args...); break;
    case 64: mq_combine_kernel<Tag, 64><<<grid, 256, 0, s>>>(args...); break;
    default: mq_combine_kernel<Tag, 128><<<grid, 256, 0, s>>>(args...); break;
  }
  return dsp_launch_status();
}

int64_t mq_tiles(int32_t max_q_len, int32_t G) { return (int64_t(max_q_len) * G + 15) / 16; }

}  // namespace

namespace dsp_detail {

// Block-table decode on the MFMA kernel (q_len 1): called by dsp_paged_decode, which has
// checked the arguments and launches its own combine over the same workspace layout.
int mq_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
              const uint16_t* v_cache, int64_t num_slots, int64_t kv_stride_slot,
              int64_t kv_stride_head, const int32_t* block_table, int64_t bt_stride,
              int32_t log2_bs, const int32_t* ctx_lens, int32_t B, int32_t KVH, int32_t G,
              int32_t D, float scale_log2, int32_t max_ctx, int32_t P, int32_t num_parts,
              float* ws_acc, float* ws_ml, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
              bool f16, int32_t* err_count, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(num_parts), static_cast<unsigned>(KVH), static_cast<unsigned>(B));
  const int32_t* no_cu = nullptr;
  if (!f16)
    return launch_mq<Bf16Tag, true>(D, grid, s, q, q_stride_b, q_stride_h, k_cache, v_cache,
                                    num_slots, kv_stride_slot, kv_stride_head, block_table,
                                    bt_stride, log2_bs, no_cu, ctx_lens, max_ctx, G, scale_log2, P,
                                    num_parts, int32_t(1), ws_acc, ws_ml, out, o_stride_b,
                                    o_stride_h, err_count);
  return launch_mq<F16Tag, true>(D, grid, s, q, q_stride_b, q_stride_h, k_cache, v_cache,
                                 num_slots, kv_stride_slot, kv_stride_head, block_table, bt_stride,
                                 log2_bs, no_cu, ctx_lens, max_ctx, G, scale_log2, P, num_parts,
                                 int32_t(1), ws_acc, ws_ml, out, o_stride_b, o_stride_h,
                                 err_count);
}

}  // namespace dsp_detail

extern "C" int dsp_paged_mq_partition_tokens(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                             int32_t max_q_len, int32_t max_ctx) {
  if (B <= 0 || KVH <= 0 || Hq % KVH != 0 || max_q_len <= 0 || max_ctx <= 0) return 128;
  const int G = Hq / KVH;
  const int64_t whole = (int64_t(max_ctx) + 127) / 128 * 128;
  // Pick the partition count n that minimises (rounds of resident workgroups) x (keys per
  // workgroup + a fixed cost) + the merge's cost per partition, in units of keys: a split
  // pays only when it fills a round of the machine that would otherwise idle.  Long query
  // blocks run on the 128-row prefill tile, two resident per CU at D 128 and four at D 64
  // (LDS and registers); short ones (verify) on 16-row tiles, three per CU.  (Verify, 32
  // sequences of ~2.3k tokens, Qwen3 heads: 62-65 us with 3 partitions, 68-71 with 7;
  // 64 sequences of 300-700 tokens: 29 us unsplit, 37-42 with 2-3 partitions.)
  const bool long_q = int64_t(max_q_len) * G >= 128;
  const int64_t base = int64_t(B) * KVH *
                       (long_q ? dsp_detail::prefill_tiles(max_q_len, G) : mq_tiles(max_q_len, G));
  const int64_t slots = (long_q ? (D <= 64 ? 4 : 2) : 3) * int64_t(dsp_detail::device_cus());
  if (base >= slots) return static_cast<int32_t>(whole);
  int64_t best_p = whole, best_cost = INT64_MAX;
  for (int n = 1; n <= kMaxParts; ++n) {
    const int64_t p = ((max_ctx + n - 1) / n + 127) / 128 * 128;
    const int64_t parts = (max_ctx + p - 1) / p;
    if (parts != n) continue;  // the same partition as a smaller n
    const int64_t rounds = (base * parts + slots - 1) / slots;
    const int64_t cost = rounds * (p + 256) + (parts > 1 ? 192 + 48 * parts : 0);
    if (cost < best_cost) best_cost = cost, best_p = p;
  }
  return static_cast<int32_t>(best_p);
}

namespace {

// Short query blocks on the balanced split-K kernel: automatic partition, no shared prefix,
// every query row of a KV head in one MFMA tile, and a shape that kernel serves.
bool balanced_verify_applies(int32_t B, int32_t Hq, int32_t KVH, int32_t D, int32_t max_q_len,
                             int32_t max_ctx, int32_t block_size) {
  return KVH > 0 && Hq % KVH == 0 && max_q_len > 0 && int64_t(max_q_len) * (Hq / KVH) <= 16 &&
         dsp_detail::balanced_decode_applies(B, KVH, D, max_ctx, block_size);
}

size_t fixed_mq_workspace_bytes(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                int32_t max_q_len, int32_t max_ctx, int32_t P) {
  const int64_t np = (int64_t(max_ctx) + P - 1) / P;
  if (np <= 1) return 0;
  return size_t(B) * KVH * mq_tiles(max_q_len, Hq / KVH) * np * 16 * (size_t(D) + 2) *
         sizeof(float);
}

}  // namespace

extern "C" size_t dsp_paged_mq_workspace_bytes(int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                                               int32_t max_q_len, int32_t max_ctx,
                                               int32_t partition_tokens) {
  if (B <= 0 || KVH <= 0 || Hq % KVH != 0 || max_q_len <= 0 || max_ctx <= 0) return 0;
  if (partition_tokens == DSP_SPLIT_BALANCED)
    return balanced_verify_applies(B, Hq, KVH, D, max_q_len, max_ctx, 16)
               ? dsp_detail::balanced_workspace_bytes(B, KVH, max_q_len * (Hq / KVH), D,
                                                      max_ctx)
               : 0;
  if (partition_tokens < 0) return 0;
  // 0: the partition the launch picks from the shape
  return fixed_mq_workspace_bytes(
      B, Hq, KVH, D, max_q_len, max_ctx,
      partition_tokens > 0 ? partition_tokens
                           : dsp_paged_mq_partition_tokens(B, Hq, KVH, D, max_q_len, max_ctx));
}

namespace {

// Both multi-query entry points.  prefix_tokens > 0: the first prefix_tokens keys are the
// same physical blocks for every sequence and every query sees them (the caller's
// precondition; a sequence with ctx - q_len < prefix_tokens is counted and zeroed); they
// are attended once for the whole batch by the prefix pass, the rest per sequence.
int mq_attention_impl(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                      const void* k_cache, const void* v_cache, int64_t num_slots,
                      int64_t kv_stride_slot, int64_t kv_stride_head, const int32_t* block_table,
                      int64_t bt_stride, int32_t block_size, const int32_t* cu_q,
                      const int32_t* ctx_lens, int32_t B, int32_t Hq, int32_t KVH, int32_t D,
                      float scale, int32_t max_q_len, int32_t max_ctx, int32_t partition_tokens,
                      void* workspace, size_t workspace_bytes, void* out, int64_t o_stride_t,
                      int64_t o_stride_h, int32_t dtype, int32_t* err_count,
                      dsp_stream_t stream, int32_t prefix_tokens) {
  DSP_HOST_CHECK(q && k_cache && v_cache && block_table && cu_q && ctx_lens && out, DSP_EINVAL);
  DSP_HOST_CHECK(B >= 0 && B <= 65535 && Hq > 0 && KVH > 0 && KVH <= 65535 && Hq % KVH == 0 &&
                     max_q_len >= 0 && max_ctx >= 0 && num_slots >= 0 && prefix_tokens >= 0,
                 DSP_EINVAL);
  DSP_HOST_CHECK(dtype == DSP_BF16 || dtype == DSP_F16 || dtype == DSP_F32, DSP_EUNSUPPORTED);
  DSP_HOST_CHECK(dsp_is_pow2(block_size), DSP_EINVAL);
  DSP_HOST_CHECK(bt_stride * block_size >= max_ctx, DSP_EINVAL);
  if (dtype == DSP_F32 || !(D == 32 || D == 64 || D == 128)) {
    // fp32 caches or head dims 8, 16, 256: the generic kernel, fixed partitions only
    DSP_HOST_CHECK(dsp_detail::generic_head_dim(D) && prefix_tokens == 0 &&
                       partition_tokens != DSP_SPLIT_BALANCED,
                   DSP_EUNSUPPORTED);
    DSP_HOST_CHECK(partition_tokens >= 0, DSP_EINVAL);
    if (B == 0 || max_q_len == 0) return DSP_OK;
    const int64_t es = dtype == DSP_F32 ? 4 : 2;
    DSP_HOST_CHECK(dsp_aligned(q, es) && dsp_aligned(k_cache, es) && dsp_aligned(v_cache, es) &&
                       dsp_aligned(out, es),
                   DSP_EALIGN);
    const int P = partition_tokens > 0
                      ? partition_tokens
                      : dsp_paged_mq_partition_tokens(B, Hq, KVH, D, max_q_len, max_ctx);
    DSP_HOST_CHECK(P > 0 && P % 128 == 0 && (max_ctx + P - 1) / P <= kMaxParts, DSP_EINVAL);
    const size_t need = dsp_detail::generic_workspace_bytes(B, Hq, D, max_q_len, max_ctx, P);
    DSP_HOST_CHECK(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                   DSP_EWORKSPACE);
    DSP_HOST_CHECK(need == 0 || dsp_aligned(workspace, 16), DSP_EALIGN);
    return dsp_detail::generic_attention(
        q, q_stride_t, q_stride_h, k_cache, v_cache, num_slots, kv_stride_slot, kv_stride_head,
        block_table, bt_stride, dsp_log2i(block_size), cu_q, ctx_lens, B, Hq, KVH, D, scale,
        max_q_len, max_ctx, P, workspace, out, o_stride_t, o_stride_h, dtype, err_count,
        static_cast<hipStream_t>(stream));
  }
  if (B == 0 || max_q_len == 0) return DSP_OK;
  DSP_HOST_CHECK(q_stride_t % 8 == 0 && q_stride_h % 8 == 0 && kv_stride_slot % 8 == 0 &&
                     kv_stride_head % 8 == 0 && dsp_aligned(q, 16) && dsp_aligned(k_cache, 16) &&
                     dsp_aligned(v_cache, 16),
                 DSP_EALIGN);
  const int G = Hq / KVH;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f16 = dtype == DSP_F16;
  if (partition_tokens == DSP_SPLIT_BALANCED) {
    // short query blocks on the balanced split: every wave takes an equal share of the keys
    DSP_HOST_CHECK(prefix_tokens == 0, DSP_EINVAL);
    DSP_HOST_CHECK(num_slots > 0 && num_slots < (int64_t(1) << 31) &&
                       balanced_verify_applies(B, Hq, KVH, D, max_q_len, max_ctx, block_size),
                   DSP_EUNSUPPORTED);
    const size_t need = dsp_detail::balanced_workspace_bytes(B, KVH, max_q_len * G, D, max_ctx);
    DSP_HOST_CHECK(workspace_bytes >= need && workspace != nullptr, DSP_EWORKSPACE);
    DSP_HOST_CHECK(dsp_aligned(workspace, 16), DSP_EALIGN);
    return dsp_detail::balanced_decode(
        static_cast<const uint16_t*>(q), q_stride_t, q_stride_h,
        static_cast<const uint16_t*>(k_cache), static_cast<const uint16_t*>(v_cache),
        num_slots, kv_stride_slot, kv_stride_head, block_table, bt_stride,
        dsp_log2i(block_size), ctx_lens, cu_q, max_q_len, B, KVH, G, D, scale_log2, max_ctx,
        static_cast<float*>(workspace), static_cast<uint16_t*>(out), o_stride_t, o_stride_h,
        f16, err_count, s);
  }
  DSP_HOST_CHECK(partition_tokens >= 0, DSP_EINVAL);
  const int64_t tiles = mq_tiles(max_q_len, G);
  int P = partition_tokens;
  if (P <= 0)
    P = prefix_tokens > 0 ? dsp_paged_mq_shared_prefix_partition_tokens(
                                B, Hq, KVH, D, max_q_len, max_ctx, prefix_tokens)
                          : dsp_paged_mq_partition_tokens(B, Hq, KVH, D, max_q_len, max_ctx);
  DSP_HOST_CHECK(P > 0 && P % 128 == 0, DSP_EINVAL);
  if (prefix_tokens > 0) {
    DSP_HOST_CHECK(prefix_tokens % P == 0 && prefix_tokens < max_ctx, DSP_EINVAL);
    DSP_HOST_CHECK(dsp_detail::shared_prefix_applies(D, block_size, B, num_slots, kv_stride_slot),
                   DSP_EUNSUPPORTED);
  }
  const int num_parts = max_ctx > 0 ? (max_ctx + P - 1) / P : 1;
  DSP_HOST_CHECK(num_parts <= kMaxParts, DSP_EINVAL);
  DSP_HOST_CHECK(tiles * num_parts < (int64_t(1) << 31) && tiles * 16 < (int64_t(1) << 31),
                 DSP_EINVAL);
  const size_t need = fixed_mq_workspace_bytes(B, Hq, KVH, D, max_q_len, max_ctx, P);
  DSP_HOST_CHECK(workspace_bytes >= need && (need == 0 || workspace != nullptr), DSP_EWORKSPACE);
  DSP_HOST_CHECK(need == 0 || dsp_aligned(workspace, 16), DSP_EALIGN);
  float* ws_acc = static_cast<float*>(workspace);
  float* ws_ml = need ? ws_acc + int64_t(B) * KVH * tiles * num_parts * 16 * D : nullptr;
  const uint16_t* qh = static_cast<const uint16_t*>(q);
  const uint16_t* kh = static_cast<const uint16_t*>(k_cache);
  const uint16_t* vh = static_cast<const uint16_t*>(v_cache);
  uint16_t* oh = static_cast<uint16_t*>(out);
  const int32_t lbs = dsp_log2i(block_size);
  const int32_t tm = static_cast<int32_t>(tiles);
  int st = DSP_OK;
  const int ws_parts = num_parts;
  if (prefix_tokens > 0) {
    // prefix and suffix tiles in one launch (the suffixes in partitions of P keys too),
    // then the merge of every row's partitions
    DSP_HOST_CHECK(dsp_detail::shared_prefix_grid(B, G, max_q_len, max_ctx, P, prefix_tokens) <
                       (int64_t(1) << 31),
                   DSP_EINVAL);
    st = dsp_detail::prefill_shared_prefix(qh, q_stride_t, q_stride_h, kh, vh, num_slots,
                                           kv_stride_slot, kv_stride_head, block_table, bt_stride,
                                           lbs, cu_q, ctx_lens, B, KVH, G, D, scale_log2,
                                           max_q_len, max_ctx, P, tm, prefix_tokens, ws_acc,
                                           ws_ml, oh, o_stride_t, o_stride_h, f16, err_count, s);
  } else if (dsp_detail::prefill_applies(D, block_size, int64_t(max_q_len) * G, num_slots,
                                         kv_stride_slot)) {
    st = dsp_detail::prefill_attention(qh, q_stride_t, q_stride_h, kh, vh, num_slots,
                                       kv_stride_slot, kv_stride_head, block_table, bt_stride, lbs,
                                       cu_q, ctx_lens, B, KVH, G, D, scale_log2, max_q_len, max_ctx,
                                       P, num_parts, tm, ws_acc, ws_ml, oh, o_stride_t, o_stride_h,
                                       f16, err_count, s);
  } else {
    dim3 grid(static_cast<unsigned>(tiles * num_parts), static_cast<unsigned>(KVH),
              static_cast<unsigned>(B));
    if (!f16)
      st = launch_mq<Bf16Tag>(D, grid, s, qh, q_stride_t, q_stride_h, kh, vh, num_slots,
                              kv_stride_slot, kv_stride_head, block_table, bt_stride, lbs, cu_q,
                              ctx_lens, max_ctx, G, scale_log2, P, num_parts, tm, ws_acc, ws_ml,
                              oh, o_stride_t, o_stride_h, err_count);
    else
      st = launch_mq<F16Tag>(D, grid, s, qh, q_stride_t, q_stride_h, kh, vh, num_slots,
                             kv_stride_slot, kv_stride_head, block_table, bt_stride, lbs, cu_q,
                             ctx_lens, max_ctx, G, scale_log2, P, num_parts, tm, ws_acc, ws_ml,
                             oh, o_stride_t, o_stride_h, err_count);
  }
  if (st != DSP_OK || ws_parts <= 1) return st;
  const int32_t rows_max = max_q_len * G;  // <= tiles * 16 < 2^31 (checked above)
  const int R = mq_combine_rows(D);
  dim3 cgrid(static_cast<unsigned>((rows_max + R - 1) / R), static_cast<unsigned>(KVH),
             static_cast<unsigned>(B));
  if (!f16)
    return launch_mq_combine<Bf16Tag>(D, cgrid, s, ws_acc, ws_ml, cu_q, ctx_lens, max_ctx, G, P,
                                      ws_parts, tm, prefix_tokens, rows_max, oh, o_stride_t,
                                      o_stride_h);
  return launch_mq_combine<F16Tag>(D, cgrid, s, ws_acc, ws_ml, cu_q, ctx_lens, max_ctx, G, P,
                                   ws_parts, tm, prefix_tokens, rows_max, oh, o_stride_t,
                                   o_stride_h);
}

}  // namespace

extern "C" int dsp_paged_mq_shared_prefix_partition_tokens(int32_t B, int32_t Hq, int32_t KVH,
                                                           int32_t D, int32_t max_q_len,
                                                           int32_t max_ctx,
                                                           int32_t prefix_tokens) {
  (void)D;
  (void)max_ctx;
  if (B <= 0 || KVH <= 0 || Hq % KVH != 0 || max_q_len <= 0 || prefix_tokens <= 0 ||
      prefix_tokens % 128 != 0)
    return 128;
  // The prefix pass runs B * max_q_len * G rows per KV head in 128-row tiles; the suffixes
  // are cut into partitions of the same length.  Split the prefix until it has a workgroup
  // for every fourth CU, in partitions that divide it: longer partitions leave the prefix
  // tiles on too few CUs, shorter ones multiply the suffix workgroups past one round of
  // resident tiles and the merge traffic (config 4, 32 forks of a 2050-token prompt, per
  // layer: 5-query verify 29.1 us at 256 keys, 27.8 at 512; decode step 24.2 at 256, 30.7
  // at 128).
  const int64_t tiles = dsp_detail::prefill_tiles(int32_t(int64_t(B) * max_q_len), Hq / KVH);
  const int64_t want = int64_t(dsp_detail::device_cus()) / 4;
  for (int p = 512; p > 128; p -= 128)
    if (prefix_tokens % p == 0 && tiles * KVH * (prefix_tokens / p) >= want) return p;
  return 128;
}

extern "C" int dsp_paged_mq_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                      const void* k_cache, const void* v_cache,
                                      int64_t num_slots, int64_t kv_stride_slot,
                                      int64_t kv_stride_head, const int32_t* block_table,
                                      int64_t bt_stride, int32_t block_size,
                                      const int32_t* cu_q, const int32_t* ctx_lens, int32_t B,
                                      int32_t Hq, int32_t KVH, int32_t D, float scale,
                                      int32_t max_q_len, int32_t max_ctx,
                                      int32_t partition_tokens, void* workspace,
                                      size_t workspace_bytes, void* out, int64_t o_stride_t,
                                      int64_t o_stride_h, int32_t dtype, int32_t* err_count,
                                      dsp_stream_t stream) {
  return mq_attention_impl(q, q_stride_t, q_stride_h, k_cache, v_cache, num_slots,
                           kv_stride_slot, kv_stride_head, block_table, bt_stride, block_size,
                           cu_q, ctx_lens, B, Hq, KVH, D, scale, max_q_len, max_ctx,
                           partition_tokens, workspace, workspace_bytes, out, o_stride_t,
                           o_stride_h, dtype, err_count, stream, 0);
}

extern "C" int dsp_paged_mq_attention_shared_prefix(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
    const void* v_cache, int64_t num_slots, int64_t kv_stride_slot, int64_t kv_stride_head,
    const int32_t* block_table, int64_t bt_stride, int32_t block_size, const int32_t* cu_q,
    const int32_t* ctx_lens, int32_t B, int32_t Hq, int32_t KVH, int32_t D, float scale,
    int32_t max_q_len, int32_t max_ctx, int32_t prefix_tokens, int32_t partition_tokens,
    void* workspace, size_t workspace_bytes, void* out, int64_t o_stride_t, int64_t o_stride_h,
    int32_t dtype, int32_t* err_count, dsp_stream_t stream) {
  DSP_HOST_CHECK(prefix_tokens > 0 && prefix_tokens % 128 == 0, DSP_EINVAL);
  return mq_attention_impl(q, q_stride_t, q_stride_h, k_cache, v_cache, num_slots,
                           kv_stride_slot, kv_stride_head, block_table, bt_stride, block_size,
                           cu_q, ctx_lens, B, Hq, KVH, D, scale, max_q_len, max_ctx,
                           partition_tokens, workspace, workspace_bytes, out, o_stride_t,
                           o_stride_h, dtype, err_count, stream, prefix_tokens);
}
