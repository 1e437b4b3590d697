// J3 on block tables: balanced split-K paged decode on MFMA.
//
// Semantics are those of dsp_paged_decode (the reference's Triton decode kernel,
// dispec/engine/triton_attn.py:59-95): one query per sequence, query head h reads KV head
// h / G (:70), fp32 online softmax (:86-92), output in the cache dtype (:94-95).
//
// Work split.  The decode work of one launch is the list of (sequence b, group of HG KV
// heads, 16-key unit) triples in sequence-major, then head-group, then key order; a
// (sequence, head group) pair is a "segment".  With C units in all and W workers -- one
// workgroup of HG waves each, at most one wave per SIMD of the GPU -- worker w takes
// units [w*C/W, (w+1)*C/W), wave i of it KV head HG*group + i of every unit.  Every wave
// therefore reads the same number of K/V bytes (to one unit) whatever the spread of context
// lengths, and all of them finish together: there is no tail of long partitions running on
// a mostly idle GPU.  C is computed on the device from ctx_lens, so the launch needs no
// host synchronisation and can be captured in a graph.
//
// A worker whose range crosses a segment boundary produces one partial result per piece
// (row max, row sum, unnormalised accumulator) per head.  Piece (s, w) -- segment s,
// worker w -- is stored at workspace slot s + w (HG heads of G rows each): along the unit
// list the pieces form a staircase in (s, w), so s + w is unique, and the workspace holds
// B*KVH/HG + W slots.  Grouping the heads (HG = 4 when KVH allows) makes the waves of a
// workgroup read the same keys' slot rows side by side: a pure read of config 3's access
// pattern runs at 6.1 TB/s with all 8 heads of a row read by one workgroup against 5.7
// TB/s for per-wave slices, and the kernel gains ~3 % (8 heads per workgroup would leave
// room for only one workgroup per CU at three waves per SIMD: slower).  A segment inside
// one worker's range is normalised and written to the output by that worker; the combine
// kernel merges the pieces of every other segment.
//
// Per 32-key chunk a wave does what the multi-query kernel of paged_mq.hip does in its
// decode mode: S^T = K . Q^T with the G query heads of the KV head packed into the 16 MFMA
// columns, K straight from HBM into the A operand, V straight into a per-wave LDS slab
// (global_load_lds_dwordx4, rows XOR-swizzled so the transposed reads are conflict-free),
// P kept in registers as the B operand of O^T = V^T . P^T, and the next chunk's K and V
// loads issued while the current chunk is still being consumed.  Block ids come from two
// 64-entry windows of the block table held one entry per lane and read as scalars
// (readlane), the second window loaded while the first is in use.
#include <float.h>

#include <atomic>

#include "dsp_common.h"
#include "dsp_internal.h"
#include "dsp_mfma.h"

namespace {

using namespace dsp_mfma;

constexpr int kLog2Unit = 4;   // 16 keys per work unit
constexpr int kOcc = 3;        // waves per SIMD the kernel is compiled for
constexpr int kMinUnits = 4;   // a worker gets at least this many units (64 keys)
constexpr int kMaxBatch = 512; // every wave scans ctx_lens: the balanced split stops here

__device__ __forceinline__ int units_of(int ctx, int max_ctx) {
  ctx = ctx < 0 ? 0 : (ctx > max_ctx ? max_ctx : ctx);
  return (ctx + (1 << kLog2Unit) - 1) >> kLog2Unit;
}

__device__ __forceinline__ int clamp_ctx(int ctx, int max_ctx) {
  return ctx < 0 ? 0 : (ctx > max_ctx ? max_ctx : ctx);
}

// Inclusive prefix sum over the 64 lanes of the wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = __lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d);
    if (lane >= d) v += o;
  }
  return v;
}

// Sum over the 64 lanes, returned as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return __builtin_amdgcn_readfirstlane(v);
}

// Work units of sequence b.  Decode (cu_q null): its clamped context.  Multi-query: none
// for an empty query block, a query block longer than max_q_len (its rows would not fit
// the workspace's max_q_len * G rows per head) or a context outside [q_len, max_ctx] (the
// merge kernel writes such a sequence's rows below max_q_len as zeros and counts it), else
// its context.
__device__ __forceinline__ bool mq_bad(int ql, int ctx, int max_q_len, int max_ctx) {
  return ql > max_q_len || ctx < ql || ctx > max_ctx;
}
__device__ __forceinline__ int units_for(bool mq, int ql, int ctx, int max_ctx, int max_q_len) {
  if (!mq) return units_of(ctx, max_ctx);
  return (ql <= 0 || mq_bad(ql, ctx, max_q_len, max_ctx)) ? 0 : units_of(ctx, max_ctx);
}
__device__ __forceinline__ int seq_units(const int32_t* __restrict__ ctx_lens,
                                         const int32_t* __restrict__ cu_q, int b, int max_ctx,
                                         int max_q_len) {
  const int ctx = ctx_lens[b];
  const int ql = cu_q ? cu_q[b + 1] - cu_q[b] : 1;
  return units_for(cu_q != nullptr, ql, ctx, max_ctx, max_q_len);
}

// Units of one KV head summed over all sequences (the whole launch is KVH times this).
__device__ __forceinline__ int64_t head_units(const int32_t* __restrict__ ctx_lens,
                                              const int32_t* __restrict__ cu_q, int B,
                                              int max_ctx, int max_q_len) {
  int64_t t = 0;
  for (int b0 = 0; b0 < B; b0 += 64) {
    const int b = b0 + __lane_id();
    t += wave_sum(b < B ? seq_units(ctx_lens, cu_q, b, max_ctx, max_q_len) : 0);
  }
  return t;
}

// Workers that get work: at most num_workers, each with at least kMinUnits units.
__device__ __forceinline__ int64_t active_workers(int64_t C, int num_workers) {
  const int64_t want = (C + kMinUnits - 1) / kMinUnits;
  return want < num_workers ? want : num_workers;
}

// block_size >= 16: a 32-key chunk starts on a multiple of 16 keys, so it touches at most
// two blocks, whose ids are read as scalars.  kOff32: every element offset into one
// layer's K or V cache fits in 31 bits, so addresses are a scalar base plus a 32-bit
// per-lane byte offset.
// HG: KV heads per workgroup.  The work list is (sequence, group of HG KV heads, unit);
// a worker is a workgroup of HG waves, wave i taking KV head HG*group + i of every piece,
// so the waves of a workgroup read the same keys' rows side by side (HG x 256 bytes of
// each 2 KiB slot row at D 128: the pool's DRAM pages are then read HG slices at a time).
template <typename Tag, int D, bool kOff32, int HG>
__global__ __launch_bounds__(64 * HG) __attribute__((amdgpu_waves_per_eu(kOcc))) void decode_balanced_kernel(
    const uint16_t* __restrict__ q, int64_t qsb, int64_t qsh, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t num_slots, int64_t kvs_slot, int64_t kvs_head,
    const int32_t* __restrict__ bt, int64_t bt_stride, int32_t log2_bs,
    const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ cu_q, int32_t B,
    int32_t KVH, int32_t G, int32_t RPH, int32_t max_ctx, float scale_log2,
    int32_t num_workers, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    uint16_t* __restrict__ out, int64_t osb, int64_t osh, int32_t* __restrict__ err_count) {
  constexpr int NKK = D / 32;       // 32-dim K steps of the score MFMA
  constexpr int NT = D / 16;        // 16-dim output tiles
  constexpr int CPR = D / 8;        // 16-byte chunks per K/V row
  constexpr int ROWB = 2 * D;       // bytes of one K/V row
  constexpr int SLAB = 32 * ROWB;   // one 32-key V chunk
  constexpr int VINS = SLAB / 1024; // 1-KiB DMA loads per V chunk
  constexpr int RPI = 1024 / ROWB;  // V rows per DMA load
  __shared__ __attribute__((aligned(1024))) char slab[HG][SLAB];

  const int lane = threadIdx.x & 63;
  const int hw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // head within the group
  const int NG = KVH / HG;                                          // head groups
  const int n = lane & 15;   // packed row (MFMA N index): query qi = n / G, head g = n % G
  const int grp = lane >> 4; // lane group: K sub-range of the MFMA operands

  // ---- this worker's unit range and where it starts
  const int maxq = RPH / G;  // max_q_len: the workspace's query rows per head / G
  const int64_t C = head_units(ctx_lens, cu_q, B, max_ctx, maxq) * NG;
  const int64_t W = active_workers(C, num_workers);
  const int64_t w = blockIdx.x;
  if (w >= W) return;
  int64_t U = w * C / W;
  int64_t left = (w + 1) * C / W - U;
  int b = 0, ctx = 0, nb = 0;
  {
    int64_t base = 0;  // per-head units of the sequences before this 64-sequence chunk
    for (int b0 = 0; b0 < B; b0 += 64) {
      const int bb = b0 + lane;
      const int c = bb < B ? clamp_ctx(ctx_lens[bb], max_ctx) : 0;
      const int v = bb < B ? seq_units(ctx_lens, cu_q, bb, max_ctx, maxq) : 0;
      const int incl = wave_incl_scan(v);
      const uint64_t hit = __ballot(int64_t(NG) * (base + incl) > U);
      if (hit) {
        const int f = __builtin_amdgcn_readfirstlane(
            __ffsll(static_cast<unsigned long long>(hit)) - 1);
        b = b0 + f;
        ctx = __builtin_amdgcn_readlane(c, f);
        nb = __builtin_amdgcn_readlane(v, f);
        U -= int64_t(NG) * (base + __builtin_amdgcn_readlane(incl, f) - nb);  // inside b
        break;
      }
      base += __builtin_amdgcn_readlane(incl, 63);
    }
  }
  if (nb == 0) return;  // unreachable: unit U < C lies in a non-empty sequence
  int kvg = static_cast<int>(U / nb);
  int u = static_cast<int>(U % nb);

  const int bmask = (1 << log2_bs) - 1;
  char* const slab_l = slab[hw];
  auto swz = [](int r, int c) { return c ^ ((2 * ((r >> 2) & 3)) & (CPR - 1)); };
  bool any_bad = false;

  for (;;) {
    // ---- piece: units [u, u1) of segment (b, kvh), keys [kb, ke)
    const int u1 = static_cast<int>(left < int64_t(nb - u) ? u + left : nb);
    const int kb = u << kLog2Unit;
    const int ke = min(u1 << kLog2Unit, ctx);
    const bool whole = u == 0 && u1 == nb;
    const int kvh = kvg * HG + hw;
    const int64_t bt_row = int64_t(b) * bt_stride;
    const int64_t head_off = int64_t(kvh) * kvs_head;
    // query rows of sequence b: token q0 + qi, head kvh*G + g; row qi sees keys < lim
    const int q0 = cu_q ? cu_q[b] : b;
    const int ql = cu_q ? cu_q[b + 1] - q0 : 1;
    const bool row_ok = n < ql * G;
    const int qi = row_ok ? n / G : 0;
    const int g = row_ok ? n - qi * G : 0;
    const int lim = min(ke, ctx - ql + qi + 1);

    dsp_u32x4 qop[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
      qop[kk] = row_ok ? *reinterpret_cast<const dsp_u32x4*>(q + int64_t(q0 + qi) * qsb +
                                                             int64_t(kvh * G + g) * qsh + 32 * kk +
                                                             8 * grp)
                       : dsp_u32x4{0u, 0u, 0u, 0u};

    // Block-table windows: lane i holds the id of block wblk + i (win) and wblk + 64 + i
    // (win2).  Chunks advance by 32 keys, i.e. by at most 32 blocks, so a chunk always
    // lies within win and win2 once the windows have been advanced for its first key.
    int wblk = kb >> log2_bs;
    auto load_win = [&](int first) -> int32_t {
      const int64_t j = int64_t(first) + lane;
      return j < bt_stride ? bt[bt_row + j] : -1;
    };
    int32_t win = load_win(wblk), win2 = load_win(wblk + 64);
    auto advance = [&](int key) {
      if ((key >> log2_bs) - wblk >= 64) {
        wblk += 64;
        win = win2;
        win2 = load_win(wblk + 64);
      }
    };
    // Block ids of the chunk starting at t0: its first block and the next one (scalars).
    int32_t cb0 = 0, cb1 = 0;
    auto chunk_blocks = [&](int t0) {
      const int j = (t0 >> log2_bs) - wblk;  // < 64 after advance(t0); j + 1 < 128
      cb0 = j < 64 ? __builtin_amdgcn_readlane(win, j) : __builtin_amdgcn_readlane(win2, j - 64);
      cb1 = j + 1 < 64 ? __builtin_amdgcn_readlane(win, j + 1)
                       : __builtin_amdgcn_readlane(win2, j + 1 - 64);
    };
    // Element offset of `key` of the chunk starting at t0 in one layer's cache (head
    // included), -1 when its block id is out of range.
    auto elem_of = [&](int t0, int key) -> int64_t {
      const int32_t blk = ((key >> log2_bs) != (t0 >> log2_bs)) ? cb1 : cb0;
      const int64_t sl = int64_t(blk) * (bmask + 1) + (key & bmask);
      return (sl >= 0 && sl < num_slots) ? sl * kvs_slot + head_off : int64_t(-1);
    };
    auto addr = [&](const uint16_t* base, int64_t e) -> const uint16_t* {
      if constexpr (kOff32)
        return reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(base) +
                                                 (static_cast<uint32_t>(e) << 1));
      else
        return base + e;
    };

    dsp_u32x4 kop[2][NKK];
    // K operands of the two 16-key halves of chunk t0 (lane: key t0 + 16*st + n, dims
    // 8*grp + 32*kk).  Keys past ke load row ke - 1 (their scores are masked to -inf
    // below), a bad block id row 0: the loads are unconditional, so the loop head waits
    // for exactly these loads and nothing else.
    auto load_k = [&](int t0) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int key = t0 + 16 * st + n;
        const int64_t e = elem_of(t0, min(key, ke - 1));
        any_bad |= key < ke && e < 0;
        const int64_t ee = e >= 0 ? e : 0;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
          kop[st][kk] = *reinterpret_cast<const dsp_u32x4*>(addr(kc, ee + 32 * kk + 8 * grp));
      }
    };
    // V rows of chunk t0 into the slab: chunk c of row r at slot c ^ 2*((r >> 2) & 3).
    // Rows past ke repeat row ke - 1 (finite data, probability exactly 0).  Non-temporal
    // (aux 2): a layer's V is read once per step and other layers evict it before the next,
    // so keeping it in the caches only costs (same-box A/B over multi-layer loops: config 3
    // 361.8-364.9 -> 351.0 us, config 2 41.0-41.3 -> 39.4-39.6, the skewed and mixed batches
    // and the skewed verify 4-5 % faster; non-temporal K loads as well gained on config 2 but
    // lost 2 % on config 3).
    auto load_v = [&](int t0) {
#pragma unroll
      for (int i = 0; i < VINS; ++i) {
        const int row = i * RPI + lane / CPR, sl = lane % CPR;
        const int64_t e = elem_of(t0, min(t0 + row, ke - 1));
        const uint16_t* src = addr(vc, (e >= 0 ? e : 0) + 8 * swz(row, sl));
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                         (__attribute__((address_space(3))) void*)(slab_l + i * 1024),
                                         16, 0, 2);
      }
    };

    int vbase[NT < 4 ? NT : 4];  // lane's V^T read offsets for nt & 3 (see the P.V loop)
#pragma unroll
    for (int j = 0; j < (NT < 4 ? NT : 4); ++j)
      vbase[j] = 4 * grp * ROWB + 32 * (j ^ (((2 * grp) & (CPR - 1)) >> 1)) + 16 * (n >> 3) +
                 2 * (n & 7);

    float m = -INFINITY, lpart = 0.f;
    f32x4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // K before V, as inside the loop: the loop head then waits for K only (vmcnt(VINS)),
    // with this chunk's V still in flight, on entry and on every later iteration alike.
    chunk_blocks(kb);
    load_k(kb);
    load_v(kb);
    for (int t0 = kb; t0 < ke; t0 += 32) {
      const int tn = t0 + 32;
      const bool prefetch = tn < ke;
      f32x4 sc[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        sc[st] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) sc[st] = mfma32<Tag>(kop[st][kk], qop[kk], sc[st]);
      }
      if (prefetch) {
        advance(tn);
        chunk_blocks(tn);
        load_k(tn);
      }
      // Scale and mask; lane holds keys t0 + 16*st + 4*grp + j of packed row n.
      float s[2][4];
      float mx = -INFINITY;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = t0 + 16 * st + 4 * grp + j;
          s[st][j] = (row_ok && key < lim) ? sc[st][j] * scale_log2 : -INFINITY;
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
      const dsp_u32x4 pop = dsp_u32x4{pack2(pb[0], pb[1]), pack2(pb[2], pb[3]),
                                      pack2(pb[4], pb[5]), pack2(pb[6], pb[7])};
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] *= alpha;

      // This chunk's V has landed once at most the next chunk's K loads (2 * NKK) and a
      // window load remain outstanding; loads complete in issue order.
      if (prefetch)
        __builtin_amdgcn_s_waitcnt(dsp_waitcnt_vm<2 * NKK>());
      else
        __builtin_amdgcn_s_waitcnt(dsp_waitcnt_vm<0>());
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // V^T operand: lane needs dim 16*nt + n of keys {4*grp+u} (u<4) and {16+4*grp+u-4}.
      // Those rows all have (row >> 2) & 3 == grp, so their swizzle is one XOR with
      // 2*grp: dim d sits at byte 32*(nt ^ y) + 16*(n >> 3) + 2*(n & 7) of the row, with
      // y = (2*grp & (CPR-1)) / 2 < 4.  Per lane that is one base per nt & 3 plus
      // compile-time offsets (row, nt & ~3), i.e. LDS immediates.
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        uint16_t v[8];
#pragma unroll
        for (int uu = 0; uu < 8; ++uu) {
          const int krow = uu < 4 ? uu : 12 + uu;  // row minus 4*grp
          v[uu] = *reinterpret_cast<const uint16_t*>(
              slab_l + vbase[nt & 3] + krow * ROWB + 32 * (nt & ~3));
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
    }

    // Row sums: this lane's keys only so far; add the other three lane groups.
    lpart += dsp_shfl_xor(lpart, 16);
    lpart += dsp_shfl_xor(lpart, 32);
    if (row_ok) {
      if (whole) {
        const float inv = lpart > 0.f ? 1.f / lpart : 0.f;
        uint16_t* o = out + int64_t(q0 + qi) * osb + int64_t(kvh * G + g) * osh + 4 * grp;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int j = 0; j < 4; ++j) o[16 * nt + j] = narrow<Tag>(acc[nt][j] * inv);
      } else {
        // piece (segment s = b*NG + kvg, worker w) is slot s + w; its head hw, row n
        const int64_t row = ((int64_t(b) * NG + kvg + w) * HG + hw) * RPH + n;
        float* a = ws_acc + row * D + 4 * grp;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) *reinterpret_cast<f32x4*>(a + 16 * nt) = acc[nt];
        if (grp == 0) {
          ws_ml[2 * row] = m;
          ws_ml[2 * row + 1] = lpart;
        }
      }
    }

    left -= u1 - u;
    if (left <= 0) break;
    // next segment: the next head group of b, or the first of the next non-empty sequence
    // (one exists: units remain)
    u = 0;
    if (++kvg == NG) {
      kvg = 0;
      do {
        if (++b >= B) break;
        ctx = clamp_ctx(ctx_lens[b], max_ctx);
        nb = seq_units(ctx_lens, cu_q, b, max_ctx, maxq);
      } while (nb == 0);
      if (b >= B) break;
    }
  }
  if (err_count && __ballot(any_bad) && lane == 0) atomicAdd(err_count, 1);
}

// One workgroup (4 waves) per (sequence b, query head h, query i).  Merges the pieces of
// segment (b, h / G) when more than one worker covered it, writes zeros for an empty
// context, and counts a bad length once per sequence: for decode (cu_q null, one query per
// sequence) a context outside [0, max_ctx]; for multi-query a context outside
// [q_len, max_ctx], whose rows are written as zeros.  One pass with online
// rescaling: wave w takes pieces w, w + 4, ..., each lane loading the (max, sum) pair and
// its dims of the accumulator of up to 16 pieces at once, so the merge costs two dependent
// memory round trips (ctx_lens, then the pieces) for up to 64 pieces; the waves' partial
// merges meet in LDS.  The piece count is known (and wave-uniform) before the pieces are
// loaded, so a wave issues loads for its own pieces only: loading all 16 through clamped
// addresses and discarding the extra ones by a select cost ~1.3 us of L1 bandwidth per
// launch on config 2 (9 pieces a segment).
template <typename Tag, int D>
__global__ __launch_bounds__(256) void decode_balanced_combine_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
    const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ cu_q, int32_t B,
    int32_t KVH, int32_t G, int32_t RPH, int32_t max_ctx, int32_t num_workers, int32_t HG,
    uint16_t* __restrict__ out, int64_t osb, int64_t osh, int32_t* __restrict__ err_count) {
  constexpr int NV = D > 64 ? 2 : 1;  // dims per lane: lane, lane + 64
  constexpr int kInFlight = 16;       // pieces loaded per lane before they are folded in
  __shared__ float s_acc[4][NV * 64];
  __shared__ float s_ml[4][2];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int h = blockIdx.x, b = blockIdx.y, i = blockIdx.z;
  const int maxq = RPH / G;  // max_q_len (the grid's z extent)
  // One scan per 64 sequences gives the total units and the units of the sequences before
  // b; sequence b's own lengths are read out of the same lanes (readlane), so the merge
  // waits on one memory round trip before its pieces: no separate loads of cu_q[b] or
  // ctx_lens[b] ahead of the scan or behind it.
  int64_t total = 0, pre = 0;
  int q0 = b, ql = 1, raw = 0, nb = 0;
  const bool mq = cu_q != nullptr;
  for (int b0 = 0; b0 < B; b0 += 64) {
    const int bb = b0 + lane;
    const bool in = bb < B;
    const int ctx = in ? ctx_lens[bb] : 0;
    const int c0 = in && mq ? cu_q[bb] : bb;
    const int c1 = in && mq ? cu_q[bb + 1] : bb + 1;
    const int u = in ? units_for(mq, c1 - c0, ctx, max_ctx, maxq) : 0;
    const int incl = wave_incl_scan(u);
    if (b >= b0 && b < b0 + 64) {  // wave-uniform
      const int l = b - b0;
      pre = total + (l > 0 ? __builtin_amdgcn_readlane(incl, l - 1) : 0);
      q0 = __builtin_amdgcn_readlane(c0, l);
      ql = __builtin_amdgcn_readlane(c1, l) - q0;
      raw = __builtin_amdgcn_readlane(ctx, l);
      nb = __builtin_amdgcn_readlane(u, l);
    }
    total += __builtin_amdgcn_readlane(incl, 63);
  }
  if (i >= ql) return;
  const bool bad = mq ? mq_bad(ql, raw, maxq, max_ctx) : (raw < 0 || raw > max_ctx);
  if (h == 0 && i == 0 && threadIdx.x == 0 && err_count && bad) atomicAdd(err_count, 1);
  uint16_t* o = out + int64_t(q0 + i) * osb + int64_t(h) * osh;
  if (nb == 0) {
    if (threadIdx.x < D) o[threadIdx.x] = 0;
    return;
  }
  const int NG = KVH / HG;
  const int64_t C = total * NG;
  const int64_t W = active_workers(C, num_workers);
  const int kvh = h / G, g = h % G, kvg = kvh / HG, hw = kvh % HG;
  const int64_t cs = int64_t(NG) * pre + int64_t(kvg) * nb, ce = cs + nb;
  const int64_t w0 = ((cs + 1) * W - 1) / C, w1 = (ce * W - 1) / C;
  if (w0 == w1) return;  // one worker covered the segment and wrote the output
  const int np = static_cast<int>(w1 - w0 + 1);
  // piece p is slot (b*NG + kvg) + w0 + p; its head hw, row i*G + g
  const int64_t row0 = ((int64_t(b) * NG + kvg + w0) * HG + hw) * RPH + i * G + g;
  const int64_t pstride = int64_t(HG) * RPH;  // rows between consecutive slots
  const bool act = lane < D;
  const float* src = ws_acc + row0 * D + (act ? lane : 0);
  const float* ml = ws_ml + 2 * row0;

  float Mw = -INFINITY, Lw = 0.f, A[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) A[j] = 0.f;
  const int npw = np > wave ? (np - wave + 3) >> 2 : 0;  // this wave's pieces: wave + 4k
  for (int k0 = 0; k0 < npw; k0 += kInFlight) {
    float mv[kInFlight], lv[kInFlight], v[kInFlight][NV];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      if (k0 + u < npw) {  // wave-uniform: the loads of absent pieces are not issued
        const int64_t r = int64_t(wave + 4 * (k0 + u)) * pstride;
        mv[u] = ml[2 * r];
        lv[u] = ml[2 * r + 1];
#pragma unroll
        for (int j = 0; j < NV; ++j) v[u][j] = src[r * D + 64 * j];
      } else {
        mv[u] = -INFINITY;
        lv[u] = 0.f;
#pragma unroll
        for (int j = 0; j < NV; ++j) v[u][j] = 0.f;
      }
    }
    float bm = Mw;
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) bm = fmaxf(bm, mv[u]);
    const float bmu = bm == -INFINITY ? 0.f : bm;
    const float keep = dsp_exp2(Mw - bmu);
    Lw *= keep;
#pragma unroll
    for (int j = 0; j < NV; ++j) A[j] *= keep;
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      const float wk = dsp_exp2(mv[u] - bmu);
      Lw = fmaf(lv[u], wk, Lw);
#pragma unroll
      for (int j = 0; j < NV; ++j) A[j] = fmaf(v[u][j], wk, A[j]);
    }
    Mw = bm;
  }
  if (lane == 0) {
    s_ml[wave][0] = Mw;
    s_ml[wave][1] = Lw;
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) s_acc[wave][lane + 64 * j] = A[j];
  __syncthreads();
  if (threadIdx.x < D) {
    const int d = threadIdx.x;
    const float M = fmaxf(fmaxf(s_ml[0][0], s_ml[1][0]), fmaxf(s_ml[2][0], s_ml[3][0]));
    const float Mu = M == -INFINITY ? 0.f : M;
    float Lt = 0.f, At = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float wk = dsp_exp2(s_ml[w][0] - Mu);
      Lt = fmaf(s_ml[w][1], wk, Lt);
      At = fmaf(s_acc[w][d], wk, At);
    }
    o[d] = narrow<Tag>(At * (Lt > 0.f ? 1.f / Lt : 0.f));
  }
}

template <typename Tag, int D, int HG>
int launch_balanced_hg(int W, const uint16_t* q, int64_t qsb, int64_t qsh, const uint16_t* kc,
                       const uint16_t* vc, int64_t num_slots, int64_t kvs_slot, int64_t kvs_head,
                       const int32_t* bt, int64_t bt_stride, int32_t log2_bs,
                       const int32_t* ctx_lens, const int32_t* cu_q, int32_t max_q_len,
                       int32_t B, int32_t KVH, int32_t G, int32_t max_ctx, float scale_log2,
                       float* ws_acc, float* ws_ml, uint16_t* out, int64_t osb, int64_t osh,
                       int32_t* err_count, hipStream_t s) {
  const int Wg = W / HG > 0 ? W / HG : 1;  // workgroups of HG waves
  const int RPH = max_q_len * G;           // workspace rows per head
  // largest element offset: last slot's last head's row end
  const bool off32 = num_slots * kvs_slot + KVH * kvs_head + D < (int64_t(1) << 31);
  if (off32)
    decode_balanced_kernel<Tag, D, true, HG><<<dim3(static_cast<unsigned>(Wg)), 64 * HG, 0, s>>>(
        q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head, bt, bt_stride, log2_bs, ctx_lens,
        cu_q, B, KVH, G, RPH, max_ctx, scale_log2, Wg, ws_acc, ws_ml, out, osb, osh, err_count);
  else
    decode_balanced_kernel<Tag, D, false, HG><<<dim3(static_cast<unsigned>(Wg)), 64 * HG, 0, s>>>(
        q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head, bt, bt_stride, log2_bs, ctx_lens,
        cu_q, B, KVH, G, RPH, max_ctx, scale_log2, Wg, ws_acc, ws_ml, out, osb, osh, err_count);
  const int st = dsp_launch_status();
  if (st != DSP_OK) return st;
  const int Hq = KVH * G;
  decode_balanced_combine_kernel<Tag, D><<<dim3(Hq, B, max_q_len), 256, 0, s>>>(
      ws_acc, ws_ml, ctx_lens, cu_q, B, KVH, G, RPH, max_ctx, Wg, HG, out, osb, osh, err_count);
  return dsp_launch_status();
}

template <typename Tag, int D>
int launch_balanced_d(int W, const uint16_t* q, int64_t qsb, int64_t qsh, const uint16_t* kc,
                      const uint16_t* vc, int64_t num_slots, int64_t kvs_slot, int64_t kvs_head,
                      const int32_t* bt, int64_t bt_stride, int32_t log2_bs,
                      const int32_t* ctx_lens, const int32_t* cu_q, int32_t max_q_len,
                      int32_t B, int32_t KVH, int32_t G, int32_t max_ctx, float scale_log2,
                      float* ws_acc, float* ws_ml, uint16_t* out, int64_t osb, int64_t osh,
                      int32_t* err_count, hipStream_t s) {
  switch (dsp_detail::balanced_head_group(KVH)) {
    case 8:
      return launch_balanced_hg<Tag, D, 8>(W, q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head,
                                           bt, bt_stride, log2_bs, ctx_lens, cu_q, max_q_len, B,
                                           KVH, G, max_ctx, scale_log2, ws_acc, ws_ml, out, osb,
                                           osh, err_count, s);
    case 4:
      return launch_balanced_hg<Tag, D, 4>(W, q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head,
                                           bt, bt_stride, log2_bs, ctx_lens, cu_q, max_q_len, B,
                                           KVH, G, max_ctx, scale_log2, ws_acc, ws_ml, out, osb,
                                           osh, err_count, s);
    case 2:
      return launch_balanced_hg<Tag, D, 2>(W, q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head,
                                           bt, bt_stride, log2_bs, ctx_lens, cu_q, max_q_len, B,
                                           KVH, G, max_ctx, scale_log2, ws_acc, ws_ml, out, osb,
                                           osh, err_count, s);
    default:
      return launch_balanced_hg<Tag, D, 1>(W, q, qsb, qsh, kc, vc, num_slots, kvs_slot, kvs_head,
                                           bt, bt_stride, log2_bs, ctx_lens, cu_q, max_q_len, B,
                                           KVH, G, max_ctx, scale_log2, ws_acc, ws_ml, out, osb,
                                           osh, err_count, s);
  }
}

template <typename Tag, typename... A>
int launch_balanced(int D, A... args) {
  switch (D) {
    case 32: return launch_balanced_d<Tag, 32>(args...);
    case 64: return launch_balanced_d<Tag, 64>(args...);
    case 128: return launch_balanced_d<Tag, 128>(args...);
    default: return DSP_EUNSUPPORTED;
  }
}

}  // namespace

namespace dsp_detail {

int device_cus() {
  // a device property: queried once per device (a race only repeats the same query)
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < kMaxDevices) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;
  if (dev >= 0 && dev < kMaxDevices) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}


// KV heads per workgroup of the balanced kernel: the largest of 4, 2, 1 dividing KVH.
int balanced_head_group(int32_t KVH) {
  return KVH % 4 == 0 ? 4 : (KVH % 2 == 0 ? 2 : 1);
}

bool balanced_decode_applies(int32_t B, int32_t KVH, int32_t D, int32_t max_ctx,
                             int32_t block_size) {
  if (B < 1 || B > kMaxBatch || KVH < 1 || max_ctx < 1) return false;
  if (block_size < (1 << kLog2Unit)) return false;
  if (D != 32 && D != 64 && D != 128) return false;
  // the unit scans (here and in the merge) add up 64 sequences' unit counts in 32-bit
  // lanes: at most 64 x (2^25 - 1) units, i.e. contexts below 2^29 - 15 tokens
  if (max_ctx > (1 << 29) - 16) return false;
  // w * C stays far inside int64 for every worker index w
  const int64_t cmax = int64_t(B) * KVH * ((int64_t(max_ctx) + 15) >> kLog2Unit);
  return cmax < (int64_t(1) << 40);
}

int32_t balanced_workers(int32_t B, int32_t KVH, int32_t max_ctx) {
  // One worker wave per SIMD: every CU gets the same number of workgroups (4 / HG of
  // them), and fewer, longer key streams over the randomly placed blocks read faster than
  // three waves per SIMD (config 3 387 -> 377-379 us, one 32k context among 15 short
  // 50.5 -> 46-47, config 2 -1 %); 1.5 or 0.75 waves per SIMD load the CUs unevenly
  // (config 3 410-414 us).
  const int64_t cap = int64_t(dsp_detail::device_cus()) * 4;
  const int64_t cmax = int64_t(B) * KVH * ((int64_t(max_ctx) + 15) >> kLog2Unit);
  int64_t want = (cmax + kMinUnits - 1) / kMinUnits;
  if (want < 1) want = 1;
  return static_cast<int32_t>(want < cap ? want : cap);
}

size_t balanced_workspace_bytes(int32_t B, int32_t KVH, int32_t rows_per_head, int32_t D,
                                int32_t max_ctx) {
  const int64_t slots = int64_t(B) * KVH + balanced_workers(B, KVH, max_ctx);
  return size_t(slots) * rows_per_head * (size_t(D) + 2) * sizeof(float);
}

int balanced_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                    const uint16_t* k_cache, const uint16_t* v_cache, int64_t num_slots,
                    int64_t kv_stride_slot, int64_t kv_stride_head, const int32_t* block_table,
                    int64_t bt_stride, int32_t log2_bs, const int32_t* ctx_lens,
                    const int32_t* cu_q, int32_t max_q_len, int32_t B, int32_t KVH, int32_t G,
                    int32_t D, float scale_log2, int32_t max_ctx, float* workspace,
                    uint16_t* out, int64_t o_stride_b, int64_t o_stride_h, bool f16,
                    int32_t* err_count, hipStream_t s) {
  const int32_t W = balanced_workers(B, KVH, max_ctx);
  float* ws_acc = workspace;
  float* ws_ml = ws_acc + (int64_t(B) * KVH + W) * max_q_len * G * D;
  if (!f16)
    return launch_balanced<Bf16Tag>(D, W, q, q_stride_b, q_stride_h, k_cache, v_cache,
                                    num_slots, kv_stride_slot, kv_stride_head, block_table,
                                    bt_stride, log2_bs, ctx_lens, cu_q, max_q_len, B, KVH, G,
                                    max_ctx, scale_log2, ws_acc, ws_ml, out, o_stride_b,
                                    o_stride_h, err_count, s);
  return launch_balanced<F16Tag>(D, W, q, q_stride_b, q_stride_h, k_cache, v_cache, num_slots,
                                 kv_stride_slot, kv_stride_head, block_table, bt_stride, log2_bs,
                                 ctx_lens, cu_q, max_q_len, B, KVH, G, max_ctx, scale_log2,
                                 ws_acc, ws_ml, out, o_stride_b, o_stride_h, err_count, s);
}

}  // namespace dsp_detail
