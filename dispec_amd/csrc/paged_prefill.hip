// J4 for long query blocks (chunked prefill over the paged cache): a FlashAttention-style
// tile of 128 packed rows per workgroup on v_mfma_f32_32x32x16.
//
// Semantics are dsp_paged_mq_attention's (ModelRunner._attention's native branch,
// dispec/engine/model_runner.py:160-185): per sequence, SDPA over the paged context with
// causal_lower_right(q_len, ctx) and GQA; packed row r of a (sequence, KV head) is query
// r / G of query head kvh*G + r % G.
//
// Why a second kernel: the multi-query kernel of paged_mq.hip gives each workgroup 16 rows
// and streams K/V through registers, which suits verify (q_len <= 16 / G) but caps a
// 512-token prefill chunk at ~200 TFLOP/s: every 16-row tile re-reads the whole context
// from L2 (16 flop per K/V byte).  Here four waves share each 64-key chunk of K and V,
// loaded once per workgroup straight into LDS (global_load_lds_dwordx4, double-buffered,
// 64 KiB: two workgroups per CU), so a chunk feeds 128 rows.
//
// Per wave (32 rows) and chunk:
//  * S^T = K . Q^T: 2 (keys) x D/16 (dims) MFMAs 32x32x16; K rows come from LDS as the A
//    operand (16-byte chunks XOR-swizzled by row: conflict-free), Q^T stays in registers.
//  * Lane l holds row l % 32 and, per 16-key step, keys 4*(l/32) + {0..3, 8..11} -- exactly
//    the B operand of O^T += V^T . P^T for a 16-key step whose K index is permuted the same
//    way, so P never leaves registers; V^T is read from LDS 2 bytes at a time in that
//    order (rows swizzled so the two lane groups hit different banks).
//  * Online softmax in base 2 per row; the row max needs one exchange between the lane
//    halves.
// Partials go to the multi-query kernel's workspace layout (16-row tiles), so its merge
// kernel combines the key partitions.
#include <float.h>

#include "dsp_common.h"
#include "dsp_internal.h"
#include "dsp_mfma.h"

namespace {

using namespace dsp_mfma;

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4, kThreads = 64 * kWaves;
constexpr int kRows = 32 * kWaves;  // packed rows per workgroup
constexpr int kChunk = 64;          // keys per LDS chunk
constexpr int kMaxSharedSeqs = 1024;  // sequences of a shared-prefix launch (cu_q in LDS)

template <typename Tag>
__device__ __forceinline__ f32x16 mfma32x32(dsp_u32x4 a, dsp_u32x4 b, f32x16 c) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void lds_void_t;

// One LDS DMA (global_load_lds_dwordx4): 16 bytes per lane from sbase + voff into LDS at
// m0 + 16 * lane.  It is issued from inline assembly so that the compiler does not make
// later LDS reads wait for it: its waitcnt pass cannot tell the DMA's target buffer from
// the one being read and would wait for the whole DMA.  The kernel waits for it itself
// (vmcnt) before the barrier that publishes the chunk.  M0 has no other user here.
// kNonTemporal marks the load nt: a shared-prefix launch reads most of its keys once (the
// prefix by one or a few packed tiles, each suffix by its sequence's tiles), so keeping them
// in the caches only evicts what other launches reuse (fork decode 23.5-23.8 -> 21.4 us
// per layer, verify unchanged).  An unshared prefill re-reads a sequence's keys from every
// 128-row tile of its queries and keeps the ordinary load (nt costs it 3-8 %).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool kNonTemporal>
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t m0) {
  if constexpr (kNonTemporal)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(voff), "s"(sbase), "s"(m0)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(m0)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;

// kShared: a shared-prefix (cascade) launch, two kinds of workgroup in one grid.  For
// x < prefix_x (per KV head) a workgroup is a prefix tile: packed row r is token r / G of
// the whole batch (every sequence's queries), query head kvh*G + r % G; the keys are the
// first prefix_tokens of block-table row 0, which every sequence shares and every query
// sees whole (no mask); partition `part` covers keys [part*P, part*P + P) and is written,
// for every row, to that row's own (sequence, 16-row tile) slot of the merge layout.  The
// other workgroups are suffix tiles: one sequence's rows over one partition of P of its
// keys from prefix_tokens on (causal), numbered on from the prefix's partitions (keys
// [part*P, part*P + P) again).  Both kinds run side by side; the merge then folds every
// partition up to a row's last visible key, as for an unshared launch.
template <typename Tag, int D, bool kShared>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void paged_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t qst, int64_t qsh, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int64_t num_slots, int64_t kvs_slot, int64_t kvs_head,
    const int32_t* __restrict__ bt, int64_t bt_stride, int32_t log2_bs,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ ctx_lens, int32_t max_ctx,
    int32_t G, float scale_log2, int32_t P, int32_t num_parts, int32_t tiles16_max,
    float* __restrict__ ws_acc, float* __restrict__ ws_ml, uint16_t* __restrict__ out,
    int64_t ost, int64_t osh, int32_t* __restrict__ err_count, int32_t nseq,
    int32_t prefix_tokens, int32_t ws_parts, int32_t prefix_x) {
  constexpr int NKS = D / 16;        // 16-dim steps of the score MFMA
  constexpr int NDT = D / 32;        // 32-dim output tiles
  constexpr int CPR = D / 8;         // 16-byte chunks per K/V row
  constexpr int ROWB = 2 * D;        // bytes per K/V row
  constexpr int SLAB = kChunk * ROWB;            // one K (or V) chunk
  constexpr int RPI = 1024 / ROWB;               // rows per 1-KiB DMA load
  constexpr int LPW = SLAB / 1024 / kWaves;      // DMA loads per wave per slab
  static_assert(LPW >= 1, "every wave loads part of a chunk");
  __shared__ __attribute__((aligned(1024))) char lds[2][2][SLAB];  // [buffer][K | V]
  __shared__ int32_t s_cu[kShared ? kMaxSharedSeqs + 1 : 1];         // cu_q, prefix pass

  // XCD-aware order: the dispatcher hands workgroup `lin` to XCD lin % 8.  Each XCD gets a
  // contiguous range of logical ids, so the tiles of one (sequence, KV head) -- which read
  // the same K/V -- run on one XCD and share its L2.  Within a (sequence, KV head) the
  // heaviest tiles (the last rows see the most keys) come first.
  const int X = gridDim.x, KVH = gridDim.y;
  const int64_t nwg = int64_t(X) * KVH * gridDim.z;
  const int64_t lin = blockIdx.x + int64_t(X) * (blockIdx.y + int64_t(KVH) * blockIdx.z);
  const int64_t q8 = nwg / 8, r8 = nwg % 8, xcd = lin % 8, pos = lin / 8;
  const int64_t lg = xcd < r8 ? xcd * (q8 + 1) + pos : r8 * (q8 + 1) + (xcd - r8) * q8 + pos;
  const int xl = int(lg % X);
  const int kvh = int((lg / X) % KVH);
  int b = int(lg / X / KVH), part, tile;
  bool pre = false;  // a prefix tile of a shared-prefix launch
  if constexpr (kShared) {
    pre = xl < prefix_x;
    if (pre) {
      part = xl % num_parts;
      tile = prefix_x / num_parts - 1 - xl / num_parts;
    } else {
      // suffix tiles: per sequence tiles_s row tiles x nsp partitions of its keys past the
      // prefix (partition index continues the prefix's: key range [part*P, part*P + P))
      const int first = prefix_tokens / P, nsp = ws_parts - first;
      const int per_seq = (X - prefix_x) / nseq, idx = xl - prefix_x;
      const int tiles_s = per_seq / nsp, k = idx % per_seq;
      b = idx / per_seq;
      tile = tiles_s - 1 - k / nsp;
      part = first + k % nsp;
    }
  } else {
    const int ntiles = X / num_parts;
    part = xl % num_parts;
    tile = ntiles - 1 - xl / num_parts;
  }
  // The first two chunks' block ids are loaded now, beside the lengths below: chunk keys
  // start at part * P whatever the lengths are (clamped into the table's width here; a
  // wave whose rows turn out to start past the partition's end reloads its id below).
  const int wave_e = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t bt_row_e = int64_t(b) * bt_stride;
  const int key_cap = max(max_ctx - 1, 0);
  auto early_blk = [&](int t) {
    return bt[bt_row_e + (min(t + 16 * wave_e, key_cap) >> log2_bs)];
  };
  int32_t blk_first = early_blk(part * P), blk_second = early_blk(part * P + kChunk);
  int q0, qlen, ctx, kend = 0;
  if (pre) {
    // all tokens of the batch; the causal limit never binds (ctx - qlen + qi >= max_ctx)
    q0 = 0;
    qlen = cu_q[nseq];
    ctx = qlen + max_ctx;
    kend = prefix_tokens;
    // staged for the epilogue's row -> sequence search (published by the first chunk's
    // barrier: every workgroup that gets past the checks below runs at least one chunk)
    for (int i = threadIdx.x; i <= nseq; i += kThreads) s_cu[i] = cu_q[i];
  } else {
    q0 = cu_q[b];
    qlen = cu_q[b + 1] - q0;
    ctx = ctx_lens[b];
  }
  const int rows = qlen * G;
  const int r0 = tile * kRows;
  if (qlen <= 0 || r0 >= rows) return;
  if (!pre) {
    // bad lengths (and, in a shared-prefix launch, queries that start inside the prefix):
    // counted once, the rows are zeros
    if (ctx > max_ctx || ctx < qlen || (kShared && ctx - qlen < prefix_tokens)) {
      if (!kShared && part != 0) return;
      if (threadIdx.x == 0 && tile == 0 && kvh == 0 && err_count) atomicAdd(err_count, 1);
      for (int i = threadIdx.x; i < kRows * D; i += kThreads) {
        const int rr = r0 + i / D;
        if (rr < rows)
          out[int64_t(q0 + rr / G) * ost + int64_t(kvh * G + rr % G) * osh + i % D] = 0;
      }
      return;
    }
    const int r_last = min(r0 + kRows - 1, rows - 1);
    kend = ctx - qlen + r_last / G + 1;  // keys any row of the tile sees
  }
  // partition `part` covers keys [part*P, part*P + P) of the tile's visible range (a
  // suffix tile's partitions start at the prefix's end, which is a multiple of P)
  const int kbeg = part * P;
  if (kbeg >= kend) return;
  const int kfin = min(kbeg + P, kend);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hl = lane >> 5;        // lane half: key sub-range of the operands
  const int col = lane & 31;       // this lane's row within the wave
  const int r = r0 + 32 * wave + col;
  const bool row_ok = r < rows;
  const bool wave_has_rows = r0 + 32 * wave < rows;  // wave-uniform
  const int qi = row_ok ? r / G : 0;
  const int h = kvh * G + (row_ok ? r % G : 0);
  // Keys 0..lim are visible to this row (causal limit, and the partition's end); lim_min
  // is the smallest limit among the wave's rows (its first row), wave-uniform.  Rows past
  // `rows` have q = 0: finite scores, never stored.
  const int lim = min(ctx - qlen + qi, kfin - 1);
  const int lim_min = min(ctx - qlen + (r0 + 32 * wave) / G, kfin - 1);
  const int64_t bt_row = int64_t(b) * bt_stride;
  const int64_t head_off = int64_t(kvh) * kvs_head;
  const int bmask = (1 << log2_bs) - 1;

  // Q^T (B operand): lane holds dims 16*ks + 8*hl .. +8 of its row.
  dsp_u32x4 qop[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
    qop[ks] = row_ok ? *reinterpret_cast<const dsp_u32x4*>(q + int64_t(q0 + qi) * qst +
                                                           int64_t(h) * qsh + 16 * ks + 8 * hl)
                     : dsp_u32x4{0u, 0u, 0u, 0u};

  // K/V chunk rows into LDS: load j of this wave covers rows (wave*LPW + j)*RPI ..; lane l
  // fills slot l % CPR of row l / CPR with global chunk slot ^ swz(row).  K rows are
  // swizzled by (row & (CPR-1)) for the A-operand reads (32 rows, one 16-byte chunk each);
  // V rows by whole 64-byte groups (4 chunks): 4*(row & 3) at D 128 and 4*((row >> 1) & 1)
  // at D 64, so each half-wave of a transposing read (4 consecutive rows x 64 bytes) covers
  // all 64 banks once.  Rows past kfin repeat the last key's row (finite data, masked);
  // an out-of-range slot reads slot 0.
  auto kswz = [](int row) { return row & (CPR - 1); };
  auto vswz = [](int row) { return D == 128 ? 4 * (row & 3) : 4 * ((row >> 1) & 1); };
  // Wave w loads rows 16*w .. 16*w + 15 of each chunk.  Chunks start at multiples of 64
  // keys and blocks hold a multiple of 16 tokens, so those rows lie in one block: its id
  // is wave-uniform and the addresses are a scalar base plus per-lane constants.  Rows past
  // kfin read other slots of the same block (finite data, masked); an out-of-range block
  // reads slots 0..15.
  static_assert(LPW * RPI == 16, "16 rows per wave per chunk");
  uint32_t koff[LPW], voff[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int rw = j * RPI + lane / CPR, row = 16 * wave + rw, sl = lane % CPR;
    koff[j] = uint32_t(rw * kvs_slot * 2 + 16 * (sl ^ kswz(row)));
    voff[j] = uint32_t(rw * kvs_slot * 2 + 16 * (sl ^ vswz(row)));
  }
  const uint32_t lds_base = uint32_t(reinterpret_cast<uintptr_t>((lds_void_t*)&lds[0][0][0]));
  auto load_blk = [&](int t0) {
    return bt[bt_row + (min(t0 + 16 * wave, kfin - 1) >> log2_bs)];
  };
  bool any_bad = false;  // (wave-uniform) a block id of visible keys lay outside the cache
  auto issue = [&](int buf, int t0, int32_t blk_v) {
    const int32_t blk = __builtin_amdgcn_readfirstlane(blk_v);
    int64_t slot0 = int64_t(blk) * (bmask + 1) + ((t0 + 16 * wave) & bmask);
    if (blk < 0 || (int64_t(blk) + 1) * (bmask + 1) > num_slots) {
      slot0 = 0;
      any_bad |= t0 + 16 * wave < kfin;
    }
    const int64_t e = slot0 * kvs_slot + head_off;
    const char* kb = reinterpret_cast<const char*>(kc + e);
    const char* vb = reinterpret_cast<const char*>(vc + e);
    const uint32_t m0 = lds_base + uint32_t(buf * 2 * SLAB + wave * LPW * 1024);
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      dma16<kShared>(kb, koff[j], m0 + j * 1024);
      dma16<kShared>(vb, voff[j], m0 + SLAB + j * 1024);
    }
  };

  float m = -INFINITY, lpart = 0.f;
  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[dt][j] = 0.f;

  const int nch = (kfin - kbeg + kChunk - 1) / kChunk;
  // block ids run one chunk ahead of the DMAs, which run one chunk ahead of the MFMAs; the
  // first two were loaded at entry for the unclamped keys, which load_blk would clamp to
  // kfin - 1 only for a wave whose rows start past kfin (then reloaded, as load_blk does)
  if (kbeg + 16 * wave > kfin - 1) blk_first = load_blk(kbeg);
  issue(0, kbeg, blk_first);
  int32_t blk = blk_second;
  if (nch > 1 && kbeg + kChunk + 16 * wave > kfin - 1) blk = load_blk(kbeg + kChunk);
  for (int c = 0; c < nch; ++c) {
    const int t0 = kbeg + c * kChunk;
    // this wave's DMAs of chunk c (and the block ids of chunk c + 1) are in; after the
    // barrier every wave's are, and every wave is done reading chunk c - 1, whose buffer
    // the next DMA overwrites
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(dsp_waitcnt_vm<0>());
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < nch) {
      issue((c + 1) & 1, t0 + kChunk, blk);
      if (c + 2 < nch) blk = load_blk(t0 + 2 * kChunk);
    }
    // A wave whose 32 rows all lie past the tile's rows (a short query block: a verify
    // tile of 10 rows leaves three of four waves empty) only loads its share of each chunk.
    if (!wave_has_rows) continue;
    const char* ks_lds = &lds[c & 1][0][0];
    const char* vs_lds = &lds[c & 1][1][0];

    // ---- scores S^T (keys x rows): two 32-key halves
    f32x16 sc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int j = 0; j < 16; ++j) sc[mt][j] = 0.f;
      const int krow = 32 * mt + col;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const dsp_u32x4 kop = *reinterpret_cast<const dsp_u32x4*>(
            ks_lds + krow * ROWB + 16 * ((2 * ks + hl) ^ kswz(krow)));
        sc[mt] = mfma32x32<Tag>(kop, qop[ks], sc[mt]);
      }
    }
    // ---- mask (only chunks that reach past a row's causal limit or past kfin), row max.
    // sc[mt][j] is key 32*mt + 8*(j/4) + 4*hl + j%4 of this lane's row.
    if (t0 + kChunk - 1 > lim_min) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = t0 + 32 * mt + 8 * (j >> 2) + 4 * hl + (j & 3);
          sc[mt][j] = key <= lim ? sc[mt][j] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sc[mt][j]);
    mx = fmaxf(mx, dsp_shfl_xor(mx, 32)) * scale_log2;  // base-2 units; -inf stays -inf
    // Lazy rescale: the running max m only moves when some row's chunk max exceeds it by
    // more than 8 (so p <= 2^8); the result is exact either way, since l and acc share m.
    if (__builtin_amdgcn_ballot_w64(mx > m + 8.f) != 0) {
      const float m_new = fmaxf(m, mx);
      const float alpha = m_new == -INFINITY ? 1.f : dsp_exp2(m - m_new);
      m = m_new;
      lpart *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
    }
    const float neg_m = m == -INFINITY ? 0.f : -m;
    // P^T operands of the four 16-key steps: step ps = 2*mt + half takes registers
    // j = 8*half .. 8*half + 7, i.e. keys 16*ps + 4*hl + {0..3, 8..11}.
    dsp_u32x4 pop[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint16_t pb[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float p = dsp_exp2(fmaf(sc[mt][8 * half + i], scale_log2, neg_m));
          lpart += p;
          pb[i] = narrow<Tag>(p);
        }
        pop[2 * mt + half] = dsp_u32x4{pack2(pb[0], pb[1]), pack2(pb[2], pb[3]),
                                       pack2(pb[4], pb[5]), pack2(pb[6], pb[7])};
      }

    // ---- O^T += V^T . P^T.  Per 16-key step ps the V^T operand is dim 32*dt + col, K index
    // 8*hl + i <-> key 16*ps + 8*(i/4) + 4*hl + i%4 (the P^T order).  In ds_read_b64_tr_b16,
    // lane g + 4a + e of each 16-lane group g receives element e of the 4-element segments
    // addressed by lanes g + a + 4j (j = 0..3); so lane s addresses key 16*ps + 8*inst +
    // 4*hl + (s%16)/4, dims 32*dt + 16*((s/16)%2) + 4*(s%4) .. +3, for inst = 0, 1.
#pragma unroll
    for (int ps = 0; ps < 4; ++ps) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        v4i16 vh[2];
#pragma unroll
        for (int inst = 0; inst < 2; ++inst) {
          const int kr = 16 * ps + 8 * inst + 4 * hl + ((lane & 15) >> 2);
          const int dim0 = 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
          vh[inst] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(
              vs_lds + kr * ROWB + 16 * ((dim0 >> 3) ^ vswz(kr)) + 2 * (dim0 & 7)));
        }
        acc[dt] = mfma32x32<Tag>(__builtin_bit_cast(dsp_u32x4, vh), pop[ps], acc[dt]);
      }
    }
  }

  if (err_count && any_bad && lane == 0) atomicAdd(err_count, 1);  // once per wave

  // ---- epilogue: row sums over the two lane halves; acc[dt][j] = O[row col][dim 32*dt +
  // 8*(j/4) + 4*hl + j%4]
  lpart += dsp_shfl_xor(lpart, 32);
  if (!row_ok) return;
  int sb = b, lr = r;  // the row's sequence and its packed row there
  if (pre) {
    int lo = 0, hi = nseq - 1;  // last sequence whose first token is <= qi
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_cu[mid] <= qi) lo = mid; else hi = mid - 1;
    }
    sb = lo;
    lr = (qi - s_cu[lo]) * G + (r % G);
  }
  const int st = lr / 16, rr = lr % 16;                  // 16-row tile of the merge layout
  if (st >= tiles16_max) return;  // q_len past the caller's max_q_len: rows not covered
  if constexpr (!kShared) {
    const int r_last16 = min(st * 16 + 15, rows - 1);
    const int kend16 = ctx - qlen + r_last16 / G + 1;
    const int nparts16 = (kend16 + P - 1) / P;
    if (part >= nparts16) return;  // the merge for this 16-row tile does not read it
    if (nparts16 == 1) {
      const float inv = lpart > 0.f ? 1.f / lpart : 0.f;
      uint16_t* o = out + int64_t(q0 + qi) * ost + int64_t(h) * osh;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          o[32 * dt + 8 * (j >> 2) + 4 * hl + (j & 3)] = narrow<Tag>(acc[dt][j] * inv);
      return;
    }
  }
  const int64_t slot = ((int64_t(sb) * KVH + kvh) * tiles16_max + st) * ws_parts + part;
  float* a = ws_acc + (slot * 16 + rr) * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4)
      *reinterpret_cast<f32x4*>(a + 32 * dt + 8 * j4 + 4 * hl) =
          f32x4{acc[dt][4 * j4], acc[dt][4 * j4 + 1], acc[dt][4 * j4 + 2], acc[dt][4 * j4 + 3]};
  if (hl == 0) {
    ws_ml[2 * (slot * 16 + rr)] = m;
    ws_ml[2 * (slot * 16 + rr) + 1] = lpart;
  }
}

template <bool kShared, typename... A>
int launch_prefill(int D, bool f16, dim3 grid, hipStream_t s, A... args) {
  if (D == 128) {
    if (f16) paged_prefill_kernel<F16Tag, 128, kShared><<<grid, kThreads, 0, s>>>(args...);
    else paged_prefill_kernel<Bf16Tag, 128, kShared><<<grid, kThreads, 0, s>>>(args...);
  } else {
    if (f16) paged_prefill_kernel<F16Tag, 64, kShared><<<grid, kThreads, 0, s>>>(args...);
    else paged_prefill_kernel<Bf16Tag, 64, kShared><<<grid, kThreads, 0, s>>>(args...);
  }
  return dsp_launch_status();
}

}  // namespace

namespace dsp_detail {

bool prefill_applies(int32_t D, int32_t block_size, int64_t max_rows, int64_t num_slots,
                     int64_t kv_stride_slot) {
  return (D == 64 || D == 128) && block_size >= 16 && max_rows >= kRows && num_slots >= 16 &&
         kv_stride_slot < (int64_t(1) << 25);  // 16-row lane offsets fit 32 bits
}

int64_t prefill_tiles(int32_t max_q_len, int32_t G) {
  return (int64_t(max_q_len) * G + kRows - 1) / kRows;
}

int prefill_attention(const uint16_t* q, int64_t q_stride_t, int64_t q_stride_h,
                      const uint16_t* k_cache, const uint16_t* v_cache, int64_t num_slots,
                      int64_t kv_stride_slot, int64_t kv_stride_head, const int32_t* block_table,
                      int64_t bt_stride, int32_t log2_bs, const int32_t* cu_q,
                      const int32_t* ctx_lens, int32_t B, int32_t KVH, int32_t G, int32_t D,
                      float scale_log2, int32_t max_q_len, int32_t max_ctx, int32_t P,
                      int32_t num_parts, int32_t tiles16_max, float* ws_acc, float* ws_ml,
                      uint16_t* out, int64_t o_stride_t, int64_t o_stride_h, bool f16,
                      int32_t* err_count, hipStream_t s) {
  const int64_t tiles = prefill_tiles(max_q_len, G);
  dim3 grid(static_cast<unsigned>(tiles * num_parts), static_cast<unsigned>(KVH),
            static_cast<unsigned>(B));
  return launch_prefill<false>(D, f16, grid, s, q, q_stride_t, q_stride_h, k_cache, v_cache,
                               num_slots, kv_stride_slot, kv_stride_head, block_table, bt_stride,
                               log2_bs, cu_q, ctx_lens, max_ctx, G, scale_log2, P, num_parts,
                               tiles16_max, ws_acc, ws_ml, out, o_stride_t, o_stride_h,
                               err_count, B, int32_t(0), num_parts, int32_t(0));
}

int prefill_shared_prefix(const uint16_t* q, int64_t q_stride_t, int64_t q_stride_h,
                          const uint16_t* k_cache, const uint16_t* v_cache, int64_t num_slots,
                          int64_t kv_stride_slot, int64_t kv_stride_head,
                          const int32_t* block_table, int64_t bt_stride, int32_t log2_bs,
                          const int32_t* cu_q, const int32_t* ctx_lens, int32_t B, int32_t KVH,
                          int32_t G, int32_t D, float scale_log2, int32_t max_q_len,
                          int32_t max_ctx, int32_t P, int32_t tiles16_max,
                          int32_t prefix_tokens, float* ws_acc, float* ws_ml, uint16_t* out,
                          int64_t o_stride_t, int64_t o_stride_h, bool f16, int32_t* err_count,
                          hipStream_t s) {
  const int32_t prefix_parts = prefix_tokens / P;
  const int32_t suffix_parts = (max_ctx - prefix_tokens + P - 1) / P;
  const int64_t tiles_p = (int64_t(B) * max_q_len * G + kRows - 1) / kRows;
  const int64_t prefix_x = tiles_p * prefix_parts;
  const int64_t suffix_x = int64_t(B) * prefill_tiles(max_q_len, G) * suffix_parts;
  dim3 grid(static_cast<unsigned>(prefix_x + suffix_x), static_cast<unsigned>(KVH), 1u);
  return launch_prefill<true>(D, f16, grid, s, q, q_stride_t, q_stride_h, k_cache, v_cache,
                              num_slots, kv_stride_slot, kv_stride_head, block_table, bt_stride,
                              log2_bs, cu_q, ctx_lens, max_ctx, G, scale_log2, P, prefix_parts,
                              tiles16_max, ws_acc, ws_ml, out, o_stride_t, o_stride_h, err_count,
                              B, prefix_tokens, prefix_parts + suffix_parts,
                              static_cast<int32_t>(prefix_x));
}

int64_t shared_prefix_grid(int32_t B, int32_t G, int32_t max_q_len, int32_t max_ctx, int32_t P,
                           int32_t prefix_tokens) {
  const int64_t tiles_p = (int64_t(B) * max_q_len * G + kRows - 1) / kRows;
  return tiles_p * (prefix_tokens / P) +
         int64_t(B) * prefill_tiles(max_q_len, G) * ((max_ctx - prefix_tokens + P - 1) / P);
}

bool shared_prefix_applies(int32_t D, int32_t block_size, int32_t B, int64_t num_slots,
                           int64_t kv_stride_slot) {
  return (D == 64 || D == 128) && block_size >= 16 && B >= 1 && B <= kMaxSharedSeqs &&
         num_slots >= 16 && kv_stride_slot < (int64_t(1) << 25);
}

}  // namespace dsp_detail
