// Byte-exact KV moves on the paged pool: append (J1), block copy (J2), transport
// gather (J5a) and scatter (J5c).  All four are HBM-bound copies: every lane moves
// VEC-byte vectors (16 B = one dwordx4 when strides allow), 64-bit offsets throughout
// (a full-size pool is far beyond 4 GiB), and each thread issues its loads before its
// stores so several vectors per lane are in flight.
#include "dsp_common.h"

namespace {

constexpr int kThreads = 256;

// Where the append kernel's stores of a row with an out-of-range slot go (their values are
// never read): one 4 KiB region per device, shared by every launch.
constexpr int kDroppedBytes = 4096;
__device__ __attribute__((aligned(16))) char g_dropped_rows[kDroppedBytes];

// ------------------------------------------------------------------------------- J1
// One group of `lanes_per_row` lanes per token row; blockIdx.y selects K (0) or V (1).
// kScatter: dense rows -> pool slots (append); otherwise pool slots -> dense rows.
// The append's lane groups take R rows each (rows g, g + rows_per_wg, ...): R = 2 for
// launches of up to kSmallAppend rows, 1 above.  Same-box A/B (cold cache, 2 KiB rows):
// 8781 rows 4.0 TB/s at R 1, 4.3 at R 2, 4.2 at R 4, 4.05 at R 8; 32768 rows 5.1-5.2 at
// R 1, 5.0 at R 2 and 4.
constexpr int64_t kSmallAppend = 16384;
template <int VEC, bool kScatter, int R>
__global__ __launch_bounds__(kThreads) void slot_rows_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t num_slots,
    int64_t pool_stride, const char* __restrict__ k, const char* __restrict__ v,
    int64_t src_stride, const int64_t* __restrict__ slots, int64_t num_tokens,
    int32_t chunks_per_row, int32_t lanes_per_row, int32_t rows_per_wg,
    int32_t* __restrict__ err_count) {
  using V = typename dsp_vec<VEC>::type;
  const int lane = threadIdx.x % lanes_per_row;
  const char* plane_src = blockIdx.y == 0 ? k : v;
  char* plane_pool = blockIdx.y == 0 ? k_pool : v_pool;
  if constexpr (kScatter) {
    // The dense source rows do not depend on the slots: each lane's first vector of its
    // R rows is loaded together with the rows' slot indices, so the launch pays
    // one memory round trip before its stores.  No branch on a slot lies between those
    // loads and their stores (the compiler would sink the loads below it): a row with a bad
    // slot, a row past the end and a lane past a row's end store into g_dropped_rows
    // instead; bad rows are counted after the stores.
    const int64_t row0 =
        int64_t(blockIdx.x) * rows_per_wg * R + threadIdx.x / lanes_per_row;
    const int c = lane;
    V first[R];
    int64_t slot[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t row = min(row0 + int64_t(i) * rows_per_wg, num_tokens - 1);
      first[i] = dsp_ld_stream(reinterpret_cast<const V*>(plane_src + row * src_stride) +
                               min(c, chunks_per_row - 1));
    }
    __builtin_amdgcn_sched_barrier(0);  // issued before the slot loads, not after their wait
#pragma unroll
    for (int i = 0; i < R; ++i)
      slot[i] = slots[min(row0 + int64_t(i) * rows_per_wg, num_tokens - 1)];
    V* const drop = reinterpret_cast<V*>(g_dropped_rows);
    constexpr int kDropMask = kDroppedBytes / VEC - 1;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t row = row0 + int64_t(i) * rows_per_wg;
      const bool live = row < num_tokens;
      const bool ok = live && slot[i] >= 0 && slot[i] < num_slots;
      bad += live && !ok;
      V* pooled = reinterpret_cast<V*>(plane_pool + (ok ? slot[i] : 0) * pool_stride);
      dsp_st_stream(first[i], ok && c < chunks_per_row ? pooled + c : drop + (c & kDropMask));
      if (ok) {  // rows longer than the lane group: the rest, one vector per lane at a time
        const V* src = reinterpret_cast<const V*>(plane_src + row * src_stride);
        for (int cc = c + lanes_per_row; cc < chunks_per_row; cc += lanes_per_row)
          dsp_st_stream(dsp_ld_stream(src + cc), pooled + cc);
      }
    }
    if (bad && lane == 0 && blockIdx.y == 0 && err_count) atomicAdd(err_count, bad);
    return;
  }
  const int64_t row = int64_t(blockIdx.x) * rows_per_wg + threadIdx.x / lanes_per_row;
  if (row >= num_tokens) return;
  const int64_t slot = slots[row];
  if (slot < 0 || slot >= num_slots) {
    if (lane == 0 && blockIdx.y == 0 && err_count) atomicAdd(err_count, 1);
    return;
  }
  const V* src = reinterpret_cast<const V*>(plane_pool + slot * pool_stride);
  V* dst = reinterpret_cast<V*>(const_cast<char*>(plane_src) + row * src_stride);
  // Full rounds: U vectors per lane, all loads issued before the stores.
  constexpr int U = 4;
  int c = lane;
  for (; c + (U - 1) * lanes_per_row < chunks_per_row; c += U * lanes_per_row) {
    V buf[U];
#pragma unroll
    for (int u = 0; u < U; ++u) buf[u] = dsp_ld_stream(src + c + u * lanes_per_row);
#pragma unroll
    for (int u = 0; u < U; ++u) dsp_st_stream(buf[u], dst + c + u * lanes_per_row);
  }
  for (; c < chunks_per_row; c += lanes_per_row) dsp_st_stream(dsp_ld_stream(src + c), dst + c);
}

// A one-shot workgroup per 4 KiB piece: each thread loads its 4 KiB / (256 * VEC) vectors,
// stores them and exits.  On gfx950 this beats a workgroup per whole 32 KiB block with
// eight vectors per thread by 11 % on the transport gather and scatter (6.22 against 5.58
// and 5.78 against 5.22 TB/s at 8 x 4096 tokens of 28/36 layers); block copies between
// random blocks run at the same ~5.2 TB/s either way (random destinations bound them).
constexpr int64_t kPiece = 4096;

template <int VEC>
__device__ __forceinline__ void piece_copy(const char* __restrict__ src, char* __restrict__ dst,
                                           int64_t bytes) {
  using V = typename dsp_vec<VEC>::type;
  constexpr int U = int(kPiece / (kThreads * VEC));
  const int64_t n = bytes / VEC;
  const V* s = reinterpret_cast<const V*>(src);
  V* d = reinterpret_cast<V*>(dst);
  V buf[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (threadIdx.x + u * kThreads < n) buf[u] = dsp_ld_stream(s + threadIdx.x + u * kThreads);
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (threadIdx.x + u * kThreads < n) dsp_st_stream(buf[u], d + threadIdx.x + u * kThreads);
}

// ------------------------------------------------------------------------------- J2
// grid = (num_pairs * pieces per block, num_layers, 2 planes): one 4 KiB piece of one
// block of one layer per workgroup.
template <int VEC>
__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(
    const char* __restrict__ src_k, const char* __restrict__ src_v, int64_t src_layer_stride,
    int64_t src_num_blocks, char* __restrict__ dst_k, char* __restrict__ dst_v,
    int64_t dst_layer_stride, int64_t dst_num_blocks, int64_t block_bytes,
    const int32_t* __restrict__ src_blocks, const int32_t* __restrict__ dst_blocks,
    int32_t pieces_per_block, int32_t* __restrict__ err_count) {
  const int64_t p = blockIdx.x / pieces_per_block;
  const int64_t off = (blockIdx.x % pieces_per_block) * kPiece;
  const int64_t s = src_blocks[p], d = dst_blocks[p];
  if (s < 0 || s >= src_num_blocks || d < 0 || d >= dst_num_blocks) {
    if (threadIdx.x == 0 && off == 0 && blockIdx.y == 0 && blockIdx.z == 0 && err_count)
      atomicAdd(err_count, 1);
    return;
  }
  const int64_t l = blockIdx.y;
  const char* src =
      (blockIdx.z == 0 ? src_k : src_v) + l * src_layer_stride + s * block_bytes + off;
  char* dst = (blockIdx.z == 0 ? dst_k : dst_v) + l * dst_layer_stride + d * block_bytes + off;
  piece_copy<VEC>(src, dst, min(kPiece, block_bytes - off));
}

// grid = (ceil(num_dst / kFanOut) * pieces per block, num_layers, 2 planes): one 4 KiB
// piece of the source block, copied to kFanOut destinations.  Each thread loads its
// vectors of the piece once and stores them kFanOut times (the fork of one block into
// many sequences reads the source once per kFanOut copies, not once per copy).  The
// destination ids come in one round trip: lane i loads id i, every wave reads them back as
// scalars; ids past num_dst or out of range store nothing (an out-of-range id is counted).
constexpr int kFanOut = 8;
template <int VEC>
__global__ __launch_bounds__(kThreads) void fanout_block_kernel(
    const char* __restrict__ src_k, const char* __restrict__ src_v, int64_t src_layer_stride,
    char* __restrict__ dst_k, char* __restrict__ dst_v, int64_t dst_layer_stride,
    int64_t dst_num_blocks, int64_t block_bytes, int64_t src_block,
    const int32_t* __restrict__ dst_blocks, int64_t num_dst, int32_t pieces_per_block,
    int32_t* __restrict__ err_count) {
  using V = typename dsp_vec<VEC>::type;
  constexpr int U = int(kPiece / (kThreads * VEC));
  const int64_t g = blockIdx.x / pieces_per_block;
  const int64_t off = (blockIdx.x % pieces_per_block) * kPiece;
  const int64_t l = blockIdx.y;
  const int64_t n = min(kPiece, block_bytes - off) / VEC;
  const int64_t il = min(g * kFanOut + (threadIdx.x & (kFanOut - 1)), num_dst - 1);
  const int32_t db_l = dst_blocks[il];
  const V* src = reinterpret_cast<const V*>((blockIdx.z == 0 ? src_k : src_v) +
                                            l * src_layer_stride + src_block * block_bytes + off);
  char* dbase = (blockIdx.z == 0 ? dst_k : dst_v) + l * dst_layer_stride + off;
  V buf[U];
#pragma unroll
  for (int u = 0; u < U; ++u) buf[u] = dsp_ld_stream(src + min(int64_t(threadIdx.x + u * kThreads), n - 1));
#pragma unroll
  for (int p = 0; p < kFanOut; ++p) {
    const int64_t db = __builtin_amdgcn_readlane(db_l, p);
    const bool in = g * kFanOut + p < num_dst;
    const bool ok = db >= 0 && db < dst_num_blocks;
    if (in && !ok && threadIdx.x == 0 && off == 0 && l == 0 && blockIdx.z == 0 && err_count)
      atomicAdd(err_count, 1);
    V* dst = reinterpret_cast<V*>(dbase + (in && ok ? db : 0) * block_bytes);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (in && ok && threadIdx.x + u * kThreads < n)
        dsp_st_stream(buf[u], dst + threadIdx.x + u * kThreads);
  }
}

// --------------------------------------------------------------------------- J5a/J5c
// grid = (max blocks per sequence * pieces per block, num_layers, 2 * num_seqs).  Block j
// of sequence b in layer l covers tokens [j*bs, min((j+1)*bs, T_b)): contiguous in the pool
// (one block) and contiguous in the transport buffer, so it is one segment, copied in
// 4 KiB pieces.
template <int VEC, bool kGather>
__global__ __launch_bounds__(kThreads) void transport_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t layer_stride,
    int64_t num_blocks, int64_t row_bytes, int32_t log2_bs,
    const int32_t* __restrict__ block_tables, int64_t bt_stride,
    const int64_t* __restrict__ cu_seqlens, int64_t num_layers, char* __restrict__ k_buf,
    char* __restrict__ v_buf, int32_t pieces_per_block, int32_t* __restrict__ err_count) {
  const int64_t j = blockIdx.x / pieces_per_block;
  const int64_t off = (blockIdx.x % pieces_per_block) * kPiece;
  const int64_t l = blockIdx.y;
  const int b = blockIdx.z >> 1;
  const int plane = blockIdx.z & 1;
  // The block id does not depend on the lengths (j < bt_stride: the launch covers at most
  // ceil(max_seqlen / bs) blocks per sequence): it is loaded beside them, and one branch
  // tests both, so the copy starts one memory round trip after the workgroup does.
  const int64_t blk = block_tables[int64_t(b) * bt_stride + j];
  const int64_t t0 = cu_seqlens[b];
  const int64_t T = cu_seqlens[b + 1] - t0;
  const int64_t first = j << log2_bs;
  const int64_t seg = first < T ? min(int64_t(1) << log2_bs, T - first) * row_bytes : 0;
  if (off >= seg || blk < 0 || blk >= num_blocks) {
    if (off < seg && threadIdx.x == 0 && off == 0 && l == 0 && plane == 0 && err_count)
      atomicAdd(err_count, 1);
    return;
  }
  char* pool = (plane == 0 ? k_pool : v_pool) + l * layer_stride +
               (blk << log2_bs) * row_bytes + off;
  char* buf = (plane == 0 ? k_buf : v_buf) + (num_layers * t0 + l * T + first) * row_bytes + off;
  const int64_t bytes = min(kPiece, seg - off);
  if constexpr (kGather)
    piece_copy<VEC>(pool, buf, bytes);
  else
    piece_copy<VEC>(buf, pool, bytes);
}

// ------------------------------------------------------------------ J5c, by destination
// The scatter with its workgroups in physical-block order.  Sequence order makes the pool
// writes land on random blocks (the tables are scattered over the pool); visited by
// destination block, the writes run through each layer in address order and the reads
// (32 KiB runs of the contiguous transport buffer) become the random side -- the gather's
// pattern, whose random side is the cheaper one to make random.  owner[p] = b * nblk + j
// for the table entry (b, j) naming block p (-1: none); two entries naming one block are
// resolved to the later one in table order, as a sequential import would leave it.
__global__ __launch_bounds__(256) void block_owner_fill_kernel(int32_t* __restrict__ owner,
                                                               int64_t num_blocks) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < num_blocks) owner[i] = -1;
}

__global__ __launch_bounds__(256) void block_owner_kernel(
    int32_t* __restrict__ owner, int64_t num_blocks, const int32_t* __restrict__ block_tables,
    int64_t bt_stride, const int64_t* __restrict__ cu_seqlens, int32_t num_seqs,
    int32_t log2_bs, int64_t nblk, int32_t* __restrict__ err_count) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= num_seqs * nblk) return;
  const int b = int(i / nblk);
  const int64_t j = i - int64_t(b) * nblk;
  if ((j << log2_bs) >= cu_seqlens[b + 1] - cu_seqlens[b]) return;   // no tokens here
  const int32_t blk = block_tables[int64_t(b) * bt_stride + j];
  if (blk < 0 || blk >= num_blocks) {
    if (err_count) atomicAdd(err_count, 1);
    return;
  }
  atomicMax(owner + blk, int32_t(i));
}

// grid = (num_blocks * pieces per block, num_layers, 2 planes); block p's rows come from
// the transport buffer segment of its owner (b, j), exactly as transport_kernel copies them.
template <int VEC>
__global__ __launch_bounds__(kThreads) void scatter_by_block_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t layer_stride,
    int64_t row_bytes, int32_t log2_bs, const int64_t* __restrict__ cu_seqlens,
    int64_t num_layers, const char* __restrict__ k_buf, const char* __restrict__ v_buf,
    int32_t pieces_per_block, const int32_t* __restrict__ owner, int64_t nblk) {
  const int64_t p = blockIdx.x / pieces_per_block;
  const int64_t off = (blockIdx.x % pieces_per_block) * kPiece;
  const int64_t l = blockIdx.y;
  const int plane = blockIdx.z;
  const int32_t own = owner[p];
  if (own < 0) return;
  const int b = int(own / nblk);
  const int64_t j = own - int64_t(b) * nblk;
  const int64_t t0 = cu_seqlens[b];
  const int64_t T = cu_seqlens[b + 1] - t0;
  const int64_t first = j << log2_bs;
  const int64_t seg = min(int64_t(1) << log2_bs, T - first) * row_bytes;   // > 0: j has tokens
  if (off >= seg) return;
  char* pool = (plane == 0 ? k_pool : v_pool) + l * layer_stride + (p << log2_bs) * row_bytes + off;
  const char* buf =
      (plane == 0 ? k_buf : v_buf) + (num_layers * t0 + l * T + first) * row_bytes + off;
  piece_copy<VEC>(buf, pool, min(kPiece, seg - off));
}

template <bool kGather>
int launch_transport(void* k_pool, void* v_pool, int64_t num_layers, int64_t layer_stride,
                     int64_t num_blocks, int64_t row_bytes, int32_t block_size,
                     const int32_t* block_tables, int64_t bt_stride, const int64_t* cu_seqlens,
                     int32_t num_seqs, int64_t max_seqlen, void* k_buf, void* v_buf,
                     int32_t* err_count, hipStream_t stream) {
  DSP_HOST_CHECK(k_pool && v_pool && k_buf && v_buf && block_tables && cu_seqlens, DSP_EINVAL);
  DSP_HOST_CHECK(num_layers > 0 && num_layers <= 65535 && num_blocks > 0 && row_bytes > 0 &&
                     num_seqs >= 0 && 2 * int64_t(num_seqs) <= 65535 && max_seqlen >= 0,
                 DSP_EINVAL);
  DSP_HOST_CHECK(dsp_is_pow2(block_size), DSP_EINVAL);
  DSP_HOST_CHECK(bt_stride * block_size >= max_seqlen, DSP_EINVAL);
  DSP_HOST_CHECK(layer_stride >= num_blocks * block_size * row_bytes, DSP_EINVAL);
  if (num_seqs == 0 || max_seqlen == 0) return DSP_OK;
  const int vec = dsp_vec_width({row_bytes, layer_stride, int64_t(reinterpret_cast<uintptr_t>(k_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(v_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(k_buf)),
                                 int64_t(reinterpret_cast<uintptr_t>(v_buf))});
  const int64_t nblk = (max_seqlen + block_size - 1) / block_size;
  const int64_t ppb = (block_size * row_bytes + kPiece - 1) / kPiece;
  DSP_HOST_CHECK(nblk * ppb < (int64_t(1) << 31), DSP_EINVAL);
  dim3 grid(static_cast<unsigned>(nblk * ppb), static_cast<unsigned>(num_layers),
            2u * num_seqs);
  const int32_t lbs = dsp_log2i(block_size);
  char* kp = static_cast<char*>(k_pool);
  char* vp = static_cast<char*>(v_pool);
  char* kb = static_cast<char*>(k_buf);
  char* vb = static_cast<char*>(v_buf);
#define DSP_TRANSPORT(V)                                                                      \
  transport_kernel<V, kGather><<<grid, kThreads, 0, stream>>>(                                \
      kp, vp, layer_stride, num_blocks, row_bytes, lbs, block_tables, bt_stride, cu_seqlens, \
      num_layers, kb, vb, static_cast<int32_t>(ppb), err_count)
  switch (vec) {
    case 16: DSP_TRANSPORT(16); break;
    case 8: DSP_TRANSPORT(8); break;
    case 4: DSP_TRANSPORT(4); break;
    case 2: DSP_TRANSPORT(2); break;
    default: DSP_TRANSPORT(1); break;
  }
#undef DSP_TRANSPORT
  return dsp_launch_status();
}

// The scatter in destination-block order when the tables can name at least half the pool's
// blocks (its grid covers every block of the pool, so a small import into a large pool
// keeps the sequence-order kernel).  Same-box A/B, config 5 (8 x 4096 tokens into a pool
// 1.25x their blocks, 36 layers): 1550-1565 against 1662-1667 us.
int launch_scatter_ordered(void* k_pool, void* v_pool, int64_t num_layers, int64_t layer_stride,
                           int64_t num_blocks, int64_t row_bytes, int32_t block_size,
                           const int32_t* block_tables, int64_t bt_stride,
                           const int64_t* cu_seqlens, int32_t num_seqs, int64_t max_seqlen,
                           const void* k_buf, const void* v_buf, int32_t* block_owner,
                           int32_t* err_count, hipStream_t stream) {
  DSP_HOST_CHECK(block_owner, DSP_EINVAL);
  DSP_HOST_CHECK(num_blocks > 0 && num_seqs >= 0 && max_seqlen >= 0 && dsp_is_pow2(block_size),
                 DSP_EINVAL);
  const int64_t nblk = (max_seqlen + block_size - 1) / block_size;
  const int64_t ppb = (block_size * row_bytes + kPiece - 1) / kPiece;
  const bool ordered = 2 * int64_t(num_seqs) * nblk >= num_blocks &&
                       int64_t(num_seqs) * nblk < (int64_t(1) << 31) &&
                       num_blocks * ppb < (int64_t(1) << 31);
  if (!ordered)
    return launch_transport<false>(k_pool, v_pool, num_layers, layer_stride, num_blocks,
                                   row_bytes, block_size, block_tables, bt_stride, cu_seqlens,
                                   num_seqs, max_seqlen, const_cast<void*>(k_buf),
                                   const_cast<void*>(v_buf), err_count, stream);
  // the same argument checks as the sequence-order kernel
  DSP_HOST_CHECK(k_pool && v_pool && k_buf && v_buf && block_tables && cu_seqlens, DSP_EINVAL);
  DSP_HOST_CHECK(num_layers > 0 && num_layers <= 65535 && row_bytes > 0, DSP_EINVAL);
  DSP_HOST_CHECK(bt_stride * block_size >= max_seqlen, DSP_EINVAL);
  DSP_HOST_CHECK(layer_stride >= num_blocks * block_size * row_bytes, DSP_EINVAL);
  if (num_seqs == 0 || max_seqlen == 0) return DSP_OK;
  const int vec = dsp_vec_width({row_bytes, layer_stride, int64_t(reinterpret_cast<uintptr_t>(k_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(v_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(k_buf)),
                                 int64_t(reinterpret_cast<uintptr_t>(v_buf))});
  const int32_t lbs = dsp_log2i(block_size);
  block_owner_fill_kernel<<<static_cast<unsigned>((num_blocks + 255) / 256), 256, 0, stream>>>(
      block_owner, num_blocks);
  block_owner_kernel<<<static_cast<unsigned>((num_seqs * nblk + 255) / 256), 256, 0, stream>>>(
      block_owner, num_blocks, block_tables, bt_stride, cu_seqlens, num_seqs, lbs, nblk,
      err_count);
  dim3 grid(static_cast<unsigned>(num_blocks * ppb), static_cast<unsigned>(num_layers), 2u);
  char* kp = static_cast<char*>(k_pool);
  char* vp = static_cast<char*>(v_pool);
  const char* kb = static_cast<const char*>(k_buf);
  const char* vb = static_cast<const char*>(v_buf);
#define DSP_BY_BLOCK(V)                                                                     \
  scatter_by_block_kernel<V><<<grid, kThreads, 0, stream>>>(kp, vp, layer_stride, row_bytes, \
                                                            lbs, cu_seqlens, num_layers, kb, \
                                                            vb, static_cast<int32_t>(ppb),   \
                                                            block_owner, nblk)
  switch (vec) {
    case 16: DSP_BY_BLOCK(16); break;
    case 8: DSP_BY_BLOCK(8); break;
    case 4: DSP_BY_BLOCK(4); break;
    case 2: DSP_BY_BLOCK(2); break;
    default: DSP_BY_BLOCK(1); break;
  }
#undef DSP_BY_BLOCK
  return dsp_launch_status();
}

}  // namespace

namespace {

template <bool kScatter>
int launch_slot_rows(void* k_pool, void* v_pool, int64_t num_slots, int64_t pool_stride,
                     const void* k, const void* v, int64_t dense_stride, const int64_t* slots,
                     int64_t num_tokens, int64_t row_bytes, int32_t* err_count,
                     hipStream_t s) {
  DSP_HOST_CHECK(k_pool && v_pool && k && v && (slots || num_tokens == 0), DSP_EINVAL);
  DSP_HOST_CHECK(num_slots >= 0 && num_tokens >= 0 && row_bytes > 0, DSP_EINVAL);
  DSP_HOST_CHECK(pool_stride >= row_bytes && dense_stride >= 0, DSP_EINVAL);
  if (num_tokens == 0) return DSP_OK;
  const int vec = dsp_vec_width({row_bytes, pool_stride, dense_stride,
                                 int64_t(reinterpret_cast<uintptr_t>(k_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(v_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(k)),
                                 int64_t(reinterpret_cast<uintptr_t>(v))});
  const int64_t chunks = row_bytes / vec;
  DSP_HOST_CHECK(chunks < (int64_t(1) << 30), DSP_EINVAL);
  int lanes = 1;
  while (lanes < chunks && lanes < kThreads) lanes <<= 1;
  const int rows_per_wg = kThreads / lanes;
  const int R = kScatter && num_tokens <= kSmallAppend ? 2 : 1;
  const int64_t nwg = (num_tokens + int64_t(rows_per_wg) * R - 1) / (int64_t(rows_per_wg) * R);
  DSP_HOST_CHECK(nwg < (int64_t(1) << 31), DSP_EINVAL);
  dim3 grid(static_cast<unsigned>(nwg), 2u, 1u);
  char* kp = static_cast<char*>(k_pool);
  char* vp = static_cast<char*>(v_pool);
  const char* kd = static_cast<const char*>(k);
  const char* vd = static_cast<const char*>(v);
#define DSP_ROWS(V)                                                                          \
  if (R == 2)                                                                                \
    slot_rows_kernel<V, kScatter, 2><<<grid, kThreads, 0, s>>>(                              \
        kp, vp, num_slots, pool_stride, kd, vd, dense_stride, slots, num_tokens,             \
        static_cast<int32_t>(chunks), lanes, rows_per_wg, err_count);                        \
  else                                                                                       \
    slot_rows_kernel<V, kScatter, 1><<<grid, kThreads, 0, s>>>(                              \
        kp, vp, num_slots, pool_stride, kd, vd, dense_stride, slots, num_tokens,             \
        static_cast<int32_t>(chunks), lanes, rows_per_wg, err_count)
  switch (vec) {
    case 16: DSP_ROWS(16); break;
    case 8: DSP_ROWS(8); break;
    case 4: DSP_ROWS(4); break;
    case 2: DSP_ROWS(2); break;
    default: DSP_ROWS(1); break;
  }
#undef DSP_ROWS
  return dsp_launch_status();
}

}  // namespace

extern "C" int dsp_kv_append(void* k_pool, void* v_pool, int64_t num_slots,
                             int64_t pool_slot_stride_bytes, const void* k, const void* v,
                             int64_t src_token_stride_bytes, const int64_t* slots,
                             int64_t num_tokens, int64_t row_bytes, int32_t* err_count,
                             dsp_stream_t stream) {
  return launch_slot_rows<true>(k_pool, v_pool, num_slots, pool_slot_stride_bytes, k, v,
                                src_token_stride_bytes, slots, num_tokens, row_bytes,
                                err_count, static_cast<hipStream_t>(stream));
}

extern "C" int dsp_kv_gather_slots(const void* k_pool, const void* v_pool, int64_t num_slots,
                                   int64_t pool_slot_stride_bytes, const int64_t* slots,
                                   int64_t num_tokens, int64_t row_bytes, void* k_out,
                                   void* v_out, int64_t out_token_stride_bytes,
                                   int32_t* err_count, dsp_stream_t stream) {
  return launch_slot_rows<false>(const_cast<void*>(k_pool), const_cast<void*>(v_pool),
                                 num_slots, pool_slot_stride_bytes, k_out, v_out,
                                 out_token_stride_bytes, slots, num_tokens, row_bytes,
                                 err_count, static_cast<hipStream_t>(stream));
}

extern "C" int dsp_kv_copy_blocks(const void* src_k_pool, const void* src_v_pool,
                                  int64_t src_layer_stride_bytes, int64_t src_num_blocks,
                                  void* dst_k_pool, void* dst_v_pool,
                                  int64_t dst_layer_stride_bytes, int64_t dst_num_blocks,
                                  int64_t num_layers, int64_t block_bytes,
                                  const int32_t* src_blocks, const int32_t* dst_blocks,
                                  int64_t num_pairs, int32_t* err_count, dsp_stream_t stream) {
  DSP_HOST_CHECK(src_k_pool && src_v_pool && dst_k_pool && dst_v_pool, DSP_EINVAL);
  DSP_HOST_CHECK((src_blocks && dst_blocks) || num_pairs == 0, DSP_EINVAL);
  DSP_HOST_CHECK(num_layers > 0 && num_layers <= 65535 && src_num_blocks >= 0 &&
                     dst_num_blocks >= 0 && block_bytes > 0 && num_pairs >= 0 &&
                     num_pairs < (int64_t(1) << 31),
                 DSP_EINVAL);
  DSP_HOST_CHECK(src_layer_stride_bytes >= src_num_blocks * block_bytes &&
                     dst_layer_stride_bytes >= dst_num_blocks * block_bytes,
                 DSP_EINVAL);
  if (num_pairs == 0) return DSP_OK;
  const int vec = dsp_vec_width({block_bytes, src_layer_stride_bytes, dst_layer_stride_bytes,
                                 int64_t(reinterpret_cast<uintptr_t>(src_k_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(src_v_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(dst_k_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(dst_v_pool))});
  const int64_t ppb = (block_bytes + kPiece - 1) / kPiece;
  DSP_HOST_CHECK(num_pairs * ppb < (int64_t(1) << 31), DSP_EINVAL);
  dim3 grid(static_cast<unsigned>(num_pairs * ppb), static_cast<unsigned>(num_layers), 2u);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* sk = static_cast<const char*>(src_k_pool);
  const char* sv = static_cast<const char*>(src_v_pool);
  char* dk = static_cast<char*>(dst_k_pool);
  char* dv = static_cast<char*>(dst_v_pool);
#define DSP_COPY(V)                                                                        \
  copy_blocks_kernel<V><<<grid, kThreads, 0, s>>>(sk, sv, src_layer_stride_bytes,          \
                                                  src_num_blocks, dk, dv,                  \
                                                  dst_layer_stride_bytes, dst_num_blocks,  \
                                                  block_bytes, src_blocks, dst_blocks,     \
                                                  static_cast<int32_t>(ppb), err_count)
  switch (vec) {
    case 16: DSP_COPY(16); break;
    case 8: DSP_COPY(8); break;
    case 4: DSP_COPY(4); break;
    case 2: DSP_COPY(2); break;
    default: DSP_COPY(1); break;
  }
#undef DSP_COPY
  return dsp_launch_status();
}

extern "C" int dsp_kv_copy_block_fanout(const void* src_k_pool, const void* src_v_pool,
                                        int64_t src_layer_stride_bytes, int64_t src_num_blocks,
                                        void* dst_k_pool, void* dst_v_pool,
                                        int64_t dst_layer_stride_bytes, int64_t dst_num_blocks,
                                        int64_t num_layers, int64_t block_bytes,
                                        int32_t src_block, const int32_t* dst_blocks,
                                        int64_t num_dst, int32_t* err_count,
                                        dsp_stream_t stream) {
  DSP_HOST_CHECK(src_k_pool && src_v_pool && dst_k_pool && dst_v_pool, DSP_EINVAL);
  DSP_HOST_CHECK(dst_blocks || num_dst == 0, DSP_EINVAL);
  DSP_HOST_CHECK(num_layers > 0 && num_layers <= 65535 && src_num_blocks >= 0 &&
                     dst_num_blocks >= 0 && block_bytes > 0 && num_dst >= 0 &&
                     num_dst < (int64_t(1) << 31),
                 DSP_EINVAL);
  DSP_HOST_CHECK(src_layer_stride_bytes >= src_num_blocks * block_bytes &&
                     dst_layer_stride_bytes >= dst_num_blocks * block_bytes,
                 DSP_EINVAL);
  if (num_dst == 0) return DSP_OK;
  // the source id is a host value: checked here, not counted
  DSP_HOST_CHECK(src_block >= 0 && src_block < src_num_blocks, DSP_EINVAL);
  const int vec = dsp_vec_width({block_bytes, src_layer_stride_bytes, dst_layer_stride_bytes,
                                 int64_t(reinterpret_cast<uintptr_t>(src_k_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(src_v_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(dst_k_pool)),
                                 int64_t(reinterpret_cast<uintptr_t>(dst_v_pool))});
  const int64_t ppb = (block_bytes + kPiece - 1) / kPiece;
  const int64_t groups = (num_dst + kFanOut - 1) / kFanOut;
  DSP_HOST_CHECK(groups * ppb < (int64_t(1) << 31), DSP_EINVAL);
  dim3 grid(static_cast<unsigned>(groups * ppb), static_cast<unsigned>(num_layers), 2u);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* sk = static_cast<const char*>(src_k_pool);
  const char* sv = static_cast<const char*>(src_v_pool);
  char* dk = static_cast<char*>(dst_k_pool);
  char* dv = static_cast<char*>(dst_v_pool);
#define DSP_FAN(V)                                                                         \
  fanout_block_kernel<V><<<grid, kThreads, 0, s>>>(sk, sv, src_layer_stride_bytes, dk, dv,  \
                                                   dst_layer_stride_bytes, dst_num_blocks,  \
                                                   block_bytes, src_block, dst_blocks,      \
                                                   num_dst, static_cast<int32_t>(ppb),      \
                                                   err_count)
  switch (vec) {
    case 16: DSP_FAN(16); break;
    case 8: DSP_FAN(8); break;
    case 4: DSP_FAN(4); break;
    case 2: DSP_FAN(2); break;
    default: DSP_FAN(1); break;
  }
#undef DSP_FAN
  return dsp_launch_status();
}

extern "C" int dsp_kv_gather(const void* k_pool, const void* v_pool, int64_t num_layers,
                             int64_t pool_layer_stride_bytes, int64_t num_blocks,
                             int64_t row_bytes, int32_t block_size,
                             const int32_t* block_tables, int64_t bt_stride,
                             const int64_t* cu_seqlens, int32_t num_seqs, int64_t max_seqlen,
                             void* k_buf, void* v_buf, int32_t* err_count,
                             dsp_stream_t stream) {
  return launch_transport<true>(const_cast<void*>(k_pool), const_cast<void*>(v_pool),
                                num_layers, pool_layer_stride_bytes, num_blocks, row_bytes,
                                block_size, block_tables, bt_stride, cu_seqlens, num_seqs,
                                max_seqlen, k_buf, v_buf, err_count,
                                static_cast<hipStream_t>(stream));
}

extern "C" int dsp_kv_scatter(void* k_pool, void* v_pool, int64_t num_layers,
                              int64_t pool_layer_stride_bytes, int64_t num_blocks,
                              int64_t row_bytes, int32_t block_size,
                              const int32_t* block_tables, int64_t bt_stride,
                              const int64_t* cu_seqlens, int32_t num_seqs, int64_t max_seqlen,
                              const void* k_buf, const void* v_buf, int32_t* err_count,
                              dsp_stream_t stream) {
  return launch_transport<false>(k_pool, v_pool, num_layers, pool_layer_stride_bytes,
                                 num_blocks, row_bytes, block_size, block_tables, bt_stride,
                                 cu_seqlens, num_seqs, max_seqlen, const_cast<void*>(k_buf),
                                 const_cast<void*>(v_buf), err_count,
                                 static_cast<hipStream_t>(stream));
}

extern "C" int dsp_kv_scatter_ordered(void* k_pool, void* v_pool, int64_t num_layers,
                                      int64_t pool_layer_stride_bytes, int64_t num_blocks,
                                      int64_t row_bytes, int32_t block_size,
                                      const int32_t* block_tables, int64_t bt_stride,
                                      const int64_t* cu_seqlens, int32_t num_seqs,
                                      int64_t max_seqlen, const void* k_buf, const void* v_buf,
                                      int32_t* block_owner, int32_t* err_count,
                                      dsp_stream_t stream) {
  return launch_scatter_ordered(k_pool, v_pool, num_layers, pool_layer_stride_bytes, num_blocks,
                                row_bytes, block_size, block_tables, bt_stride, cu_seqlens,
                                num_seqs, max_seqlen, k_buf, v_buf, block_owner, err_count,
                                static_cast<hipStream_t>(stream));
}
