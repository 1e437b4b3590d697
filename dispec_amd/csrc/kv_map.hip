// J5b: the cross-model KV map -- an MFMA GEMM whose A operand is the design row
// gathered from several source layers, with epilogues that round exactly where the
// reference's bf16 torch ops round, plus the fp32 RoPE strip/apply pass.
//
// Reference: CrossModelKVMap.map/_apply and LayerMap.apply (dispec/kv/transfer.py:
// 243-283, 104-112), strip_rope/apply_rope (:66-80).
//
// GEMM: C[M, N] = epilogue(A[M, K] . Bt[N, K]^T), bf16 in, fp32 accumulate.
//  * A row m, column k lives at a + seg_off[k / seg_len] + m * lda + k % seg_len: the
//    design row of transfer.py:249 (source layers in map order, each a KVH*D row) is
//    read straight from the contiguous source buffer, never materialised.
//  * Bt is the weight stored N x K (K contiguous): W^T for x @ W (transposed once when
//    the map is loaded), or the F.linear weight itself.
//  * 128 x 128 output tile per 256-thread workgroup, 64 x 64 per wave as 4 x 4
//    v_mfma_f32_16x16x32 tiles, K in steps of 32 staged through double-buffered LDS
//    (row pitch padded to 40 elements: the 16-byte fragment reads are conflict-free).
//  * Epilogue, per element, in the order the reference rounds:
//      acc -> [bias mode 1: bf16(bf16(acc) + b)  (x @ W + b, two bf16 ops)]
//             [bias mode 2: bf16(acc + b)        (F.linear / addmm, one rounding)]
//             [bias mode 0: bf16(acc)]
//          -> [act 1: bf16(gelu(y)), exact erf form]
//          -> [accumulate: bf16(c_old + y)]
#include <math.h>

#include "dsp_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int PITCH = BK + 8;  // LDS row pitch in bf16 elements
constexpr int kMaxSegments = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct SegOffsets {
  int64_t off[kMaxSegments];
  // Offset of segment i without dynamic indexing (which would put the array in scratch).
  __device__ __forceinline__ int64_t get(int64_t i) const {
    int64_t r = off[0];
#pragma unroll
    for (int j = 1; j < kMaxSegments; ++j) r = (i == j) ? off[j] : r;
    return r;
  }
};

__device__ __forceinline__ float bf16_round(float x) {
  return __uint_as_float(uint32_t(dsp_f32_to_bf16(x)) << 16);
}

// Bias of the four consecutive columns nb..nb+3 (clipped at N) as floats: one 8-byte load
// when it can, so an epilogue issues its bias loads together instead of one short load and
// one wait per element.
__device__ __forceinline__ void load_bias4(const uint16_t* __restrict__ bias, int64_t nb, int64_t N,
                                           float b4[4]) {
  if (nb + 3 < N && dsp_aligned(bias + nb, 8)) {
    const dsp_u32x2 u = *reinterpret_cast<const dsp_u32x2*>(bias + nb);
    b4[0] = dsp_bf16lo(u[0]);
    b4[1] = dsp_bf16hi(u[0]);
    b4[2] = dsp_bf16lo(u[1]);
    b4[3] = dsp_bf16hi(u[1]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) b4[e] = nb + e < N ? dsp_bf16lo(bias[nb + e]) : 0.f;
  }
}

// Bias and activation of one output, in the order the reference rounds (see the header
// comment); the result is a bf16 value held in a float.  Accumulation into C comes after.
__device__ __forceinline__ float epi_bias_act(float y, float b, int32_t bias_mode, int32_t act) {
  if (bias_mode == 1) {
    y = bf16_round(bf16_round(y) + b);
  } else if (bias_mode == 2) {
    y = bf16_round(y + b);
  } else {
    y = bf16_round(y);
  }
  if (act == 1) y = bf16_round(0.5f * y * (1.f + erff(y * 0.70710678118654752f)));
  return y;
}

// Epilogue of four consecutive outputs (row crow, columns nb..nb+3, clipped at N) in the
// order the reference rounds (see the header comment); b4 is their bias (bias_mode != 0).
__device__ __forceinline__ void store_c4(const f32x4& v, uint16_t* __restrict__ crow, int64_t nb,
                                         int64_t N, const float b4[4], int32_t bias_mode,
                                         int32_t act, int32_t accumulate) {
  // (the callers pass compile-time flags where they can, which prunes the branches)
  uint16_t* dst = crow + nb;
  const bool full = nb + 3 < N && dsp_aligned(dst, 8);
  uint16_t old[4] = {0, 0, 0, 0};
  if (accumulate) {
    if (full) {
      const dsp_u32x2 u = *reinterpret_cast<const dsp_u32x2*>(dst);
      old[0] = uint16_t(u[0]);
      old[1] = uint16_t(u[0] >> 16);
      old[2] = uint16_t(u[1]);
      old[3] = uint16_t(u[1] >> 16);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nb + e < N) old[e] = dst[e];
    }
  }
  uint16_t ybits[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float y = epi_bias_act(v[e], b4[e], bias_mode, act);
    if (accumulate) y = bf16_round(dsp_bf16lo(old[e]) + y);
    ybits[e] = dsp_f32_to_bf16(y);
  }
  if (full) {
    *reinterpret_cast<dsp_u32x2*>(dst) = dsp_u32x2{uint32_t(ybits[0]) | (uint32_t(ybits[1]) << 16),
                                                uint32_t(ybits[2]) | (uint32_t(ybits[3]) << 16)};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (nb + e < N) dst[e] = ybits[e];
  }
}

// Load the 16-byte chunk (8 elements) of A or Bt at (row, k); zero outside the matrix.
// kVec: `base` already points at the K tile's segment (the tile never straddles two)
// and `k` is the column inside it.  Otherwise column k is element k % seg_len of
// segment k / seg_len and each element is fetched on its own (small, unaligned maps).
template <bool kVec>
__device__ __forceinline__ dsp_u32x4 load_chunk(const uint16_t* __restrict__ base,
                                            const SegOffsets& seg, int64_t seg_len, int64_t ld,
                                            int64_t row, int64_t rows, int64_t k, int64_t kabs,
                                            int64_t K) {
  if (row >= rows || kabs >= K) return dsp_u32x4{0u, 0u, 0u, 0u};
  if constexpr (kVec) {
    return *reinterpret_cast<const dsp_u32x4*>(base + k + row * ld);
  } else {
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t kk = kabs + i;
      const int64_t s = kk / seg_len;
      e[i] = kk < K ? base[seg.off[s] + (kk - s * seg_len) + row * ld] : uint16_t(0);
    }
    return dsp_u32x4{uint32_t(e[0]) | (uint32_t(e[1]) << 16), uint32_t(e[2]) | (uint32_t(e[3]) << 16),
                      uint32_t(e[4]) | (uint32_t(e[5]) << 16), uint32_t(e[6]) | (uint32_t(e[7]) << 16)};
  }
}

template <bool kVec>
__global__ __launch_bounds__(kThreads) void map_gemm_kernel(
    const uint16_t* __restrict__ a, SegOffsets a_seg, int64_t a_seg_len, int64_t lda,
    const uint16_t* __restrict__ bt, int64_t ldb, uint16_t* __restrict__ c, int64_t ldc,
    int64_t M, int64_t N, int64_t K, const uint16_t* __restrict__ bias, int32_t bias_mode,
    int32_t act, int32_t accumulate, int64_t a_batch_stride, int64_t c_batch_stride) {
  __shared__ uint16_t sa[2][BM][PITCH];
  a += int64_t(blockIdx.z) * a_batch_stride;
  c += int64_t(blockIdx.z) * c_batch_stride;
  __shared__ uint16_t sb[2][BN][PITCH];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = int64_t(blockIdx.y) * BM, n0 = int64_t(blockIdx.x) * BN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

  // Each thread stages 2 chunks of A and 2 of Bt per K step: rows tid/4 and tid/4 + 64,
  // chunk tid % 4 (8 elements) of the 32-wide K slice.
  const int lr = tid >> 2, lc = (tid & 3) * 8;
  dsp_u32x4 ra[2], rb[2];
  SegOffsets b_seg{};
  auto fetch = [&](int64_t k0) {
    // k0 is uniform across the workgroup, so the segment lookup stays scalar.
    const int64_t s = k0 / a_seg_len;
    const uint16_t* abase = kVec ? a + a_seg.off[s] : a;
    const int64_t ak = kVec ? k0 - s * a_seg_len + lc : 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ra[i] = load_chunk<kVec>(abase, a_seg, a_seg_len, lda, m0 + lr + 64 * i, M, ak, k0 + lc, K);
      rb[i] = load_chunk<kVec>(bt, b_seg, K, ldb, n0 + lr + 64 * i, N, k0 + lc, k0 + lc, K);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *reinterpret_cast<dsp_u32x4*>(&sa[buf][lr + 64 * i][lc]) = ra[i];
      *reinterpret_cast<dsp_u32x4*>(&sb[buf][lr + 64 * i][lc]) = rb[i];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t nk = (K + BK - 1) / BK;
  fetch(0);
  stash(0);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;  // fragment row and k offset
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) fetch((kt + 1) * BK);
    dsp_u32x4 fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i] = *reinterpret_cast<const dsp_u32x4*>(&sa[buf][wm + 16 * i + fr][fk]);
      fb[i] = *reinterpret_cast<const dsp_u32x4*>(&sb[buf][wn + 16 * i + fr][fk]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fb[j]),
                                                            __builtin_bit_cast(bf16x8, fa[i]),
                                                            acc[i][j], 0, 0, 0);
    if (kt + 1 < nk) {
      stash(buf ^ 1);
      __syncthreads();
    }
  }

  // acc[i][j] = C^T tile: lane holds rows n = wn + 16j + 4*(lane/16) + e, column
  // m = wm + 16i + lane%16 (the MFMA was fed Bt as its A operand).
  float b4[4][4] = {};
  if (bias_mode != 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) load_bias4(bias, n0 + wn + 16 * j + 4 * (lane >> 4), N, b4[j]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + wm + 16 * i + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      store_c4(acc[i][j], c + m * ldc, n0 + wn + 16 * j + 4 * (lane >> 4), N, b4[j], bias_mode,
               act, accumulate);
  }
}

// ---- large problems ---------------------------------------------------------------------
// 256 x 256 output tile per 512-thread workgroup: 8 waves as 4 (M) x 2 (N), 64 x 128 each
// as 4 x 8 v_mfma_f32_16x16x32 tiles.  K advances in 64-wide stages that go from global
// memory straight into LDS (global_load_lds_dwordx4: no VGPR staging, no ds_write), two
// stages resident (128 KiB).  A tile row is 128 bytes = 8 chunks of 16 bytes; chunk c of
// row r is stored at slot c ^ (r & 7), so both the DMA writes (64 consecutive chunks per
// instruction) and the MFMA fragment reads (16 rows x 4 chunks per wave) hit distinct
// banks.  Each output still accumulates over K in 32-wide MFMA steps in increasing k, the
// same order as map_gemm_kernel, so the two kernels give bit-identical results.
namespace big {
constexpr int kBM = 256, kBN = 256, kBK = 64, kWN = 2, kNW = 8, kNT = 64 * kNW;
constexpr int kCPR = kBK / 8;                // 16-byte chunks per tile row
constexpr int kRowB = kBK * 2;               // bytes per tile row
constexpr int kStageB = (kBM + kBN) * kRowB;
constexpr int kLPW = (kBM + kBN) * kCPR / 64 / kNW;  // 1-KiB DMA loads per wave per stage
constexpr int kTM = 64, kTN = 128, kFM = kTM / 16, kFN = kTN / 16, kKS = kBK / 32;
static_assert(kBM * kCPR % (64 * kLPW) == 0, "a wave loads rows of one operand only");
}  // namespace big

typedef __attribute__((address_space(3))) void lds_void_t;

// Where the rows of C go when they are scattered into a paged pool instead of a dense
// matrix (kPool): row m of problem z is pool slot block_tables[z][m / bs] * bs + m % bs of
// one layer, whose rows are ldc elements apart; a row whose block id lies outside the pool
// is skipped and counted.  rope_cos / rope_sin (kRope): fp32 tables [M][head_dim], row m
// the position of row m, applied after the bias (RoPE on each head of the row).
struct PoolOut {
  const int32_t* block_tables = nullptr;
  int64_t bt_stride = 0;
  int32_t log2_bs = 0;
  int64_t num_slots = 0;
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  int32_t head_dim = 0;
  int32_t* err_count = nullptr;
};

// out = x*cos + rotate_half(x)*sin for one element, x_partner the element half a head
// away (rotate_half(x) = cat(-x2, x1)); the two products and the sum are each rounded to
// fp32, the order of the reference's elementwise torch ops (transfer.py:76-80).
__device__ __forceinline__ float rope_apply1(float x, float x_partner, float c, float sn,
                                             bool first_half) {
#pragma clang fp contract(off)
  const float t1 = x * c;
  const float t2 = x_partner * sn;
  return first_half ? t1 - t2 : t1 + t2;
}

// The epilogue flags are template parameters: with all three variants compiled into one
// body the epilogue's live ranges push the kernel past 256 VGPRs.  kRope / kPool: the
// fused target-RoPE and pool-scatter epilogue of dsp_kv_map_gemm_to_pool.
template <int kBias, int kAct, int kAccum, int kRope = 0, int kPool = 0>
__global__ __launch_bounds__(big::kNT) void map_gemm_big_kernel(
    const uint16_t* __restrict__ a, SegOffsets a_seg, int64_t a_seg_len, int64_t lda,
    const uint16_t* __restrict__ bt, int64_t ldb, uint16_t* __restrict__ c, int64_t ldc,
    int64_t M, int64_t N, int64_t K, const uint16_t* __restrict__ bias,
    int64_t a_batch_stride, int64_t c_batch_stride, PoolOut po = PoolOut()) {
  __shared__ __attribute__((aligned(1024))) char lds[2 * big::kStageB];
  // 1-D grid over (batch, m tile, n tile), n fastest.  Workgroup ids are dealt to the 8
  // XCDs round-robin; remap so each XCD gets a contiguous run of tiles and the n tiles
  // sharing one A row block run on the same L2.
  const int tn = int((N + big::kBN - 1) / big::kBN), tm = int((M + big::kBM - 1) / big::kBM);
  int t = int(blockIdx.x);
  const int full = int(gridDim.x) & ~7;
  if (t < full) t = (t & 7) * (full >> 3) + (t >> 3);
  const int bx = t % tn, by = (t / tn) % tm, bz = t / (tn * tm);
  a += int64_t(bz) * a_batch_stride;
  if (!kPool) c += int64_t(bz) * c_batch_stride;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t m0 = int64_t(by) * big::kBM, n0 = int64_t(bx) * big::kBN;

  // This wave's loads: instruction j covers tile rows 8 * (wave * kLPW + j) .. +7 (A rows
  // for waves 0-3, Bt rows for waves 4-7); lane l fills slot l % 8 of row l / 8, i.e.
  // chunk (l % 8) ^ (row & 7).  Rows past M / N are clamped to the last row (their outputs are
  // never stored).  Element offsets fit 32 bits (checked on the host).
  const bool loads_a = wave * big::kLPW * 64 < big::kBM * big::kCPR;
  uint32_t off[big::kLPW];
#pragma unroll
  for (int j = 0; j < big::kLPW; ++j) {
    const int r = (wave * big::kLPW + j) * (64 / big::kCPR) + lane / big::kCPR;
    const int chunk = (lane % big::kCPR) ^ (r & 7);
    const int64_t row = loads_a ? min<int64_t>(m0 + r, M - 1) : min<int64_t>(n0 + r - big::kBM, N - 1);
    off[j] = uint32_t(row * (loads_a ? lda : ldb) + chunk * 8);
  }
  // Stages are issued in order; the A source (segment seg_i, column seg_k inside it) is
  // advanced incrementally, so a segment offset is fetched once per segment boundary
  // rather than divided out and loaded at every stage (a stage never straddles segments).
  int64_t seg_i = 0, seg_k = 0;
  const uint16_t* a_src = a + a_seg.off[0];
  auto issue = [&](int buf, int64_t k0) {
    const uint16_t* src = loads_a ? a_src + seg_k : bt + k0;
    char* dst = lds + buf * big::kStageB + wave * big::kLPW * 1024;
#pragma unroll
    for (int j = 0; j < big::kLPW; ++j)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + off[j]),
                                       (lds_void_t*)(dst + j * 1024), 16, 0, 0);
    seg_k += big::kBK;
    if (seg_k == a_seg_len && k0 + big::kBK < K) {
      seg_k = 0;
      a_src = a + a_seg.get(++seg_i);
    }
  };

  f32x4 acc[big::kFM][big::kFN];
#pragma unroll
  for (int i = 0; i < big::kFM; ++i)
#pragma unroll
    for (int j = 0; j < big::kFN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int wm = (wave / big::kWN) * big::kTM, wn = (wave % big::kWN) * big::kTN;
  const int fr = lane & 15, fq = lane >> 4;
  dsp_u32x4 fa[2][big::kFM], fb[2][big::kFN];
  auto read_frags = [&](const char* sa, int ks, int slot) {
    const char* sb = sa + big::kBM * big::kRowB;
    const int chunk = ks * 4 + fq;
#pragma unroll
    for (int i = 0; i < big::kFM; ++i) {
      const int r = wm + 16 * i + fr;
      fa[slot][i] = *reinterpret_cast<const dsp_u32x4*>(sa + r * big::kRowB + ((chunk ^ (r & 7)) * 16));
    }
#pragma unroll
    for (int j = 0; j < big::kFN; ++j) {
      const int r = wn + 16 * j + fr;
      fb[slot][j] = *reinterpret_cast<const dsp_u32x4*>(sb + r * big::kRowB + ((chunk ^ (r & 7)) * 16));
    }
  };

  const int nk = int(K / big::kBK);
  issue(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt has landed for every wave, and every wave is done reading stage kt - 1,
    // whose buffer the next DMA overwrites
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    const char* sa = lds + (kt & 1) * big::kStageB;
    read_frags(sa, 0, 0);
    if (kt + 1 < nk) issue((kt + 1) & 1, int64_t(kt + 1) * big::kBK);
#pragma unroll
    for (int ks = 0; ks < big::kKS; ++ks) {
      if (ks + 1 < big::kKS) read_frags(sa, ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < big::kFM; ++i)
#pragma unroll
        for (int j = 0; j < big::kFN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fb[ks & 1][j]),
                                                              __builtin_bit_cast(bf16x8, fa[ks & 1][i]),
                                                              acc[i][j], 0, 0, 0);
      if (ks + 1 < big::kKS) {
        // issue the next slice's fragment reads between this slice's MFMAs
#pragma unroll
        for (int q = 0; q < big::kFM + big::kFN; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, big::kFM * big::kFN - (big::kFM + big::kFN), 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // Epilogue through LDS.  acc[i][j] is a C^T tile: lane holds columns
  // n = wn + 16j + 4*(lane/16) + e of row m = wm + 16i + lane%16, so stores straight from
  // it write 16 rows x 32 bytes per instruction.  Instead each wave rounds its 64 x 128
  // outputs into its own 16 KiB of the (now idle) stage buffers as bf16 rows of 256 bytes
  // (16-byte chunk c of row r at slot c ^ (r & 15), its two 8-byte halves swapped in rows
  // with r & 8: the 16 lanes of an 8-byte write, rows r0 .. r0 + 15 at one column, then hit
  // 16 distinct bank pairs, where rows r and r + 8 shared one) and reads them
  // back four whole rows per instruction, so C is written in full 256-byte row runs with
  // 16-byte lanes -- half the store instructions, every cache line written whole -- with
  // non-temporal stores (same-box A/B, config 5: 73.4-74.7 against 75.7-76.8 us a launch).
  static_assert(big::kNW * big::kTM * big::kTN * 2 <= 2 * big::kStageB, "C tile fits the stages");
  float b4[big::kFN][4] = {};
  if (kBias) {
#pragma unroll
    for (int j = 0; j < big::kFN; ++j) load_bias4(bias, n0 + wn + 16 * j + 4 * fq, N, b4[j]);
  }
  __syncthreads();   // every wave is done reading the last stage
  char* ct = lds + wave * (big::kTM * big::kTN * 2);
#pragma unroll
  for (int i = 0; i < big::kFM; ++i) {
    const int r = 16 * i + fr;
#pragma unroll
    for (int j = 0; j < big::kFN; ++j) {
      uint16_t yb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        yb[e] = dsp_f32_to_bf16(epi_bias_act(acc[i][j][e], b4[j][e], kBias, kAct));
      const int col = 16 * j + 4 * fq;
      *reinterpret_cast<dsp_u32x2*>(ct + r * (big::kTN * 2) + (((col >> 3) ^ (r & 15)) * 16) +
                                    (((col & 7) * 2) ^ (r & 8))) =
          dsp_u32x2{uint32_t(yb[0]) | (uint32_t(yb[1]) << 16),
                    uint32_t(yb[2]) | (uint32_t(yb[3]) << 16)};
    }
  }
  const int cl = lane & 15;
  const int64_t n = n0 + wn + 8 * cl;
  const bool vec_c = n + 7 < N;
  // kPool: the pool slot of each of this lane's 16 rows (loads issued together)
  int64_t slot_q[kPool ? big::kTM / 4 : 1];
  if constexpr (kPool) {
    const int32_t* btz = po.block_tables + int64_t(bz) * po.bt_stride;
    const int bmask = (1 << po.log2_bs) - 1;
#pragma unroll
    for (int q = 0; q < big::kTM / 4; ++q) {
      const int64_t m = min<int64_t>(m0 + wm + 4 * q + (lane >> 4), M - 1);
      slot_q[q] = (int64_t(btz[m >> po.log2_bs]) << po.log2_bs) | (m & bmask);
    }
  }
  // kRope: this lane's 8 columns are dims d0 .. d0 + 7 of one head; the partner chunk (half
  // a head away) is chunk cl ^ (head_dim / 16) of the same wave tile (tiles are head-aligned)
  const int hd = kRope ? po.head_dim : 8;
  const int d0 = int((n0 + wn + 8 * cl) % hd);
  const bool first_half = d0 < hd / 2;
  const int pcl = cl ^ (hd / 16);
#pragma unroll
  for (int q = 0; q < big::kTM / 4; ++q) {
    const int r = 4 * q + (lane >> 4);
    // r & 8 is bit 1 of q for every lane (r = 4q + 0..3): a fixed register swap
    const bool swapped = (q >> 1) & 1;
    auto unswap = [swapped](dsp_u32x4 u) {
      return swapped ? dsp_u32x4{u[2], u[3], u[0], u[1]} : u;
    };
    dsp_u32x4 v = unswap(
        *reinterpret_cast<const dsp_u32x4*>(ct + r * (big::kTN * 2) + ((cl ^ (r & 15)) * 16)));
    const int64_t m = m0 + wm + r;
    if (m >= M) continue;
    if constexpr (kRope) {
      const dsp_u32x4 vp = unswap(
          *reinterpret_cast<const dsp_u32x4*>(ct + r * (big::kTN * 2) + ((pcl ^ (r & 15)) * 16)));
      const float* cr = po.rope_cos + m * hd + d0;
      const float* sr = po.rope_sin + m * hd + d0;
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(cr), c1 = *reinterpret_cast<const f32x4*>(cr + 4);
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(sr), s1 = *reinterpret_cast<const f32x4*>(sr + 4);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float clo = w < 2 ? c0[2 * w] : c1[2 * w - 4], chi = w < 2 ? c0[2 * w + 1] : c1[2 * w - 3];
        const float slo = w < 2 ? s0[2 * w] : s1[2 * w - 4], shi = w < 2 ? s0[2 * w + 1] : s1[2 * w - 3];
        const uint16_t lo = dsp_f32_to_bf16(
            rope_apply1(dsp_bf16lo(v[w]), dsp_bf16lo(vp[w]), clo, slo, first_half));
        const uint16_t hi = dsp_f32_to_bf16(
            rope_apply1(dsp_bf16hi(v[w]), dsp_bf16hi(vp[w]), chi, shi, first_half));
        v[w] = uint32_t(lo) | (uint32_t(hi) << 16);
      }
    }
    uint16_t* dst;
    if constexpr (kPool) {
      const int64_t slot = slot_q[q];
      if (slot < 0 || slot >= po.num_slots) {
        if (cl == 0 && po.err_count) atomicAdd(po.err_count, 1);
        continue;
      }
      dst = c + slot * ldc + n;
    } else {
      dst = c + m * ldc + n;
    }
    if (vec_c && dsp_aligned(dst, 16)) {
      dsp_u32x4 w = v;
      if (kAccum) {
        const dsp_u32x4 old = *reinterpret_cast<const dsp_u32x4*>(dst);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint16_t lo = dsp_f32_to_bf16(bf16_round(dsp_bf16lo(old[e]) + dsp_bf16lo(v[e])));
          const uint16_t hi = dsp_f32_to_bf16(bf16_round(dsp_bf16hi(old[e]) + dsp_bf16hi(v[e])));
          w[e] = uint32_t(lo) | (uint32_t(hi) << 16);
        }
      }
      dsp_st_stream(w, reinterpret_cast<dsp_u32x4*>(dst));  // C is not read back here
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (n + e >= N) break;
        const uint32_t word = v[e >> 1];
        uint16_t y = uint16_t((e & 1) ? word >> 16 : word);
        if (kAccum) y = dsp_f32_to_bf16(bf16_round(dsp_bf16lo(dst[e]) + dsp_bf16lo(y)));
        dst[e] = y;
      }
    }
  }
}

// RoPE on (L, T, H, D) rows in fp32: out = x*cos + sign*rot(x)*sin, with
// rot(x) = cat(-x2, x1) over the two halves of head_dim (transfer.py:61-80: sign -1
// strips, +1 applies).  Input bf16 or fp32; output fp32, or bf16 rounded to nearest
// even.  One thread per pair (d, d + D/2) of one head of one token of one layer.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void rope_kernel(const TI* __restrict__ x, TO* __restrict__ y,
                                                   int64_t L, int64_t T, int64_t H, int64_t D,
                                                   int64_t x_layer_stride, int64_t y_layer_stride,
                                                   const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t, float sign) {
#pragma clang fp contract(off)
  const int64_t half = D / 2;
  const int64_t per_layer = T * H * half;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= L * per_layer) return;
  const int64_t l = idx / per_layer;
  int64_t r = idx - l * per_layer;
  const int64_t t = r / (H * half);
  r -= t * H * half;
  const int64_t h = r / half, d = r - h * half;
  const int64_t xo = l * x_layer_stride + (t * H + h) * D;
  const int64_t yo = l * y_layer_stride + (t * H + h) * D;
  auto ld = [](TI v) -> float {
    if constexpr (sizeof(TI) == 2) return dsp_bf16lo(v); else return v;
  };
  auto st = [](float v) -> TO {
    if constexpr (sizeof(TO) == 2) return dsp_f32_to_bf16(v); else return v;
  };
  const float x1 = ld(x[xo + d]), x2 = ld(x[xo + d + half]);
  const float c1 = cos_t[t * D + d], s1 = sin_t[t * D + d];
  const float c2 = cos_t[t * D + d + half], s2 = sin_t[t * D + d + half];
  // x * cos and rot(x) * sin are rounded separately, then added (contraction into a fused
  // multiply-add is off for this kernel): the operation order of the reference's
  // elementwise torch ops.
  const float o1 = x1 * c1 + sign * (-x2 * s1);
  const float o2 = x2 * c2 + sign * (x1 * s2);
  y[yo + d] = st(o1);
  y[yo + d + half] = st(o2);
}

}  // namespace

extern "C" int dsp_kv_map_gemm(const void* a, const int64_t* a_segment_offsets,
                               int32_t num_segments, int64_t segment_len, int64_t lda,
                               const void* bt, int64_t ldb, void* c, int64_t ldc, int64_t M,
                               int64_t N, int64_t K, int32_t batch, int64_t a_batch_stride,
                               int64_t c_batch_stride, const void* bias, int32_t bias_mode,
                               int32_t activation, int32_t accumulate, int32_t dtype,
                               dsp_stream_t stream) {
  DSP_HOST_CHECK(a && bt && c && a_segment_offsets, DSP_EINVAL);
  DSP_HOST_CHECK(M >= 0 && N >= 0 && K >= 0 && lda >= 0 && ldb >= K && ldc >= N, DSP_EINVAL);
  DSP_HOST_CHECK(num_segments >= 1 && num_segments <= kMaxSegments && segment_len > 0 &&
                     int64_t(num_segments) * segment_len == K,
                 DSP_EINVAL);
  DSP_HOST_CHECK(bias_mode >= 0 && bias_mode <= 2 && (bias_mode == 0 || bias) &&
                     (activation == 0 || activation == 1),
                 DSP_EINVAL);
  DSP_HOST_CHECK(dtype == DSP_BF16, DSP_EUNSUPPORTED);
  DSP_HOST_CHECK(batch >= 0 && batch <= 65535 && a_batch_stride >= 0 && c_batch_stride >= 0,
                 DSP_EINVAL);
  if (M == 0 || N == 0 || batch == 0) return DSP_OK;
  SegOffsets seg{};
  bool vec = dsp_aligned(a, 16) && dsp_aligned(bt, 16) && segment_len % BK == 0 &&
             lda % 8 == 0 && ldb % 8 == 0 && a_batch_stride % 8 == 0;
  for (int i = 0; i < num_segments; ++i) {
    seg.off[i] = a_segment_offsets[i];
    vec = vec && (seg.off[i] % 8 == 0);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* ah = static_cast<const uint16_t*>(a);
  const uint16_t* bh = static_cast<const uint16_t*>(bt);
  uint16_t* ch = static_cast<uint16_t*>(c);
  const uint16_t* biash = static_cast<const uint16_t*>(bias);
  // Large problems (enough 256 x 256 tiles to cover the chip half a time) take the
  // direct-to-LDS kernel; it needs 64-aligned K stages and 32-bit element offsets.
  const int64_t big_tiles = ((M + big::kBM - 1) / big::kBM) * ((N + big::kBN - 1) / big::kBN) * batch;
  int64_t max_a_off = 0;
  for (int i = 0; i < num_segments; ++i) max_a_off = max(max_a_off, seg.off[i]);
  // (bias mode 1 with gelu and accumulate -- a form no map uses -- would spill: excluded)
  const bool use_big = vec && big_tiles >= 128 && big_tiles < (int64_t(1) << 31) &&
                       !(bias_mode == 1 && activation == 1 && accumulate) &&
                       K % big::kBK == 0 && segment_len % big::kBK == 0 &&
                       max_a_off + (M - 1) * lda + segment_len <= int64_t(UINT32_MAX) &&
                       (N - 1) * ldb + K <= int64_t(UINT32_MAX);
  if (use_big) {
    const unsigned grid = static_cast<unsigned>(big_tiles);
#define DSP_BIG(B, A, C)                                                                       \
  map_gemm_big_kernel<B, A, C><<<grid, big::kNT, 0, s>>>(ah, seg, segment_len, lda, bh, ldb, ch, \
                                                         ldc, M, N, K, biash, a_batch_stride,  \
                                                         c_batch_stride)
#define DSP_BIG_B(A, C)                \
  if (bias_mode == 0) DSP_BIG(0, A, C); \
  else if (bias_mode == 1) DSP_BIG(1, A, C); \
  else DSP_BIG(2, A, C)
    if (activation == 0 && !accumulate) { DSP_BIG_B(0, 0); }
    else if (activation == 0) { DSP_BIG_B(0, 1); }
    else if (!accumulate) { DSP_BIG_B(1, 0); }
    else if (bias_mode == 0) { DSP_BIG(0, 1, 1); }
    else { DSP_BIG(2, 1, 1); }
#undef DSP_BIG_B
#undef DSP_BIG
    return dsp_launch_status();
  }
  const int64_t gm = (M + BM - 1) / BM, gn = (N + BN - 1) / BN;
  DSP_HOST_CHECK(gm < (int64_t(1) << 31) && gn <= 65535, DSP_EINVAL);
  dim3 grid(static_cast<unsigned>(gn), static_cast<unsigned>(gm), static_cast<unsigned>(batch));
  if (vec)
    map_gemm_kernel<true><<<grid, kThreads, 0, s>>>(ah, seg, segment_len, lda, bh, ldb, ch, ldc, M,
                                                    N, K, biash, bias_mode, activation, accumulate,
                                                    a_batch_stride, c_batch_stride);
  else
    map_gemm_kernel<false><<<grid, kThreads, 0, s>>>(ah, seg, segment_len, lda, bh, ldb, ch, ldc,
                                                     M, N, K, biash, bias_mode, activation,
                                                     accumulate, a_batch_stride, c_batch_stride);
  return dsp_launch_status();
}

extern "C" int dsp_kv_map_gemm_to_pool(
    const void* a, const int64_t* a_segment_offsets, int32_t num_segments, int64_t segment_len,
    int64_t lda, const void* bt, int64_t ldb, void* pool, int64_t pool_row_stride,
    int64_t num_slots, const int32_t* block_tables, int64_t bt_stride, int32_t block_size,
    int64_t M, int64_t N, int64_t K, int32_t batch, int64_t a_batch_stride, const void* bias,
    const float* rope_cos, const float* rope_sin, int32_t head_dim, int32_t dtype,
    int32_t* err_count, dsp_stream_t stream) {
  DSP_HOST_CHECK(a && bt && pool && a_segment_offsets && block_tables, DSP_EINVAL);
  DSP_HOST_CHECK(M >= 0 && N > 0 && K > 0 && lda >= 0 && ldb >= K && pool_row_stride >= N &&
                     num_slots >= 0 && bt_stride >= 0,
                 DSP_EINVAL);
  DSP_HOST_CHECK(num_segments >= 1 && num_segments <= kMaxSegments && segment_len > 0 &&
                     int64_t(num_segments) * segment_len == K,
                 DSP_EINVAL);
  DSP_HOST_CHECK(dsp_is_pow2(block_size) && bt_stride * block_size >= M, DSP_EINVAL);
  DSP_HOST_CHECK((rope_cos == nullptr) == (rope_sin == nullptr), DSP_EINVAL);
  DSP_HOST_CHECK(dtype == DSP_BF16, DSP_EUNSUPPORTED);
  DSP_HOST_CHECK(batch >= 0 && batch <= 65535 && a_batch_stride >= 0, DSP_EINVAL);
  if (M == 0 || batch == 0) return DSP_OK;
  const bool rope = rope_cos != nullptr;
  // one head per 128-column wave tile (or two of 64): tiles are head-aligned
  DSP_HOST_CHECK(!rope || ((head_dim == 64 || head_dim == 128) && N % head_dim == 0 &&
                           dsp_aligned(rope_cos, 16) && dsp_aligned(rope_sin, 16)),
                 DSP_EUNSUPPORTED);
  SegOffsets seg{};
  int64_t max_a_off = 0;
  bool ok = dsp_aligned(a, 16) && dsp_aligned(bt, 16) && dsp_aligned(pool, 16) && lda % 8 == 0 &&
            ldb % 8 == 0 && a_batch_stride % 8 == 0 && pool_row_stride % 8 == 0 && N % 8 == 0 &&
            K % big::kBK == 0 && segment_len % big::kBK == 0;
  for (int i = 0; i < num_segments; ++i) {
    seg.off[i] = a_segment_offsets[i];
    ok = ok && seg.off[i] % 8 == 0;
    max_a_off = max(max_a_off, seg.off[i]);
  }
  // the large-tile kernel's preconditions (16-byte operand rows, 64-wide K stages, 32-bit
  // element offsets); nothing else carries this epilogue
  const int64_t tiles = ((M + big::kBM - 1) / big::kBM) * ((N + big::kBN - 1) / big::kBN) * batch;
  DSP_HOST_CHECK(ok && tiles < (int64_t(1) << 31) &&
                     max_a_off + (M - 1) * lda + segment_len <= int64_t(UINT32_MAX) &&
                     (N - 1) * ldb + K <= int64_t(UINT32_MAX),
                 DSP_EUNSUPPORTED);
  PoolOut po;
  po.block_tables = block_tables;
  po.bt_stride = bt_stride;
  po.log2_bs = dsp_log2i(block_size);
  po.num_slots = num_slots;
  po.rope_cos = rope_cos;
  po.rope_sin = rope_sin;
  po.head_dim = head_dim;
  po.err_count = err_count;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(tiles);
  const uint16_t* ah = static_cast<const uint16_t*>(a);
  const uint16_t* bh = static_cast<const uint16_t*>(bt);
  uint16_t* ch = static_cast<uint16_t*>(pool);
  const uint16_t* biash = static_cast<const uint16_t*>(bias);
#define DSP_POOL(B, R)                                                                    \
  map_gemm_big_kernel<B, 0, 0, R, 1><<<grid, big::kNT, 0, s>>>(                            \
      ah, seg, segment_len, lda, bh, ldb, ch, pool_row_stride, M, N, K, biash, a_batch_stride, \
      0, po)
  if (bias) {
    if (rope) DSP_POOL(1, 1); else DSP_POOL(1, 0);
  } else {
    if (rope) DSP_POOL(0, 1); else DSP_POOL(0, 0);
  }
#undef DSP_POOL
  return dsp_launch_status();
}

extern "C" int dsp_kv_rope(const void* x, int64_t x_layer_stride, void* y,
                           int64_t y_layer_stride, int64_t L, int64_t T, int64_t H, int64_t D,
                           const float* cos_table, const float* sin_table, int32_t direction,
                           int32_t in_dtype, int32_t out_dtype, dsp_stream_t stream) {
  DSP_HOST_CHECK(x && y && cos_table && sin_table, DSP_EINVAL);
  DSP_HOST_CHECK(L >= 0 && T >= 0 && H >= 0 && D > 0 && D % 2 == 0, DSP_EINVAL);
  DSP_HOST_CHECK(x_layer_stride >= T * H * D && y_layer_stride >= T * H * D, DSP_EINVAL);
  DSP_HOST_CHECK(direction == 1 || direction == -1, DSP_EINVAL);
  DSP_HOST_CHECK((in_dtype == DSP_BF16 || in_dtype == DSP_F32) &&
                     (out_dtype == DSP_BF16 || out_dtype == DSP_F32),
                 DSP_EUNSUPPORTED);
  const int64_t n = L * T * H * (D / 2);
  if (n == 0) return DSP_OK;
  const int64_t blocks = (n + 255) / 256;
  DSP_HOST_CHECK(blocks < (int64_t(1) << 31), DSP_EINVAL);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned nb = static_cast<unsigned>(blocks);
  const float sg = float(direction);
#define DSP_ROPE(TI, TO)                                                                      \
  rope_kernel<TI, TO><<<nb, 256, 0, s>>>(static_cast<const TI*>(x), static_cast<TO*>(y), L, T, \
                                         H, D, x_layer_stride, y_layer_stride, cos_table,    \
                                         sin_table, sg)
  if (in_dtype == DSP_BF16 && out_dtype == DSP_BF16) DSP_ROPE(uint16_t, uint16_t);
  else if (in_dtype == DSP_BF16) DSP_ROPE(uint16_t, float);
  else if (out_dtype == DSP_BF16) DSP_ROPE(float, uint16_t);
  else DSP_ROPE(float, float);
#undef DSP_ROPE
  return dsp_launch_status();
}
