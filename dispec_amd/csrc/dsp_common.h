// Shared helpers for the gfx950 kernels of libdispec_hip.so (device + host side).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dispec_hip.h"

#define DSP_HOST_CHECK(cond, code) \
  do {                             \
    if (!(cond)) return (code);    \
  } while (0)

// Launch status: a positive hipError_t, or DSP_OK.
static inline int dsp_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DSP_OK : static_cast<int>(e);
}

__host__ __device__ static inline bool dsp_aligned(const void* p, int64_t a) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(a)) == 0;
}

static inline bool dsp_is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

static inline int dsp_log2i(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}

// Largest vector width in {16, 8, 4, 2, 1} bytes dividing every value given.
static inline int dsp_vec_width(std::initializer_list<int64_t> vals) {
  int w = 16;
  for (int64_t v : vals) {
    while (w > 1 && (v % w) != 0) w >>= 1;
  }
  return w;
}

// s_waitcnt immediate that waits until at most VM vector-memory operations of this wave
// are outstanding and does not wait on the export or LDS/scalar counters.  gfx9
// encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4] (7 = no wait), lgkmcnt [11:8]
// (15 = no wait).  The vmcnt field holds 0..63: a count beyond it is a compile error, not
// a silently wrapped wait.
template <int VM>
constexpr int dsp_waitcnt_vm() {
  static_assert(VM >= 0 && VM <= 63, "vmcnt holds 0..63 outstanding loads on gfx9");
  return (VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8);
}
static_assert(dsp_waitcnt_vm<0>() == 0x0F70 && dsp_waitcnt_vm<8>() == 0x0F78 &&
                  dsp_waitcnt_vm<17>() == 0x4F71,
              "s_waitcnt encoding");

// ---------------------------------------------------------------- device helpers
// Byte vectors used for coalesced copies.  16 B per lane is one global_load_dwordx4.
// Native clang vectors, not HIP's uint4/uint2 structs: conditional loads of the struct
// types do not if-convert and serialise behind per-load waits.
typedef uint32_t dsp_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t dsp_u32x2 __attribute__((ext_vector_type(2)));
template <int VEC> struct dsp_vec;
template <> struct dsp_vec<16> { using type = dsp_u32x4; };
template <> struct dsp_vec<8> { using type = dsp_u32x2; };
template <> struct dsp_vec<4> { using type = uint32_t; };
template <> struct dsp_vec<2> { using type = uint16_t; };
template <> struct dsp_vec<1> { using type = uint8_t; };

// Streaming (non-temporal) load/store for data touched once: keeps the copy out of the
// caches' way.
template <typename V>
__device__ __forceinline__ V dsp_ld_stream(const V* p) { return __builtin_nontemporal_load(p); }
template <typename V>
__device__ __forceinline__ void dsp_st_stream(V v, V* p) { __builtin_nontemporal_store(v, p); }

// bf16 / fp16 <-> fp32.  bf16 widening is exact (a shift); narrowing rounds to nearest
// even, as torch's .to(torch.bfloat16) does (NaN kept quiet).
__device__ __forceinline__ float dsp_bf16lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float dsp_bf16hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// fp32 -> bf16, round to nearest even: one v_cvt_pk_bf16_f32 on gfx950 (NaN stays a quiet
// NaN; finite values round exactly as the bit-twiddling form u + 0x7fff + lsb would).
__device__ __forceinline__ uint16_t dsp_f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float dsp_f16lo(uint32_t u) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u & 0xffffu)));
}
__device__ __forceinline__ float dsp_f16hi(uint32_t u) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u >> 16)));
}
__device__ __forceinline__ uint16_t dsp_f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // round to nearest even
}

// Cross-lane helpers on one 64-wide wavefront.  DPP row ops act within rows of 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dsp_dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HMIRROR = 0x141; // lane i <- lane 7-i within each half-row
constexpr int DPP_ROW_MIRROR = 0x140;  // lane i <- lane 15-i within each row

// Sum over the aligned group of N consecutive lanes (N in 1,2,4,8,16); every lane of
// the group ends with the group total.
template <int N>
__device__ __forceinline__ float dsp_group_sum(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group of 1..16 lanes");
  if constexpr (N >= 2) x += dsp_dpp<DPP_QUAD_XOR1>(x);
  if constexpr (N >= 4) x += dsp_dpp<DPP_QUAD_XOR2>(x);
  if constexpr (N >= 8) x += dsp_dpp<DPP_ROW_HMIRROR>(x);
  if constexpr (N >= 16) x += dsp_dpp<DPP_ROW_MIRROR>(x);
  return x;
}

__device__ __forceinline__ float dsp_shfl_xor(float x, int mask) {
  int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

__device__ __forceinline__ float dsp_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
