// MFMA helpers shared by the attention kernels (gfx950, 64-wide waves).
#pragma once

#include <type_traits>

#include "dsp_common.h"

namespace dsp_mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Bf16Tag {};
struct F16Tag {};

// One v_mfma_f32_16x16x32_{bf16,f16}: c += a . b with 8 packed 16-bit values per lane in
// each operand (lane l: row l % 16, k range 8 * (l / 16) .. +8).
template <typename Tag>
__device__ __forceinline__ f32x4 mfma32(dsp_u32x4 a, dsp_u32x4 b, f32x4 c) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// fp32 -> the cache dtype, round to nearest even.
template <typename Tag>
__device__ __forceinline__ uint16_t narrow(float f) {
  if constexpr (std::is_same<Tag, Bf16Tag>::value)
    return dsp_f32_to_bf16(f);
  else
    return dsp_f32_to_f16(f);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return uint32_t(lo) | (uint32_t(hi) << 16);
}

}  // namespace dsp_mfma
