// Shared definitions for the gfx950 TriS-MoE grouped expert kernels.
//
// Format constants follow the reference's block-GR / compact3 layout
// (TriSMoE_cuda_kernel.cu:55-79, qlinear_cuda.py:486-494): a GR block covers
// 64 input columns (2 packed rows of 32 bits) x 64 outputs = 128 words.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "tris_moe_hip.h"

namespace tris {

constexpr int kTileK = 64;            // input columns per GR block / K tile
constexpr int kTileOut = 64;          // outputs per GR block / N tile
constexpr int kGrPackedRows = 2;      // packed 32-bit rows per GR block
constexpr int kGrWords = 128;         // decoded words per GR block
constexpr int kGrBits = kGrWords * 32;
constexpr int kMetaKMask = 0xF;
constexpr int kMetaRaw = 1 << 4;
constexpr int kMetaOnesShift = 8;
constexpr int kMaxParallelK = 7;      // encoder's largest k; larger k decode serially
constexpr int kWave = 64;

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// fp16 bits <-> float, exact.
__device__ __forceinline__ float h2f(uint16_t bits) {
  return __half2float(__ushort_as_half(bits));
}
__device__ __forceinline__ uint16_t f2h_bits(float v) {
  return __half_as_ushort(__float2half(v));
}
// Correctly rounded fp16 product / sum (RNE), matching __hmul/__hadd.
__device__ __forceinline__ uint16_t hmul_bits(uint16_t a, uint16_t b) {
  return __half_as_ushort(__hmul(__ushort_as_half(a), __ushort_as_half(b)));
}
__device__ __forceinline__ uint16_t hadd_bits(uint16_t a, uint16_t b) {
  return __half_as_ushort(__hadd(__ushort_as_half(a), __ushort_as_half(b)));
}

// The reference's gated activation act_fn(g) * u for fp16 g, u (modeling_mixtral.py:496): SiLU in fp32
// rounded to fp16, then the fp16 product.
__device__ __forceinline__ uint16_t swiglu_bits(uint16_t g16, uint16_t u16) {
  const float g = h2f(g16);
  const float sg = h2f(f2h_bits(g / (1.0f + expf(-g))));
  return f2h_bits(sg * h2f(u16));
}

__device__ __forceinline__ uint32_t low_mask(int bits) {
  return bits >= 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u);
}

// Host-side error reporting shared by every C-ABI entry point.
void set_error(const char* fmt, ...);
int check_launch(const char* what);

}  // namespace tris

#define TRIS_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::tris::set_error(__VA_ARGS__);    \
      return TRIS_ERR_INVALID;           \
    }                                    \
  } while (0)
