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

// Typed views of generic pointers for loads whose address space the compiler cannot infer (pointers taken from
// a struct indexed at run time, or selected between two arrays).  A generic (flat) load counts in the LDS
// counter as well as the vector-memory one, so each later wait for an LDS read would also wait for it: a global
// load issued ahead of a computation on LDS must be a global_load to stay in flight across it.
typedef const __attribute__((address_space(1))) int32_t gmem_i32;
typedef const __attribute__((address_space(3))) int32_t lds_i32;
__device__ __forceinline__ gmem_i32* as_gmem(const int32_t* p) { return (gmem_i32*)p; }
__device__ __forceinline__ lds_i32* as_lds(const int32_t* p) { return (lds_i32*)p; }

// fp16 bits <-> float, exact.
__device__ __forceinline__ float h2f(uint16_t bits) {
  return __half2float(__ushort_as_half(bits));
}
__device__ __forceinline__ uint16_t f2h_bits(float v) {
  return __half_as_ushort(__float2half(v));
}
// float -> bf16 bits, round to nearest even (NaN stays a quiet NaN), as torch's .to(bfloat16).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
// Correctly rounded fp16 product / sum (RNE), matching __hmul/__hadd.
__device__ __forceinline__ uint16_t hmul_bits(uint16_t a, uint16_t b) {
  return __half_as_ushort(__hmul(__ushort_as_half(a), __ushort_as_half(b)));
}
__device__ __forceinline__ uint16_t hadd_bits(uint16_t a, uint16_t b) {
  return __half_as_ushort(__hadd(__ushort_as_half(a), __ushort_as_half(b)));
}

// The reference's gated activation act_fn(g) * u for fp16 g, u (modeling_mixtral.py:496): SiLU in fp32
// rounded to fp16, then the fp16 product.  silu(g) = g / (1 + e^-g) is evaluated with the hardware's base-2
// exponential and reciprocal (e^x = 2^(x log2 e), v_exp_f32 and v_rcp_f32, about 1 ulp each): the fp32 value is
// within a few tens of fp32 ulps of the correctly rounded quotient, so after the rounding to fp16 it is the
// IEEE-division value or one fp16 ulp from it (inf, -inf, NaN and the overflow of e^-g give the same results:
// -inf / inf is NaN, g / inf is -0).  The division sequence took about 30 VALU per element, which bounded the
// prefill kernels that form the product in their operand staging.  The quotient is formed from |g| and takes g's
// sign bit afterwards: the compiler turns a rounded fp16 product into v_fma_mix with a +0 addend, which would make
// silu(-0) = -0 a +0.
__device__ __forceinline__ uint16_t swiglu_bits(uint16_t g16, uint16_t u16) {
  const float g = h2f(g16);
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);  // e^-g
  const uint16_t mag = f2h_bits(__builtin_fabsf(g) * __builtin_amdgcn_rcpf(1.0f + e));
  const uint16_t sg = static_cast<uint16_t>(mag | (g16 & 0x8000u));
  return f2h_bits(h2f(sg) * h2f(u16));
}

constexpr uint32_t kBufferWord3 = 0x00020000;  // raw buffer resource, gfx9 family

// A raw buffer resource over [base, base + bytes): loads at or past `bytes` read zeros and stores there are
// dropped, without a memory access.  Every caller passes wave-uniform values; reading them back from the first
// lane lets the compiler keep the resource in scalar registers (a resource it cannot prove uniform costs a
// waterfall loop per access).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32)));
  const int n = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  void* ub = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, n, kBufferWord3);
}

__device__ __forceinline__ uint32_t low_mask(int bits) {
  return bits >= 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u);
}

// DPP lane move (register to register, no LDS round trip): lanes whose source lies outside their row, or
// whose row is masked off by RowMask, take `identity`.  Every lane of the wavefront must be active.
template <int Ctrl, int RowMask>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t identity, uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(identity), static_cast<int>(v), Ctrl, RowMask, 0xF, false));
}

// Inclusive scan over the 64 lanes of a wavefront (all active): row shifts within each row of 16, then the
// row-15 and row-31 broadcasts carry the row totals forward.  op(own, earlier) combines a lane's value with
// the combined value of the lanes before it; the tree is fixed, so every run combines in the same order.
template <typename Op>
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, uint32_t identity, Op op) {
  v = op(v, dpp_mov<0x111, 0xF>(identity, v));  // row_shr:1
  v = op(v, dpp_mov<0x112, 0xF>(identity, v));  // row_shr:2
  v = op(v, dpp_mov<0x114, 0xF>(identity, v));  // row_shr:4
  v = op(v, dpp_mov<0x118, 0xF>(identity, v));  // row_shr:8
  v = op(v, dpp_mov<0x142, 0xA>(identity, v));  // row_bcast:15 into rows 1 and 3
  v = op(v, dpp_mov<0x143, 0xC>(identity, v));  // row_bcast:31 into rows 2 and 3
  return v;
}

__device__ __forceinline__ int wave_incl_sum_i32(int v) {
  return static_cast<int>(
      wave_incl_scan(static_cast<uint32_t>(v), 0u, [](uint32_t own, uint32_t earlier) { return own + earlier; }));
}

// The wave-uniform maximum of int keys whose maximum is known to be >= 0 (every lane active): row maxima by
// DPP row shifts (a lane whose source lies outside its row takes 0, which cannot exceed that maximum), then
// the four rows' last lanes combined in scalar registers.
__device__ __forceinline__ int wave_max_nonneg_i32(int v) {
  v = max(v, static_cast<int>(dpp_mov<0x111, 0xF>(0u, static_cast<uint32_t>(v))));  // row_shr:1
  v = max(v, static_cast<int>(dpp_mov<0x112, 0xF>(0u, static_cast<uint32_t>(v))));  // row_shr:2
  v = max(v, static_cast<int>(dpp_mov<0x114, 0xF>(0u, static_cast<uint32_t>(v))));  // row_shr:4
  v = max(v, static_cast<int>(dpp_mov<0x118, 0xF>(0u, static_cast<uint32_t>(v))));  // row_shr:8
  const int a = __builtin_amdgcn_readlane(v, 15);
  const int b = __builtin_amdgcn_readlane(v, 31);
  const int c = __builtin_amdgcn_readlane(v, 47);
  const int d = __builtin_amdgcn_readlane(v, 63);
  return max(max(a, b), max(c, d));
}

// Wave-uniform reductions (the scan's last lane, read into a scalar register).
__device__ __forceinline__ float wave_max_f32(float v) {
  const uint32_t r = wave_incl_scan(__float_as_uint(v), __float_as_uint(-INFINITY), [](uint32_t own, uint32_t e) {
    return __float_as_uint(fmaxf(__uint_as_float(own), __uint_as_float(e)));
  });
  return __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(r), kWave - 1)));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  const uint32_t r = wave_incl_scan(__float_as_uint(v), 0u, [](uint32_t own, uint32_t e) {
    return __float_as_uint(__uint_as_float(own) + __uint_as_float(e));
  });
  return __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(r), kWave - 1)));
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
