// Routing-weighted combine of the grouped expert outputs.
//
// Replaces the reference's scatter-add (modeling_mixtral.py:529-536):
//   final.index_add_(0, grouped_token_indices, (down_out * routing).to(bf16))
// which rounds every routed contribution to bf16 and accumulates in bf16.
// Here each token's top-k contributions (fp16 products down_out * w, as in the
// reference) are gathered through the inverse route permutation, summed in
// fp32 together with an optional unrouted shared-expert output, and rounded
// once to bf16.  One thread produces 8 consecutive features; reads are
// 16-byte vector loads.
#include "tris_common.h"

namespace tris {

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ expert_out,
                                                          const int32_t* __restrict__ inverse_perm,
                                                          const uint16_t* __restrict__ weights,
                                                          const uint16_t* __restrict__ shared, int tokens, int top_k,
                                                          int hidden, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (t >= tokens || h0 >= hidden) return;
  const bool vec = (hidden % 8) == 0;
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.0f;
  for (int s = 0; s < top_k; ++s) {
    const int row = inverse_perm[t * top_k + s];
    const __half w = __ushort_as_half(weights[t * top_k + s]);
    const uint16_t* src = expert_out + static_cast<int64_t>(row) * hidden + h0;
    uint16_t v[8];
    if (vec) {
      *reinterpret_cast<uint4*>(v) = *reinterpret_cast<const uint4*>(src);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = (h0 + u < hidden) ? src[u] : 0;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += __half2float(__hmul(__ushort_as_half(v[u]), w));
  }
  if (shared != nullptr) {
    const uint16_t* src = shared + static_cast<int64_t>(t) * hidden + h0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (h0 + u < hidden) acc[u] += h2f(src[u]);
    }
  }
  uint16_t* dst = out + static_cast<int64_t>(t) * hidden + h0;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (h0 + u < hidden) dst[u] = f32_to_bf16_rne(acc[u]);
  }
}

// out = act_fn(gate) * up, 8 consecutive elements per thread (16-byte loads when aligned).
__global__ __launch_bounds__(256) void swiglu_mul_kernel(const uint16_t* __restrict__ gate,
                                                         const uint16_t* __restrict__ up, int64_t count,
                                                         uint16_t* __restrict__ out) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i0 >= count) return;
  if (i0 + 8 <= count) {
    const uint4 gv = *reinterpret_cast<const uint4*>(gate + i0);
    const uint4 uv = *reinterpret_cast<const uint4*>(up + i0);
    const uint32_t g[4] = {gv.x, gv.y, gv.z, gv.w};
    const uint32_t u[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = swiglu_bits(static_cast<uint16_t>(g[k]), static_cast<uint16_t>(u[k]));
      const uint32_t hi = swiglu_bits(static_cast<uint16_t>(g[k] >> 16), static_cast<uint16_t>(u[k] >> 16));
      o[k] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(out + i0) = make_uint4(o[0], o[1], o[2], o[3]);
    return;
  }
  for (int64_t i = i0; i < count; ++i) out[i] = swiglu_bits(gate[i], up[i]);
}

}  // namespace tris

using namespace tris;

extern "C" int tris_swiglu_mul(const uint16_t* gate, const uint16_t* up, int64_t count, uint16_t* out, void* stream) {
  TRIS_REQUIRE(count >= 0, "tris_swiglu_mul: negative count");
  if (count == 0) return TRIS_OK;
  TRIS_REQUIRE(gate && up && out, "tris_swiglu_mul: null pointer");
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(gate) % 16 == 0 && reinterpret_cast<uintptr_t>(up) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0,
               "tris_swiglu_mul: tensors must be 16-byte aligned");
  const int64_t threads = 256;
  const int64_t blocks = (count + 8 * threads - 1) / (8 * threads);
  TRIS_REQUIRE(blocks <= 2147483647LL, "tris_swiglu_mul: too many elements");
  hipLaunchKernelGGL(swiglu_mul_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), gate, up, count, out);
  return check_launch("swiglu_mul_kernel");
}

extern "C" int tris_moe_combine(const uint16_t* expert_out, const int32_t* inverse_perm, const uint16_t* weights,
                                const uint16_t* shared, int32_t tokens, int32_t top_k, int32_t hidden,
                                uint16_t* out, void* stream) {
  TRIS_REQUIRE(tokens >= 0 && top_k >= 0 && hidden >= 0, "tris_moe_combine: negative shape");
  if (tokens == 0 || hidden == 0) return TRIS_OK;
  TRIS_REQUIRE(out != nullptr && (top_k == 0 || (expert_out && inverse_perm && weights)),
               "tris_moe_combine: null pointer");
  TRIS_REQUIRE(tokens <= 65535, "tris_moe_combine: too many tokens per launch (%d)", tokens);
  TRIS_REQUIRE(hidden % 8 != 0 || reinterpret_cast<uintptr_t>(expert_out) % 16 == 0,
               "tris_moe_combine: expert_out must be 16-byte aligned");
  const int threads = 256;
  dim3 grid(ceil_div(ceil_div(hidden, 8), threads), tokens);
  hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(threads), 0, static_cast<hipStream_t>(stream), expert_out,
                     inverse_perm, weights, shared, tokens, top_k, hidden, out);
  return check_launch("moe_combine_kernel");
}
