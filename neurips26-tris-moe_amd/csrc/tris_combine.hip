// Routing-weighted combine of the grouped expert outputs.
//
// Replaces the reference's scatter-add (modeling_mixtral.py:529-536):
//   final.index_add_(0, grouped_token_indices, (down_out * routing).to(bf16))
// which rounds every routed contribution to bf16 and accumulates in bf16.
// Here each token's top-k contributions (fp16 products down_out * w, as in the
// reference) are gathered through the inverse route permutation, summed in
// fp32 together with an optional unrouted shared-expert output, and rounded
// once to the output dtype (bf16, or fp16 for fp16 models).  One thread
// produces 8 consecutive features; reads are 16-byte vector loads.  The
// compensated variants first add a null-space compensation term to each
// expert output row (fp16(out + comp), the reference's out.add_(compensation),
// qlinear_cuda.py:2322-2334), so that the term computed beside the grouped GEMM
// joins it without a launch of its own.  The gated variant joins a shared
// expert through its sigmoid gate, as the Qwen blocks do
// (modeling_qwen2_moe.py:815-818, modeling_qwen3_5_moe.py:186-188).
#include <type_traits>

#include "tris_common.h"

// Every fp16 / bf16 rounding written here is one the reference performs (each torch op rounds its result), so
// the compiler may not fuse a rounded product into the following add: without this, fp16(a + fp16(g * s))
// compiles to one v_fma_f16 and the product's rounding is lost.
#pragma clang fp contract(off)

namespace tris {


// fp16(a + b) for fp16 bit patterns: the exact sum rounded once, as torch's fp16 add_.
__device__ __forceinline__ uint16_t f16_add_bits(uint16_t a, uint16_t b) { return f2h_bits(h2f(a) + h2f(b)); }

// Model-dtype (bf16 or fp16) bit patterns <-> float: exact widening, round-to-nearest-even narrowing.
template <bool kBf16>
__device__ __forceinline__ float dt_to_f32(uint16_t b) {
  return kBf16 ? __uint_as_float(static_cast<uint32_t>(b) << 16) : h2f(b);
}
template <bool kBf16>
__device__ __forceinline__ uint16_t f32_to_dt(float f) {
  return kBf16 ? f32_to_bf16_rne(f) : f2h_bits(f);
}
template <bool kBf16>
__device__ __forceinline__ float round_dt(float f) {
  return dt_to_f32<kBf16>(f32_to_dt<kBf16>(f));
}

// The routed combine, one token per hblocks workgroups of 256 threads, 8 features per thread.  kBf16: the
// output (and, when kGated, the gate's input and weight) are bf16, else fp16.  kGated: the shared expert
// joins through its gate, as the Qwen blocks add it (modeling_qwen2_moe.py:815-818,
// modeling_qwen3_5_moe.py:186-188):
//   final  = dt(routed)                                   the routed sum in the output dtype
//   gate   = dt(sigmoid(dt(gate_in[t] . gate_w)))         the one-output gate Linear, then sigmoid
//   out    = dt(final + dt(gate * dt(shared)))            shared_expert(h).to(dt), gated, added
// Every workgroup of a token reduces the gate's dot product itself (fixed order: per-thread fp32 sums of
// exact products, the wavefront sum, then the four wavefronts in order), so no launch or grid-wide step is
// added.  Without kGated, the shared output (if any) is added to the fp32 routed sum before the one rounding.
// kK > 0: top_k == kK, every pick's row loaded together; kK == 0: any top_k, one pick at a time.
template <bool kBf16, bool kGated, int kK>
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ expert_out,
                                                          const uint16_t* __restrict__ expert_comp,
                                                          const int32_t* __restrict__ inverse_perm,
                                                          const uint16_t* __restrict__ weights,
                                                          const uint16_t* __restrict__ shared,
                                                          const uint16_t* __restrict__ gate_in,
                                                          const uint16_t* __restrict__ gate_w, int tokens, int top_k,
                                                          int hidden, int hblocks, uint16_t* __restrict__ out) {
  const int t = static_cast<int>(blockIdx.x) / hblocks;
  const int h0 = ((static_cast<int>(blockIdx.x) - t * hblocks) * static_cast<int>(blockDim.x) + threadIdx.x) * 8;
  const bool vec = (hidden % 8) == 0;
  // the routed rows first (their loads in flight while the gate's dot product is reduced), then the gate,
  // in which every thread of the workgroup takes part, then the early exit
  const bool valid = t < tokens && h0 < hidden;
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.0f;
  // one slot's rows (and compensation) at column h0 into v, c
  auto load_row = [&](int row, uint16_t v[8], uint16_t c[8]) {
    const uint16_t* src = expert_out + static_cast<int64_t>(row) * hidden + h0;
    if (vec) {
      *reinterpret_cast<uint4*>(v) = *reinterpret_cast<const uint4*>(src);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = (h0 + u < hidden) ? src[u] : 0;
    }
    if (expert_comp != nullptr) {
      const uint16_t* csrc = expert_comp + static_cast<int64_t>(row) * hidden + h0;
      if (vec) {
        *reinterpret_cast<uint4*>(c) = *reinterpret_cast<const uint4*>(csrc);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) c[u] = (h0 + u < hidden) ? csrc[u] : 0;
      }
    }
  };
  auto add_row = [&](uint16_t v[8], const uint16_t c[8], __half w) {
    if (expert_comp != nullptr) {
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = f16_add_bits(v[u], c[u]);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += __half2float(__hmul(__ushort_as_half(v[u]), w));
  };
  const int32_t* inv = inverse_perm + static_cast<int64_t>(t) * top_k;
  const uint16_t* wts = weights + static_cast<int64_t>(t) * top_k;
  if (valid) {
  if constexpr (kK > 0) {
    // every pick's index and weight, then every pick's row, in flight together (a pick the route left out,
    // index -1, reads row 0 and adds nothing); the sum keeps pick order
    int rows[kK];
    uint16_t wbits[kK];
#pragma unroll
    for (int s = 0; s < kK; ++s) {
      rows[s] = inv[s];
      wbits[s] = wts[s];
    }
    uint16_t v[kK][8], c[kK][8];
#pragma unroll
    for (int s = 0; s < kK; ++s) load_row(rows[s] >= 0 ? rows[s] : 0, v[s], c[s]);
#pragma unroll
    for (int s = 0; s < kK; ++s) {
      if (rows[s] >= 0) add_row(v[s], c[s], __ushort_as_half(wbits[s]));
    }
  } else {
    for (int s = 0; s < top_k; ++s) {
      const int row = inv[s];
      if (row < 0) continue;  // a pick the route left out (expert id outside [0, num_experts))
      uint16_t v[8], c[8];
      load_row(row, v, c);
      add_row(v, c, __ushort_as_half(wts[s]));
    }
  }
  }
  // the shared expert's output at these columns, in flight with the gate's loads
  uint16_t sh16[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const uint16_t* ssrc = shared != nullptr ? shared + static_cast<int64_t>(t) * hidden + h0 : nullptr;
  if (valid && ssrc != nullptr) {
    if (vec) {
      *reinterpret_cast<uint4*>(sh16) = *reinterpret_cast<const uint4*>(ssrc);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) sh16[u] = (h0 + u < hidden) ? ssrc[u] : 0;
    }
  }
  float gate = 0.0f;
  if constexpr (kGated) {
    __shared__ float wave_part[4];
    const uint16_t* xr = gate_in + static_cast<int64_t>(t) * hidden;
    float s = 0.0f;
    for (int h = static_cast<int>(threadIdx.x) * 8; h < hidden; h += static_cast<int>(blockDim.x) * 8) {
      uint16_t xv[8], wv[8];
      if (vec) {
        *reinterpret_cast<uint4*>(xv) = *reinterpret_cast<const uint4*>(xr + h);
        *reinterpret_cast<uint4*>(wv) = *reinterpret_cast<const uint4*>(gate_w + h);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          xv[u] = (h + u < hidden) ? xr[h + u] : 0;
          wv[u] = (h + u < hidden) ? gate_w[h + u] : 0;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) s += dt_to_f32<kBf16>(xv[u]) * dt_to_f32<kBf16>(wv[u]);  // exact products
    }
    s = wave_sum_f32(s);
    if ((threadIdx.x & (kWave - 1)) == 0) wave_part[threadIdx.x / kWave] = s;
    __syncthreads();
    const float dot = ((wave_part[0] + wave_part[1]) + wave_part[2]) + wave_part[3];
    const float logit = round_dt<kBf16>(dot);
    gate = round_dt<kBf16>(1.0f / (1.0f + expf(-logit)));
  }
  if (!valid) return;
  uint16_t* dst = out + static_cast<int64_t>(t) * hidden + h0;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (h0 + u >= hidden) continue;
    float v = acc[u];
    if constexpr (kGated) {
      const float sh = round_dt<kBf16>(h2f(sh16[u]));
      v = round_dt<kBf16>(v) + round_dt<kBf16>(gate * sh);
    } else {
      if (ssrc != nullptr) v += h2f(sh16[u]);
    }
    dst[u] = f32_to_dt<kBf16>(v);
  }
}

// One element of act_fn(gate') * up' with gate' = fp16(gate + comp_gate), up' = fp16(up + comp_up) where a
// compensation is given.
__device__ __forceinline__ uint16_t swiglu_comp_bits(uint16_t g, uint16_t u, const uint16_t* cg, const uint16_t* cu,
                                                     int64_t i) {
  if (cg != nullptr) g = f16_add_bits(g, cg[i]);
  if (cu != nullptr) u = f16_add_bits(u, cu[i]);
  return swiglu_bits(g, u);
}

// 8 fp16 values of a 16-byte-aligned tensor, or zeros for a missing one.
__device__ __forceinline__ void load8(const uint16_t* p, int64_t i0, uint32_t w[4]) {
  if (p == nullptr) {
    w[0] = w[1] = w[2] = w[3] = 0u;
    return;
  }
  const uint4 v = *reinterpret_cast<const uint4*>(p + i0);
  w[0] = v.x;
  w[1] = v.y;
  w[2] = v.z;
  w[3] = v.w;
}

// out = act_fn(gate) * up, 8 consecutive elements per thread (16-byte loads when aligned); with comp_gate /
// comp_up, the compensation is added to each operand first.
__global__ __launch_bounds__(256) void swiglu_mul_kernel(const uint16_t* __restrict__ gate,
                                                         const uint16_t* __restrict__ up,
                                                         const uint16_t* __restrict__ comp_gate,
                                                         const uint16_t* __restrict__ comp_up, int64_t count,
                                                         uint16_t* __restrict__ out) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i0 >= count) return;
  if (i0 + 8 <= count) {
    uint32_t g[4], u[4], cg[4], cu[4];
    load8(gate, i0, g);
    load8(up, i0, u);
    load8(comp_gate, i0, cg);
    load8(comp_up, i0, cu);
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint16_t gl = static_cast<uint16_t>(g[k]), gh = static_cast<uint16_t>(g[k] >> 16);
      uint16_t ul = static_cast<uint16_t>(u[k]), uh = static_cast<uint16_t>(u[k] >> 16);
      if (comp_gate != nullptr) {
        gl = f16_add_bits(gl, static_cast<uint16_t>(cg[k]));
        gh = f16_add_bits(gh, static_cast<uint16_t>(cg[k] >> 16));
      }
      if (comp_up != nullptr) {
        ul = f16_add_bits(ul, static_cast<uint16_t>(cu[k]));
        uh = f16_add_bits(uh, static_cast<uint16_t>(cu[k] >> 16));
      }
      o[k] = static_cast<uint32_t>(swiglu_bits(gl, ul)) | (static_cast<uint32_t>(swiglu_bits(gh, uh)) << 16);
    }
    *reinterpret_cast<uint4*>(out + i0) = make_uint4(o[0], o[1], o[2], o[3]);
    return;
  }
  for (int64_t i = i0; i < count; ++i) out[i] = swiglu_comp_bits(gate[i], up[i], comp_gate, comp_up, i);
}

}  // namespace tris

using namespace tris;

static int swiglu_launch(const char* who, const uint16_t* gate, const uint16_t* up, const uint16_t* comp_gate,
                         const uint16_t* comp_up, int64_t count, uint16_t* out, void* stream) {
  TRIS_REQUIRE(count >= 0, "%s: negative count", who);
  if (count == 0) return TRIS_OK;
  TRIS_REQUIRE(gate && up && out, "%s: null pointer", who);
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  TRIS_REQUIRE(a16(gate) && a16(up) && a16(out) && a16(comp_gate) && a16(comp_up), "%s: tensors must be 16-byte aligned",
               who);
  const int64_t threads = 256;
  const int64_t blocks = (count + 8 * threads - 1) / (8 * threads);
  TRIS_REQUIRE(blocks <= 2147483647LL, "%s: too many elements", who);
  hipLaunchKernelGGL(swiglu_mul_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), gate, up, comp_gate, comp_up, count, out);
  return check_launch(who);
}

extern "C" int tris_swiglu_mul(const uint16_t* gate, const uint16_t* up, int64_t count, uint16_t* out, void* stream) {
  return swiglu_launch("tris_swiglu_mul", gate, up, nullptr, nullptr, count, out, stream);
}

extern "C" int tris_swiglu_mul_compensated(const uint16_t* gate, const uint16_t* up, const uint16_t* comp_gate,
                                           const uint16_t* comp_up, int64_t count, uint16_t* out, void* stream) {
  return swiglu_launch("tris_swiglu_mul_compensated", gate, up, comp_gate, comp_up, count, out, stream);
}

static int combine_launch(const char* who, const uint16_t* expert_out, const uint16_t* expert_comp,
                          const int32_t* inverse_perm, const uint16_t* weights, const uint16_t* shared,
                          const uint16_t* gate_in, const uint16_t* gate_w, int32_t tokens, int32_t top_k,
                          int32_t hidden, bool out_bf16, uint16_t* out, void* stream) {
  TRIS_REQUIRE(tokens >= 0 && top_k >= 0 && hidden >= 0, "%s: negative shape", who);
  if (tokens == 0 || hidden == 0) return TRIS_OK;
  TRIS_REQUIRE(out != nullptr && (top_k == 0 || (expert_out && inverse_perm && weights)), "%s: null pointer", who);
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  TRIS_REQUIRE(hidden % 8 != 0 || (a16(expert_out) && a16(expert_comp)),
               "%s: expert_out and expert_comp must be 16-byte aligned", who);
  const bool gated = gate_w != nullptr;
  TRIS_REQUIRE(!gated || (shared != nullptr && gate_in != nullptr),
               "%s: a shared-expert gate needs the shared output and the gate input", who);
  TRIS_REQUIRE(!gated || hidden % 8 != 0 || (a16(gate_in) && a16(gate_w)),
               "%s: gate input and weight must be 16-byte aligned", who);
  const int threads = 256;
  const int hblocks = ceil_div(ceil_div(hidden, 8), threads);
  const int64_t blocks = static_cast<int64_t>(hblocks) * tokens;  // token-major, one dimension (no 65535 limit)
  TRIS_REQUIRE(blocks <= 2147483647LL, "%s: too many tokens (%d)", who, tokens);
  const dim3 grid(static_cast<unsigned>(blocks));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const auto launch = [&](auto bf16_tag, auto gated_tag, auto k_tag) {
    hipLaunchKernelGGL((moe_combine_kernel<decltype(bf16_tag)::value, decltype(gated_tag)::value,
                                           decltype(k_tag)::value>),
                       grid, dim3(threads), 0, st, expert_out, expert_comp, inverse_perm, weights, shared, gate_in,
                       gate_w, tokens, top_k, hidden, hblocks, out);
  };
  const auto by_k = [&](auto bf16_tag, auto gated_tag) {
    if (top_k == 2) {
      launch(bf16_tag, gated_tag, std::integral_constant<int, 2>{});
    } else if (top_k == 8) {
      launch(bf16_tag, gated_tag, std::integral_constant<int, 8>{});
    } else {
      launch(bf16_tag, gated_tag, std::integral_constant<int, 0>{});
    }
  };
  if (out_bf16) {
    if (gated) by_k(std::true_type{}, std::true_type{});
    else by_k(std::true_type{}, std::false_type{});
  } else {
    if (gated) by_k(std::false_type{}, std::true_type{});
    else by_k(std::false_type{}, std::false_type{});
  }
  return check_launch(who);
}

extern "C" int tris_moe_combine(const uint16_t* expert_out, const int32_t* inverse_perm, const uint16_t* weights,
                                const uint16_t* shared, int32_t tokens, int32_t top_k, int32_t hidden,
                                uint16_t* out, void* stream) {
  return combine_launch("tris_moe_combine", expert_out, nullptr, inverse_perm, weights, shared, nullptr, nullptr,
                        tokens, top_k, hidden, true, out, stream);
}

extern "C" int tris_moe_combine_compensated(const uint16_t* expert_out, const uint16_t* expert_comp,
                                            const int32_t* inverse_perm, const uint16_t* weights,
                                            const uint16_t* shared, int32_t tokens, int32_t top_k, int32_t hidden,
                                            uint16_t* out, void* stream) {
  return combine_launch("tris_moe_combine_compensated", expert_out, expert_comp, inverse_perm, weights, shared,
                        nullptr, nullptr, tokens, top_k, hidden, true, out, stream);
}

extern "C" int tris_moe_combine_gated(const uint16_t* expert_out, const uint16_t* expert_comp,
                                      const int32_t* inverse_perm, const uint16_t* weights, const uint16_t* shared,
                                      const uint16_t* shared_gate_input, const uint16_t* shared_gate_weight,
                                      int32_t tokens, int32_t top_k, int32_t hidden, int32_t out_bf16,
                                      uint16_t* out, void* stream) {
  return combine_launch("tris_moe_combine_gated", expert_out, expert_comp, inverse_perm, weights, shared,
                        shared_gate_input, shared_gate_weight, tokens, top_k, hidden, out_bf16 != 0, out, stream);
}
