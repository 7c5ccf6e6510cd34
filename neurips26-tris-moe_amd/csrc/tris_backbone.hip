// Shared fp16 backbone projection hidden = x * SV^T on MFMA.
//
// Replaces the fp16 branch of QuantLinear.compute_shared_hidden
// (qlinear_cuda.py:4454-4502), an F.linear on cuBLAS, and fuses the
// index_select gather of grouped rows (modeling_mixtral.py:467, :475-476)
// through an optional row index.
//
// Shape: out[T, rank] = x[T, in] . SV[rank, in]^T with fp16 inputs and fp32
// accumulation.  One workgroup = 4 wavefronts computes a 16-token x 16-row
// output tile over a kBbSlice-wide slice of `in`; wavefront w takes the
// 32-wide K steps w, w+4, ... and issues v_mfma_f32_16x16x32_f16 on 16-byte
// operand loads, kBbUnroll steps of loads in flight before the MFMAs.  The
// four wavefronts are reduced in LDS.  With one slice the workgroup writes
// fp16; otherwise it writes fp32 partial sums and a second kernel adds the
// slices in order and rounds to fp16 (no cross-workgroup communication inside
// a kernel, so results are deterministic).
//
// At decode (T <= 16) the projection is HBM-bound on SV (2*rank*in bytes).
#include "tris_common.h"

namespace tris {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBbWaves = 4;
constexpr int kBbThreads = kBbWaves * kWave;
constexpr int kBbKStep = 32;
constexpr int kBbSlice = 256;   // K per workgroup
constexpr int kBbUnroll = 2;    // K steps per wave per slice (kBbSlice / (kBbWaves * kBbKStep))

struct BackboneArgs {
  const uint16_t* x;
  const int64_t* row_index;
  const uint16_t* sv;
  const uint16_t* in_scale;
  uint16_t* out;
  float* partials;  // [slices, tokens, rank]
  int tokens;
  int in_features;
  int rank;
  int slices;
};

__device__ __forceinline__ f16x8 load8_tail(const uint16_t* __restrict__ src, int k, int limit, bool valid) {
  f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (valid) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (k + u < limit) v[u] = __builtin_bit_cast(_Float16, src[k + u]);
    }
  }
  return v;
}

__device__ __forceinline__ f16x8 load8_vec(const uint16_t* __restrict__ src, int k, bool valid) {
  f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (valid) v = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(src + k));
  return v;
}

__global__ __launch_bounds__(kBbThreads) void backbone_kernel(BackboneArgs a) {
  __shared__ f32x4 red[kBbWaves - 1][kWave];
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int r0 = blockIdx.x * 16;
  const int slice = blockIdx.y;
  const int t0 = blockIdx.z * 16;
  const int i = lane % 16;
  const int kg = lane / 16;

  const int t = t0 + i;
  const bool t_valid = t < a.tokens;
  int64_t xrow = 0;
  if (t_valid) xrow = a.row_index != nullptr ? a.row_index[t] : t;
  const uint16_t* xsrc = a.x + xrow * a.in_features;
  const int r = r0 + i;
  const bool r_valid = r < a.rank;
  const uint16_t* ssrc = a.sv + static_cast<int64_t>(r_valid ? r : 0) * a.in_features;

  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int kbeg = slice * kBbSlice;
  const int kend = (kbeg + kBbSlice) < a.in_features ? (kbeg + kBbSlice) : a.in_features;
  const bool full = (kend - kbeg) == kBbSlice && (a.in_features % 8) == 0;
  if (full) {
    f16x8 av[kBbUnroll], bv[kBbUnroll], sc[kBbUnroll];
#pragma unroll
    for (int u = 0; u < kBbUnroll; ++u) {
      const int k = kbeg + (u * kBbWaves + wave) * kBbKStep + kg * 8;
      av[u] = load8_vec(xsrc, k, t_valid);
      bv[u] = load8_vec(ssrc, k, r_valid);
      if (a.in_scale != nullptr) sc[u] = load8_vec(a.in_scale, k, true);
    }
#pragma unroll
    for (int u = 0; u < kBbUnroll; ++u) {
      if (a.in_scale != nullptr) av[u] = av[u] * sc[u];  // fp16 products, as x * ns_col in the reference
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u], bv[u], acc, 0, 0, 0);
    }
  } else {
    for (int k0 = kbeg + wave * kBbKStep; k0 < kend; k0 += kBbWaves * kBbKStep) {
      const int k = k0 + kg * 8;
      f16x8 av = load8_tail(xsrc, k, kend, t_valid);
      const f16x8 bv = load8_tail(ssrc, k, kend, r_valid);
      if (a.in_scale != nullptr) av = av * load8_tail(a.in_scale, k, kend, true);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
    }
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kBbWaves - 1; ++w) acc += red[w][lane];
  // acc[v] = out[t0 + 4*kg + v][r0 + i]
  const int col = r0 + i;
  if (col >= a.rank) return;
  if (a.slices == 1) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int tt = t0 + 4 * kg + v;
      if (tt < a.tokens) a.out[static_cast<int64_t>(tt) * a.rank + col] = f2h_bits(acc[v]);
    }
    return;
  }
  float* part = a.partials + static_cast<int64_t>(slice) * a.tokens * a.rank;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int tt = t0 + 4 * kg + v;
    if (tt < a.tokens) part[static_cast<int64_t>(tt) * a.rank + col] = acc[v];
  }
}

// out[t][r] = fp16(sum over slices, in slice order).
__global__ __launch_bounds__(256) void backbone_reduce_kernel(const float* __restrict__ partials,
                                                              uint16_t* __restrict__ out, int64_t count, int slices) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= count) return;
  float sum = 0.0f;
  for (int s = 0; s < slices; ++s) sum += partials[s * count + idx];
  out[idx] = f2h_bits(sum);
}

__global__ __launch_bounds__(256) void fill_zero_u16_kernel(uint16_t* __restrict__ out, int64_t count) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx < count) out[idx] = 0;
}

}  // namespace tris

using namespace tris;

extern "C" int64_t tris_backbone_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank) {
  if (tokens <= 0 || in_features <= 0 || rank <= 0) return 0;
  const int64_t slices = ceil_div(in_features, kBbSlice);
  return slices > 1 ? slices * tokens * rank * 4 : 0;
}

extern "C" int tris_backbone_linear(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                                    const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  TRIS_REQUIRE(tokens >= 0 && in_features >= 0 && rank >= 0, "tris_backbone_linear: negative shape");
  if (tokens == 0 || rank == 0) return TRIS_OK;
  TRIS_REQUIRE(out != nullptr, "tris_backbone_linear: null output");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_features == 0) {
    const int64_t count = static_cast<int64_t>(tokens) * rank;
    hipLaunchKernelGGL(fill_zero_u16_kernel, dim3(static_cast<unsigned>((count + 255) / 256)), dim3(256), 0, s, out,
                       count);
    return check_launch("fill_zero_u16_kernel");
  }
  TRIS_REQUIRE(x && sv, "tris_backbone_linear: null input");
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(sv) % 16 == 0 &&
                   (in_scale == nullptr || reinterpret_cast<uintptr_t>(in_scale) % 16 == 0),
               "tris_backbone_linear: x, sv and in_scale must be 16-byte aligned");
  const int64_t need = tris_backbone_workspace_bytes(tokens, in_features, rank);
  TRIS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
               "tris_backbone_linear: workspace of %lld bytes needed, %lld given", static_cast<long long>(need),
               static_cast<long long>(workspace_bytes));
  const int slices = ceil_div(in_features, kBbSlice);
  const int token_tiles = ceil_div(tokens, 16);
  const int row_tiles = ceil_div(rank, 16);
  TRIS_REQUIRE(token_tiles <= 65535 && slices <= 65535, "tris_backbone_linear: grid too large");
  BackboneArgs args{};
  args.x = x;
  args.row_index = row_index;
  args.sv = sv;
  args.in_scale = in_scale;
  args.out = out;
  args.partials = static_cast<float*>(workspace);
  args.tokens = tokens;
  args.in_features = in_features;
  args.rank = rank;
  args.slices = slices;
  hipLaunchKernelGGL(backbone_kernel, dim3(row_tiles, slices, token_tiles), dim3(kBbThreads), 0, s, args);
  int rc = check_launch("backbone_kernel");
  if (rc || slices == 1) return rc;
  const int64_t count = static_cast<int64_t>(tokens) * rank;
  hipLaunchKernelGGL(backbone_reduce_kernel, dim3(static_cast<unsigned>((count + 255) / 256)), dim3(256), 0, s,
                     args.partials, out, count, slices);
  return check_launch("backbone_reduce_kernel");
}
