// Shared fp16 backbone projection hidden = x * SV^T on MFMA.
//
// Replaces the fp16 branch of QuantLinear.compute_shared_hidden
// (qlinear_cuda.py:4454-4502), an F.linear on cuBLAS, and fuses the
// index_select gather of grouped rows (modeling_mixtral.py:467, :475-476)
// through an optional row index.
//
// Shape: out[T, rank] = x[T, in] . SV[rank, in]^T with fp16 inputs and fp32
// accumulation.  One workgroup = 4 wavefronts computes a 16-token x 16-row
// output tile over one K slice; wavefront w takes a contiguous quarter of the
// slice and issues its 16-byte operand loads in batches of kBbBatch 32-wide K
// steps before the v_mfma_f32_16x16x32_f16, and the four partial tiles are
// added in LDS in wavefront order.  The slice count is chosen so that a decode
// launch has a few hundred workgroups (latency, not MFMA, bounds this
// projection at decode).  With one slice the workgroup writes fp16; otherwise
// it writes fp32 partial tiles to the caller's workspace and
// backbone_reduce_kernel adds the slices in slice order and rounds once, so
// results are deterministic and no workgroups communicate inside a kernel.
// blockIdx.z selects one of up to two projections of the same rows (a gate/up
// pair in one launch).
//
// At decode (T <= 16) the projection is HBM-bound on SV (2*rank*in bytes).
#include "tris_common.h"

namespace tris {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBbWaves = 4;
constexpr int kBbThreads = kBbWaves * kWave;
constexpr int kBbKStep = 32;
constexpr int kBbBatch = 8;          // K steps of loads in flight per wavefront
constexpr int kBbTargetWgs = 512;    // aim for this many workgroups per launch
constexpr int kBbMaxSlices = 32;

struct BackboneProj {
  const uint16_t* sv;
  uint16_t* out;
};

struct BackboneArgs {
  const uint16_t* x;
  const int64_t* row_index;
  const uint16_t* in_scale;
  BackboneProj proj[2];
  float* partials;  // [nproj][slices][tokens][rank] when slices > 1
  int tokens;
  int in_features;
  int rank;
  int slices;
  int slice_k;  // K columns per slice (a multiple of kBbWaves * kBbKStep)
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

// grid = (row tiles, token tiles * slices, projections)
__global__ __launch_bounds__(kBbThreads) void backbone_kernel(BackboneArgs a) {
  __shared__ f32x4 red[kBbWaves - 1][kWave];
  const int q = blockIdx.z;
  const BackboneProj& pj = a.proj[q];
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int r0 = blockIdx.x * 16;
  const int slice = blockIdx.y % a.slices;
  const int t0 = (blockIdx.y / a.slices) * 16;
  const int i = lane % 16;
  const int kg = lane / 16;

  const int t = t0 + i;
  const bool t_valid = t < a.tokens;
  int64_t xrow = 0;
  if (t_valid) xrow = a.row_index != nullptr ? a.row_index[t] : t;
  const uint16_t* xsrc = a.x + xrow * a.in_features;
  const int r = r0 + i;
  const bool r_valid = r < a.rank;
  const uint16_t* ssrc = pj.sv + static_cast<int64_t>(r_valid ? r : 0) * a.in_features;
  const bool scaled = a.in_scale != nullptr;
  const bool vec = (a.in_features % 8) == 0;

  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int kper = a.slice_k / kBbWaves;
  const int kbeg0 = slice * a.slice_k + wave * kper;
  const int kbeg = kbeg0 < a.in_features ? kbeg0 : a.in_features;
  const int kend = (kbeg0 + kper) < a.in_features ? (kbeg0 + kper) : a.in_features;
  int k0 = kbeg;
  if (vec) {
    for (; k0 + kBbBatch * kBbKStep <= kend; k0 += kBbBatch * kBbKStep) {
      f16x8 av[kBbBatch], bv[kBbBatch];
#pragma unroll
      for (int u = 0; u < kBbBatch; ++u) {
        const int k = k0 + u * kBbKStep + kg * 8;
        av[u] = load8_vec(xsrc, k, t_valid);
        bv[u] = load8_vec(ssrc, k, r_valid);
      }
      if (scaled) {
#pragma unroll
        for (int u = 0; u < kBbBatch; ++u) {
          av[u] = av[u] * load8_vec(a.in_scale, k0 + u * kBbKStep + kg * 8, true);  // fp16 products, as x * ns_col
        }
      }
#pragma unroll
      for (int u = 0; u < kBbBatch; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u], bv[u], acc, 0, 0, 0);
    }
  }
  // remaining steps: 16-byte loads for whole runs of 8 columns, element-wise at the end of a row
  for (; k0 < kend; k0 += kBbKStep) {
    const int k = k0 + kg * 8;
    f16x8 av, bv;
    if (vec && k + 8 <= kend) {
      av = load8_vec(xsrc, k, t_valid);
      bv = load8_vec(ssrc, k, r_valid);
      if (scaled) av = av * load8_vec(a.in_scale, k, true);
    } else {
      av = load8_tail(xsrc, k, kend, t_valid);
      bv = load8_tail(ssrc, k, kend, r_valid);
      if (scaled) av = av * load8_tail(a.in_scale, k, kend, true);
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
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
      if (tt < a.tokens) pj.out[static_cast<int64_t>(tt) * a.rank + col] = f2h_bits(acc[v]);
    }
    return;
  }
  float* part = a.partials + (static_cast<int64_t>(q) * a.slices + slice) * a.tokens * a.rank;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int tt = t0 + 4 * kg + v;
    if (tt < a.tokens) part[static_cast<int64_t>(tt) * a.rank + col] = acc[v];
  }
}

// out[q][t][r] = fp16(sum over slices s = 0, 1, ... of partials[q][s][t][r]); blockIdx.y = q.
__global__ __launch_bounds__(256) void backbone_reduce_kernel(BackboneArgs a) {
  const int64_t count = static_cast<int64_t>(a.tokens) * a.rank;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= count) return;
  const int q = blockIdx.y;
  const float* src = a.partials + static_cast<int64_t>(q) * a.slices * count + idx;
  float v[kBbMaxSlices];
#pragma unroll
  for (int s = 0; s < kBbMaxSlices; ++s) v[s] = s < a.slices ? src[s * count] : 0.0f;  // loads in flight together
  float sum = 0.0f;
#pragma unroll
  for (int s = 0; s < kBbMaxSlices; ++s) {
    if (s < a.slices) sum += v[s];
  }
  a.proj[q].out[idx] = f2h_bits(sum);
}

__global__ __launch_bounds__(256) void fill_zero_u16_kernel(uint16_t* __restrict__ out, int64_t count) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx < count) out[idx] = 0;
}

// Slices per projection: enough workgroups to cover the chip at decode, at
// most one slice per kBbWaves*kBbKStep columns and kBbMaxSlices in all.  The
// count does not depend on how many projections share the launch, so a pair
// gives the same bits as two single calls.
int backbone_slices(int tokens, int in_features, int rank) {
  if (tokens <= 0 || in_features <= 0 || rank <= 0) return 1;
  const int64_t tiles = static_cast<int64_t>(ceil_div(tokens, 16)) * ceil_div(rank, 16);
  int64_t slices = (kBbTargetWgs + tiles - 1) / tiles;
  const int64_t max_by_k = ceil_div(in_features, kBbWaves * kBbKStep);
  if (slices > max_by_k) slices = max_by_k;
  if (slices > kBbMaxSlices) slices = kBbMaxSlices;
  return slices < 1 ? 1 : static_cast<int>(slices);
}

int64_t backbone_workspace_bytes(int tokens, int in_features, int rank, int nproj) {
  const int slices = backbone_slices(tokens, in_features, rank);
  return slices > 1 ? static_cast<int64_t>(nproj) * slices * tokens * rank * 4 : 0;
}

int launch_backbone(const uint16_t* x, int tokens, int in_features, const int64_t* row_index, const uint16_t* sv_a,
                    const uint16_t* sv_b, int rank, const uint16_t* in_scale, uint16_t* out_a, uint16_t* out_b,
                    void* workspace, int64_t workspace_bytes, void* stream, const char* who) {
  TRIS_REQUIRE(tokens >= 0 && in_features >= 0 && rank >= 0, "%s: negative shape", who);
  if (tokens == 0 || rank == 0) return TRIS_OK;
  TRIS_REQUIRE(out_a != nullptr && (sv_b == nullptr || out_b != nullptr), "%s: null output", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nproj = sv_b != nullptr ? 2 : 1;
  if (in_features == 0) {
    const int64_t count = static_cast<int64_t>(tokens) * rank;
    for (int q = 0; q < nproj; ++q) {
      hipLaunchKernelGGL(fill_zero_u16_kernel, dim3(static_cast<unsigned>((count + 255) / 256)), dim3(256), 0, s,
                         q ? out_b : out_a, count);
    }
    return check_launch("fill_zero_u16_kernel");
  }
  TRIS_REQUIRE(x && sv_a, "%s: null input", who);
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(sv_a) % 16 == 0 &&
                   (sv_b == nullptr || reinterpret_cast<uintptr_t>(sv_b) % 16 == 0) &&
                   (in_scale == nullptr || reinterpret_cast<uintptr_t>(in_scale) % 16 == 0),
               "%s: x, sv and in_scale must be 16-byte aligned", who);
  const int slices = backbone_slices(tokens, in_features, rank);
  const int64_t need = backbone_workspace_bytes(tokens, in_features, rank, nproj);
  TRIS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
               "%s: workspace of %lld bytes needed, %lld given", who, static_cast<long long>(need),
               static_cast<long long>(workspace_bytes));
  const int token_tiles = ceil_div(tokens, 16);
  const int row_tiles = ceil_div(rank, 16);
  TRIS_REQUIRE(static_cast<int64_t>(token_tiles) * slices <= 65535, "%s: too many tokens", who);
  BackboneArgs args{};
  args.x = x;
  args.row_index = row_index;
  args.in_scale = in_scale;
  args.proj[0] = BackboneProj{sv_a, out_a};
  args.proj[1] = BackboneProj{sv_b, out_b};
  args.partials = static_cast<float*>(workspace);
  args.tokens = tokens;
  args.in_features = in_features;
  args.rank = rank;
  args.slices = slices;
  args.slice_k = ceil_div(ceil_div(in_features, slices), kBbWaves * kBbKStep) * kBbWaves * kBbKStep;
  hipLaunchKernelGGL(backbone_kernel, dim3(row_tiles, token_tiles * slices, nproj), dim3(kBbThreads), 0, s, args);
  int rc = check_launch(who);
  if (rc || slices == 1) return rc;
  const int64_t count = static_cast<int64_t>(tokens) * rank;
  hipLaunchKernelGGL(backbone_reduce_kernel, dim3(static_cast<unsigned>((count + 255) / 256), nproj), dim3(256), 0, s,
                     args);
  return check_launch(who);
}

}  // namespace tris

using namespace tris;

extern "C" int64_t tris_backbone_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank) {
  return backbone_workspace_bytes(tokens, in_features, rank, 1);
}

extern "C" int64_t tris_backbone_pair_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank) {
  return backbone_workspace_bytes(tokens, in_features, rank, 2);
}

extern "C" int tris_backbone_linear(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                                    const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  return launch_backbone(x, tokens, in_features, row_index, sv, nullptr, rank, in_scale, out, nullptr, workspace,
                         workspace_bytes, stream, "tris_backbone_linear");
}

extern "C" int tris_backbone_linear_pair(const uint16_t* x, int32_t tokens, int32_t in_features,
                                         const int64_t* row_index, const uint16_t* sv_a, const uint16_t* sv_b,
                                         int32_t rank, uint16_t* out_a, uint16_t* out_b, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  TRIS_REQUIRE(sv_b != nullptr, "tris_backbone_linear_pair: null sv_b");
  return launch_backbone(x, tokens, in_features, row_index, sv_a, sv_b, rank, nullptr, out_a, out_b, workspace,
                         workspace_bytes, stream, "tris_backbone_linear_pair");
}
