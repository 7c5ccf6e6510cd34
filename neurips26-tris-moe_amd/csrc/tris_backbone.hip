// Shared fp16 backbone projection hidden = x * SV^T on MFMA.
//
// Replaces the fp16 branch of QuantLinear.compute_shared_hidden
// (qlinear_cuda.py:4454-4502), an F.linear on cuBLAS, and fuses the
// index_select gather of grouped rows (modeling_mixtral.py:467, :475-476)
// through an optional row index.
//
// Shape: out[T, rank] = x[T, in] . SV[rank, in]^T with fp16 inputs and fp32
// accumulation.  One workgroup = 4 wavefronts computes a 16-token x 16-row
// output tile over a 512-wide slice of `in`; each wavefront issues
// v_mfma_f32_16x16x32_f16 on 32-wide K steps (wave w takes steps w, w+4, ...),
// with 16-byte operand loads from x and SV.  Slices are reduced in LDS inside
// the workgroup and across workgroups through an fp32 partial buffer: the
// last workgroup of a tile (agent-scope counter) sums the partials in slice
// order, writes fp16 and returns its counter to zero, so results are
// deterministic and the workspace needs zeroing only once.
//
// At decode (T <= 16) this kernel is HBM-bound on SV (2*rank*in bytes).
#include "tris_common.h"

namespace tris {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBbWaves = 4;
constexpr int kBbThreads = kBbWaves * kWave;
constexpr int kBbKStep = 32;
constexpr int kBbSlice = 512;  // K per workgroup

struct BackboneArgs {
  const uint16_t* x;
  const int64_t* row_index;
  const uint16_t* sv;
  const uint16_t* in_scale;
  uint16_t* out;
  float* partials;     // [slices, tokens, rank]
  int32_t* counters;   // [token_tiles, row_tiles]
  int tokens;
  int in_features;
  int rank;
  int slices;
};

__device__ __forceinline__ f16x8 load8_f16(const uint16_t* __restrict__ src, int k, int in_features, bool valid,
                                           bool vec_ok) {
  f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (!valid) return v;
  if (vec_ok && k + 8 <= in_features) {
    const uint4 raw = *reinterpret_cast<const uint4*>(src + k);
    v = __builtin_bit_cast(f16x8, raw);
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (k + u < in_features) v[u] = __builtin_bit_cast(_Float16, src[k + u]);
    }
  }
  return v;
}

__global__ __launch_bounds__(kBbThreads) void backbone_kernel(BackboneArgs a) {
  __shared__ f32x4 red[kBbWaves - 1][kWave];
  __shared__ int is_last;
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
  int64_t xrow = t;
  if (t_valid && a.row_index != nullptr) xrow = a.row_index[t];
  const uint16_t* xsrc = a.x + xrow * a.in_features;
  const int r = r0 + i;
  const bool r_valid = r < a.rank;
  const uint16_t* ssrc = a.sv + static_cast<int64_t>(r) * a.in_features;
  const bool vec_ok = (a.in_features % 8) == 0;

  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int kbeg = slice * kBbSlice;
  const int kend = (kbeg + kBbSlice) < a.in_features ? (kbeg + kBbSlice) : a.in_features;
  for (int k0 = kbeg + wave * kBbKStep; k0 < kend; k0 += kBbWaves * kBbKStep) {
    const int k = k0 + kg * 8;
    f16x8 av = load8_f16(xsrc, k, kend, t_valid, vec_ok);
    const f16x8 bv = load8_f16(ssrc, k, kend, r_valid, vec_ok);
    if (a.in_scale != nullptr) {
      const f16x8 sc = load8_f16(a.in_scale, k, kend, true, vec_ok);
      av = av * sc;  // fp16 products, as x * ns_col in the reference
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  for (int w = 0; w < kBbWaves - 1; ++w) acc += red[w][lane];
  // acc[v] = out[t0 + 4*kg + v][r0 + i]
  const int col = r0 + i;
  if (a.slices == 1) {
    if (col < a.rank) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tt = t0 + 4 * kg + v;
        if (tt < a.tokens) a.out[static_cast<int64_t>(tt) * a.rank + col] = f2h_bits(acc[v]);
      }
    }
    return;
  }
  float* part = a.partials + static_cast<int64_t>(slice) * a.tokens * a.rank;
  if (col < a.rank) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int tt = t0 + 4 * kg + v;
      if (tt < a.tokens) part[static_cast<int64_t>(tt) * a.rank + col] = acc[v];
    }
  }
  __threadfence();
  int32_t* counter = a.counters + blockIdx.z * gridDim.x + blockIdx.x;
  if (lane == 0) is_last = (atomicAdd(counter, 1) == a.slices - 1) ? 1 : 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  if (!is_last) return;
  __threadfence();
  if (col < a.rank) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int tt = t0 + 4 * kg + v;
      if (tt < a.tokens) {
        float sum = 0.0f;
        for (int s = 0; s < a.slices; ++s) {
          sum += a.partials[(static_cast<int64_t>(s) * a.tokens + tt) * a.rank + col];
        }
        a.out[static_cast<int64_t>(tt) * a.rank + col] = f2h_bits(sum);
      }
    }
  }
  if (lane == 0) atomicExch(counter, 0);
}

}  // namespace tris

using namespace tris;

extern "C" int64_t tris_backbone_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank) {
  if (tokens <= 0 || in_features <= 0 || rank <= 0) return 0;
  const int64_t slices = ceil_div(in_features, kBbSlice);
  const int64_t counters = static_cast<int64_t>(ceil_div(tokens, 16)) * ceil_div(rank, 16);
  const int64_t part = slices > 1 ? slices * tokens * rank * 4 : 0;
  return ((counters * 4 + 255) / 256) * 256 + part;
}

extern "C" int tris_backbone_linear(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                                    const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  TRIS_REQUIRE(tokens >= 0 && in_features >= 0 && rank >= 0, "tris_backbone_linear: negative shape");
  if (tokens == 0 || rank == 0) return TRIS_OK;
  TRIS_REQUIRE(out != nullptr, "tris_backbone_linear: null output");
  if (in_features == 0) {
    hipError_t err = hipMemsetAsync(out, 0, static_cast<size_t>(tokens) * rank * 2, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) {
      set_error("tris_backbone_linear: %s", hipGetErrorString(err));
      return TRIS_ERR_HIP;
    }
    return TRIS_OK;
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
  const int64_t counter_bytes = ((static_cast<int64_t>(token_tiles) * row_tiles * 4 + 255) / 256) * 256;
  BackboneArgs args{};
  args.x = x;
  args.row_index = row_index;
  args.sv = sv;
  args.in_scale = in_scale;
  args.out = out;
  args.counters = static_cast<int32_t*>(workspace);
  args.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + counter_bytes);
  args.tokens = tokens;
  args.in_features = in_features;
  args.rank = rank;
  args.slices = slices;
  hipLaunchKernelGGL(backbone_kernel, dim3(row_tiles, slices, token_tiles), dim3(kBbThreads), 0,
                     static_cast<hipStream_t>(stream), args);
  return check_launch("backbone_kernel");
}
