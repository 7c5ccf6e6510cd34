// Shared fp16 backbone projection on MFMA: the tiling, the per-workgroup body and the slice reduction,
// shared by the standalone launches (tris_backbone.hip) and the launches that run the projection beside
// other work (the router's launch, tris_route.hip; the reduction beside the GR predecode, tris_gr.hip).
#pragma once

#include "tris_common.h"

namespace tris {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBbWaves = 4;
constexpr int kBbThreads = kBbWaves * kWave;
constexpr int kBbKStep = 32;
constexpr int kBbBatch = 8;          // K steps of loads in flight per wavefront
constexpr int kBbTargetWgs = 256;    // aim for this many workgroups per launch (MI355X: 512 and 1024 were slower
                                      // at the Mixtral decode shapes, 128 too at T <= 2)
constexpr int kBbPacked4TargetWgs = 512;  // the 4-bit backbone, which dequantises in its loop (256: Mixtral T = 16
                                          // step 108 -> 113 us)
constexpr int kBbMaxSlices = 32;        // slices of backbone_kernel
// the tiled GEMM for prefill-size batches (backbone_gemm_kernel, tris_backbone.hip)
constexpr int kBgM = 256;            // rows of a workgroup tile
constexpr int kBgN = 128;            // rank columns of a workgroup tile
constexpr int kBgK = 32;             // K columns per LDS stage
constexpr int kBgStride = kBgK;      // fp16 per staged row (64 bytes, four 16-byte chunks; see bg_chunk)

// LDS position (fp16 offset) of 16-byte chunk c (0..3) of staged row r: the chunks of a row are permuted by
// f(r) = ((r >> 1) ^ (r >> 3)) & 3, so the 16 rows an MFMA operand read touches (one chunk each) and the four
// rows x four chunks a wavefront's copy writes (16 lanes a pass) fall on distinct banks, for 32 banks and 8
// lanes a pass as for 64 banks and 16 lanes.
__device__ __forceinline__ int bg_chunk(int r, int c) {
  return r * kBgStride + 8 * (c ^ (((r >> 1) ^ (r >> 3)) & 3));
}
constexpr int kBgThreads = 256;
constexpr int kBgMinRows = 512;      // rows from which the entry points take it
constexpr int kBgMinStages = 16;     // K stages per slice at least
constexpr int kBgTargetWgs = 512;    // two workgroups per CU
constexpr int kBgMaxSlices = 16;
constexpr int kBbReduceMaxSlices = 64;  // slices backbone_reduce_at adds (backbone_swiglu_kernel uses up to 64)

struct BackboneProj {
  const uint16_t* sv;
  uint16_t* out;
  const uint16_t* in_scale;  // fp16 [in] per-column input scale of this projection, or null
  // split > 0: the projection is two stacked ones; out holds columns [0, split) as [tokens, split] and out_hi
  // columns [split, rank) as [tokens, rank - split]
  uint16_t* out_hi;
  int split;
};

// Stores output (row, col) of a projection of `rank` columns, through its column split.
__device__ __forceinline__ void bb_store(const BackboneProj& pj, int rank, int64_t row, int col, uint16_t v) {
  if (pj.split > 0 && col >= pj.split) {
    pj.out_hi[row * (rank - pj.split) + (col - pj.split)] = v;
  } else {
    pj.out[row * (pj.split > 0 ? pj.split : rank) + col] = v;
  }
}

struct BackboneArgs {
  const uint16_t* x;
  const int64_t* row_index;
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

// grid = (row tiles, token-tile groups * slices, projections).  A workgroup covers TT token tiles of 16
// rows, so each SV operand load feeds TT MFMAs (SV, the bytes that bound the projection, is read once per
// row tile and slice however many tokens there are, up to 16 * TT); B K steps of loads are in flight per
// wavefront, the last batch of a slice predicated (zero operands past its end).
//
// backbone_block: the work of workgroup (bx, by, bz) of that grid done by kBbThreads threads (tid < kBbThreads),
// with its LDS partial tiles in red.  It passes exactly one __syncthreads (also when !active, a grid slot with
// no work), so several such blocks can share one larger workgroup.
// 8 bf16 (16 bytes) -> 8 fp16, each rounded to nearest even (torch's bf16 .to(float16)).
__device__ __forceinline__ f16x8 bf16x8_to_f16x8(uint4 v) {
  f16x8 r;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[2 * i] = static_cast<_Float16>(__uint_as_float(w[i] << 16));
    r[2 * i + 1] = static_cast<_Float16>(__uint_as_float(w[i] & 0xFFFF0000u));
  }
  return r;
}

__device__ __forceinline__ f16x8 load8_vec_bf16(const uint16_t* __restrict__ src, int k, bool valid) {
  f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (valid) v = bf16x8_to_f16x8(*reinterpret_cast<const uint4*>(src + k));
  return v;
}

// kXBf16: a.x holds bf16 activations, converted to fp16 on load (in_features % 8 == 0: the vector path only).
template <int TT, int B, bool kXBf16 = false>
__device__ __forceinline__ void backbone_block(const BackboneArgs& a, bool active, int bx, int by, int bz, int tid,
                                               f32x4 (*red)[TT][kWave]) {
  const int q = bz;
  const BackboneProj& pj = a.proj[q];
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int r0 = bx * 16;
  const int slice = by % a.slices;
  const int tg0 = (by / a.slices) * TT;  // first token tile of the group
  const int i = lane % 16;
  const int kg = lane / 16;

  bool t_valid[TT];
  const uint16_t* xsrc[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) {
    const int t = (tg0 + j) * 16 + i;
    t_valid[j] = active && t < a.tokens;
    int64_t xrow = 0;
    if (t_valid[j]) xrow = a.row_index != nullptr ? a.row_index[t] : t;
    xsrc[j] = a.x + xrow * a.in_features;
  }
  const int r = r0 + i;
  const bool r_valid = active && r < a.rank;
  const uint16_t* ssrc = pj.sv + static_cast<int64_t>(r_valid ? r : 0) * a.in_features;
  const uint16_t* in_scale = pj.in_scale;
  const bool scaled = in_scale != nullptr;
  const bool vec = (a.in_features % 8) == 0;

  f32x4 acc[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int kper = a.slice_k / kBbWaves;
  const int kbeg0 = active ? slice * a.slice_k + wave * kper : a.in_features;  // an inactive block loops 0 times
  const int kbeg = kbeg0 < a.in_features ? kbeg0 : a.in_features;
  const int kend = (kbeg0 + kper) < a.in_features ? (kbeg0 + kper) : a.in_features;
  if (vec) {
    // every k is a multiple of 8 and so is kend: a 16-byte run is inside the slice iff k < kend
    for (int k0 = kbeg; k0 < kend; k0 += B * kBbKStep) {
      f16x8 bv[B], av[TT][B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int k = k0 + u * kBbKStep + kg * 8;
        const bool kv = k < kend;
        bv[u] = load8_vec(ssrc, k, r_valid && kv);
#pragma unroll
        for (int j = 0; j < TT; ++j) {
          av[j][u] = kXBf16 ? load8_vec_bf16(xsrc[j], k, t_valid[j] && kv) : load8_vec(xsrc[j], k, t_valid[j] && kv);
        }
      }
      if (scaled) {
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int k = k0 + u * kBbKStep + kg * 8;
          const f16x8 sc = load8_vec(in_scale, k, k < kend);
#pragma unroll
          for (int j = 0; j < TT; ++j) av[j][u] = av[j][u] * sc;  // fp16 products, as x * ns_col
        }
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
#pragma unroll
        for (int j = 0; j < TT; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[j][u], bv[u], acc[j], 0, 0, 0);
      }
    }
  } else {
    // rows not a multiple of 8 columns: element-wise loads
    for (int k0 = kbeg; k0 < kend; k0 += kBbKStep) {
      const int k = k0 + kg * 8;
      const f16x8 bv = load8_tail(ssrc, k, kend, r_valid);
      const f16x8 sc = scaled ? load8_tail(in_scale, k, kend, true) : f16x8{1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
      for (int j = 0; j < TT; ++j) {
        f16x8 av = load8_tail(xsrc[j], k, kend, t_valid[j]);
        if (scaled) av = av * sc;
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[j], 0, 0, 0);
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < TT; ++j) red[wave - 1][j][lane] = acc[j];
  }
  __syncthreads();
  const int col = r0 + i;
  if (active && wave == 0) {
#pragma unroll
    for (int j = 0; j < TT; ++j) {
#pragma unroll
      for (int w = 0; w < kBbWaves - 1; ++w) acc[j] += red[w][j][lane];
      // acc[j][v] = out[t0 + 4*kg + v][r0 + i], t0 the tile's first token
      const int t0 = (tg0 + j) * 16;
      float* part = a.partials + (static_cast<int64_t>(q) * a.slices + slice) * a.tokens * a.rank;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tt = t0 + 4 * kg + v;
        if (tt < a.tokens && col < a.rank) {
          if (a.slices == 1) {
            bb_store(pj, a.rank, tt, col, f2h_bits(acc[j][v]));
          } else {
            part[static_cast<int64_t>(tt) * a.rank + col] = acc[j][v];
          }
        }
      }
    }
  }
}

// Output element idx of projection q from the slices' partial sums, added in slice order and rounded once.
__device__ __forceinline__ void backbone_reduce_at(const BackboneArgs& a, int64_t idx, int q) {
  const int64_t count = static_cast<int64_t>(a.tokens) * a.rank;
  if (idx >= count) return;
  const float* src = a.partials + static_cast<int64_t>(q) * a.slices * count + idx;
  float v[kBbReduceMaxSlices];
#pragma unroll
  for (int s = 0; s < kBbReduceMaxSlices; ++s) v[s] = s < a.slices ? src[s * count] : 0.0f;  // loads in flight together
  float sum = 0.0f;
#pragma unroll
  for (int s = 0; s < kBbReduceMaxSlices; ++s) {
    if (s < a.slices) sum += v[s];
  }
  const BackboneProj& pj = a.proj[q];
  if (pj.split > 0) {
    bb_store(pj, a.rank, idx / a.rank, static_cast<int>(idx % a.rank), f2h_bits(sum));
  } else {
    pj.out[idx] = f2h_bits(sum);
  }
}


// Host-side plan of a launch (tris_backbone.hip): slices, token tiles per workgroup and the grid.
struct BackbonePlan {
  int slices;
  int tt;            // token tiles per workgroup
  int token_groups;
  int row_tiles;
  int slice_k;
};
BackbonePlan backbone_plan(int tokens, int in_features, int rank);
int64_t backbone_workspace_bytes(int tokens, int in_features, int rank, int nproj, bool use_gemm = true,
                                 int target = kBbTargetWgs);
bool backbone_gemm_fits(int tokens, int in_features, int rank);
// Validates one launch's arguments (tokens, in_features and rank > 0) and fills args and plan.
int backbone_prepare(const uint16_t* x, int tokens, int in_features, const int64_t* row_index, const uint16_t* sv_a,
                     const uint16_t* sv_b, int rank, const uint16_t* in_scale_a, const uint16_t* in_scale_b,
                     uint16_t* out_a, uint16_t* out_b, void* workspace, int64_t workspace_bytes, BackboneArgs* args,
                     BackbonePlan* plan, const char* who, bool use_gemm = false);
// The slice reduction of a launch that left its partial sums in args.partials (slices > 1).
int launch_backbone_reduce(const BackboneArgs& args, int nproj, hipStream_t s, const char* who);
// backbone_prepare for a tris_backbone_pair_job, with its column split (decode-size launches only: the tiled
// GEMM of prefill batches stores whole rows).
int backbone_prepare_job(const tris_backbone_pair_job* bb, BackboneArgs* args, BackbonePlan* plan, const char* who);

}  // namespace tris
