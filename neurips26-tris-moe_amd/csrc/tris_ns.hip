// Matrix-mode null-space compensation of the grouped expert GEMM: comp[r] = C1_e . (C2_e . x[r]) for the
// rows r of each segment (expert e), both matrices 4-bit packed per expert and concatenated
// (build_grouped_ns_compensation_payload, qlinear_cuda.py:1734-1872; applied by
// run_grouped_structured_expert_forward, :2322-2335, as out.add_(compensation)).
//
// Replaces grouped_ns_compensation_forward (TriSMoE_cuda_kernel.cu:1208-2145 GroupedPacked4LinearOffset*
// kernels).  Two launches:
//   ns_c2_kernel: hidden[r][j] = fp16(sum_c x[r][c] * W2_e[j][c]) for j < rank_e (0 beyond), one
//     workgroup per (16-row tile of one segment, 64 rank indices), four K partitions per workgroup;
//   ns_c1_kernel: comp[r][n] = fp16(sum_j hidden[r][j] * W1_e[n][j]), one workgroup per (16-row tile,
//     256 output columns), the tile's hidden rows in LDS; optionally out[r][n] = fp16(out + comp).
// Weights are the exact dequantised fp16 values fp16((q - z) * s) of PackedQuantMatrix4bit.dequantize
// (qlinear_cuda.py:2761-2786); products and sums in fp32 (the reference's kernels round the weights
// through an fp16 FMA and accumulate pairs in fp16; the oracle is the fp32 product of the exact weights,
// the reference's own fallback F.linear(F.linear(x, c2), c1), qlinear_cuda.py:1943-1946).
//
// Rows of segments routed to no expert or to an expert with rank 0 get comp = 0.  The work is small next
// to the grouped GEMM (rank_e is a few dozen), so these are plain VALU kernels.
#include "tris_common.h"

namespace tris {

constexpr int kNsRows = 16;       // rows per tile (one segment)
constexpr int kNsC2Ranks = 64;    // rank indices per C2 workgroup
constexpr int kNsC2Parts = 4;     // K partitions per C2 workgroup
constexpr int kNsC2Chunk = 256;   // input columns staged per pass
constexpr int kNsC1Cols = 256;    // output columns per C1 workgroup
constexpr int kNsMaxRank = 512;   // hidden columns staged for C1 (fp32 in LDS)

struct NsArgs {
  const uint16_t* x;        // [batch, in]
  const int32_t* expert_ids;
  const int32_t* segment_offsets;
  int num_segments;
  tris_ns_payload ns;
  uint16_t* hidden;         // [batch, max_ns_rank]
  uint16_t* out;            // [batch, out]
  int accumulate;
};

// Row tile t (tiles of <= 16 rows, segment by segment) -> segment, first row, row count; false when t is
// past the last tile.  Thread 0 scans, the workgroup reads the result from LDS.
__device__ bool ns_map_tile(const int32_t* __restrict__ seg, int nseg, int tile, int* s_out, int* row0, int* rc) {
  __shared__ int res[3];
  if (threadIdx.x == 0) {
    int base = 0, found = -1, r0 = 0, cnt = 0;
    for (int s = 0; s < nseg && found < 0; ++s) {
      const int lo = seg[s], hi = seg[s + 1];
      const int t = hi > lo ? (hi - lo + kNsRows - 1) / kNsRows : 0;
      if (tile < base + t) {
        found = s;
        r0 = lo + (tile - base) * kNsRows;
        cnt = (hi - r0) < kNsRows ? (hi - r0) : kNsRows;
      }
      base += t;
    }
    res[0] = found;
    res[1] = r0;
    res[2] = cnt;
  }
  __syncthreads();
  *s_out = res[0];
  *row0 = res[1];
  *rc = res[2];
  __syncthreads();
  return *s_out >= 0;
}

// The 8 exact weights of one packed word: fp16((q_m - z) * s) as floats.
__device__ __forceinline__ void ns_weights8(uint32_t word, int z, float s, float w[8]) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int q = static_cast<int>((word >> (4 * m)) & 0xFu);
    w[m] = h2f(f2h_bits(static_cast<float>(q - z) * s));  // exact product, one rounding
  }
}

__global__ __launch_bounds__(kNsC2Ranks * kNsC2Parts) void ns_c2_kernel(NsArgs a) {
  __shared__ uint16_t xs[kNsRows][kNsC2Chunk];
  __shared__ float part[kNsC2Parts - 1][kNsRows][kNsC2Ranks];
  int s, row0, rc;
  if (!ns_map_tile(a.segment_offsets, a.num_segments, blockIdx.x, &s, &row0, &rc)) return;
  const tris_ns_payload& ns = a.ns;
  const int e = a.expert_ids[s];
  const bool ev = e >= 0 && e < ns.num_experts;
  int rank = ev ? ns.ns_rank_per_expert[e] : 0;
  rank = rank < ns.max_ns_rank ? rank : ns.max_ns_rank;  // a malformed rank never reaches past the tiles
  const int jl = threadIdx.x % kNsC2Ranks;
  const int kp = threadIdx.x / kNsC2Ranks;
  const int j = blockIdx.y * kNsC2Ranks + jl;
  const bool jv = j < rank;
  const int in_f = ns.infeatures;
  const int groups = (in_f + ns.group_size - 1) / ns.group_size;
  const int64_t roff = ev ? ns.ns_c2_rank_offsets[e] : 0;
  const int64_t rwoff = ev ? ns.ns_c2_rank_word_offsets[e] : 0;
  float acc[kNsRows];
#pragma unroll
  for (int r = 0; r < kNsRows; ++r) acc[r] = 0.0f;
  if (rank > 0 && blockIdx.y * kNsC2Ranks < rank) {  // uniform
    for (int c0 = 0; c0 < in_f; c0 += kNsC2Chunk) {
      const int cc = (in_f - c0) < kNsC2Chunk ? (in_f - c0) : kNsC2Chunk;
      for (int idx = threadIdx.x; idx < kNsRows * kNsC2Chunk; idx += blockDim.x) {
        const int r = idx / kNsC2Chunk, c = idx % kNsC2Chunk;
        xs[r][c] = (r < rc && c < cc) ? a.x[static_cast<int64_t>(row0 + r) * in_f + c0 + c] : 0;
      }
      __syncthreads();
      if (jv) {
        // partition kp takes words kp, kp + 4, ... of the chunk (a chunk starts on a word)
        for (int p = kp; p * 8 < cc; p += kNsC2Parts) {
          const int c = c0 + p * 8;
          int g = c / ns.group_size;
          g = g < groups ? g : groups - 1;
          const uint32_t word =
              static_cast<uint32_t>(ns.ns_c2_qweight[static_cast<int64_t>(c >> 3) * ns.total_rank + roff + j]);
          const uint32_t zw =
              static_cast<uint32_t>(ns.ns_c2_qzeros[static_cast<int64_t>(g) * ns.total_rank_words + rwoff + (j >> 3)]);
          const int z = static_cast<int>((zw >> (4 * (j & 7))) & 0xFu) + 1;
          const float sc = h2f(ns.ns_c2_scales[static_cast<int64_t>(g) * ns.total_rank + roff + j]);
          float w[8];
          ns_weights8(word, z, sc, w);
#pragma unroll
          for (int r = 0; r < kNsRows; ++r) {
#pragma unroll
            for (int m = 0; m < 8; ++m) acc[r] += (p * 8 + m < cc ? h2f(xs[r][p * 8 + m]) : 0.0f) * w[m];
          }
        }
      }
      __syncthreads();
    }
  }
  if (kp > 0) {
#pragma unroll
    for (int r = 0; r < kNsRows; ++r) part[kp - 1][r][jl] = acc[r];
  }
  __syncthreads();
  if (kp != 0 || j >= ns.max_ns_rank) return;
  for (int r = 0; r < rc; ++r) {
    float v = acc[r];
#pragma unroll
    for (int q = 0; q < kNsC2Parts - 1; ++q) v += part[q][r][jl];
    a.hidden[static_cast<int64_t>(row0 + r) * ns.max_ns_rank + j] = jv ? f2h_bits(v) : 0;
  }
}

__global__ __launch_bounds__(kNsC1Cols) void ns_c1_kernel(NsArgs a) {
  __shared__ float hs[kNsRows][kNsMaxRank];
  int s, row0, rc;
  if (!ns_map_tile(a.segment_offsets, a.num_segments, blockIdx.x, &s, &row0, &rc)) return;
  const tris_ns_payload& ns = a.ns;
  const int e = a.expert_ids[s];
  const bool ev = e >= 0 && e < ns.num_experts;
  int rank = ev ? ns.ns_rank_per_expert[e] : 0;
  rank = rank < ns.max_ns_rank ? rank : ns.max_ns_rank;  // a malformed rank never reaches past the tiles
  const int out_f = ns.outfeatures;
  const int n = blockIdx.y * kNsC1Cols + threadIdx.x;
  const bool nv = n < out_f;
  for (int idx = threadIdx.x; idx < kNsRows * rank; idx += blockDim.x) {
    const int r = idx / rank, j = idx % rank;
    hs[r][j] = r < rc ? h2f(a.hidden[static_cast<int64_t>(row0 + r) * ns.max_ns_rank + j]) : 0.0f;
  }
  __syncthreads();
  float acc[kNsRows];
#pragma unroll
  for (int r = 0; r < kNsRows; ++r) acc[r] = 0.0f;
  if (nv && rank > 0) {
    const int egs = rank < ns.group_size ? rank : ns.group_size;  // a rank below the group size is one group
    const int eg = (rank + egs - 1) / egs;
    const int64_t wbase = static_cast<int64_t>(ns.ns_c1_rank_word_offsets[e]);
    const int64_t gbase = static_cast<int64_t>(ns.ns_c1_group_offsets[e]);
    const int qzc = (out_f + 7) / 8;
    for (int j0 = 0; j0 < rank; j0 += 8) {
      int g = j0 / egs;
      g = g < eg ? g : eg - 1;
      const uint32_t word = static_cast<uint32_t>(ns.ns_c1_qweight[(wbase + (j0 >> 3)) * out_f + n]);
      const uint32_t zw = static_cast<uint32_t>(ns.ns_c1_qzeros[(gbase + g) * qzc + (n >> 3)]);
      const int z = static_cast<int>((zw >> (4 * (n & 7))) & 0xFu) + 1;
      const float sc = h2f(ns.ns_c1_scales[(gbase + g) * out_f + n]);
      float w[8];
      ns_weights8(word, z, sc, w);
#pragma unroll
      for (int r = 0; r < kNsRows; ++r) {
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[r] += (j0 + m < rank ? hs[r][j0 + m] : 0.0f) * w[m];
      }
    }
  }
  if (!nv) return;
  for (int r = 0; r < rc; ++r) {
    const int64_t o = static_cast<int64_t>(row0 + r) * out_f + n;
    const uint16_t comp = f2h_bits(acc[r]);  // the compensation tensor's fp16 value
    a.out[o] = a.accumulate ? f2h_bits(h2f(a.out[o]) + h2f(comp)) : comp;  // out.add_(compensation)
  }
}

static int check_ns(const tris_ns_payload* ns, const char* who) {
  TRIS_REQUIRE(ns != nullptr, "%s: null payload", who);
  TRIS_REQUIRE(ns->num_experts >= 0 && ns->infeatures >= 0 && ns->outfeatures >= 0 && ns->max_ns_rank >= 0 &&
                   ns->total_rank >= 0 && ns->total_rank_words >= 0,
               "%s: negative shape", who);
  TRIS_REQUIRE(ns->max_ns_rank <= kNsMaxRank, "%s: max_ns_rank %d exceeds %d", who, ns->max_ns_rank, kNsMaxRank);
  if (ns->max_ns_rank > 0) {
    TRIS_REQUIRE(ns->group_size > 0, "%s: group_size must be positive", who);
    TRIS_REQUIRE(ns->ns_rank_per_expert && ns->ns_c2_rank_offsets && ns->ns_c2_rank_word_offsets &&
                     ns->ns_c1_rank_word_offsets && ns->ns_c1_group_offsets && ns->ns_c2_qweight &&
                     ns->ns_c2_qzeros && ns->ns_c2_scales && ns->ns_c1_qweight && ns->ns_c1_qzeros &&
                     ns->ns_c1_scales,
                 "%s: null tensor", who);
  }
  return TRIS_OK;
}

}  // namespace tris

using namespace tris;

extern "C" int tris_grouped_ns_compensation_forward(const uint16_t* x_grouped, int32_t batch,
                                                    const int32_t* expert_ids, const int32_t* segment_offsets,
                                                    int32_t num_segments, const tris_ns_payload* ns,
                                                    uint16_t* hidden, uint16_t* out, int32_t accumulate,
                                                    void* stream) {
  const char* who = "tris_grouped_ns_compensation_forward";
  int rc = check_ns(ns, who);
  if (rc) return rc;
  TRIS_REQUIRE(batch >= 0 && num_segments >= 0, "%s: negative batch or segment count", who);
  if (batch == 0 || num_segments == 0 || ns->outfeatures == 0) return TRIS_OK;
  TRIS_REQUIRE(out != nullptr && expert_ids != nullptr && segment_offsets != nullptr, "%s: null pointer", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  NsArgs a{};
  a.x = x_grouped;
  a.expert_ids = expert_ids;
  a.segment_offsets = segment_offsets;
  a.num_segments = num_segments;
  a.ns = *ns;
  a.hidden = hidden;
  a.out = out;
  a.accumulate = accumulate != 0;
  // row tiles: at most batch / 16 + one partial tile per segment; tiles past the last exit at once
  const int tiles = batch / kNsRows + (num_segments < batch ? num_segments : batch);
  if (ns->max_ns_rank == 0 && accumulate) return TRIS_OK;  // no expert has a compensation term
  if (ns->max_ns_rank > 0) {
    TRIS_REQUIRE(x_grouped != nullptr && hidden != nullptr, "%s: null input or hidden workspace", who);
    hipLaunchKernelGGL(ns_c2_kernel, dim3(tiles, ceil_div(ns->max_ns_rank, kNsC2Ranks)),
                       dim3(kNsC2Ranks * kNsC2Parts), 0, s, a);
    rc = check_launch(who);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(ns_c1_kernel, dim3(tiles, ceil_div(ns->outfeatures, kNsC1Cols)), dim3(kNsC1Cols), 0, s, a);
  return check_launch(who);
}
