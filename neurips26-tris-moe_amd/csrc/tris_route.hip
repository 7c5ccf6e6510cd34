// Device-side grouped route builder.
//
// Replaces build_grouped_route (TriSMoE_cuda.cpp:741-793), which runs a torch
// sort, bincount, nonzero and two cumsums and then copies the tile count to
// the host.  Here two small kernels build the same metadata on the stream
// with no host round trip:
//   1. route_histogram_kernel (one workgroup): per-expert counts in LDS,
//      a block scan over experts, compacted active expert ids,
//      segment_offsets, problem_offsets and {num_active, total_tiles}.
//   2. route_scatter_kernel (one wavefront per active expert): a stable
//      counting-sort scatter; each wave scans the flattened expert ids in
//      64-element chunks and places its expert's entries in flat order using
//      a ballot and a popcount of the lower lanes.
#include "tris_common.h"

namespace tris {

constexpr int kRouteThreads = 1024;
constexpr int kRouteMaxExperts = 16384;

__global__ __launch_bounds__(kRouteThreads) void route_histogram_kernel(
    const int64_t* __restrict__ selected, int total, int num_experts, int m_tile, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ segment_offsets, int32_t* __restrict__ problem_offsets, int32_t* __restrict__ counts) {
  extern __shared__ int cnt[];  // [num_experts]
  __shared__ int scan_active[kRouteThreads];
  __shared__ int scan_rows[kRouteThreads];
  __shared__ int scan_tiles[kRouteThreads];
  __shared__ int bad;
  const int tid = threadIdx.x;
  for (int e = tid; e < num_experts; e += kRouteThreads) cnt[e] = 0;
  if (tid == 0) bad = 0;
  __syncthreads();
  for (int i = tid; i < total; i += kRouteThreads) {
    const int64_t e = selected[i];
    if (e < 0 || e >= num_experts) {
      bad = 1;
    } else {
      atomicAdd(&cnt[e], 1);
    }
  }
  __syncthreads();
  // Each thread owns a contiguous chunk of experts.
  const int chunk = (num_experts + kRouteThreads - 1) / kRouteThreads;
  const int e0 = tid * chunk;
  const int e1 = (e0 + chunk) < num_experts ? (e0 + chunk) : num_experts;
  int na = 0, nr = 0, nt = 0;
  for (int e = e0; e < e1; ++e) {
    const int c = cnt[e];
    if (c > 0) {
      ++na;
      nr += c;
      nt += (c + m_tile - 1) / m_tile;
    }
  }
  scan_active[tid] = na;
  scan_rows[tid] = nr;
  scan_tiles[tid] = nt;
  __syncthreads();
  for (int d = 1; d < kRouteThreads; d <<= 1) {
    const int va = tid >= d ? scan_active[tid - d] : 0;
    const int vr = tid >= d ? scan_rows[tid - d] : 0;
    const int vt = tid >= d ? scan_tiles[tid - d] : 0;
    __syncthreads();
    scan_active[tid] += va;
    scan_rows[tid] += vr;
    scan_tiles[tid] += vt;
    __syncthreads();
  }
  const int num_active = scan_active[kRouteThreads - 1];
  const int rows_total = scan_rows[kRouteThreads - 1];
  const int tiles_total = scan_tiles[kRouteThreads - 1];
  int a = scan_active[tid] - na;
  int r = scan_rows[tid] - nr;
  int t = scan_tiles[tid] - nt;
  for (int e = e0; e < e1; ++e) {
    const int c = cnt[e];
    if (c > 0) {
      expert_ids[a] = e;
      segment_offsets[a] = r;
      problem_offsets[a] = t;
      ++a;
      r += c;
      t += (c + m_tile - 1) / m_tile;
    }
  }
  for (int j = num_active + tid; j < num_experts; j += kRouteThreads) expert_ids[j] = -1;
  for (int j = num_active + tid; j <= num_experts; j += kRouteThreads) {
    segment_offsets[j] = rows_total;
    problem_offsets[j] = tiles_total;
  }
  if (tid == 0) {
    counts[0] = bad ? -1 : num_active;
    counts[1] = bad ? 0 : tiles_total;
  }
  if (bad) {
    // Leave no active expert so the scatter writes nothing.
    for (int j = tid; j < num_experts; j += kRouteThreads) expert_ids[j] = -1;
  }
}

__global__ __launch_bounds__(256) void route_scatter_kernel(
    const int64_t* __restrict__ selected, int total, int top_k, int num_experts, const int32_t* __restrict__ expert_ids,
    const int32_t* __restrict__ segment_offsets, int64_t* __restrict__ perm, int64_t* __restrict__ token_idx,
    int64_t* __restrict__ slots, int32_t* __restrict__ grouped_expert_ids, int32_t* __restrict__ inverse_perm) {
  const int seg = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (seg >= num_experts) return;
  const int e = expert_ids[seg];
  if (e < 0) return;
  int pos = segment_offsets[seg];
  const uint64_t lower = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int c = 0; c < total; c += kWave) {
    const int i = c + lane;
    const bool hit = i < total && selected[i] == e;
    const uint64_t mask = __ballot(hit);
    if (hit) {
      const int dst = pos + __popcll(mask & lower);
      perm[dst] = i;
      token_idx[dst] = i / top_k;
      slots[dst] = i % top_k;
      grouped_expert_ids[dst] = e;
      if (inverse_perm != nullptr) inverse_perm[i] = dst;
    }
    pos += __popcll(mask);
  }
}

}  // namespace tris

using namespace tris;

extern "C" int tris_build_grouped_route(const int64_t* selected_experts, int32_t num_tokens, int32_t top_k,
                                        int32_t num_experts, int32_t m_tile, int64_t* perm,
                                        int64_t* grouped_token_indices, int64_t* grouped_slots,
                                        int32_t* grouped_expert_ids, int32_t* expert_ids, int32_t* segment_offsets,
                                        int32_t* problem_offsets, int32_t* counts, int32_t* inverse_perm,
                                        void* stream) {
  TRIS_REQUIRE(num_tokens >= 0 && top_k >= 0, "build_grouped_route: negative shape");
  TRIS_REQUIRE(num_experts >= 0, "num_experts must be non-negative");
  TRIS_REQUIRE(m_tile > 0, "m_tile must be positive");
  TRIS_REQUIRE(num_experts <= kRouteMaxExperts, "build_grouped_route: num_experts %d exceeds %d", num_experts,
               kRouteMaxExperts);
  const int64_t total = static_cast<int64_t>(num_tokens) * top_k;
  TRIS_REQUIRE(total <= (1LL << 30), "build_grouped_route: too many routed rows");
  TRIS_REQUIRE(counts && segment_offsets && problem_offsets && (num_experts == 0 || expert_ids),
               "build_grouped_route: null output");
  TRIS_REQUIRE(total == 0 || (selected_experts && perm && grouped_token_indices && grouped_slots && grouped_expert_ids),
               "build_grouped_route: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(route_histogram_kernel, dim3(1), dim3(kRouteThreads),
                     static_cast<size_t>(num_experts > 0 ? num_experts : 1) * sizeof(int), s, selected_experts,
                     static_cast<int>(total), num_experts, m_tile, expert_ids, segment_offsets, problem_offsets,
                     counts);
  int rc = check_launch("route_histogram_kernel");
  if (rc) return rc;
  if (total == 0 || num_experts == 0) return TRIS_OK;
  const int waves_per_block = 256 / kWave;
  hipLaunchKernelGGL(route_scatter_kernel, dim3(ceil_div(num_experts, waves_per_block)), dim3(256), 0, s,
                     selected_experts, static_cast<int>(total), top_k, num_experts, expert_ids, segment_offsets, perm,
                     grouped_token_indices, grouped_slots, grouped_expert_ids, inverse_perm);
  return check_launch("route_scatter_kernel");
}
