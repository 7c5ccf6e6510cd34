// The decode router's selection and its one-wavefront route builder, shared by the router launches
// (tris_route.hip) and the predecode launch that runs the route beside the decode (tris_gr.hip), whose
// workgroups derive the routed experts from the same logits with the same code.
#pragma once

#include "tris_common.h"

namespace tris {

constexpr int kRouteMaxTopK = 16;

struct RouteArgs;
// Validates a decode router's arguments (tris_route_topk_grouped's contract) and fills ra (tris_route.hip).
int route_prepare(const float* router_logits, int32_t num_tokens, int32_t num_experts, int32_t top_k,
                  int32_t renormalize, int32_t m_tile, uint16_t* routing_weights_f16, float* routing_weights_f32,
                  int64_t* selected_experts, int64_t* perm, int64_t* grouped_token_indices, int64_t* grouped_slots,
                  int32_t* grouped_expert_ids, int32_t* expert_ids, int32_t* segment_offsets,
                  int32_t* problem_offsets, int32_t* counts, int32_t* inverse_perm, RouteArgs* ra, const char* who);

// The fused router's arguments (tris_route_topk_grouped's outputs, see the header).
struct RouteArgs {
  const float* logits;
  int tokens, num_experts, top_k, renormalize, m_tile;
  uint16_t* weights16;
  float* weights32;
  int64_t* selected;
  int64_t* perm;
  int64_t* token_idx;
  int64_t* slots;
  int32_t* grouped_expert_ids;
  int32_t* expert_ids;
  int32_t* segment_offsets;
  int32_t* problem_offsets;
  int32_t* counts;
  int32_t* inverse_perm;
};

// Softmax of one token's logits (fp32, max-subtracted, summed in expert order) and its top-k by
// probability with ties to the lower expert id (a stable descending sort, as the oracle's argsort):
// bp[j] / be[j] for j < top_k, most probable first.
template <int K>
__device__ __forceinline__ void route_token_topk(const float* __restrict__ row, int num_experts, int top_k,
                                                 float bp[K], int be[K]) {
  float m = row[0];
  for (int e = 1; e < num_experts; ++e) m = fmaxf(m, row[e]);
  float sum = 0.0f;
  for (int e = 0; e < num_experts; ++e) sum += expf(row[e] - m);
#pragma unroll
  for (int j = 0; j < K; ++j) {
    bp[j] = -1.0f;
    be[j] = -1;
  }
  for (int e = 0; e < num_experts; ++e) {
    const float pe = expf(row[e] - m) / sum;
    // insert after every kept entry with probability >= pe (earlier experts win ties)
    if (pe > bp[top_k - 1] || be[top_k - 1] < 0) {
      float cp = pe;
      int ce = e;
      bool shifting = false;  // once placed, every later entry moves down one
#pragma unroll
      for (int j = 0; j < K; ++j) {
        if (j < top_k && (shifting || be[j] < 0 || cp > bp[j])) {
          const float tp = bp[j];
          const int te = be[j];
          bp[j] = cp;
          be[j] = ce;
          cp = tp;
          ce = te;
          shifting = true;
        }
      }
    }
  }
}

// The routing weight of pick j: renormalised over the k picks (summed in pick order) or not.
template <int K>
__device__ __forceinline__ float route_pick_weight(const float bp[K], int top_k, int renormalize, int j) {
  float denom = 0.0f;
#pragma unroll
  for (int q = 0; q < K; ++q) {
    if (q < top_k) denom += bp[q];
  }
  return renormalize ? bp[j] / denom : bp[j];
}

constexpr int kRouteWaveMaxRows = 64;     // routed rows of the one-wavefront router
constexpr int kRouteLaneMaxExperts = 8;   // its experts: a lane routes a token alone

// One wavefront, no barriers, for at most 64 routed rows and 8 experts: lane t < tokens takes token t's
// softmax and top-k (a short serial chain over few experts); lane i < tokens * top_k then holds routed
// entry i (expert sel_i); lane e <
// num_experts counts its expert by ballots, and prefix sums over lanes give the compacted active
// experts and their segment / problem offsets; entry i's place in its segment is the number of
// earlier entries of its expert.  The same outputs as route_topk_small_kernel.
// Run by the first wavefront of a workgroup (lane = thread index < 64); lg: LDS for the logits,
// kRouteWaveMaxRows * kRouteLaneMaxExperts floats.
template <int K>
__device__ __forceinline__ void route_wave_body(const RouteArgs& ra, float* lg, int lane) {
  const float* __restrict__ logits = ra.logits;
  const int tokens = ra.tokens, num_experts = ra.num_experts, top_k = ra.top_k, renormalize = ra.renormalize;
  const int m_tile = ra.m_tile;
  uint16_t* __restrict__ weights16 = ra.weights16;
  float* __restrict__ weights32 = ra.weights32;
  int64_t* __restrict__ selected = ra.selected;
  int64_t* __restrict__ perm = ra.perm;
  int64_t* __restrict__ token_idx = ra.token_idx;
  int64_t* __restrict__ slots = ra.slots;
  int32_t* __restrict__ grouped_expert_ids = ra.grouped_expert_ids;
  int32_t* __restrict__ expert_ids = ra.expert_ids;
  int32_t* __restrict__ segment_offsets = ra.segment_offsets;
  int32_t* __restrict__ problem_offsets = ra.problem_offsets;
  int32_t* __restrict__ counts = ra.counts;
  int32_t* __restrict__ inverse_perm = ra.inverse_perm;

  const int total = tokens * top_k;
  // every load in flight at once (coalesced), then each token reads its row from LDS
  const int nlog = tokens * num_experts;
  for (int u0 = 0; u0 < nlog; u0 += 8 * kWave) {  // 8 loads per lane in flight per round
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = u0 + u * kWave + lane;
      v[u] = logits[idx < nlog ? idx : 0];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = u0 + u * kWave + lane;
      if (idx < nlog) lg[idx] = v[u];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  float bp[K];
  int be[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    bp[j] = -1.0f;
    be[j] = -1;
  }
  if (lane < tokens) {
    route_token_topk<K>(lg + lane * num_experts, num_experts, top_k, bp, be);
#pragma unroll
    for (int j = 0; j < K; ++j) {
      if (j < top_k) {
        const float w = route_pick_weight<K>(bp, top_k, renormalize, j);
        const int i = lane * top_k + j;
        if (selected != nullptr) selected[i] = be[j];
        weights16[i] = f2h_bits(w);
        if (weights32 != nullptr) weights32[i] = w;
      }
    }
  }
  // entry i = t * top_k + j lives in lane t's be[j]
  int sel_i = -1;
  {
    const int t = lane / top_k;
    const int jj = lane - t * top_k;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int v = __shfl(be[j], t < kWave ? t : 0);
      if (j < top_k && j == jj && lane < total) sel_i = v;
    }
  }
  // per-expert counts (lane e) and each entry's earlier entries of its expert
  int cnt = 0, before = 0;
  const uint64_t lower = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  for (int e = 0; e < num_experts; ++e) {
    const uint64_t mask = __ballot(sel_i == e);
    if (lane == e) cnt = __popcll(mask);
    if (sel_i == e) before = __popcll(mask & lower);
  }
  const bool act = lane < num_experts && cnt > 0;
  const int tiles = act ? (cnt + m_tile - 1) / m_tile : 0;
  const uint64_t amask = __ballot(act);
  const int a = __popcll(amask & lower);  // index among active experts
  int rows_incl = cnt, tiles_incl = tiles;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int vr = __shfl_up(rows_incl, d);
    const int vt = __shfl_up(tiles_incl, d);
    if (lane >= d) {
      rows_incl += vr;
      tiles_incl += vt;
    }
  }
  const int num_active = __popcll(amask);
  const int rows_total = __shfl(rows_incl, kWave - 1);
  const int tiles_total = __shfl(tiles_incl, kWave - 1);
  const int seg_start = rows_incl - cnt;  // first row of lane e's segment
  if (act) {
    expert_ids[a] = lane;
    segment_offsets[a] = seg_start;
    problem_offsets[a] = tiles_incl - tiles;
  }
  for (int j = num_active + lane; j < num_experts; j += kWave) expert_ids[j] = -1;
  for (int j = num_active + lane; j <= num_experts; j += kWave) {
    segment_offsets[j] = rows_total;
    problem_offsets[j] = tiles_total;
  }
  if (lane == 0) {
    counts[0] = num_active;
    counts[1] = tiles_total;
  }
  const int seg_of = __shfl(seg_start, sel_i >= 0 ? sel_i : 0);
  if (lane < total) {
    const int dst = seg_of + before;
    perm[dst] = lane;
    token_idx[dst] = lane / top_k;
    slots[dst] = lane % top_k;
    grouped_expert_ids[dst] = sel_i;
    if (inverse_perm != nullptr) inverse_perm[lane] = dst;
  }
}

// The routed experts of a decode route, as route_wave_body writes them to expert_ids: the experts any
// token picked, ascending, then -1 up to num_slots.  One wavefront (every lane active; at most 64 tokens and
// 64 experts), from the router logits in memory with the same selection (route_token_topk), so a workgroup
// that needs only the expert list derives it beside the launch that builds the route, and both agree.
template <int K>
__device__ __forceinline__ void route_active_experts(const float* __restrict__ logits, int tokens, int num_experts,
                                                     int top_k, int lane, int32_t* eids, int num_slots) {
  float bp[K];
  int be[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    bp[j] = -1.0f;
    be[j] = -1;
  }
  if (lane < tokens) route_token_topk<K>(logits + lane * num_experts, num_experts, top_k, bp, be);
  bool picked = false;
  for (int e = 0; e < num_experts; ++e) {
    bool mine = false;
#pragma unroll
    for (int j = 0; j < K; ++j) mine = mine || (j < top_k && be[j] == e);
    const uint64_t m = __ballot(mine);
    if (lane == e) picked = m != 0ull;
  }
  const bool act = lane < num_experts && picked;
  const uint64_t am = __ballot(act);
  const uint64_t lower = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  if (act) eids[__popcll(am & lower)] = lane;
  for (int q = __popcll(am) + lane; q < num_slots; q += kWave) eids[q] = -1;
}

}  // namespace tris
