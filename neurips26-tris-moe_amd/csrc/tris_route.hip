// Device-side grouped route builder.
//
// Replaces build_grouped_route (TriSMoE_cuda.cpp:741-793), which runs a torch
// sort, bincount, nonzero and two cumsums and then copies the tile count to
// the host.  Here one launch builds the same metadata on the stream with no
// host round trip (route_group_scatter_kernel, one workgroup per segment
// slot, each of which runs both steps):
//   1. route_histogram_block: per-expert counts in LDS, a block scan over
//      experts, compacted active expert ids, segment_offsets,
//      problem_offsets and {num_active, total_tiles};
//   2. route_scatter_block: a stable counting-sort scatter of the slot's
//      expert; the workgroup scans the flattened expert ids in 1024-element
//      chunks and places its entries in flat order using ballots, a popcount
//      of the lower lanes and the wave totals in LDS.
// For decode-sized batches route_topk_small_kernel does the router softmax
// and top-k (modeling_mixtral.py:548-555) and all of the above in one
// workgroup and one launch.
#include "tris_backbone.h"
#include "tris_route.h"

namespace tris {

constexpr int kRouteThreads = 1024;
constexpr int kRouteMaxExperts = 16384;

// The histogram of the flattened expert ids, the scan over experts and the compacted segments, by one
// workgroup of kRouteThreads threads (cnt: num_experts ints of LDS).  With write_out the workgroup writes
// expert_ids, segment_offsets, problem_offsets and counts; it always leaves, in *slot_e / *slot_pos, the expert
// and first row of segment slot `seg` (-1 when the slot is inactive; for seg == num_experts, the end of the
// valid rows) and in *bad whether an id lay outside [0, num_experts).
__device__ __forceinline__ void route_histogram_block(const int64_t* __restrict__ selected, int total, int num_experts,
                                                      int m_tile, int* cnt, bool write_out,
                                                      int32_t* __restrict__ expert_ids,
                                                      int32_t* __restrict__ segment_offsets,
                                                      int32_t* __restrict__ problem_offsets,
                                                      int32_t* __restrict__ counts, int seg, int* slot_e,
                                                      int* slot_pos, int* bad) {
  __shared__ int scan_active[kRouteThreads];
  __shared__ int scan_rows[kRouteThreads];
  __shared__ int scan_tiles[kRouteThreads];
  const int tid = threadIdx.x;
  for (int e = tid; e < num_experts; e += kRouteThreads) cnt[e] = 0;
  if (tid == 0) {
    *bad = 0;
    *slot_e = -1;
  }
  __syncthreads();
  for (int i = tid; i < total; i += kRouteThreads) {
    const int64_t e = selected[i];
    if (e < 0 || e >= num_experts) {
      *bad = 1;
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
      if (write_out) {
        expert_ids[a] = e;
        segment_offsets[a] = r;
        problem_offsets[a] = t;
      }
      if (a == seg) {
        *slot_e = e;
        *slot_pos = r;
      }
      ++a;
      r += c;
      t += (c + m_tile - 1) / m_tile;
    }
  }
  if (tid == 0 && seg == num_experts) *slot_pos = rows_total;
  if (write_out) {
    for (int j = num_active + tid; j < num_experts; j += kRouteThreads) expert_ids[j] = -1;
    for (int j = num_active + tid; j <= num_experts; j += kRouteThreads) {
      segment_offsets[j] = rows_total;
      problem_offsets[j] = tiles_total;
    }
  }
  __syncthreads();
  if (write_out && tid == 0) {
    // An id outside [0, num_experts) is reported here; the valid entries keep their segments and the
    // scatter places the invalid ones after them (route_scatter_block).
    counts[0] = *bad ? -1 : num_active;
    counts[1] = tiles_total;
  }
}

__global__ __launch_bounds__(kRouteThreads) void route_histogram_kernel(
    const int64_t* __restrict__ selected, int total, int num_experts, int m_tile, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ segment_offsets, int32_t* __restrict__ problem_offsets, int32_t* __restrict__ counts) {
  extern __shared__ int cnt[];  // [num_experts]
  __shared__ int slot_e, slot_pos, bad;
  route_histogram_block(selected, total, num_experts, m_tile, cnt, true, expert_ids, segment_offsets, problem_offsets,
                        counts, -1, &slot_e, &slot_pos, &bad);
}

constexpr int kScatterThreads = 1024;
constexpr int kScatterWaves = kScatterThreads / kWave;

// The stable scatter of segment slot `seg` (expert e, first row pos) by one workgroup of kScatterThreads
// threads: the flattened expert ids are scanned in chunks of kScatterThreads, each chunk's hits placed in flat
// order (ballot within a wave, wave totals through LDS), so a segment's entries keep the order of the flat index
// as in a stable sort.  Slot num_experts (e == -1) places the entries whose id lies outside [0, num_experts)
// after every segment, in flat order, with their own token index and slot, grouped expert id -1 and
// inverse_perm -1: every grouped row then holds a valid token index (the backbone's row gather stays in
// bounds), no segment covers those rows, and the combine skips them.
__device__ __forceinline__ void route_scatter_block(const int64_t* __restrict__ selected, int total, int top_k,
                                                    int num_experts, int seg, int e, int pos,
                                                    int64_t* __restrict__ perm, int64_t* __restrict__ token_idx,
                                                    int64_t* __restrict__ slots, int32_t* __restrict__ grouped_expert_ids,
                                                    int32_t* __restrict__ inverse_perm) {
  __shared__ int wave_hits[2][kScatterWaves];
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const bool invalid_slot = seg == num_experts;
  const uint64_t lower = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int buf = 0;
  for (int c = 0; c < total; c += kScatterThreads) {
    const int i = c + tid;
    bool hit = false;
    if (i < total) {
      const int64_t si = selected[i];
      hit = invalid_slot ? (si < 0 || si >= num_experts) : si == e;
    }
    const uint64_t mask = __ballot(hit);
    if (lane == 0) wave_hits[buf][wave] = __popcll(mask);
    __syncthreads();  // (two buffers: the next chunk's writes do not race this chunk's reads)
    int before = 0, chunk = 0;
#pragma unroll
    for (int w = 0; w < kScatterWaves; ++w) {
      const int h = wave_hits[buf][w];
      before += w < wave ? h : 0;
      chunk += h;
    }
    if (hit) {
      const int dst = pos + before + __popcll(mask & lower);
      perm[dst] = i;
      token_idx[dst] = i / top_k;
      slots[dst] = i % top_k;
      grouped_expert_ids[dst] = e;
      if (inverse_perm != nullptr) inverse_perm[i] = invalid_slot ? -1 : dst;
    }
    pos += chunk;
    buf ^= 1;
  }
}

// The whole route from the flattened ids in one launch: workgroup seg (one per segment slot, and one for the
// invalid ids) builds the histogram and the segments itself (workgroup 0 also writes them out), then scatters
// its slot's entries.  Every workgroup reads all ids: for prefill routes of a few thousand rows that costs
// less than a second launch.
static_assert(kScatterThreads == kRouteThreads, "the histogram and the scatter share the workgroup");
__global__ __launch_bounds__(kScatterThreads) void route_group_scatter_kernel(
    const int64_t* __restrict__ selected, int total, int top_k, int num_experts, int m_tile,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ segment_offsets, int32_t* __restrict__ problem_offsets,
    int32_t* __restrict__ counts, int64_t* __restrict__ perm, int64_t* __restrict__ token_idx,
    int64_t* __restrict__ slots, int32_t* __restrict__ grouped_expert_ids, int32_t* __restrict__ inverse_perm) {
  extern __shared__ int cnt[];  // [num_experts]
  __shared__ int slot_e, slot_pos, bad;
  const int seg = blockIdx.x;
  route_histogram_block(selected, total, num_experts, m_tile, cnt, seg == 0, expert_ids, segment_offsets,
                        problem_offsets, counts, seg, &slot_e, &slot_pos, &bad);
  const bool invalid_slot = seg == num_experts;
  if (invalid_slot ? bad == 0 : slot_e < 0) return;  // every id valid / an inactive slot (the whole workgroup)
  route_scatter_block(selected, total, top_k, num_experts, seg, invalid_slot ? -1 : slot_e, slot_pos, perm, token_idx,
                      slots, grouped_expert_ids, inverse_perm);
}

constexpr int kRouteSmallMaxRows = 2048;    // tokens * top_k
constexpr int kRouteSmallMaxExperts = 1024;

// LDS of the one-workgroup router.
struct RouteSmem {
  int16_t sel[kRouteSmallMaxRows];
  int cnt[kRouteSmallMaxExperts];
  int seg_of[kRouteSmallMaxExperts];                   // segment base of each expert's next tokens
  unsigned long long tok_bits[kRouteSmallMaxExperts];  // the chunk's tokens that picked expert e
  int wave_tot[3][kRouteThreads / kWave];
};

// One token's softmax and top-k by a whole wavefront (wave-uniform call, every lane active): the same picks,
// in the same order, as route_token_topk.  Lane l holds experts l + 64 q (q < P) in registers; the max and
// the exp-sum are wave reductions (a fixed DPP tree: the serial sum's order differs, so a probability can
// differ from route_token_topk's in its last bit; the picks compare those probabilities as the oracle's
// argsort does).  Then top_k rounds, each the wave maximum of the probabilities not yet picked and, by
// ballots over q, the lowest expert holding it (ties to the lower expert id); the owner clears its slot.
// A NaN probability (NaN or infinite logits) counts as 0, so every round finds an expert in range.
// Lane j < top_k returns pick j: its expert and its weight, renormalised over the picks (summed in pick
// order) or not.  pv: the lane's logits (route_load_logits).
template <int P>
__device__ __forceinline__ void route_token_wave(float (&pv)[P], int num_experts, int top_k, int renormalize,
                                                 int& pick_e, float& pick_w);

// The logits of one token for route_token_wave: lane l takes experts l + 64 q.
template <int P>
__device__ __forceinline__ void route_load_logits(const float* __restrict__ row, int num_experts, float (&pv)[P]) {
  const int lane = static_cast<int>(__lane_id());
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int e = lane + kWave * q;
    pv[q] = e < num_experts ? row[e] : -INFINITY;
  }
}

template <int P>
__device__ __forceinline__ void route_token_wave(float (&pv)[P], int num_experts, int top_k, int renormalize,
                                                 int& pick_e, float& pick_w) {
  const int lane = static_cast<int>(__lane_id());
  float lm = pv[0];
#pragma unroll
  for (int q = 1; q < P; ++q) lm = fmaxf(lm, pv[q]);
  const float m = wave_max_f32(lm);
  float ls = 0.0f;
#pragma unroll
  for (int q = 0; q < P; ++q) {
    if (lane + kWave * q < num_experts) ls += expf(pv[q] - m);
  }
  const float sum = wave_sum_f32(ls);
  // Probabilities as int keys: a non-negative float's bits order as a signed int, and every key in range
  // is >= 0, so the -1.0f of an expert out of range or already picked sorts below them all.
  int kv[P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const float p = expf(pv[q] - m) / sum;
    kv[q] = __float_as_int(lane + kWave * q < num_experts ? (p == p ? p : 0.0f) : -1.0f);
  }
  float denom = 0.0f, my_p = 0.0f;
  int my_e = -1;
  for (int j = 0; j < top_k; ++j) {
    int lmax = kv[0];
#pragma unroll
    for (int q = 1; q < P; ++q) lmax = max(lmax, kv[q]);
    const int best = wave_max_nonneg_i32(lmax);  // an unpicked expert in range remains (top_k <= num_experts)
    int e = 0;
    bool found = false;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const uint64_t hit = __ballot(kv[q] == best);
      if (!found && hit != 0) {
        e = kWave * q + __ffsll(static_cast<unsigned long long>(hit)) - 1;
        found = true;
      }
    }
#pragma unroll
    for (int q = 0; q < P; ++q) {
      if (q == (e >> 6) && lane == (e & (kWave - 1))) kv[q] = __float_as_int(-1.0f);
    }
    const float bp = __int_as_float(best);
    if (lane == j) {
      my_p = bp;
      my_e = e;
    }
    denom += bp;
  }
  pick_e = my_e;
  pick_w = renormalize ? my_p / denom : my_p;
}

// One workgroup, one launch: per token softmax and top-k (route_token_wave, one wavefront per token: P
// experts per lane, P * 64 >= num_experts) with optional renormalisation over the k picks and fp16 weights;
// then the histogram and scan of route_histogram_kernel (thread e owns expert e: wave scans by DPP, one LDS
// exchange of the wave totals) and a stable scatter.  A token's picks are distinct experts, so an entry's
// place in its expert's segment is the number of earlier tokens that picked the expert: tokens go in chunks
// of 64, each expert's tokens of the chunk marked in a 64-bit mask, the segment bases advanced by the
// masks' popcounts after each chunk.
// Run by a whole workgroup of kRouteThreads threads (tid = thread index), with its LDS in sm.
template <int P>
__device__ __forceinline__ void route_small_body(const RouteArgs& ra, RouteSmem& sm, int tid) {
  static_assert(kRouteSmallMaxExperts == kRouteThreads, "thread e owns expert e");
  static_assert(kRouteMaxTopK * kWave <= kRouteThreads, "a chunk of 64 tokens' entries fits the workgroup");
  constexpr int kWaves = kRouteThreads / kWave;
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
  int16_t* sel = sm.sel;
  int* cnt = sm.cnt;
  int* seg_of = sm.seg_of;
  unsigned long long* tok_bits = sm.tok_bits;
  int (*wave_tot)[kRouteThreads / kWave] = sm.wave_tot;

  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int e = tid;
  if (e < num_experts) {
    cnt[e] = 0;
    tok_bits[e] = 0ull;
  }
  __syncthreads();
  // ---- softmax and top-k, one wavefront per token; lane j writes pick j.  The wave's next token's logits
  // are loaded while this one is routed.
  float nxt[P];
  if (wave < tokens) route_load_logits<P>(logits + static_cast<int64_t>(wave) * num_experts, num_experts, nxt);
  for (int t = wave; t < tokens; t += kWaves) {
    float pv[P];
#pragma unroll
    for (int q = 0; q < P; ++q) pv[q] = nxt[q];
    if (t + kWaves < tokens) {
      route_load_logits<P>(logits + static_cast<int64_t>(t + kWaves) * num_experts, num_experts, nxt);
    }
    int pe;
    float pw;
    route_token_wave<P>(pv, num_experts, top_k, renormalize, pe, pw);
    if (lane < top_k) {
      const int i = t * top_k + lane;
      sel[i] = static_cast<int16_t>(pe);
      if (selected != nullptr) selected[i] = pe;
      weights16[i] = f2h_bits(pw);
      if (weights32 != nullptr) weights32[i] = pw;
      atomicAdd(&cnt[pe], 1);
    }
  }
  __syncthreads();
  // ---- per-expert counts -> compacted active experts, segment and problem offsets
  const int c = e < num_experts ? cnt[e] : 0;
  const bool act = c > 0;
  const int tiles = act ? (c + m_tile - 1) / m_tile : 0;
  const uint64_t amask = __ballot(act);
  const uint64_t lower = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  const int rows_incl = wave_incl_sum_i32(c);
  const int tiles_incl = wave_incl_sum_i32(tiles);
  if (lane == kWave - 1) {
    wave_tot[0][wave] = __popcll(amask);
    wave_tot[1][wave] = rows_incl;
    wave_tot[2][wave] = tiles_incl;
  }
  __syncthreads();
  int a0 = 0, r0 = 0, t0 = 0, num_active = 0, rows_total = 0, tiles_total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int x = wave_tot[0][w], y = wave_tot[1][w], z = wave_tot[2][w];
    if (w < wave) {
      a0 += x;
      r0 += y;
      t0 += z;
    }
    num_active += x;
    rows_total += y;
    tiles_total += z;
  }
  const int seg = r0 + rows_incl - c;
  if (e < num_experts) seg_of[e] = seg;
  if (act) {
    const int a = a0 + __popcll(amask & lower);
    expert_ids[a] = e;
    segment_offsets[a] = seg;
    problem_offsets[a] = t0 + tiles_incl - tiles;
  }
  for (int j = num_active + tid; j < num_experts; j += kRouteThreads) expert_ids[j] = -1;
  for (int j = num_active + tid; j <= num_experts; j += kRouteThreads) {
    segment_offsets[j] = rows_total;
    problem_offsets[j] = tiles_total;
  }
  if (tid == 0) {
    counts[0] = num_active;
    counts[1] = tiles_total;
  }
  __syncthreads();
  // ---- stable scatter, 64 tokens at a time: thread u takes entry chunk * 64 * top_k + u
  for (int tc = 0; tc < tokens; tc += kWave) {
    const int i = tc * top_k + tid;
    const int t = i / top_k;
    const bool mine = tid < kWave * top_k && t < tokens;
    const int ex = mine ? sel[i] : 0;
    const uint64_t bit = 1ull << (mine ? t - tc : 0);
    if (mine) atomicOr(&tok_bits[ex], static_cast<unsigned long long>(bit));
    __syncthreads();
    if (mine) {
      const int dst = seg_of[ex] + __popcll(tok_bits[ex] & (bit - 1ull));
      perm[dst] = i;
      token_idx[dst] = t;
      slots[dst] = i - t * top_k;
      grouped_expert_ids[dst] = ex;
      if (inverse_perm != nullptr) inverse_perm[i] = dst;
    }
    __syncthreads();
    if (e < num_experts) {
      seg_of[e] += __popcll(tok_bits[e]);
      tok_bits[e] = 0ull;
    }
    __syncthreads();
  }
}

template <int K>
__global__ __launch_bounds__(kWave) void route_topk_wave_kernel(RouteArgs ra) {
  __shared__ float lg[kRouteWaveMaxRows * kRouteLaneMaxExperts];  // the logits, [tokens][num_experts]
  route_wave_body<K>(ra, lg, static_cast<int>(threadIdx.x));
}

template <int P>
__global__ __launch_bounds__(kRouteThreads) void route_topk_small_kernel(RouteArgs ra) {
  __shared__ RouteSmem sm;
  route_small_body<P>(ra, sm, static_cast<int>(threadIdx.x));
}

// Softmax / top-k / renormalisation only, for batches past the one-launch router: one wavefront per token
// (route_token_wave, P experts a lane), tokens spread over the grid; the route is then built by
// route_group_scatter_kernel.  Each wavefront loads its next token's logits while it
// routes the current one.
constexpr int kRouteTokThreads = 256;
constexpr int kRouteTokWaves = kRouteTokThreads / kWave;

template <int P>
__global__ __launch_bounds__(kRouteTokThreads) void route_topk_tokens_kernel(RouteArgs ra) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int stride = static_cast<int>(gridDim.x) * kRouteTokWaves;
  int t = static_cast<int>(blockIdx.x) * kRouteTokWaves + static_cast<int>(threadIdx.x) / kWave;
  float nxt[P];
  if (t < ra.tokens) route_load_logits<P>(ra.logits + static_cast<int64_t>(t) * ra.num_experts, ra.num_experts, nxt);
  for (; t < ra.tokens; t += stride) {
    float pv[P];
#pragma unroll
    for (int q = 0; q < P; ++q) pv[q] = nxt[q];
    if (t + stride < ra.tokens) {
      route_load_logits<P>(ra.logits + static_cast<int64_t>(t + stride) * ra.num_experts, ra.num_experts, nxt);
    }
    int pe;
    float pw;
    route_token_wave<P>(pv, ra.num_experts, ra.top_k, ra.renormalize, pe, pw);
    if (lane < ra.top_k) {
      const int64_t i = static_cast<int64_t>(t) * ra.top_k + lane;
      ra.selected[i] = pe;
      ra.weights16[i] = f2h_bits(pw);
      if (ra.weights32 != nullptr) ra.weights32[i] = pw;
    }
  }
}

// Router variants: the one-wavefront router with pick lists of 2, 8 or 16 entries (the smallest that holds
// top_k: shorter unrolled insertion chains), or the workgroup router with 1, 2, 4, 8 or 16 experts a lane
// (the smallest that covers num_experts: fewer registers of probabilities and ballots per pick).
enum RouteKind : int {
  kRouteWave2, kRouteWave8, kRouteWave16, kRouteSmall1, kRouteSmall2, kRouteSmall4, kRouteSmall8, kRouteSmall16
};

static int route_variant(int tokens, int num_experts, int top_k) {
  if (static_cast<int64_t>(tokens) * top_k <= kRouteWaveMaxRows && num_experts <= kRouteLaneMaxExperts) {
    return top_k <= 2 ? kRouteWave2 : top_k <= 8 ? kRouteWave8 : kRouteWave16;
  }
  const int per_lane = ceil_div(num_experts, kWave);
  return per_lane <= 1   ? kRouteSmall1
         : per_lane <= 2 ? kRouteSmall2
         : per_lane <= 4 ? kRouteSmall4
         : per_lane <= 8 ? kRouteSmall8
                         : kRouteSmall16;
}

// The router in a workgroup of kRouteThreads threads (the one-wavefront variants use its first wavefront).
__device__ __forceinline__ void route_dispatch(const RouteArgs& ra, int kind, RouteSmem& sm, float* lg, int tid) {
  switch (kind) {
    case kRouteWave2: if (tid < kWave) route_wave_body<2>(ra, lg, tid); break;
    case kRouteWave8: if (tid < kWave) route_wave_body<8>(ra, lg, tid); break;
    case kRouteWave16: if (tid < kWave) route_wave_body<kRouteMaxTopK>(ra, lg, tid); break;
    case kRouteSmall1: route_small_body<1>(ra, sm, tid); break;
    case kRouteSmall2: route_small_body<2>(ra, sm, tid); break;
    case kRouteSmall4: route_small_body<4>(ra, sm, tid); break;
    case kRouteSmall8: route_small_body<8>(ra, sm, tid); break;
    default: route_small_body<kRouteSmallMaxExperts / kWave>(ra, sm, tid); break;
  }
}

// The router and the shared backbone projection of the same tokens in one launch (they do not depend on
// each other): workgroup 0 routes; every other workgroup runs kRbSub blocks of the backbone's grid
// (backbone_block, 256 threads each, sharing the workgroup's one barrier).  The two roles never share a
// workgroup, so their LDS is one union.
constexpr int kRbSub = kRouteThreads / kBbThreads;

template <int TT>
union RouteBackboneSmem {
  RouteSmem r;
  float lg[kRouteWaveMaxRows * kRouteLaneMaxExperts];
  f32x4 red[kRbSub][kBbWaves - 1][TT][kWave];
};

template <int TT, int B>
__global__ __launch_bounds__(kRouteThreads) void route_backbone_kernel(RouteArgs ra, int kind, BackboneArgs ba,
                                                                      int bb_blocks, int gx, int gy) {
  __shared__ RouteBackboneSmem<TT> sm;
  const int tid = static_cast<int>(threadIdx.x);
  if (blockIdx.x == 0) {
    route_dispatch(ra, kind, sm.r, sm.lg, tid);
    return;
  }
  const int sub = tid / kBbThreads;
  const int vb = (static_cast<int>(blockIdx.x) - 1) * kRbSub + sub;
  const bool active = vb < bb_blocks;
  const int v = active ? vb : 0;
  backbone_block<TT, B>(ba, active, v % gx, (v / gx) % gy, v / (gx * gy), tid % kBbThreads, sm.red[sub]);
}

// ---- The block's prologue: the router Linear and the expert kernels' input cast in one launch
// (modeling_mixtral.py:546-553: router_logits = self.gate(hidden_states) in the model dtype; hidden_states
// cast to fp16 for the quantised kernels, :83-90).  Workgroup (ex, ty) computes the 16 x 16 tile of logits of
// tokens 16 ty.. and experts 16 ex.. on v_mfma_f32_16x16x32_{bf16,f16} (products exact in fp32, fp32 sums):
// its 16 wavefronts split the hidden dimension, each with kRlBatch K steps of loads in flight, and wavefront 0
// adds the others' partial tiles in wavefront order.  Each logit is rounded once to the model dtype and
// written twice: in that dtype (the block's router_logits output) and widened to fp32 (the softmax input,
// F.softmax(router_logits, dtype=float)).  The workgroups of the first expert tile also write fp16(x) of
// their tokens from the very operands they load (bf16 -> fp32 -> fp16, round to nearest even, as torch's
// .to(float16)), so the cast reads nothing more.  Used for large batches and for rows wider than
// router_linear_small_kernel holds.
constexpr int kRlWaves = 16;
constexpr int kRlThreads = kRlWaves * kWave;
constexpr int kRlBatch = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint4 rl_load16(const uint16_t* __restrict__ p, bool valid) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return valid ? v : make_uint4(0u, 0u, 0u, 0u);
}

// Two bf16 (one word) -> two fp16 (one word), each rounded to nearest even.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
  const float lo = __uint_as_float(w << 16);
  const float hi = __uint_as_float(w & 0xFFFF0000u);
  return static_cast<uint32_t>(f2h_bits(lo)) | (static_cast<uint32_t>(f2h_bits(hi)) << 16);
}

template <bool kBf16>
__global__ __launch_bounds__(kRlThreads) void router_linear_kernel(const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ w, int tokens,
                                                                   int hidden, int num_experts, int kper,
                                                                   uint16_t* __restrict__ logits_out,
                                                                   float* __restrict__ logits_f32,
                                                                   uint16_t* __restrict__ x16) {
  __shared__ f32x4 red[kRlWaves - 1][kWave];
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int i = lane % 16;
  const int kg = lane / 16;
  const int t = static_cast<int>(blockIdx.y) * 16 + i;  // token of this lane's A row
  const int e = static_cast<int>(blockIdx.x) * 16 + i;  // expert of this lane's B column
  const bool tv = t < tokens;
  const bool ev = e < num_experts;
  const uint16_t* xr = x + static_cast<int64_t>(tv ? t : 0) * hidden;
  const uint16_t* wr = w + static_cast<int64_t>(ev ? e : 0) * hidden;
  const bool cast = kBf16 && x16 != nullptr && blockIdx.x == 0 && tv;
  uint16_t* cr = cast ? x16 + static_cast<int64_t>(t) * hidden : nullptr;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int kb = wave * kper;
  const int ke = (kb + kper) < hidden ? (kb + kper) : hidden;
  for (int k0 = kb; k0 < ke; k0 += kRlBatch * 32) {
    uint4 av[kRlBatch], bv[kRlBatch];
#pragma unroll
    for (int u = 0; u < kRlBatch; ++u) {
      const int k = k0 + u * 32 + kg * 8;
      const bool kv = k < ke;  // hidden % 8 == 0: a 16-byte run lies inside the row iff it starts before ke
      av[u] = rl_load16(xr + (kv ? k : 0), kv && tv);
      bv[u] = rl_load16(wr + (kv ? k : 0), kv && ev);
    }
    if (cast) {
#pragma unroll
      for (int u = 0; u < kRlBatch; ++u) {
        const int k = k0 + u * 32 + kg * 8;
        if (k < ke) {
          *reinterpret_cast<uint4*>(cr + k) = make_uint4(bf16x2_to_f16x2(av[u].x), bf16x2_to_f16x2(av[u].y),
                                                         bf16x2_to_f16x2(av[u].z), bf16x2_to_f16x2(av[u].w));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kRlBatch; ++u) {
      if constexpr (kBf16) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[u]),
                                                      __builtin_bit_cast(bf16x8, bv[u]), acc, 0, 0, 0);
      } else {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av[u]),
                                                     __builtin_bit_cast(f16x8, bv[u]), acc, 0, 0, 0);
      }
    }
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int q = 0; q < kRlWaves - 1; ++q) acc += red[q][lane];
  // acc[v] = logit of token 16 ty + 4 kg + v, expert e
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int tt = static_cast<int>(blockIdx.y) * 16 + 4 * kg + v;
    if (tt < tokens && ev) {
      uint16_t bits;
      float val;
      if constexpr (kBf16) {
        uint32_t u = __float_as_uint(acc[v]);
        if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) {
          bits = static_cast<uint16_t>((u >> 16) | 0x40u);  // NaN stays NaN
        } else {
          u += 0x7FFFu + ((u >> 16) & 1u);
          bits = static_cast<uint16_t>(u >> 16);
        }
        val = __uint_as_float(static_cast<uint32_t>(bits) << 16);
      } else {
        bits = f2h_bits(acc[v]);
        val = h2f(bits);
      }
      const int64_t o = static_cast<int64_t>(tt) * num_experts + e;
      logits_out[o] = bits;
      logits_f32[o] = val;
    }
  }
}

// The same outputs for batches up to kRlsMaxTokens (rows of up to 8192 columns), spread over many workgroups:
// workgroup (t, eg) computes token t's
// logits of experts 8 eg .. 8 eg + 7 with VALU dot products.  Thread j takes the 16-byte runs j, j + 256, ...
// of the row; all its loads (x and the 8 weight rows) are issued before any product, each thread sums its
// products in fp32 in run order, the wavefronts reduce by a fixed DPP tree and wavefront 0 adds the four
// wavefront sums in order.  The workgroups of expert group 0 write fp16(x) of their token.
constexpr int kRlsThreads = 256;
constexpr int kRlsExperts = 8;
constexpr int kRlsMaxRuns = 4;  // 16-byte runs per thread held in registers: hidden <= 4 * 256 * 8 = 8192

template <bool kBf16>
__device__ __forceinline__ float rl_dt(uint32_t w, int half) {
  const uint32_t b = half ? (w >> 16) : (w & 0xFFFFu);
  return kBf16 ? __uint_as_float(b << 16) : h2f(static_cast<uint16_t>(b));
}

// Workgroup-part body of router_linear_small_kernel: item (t, eg) by kRlsThreads threads (tid < kRlsThreads),
// with its wavefront sums in part.  It passes exactly one __syncthreads (also when !active), so several items
// can share one larger workgroup.
template <bool kBf16>
__device__ __forceinline__ void router_linear_item(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                   int hidden, int num_experts, int t, int eg, bool active, int tid,
                                                   float (*part)[kRlsExperts], uint16_t* __restrict__ logits_out,
                                                   float* __restrict__ logits_f32, uint16_t* __restrict__ x16) {
  const int e0 = eg * kRlsExperts;
  const int runs = active ? hidden / 8 : 0;
  const uint16_t* xr = x + static_cast<int64_t>(active ? t : 0) * hidden;
  uint4 xv[kRlsMaxRuns], wv[kRlsMaxRuns][kRlsExperts];
#pragma unroll
  for (int m = 0; m < kRlsMaxRuns; ++m) {
    const int c = tid + m * kRlsThreads;
    const bool cv = c < runs;
    xv[m] = rl_load16(xr + (cv ? c : 0) * 8, cv);
#pragma unroll
    for (int q = 0; q < kRlsExperts; ++q) {
      const int e = e0 + q;
      const bool v = cv && e < num_experts;
      wv[m][q] = rl_load16(w + static_cast<int64_t>(e < num_experts ? e : 0) * hidden + (cv ? c : 0) * 8, v);
    }
  }
  if (kBf16 && x16 != nullptr && eg == 0) {
#pragma unroll
    for (int m = 0; m < kRlsMaxRuns; ++m) {
      const int c = tid + m * kRlsThreads;
      if (c < runs) {
        *reinterpret_cast<uint4*>(x16 + static_cast<int64_t>(t) * hidden + c * 8) =
            make_uint4(bf16x2_to_f16x2(xv[m].x), bf16x2_to_f16x2(xv[m].y), bf16x2_to_f16x2(xv[m].z),
                       bf16x2_to_f16x2(xv[m].w));
      }
    }
  }
  float acc[kRlsExperts];
#pragma unroll
  for (int q = 0; q < kRlsExperts; ++q) acc[q] = 0.0f;
#pragma unroll
  for (int m = 0; m < kRlsMaxRuns; ++m) {
    const uint32_t xs[4] = {xv[m].x, xv[m].y, xv[m].z, xv[m].w};
#pragma unroll
    for (int q = 0; q < kRlsExperts; ++q) {
      const uint32_t ws[4] = {wv[m][q].x, wv[m][q].y, wv[m][q].z, wv[m][q].w};
#pragma unroll
      for (int h = 0; h < 8; ++h) acc[q] += rl_dt<kBf16>(xs[h / 2], h & 1) * rl_dt<kBf16>(ws[h / 2], h & 1);
    }
  }
  const int wave = tid / kWave;
#pragma unroll
  for (int q = 0; q < kRlsExperts; ++q) {
    const float v = wave_sum_f32(acc[q]);
    if ((tid & (kWave - 1)) == 0) part[wave][q] = v;
  }
  __syncthreads();
  if (active && tid < kRlsExperts && e0 + tid < num_experts) {
    const float dot = ((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid];
    uint16_t bits;
    float val;
    if constexpr (kBf16) {
      uint32_t u = __float_as_uint(dot);
      if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) {
        bits = static_cast<uint16_t>((u >> 16) | 0x40u);
      } else {
        u += 0x7FFFu + ((u >> 16) & 1u);
        bits = static_cast<uint16_t>(u >> 16);
      }
      val = __uint_as_float(static_cast<uint32_t>(bits) << 16);
    } else {
      bits = f2h_bits(dot);
      val = h2f(bits);
    }
    const int64_t o = static_cast<int64_t>(t) * num_experts + e0 + tid;
    logits_out[o] = bits;
    logits_f32[o] = val;
  }
}

template <bool kBf16>
__global__ __launch_bounds__(kRlsThreads) void router_linear_small_kernel(const uint16_t* __restrict__ x,
                                                                          const uint16_t* __restrict__ w,
                                                                          int hidden, int num_experts,
                                                                          uint16_t* __restrict__ logits_out,
                                                                          float* __restrict__ logits_f32,
                                                                          uint16_t* __restrict__ x16) {
  __shared__ float part[kRlsThreads / kWave][kRlsExperts];
  router_linear_item<kBf16>(x, w, hidden, num_experts, static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y),
                            true, static_cast<int>(threadIdx.x), part, logits_out, logits_f32, x16);
}

// The block's first launch at decode: the router Linear (router_linear_item) and the gate/up backbone
// projections of the same tokens (backbone_block), which do not depend on each other, one item or block per
// workgroup of kBbThreads threads (a 1024-thread workgroup would cap the router body's registers below what
// its loads in flight hold).  The backbone reads the bf16 activations and converts them on load (the bits x16
// holds), since x16 is written in this same launch.  Workgroups [0, rl_items) take the router items (t, eg),
// t-major; the rest the backbone's grid.
template <int TT>
union RouterBackboneSmem {
  float part[kRlsThreads / kWave][kRlsExperts];
  f32x4 red[kBbWaves - 1][TT][kWave];
};

template <int TT, int B>
__global__ __launch_bounds__(kBbThreads) void router_backbone_kernel(const uint16_t* __restrict__ x,
                                                                    const uint16_t* __restrict__ w, int hidden,
                                                                    int num_experts, int rl_items,
                                                                    uint16_t* __restrict__ logits_out,
                                                                    float* __restrict__ logits_f32,
                                                                    uint16_t* __restrict__ x16, BackboneArgs ba,
                                                                    int gx, int gy) {
  static_assert(kRlsThreads == kBbThreads, "one router item or one backbone block per workgroup");
  __shared__ RouterBackboneSmem<TT> sm;
  const int tid = static_cast<int>(threadIdx.x);
  const int b = static_cast<int>(blockIdx.x);
  if (b < rl_items) {
    const int groups = ceil_div(num_experts, kRlsExperts);
    router_linear_item<true>(x, w, hidden, num_experts, b / groups, b % groups, true, tid, sm.part, logits_out,
                             logits_f32, x16);
    return;
  }
  const int v = b - rl_items;
  backbone_block<TT, B, true>(ba, true, v % gx, (v / gx) % gy, v / (gx * gy), tid, sm.red);
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
  const size_t lds = static_cast<size_t>(num_experts > 0 ? num_experts : 1) * sizeof(int);
  if (total == 0) {
    hipLaunchKernelGGL(route_histogram_kernel, dim3(1), dim3(kRouteThreads), lds, s, selected_experts, 0,
                       num_experts, m_tile, expert_ids, segment_offsets, problem_offsets, counts);
    return check_launch("route_histogram_kernel");
  }
  hipLaunchKernelGGL(route_group_scatter_kernel, dim3(num_experts + 1), dim3(kScatterThreads), lds, s,
                     selected_experts, static_cast<int>(total), top_k, num_experts, m_tile, expert_ids, segment_offsets,
                     problem_offsets, counts, perm, grouped_token_indices, grouped_slots, grouped_expert_ids,
                     inverse_perm);
  return check_launch("route_group_scatter_kernel");
}

// Validates tris_route_topk_grouped's arguments and fills ra.
int tris::route_prepare(const float* router_logits, int32_t num_tokens, int32_t num_experts, int32_t top_k,
                         int32_t renormalize, int32_t m_tile, uint16_t* routing_weights_f16, float* routing_weights_f32,
                         int64_t* selected_experts, int64_t* perm, int64_t* grouped_token_indices,
                         int64_t* grouped_slots, int32_t* grouped_expert_ids, int32_t* expert_ids,
                         int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts, int32_t* inverse_perm,
                         RouteArgs* ra, const char* who) {
  TRIS_REQUIRE(num_tokens >= 0 && num_experts > 0 && top_k > 0, "%s: bad shape", who);
  TRIS_REQUIRE(top_k <= num_experts && top_k <= kRouteMaxTopK, "%s: top_k %d (at most %d and num_experts)", who,
               top_k, kRouteMaxTopK);
  TRIS_REQUIRE(num_experts <= kRouteSmallMaxExperts, "%s: num_experts %d exceeds %d", who, num_experts,
               kRouteSmallMaxExperts);
  TRIS_REQUIRE(static_cast<int64_t>(num_tokens) * top_k <= kRouteSmallMaxRows,
               "%s: %lld routed rows exceed %d (use tris_build_grouped_route)", who,
               static_cast<long long>(num_tokens) * top_k, kRouteSmallMaxRows);
  TRIS_REQUIRE(m_tile > 0, "m_tile must be positive");
  TRIS_REQUIRE(counts && segment_offsets && problem_offsets && expert_ids, "%s: null output", who);
  TRIS_REQUIRE(num_tokens == 0 || (router_logits && routing_weights_f16 && perm && grouped_token_indices &&
                                   grouped_slots && grouped_expert_ids),
               "%s: null pointer", who);
  *ra = RouteArgs{router_logits, num_tokens, num_experts, top_k, renormalize, m_tile, routing_weights_f16,
                  routing_weights_f32, selected_experts, perm, grouped_token_indices, grouped_slots,
                  grouped_expert_ids, expert_ids, segment_offsets, problem_offsets, counts, inverse_perm};
  return TRIS_OK;
}

static int launch_route(const RouteArgs& ra, hipStream_t s, const char* who) {
  switch (route_variant(ra.tokens, ra.num_experts, ra.top_k)) {
    case kRouteWave2: hipLaunchKernelGGL((route_topk_wave_kernel<2>), dim3(1), dim3(kWave), 0, s, ra); break;
    case kRouteWave8: hipLaunchKernelGGL((route_topk_wave_kernel<8>), dim3(1), dim3(kWave), 0, s, ra); break;
    case kRouteWave16:
      hipLaunchKernelGGL((route_topk_wave_kernel<kRouteMaxTopK>), dim3(1), dim3(kWave), 0, s, ra);
      break;
    case kRouteSmall1: hipLaunchKernelGGL((route_topk_small_kernel<1>), dim3(1), dim3(kRouteThreads), 0, s, ra); break;
    case kRouteSmall2: hipLaunchKernelGGL((route_topk_small_kernel<2>), dim3(1), dim3(kRouteThreads), 0, s, ra); break;
    case kRouteSmall4: hipLaunchKernelGGL((route_topk_small_kernel<4>), dim3(1), dim3(kRouteThreads), 0, s, ra); break;
    case kRouteSmall8: hipLaunchKernelGGL((route_topk_small_kernel<8>), dim3(1), dim3(kRouteThreads), 0, s, ra); break;
    default:
      hipLaunchKernelGGL((route_topk_small_kernel<kRouteSmallMaxExperts / kWave>), dim3(1), dim3(kRouteThreads), 0, s,
                         ra);
      break;
  }
  return check_launch(who);
}

extern "C" int tris_route_topk_grouped(const float* router_logits, int32_t num_tokens, int32_t num_experts,
                                       int32_t top_k, int32_t renormalize, int32_t m_tile,
                                       uint16_t* routing_weights_f16, float* routing_weights_f32,
                                       int64_t* selected_experts, int64_t* perm, int64_t* grouped_token_indices,
                                       int64_t* grouped_slots, int32_t* grouped_expert_ids, int32_t* expert_ids,
                                       int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts,
                                       int32_t* inverse_perm, void* stream) {
  const char* who = "tris_route_topk_grouped";
  RouteArgs ra;
  int rc = route_prepare(router_logits, num_tokens, num_experts, top_k, renormalize, m_tile, routing_weights_f16,
                         routing_weights_f32, selected_experts, perm, grouped_token_indices, grouped_slots,
                         grouped_expert_ids, expert_ids, segment_offsets, problem_offsets, counts, inverse_perm, &ra,
                         who);
  if (rc) return rc;
  return launch_route(ra, static_cast<hipStream_t>(stream), who);
}

extern "C" int tris_route_topk(const float* router_logits, int32_t num_tokens, int32_t num_experts, int32_t top_k,
                               int32_t renormalize, uint16_t* routing_weights_f16, float* routing_weights_f32,
                               int64_t* selected_experts, void* stream) {
  const char* who = "tris_route_topk";
  TRIS_REQUIRE(num_tokens >= 0 && num_experts > 0 && top_k > 0, "%s: bad shape", who);
  TRIS_REQUIRE(top_k <= num_experts && top_k <= kRouteMaxTopK, "%s: top_k %d (at most %d and num_experts)", who,
               top_k, kRouteMaxTopK);
  TRIS_REQUIRE(num_experts <= kRouteSmallMaxExperts, "%s: num_experts %d exceeds %d", who, num_experts,
               kRouteSmallMaxExperts);
  if (num_tokens == 0) return TRIS_OK;
  TRIS_REQUIRE(router_logits && routing_weights_f16 && selected_experts, "%s: null pointer", who);
  RouteArgs ra{};
  ra.logits = router_logits;
  ra.tokens = num_tokens;
  ra.num_experts = num_experts;
  ra.top_k = top_k;
  ra.renormalize = renormalize;
  ra.weights16 = routing_weights_f16;
  ra.weights32 = routing_weights_f32;
  ra.selected = selected_experts;
  // every token's wavefront resident at once up to 8192 workgroups (32768 tokens), then a grid-stride loop
  const int64_t wgs = (static_cast<int64_t>(num_tokens) + kRouteTokWaves - 1) / kRouteTokWaves;
  const dim3 grid(static_cast<unsigned>(wgs < 8192 ? wgs : 8192));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int per_lane = ceil_div(num_experts, kWave);
  if (per_lane <= 1) {
    hipLaunchKernelGGL((route_topk_tokens_kernel<1>), grid, dim3(kRouteTokThreads), 0, s, ra);
  } else if (per_lane <= 2) {
    hipLaunchKernelGGL((route_topk_tokens_kernel<2>), grid, dim3(kRouteTokThreads), 0, s, ra);
  } else if (per_lane <= 4) {
    hipLaunchKernelGGL((route_topk_tokens_kernel<4>), grid, dim3(kRouteTokThreads), 0, s, ra);
  } else if (per_lane <= 8) {
    hipLaunchKernelGGL((route_topk_tokens_kernel<8>), grid, dim3(kRouteTokThreads), 0, s, ra);
  } else {
    hipLaunchKernelGGL((route_topk_tokens_kernel<kRouteSmallMaxExperts / kWave>), grid, dim3(kRouteTokThreads), 0, s,
                       ra);
  }
  return check_launch(who);
}

// Backbone token tiles per workgroup in the merged launch: the 1024-thread workgroup caps the kernel at 128
// VGPRs, which the 8-step load batches fit with one token tile only.
constexpr int kRbMaxTokens = 64;

extern "C" int tris_route_topk_backbone(const float* router_logits, int32_t num_tokens, int32_t num_experts,
                                        int32_t top_k, int32_t renormalize, int32_t m_tile,
                                        uint16_t* routing_weights_f16, float* routing_weights_f32,
                                        int64_t* selected_experts, int64_t* perm, int64_t* grouped_token_indices,
                                        int64_t* grouped_slots, int32_t* grouped_expert_ids, int32_t* expert_ids,
                                        int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts,
                                        int32_t* inverse_perm, const tris_backbone_pair_job* bb,
                                        int32_t defer_reduce, void* stream) {
  const char* who = "tris_route_topk_backbone";
  RouteArgs ra;
  int rc = route_prepare(router_logits, num_tokens, num_experts, top_k, renormalize, m_tile, routing_weights_f16,
                         routing_weights_f32, selected_experts, perm, grouped_token_indices, grouped_slots,
                         grouped_expert_ids, expert_ids, segment_offsets, problem_offsets, counts, inverse_perm, &ra,
                         who);
  if (rc) return rc;
  TRIS_REQUIRE(bb != nullptr, "%s: null backbone job", who);
  TRIS_REQUIRE(bb->tokens == num_tokens, "%s: the backbone's %d tokens differ from the router's %d", who, bb->tokens,
               num_tokens);
  TRIS_REQUIRE(num_tokens <= kRbMaxTokens, "%s: %d tokens exceed the merged launch's %d", who, num_tokens,
               kRbMaxTokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (num_tokens == 0) return TRIS_OK;
  BackboneArgs ba;
  BackbonePlan pl;
  rc = backbone_prepare_job(bb, &ba, &pl, who);
  if (rc) return rc;
  const int nproj = bb->sv_b != nullptr ? 2 : 1;
  const int gx = pl.row_tiles;
  const int gy = pl.token_groups * pl.slices;
  const int64_t blocks = static_cast<int64_t>(gx) * gy * nproj;
  TRIS_REQUIRE(blocks < (int64_t{1} << 28), "%s: backbone grid too large", who);
  const dim3 grid(static_cast<unsigned>(1 + ceil_div(static_cast<int>(blocks), kRbSub)));
  const int kind = route_variant(num_tokens, num_experts, top_k);
  switch (pl.tt) {
    case 1:
      hipLaunchKernelGGL((route_backbone_kernel<1, 8>), grid, dim3(kRouteThreads), 0, s, ra, kind, ba,
                         static_cast<int>(blocks), gx, gy);
      break;
    case 2:
      hipLaunchKernelGGL((route_backbone_kernel<2, 4>), grid, dim3(kRouteThreads), 0, s, ra, kind, ba,
                         static_cast<int>(blocks), gx, gy);
      break;
    case 3:
      hipLaunchKernelGGL((route_backbone_kernel<3, 4>), grid, dim3(kRouteThreads), 0, s, ra, kind, ba,
                         static_cast<int>(blocks), gx, gy);
      break;
    default:
      hipLaunchKernelGGL((route_backbone_kernel<4, 4>), grid, dim3(kRouteThreads), 0, s, ra, kind, ba,
                         static_cast<int>(blocks), gx, gy);
      break;
  }
  rc = check_launch(who);
  if (rc || pl.slices == 1 || defer_reduce) return rc;
  return launch_backbone_reduce(ba, nproj, s, who);
}

// Batches up to this many tokens take router_linear_small_kernel.
constexpr int kRlsMaxTokens = 512;

extern "C" int tris_router_linear(const uint16_t* x, const uint16_t* router_weight, int32_t tokens, int32_t hidden,
                                  int32_t num_experts, int32_t model_bf16, uint16_t* router_logits,
                                  float* logits_f32, uint16_t* x16, void* stream) {
  const char* who = "tris_router_linear";
  TRIS_REQUIRE(tokens >= 0 && hidden > 0 && num_experts > 0, "%s: bad shape", who);
  if (tokens == 0) return TRIS_OK;
  TRIS_REQUIRE(x && router_weight && router_logits && logits_f32, "%s: null pointer", who);
  TRIS_REQUIRE(hidden % 8 == 0, "%s: hidden %d must be a multiple of 8", who, hidden);
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  TRIS_REQUIRE(a16(x) && a16(router_weight) && a16(x16), "%s: x, the weight and x16 must be 16-byte aligned", who);
  TRIS_REQUIRE(model_bf16 || x16 == nullptr, "%s: x16 is written only for a bf16 model (fp16 x is the input)", who);
  TRIS_REQUIRE(ceil_div(tokens, 16) <= 65535, "%s: %d tokens exceed the grid", who, tokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tokens <= kRlsMaxTokens && hidden <= kRlsMaxRuns * kRlsThreads * 8) {
    // one workgroup per token and 8 experts: T x E/8 workgroups spread small batches over the GPU (the MFMA
    // tile kernel has T/16 of them: at T = 16, 11.7 against 5.7 us); for large batches each of them re-reading
    // the 8 weight rows costs more (T = 2048: 19.6 against the tile kernel's 15.6 us)
    const dim3 g(static_cast<unsigned>(tokens), static_cast<unsigned>(ceil_div(num_experts, kRlsExperts)));
    if (model_bf16) {
      hipLaunchKernelGGL((router_linear_small_kernel<true>), g, dim3(kRlsThreads), 0, s, x, router_weight, hidden,
                         num_experts, router_logits, logits_f32, x16);
    } else {
      hipLaunchKernelGGL((router_linear_small_kernel<false>), g, dim3(kRlsThreads), 0, s, x, router_weight, hidden,
                         num_experts, router_logits, logits_f32, x16);
    }
    return check_launch(who);
  }
  const int kper = ceil_div(ceil_div(hidden, kRlWaves), 32) * 32;
  const dim3 grid(static_cast<unsigned>(ceil_div(num_experts, 16)), static_cast<unsigned>(ceil_div(tokens, 16)));
  if (model_bf16) {
    hipLaunchKernelGGL((router_linear_kernel<true>), grid, dim3(kRlThreads), 0, s, x, router_weight, tokens, hidden,
                       num_experts, kper, router_logits, logits_f32, x16);
  } else {
    hipLaunchKernelGGL((router_linear_kernel<false>), grid, dim3(kRlThreads), 0, s, x, router_weight, tokens, hidden,
                       num_experts, kper, router_logits, logits_f32, x16);
  }
  return check_launch(who);
}

extern "C" int tris_router_backbone(const uint16_t* x, const uint16_t* router_weight, int32_t tokens, int32_t hidden,
                                    int32_t num_experts, uint16_t* router_logits, float* logits_f32, uint16_t* x16,
                                    const tris_backbone_pair_job* bb, void* stream) {
  const char* who = "tris_router_backbone";
  TRIS_REQUIRE(tokens > 0 && hidden > 0 && num_experts > 0, "%s: bad shape", who);
  TRIS_REQUIRE(x && router_weight && router_logits && logits_f32 && x16 && bb, "%s: null pointer", who);
  TRIS_REQUIRE(hidden % 8 == 0 && hidden <= kRlsMaxRuns * kRlsThreads * 8,
               "%s: hidden %d must be a multiple of 8 and at most %d", who, hidden, kRlsMaxRuns * kRlsThreads * 8);
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  TRIS_REQUIRE(a16(x) && a16(router_weight) && a16(x16), "%s: x, the weight and x16 must be 16-byte aligned", who);
  TRIS_REQUIRE(bb->x == x && bb->tokens == tokens && bb->in_features == hidden,
               "%s: the backbone job must project the router's input (job x == x, same tokens and columns)", who);
  TRIS_REQUIRE(tokens <= kRbMaxTokens, "%s: %d tokens exceed the merged launch's %d", who, tokens, kRbMaxTokens);
  BackboneArgs ba;
  BackbonePlan pl;
  int rc = backbone_prepare_job(bb, &ba, &pl, who);
  if (rc) return rc;
  const int nproj = bb->sv_b != nullptr ? 2 : 1;
  const int gx = pl.row_tiles;
  const int gy = pl.token_groups * pl.slices;
  const int64_t blocks = static_cast<int64_t>(gx) * gy * nproj;
  TRIS_REQUIRE(blocks < (int64_t{1} << 28), "%s: backbone grid too large", who);
  const int rl_items = tokens * ceil_div(num_experts, kRlsExperts);
  const dim3 grid(static_cast<unsigned>(rl_items + blocks));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TRIS_RB_LAUNCH(TT, B)                                                                                      \
  hipLaunchKernelGGL((router_backbone_kernel<TT, B>), grid, dim3(kBbThreads), 0, s, x, router_weight, hidden,      \
                     num_experts, rl_items, router_logits, logits_f32, x16, ba, gx, gy)
  switch (pl.tt) {
    case 1: TRIS_RB_LAUNCH(1, 8); break;
    case 2: TRIS_RB_LAUNCH(2, 4); break;
    case 3: TRIS_RB_LAUNCH(3, 4); break;
    default: TRIS_RB_LAUNCH(4, 4); break;
  }
#undef TRIS_RB_LAUNCH
  return check_launch(who);
}
