// Block-GR predecode and dense-decode kernels.
//
// Predecode replaces Compact3TriSMoEGroupedBlockGRPredecodeKernel
// (TriSMoE_cuda_kernel.cu:4683-4718), which decodes each block serially on
// thread 0.  Here a workgroup builds the byte decode table in LDS once, then
// every group of S lanes decodes one block (tris_gr_span.h), so a 256-lane
// workgroup decodes 256/S blocks at once; the decoded words leave LDS as
// coalesced stores.  Work per block hardly depends on S; more lanes per block
// shorten each lane's walk (latency), fewer cut the scan steps, so S is chosen
// from the block count.
#include "tris_backbone.h"
#include "tris_gr_span.h"
#include "tris_moe_hip.h"
#include "tris_route.h"

namespace tris {

constexpr int kSpanThreads = 256;
constexpr int kSpanWaves = kSpanThreads / kWave;
constexpr int kSpanWgTarget = 1280;  // persistent workgroups per launch: five per CU (LDS and VGPRs allow five)

// One projection's stream; jobs of one launch share the routed expert list.
struct GrJob {
  int32_t* out;
  const int32_t* words;
  const int32_t* offsets;
  const int32_t* meta;
  int num_experts;
  int words_stride;
  int nblk;
  int num_out_blocks;
  int dense_rows;  // 0: predecode layout [slot][block][128]; else dense [slot][packed_rows][N]
  int dense_cols;
};

struct GrJobs {
  GrJob job[TRIS_MAX_PREDECODE_JOBS];
};

// Work items: (job, slot, batch of kWave / S blocks), job-major, then slot, then batch; an item is one
// wavefront's.  The grid is persistent over them: a workgroup copies the tables and the slots' expert ids to
// LDS once, then each wavefront takes items on its own (no workgroup barrier after the copy): it zeroes its
// blocks' LDS bitmaps, decodes them and stores them with 16-byte stores.  The next item's block headers are
// loaded before the current item is decoded and its span words after, so their latency overlaps the decode;
// the first item's headers are loaded before the table copy.
struct GrWork {
  int num_jobs;
  int num_slots;
  int first[TRIS_MAX_PREDECODE_JOBS + 1];  // first item of each job; first[num_jobs] = all items
  int reduce_wgs;  // workgroups that reduce a backbone's slices (GrReduce), dispatched before the decoders
  int decode_wgs;  // workgroups that decode, after them
};

// The decode route built in the same launch (tris_route_predecode_multi_reduce): workgroup 0 runs
// route_wave_body, and every decode workgroup derives its slots' experts from the
// same logits (route_active_experts) instead of reading expert_ids, which that workgroup is still writing; with
// decode_all (tris_route_predecode_all_reduce) the decoders take every expert, slot e for expert e, and read
// nothing the route writes.
struct GrRoute {
  RouteArgs ra;
  int k_variant;  // the route_wave_body instance: 2, 8 or kRouteMaxTopK (by top_k, as tris_route_topk_grouped)
  int wg;         // its workgroup index (0: the decoders follow it), or -1: no route in this launch
  int decode_all;  // 1: the decoders take every expert, slot = expert id, and do not read the logits
};

// A backbone projection's slice reduction run by workgroups of the same launch, dispatched after the route's and
// before the decoders (independent work): blocks_per_proj workgroups of kSpanThreads output elements for each of
// nproj projections.
struct GrReduce {
  BackboneArgs bb;
  int blocks_per_proj;
};

constexpr int kSpanLdsSlots = 256;  // expert ids staged in LDS (later slots read from memory)

template <int S>
struct GrItem {
  int q, slot, block0;
  GrSpan<S> sp;
};

// Item w's job, slot and first block, and its block headers (an empty item past the last).  eids: the slots'
// expert ids in LDS (the first kSpanLdsSlots), or null: every id read from expert_ids.
template <int S>
__device__ __forceinline__ void gr_item_header(const GrJobs& jobs, const GrWork& wk, const int32_t* __restrict__ eids,
                                               const int32_t* __restrict__ expert_ids, int w, int g, GrItem<S>& it) {
  constexpr int kBlocksPerItem = kWave / S;
  const bool exists = w < wk.first[wk.num_jobs];
  const int wv = exists ? w : 0;
  int q = 0;
#pragma unroll
  for (int i = 1; i < TRIS_MAX_PREDECODE_JOBS; ++i) q += (i < wk.num_jobs && wv >= wk.first[i]) ? 1 : 0;
  const GrJob& jb = jobs.job[q];
  const int nblk = jb.nblk;
  const int batches = ceil_div(nblk, kBlocksPerItem);
  const int local = wv - wk.first[q];
  it.q = q;
  it.slot = local / batches;
  it.block0 = (local - it.slot * batches) * kBlocksPerItem;
  // the slot is wave-uniform: one LDS read or one global load, not a load through a pointer selected
  // between LDS and memory (a flat load, which each later LDS wait would wait for)
  int expert;
  if (eids != nullptr && it.slot < kSpanLdsSlots) {
    expert = as_lds(eids)[it.slot];
  } else {
    expert = as_gmem(expert_ids)[it.slot];
  }
  const bool ev = exists && expert >= 0 && expert < jb.num_experts;
  const int ex = ev ? expert : 0;
  gr_span_header<S>(it.sp, jb.words + static_cast<int64_t>(ex) * jb.words_stride,
                    jb.offsets + static_cast<int64_t>(ex) * (nblk + 1), jb.meta + static_cast<int64_t>(ex) * nblk,
                    it.block0 + g, ev && it.block0 + g < nblk, expert_ids);
}

template <int S>
__global__ __launch_bounds__(kSpanThreads) __attribute__((amdgpu_waves_per_eu(5))) void gr_decode_span_kernel(GrJobs jobs, GrWork wk,
                                                                      const int32_t* __restrict__ expert_ids,
                                                                      GrReduce red, GrRoute rt) {
  constexpr int kBlocksPerItem = kWave / S;
  constexpr int kItemVec4 = kBlocksPerItem * kGrWords / 4;
  static_assert(kGrBlockStride % 4 == 0 && kGrPadFront % 4 == 0, "16-byte aligned block bitmaps");
  static_assert(kSpanWaves * kBlocksPerItem * kGrBlockStride >= kRouteWaveMaxRows * kRouteLaneMaxExperts,
                "the route workgroup's logits fit the decode buffers");
  __shared__ GrTables tab;
  __shared__ GrTables4 tab4;
  __shared__ __attribute__((aligned(16))) uint32_t outb[kSpanWaves][kBlocksPerItem * kGrBlockStride];
  __shared__ int32_t eids[kSpanLdsSlots];
  __shared__ int32_t weids[kSpanWaves][kRouteLaneMaxExperts];  // each wavefront's expert list (route in launch)
  const int tid = threadIdx.x;
  // with a route in the launch, workgroup 0 builds it (dispatched first, so its latency overlaps the decode);
  // the reduction workgroups follow, then the decoders (so the reductions are resident from the start, not
  // queued behind a grid of decoders that fills every CU)
  const int rbid = static_cast<int>(blockIdx.x) - (rt.wg >= 0 ? 1 : 0);
  if (rbid < wk.reduce_wgs) {
    if (rbid < 0) {  // the route (its logits staged in the decode buffers' LDS)
      float* lg = reinterpret_cast<float*>(&outb[0][0]);
      if (tid < kWave) {
        if (rt.k_variant == 2) route_wave_body<2>(rt.ra, lg, tid);
        else if (rt.k_variant == 8) route_wave_body<8>(rt.ra, lg, tid);
        else route_wave_body<kRouteMaxTopK>(rt.ra, lg, tid);
      }
      return;
    }
    const int q = rbid / red.blocks_per_proj;
    backbone_reduce_at(red.bb, static_cast<int64_t>(rbid % red.blocks_per_proj) * kSpanThreads + threadIdx.x, q);
    return;
  }
  const int bid = rbid - wk.reduce_wgs;
  const int total = wk.first[wk.num_jobs];
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform: what it selects stays scalar
  const int lane = tid % kWave;
  const int g = lane / S;
  const int j = lane % S;
  const int stride = wk.decode_wgs * kSpanWaves;
  int w = bid * kSpanWaves + wave;
  GrItem<S> cur;
  const int32_t* my_eids = eids;
  if (rt.wg >= 0) {
    // Each wavefront derives the slots' experts from the logits itself (the route workgroup writes expert_ids
    // meanwhile): the logits staged in its own decode buffer (one coalesced read; the host bounds tokens x
    // experts by that buffer), the router's selection on them, the list in its own LDS words.  Every slot of a
    // decode route is listed (num_slots <= kRouteLaneMaxExperts), so expert_ids is never read.  Its first
    // header is then in flight during the table copy, as without a route.
    expert_ids = reinterpret_cast<const int32_t*>(rt.ra.logits);  // any readable word, for invalid headers
    if (rt.decode_all) {
      // every expert in its own slot (num_slots = num_experts): nothing waits for the logits
      for (int i = lane; i < wk.num_slots; i += kWave) weids[wave][i] = i;
    } else {
      float* wl = reinterpret_cast<float*>(outb[wave]);
      const int nlog = rt.ra.tokens * rt.ra.num_experts;
      for (int i = lane; i < nlog; i += kWave) wl[i] = rt.ra.logits[i];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      if (rt.k_variant == 2) {
        route_active_experts<2>(wl, rt.ra.tokens, rt.ra.num_experts, rt.ra.top_k, lane, weids[wave], wk.num_slots);
      } else if (rt.k_variant == 8) {
        route_active_experts<8>(wl, rt.ra.tokens, rt.ra.num_experts, rt.ra.top_k, lane, weids[wave], wk.num_slots);
      } else {
        route_active_experts<kRouteMaxTopK>(wl, rt.ra.tokens, rt.ra.num_experts, rt.ra.top_k, lane, weids[wave],
                                            wk.num_slots);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    my_eids = weids[wave];
    gr_item_header<S>(jobs, wk, my_eids, expert_ids, w, g, cur);  // in flight during the copies below
    gr_tables_to_lds(&tab);
    gr_tables4_to_lds(&tab4);
    gr_span_words<S>(cur.sp, j);
    __syncthreads();
  } else {
    gr_item_header<S>(jobs, wk, nullptr, expert_ids, w, g, cur);  // in flight during the copies below
    const int nl = wk.num_slots < kSpanLdsSlots ? wk.num_slots : kSpanLdsSlots;
    for (int i = tid; i < nl; i += kSpanThreads) eids[i] = expert_ids[i];
    gr_tables_to_lds(&tab);
    gr_tables4_to_lds(&tab4);
    gr_span_words<S>(cur.sp, j);
    __syncthreads();
  }
  uint32_t* ob = outb[wave];
  for (; w < total; w += stride) {
    uint4* z = reinterpret_cast<uint4*>(ob);
    for (int q = lane; q < kBlocksPerItem * kGrBlockStride / 4; q += kWave) z[q] = make_uint4(0u, 0u, 0u, 0u);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    GrItem<S> nx;
    gr_item_header<S>(jobs, wk, my_eids, expert_ids, w + stride, g, nx);
    gr_decode_block_group<S>(cur.sp, &tab, ob + g * kGrBlockStride + kGrPadFront, j, &tab4);
    gr_span_words<S>(nx.sp, j);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const GrJob& jb = jobs.job[cur.q];
    const int nblk = jb.nblk;
    const int block0 = cur.block0;
    const int slot = cur.slot;
    if (jb.dense_rows == 0) {
      // the item's blocks are consecutive in [slot][block][128]: one contiguous run of 16-byte stores
      uint4* dst = reinterpret_cast<uint4*>(jb.out + (static_cast<int64_t>(slot) * nblk + block0) * kGrWords);
#pragma unroll
      for (int q = lane; q < kItemVec4; q += kWave) {
        const int b = q / (kGrWords / 4);
        if (block0 + b < nblk) {
          dst[q] = *reinterpret_cast<const uint4*>(ob + b * kGrBlockStride + kGrPadFront + 4 * (q % (kGrWords / 4)));
        }
      }
    } else {
      int32_t* dst = jb.out + static_cast<int64_t>(slot) * jb.dense_rows * jb.dense_cols;
      for (int idx = lane; idx < kBlocksPerItem * kGrWords; idx += kWave) {
        const int b = block0 + idx / kGrWords;
        if (b >= nblk) continue;
        const int wd = idx % kGrWords;
        const int row = (b / jb.num_out_blocks) * kGrPackedRows + wd / kTileOut;
        const int col = (b % jb.num_out_blocks) * kTileOut + wd % kTileOut;
        if (row < jb.dense_rows && col < jb.dense_cols) {
          dst[static_cast<int64_t>(row) * jb.dense_cols + col] =
              static_cast<int32_t>(ob[(idx / kGrWords) * kGrBlockStride + kGrPadFront + wd]);
        }
      }
    }
    cur = nx;
    // the stores' LDS reads come before the next item's zeroing in this wavefront's LDS order
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
}

// Fills job from one projection's arguments; returns the job's block count (0: nothing to do).
int make_gr_job(GrJob* job, int32_t* out, const int32_t* words, const int32_t* offsets, const int32_t* meta,
                int num_experts, int words_stride, int packed_rows, int outfeatures, bool dense, const char* who) {
  TRIS_REQUIRE(packed_rows >= 0 && outfeatures >= 0 && words_stride >= 0 && num_experts >= 0,
               "%s: negative size", who);
  const int nob = ceil_div(outfeatures, kTileOut);
  const int nblk = ceil_div(packed_rows, kGrPackedRows) * nob;
  *job = GrJob{out, words, offsets, meta, num_experts, words_stride, nblk, nob, dense ? packed_rows : 0,
               dense ? outfeatures : 0};
  if (nblk == 0) return TRIS_OK;
  TRIS_REQUIRE(out && offsets && meta && words, "%s: null pointer", who);
  return TRIS_OK;
}

// reduce: a backbone launch's deferred slice reduction to run in the same launch (or null); route: the decode
// route to build in the same launch (or null: expert_ids holds it already).
int launch_gr_jobs(const GrJobs& jobs, int num_jobs, const int32_t* expert_ids, int num_slots, void* stream,
                   const char* who, const BackboneArgs* reduce = nullptr, int reduce_nproj = 0,
                   const GrRoute* route = nullptr) {
  int max_nblk = 0;
  int64_t total = 0;
  for (int q = 0; q < num_jobs; ++q) {
    max_nblk = jobs.job[q].nblk > max_nblk ? jobs.job[q].nblk : max_nblk;
    total += static_cast<int64_t>(jobs.job[q].nblk) * num_slots;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  TRIS_REQUIRE(route == nullptr || num_slots <= kRouteLaneMaxExperts,
               "%s: a route in the predecode launch takes at most %d slots", who, kRouteLaneMaxExperts);
  if (route == nullptr && (num_slots == 0 || max_nblk == 0)) {
    return reduce != nullptr ? launch_backbone_reduce(*reduce, reduce_nproj, s, who) : TRIS_OK;
  }
  if (max_nblk == 0) num_slots = 0;  // a route (and a reduction) with nothing to decode: no decode workgroups
  TRIS_REQUIRE(route != nullptr || expert_ids != nullptr, "%s: null expert ids", who);
  TRIS_REQUIRE(num_slots <= 65535, "%s: too many experts (%d)", who, num_slots);
  // lanes per block: more lanes shorten each block's walk, fewer spread the per-workgroup table copy
  // over more blocks
  // with a route in the launch each wavefront stages the logits in its decode buffer (kWave / S blocks)
  const int64_t route_floats = route != nullptr ? static_cast<int64_t>(route->ra.tokens) * route->ra.num_experts : 0;
  const int S = (total > 8192 || route_floats > (kWave / 32) * kGrBlockStride) ? 16 : 32;
  TRIS_REQUIRE(route_floats <= (kWave / 16) * kGrBlockStride, "%s: %lld router logits exceed a wavefront's buffer",
               who, static_cast<long long>(route_floats));
  const int per_item = kWave / S;
  GrWork wk{};
  wk.num_jobs = num_jobs;
  wk.num_slots = num_slots;
  int64_t items = 0;
  for (int q = 0; q < num_jobs; ++q) {
    wk.first[q] = static_cast<int>(items);
    items += static_cast<int64_t>(num_slots) * ceil_div(jobs.job[q].nblk, per_item);
  }
  TRIS_REQUIRE(items < (1LL << 30), "%s: too many blocks", who);
  for (int q = num_jobs; q <= TRIS_MAX_PREDECODE_JOBS; ++q) wk.first[q] = static_cast<int>(items);
  GrReduce red{};
  int64_t reduce_wgs = 0;
  if (reduce != nullptr) {
    red.bb = *reduce;
    const int64_t per_proj = (static_cast<int64_t>(reduce->tokens) * reduce->rank + kSpanThreads - 1) / kSpanThreads;
    TRIS_REQUIRE(per_proj < (1LL << 30), "%s: backbone reduction too large", who);
    red.blocks_per_proj = static_cast<int>(per_proj);
    reduce_wgs = per_proj * reduce_nproj;
  }
  red.blocks_per_proj = red.blocks_per_proj > 0 ? red.blocks_per_proj : 1;
  TRIS_REQUIRE(reduce_wgs < (1LL << 30), "%s: too many reduction workgroups", who);
  wk.reduce_wgs = static_cast<int>(reduce_wgs);
  // persistent workgroups: one wavefront per item up to what is resident beside the route and reduction
  // workgroups (kSpanWgTarget in all), so every item that can run at once does; past that each wavefront takes
  // several
  const int64_t wgs = (items + kSpanWaves - 1) / kSpanWaves;
  const int64_t others = reduce_wgs + (route != nullptr ? 1 : 0);
  const int64_t cap = kSpanWgTarget - others > kSpanWgTarget / 2 ? kSpanWgTarget - others : kSpanWgTarget / 2;
  const int64_t grid = wgs < cap ? wgs : cap;
  wk.decode_wgs = static_cast<int>(grid);
  GrRoute rt{};
  rt.wg = -1;
  if (route != nullptr) {
    rt = *route;
    rt.wg = 0;
  }
  const int64_t all = grid + reduce_wgs + (route != nullptr ? 1 : 0);
  TRIS_REQUIRE(all < (1LL << 31), "%s: too many workgroups", who);
  const dim3 g3(static_cast<unsigned>(all));
  if (S == 16) {
    hipLaunchKernelGGL((gr_decode_span_kernel<16>), g3, dim3(kSpanThreads), 0, s, jobs, wk, expert_ids, red, rt);
  } else {
    hipLaunchKernelGGL((gr_decode_span_kernel<32>), g3, dim3(kSpanThreads), 0, s, jobs, wk, expert_ids, red, rt);
  }
  return check_launch(who);
}

}  // namespace tris

using namespace tris;

extern "C" int tris_grouped_block_gr_predecode(int32_t* decoded, const int32_t* expert_ids, int32_t num_active,
                                               const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                                               const int32_t* q_gmap_gr_meta, int32_t num_experts,
                                               int32_t words_stride, int32_t packed_rows, int32_t outfeatures,
                                               void* stream) {
  const char* who = "tris_grouped_block_gr_predecode";
  TRIS_REQUIRE(num_active >= 0, "%s: negative size", who);
  GrJobs jobs{};
  int rc = make_gr_job(&jobs.job[0], decoded, q_gmap_gr_words, q_gmap_gr_offsets, q_gmap_gr_meta, num_experts,
                       words_stride, packed_rows, outfeatures, false, who);
  if (rc) return rc;
  return launch_gr_jobs(jobs, 1, expert_ids, num_active, stream, who);
}

extern "C" int tris_grouped_block_gr_predecode_multi(const tris_gr_predecode_job* jobs, int32_t num_jobs,
                                                     const int32_t* expert_ids, int32_t num_active, void* stream) {
  const char* who = "tris_grouped_block_gr_predecode_multi";
  TRIS_REQUIRE(num_active >= 0, "%s: negative size", who);
  TRIS_REQUIRE(num_jobs >= 0 && num_jobs <= TRIS_MAX_PREDECODE_JOBS, "%s: %d jobs (at most %d)", who, num_jobs,
               TRIS_MAX_PREDECODE_JOBS);
  TRIS_REQUIRE(num_jobs == 0 || jobs != nullptr, "%s: null jobs", who);
  GrJobs g{};
  for (int q = 0; q < num_jobs; ++q) {
    const tris_gr_predecode_job& j = jobs[q];
    int rc = make_gr_job(&g.job[q], j.decoded, j.q_gmap_gr_words, j.q_gmap_gr_offsets, j.q_gmap_gr_meta,
                         j.num_experts, j.words_stride, j.packed_rows, j.outfeatures, false, who);
    if (rc) return rc;
  }
  return launch_gr_jobs(g, num_jobs, expert_ids, num_active, stream, who);
}

extern "C" int tris_grouped_block_gr_predecode_multi_reduce(const tris_gr_predecode_job* jobs, int32_t num_jobs,
                                                            const int32_t* expert_ids, int32_t num_active,
                                                            const tris_backbone_pair_job* bb, void* stream) {
  const char* who = "tris_grouped_block_gr_predecode_multi_reduce";
  TRIS_REQUIRE(num_active >= 0, "%s: negative size", who);
  TRIS_REQUIRE(num_jobs >= 0 && num_jobs <= TRIS_MAX_PREDECODE_JOBS, "%s: %d jobs (at most %d)", who, num_jobs,
               TRIS_MAX_PREDECODE_JOBS);
  TRIS_REQUIRE(num_jobs == 0 || jobs != nullptr, "%s: null jobs", who);
  GrJobs g{};
  for (int q = 0; q < num_jobs; ++q) {
    const tris_gr_predecode_job& j = jobs[q];
    int rc = make_gr_job(&g.job[q], j.decoded, j.q_gmap_gr_words, j.q_gmap_gr_offsets, j.q_gmap_gr_meta,
                         j.num_experts, j.words_stride, j.packed_rows, j.outfeatures, false, who);
    if (rc) return rc;
  }
  if (bb == nullptr || bb->tokens == 0 || bb->rank == 0) {
    return launch_gr_jobs(g, num_jobs, expert_ids, num_active, stream, who);
  }
  BackboneArgs ba;
  BackbonePlan pl;
  int rc = backbone_prepare_job(bb, &ba, &pl, who);
  if (rc) return rc;
  if (pl.slices == 1) return launch_gr_jobs(g, num_jobs, expert_ids, num_active, stream, who);  // nothing deferred
  return launch_gr_jobs(g, num_jobs, expert_ids, num_active, stream, who, &ba, bb->sv_b != nullptr ? 2 : 1);
}

extern "C" int tris_gr_decode_dense(const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                                    const int32_t* q_gmap_gr_meta, int32_t num_experts, int32_t words_stride,
                                    const int32_t* expert_ids, int32_t num, int32_t packed_rows,
                                    int32_t outfeatures, int32_t* dense, void* stream) {
  const char* who = "tris_gr_decode_dense";
  TRIS_REQUIRE(num >= 0, "%s: negative size", who);
  GrJobs jobs{};
  int rc = make_gr_job(&jobs.job[0], dense, q_gmap_gr_words, q_gmap_gr_offsets, q_gmap_gr_meta, num_experts,
                       words_stride, packed_rows, outfeatures, true, who);
  if (rc) return rc;
  return launch_gr_jobs(jobs, 1, expert_ids, num, stream, who);
}

static int route_predecode(const float* router_logits, int32_t num_tokens, int32_t num_experts,
                                                 int32_t top_k, int32_t renormalize, int32_t m_tile,
                                                 uint16_t* routing_weights_f16, float* routing_weights_f32,
                                                 int64_t* selected_experts, int64_t* perm,
                                                 int64_t* grouped_token_indices, int64_t* grouped_slots,
                                                 int32_t* grouped_expert_ids, int32_t* expert_ids,
                                                 int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts,
                                                 int32_t* inverse_perm, const tris_gr_predecode_job* jobs,
                                                 int32_t num_jobs, int32_t num_slots, const tris_backbone_pair_job* bb,
                                                 void* stream, bool decode_all, const char* who) {
  GrRoute route{};
  int rc = route_prepare(router_logits, num_tokens, num_experts, top_k, renormalize, m_tile, routing_weights_f16,
                         routing_weights_f32, selected_experts, perm, grouped_token_indices, grouped_slots,
                         grouped_expert_ids, expert_ids, segment_offsets, problem_offsets, counts, inverse_perm,
                         &route.ra, who);
  if (rc) return rc;
  TRIS_REQUIRE(num_tokens > 0 && static_cast<int64_t>(num_tokens) * top_k <= kRouteWaveMaxRows &&
                   num_experts <= kRouteLaneMaxExperts,
               "%s: the one-wavefront route takes at most %d routed rows and %d experts", who, kRouteWaveMaxRows,
               kRouteLaneMaxExperts);
  const int rows = num_tokens * top_k;
  if (decode_all) {
    TRIS_REQUIRE(num_slots == num_experts, "%s: num_slots must be num_experts = %d", who, num_experts);
  } else {
    TRIS_REQUIRE(num_slots == (num_experts < rows ? num_experts : rows),
                 "%s: num_slots must be min(num_experts, tokens * top_k) = %d", who,
                 num_experts < rows ? num_experts : rows);
  }
  route.decode_all = decode_all ? 1 : 0;
  route.k_variant = top_k <= 2 ? 2 : (top_k <= 8 ? 8 : kRouteMaxTopK);
  TRIS_REQUIRE(num_jobs >= 0 && num_jobs <= TRIS_MAX_PREDECODE_JOBS && (num_jobs == 0 || jobs != nullptr),
               "%s: %d jobs (0 to %d)", who, num_jobs, TRIS_MAX_PREDECODE_JOBS);
  GrJobs g{};
  for (int q = 0; q < num_jobs; ++q) {
    const tris_gr_predecode_job& j = jobs[q];
    rc = make_gr_job(&g.job[q], j.decoded, j.q_gmap_gr_words, j.q_gmap_gr_offsets, j.q_gmap_gr_meta, j.num_experts,
                     j.words_stride, j.packed_rows, j.outfeatures, false, who);
    if (rc) return rc;
    TRIS_REQUIRE(g.job[q].nblk > 0, "%s: job %d has no blocks", who, q);
  }
  if (bb == nullptr || bb->tokens == 0 || bb->rank == 0) {
    return launch_gr_jobs(g, num_jobs, nullptr, num_slots, stream, who, nullptr, 0, &route);
  }
  BackboneArgs ba;
  BackbonePlan pl;
  rc = backbone_prepare_job(bb, &ba, &pl, who);
  if (rc) return rc;
  if (pl.slices == 1) return launch_gr_jobs(g, num_jobs, nullptr, num_slots, stream, who, nullptr, 0, &route);
  return launch_gr_jobs(g, num_jobs, nullptr, num_slots, stream, who, &ba, bb->sv_b != nullptr ? 2 : 1, &route);
}

extern "C" int tris_route_predecode_multi_reduce(const float* router_logits, int32_t num_tokens, int32_t num_experts,
                                                 int32_t top_k, int32_t renormalize, int32_t m_tile,
                                                 uint16_t* routing_weights_f16, float* routing_weights_f32,
                                                 int64_t* selected_experts, int64_t* perm,
                                                 int64_t* grouped_token_indices, int64_t* grouped_slots,
                                                 int32_t* grouped_expert_ids, int32_t* expert_ids,
                                                 int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts,
                                                 int32_t* inverse_perm, const tris_gr_predecode_job* jobs,
                                                 int32_t num_jobs, int32_t num_slots, const tris_backbone_pair_job* bb,
                                                 void* stream) {
  return route_predecode(router_logits, num_tokens, num_experts, top_k, renormalize, m_tile, routing_weights_f16,
                         routing_weights_f32, selected_experts, perm, grouped_token_indices, grouped_slots,
                         grouped_expert_ids, expert_ids, segment_offsets, problem_offsets, counts, inverse_perm, jobs,
                         num_jobs, num_slots, bb, stream, false, "tris_route_predecode_multi_reduce");
}

extern "C" int tris_route_predecode_all_reduce(const float* router_logits, int32_t num_tokens, int32_t num_experts,
                                               int32_t top_k, int32_t renormalize, int32_t m_tile,
                                               uint16_t* routing_weights_f16, float* routing_weights_f32,
                                               int64_t* selected_experts, int64_t* perm,
                                               int64_t* grouped_token_indices, int64_t* grouped_slots,
                                               int32_t* grouped_expert_ids, int32_t* expert_ids,
                                               int32_t* segment_offsets, int32_t* problem_offsets, int32_t* counts,
                                               int32_t* inverse_perm, const tris_gr_predecode_job* jobs,
                                               int32_t num_jobs, const tris_backbone_pair_job* bb, void* stream) {
  return route_predecode(router_logits, num_tokens, num_experts, top_k, renormalize, m_tile, routing_weights_f16,
                         routing_weights_f32, selected_experts, perm, grouped_token_indices, grouped_slots,
                         grouped_expert_ids, expert_ids, segment_offsets, problem_offsets, counts, inverse_perm, jobs,
                         num_jobs, num_experts, bb, stream, true, "tris_route_predecode_all_reduce");
}
