// Matrix-mode null-space compensation of the grouped expert GEMM: comp[r] = C1_e . (C2_e . x[r]) for the
// rows r of each segment (expert e), both matrices 4-bit packed per expert and concatenated
// (build_grouped_ns_compensation_payload, qlinear_cuda.py:1734-1872; applied by
// run_grouped_structured_expert_forward, :2322-2335, as out.add_(compensation)).
//
// Replaces grouped_ns_compensation_forward (TriSMoE_cuda_kernel.cu:1208-2145 GroupedPacked4LinearOffset*
// kernels).  Two launches, each over one or two payloads that share the input rows and the routing (the
// gate and up projections):
//   ns_c2_kernel: fp32 partial sums part[slice][r][j] = sum over the slice's input columns of
//     x[r][c] * W2_e[j][c]; one workgroup per (16-row tile of one segment, 32 rank indices, K slice,
//     payload), eight K partitions per workgroup.  The slice count fills the GPU at decode, where a few
//     rows per expert leave the work far too small to hide load latency otherwise;
//   ns_c1_kernel: hidden[r][j] = fp16(sum of the slices in slice order) into LDS, then
//     comp[r][n] = fp16(sum_j hidden[r][j] * W1_e[n][j]); one workgroup per (16-row tile, 256 output
//     columns, payload); optionally out[r][n] = fp16(out + comp).
// Weights are the exact dequantised fp16 values fp16((q - z) * s) of PackedQuantMatrix4bit.dequantize
// (qlinear_cuda.py:2761-2786), the scale and zero point of element c taken from group c / group_size
// (dot8_packed4_uniform_shared_stride, TriSMoE_cuda_kernel.cu:1119-1160); products and sums in fp32 (the
// reference's kernels round the weights through an fp16 FMA and accumulate pairs in fp16; the oracle is
// the fp32 product of the exact weights, the reference's own fallback F.linear(F.linear(x, c2), c1),
// qlinear_cuda.py:1943-1946).  The partial sums are added in a fixed order, so results do not depend on
// scheduling.
//
// Rows of segments routed to no expert or to an expert with rank 0 get comp = 0.  The work is small next
// to the grouped GEMM (rank_e is a few dozen), so these are VALU kernels shaped for load latency: every
// global load of a pass is issued before the first use.
#include "tris_common.h"

namespace tris {

constexpr int kNsRows = 16;                              // rows per tile (one segment)
constexpr int kNsC2Ranks = 32;                           // rank indices per C2 workgroup
constexpr int kNsC2Parts = 8;                            // K partitions per C2 workgroup (a word stride each)
constexpr int kNsC2Chunk = 256;                          // input columns staged per pass
constexpr int kNsC2Words = kNsC2Chunk / 8 / kNsC2Parts;  // packed words per partition per pass
constexpr int kNsC2Threads = kNsC2Ranks * kNsC2Parts;
constexpr int kNsC2Units = kNsRows * kNsC2Chunk / 8 / kNsC2Threads;  // 16-byte x loads per thread per pass
constexpr int kNsC1Cols = 256;                           // output columns per C1 workgroup
constexpr int kNsC1Batch = 4;                            // C1 rank words loaded together
constexpr int kNsC1Slices = 16;                          // C2 partial sums per hidden element loaded together
constexpr int kNsMaxRank = 512;                          // hidden columns staged for C1 (fp32 in LDS)
constexpr int kNsTargetWgs = 512;                        // C2 workgroups aimed for
constexpr int kNsMaxSlices = 16;                         // = kNsC1Slices: C1 loads every partial sum at once
static_assert(kNsC2Units * kNsC2Threads * 8 == kNsRows * kNsC2Chunk, "x staging covers the tile");
static_assert(kNsMaxSlices <= kNsC1Slices, "C1 loads every slice's partial sum in one batch");

struct NsArgs {
  const uint16_t* x;          // [batch, in] (or [*, in] rows picked by row_index), rows 16-byte aligned
  const int64_t* row_index;   // input row of grouped row r, or NULL: x is already grouped
  int x_rows;                 // rows of x (row_index values outside [0, x_rows) read row 0)
  const int32_t* expert_ids;
  const int32_t* segment_offsets;
  int num_segments;
  int batch;
  int slices;      // C2 K slices per payload
  int slice_cols;  // input columns per slice (a multiple of kNsC2Chunk)
  int c1_blocks;   // C1 column blocks per payload
  int accumulate;
  tris_ns_payload ns[2];
  float* part[2];  // [slices][batch][max_ns_rank] fp32 partial sums of C2 . x, per payload
  const uint16_t* hidden16;  // C1 only: fp16 hidden [batch, max_ns_rank] given instead of the partial sums
  uint16_t* out[2];
};

// A workgroup's row tile: its segment's expert, first row and row count, and that expert's rank and two
// offsets into the packed payload (rank 0 when the segment has no expert).
struct NsTile {
  int e, row0, rc, rank;
  int64_t off_a, off_b;
};

// Row tile t (tiles of <= 16 rows, segment by segment) -> NsTile; false when t is past the last tile.  Wave 0
// loads the offsets and experts of 64 segments and the rank and offsets of experts 0..63 in one round trip
// (clamped addresses: every load is valid, so none waits behind a branch), finds t by a prefix sum of the
// segments' tile counts, and leaves the result in LDS.
__device__ bool ns_map_tile(const int32_t* __restrict__ seg, const int32_t* __restrict__ expert_ids, int nseg,
                            int tile, const int32_t* __restrict__ ranks, const int32_t* __restrict__ off_a,
                            const int32_t* __restrict__ off_b, int num_experts, int max_rank, NsTile* t_out) {
  __shared__ int res[7];
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int xr = 0, xa = 0, xb = 0;
    if (num_experts > 0) {  // uniform
      const int le = lane < num_experts ? lane : num_experts - 1;
      xr = ranks[le];
      xa = off_a[le];
      xb = off_b[le];
    }
    int base = 0, found = -1, r0 = 0, cnt = 0, ex = -1;
    for (int s0 = 0; s0 < nseg; s0 += 64) {
      const int s = s0 + lane;
      const int sc = s < nseg ? s : nseg - 1;
      int lo = seg[sc], hi = seg[sc + 1];
      int el = expert_ids[sc];
      asm volatile("" : "+v"(el));  // keeps the load beside the offsets' (not sunk into the hit branch)
      if (s >= nseg) hi = lo;
      const int t = hi > lo ? (hi - lo + kNsRows - 1) / kNsRows : 0;
      int incl = t;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
      }
      const int first = base + incl - t;
      const unsigned long long hit = __ballot(tile >= first && tile < base + incl);
      if (hit != 0ull) {  // uniform: exactly one segment holds the tile
        const int src = __ffsll(static_cast<long long>(hit)) - 1;
        found = __shfl(s, src);
        ex = __shfl(el, src);
        const int lo_s = __shfl(lo, src), hi_s = __shfl(hi, src), first_s = __shfl(first, src);
        r0 = lo_s + (tile - first_s) * kNsRows;
        cnt = (hi_s - r0) < kNsRows ? (hi_s - r0) : kNsRows;
        break;
      }
      base += __shfl(incl, 63);
    }
    int vr = 0, va = 0, vb = 0;
    if (ex >= 0 && ex < num_experts) {  // uniform
      if (ex < 64) {
        vr = __shfl(xr, ex);
        va = __shfl(xa, ex);
        vb = __shfl(xb, ex);
      } else {
        vr = ranks[ex];
        va = off_a[ex];
        vb = off_b[ex];
      }
    }
    if (lane == 0) {
      res[0] = found;
      res[1] = r0;
      res[2] = cnt;
      res[3] = ex;
      res[4] = vr < max_rank ? vr : max_rank;  // a malformed rank never reaches past the tiles
      res[5] = va;
      res[6] = vb;
    }
  }
  __syncthreads();
  // workgroup-uniform: scalar registers, so branches on them are scalar branches
  t_out->e = __builtin_amdgcn_readfirstlane(res[3]);
  t_out->row0 = __builtin_amdgcn_readfirstlane(res[1]);
  t_out->rc = __builtin_amdgcn_readfirstlane(res[2]);
  t_out->rank = __builtin_amdgcn_readfirstlane(res[4]);
  t_out->off_a = __builtin_amdgcn_readfirstlane(res[5]);
  t_out->off_b = __builtin_amdgcn_readfirstlane(res[6]);
  return __builtin_amdgcn_readfirstlane(res[0]) >= 0;
}

// The exact weight fp16((q - z) * s) as a float: one rounding of an exact product.
__device__ __forceinline__ float ns_weight(int q, int z, float s) {
  return h2f(f2h_bits(static_cast<float>(q - z) * s));
}

// Zero point of packed row `row` from its qzeros word ((z - 1) & 0xF per 4 bits).
__device__ __forceinline__ int ns_zero(uint32_t zw, int row) {
  return static_cast<int>((zw >> (4 * (row & 7))) & 0xFu) + 1;
}

// The 8 weights of one packed word whose elements all lie in one group.
__device__ __forceinline__ void ns_weights8(uint32_t word, int z, float s, float w[8]) {
#pragma unroll
  for (int m = 0; m < 8; ++m) w[m] = ns_weight(static_cast<int>((word >> (4 * m)) & 0xFu), z, s);
}

// One C2 pass's operands in registers: this thread's packed words with their zero words and scale bits,
// and its 16-byte units of the x tile.
struct NsC2Pass {
  uint32_t wd[kNsC2Words], zw[kNsC2Words];
  uint16_t sb[kNsC2Words];
  uint4 xv[kNsC2Units];
};

// Loads the pass at input column c0 (cc columns): every address valid (clamped), all in flight together.
__device__ __forceinline__ void ns_c2_load(NsC2Pass& p, const int32_t* __restrict__ qw, const int32_t* __restrict__ qz,
                                           const uint16_t* __restrict__ qs, int total_rank, int total_rank_words,
                                           int gs, int groups, int kp, int c0, int cc,
                                           const uint16_t* __restrict__ x, const int64_t* xrow, int in_f) {
#pragma unroll
  for (int i = 0; i < kNsC2Words; ++i) {
    const int w = kp + i * kNsC2Parts;  // word of the chunk
    const int c = c0 + (w * 8 < cc ? w * 8 : 0);
    int g = c / gs;
    g = g < groups ? g : groups - 1;
    p.wd[i] = static_cast<uint32_t>(qw[static_cast<int64_t>(c >> 3) * total_rank]);
    p.zw[i] = static_cast<uint32_t>(qz[static_cast<int64_t>(g) * total_rank_words]);
    p.sb[i] = qs[static_cast<int64_t>(g) * total_rank];
  }
#pragma unroll
  for (int i = 0; i < kNsC2Units; ++i) {
    const int cu = (static_cast<int>(threadIdx.x) + i * kNsC2Threads) % (kNsC2Chunk / 8);
    const int cl = cu * 8 < cc ? cu * 8 : 0;
    p.xv[i] = *reinterpret_cast<const uint4*>(x + xrow[i] * in_f + c0 + cl);
  }
}

__global__ __launch_bounds__(kNsC2Threads) void ns_c2_kernel(NsArgs a) {
  __shared__ float xs[kNsRows][kNsC2Chunk];
  __shared__ float part[kNsC2Parts - 1][kNsRows][kNsC2Ranks];
  const int which = static_cast<int>(blockIdx.z) / a.slices;
  const int slice = static_cast<int>(blockIdx.z) % a.slices;
  const tris_ns_payload& ns = which ? a.ns[1] : a.ns[0];
  NsTile tl;
  if (!ns_map_tile(a.segment_offsets, a.expert_ids, a.num_segments, blockIdx.x, ns.ns_rank_per_expert,
                   ns.ns_c2_rank_offsets, ns.ns_c2_rank_word_offsets, ns.num_experts, ns.max_ns_rank, &tl))
    return;
  const int rank = tl.rank, row0 = tl.row0, rc = tl.rc;
  if (rank <= 0 || static_cast<int>(blockIdx.y) * kNsC2Ranks >= rank) return;  // uniform
  const int jl = threadIdx.x % kNsC2Ranks;
  const int kp = threadIdx.x / kNsC2Ranks;
  const int j = blockIdx.y * kNsC2Ranks + jl;
  const bool jv = j < rank;
  const int jc = jv ? j : rank - 1;  // lanes past the rank load a valid row and use nothing
  const int in_f = ns.infeatures;
  const int gs = ns.group_size;
  const int groups = (in_f + gs - 1) / gs;
  const bool word_groups = gs % 8 == 0;  // every packed word inside one group
  const int32_t* __restrict__ qw = ns.ns_c2_qweight + tl.off_a + jc;         // word w at qw[w * total_rank]
  const int32_t* __restrict__ qz = ns.ns_c2_qzeros + tl.off_b + (jc >> 3);   // group g at qz[g * total_rank_words]
  const uint16_t* __restrict__ qs = ns.ns_c2_scales + tl.off_a + jc;         // group g at qs[g * total_rank]
  // the input row of each x unit this thread stages (the same in every chunk)
  int64_t xrow[kNsC2Units];
#pragma unroll
  for (int i = 0; i < kNsC2Units; ++i) {
    const int r = (static_cast<int>(threadIdx.x) + i * kNsC2Threads) / (kNsC2Chunk / 8);
    const int rl = row0 + (r < rc ? r : 0);
    int64_t xr = rl;
    if (a.row_index != nullptr) {  // uniform
      xr = a.row_index[rl];
      xr = (xr >= 0 && xr < a.x_rows) ? xr : 0;
    }
    xrow[i] = xr;
  }
  float acc[kNsRows];
#pragma unroll
  for (int r = 0; r < kNsRows; ++r) acc[r] = 0.0f;
  const int cbeg = slice * a.slice_cols;
  const int cend = (cbeg + a.slice_cols) < in_f ? (cbeg + a.slice_cols) : in_f;
  // the operands of the first pass; each pass then loads the next one's before computing its own
  NsC2Pass cur;
  if (cbeg < cend)
    ns_c2_load(cur, qw, qz, qs, ns.total_rank, ns.total_rank_words, gs, groups, kp, cbeg,
               (cend - cbeg) < kNsC2Chunk ? (cend - cbeg) : kNsC2Chunk, a.x, xrow, in_f);
  for (int c0 = cbeg; c0 < cend; c0 += kNsC2Chunk) {
    const int cc = (cend - c0) < kNsC2Chunk ? (cend - c0) : kNsC2Chunk;  // a multiple of 8
#pragma unroll
    for (int i = 0; i < kNsC2Units; ++i) {
      const int u = threadIdx.x + i * kNsC2Threads;
      const int r = u / (kNsC2Chunk / 8), cu = u % (kNsC2Chunk / 8);
      if (r < rc) {
        const bool v = cu * 8 < cc;
        const uint4 xv = cur.xv[i];
        const uint32_t h[4] = {v ? xv.x : 0u, v ? xv.y : 0u, v ? xv.z : 0u, v ? xv.w : 0u};
        float4* d = reinterpret_cast<float4*>(&xs[r][cu * 8]);
        d[0] = make_float4(h2f(h[0] & 0xFFFFu), h2f(h[0] >> 16), h2f(h[1] & 0xFFFFu), h2f(h[1] >> 16));
        d[1] = make_float4(h2f(h[2] & 0xFFFFu), h2f(h[2] >> 16), h2f(h[3] & 0xFFFFu), h2f(h[3] >> 16));
      }
    }
    const bool more = c0 + kNsC2Chunk < cend;  // uniform
    NsC2Pass nxt;
    if (more) {
      const int c1 = c0 + kNsC2Chunk;
      ns_c2_load(nxt, qw, qz, qs, ns.total_rank, ns.total_rank_words, gs, groups, kp, c1,
                 (cend - c1) < kNsC2Chunk ? (cend - c1) : kNsC2Chunk, a.x, xrow, in_f);
    }
    const uint32_t* wd = cur.wd;
    const uint32_t* zw = cur.zw;
    const uint16_t* sb = cur.sb;
    __syncthreads();
    if (jv) {
#pragma unroll
      for (int i = 0; i < kNsC2Words; ++i) {
        const int p = kp + i * kNsC2Parts;
        if (p * 8 < cc) {
          float w[8];
          if (word_groups) {
            ns_weights8(wd[i], ns_zero(zw[i], j), h2f(sb[i]), w);
          } else {  // group boundaries inside a word: the scale and zero point per element
            const int c = c0 + p * 8;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
              int g = (c + m) / gs;
              g = g < groups ? g : groups - 1;
              const int z = ns_zero(static_cast<uint32_t>(qz[static_cast<int64_t>(g) * ns.total_rank_words]), j);
              w[m] = ns_weight(static_cast<int>((wd[i] >> (4 * m)) & 0xFu), z,
                               h2f(qs[static_cast<int64_t>(g) * ns.total_rank]));
            }
          }
          // rows in groups of 4 under one scalar branch each (rows past rc hold stale LDS values: their
          // sums are never stored)
#pragma unroll
          for (int rg = 0; rg < kNsRows; rg += 4) {
            if (rg < rc) {
#pragma unroll
              for (int r = rg; r < rg + 4; ++r) {
                const float4 x0 = *reinterpret_cast<const float4*>(&xs[r][p * 8]);
                const float4 x1 = *reinterpret_cast<const float4*>(&xs[r][p * 8 + 4]);
                float v = acc[r];
                v += x0.x * w[0];
                v += x0.y * w[1];
                v += x0.z * w[2];
                v += x0.w * w[3];
                v += x1.x * w[4];
                v += x1.y * w[5];
                v += x1.z * w[6];
                v += x1.w * w[7];
                acc[r] = v;
              }
            }
          }
        }
      }
    }
    __syncthreads();
    if (more) cur = nxt;
  }
  if (kp > 0) {
#pragma unroll
    for (int r = 0; r < kNsRows; ++r) part[kp - 1][r][jl] = acc[r];
  }
  __syncthreads();
  if (kp != 0 || !jv) return;
  float* dst = (which ? a.part[1] : a.part[0]) + static_cast<int64_t>(slice) * a.batch * ns.max_ns_rank;
#pragma unroll
  for (int r = 0; r < kNsRows; ++r) {
    if (r < rc) {
      float v = acc[r];
#pragma unroll
      for (int q = 0; q < kNsC2Parts - 1; ++q) v += part[q][r][jl];
      dst[static_cast<int64_t>(row0 + r) * ns.max_ns_rank + j] = v;
    }
  }
}

// C1 packed words w0 .. w0 + kNsC1Batch - 1 of one output column: weights, zero words and scale bits,
// loaded at clamped (valid) addresses so that none waits behind a branch.
struct NsC1Batch {
  uint32_t wd[kNsC1Batch], zw[kNsC1Batch];
  uint16_t sb[kNsC1Batch];
};

__device__ __forceinline__ void ns_c1_load(NsC1Batch& b, const int32_t* __restrict__ qw, const int32_t* __restrict__ qz,
                                           const uint16_t* __restrict__ qs, int w0, int words, int egs, int eg,
                                           int out_f, int qzc) {
#pragma unroll
  for (int i = 0; i < kNsC1Batch; ++i) {
    const int w = (w0 + i) < words ? (w0 + i) : words - 1;
    int g = w * 8 / egs;
    g = g < eg ? g : eg - 1;
    b.wd[i] = static_cast<uint32_t>(qw[static_cast<int64_t>(w) * out_f]);
    b.zw[i] = static_cast<uint32_t>(qz[static_cast<int64_t>(g) * qzc]);
    b.sb[i] = qs[static_cast<int64_t>(g) * out_f];
  }
}

__global__ __launch_bounds__(kNsC1Cols) void ns_c1_kernel(NsArgs a) {
  __shared__ float hs[kNsRows][kNsMaxRank];
  const int which = static_cast<int>(blockIdx.y) / a.c1_blocks;
  const int nblk = static_cast<int>(blockIdx.y) % a.c1_blocks;
  const tris_ns_payload& ns = which ? a.ns[1] : a.ns[0];
  uint16_t* __restrict__ out = which ? a.out[1] : a.out[0];
  const int out_f = ns.outfeatures;
  if (nblk * kNsC1Cols >= out_f) return;  // uniform: past this payload's columns
  NsTile tl;
  if (!ns_map_tile(a.segment_offsets, a.expert_ids, a.num_segments, blockIdx.x, ns.ns_rank_per_expert,
                   ns.ns_c1_rank_word_offsets, ns.ns_c1_group_offsets, ns.num_experts, ns.max_ns_rank, &tl))
    return;
  const int rank = tl.rank, row0 = tl.row0, rc = tl.rc;
  const int n = nblk * kNsC1Cols + threadIdx.x;
  const bool nv = n < out_f;
  if (rank <= 0) {  // uniform: comp = 0
    if (nv && !a.accumulate) {
      for (int r = 0; r < rc; ++r) out[static_cast<int64_t>(row0 + r) * out_f + n] = 0;
    }
    return;
  }
  const int egs = rank < ns.group_size ? rank : ns.group_size;  // a rank below the group size is one group
  const int eg = (rank + egs - 1) / egs;
  const bool word_groups = eg == 1 || egs % 8 == 0;  // every packed word inside one group
  const int words = (rank + 7) / 8;
  const int qzc = (out_f + 7) / 8;
  const int nc = nv ? n : 0;  // columns past the end load column 0 and store nothing
  const int32_t* __restrict__ qw = ns.ns_c1_qweight + tl.off_a * out_f + nc;     // word w at qw[w * out_f]
  const int32_t* __restrict__ qz = ns.ns_c1_qzeros + tl.off_b * qzc + (nc >> 3); // group g at qz[g * qzc]
  const uint16_t* __restrict__ qs = ns.ns_c1_scales + tl.off_b * out_f + nc;    // group g at qs[g * out_f]
  // hidden = fp16(C2 . x): the slices' partial sums added in slice order.  In flight together: the first
  // kNsC1Slices partial sums of this thread's first hidden element, the first words of the weights and
  // the tile's rows of out (in that order, the order of their use).
  const float* __restrict__ part = which ? a.part[1] : a.part[0];
  const int64_t sstride = static_cast<int64_t>(a.batch) * ns.max_ns_rank;
  const int nst = rc * rank;
  const bool has0 = static_cast<int>(threadIdx.x) < nst;
  const int hr0 = has0 ? static_cast<int>(threadIdx.x) / rank : 0, hj0 = has0 ? static_cast<int>(threadIdx.x) % rank : 0;
  const int64_t hoff0 = static_cast<int64_t>(row0 + hr0) * ns.max_ns_rank + hj0;
  const bool given = a.hidden16 != nullptr;  // uniform
  float t0[kNsC1Slices];
  uint32_t hraw0 = 0;
  if (given) {
    hraw0 = a.hidden16[hoff0];
  } else {
#pragma unroll
    for (int k = 0; k < kNsC1Slices; ++k) t0[k] = part[hoff0 + (k < a.slices ? k : a.slices - 1) * sstride];
  }
  NsC1Batch cur;
  ns_c1_load(cur, qw, qz, qs, 0, words, egs, eg, out_f, qzc);
  uint32_t prev[kNsRows];  // one register per row: no packing, hence no wait, until the final add
  if (a.accumulate) {  // uniform
#pragma unroll
    for (int r = 0; r < kNsRows; ++r) prev[r] = out[static_cast<int64_t>(row0 + (r < rc ? r : 0)) * out_f + nc];
  }
  if (has0) {  // a.slices <= kNsC1Slices: every partial sum is in t0
    if (given) {
      hs[hr0][hj0] = h2f(static_cast<uint16_t>(hraw0));
    } else {
      float v = 0.0f;
#pragma unroll
      for (int k = 0; k < kNsC1Slices; ++k) {
        if (k < a.slices) v += t0[k];
      }
      hs[hr0][hj0] = h2f(f2h_bits(v));  // the hidden tensor's fp16 value (F.linear(x, c2))
    }
  }
  for (int idx = threadIdx.x + kNsC1Cols; idx < nst; idx += kNsC1Cols) {  // tiles of more rows or ranks
    const int r = idx / rank, j = idx % rank;
    if (given) {
      hs[r][j] = h2f(a.hidden16[static_cast<int64_t>(row0 + r) * ns.max_ns_rank + j]);
      continue;
    }
    const float* src = part + static_cast<int64_t>(row0 + r) * ns.max_ns_rank + j;
    float t[kNsC1Slices];
#pragma unroll
    for (int k = 0; k < kNsC1Slices; ++k) t[k] = src[(k < a.slices ? k : a.slices - 1) * sstride];
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < kNsC1Slices; ++k) {
      if (k < a.slices) v += t[k];
    }
    hs[r][j] = h2f(f2h_bits(v));
  }
  if (static_cast<int>(threadIdx.x) < rc * 8) {  // the last word's padding columns: zero, not stale LDS
    const int r = threadIdx.x / 8, j = rank + threadIdx.x % 8;
    if (j < words * 8) hs[r][j] = 0.0f;
  }
  __syncthreads();
  float acc[kNsRows];
#pragma unroll
  for (int r = 0; r < kNsRows; ++r) acc[r] = 0.0f;
  for (int w0 = 0; w0 < words; w0 += kNsC1Batch) {
    NsC1Batch nxt;
    const bool more = w0 + kNsC1Batch < words;
    if (more) ns_c1_load(nxt, qw, qz, qs, w0 + kNsC1Batch, words, egs, eg, out_f, qzc);
#pragma unroll
    for (int i = 0; i < kNsC1Batch; ++i) {
      const int w = w0 + i;
      if (w < words) {  // uniform
        const int j0 = w * 8;
        float wt[8];
        if (word_groups) {
          ns_weights8(cur.wd[i], ns_zero(cur.zw[i], nc), h2f(cur.sb[i]), wt);
        } else {  // group boundaries inside a word: the scale and zero point per element
#pragma unroll
          for (int m = 0; m < 8; ++m) {
            int g = (j0 + m) / egs;
            g = g < eg ? g : eg - 1;
            const int z = ns_zero(static_cast<uint32_t>(qz[static_cast<int64_t>(g) * qzc]), nc);
            wt[m] = ns_weight(static_cast<int>((cur.wd[i] >> (4 * m)) & 0xFu), z,
                              h2f(qs[static_cast<int64_t>(g) * out_f]));
          }
        }
        const int valid = rank - j0;  // the padding of the last word contributes nothing
#pragma unroll
        for (int m = 0; m < 8; ++m) wt[m] = m < valid ? wt[m] : 0.0f;
        // rows in groups of 4 under one scalar branch each (rows past rc: never stored)
#pragma unroll
        for (int rg = 0; rg < kNsRows; rg += 4) {
          if (rg < rc) {
#pragma unroll
            for (int r = rg; r < rg + 4; ++r) {
              const float4 h0 = *reinterpret_cast<const float4*>(&hs[r][j0]);
              const float4 h1 = *reinterpret_cast<const float4*>(&hs[r][j0 + 4]);
              float v = acc[r];
              v += h0.x * wt[0];
              v += h0.y * wt[1];
              v += h0.z * wt[2];
              v += h0.w * wt[3];
              v += h1.x * wt[4];
              v += h1.y * wt[5];
              v += h1.z * wt[6];
              v += h1.w * wt[7];
              acc[r] = v;
            }
          }
        }
      }
    }
    if (more) cur = nxt;
  }
  if (!nv) return;
#pragma unroll
  for (int r = 0; r < kNsRows; ++r) {
    if (r < rc) {
      const uint16_t comp = f2h_bits(acc[r]);  // the compensation tensor's fp16 value
      out[static_cast<int64_t>(row0 + r) * out_f + n] =
          a.accumulate ? f2h_bits(h2f(static_cast<uint16_t>(prev[r])) + h2f(comp)) : comp;  // out.add_(compensation)
    }
  }
}

static int check_ns(const tris_ns_payload* ns, const char* who) {
  TRIS_REQUIRE(ns != nullptr, "%s: null payload", who);
  TRIS_REQUIRE(ns->num_experts >= 0 && ns->infeatures >= 0 && ns->outfeatures >= 0 && ns->max_ns_rank >= 0 &&
                   ns->total_rank >= 0 && ns->total_rank_words >= 0,
               "%s: negative shape", who);
  TRIS_REQUIRE(ns->max_ns_rank <= kNsMaxRank, "%s: max_ns_rank %d exceeds %d", who, ns->max_ns_rank, kNsMaxRank);
  TRIS_REQUIRE(ns->infeatures % 8 == 0, "%s: infeatures %d must be a multiple of 8", who, ns->infeatures);
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

// Row tiles: at most batch / 16 + one partial tile per segment; tiles past the last exit at once.
static int ns_tiles(int batch, int num_segments) {
  return batch / kNsRows + (num_segments < batch ? num_segments : batch);
}

// Input columns per C2 slice (a multiple of the staged chunk): enough slices that the row tiles times the
// slices reach the target workgroup count.  It depends on the rows, segments and input width only, so a
// payload's sums (and bits) are the same in a single and in a pair launch.
static int ns_slice_cols(int batch, int num_segments, int infeatures) {
  const int tiles = ns_tiles(batch, num_segments);
  const int64_t wgs = tiles > 0 ? tiles : 1;
  int64_t slices = (kNsTargetWgs + wgs - 1) / wgs;
  slices = slices < kNsMaxSlices ? slices : kNsMaxSlices;
  slices = slices < 1 ? 1 : slices;
  const int in_f = infeatures > 0 ? infeatures : 1;
  return ceil_div(ceil_div(in_f, static_cast<int>(slices)), kNsC2Chunk) * kNsC2Chunk;
}

// Slices covering the input columns (none of them empty).
static int ns_slices(int batch, int num_segments, int infeatures) {
  return ceil_div(infeatures > 0 ? infeatures : 1, ns_slice_cols(batch, num_segments, infeatures));
}

static int64_t ns_part_bytes(int slices, int batch, int max_rank) {
  const int64_t b = static_cast<int64_t>(slices) * batch * max_rank * 4;
  return (b + 255) / 256 * 256;
}

static int64_t ns_workspace(int batch, int num_segments, int infeatures, int rank_a, int rank_b, int count) {
  if (batch <= 0) return 0;
  const int mr = rank_a > rank_b ? rank_a : rank_b;
  if (mr <= 0) return 0;
  const int slices = ns_slices(batch, num_segments, infeatures);
  return ns_part_bytes(slices, batch, rank_a) + (count > 1 ? ns_part_bytes(slices, batch, rank_b) : 0);
}

static int ns_forward(const char* who, const uint16_t* x, int32_t x_rows, const int64_t* row_index, int32_t batch,
                      const int32_t* expert_ids,
                      const int32_t* segment_offsets, int32_t num_segments, const tris_ns_payload* const* ns,
                      int count, void* workspace, int64_t workspace_bytes, uint16_t* const* out, int32_t accumulate,
                      hipStream_t stream) {
  for (int i = 0; i < count; ++i) {
    const int rc = check_ns(ns[i], who);
    if (rc) return rc;
  }
  TRIS_REQUIRE(count == 1 || ns[0]->infeatures == ns[1]->infeatures, "%s: the two payloads' infeatures differ (%d, %d)",
               who, ns[0]->infeatures, ns[count - 1]->infeatures);
  TRIS_REQUIRE(batch >= 0 && num_segments >= 0, "%s: negative batch or segment count", who);
  int max_rank = 0, max_out = 0;
  for (int i = 0; i < count; ++i) {
    max_rank = ns[i]->max_ns_rank > max_rank ? ns[i]->max_ns_rank : max_rank;
    max_out = ns[i]->outfeatures > max_out ? ns[i]->outfeatures : max_out;
  }
  if (batch == 0 || num_segments == 0 || max_out == 0) return TRIS_OK;
  TRIS_REQUIRE(expert_ids != nullptr && segment_offsets != nullptr, "%s: null routing", who);
  for (int i = 0; i < count; ++i) TRIS_REQUIRE(out[i] != nullptr || ns[i]->outfeatures == 0, "%s: null out", who);
  if (max_rank == 0 && accumulate) return TRIS_OK;  // no expert has a compensation term
  NsArgs a{};
  a.x = x;
  a.row_index = row_index;
  a.x_rows = row_index != nullptr ? x_rows : batch;
  a.expert_ids = expert_ids;
  a.segment_offsets = segment_offsets;
  a.num_segments = num_segments;
  a.batch = batch;
  a.accumulate = accumulate != 0;
  const int in_f = ns[0]->infeatures;
  a.slice_cols = ns_slice_cols(batch, num_segments, in_f);
  a.slices = ns_slices(batch, num_segments, in_f);
  a.c1_blocks = ceil_div(max_out, kNsC1Cols);
  for (int i = 0; i < 2; ++i) {
    a.ns[i] = *ns[i < count ? i : 0];
    a.out[i] = out[i < count ? i : 0];
  }
  const int tiles = ns_tiles(batch, num_segments);
  if (max_rank > 0) {
    const int64_t need = ns_workspace(batch, num_segments, in_f, ns[0]->max_ns_rank,
                                      count > 1 ? ns[1]->max_ns_rank : 0, count);
    TRIS_REQUIRE(x != nullptr && (reinterpret_cast<uintptr_t>(x) & 15u) == 0,
                 "%s: x_grouped must be non-null and 16-byte aligned", who);
    TRIS_REQUIRE(row_index == nullptr || x_rows > 0, "%s: row_index given with x_rows %d", who, x_rows);
    TRIS_REQUIRE(workspace != nullptr && workspace_bytes >= need, "%s: workspace of %lld bytes needed (%lld given)",
                 who, static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    a.part[0] = static_cast<float*>(workspace);
    a.part[1] = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                         ns_part_bytes(a.slices, batch, ns[0]->max_ns_rank));
    hipLaunchKernelGGL(ns_c2_kernel, dim3(tiles, ceil_div(max_rank, kNsC2Ranks), a.slices * count),
                       dim3(kNsC2Threads), 0, stream, a);
    const int rc = check_launch(who);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(ns_c1_kernel, dim3(tiles, a.c1_blocks * count), dim3(kNsC1Cols), 0, stream, a);
  return check_launch(who);
}

// out[b][n] = sum_k in[b][k] * W[n][k] in fp32 with no rounding (in fp16 or fp32, W fp16 [N, K]): the
// non-expert linear's null-space term, whose C2 product stays in fp32 and whose C1 product joins the fp32
// accumulator (kernel.cu:2252-2316).  One wavefront per output, lanes striding K (coalesced), a fixed
// butterfly reduction (deterministic).
__global__ __launch_bounds__(256) void dense_linear_f32_kernel(const uint16_t* __restrict__ in16,
                                                               const float* __restrict__ in32, int batch, int K,
                                                               const uint16_t* __restrict__ w, int N,
                                                               float* __restrict__ out) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64;
  if (o >= static_cast<int64_t>(batch) * N) return;  // uniform over the wavefront
  const int lane = threadIdx.x % 64;
  const int b = static_cast<int>(o / N), n = static_cast<int>(o % N);
  const uint16_t* wr = w + static_cast<int64_t>(n) * K;
  float v = 0.0f;
  if (in32 != nullptr) {
    const float* xr = in32 + static_cast<int64_t>(b) * K;
    for (int k = lane; k < K; k += 64) v += xr[k] * h2f(wr[k]);
  } else {
    const uint16_t* xr = in16 + static_cast<int64_t>(b) * K;
    for (int k = lane; k < K; k += 64) v += h2f(xr[k]) * h2f(wr[k]);
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d);
  if (lane == 0) out[o] = v;
}

// The C1 half of a payload (what tris_grouped_ns_c1_forward reads).
static int check_ns_c1(const tris_ns_payload* ns, const char* who) {
  TRIS_REQUIRE(ns != nullptr, "%s: null payload", who);
  TRIS_REQUIRE(ns->num_experts >= 0 && ns->outfeatures >= 0 && ns->max_ns_rank >= 0, "%s: negative shape", who);
  TRIS_REQUIRE(ns->max_ns_rank <= kNsMaxRank, "%s: max_ns_rank %d exceeds %d", who, ns->max_ns_rank, kNsMaxRank);
  if (ns->max_ns_rank > 0) {
    TRIS_REQUIRE(ns->group_size > 0, "%s: group_size must be positive", who);
    TRIS_REQUIRE(ns->ns_rank_per_expert && ns->ns_c1_rank_word_offsets && ns->ns_c1_group_offsets &&
                     ns->ns_c1_qweight && ns->ns_c1_qzeros && ns->ns_c1_scales,
                 "%s: null C1 tensor", who);
  }
  return TRIS_OK;
}

}  // namespace tris

using namespace tris;

extern "C" int tris_dense_linear_f32(const uint16_t* input_f16, const float* input_f32, int32_t batch,
                                     int32_t in_features, const uint16_t* weight, int32_t out_features, float* output,
                                     void* stream) {
  const char* who = "tris_dense_linear_f32";
  TRIS_REQUIRE(batch >= 0 && in_features >= 0 && out_features >= 0, "%s: negative shape", who);
  if (batch == 0 || out_features == 0) return TRIS_OK;
  TRIS_REQUIRE((input_f16 == nullptr) != (input_f32 == nullptr), "%s: give exactly one of the fp16 / fp32 inputs",
               who);
  TRIS_REQUIRE(output != nullptr && (in_features == 0 || weight != nullptr), "%s: null pointer", who);
  const int64_t outs = static_cast<int64_t>(batch) * out_features;
  const int64_t blocks = (outs + 3) / 4;
  TRIS_REQUIRE(blocks <= 2147483647LL, "%s: too many outputs", who);
  hipLaunchKernelGGL(dense_linear_f32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), input_f16, input_f32, batch, in_features, weight, out_features,
                     output);
  return check_launch(who);
}

extern "C" int tris_grouped_ns_c1_forward(const uint16_t* hidden, int32_t batch, const int32_t* expert_ids,
                                          const int32_t* segment_offsets, int32_t num_segments,
                                          const tris_ns_payload* ns, uint16_t* out, int32_t accumulate,
                                          void* stream) {
  const char* who = "tris_grouped_ns_c1_forward";
  int rc = check_ns_c1(ns, who);
  if (rc) return rc;
  TRIS_REQUIRE(batch >= 0 && num_segments >= 0, "%s: negative batch or segment count", who);
  if (batch == 0 || num_segments == 0 || ns->outfeatures == 0) return TRIS_OK;
  TRIS_REQUIRE(expert_ids != nullptr && segment_offsets != nullptr && out != nullptr, "%s: null pointer", who);
  if (ns->max_ns_rank == 0 && accumulate) return TRIS_OK;
  TRIS_REQUIRE(ns->max_ns_rank == 0 || hidden != nullptr, "%s: null hidden", who);
  NsArgs a{};
  a.expert_ids = expert_ids;
  a.segment_offsets = segment_offsets;
  a.num_segments = num_segments;
  a.batch = batch;
  a.accumulate = accumulate != 0;
  a.slices = 1;
  a.c1_blocks = ceil_div(ns->outfeatures, kNsC1Cols);
  a.ns[0] = a.ns[1] = *ns;
  a.hidden16 = hidden;
  a.out[0] = a.out[1] = out;
  hipLaunchKernelGGL(ns_c1_kernel, dim3(ns_tiles(batch, num_segments), a.c1_blocks), dim3(kNsC1Cols), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch(who);
}

extern "C" int64_t tris_grouped_ns_workspace_bytes(int32_t batch, int32_t num_segments, int32_t infeatures,
                                                   int32_t max_ns_rank) {
  return ns_workspace(batch, num_segments, infeatures, max_ns_rank, 0, 1);
}

extern "C" int64_t tris_grouped_ns_pair_workspace_bytes(int32_t batch, int32_t num_segments, int32_t infeatures,
                                                        int32_t max_ns_rank_a, int32_t max_ns_rank_b) {
  return ns_workspace(batch, num_segments, infeatures, max_ns_rank_a, max_ns_rank_b, 2);
}

extern "C" int tris_grouped_ns_compensation_forward(const uint16_t* x_grouped, int32_t batch,
                                                    const int32_t* expert_ids, const int32_t* segment_offsets,
                                                    int32_t num_segments, const tris_ns_payload* ns,
                                                    void* workspace, int64_t workspace_bytes, uint16_t* out,
                                                    int32_t accumulate, void* stream) {
  const tris_ns_payload* p[1] = {ns};
  uint16_t* o[1] = {out};
  return ns_forward("tris_grouped_ns_compensation_forward", x_grouped, batch, nullptr, batch, expert_ids,
                    segment_offsets,
                    num_segments, p, 1, workspace, workspace_bytes, o, accumulate, static_cast<hipStream_t>(stream));
}

extern "C" int tris_grouped_ns_compensation_pair_forward(const uint16_t* x, int32_t x_rows, const int64_t* row_index,
                                                         int32_t batch,
                                                         const int32_t* expert_ids, const int32_t* segment_offsets,
                                                         int32_t num_segments, const tris_ns_payload* ns_a,
                                                         const tris_ns_payload* ns_b, void* workspace,
                                                         int64_t workspace_bytes, uint16_t* out_a, uint16_t* out_b,
                                                         int32_t accumulate, void* stream) {
  const tris_ns_payload* p[2] = {ns_a, ns_b};
  uint16_t* o[2] = {out_a, out_b};
  return ns_forward("tris_grouped_ns_compensation_pair_forward", x, x_rows, row_index, batch, expert_ids,
                    segment_offsets,
                    num_segments, p, 2, workspace, workspace_bytes, o, accumulate, static_cast<hipStream_t>(stream));
}
