// Shared fp16 backbone projection hidden = x * SV^T on MFMA.
//
// Replaces the fp16 branch of QuantLinear.compute_shared_hidden
// (qlinear_cuda.py:4454-4502), an F.linear on cuBLAS, and fuses the
// index_select gather of grouped rows (modeling_mixtral.py:467, :475-476)
// through an optional row index.
//
// Shape: out[T, rank] = x[T, in] . SV[rank, in]^T with fp16 inputs and fp32
// accumulation.  One workgroup = 4 wavefronts computes up to 4 16-token x
// 16-row output tiles over one K slice, so each SV operand load feeds every
// token tile (SV is read once per row tile and slice); wavefront w takes a
// contiguous quarter of the slice and issues its 16-byte operand loads in
// batches of 4 or 8 32-wide K steps (the last batch predicated) before the
// v_mfma_f32_16x16x32_f16, and the four partial tiles are added in LDS in
// wavefront order.  The slice count is chosen so that a decode
// launch has a few hundred workgroups (latency, not MFMA, bounds this
// projection at decode).  With one slice the workgroup writes fp16; otherwise
// it writes fp32 partial tiles to the caller's workspace and
// backbone_reduce_kernel adds the slices in slice order and rounds once, so
// results are deterministic and no workgroups communicate inside a kernel (an
// in-kernel last-arriver reduction needs device-scope release fences, which
// write back the L2 on this GPU: measured far slower than the extra launch).
// blockIdx.z selects one of up to two projections of the same rows (a gate/up
// pair in one launch).
//
// At decode (T <= 16) the projection is HBM-bound on SV (2*rank*in bytes).
#include <mutex>

#include "tris_backbone.h"

namespace tris {

template <int TT, int B>
__global__ __launch_bounds__(kBbThreads) void backbone_kernel(BackboneArgs a) {
  __shared__ f32x4 red[kBbWaves - 1][TT][kWave];
  backbone_block<TT, B>(a, true, blockIdx.x, blockIdx.y, blockIdx.z, threadIdx.x, red);
}

__global__ __launch_bounds__(256) void backbone_reduce_kernel(BackboneArgs a) {
  backbone_reduce_at(a, static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x, blockIdx.y);
}

__global__ __launch_bounds__(256) void fill_zero_u16_kernel(uint16_t* __restrict__ out, int64_t count) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx < count) out[idx] = 0;
}

// Slices per projection: enough workgroups to cover the chip at decode, at
// most one slice per kBbWaves*kBbKStep columns and kBbMaxSlices in all.  The
// count does not depend on how many projections share the launch, so a pair
// gives the same bits as two single calls.
// Token tiles per workgroup: all of them up to 4 (one SV read per row tile and slice).
static int backbone_token_group(int tokens) {
  const int tiles = ceil_div(tokens > 0 ? tokens : 1, 16);
  return tiles < 4 ? tiles : 4;
}

// target: the workgroups a launch aims at (kBbTargetWgs; the 4-bit backbone kBbPacked4TargetWgs).
int backbone_slices(int tokens, int in_features, int rank, int target = kBbTargetWgs) {
  if (tokens <= 0 || in_features <= 0 || rank <= 0) return 1;
  const int64_t tiles =
      static_cast<int64_t>(ceil_div(ceil_div(tokens, 16), backbone_token_group(tokens))) * ceil_div(rank, 16);
  int64_t slices = (target + tiles - 1) / tiles;
  const int64_t max_by_k = ceil_div(in_features, kBbWaves * kBbKStep);
  if (slices > max_by_k) slices = max_by_k;
  if (slices > kBbMaxSlices) slices = kBbMaxSlices;
  return slices < 1 ? 1 : static_cast<int>(slices);
}

static int backbone_gemm_slice_k(int tokens, int in_features, int rank, int* slices);

// use_gemm: the entry may take the tiled GEMM for prefill-size batches (backbone_gemm_fits).
int64_t backbone_workspace_bytes(int tokens, int in_features, int rank, int nproj, bool use_gemm, int target) {
  int slices = backbone_slices(tokens, in_features, rank, target);
  if (use_gemm && backbone_gemm_fits(tokens, in_features, rank)) backbone_gemm_slice_k(tokens, in_features, rank, &slices);
  return slices > 1 ? static_cast<int64_t>(nproj) * slices * tokens * rank * 4 : 0;
}

BackbonePlan backbone_plan(int tokens, int in_features, int rank) {
  BackbonePlan p{};
  p.slices = backbone_slices(tokens, in_features, rank);
  p.tt = backbone_token_group(tokens);
  p.token_groups = ceil_div(ceil_div(tokens, 16), p.tt);
  p.row_tiles = ceil_div(rank, 16);
  p.slice_k = ceil_div(ceil_div(in_features, p.slices), kBbWaves * kBbKStep) * kBbWaves * kBbKStep;
  return p;
}

int backbone_prepare(const uint16_t* x, int tokens, int in_features, const int64_t* row_index, const uint16_t* sv_a,
                     const uint16_t* sv_b, int rank, const uint16_t* in_scale_a, const uint16_t* in_scale_b,
                     uint16_t* out_a, uint16_t* out_b, void* workspace, int64_t workspace_bytes, BackboneArgs* args,
                     BackbonePlan* plan, const char* who, bool use_gemm) {
  TRIS_REQUIRE(tokens > 0 && in_features > 0 && rank > 0, "%s: empty projection", who);
  TRIS_REQUIRE(out_a != nullptr && (sv_b == nullptr || out_b != nullptr), "%s: null output", who);
  TRIS_REQUIRE(x && sv_a, "%s: null input", who);
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(sv_a) % 16 == 0 &&
                   (sv_b == nullptr || reinterpret_cast<uintptr_t>(sv_b) % 16 == 0) &&
                   reinterpret_cast<uintptr_t>(in_scale_a) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(in_scale_b) % 16 == 0,
               "%s: x, sv and in_scale must be 16-byte aligned", who);
  const int nproj = sv_b != nullptr ? 2 : 1;
  const BackbonePlan pl = backbone_plan(tokens, in_features, rank);
  const int64_t need = backbone_workspace_bytes(tokens, in_features, rank, nproj, use_gemm);
  TRIS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
               "%s: workspace of %lld bytes needed, %lld given", who, static_cast<long long>(need),
               static_cast<long long>(workspace_bytes));
  TRIS_REQUIRE((use_gemm && backbone_gemm_fits(tokens, in_features, rank)) ||
                   static_cast<int64_t>(pl.token_groups) * pl.slices <= 65535,
               "%s: too many tokens", who);
  BackboneArgs a{};
  a.x = x;
  a.row_index = row_index;
  a.proj[0] = BackboneProj{sv_a, out_a, in_scale_a, nullptr, 0};
  a.proj[1] = BackboneProj{sv_b, out_b, in_scale_b, nullptr, 0};
  a.partials = static_cast<float*>(workspace);
  a.tokens = tokens;
  a.in_features = in_features;
  a.rank = rank;
  a.slices = pl.slices;
  a.slice_k = pl.slice_k;
  *args = a;
  *plan = pl;
  return TRIS_OK;
}

int backbone_prepare_job(const tris_backbone_pair_job* bb, BackboneArgs* args, BackbonePlan* plan, const char* who) {
  const int rc = backbone_prepare(bb->x, bb->tokens, bb->in_features, nullptr, bb->sv_a, bb->sv_b, bb->rank,
                                  bb->in_scale_a, bb->in_scale_b, bb->out_a, bb->out_b, bb->workspace,
                                  bb->workspace_bytes, args, plan, who);
  if (rc) return rc;
  TRIS_REQUIRE(bb->split >= 0 && bb->split < bb->rank, "%s: column split %d outside [0, %d)", who, bb->split,
               bb->rank);
  if (bb->split > 0) {
    TRIS_REQUIRE(bb->out_a_hi != nullptr && (bb->sv_b == nullptr || bb->out_b_hi != nullptr),
                 "%s: a column split needs out_a_hi (and out_b_hi for two projections)", who);
    args->proj[0].out_hi = bb->out_a_hi;
    args->proj[0].split = bb->split;
    args->proj[1].out_hi = bb->out_b_hi;
    args->proj[1].split = bb->sv_b != nullptr ? bb->split : 0;
  }
  return TRIS_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Prefill-size backbone: a tiled split-K MFMA GEMM, hidden[m][n] = sum_k a[m][k] SV[n][k] over one K slice, with
// a[m][k] = fp16(x[row(m)][k] * in_scale[k]) (row(m) = row_index[m] when given).  A workgroup computes a
// 256 x 128 tile (rows x rank columns) of one projection and slice;
// its four wavefronts each own a 128 x 64 quadrant (8 x 4 tiles of v_mfma_f32_16x16x32_f16), so every 16-byte
// LDS read feeds 4 or 8 MFMAs: per 32-column stage a CU (two workgroups) reads 96 KB and writes 48 KB of LDS
// for 2 x 512 MFMA cycles per SIMD.  Stages are double-buffered in LDS (48 KB a workgroup) with one barrier a
// stage; the global loads of the next two stages are in flight in registers meanwhile.  Tiles are ordered
// (projection, slice, row tile, column tile) and handed out XCD-major: the four column tiles of a row tile run
// on one XCD, whose L2 then serves the row tile's activations to all four.  Slices write fp32 partial tiles
// that backbone_reduce_kernel adds in slice order (one slice writes fp16 directly), so the result does not
// depend on the launch shape beyond the slice count, which depends on the problem shape only.

struct BgArgs {
  BackboneArgs b;       // x (g for the SwiGLU form), row_index, proj[], partials, tokens, in_features, rank, slices
  const uint16_t* x2;   // u for the SwiGLU form
  int ks;               // K columns per slice, a multiple of kBgK
  int m_tiles, n_tiles;
  int direct;           // one slice and no scatter: the tile is written as fp16 to proj[].out
};

bool backbone_gemm_fits(int tokens, int in_features, int rank) {
  return tokens >= kBgMinRows && rank % kBgN == 0 && rank > 0 && in_features % kBgK == 0 && in_features > 0;
}

// The slice count depends on the shape only (not on the projection count), so a pair launch gives each
// projection the bits of its single launch.
static int backbone_gemm_slices(int tokens, int in_features, int rank) {
  const int64_t tiles = static_cast<int64_t>(ceil_div(tokens, kBgM)) * (rank / kBgN);
  int64_t s = (kBgTargetWgs + tiles - 1) / tiles;
  const int64_t max_by_k = in_features / (kBgK * kBgMinStages);
  s = s < max_by_k ? s : max_by_k;
  s = s < kBgMaxSlices ? s : kBgMaxSlices;
  return s < 1 ? 1 : static_cast<int>(s);
}

static int backbone_gemm_slice_k(int tokens, int in_features, int rank, int* slices) {
  const int s0 = backbone_gemm_slices(tokens, in_features, rank);
  const int ks = ceil_div(in_features / kBgK, s0) * kBgK;
  *slices = ceil_div(in_features, ks);
  return ks;
}

constexpr int kXcdCount = 8;  // MI355X: workgroup w runs on XCD w % 8

struct BgStage {
  uint4 a[4];  // the x runs
  uint4 b[2];  // the SV runs
  uint4 sc;    // in_scale of the thread's 8 columns
};

__global__ __launch_bounds__(kBgThreads, 2) void backbone_gemm_kernel(BgArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t la0[kBgM * kBgStride];
  __shared__ __attribute__((aligned(16))) uint16_t la1[kBgM * kBgStride];
  __shared__ __attribute__((aligned(16))) uint16_t lb0[kBgN * kBgStride];
  __shared__ __attribute__((aligned(16))) uint16_t lb1[kBgN * kBgStride];
  const BackboneArgs& a = g.b;
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int wm = wave >> 1, wn = wave & 1;
  const int i16 = lane & 15, kg = lane >> 4;
  // XCD-major virtual tile index, column tile fastest
  int v;
  {
    const int w = static_cast<int>(blockIdx.x);
    const int W = static_cast<int>(gridDim.x);
    const int x = w % kXcdCount, q = W / kXcdCount, r = W % kXcdCount;
    v = x * q + (x < r ? x : r) + w / kXcdCount;
  }
  const int nt = v % g.n_tiles;
  v /= g.n_tiles;
  const int mt = v % g.m_tiles;
  v /= g.m_tiles;
  const int sl = v % a.slices;
  const int q = v / a.slices;
  const BackboneProj pj = q == 0 ? a.proj[0] : a.proj[1];  // selected, not indexed: no private copy of the args
  const int m0 = mt * kBgM;
  const int n0 = nt * kBgN;
  const int K = a.in_features;
  const int kbeg = sl * g.ks;
  const int kn = (K - kbeg) < g.ks ? (K - kbeg) : g.ks;  // > 0, a multiple of kBgK
  const int nstage = kn / kBgK;
  // copy slots: run i of the thread is row (tid / 4) + 64 i of the tile, columns 8 (tid % 4) .. + 8 of the stage;
  // rows past the batch read the batch's last row (their outputs are not written)
  const int crow = tid >> 2, cchunk = tid & 3, ccol = cchunk * 8;
  const uint16_t* xsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int m = m0 + crow + 64 * i;
    m = m < a.tokens ? m : a.tokens - 1;
    const int64_t xrow = a.row_index != nullptr ? a.row_index[m] : m;
    xsrc[i] = a.x + xrow * K + kbeg + ccol;
  }
  const uint16_t* ssrc0 = pj.sv + static_cast<int64_t>(n0 + crow) * K + kbeg + ccol;
  const uint16_t* ssrc1 = ssrc0 + static_cast<int64_t>(64) * K;
  const uint16_t* scale = pj.in_scale != nullptr ? pj.in_scale + kbeg + ccol : nullptr;

  auto issue = [&](int st, BgStage& R) {
    const int ko = st * kBgK;
#pragma unroll
    for (int i = 0; i < 4; ++i) R.a[i] = *reinterpret_cast<const uint4*>(xsrc[i] + ko);
    R.b[0] = *reinterpret_cast<const uint4*>(ssrc0 + ko);
    R.b[1] = *reinterpret_cast<const uint4*>(ssrc1 + ko);
    R.sc = scale != nullptr ? *reinterpret_cast<const uint4*>(scale + ko)
                            : make_uint4(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u);
  };
  // the stage's operands into LDS: a = fp16(x * in_scale) (fp16 products; a scale of 1.0 is exact)
  auto write = [&](const BgStage& R, uint16_t* la, uint16_t* lb) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t sw[4] = {R.sc.x, R.sc.y, R.sc.z, R.sc.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t xw[4] = {R.a[i].x, R.a[i].y, R.a[i].z, R.a[i].w};
      uint32_t pw[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        pw[h] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, xw[h]) * __builtin_bit_cast(h2, sw[h]));
      }
      *reinterpret_cast<uint4*>(&la[bg_chunk(crow + 64 * i, cchunk)]) = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    }
    *reinterpret_cast<uint4*>(&lb[bg_chunk(crow, cchunk)]) = R.b[0];
    *reinterpret_cast<uint4*>(&lb[bg_chunk(crow + 64, cchunk)]) = R.b[1];
  };
  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  auto compute = [&](const uint16_t* la, const uint16_t* lb) {
    f16x8 bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bv[j] = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&lb[bg_chunk(64 * wn + 16 * j + i16, kg)]));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f16x8 av =
          __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&la[bg_chunk(128 * wm + 16 * i + i16, kg)]));
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv[j], acc[i][j], 0, 0, 0);
    }
  };

  // One stage: the MFMAs of the buffer in LDS, the LDS writes of the next stage (registers loaded a stage
  // ago) into the other buffer and the global loads of the stage after it, interleaved so the matrix cores
  // keep issuing while the copies move.  Stage indices past the slice are clamped (a re-read, never used),
  // and the extra write lands in a buffer nobody reads before the next barrier.
  auto half = [&](const uint16_t* la, const uint16_t* lb, const BgStage& Rw, uint16_t* law, uint16_t* lbw, int sti,
                  BgStage& Ri) {
    issue(sti, Ri);
    compute(la, lb);
    write(Rw, law, lbw);
    __builtin_amdgcn_sched_group_barrier(0x020, 7, 0);  // the global loads first
    __builtin_amdgcn_sched_group_barrier(0x100, 5, 0);  // B fragments and the first A fragment
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // the MFMAs of A fragment i
      if (i < 7) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (i < 6) {
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
    }
  };
  // stage st sits in buffer st % 2; register set st % 2 carries it from its loads (two stages ahead) to LDS
  BgStage R0, R1;
  issue(0, R0);
  issue(nstage > 1 ? 1 : 0, R1);
  write(R0, la0, lb0);
  __syncthreads();
  for (int st = 0; st < nstage; st += 2) {
    half(la0, lb0, R1, la1, lb1, st + 2 < nstage ? st + 2 : nstage - 1, R0);
    __syncthreads();
    if (st + 1 < nstage) {
      half(la1, lb1, R0, la0, lb0, st + 3 < nstage ? st + 3 : nstage - 1, R1);
      __syncthreads();
    }
  }
  // acc[i][j][v] = hidden[m0 + 128 wm + 16 i + 4 kg + v][n0 + 64 wn + 16 j + i16], stored through a buffer
  // resource over the tile's rows (rows past the batch drop their stores through its size: no per-row test)
  const int mrows = a.tokens - m0 < kBgM ? a.tokens - m0 : kBgM;
  const uint32_t lane_off = static_cast<uint32_t>((wm * 128 + kg * 4) * a.rank + n0 + wn * 64 + i16);
  if (g.direct) {
    const __amdgpu_buffer_rsrc_t r =
        make_rsrc(pj.out + static_cast<int64_t>(m0) * a.rank, static_cast<uint32_t>(mrows) * a.rank * 2u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          __builtin_amdgcn_raw_buffer_store_b16(
              f2h_bits(acc[i][j][vv]), r,
              (lane_off + static_cast<uint32_t>((i * 16 + vv) * a.rank + j * 16)) * 2u, 0u, 0);
        }
      }
    }
  } else {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(
        a.partials + ((static_cast<int64_t>(q) * a.slices + sl) * a.tokens + m0) * a.rank,
        static_cast<uint32_t>(mrows) * a.rank * 4u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          __builtin_amdgcn_raw_buffer_store_b32(
              __float_as_uint(acc[i][j][vv]), r,
              (lane_off + static_cast<uint32_t>((i * 16 + vv) * a.rank + j * 16)) * 4u, 0u, 0);
        }
      }
    }
  }
}

// The slice reductions of the tiled GEMMs (rank a multiple of 128): four neighbouring outputs a thread, each the
// slices' partial sums added in slice order and rounded once (the bits of backbone_reduce_kernel), 16-byte loads.
// With inv (the route's inverse_perm) element (t, n) of projection q is stored to row inv[t * top_k + j] of
// proj[q].out for every slot j (the rows the route sends token t to; -1 and rows past out_rows are skipped).
__global__ __launch_bounds__(256) void backbone_reduce4_kernel(BackboneArgs a, const int32_t* __restrict__ inv,
                                                               int top_k, int out_rows) {
  const int q = static_cast<int>(blockIdx.y);
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const int64_t count = static_cast<int64_t>(a.tokens) * a.rank;
  if (i4 >= count) return;
  const float* src = a.partials + static_cast<int64_t>(q) * a.slices * count + i4;
  float4 v[kBgMaxSlices];
#pragma unroll
  for (int sl = 0; sl < kBgMaxSlices; ++sl) {
    v[sl] = sl < a.slices ? *reinterpret_cast<const float4*>(src + sl * count) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int sl = 0; sl < kBgMaxSlices; ++sl) {
    if (sl < a.slices) {
      sum.x += v[sl].x;
      sum.y += v[sl].y;
      sum.z += v[sl].z;
      sum.w += v[sl].w;
    }
  }
  const uint2 h = make_uint2(static_cast<uint32_t>(f2h_bits(sum.x)) | (static_cast<uint32_t>(f2h_bits(sum.y)) << 16),
                             static_cast<uint32_t>(f2h_bits(sum.z)) | (static_cast<uint32_t>(f2h_bits(sum.w)) << 16));
  uint16_t* out = q == 0 ? a.proj[0].out : a.proj[1].out;
  if (inv == nullptr) {
    *reinterpret_cast<uint2*>(out + i4) = h;
    return;
  }
  const int t = static_cast<int>(i4 / a.rank);
  const int n = static_cast<int>(i4 - static_cast<int64_t>(t) * a.rank);
  for (int j = 0; j < top_k; ++j) {
    const int row = inv[static_cast<int64_t>(t) * top_k + j];
    if (row >= 0 && row < out_rows) *reinterpret_cast<uint2*>(out + static_cast<int64_t>(row) * a.rank + n) = h;
  }
}

static int launch_backbone_reduce4(const BackboneArgs& args, int nproj, hipStream_t s, const char* who,
                                   const int32_t* inv = nullptr, int top_k = 0, int out_rows = 0) {
  const int64_t quads = static_cast<int64_t>(args.tokens) * args.rank / 4;
  hipLaunchKernelGGL(backbone_reduce4_kernel, dim3(static_cast<unsigned>((quads + 255) / 256), nproj), dim3(256), 0,
                     s, args, inv, top_k, out_rows);
  return check_launch(who);
}

// The SwiGLU form of the tiled GEMM with each product formed once: a workgroup of eight wavefronts covers a
// 128 x 512 tile (rows x rank columns; wavefront (wm, wn) of 2 x 4 owns a 64 x 128 quadrant, 4 x 8 tiles of
// v_mfma_f32_16x16x32_f16), so act_fn(g) * u of a row is formed by one workgroup per K slice, not by every
// 128-column tile of the rank (SiLU's exponential and reciprocal run at a quarter of the VALU rate).  Per
// 32-column stage a thread forms 8 products and copies four 16-byte SV runs; stages are double-buffered in LDS
// (80 KB, one workgroup per CU) and their global loads issued two stages ahead.  Rank columns past the rank are computed on clamped SV
// rows and not written.  Tiles are ordered (slice, row tile, column tile) and handed out XCD-major, so the
// workgroups of one K slice share its SV rows through one L2.
constexpr int kBwM = 128;
constexpr int kBwN = 512;
constexpr int kBwThreads = 512;
constexpr int kBwTargetWgs = 256;

static int backbone_wide_slice_k(int rows, int in_features, int rank, int* slices) {
  const int64_t tiles = static_cast<int64_t>(ceil_div(rows, kBwM)) * ceil_div(rank, kBwN);
  int64_t sl = (kBwTargetWgs + tiles - 1) / tiles;
  const int64_t max_by_k = in_features / (kBgK * kBgMinStages);
  sl = sl < max_by_k ? sl : max_by_k;
  sl = sl < kBgMaxSlices ? sl : kBgMaxSlices;
  sl = sl < 1 ? 1 : sl;
  const int ks = ceil_div(in_features / kBgK, static_cast<int>(sl)) * kBgK;
  *slices = ceil_div(in_features, ks);
  return ks;
}

__global__ __launch_bounds__(kBwThreads, 1) void backbone_swiglu_gemm_kernel(BgArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t la0[kBwM * kBgStride];
  __shared__ __attribute__((aligned(16))) uint16_t la1[kBwM * kBgStride];
  __shared__ __attribute__((aligned(16))) uint16_t lb0[kBwN * kBgStride];
  __shared__ __attribute__((aligned(16))) uint16_t lb1[kBwN * kBgStride];
  const BackboneArgs& a = g.b;
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int wm = wave >> 2, wn = wave & 3;
  const int i16 = lane & 15, kg = lane >> 4;
  int v;
  {
    const int w = static_cast<int>(blockIdx.x);
    const int W = static_cast<int>(gridDim.x);
    const int x = w % kXcdCount, q = W / kXcdCount, r = W % kXcdCount;
    v = x * q + (x < r ? x : r) + w / kXcdCount;
  }
  const int nt = v % g.n_tiles;
  v /= g.n_tiles;
  const int mt = v % g.m_tiles;
  const int sl = v / g.m_tiles;
  const BackboneProj& pj = a.proj[0];
  const int m0 = mt * kBwM;
  const int n0 = nt * kBwN;
  const int K = a.in_features;
  const int kbeg = sl * g.ks;
  const int kn = (K - kbeg) < g.ks ? (K - kbeg) : g.ks;
  const int nstage = kn / kBgK;
  // copy slots: the thread's g/u run is row tid / 4 of the tile, its SV runs rows tid / 4 + 128 i, columns
  // 8 (tid % 4) .. + 8 of the stage (rows past the batch or the rank read the last valid row)
  const int crow = tid >> 2, cchunk = tid & 3, ccol = cchunk * 8;
  int m = m0 + crow;
  m = m < a.tokens ? m : a.tokens - 1;
  const uint16_t* gsrc = a.x + static_cast<int64_t>(m) * K + kbeg + ccol;
  const uint16_t* usrc = g.x2 + static_cast<int64_t>(m) * K + kbeg + ccol;
  const uint16_t* ssrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int n = n0 + crow + 128 * i;
    n = n < a.rank ? n : a.rank - 1;
    ssrc[i] = pj.sv + static_cast<int64_t>(n) * K + kbeg + ccol;
  }
  const uint16_t* scale = pj.in_scale != nullptr ? pj.in_scale + kbeg + ccol : nullptr;
  struct Regs {
    uint4 g, u, b[4], sc;
  };
  auto issue = [&](int st, Regs& R) {
    const int ko = st * kBgK;
    R.g = *reinterpret_cast<const uint4*>(gsrc + ko);
    R.u = *reinterpret_cast<const uint4*>(usrc + ko);
#pragma unroll
    for (int i = 0; i < 4; ++i) R.b[i] = *reinterpret_cast<const uint4*>(ssrc[i] + ko);
    R.sc = scale != nullptr ? *reinterpret_cast<const uint4*>(scale + ko)
                            : make_uint4(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u);
  };
  auto write = [&](const Regs& R, uint16_t* la, uint16_t* lb) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t gw[4] = {R.g.x, R.g.y, R.g.z, R.g.w};
    const uint32_t uw[4] = {R.u.x, R.u.y, R.u.z, R.u.w};
    const uint32_t sw[4] = {R.sc.x, R.sc.y, R.sc.z, R.sc.w};
    uint32_t pw[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const uint32_t lo = swiglu_bits(static_cast<uint16_t>(gw[h]), static_cast<uint16_t>(uw[h]));
      const uint32_t hi = swiglu_bits(static_cast<uint16_t>(gw[h] >> 16), static_cast<uint16_t>(uw[h] >> 16));
      pw[h] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, lo | (hi << 16)) * __builtin_bit_cast(h2, sw[h]));
    }
    *reinterpret_cast<uint4*>(&la[bg_chunk(crow, cchunk)]) = make_uint4(pw[0], pw[1], pw[2], pw[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&lb[bg_chunk(crow + 128 * i, cchunk)]) = R.b[i];
  };
  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  auto compute = [&](const uint16_t* la, const uint16_t* lb) {
    f16x8 bv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bv[j] = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&lb[bg_chunk(128 * wn + 16 * j + i16, kg)]));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x8 av =
          __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&la[bg_chunk(64 * wm + 16 * i + i16, kg)]));
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv[j], acc[i][j], 0, 0, 0);
    }
  };
  // one stage as in backbone_gemm_kernel: MFMAs, the next stage's SwiGLU products and LDS writes, and the global
  // loads of the stage after it, interleaved
  auto half = [&](const uint16_t* la, const uint16_t* lb, const Regs& Rw, uint16_t* law, uint16_t* lbw, int sti,
                  Regs& Ri) {
    issue(sti, Ri);
    compute(la, lb);
    write(Rw, law, lbw);
    __builtin_amdgcn_sched_group_barrier(0x020, 7, 0);  // the global loads first
    __builtin_amdgcn_sched_group_barrier(0x100, 9, 0);  // B fragments and the first A fragment
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // SwiGLU products
      }
      if (i < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (i == 0) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
  };
  // stage st sits in buffer st % 2; register set st % 2 carries it from its loads (two stages ahead) to LDS
  Regs R0, R1;
  issue(0, R0);
  issue(nstage > 1 ? 1 : 0, R1);
  write(R0, la0, lb0);
  __syncthreads();
  for (int st = 0; st < nstage; st += 2) {
    half(la0, lb0, R1, la1, lb1, st + 2 < nstage ? st + 2 : nstage - 1, R0);
    __syncthreads();
    if (st + 1 < nstage) {
      half(la1, lb1, R0, la0, lb0, st + 3 < nstage ? st + 3 : nstage - 1, R1);
      __syncthreads();
    }
  }
  // acc[i][j][vv] = hidden[m0 + 64 wm + 16 i + 4 kg + vv][n0 + 128 wn + 16 j + i16], stored through a buffer
  // resource over the tile's rows (rows past the batch drop their stores through its size); columns past the
  // rank (a rank that is not a multiple of 512) get an offset past it
  const int mrows = a.tokens - m0 < kBwM ? a.tokens - m0 : kBwM;
  const uint32_t row_off = static_cast<uint32_t>((wm * 64 + kg * 4) * a.rank);
  uint32_t col_off[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int n = n0 + wn * 128 + j * 16 + i16;
    col_off[j] = n < a.rank ? static_cast<uint32_t>(n) : 0x10000000u;  // x 4 bytes stays below 2^32
  }
  const __amdgpu_buffer_rsrc_t r =
      g.direct ? make_rsrc(pj.out + static_cast<int64_t>(m0) * a.rank, static_cast<uint32_t>(mrows) * a.rank * 2u)
               : make_rsrc(a.partials + (static_cast<int64_t>(sl) * a.tokens + m0) * a.rank,
                           static_cast<uint32_t>(mrows) * a.rank * 4u);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t e = row_off + static_cast<uint32_t>((i * 16 + vv) * a.rank) + col_off[j];
        if (g.direct) {
          __builtin_amdgcn_raw_buffer_store_b16(f2h_bits(acc[i][j][vv]), r, e * 2u, 0u, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][vv]), r, e * 4u, 0u, 0);
        }
      }
    }
  }
}

// base: g, proj[0] (sv, out, in_scale), partials, rows (tokens), in_features, rank.
static int launch_backbone_swiglu_gemm(const BackboneArgs& base, const uint16_t* up, hipStream_t s, const char* who) {
  BgArgs g{};
  g.b = base;
  g.x2 = up;
  int slices = 1;
  g.ks = backbone_wide_slice_k(base.tokens, base.in_features, base.rank, &slices);
  g.b.slices = slices;
  g.m_tiles = ceil_div(base.tokens, kBwM);
  g.n_tiles = ceil_div(base.rank, kBwN);
  g.direct = slices == 1;
  const int64_t wgs = static_cast<int64_t>(g.m_tiles) * g.n_tiles * slices;
  TRIS_REQUIRE(wgs <= 2147483647, "%s: grid too large", who);
  hipLaunchKernelGGL(backbone_swiglu_gemm_kernel, dim3(static_cast<unsigned>(wgs)), dim3(kBwThreads), 0, s, g);
  int rc = check_launch(who);
  if (rc || g.direct) return rc;
  return launch_backbone_reduce4(g.b, 1, s, who);
}

// base: x, row_index, proj[], partials, tokens, in_features, rank; slices are set here.
// scatter (inverse_perm, top_k, out_rows): the token rows' projections go to their routed rows.
static int launch_backbone_gemm(const BackboneArgs& base, int nproj, hipStream_t s, const char* who,
                                const int32_t* scatter = nullptr, int top_k = 0, int out_rows = 0) {
  BgArgs g{};
  g.b = base;
  int slices = 1;
  g.ks = backbone_gemm_slice_k(base.tokens, base.in_features, base.rank, &slices);
  g.b.slices = slices;
  g.m_tiles = ceil_div(base.tokens, kBgM);
  g.n_tiles = base.rank / kBgN;
  g.direct = slices == 1 && scatter == nullptr;
  const int64_t wgs = static_cast<int64_t>(g.m_tiles) * g.n_tiles * slices * nproj;
  TRIS_REQUIRE(wgs <= 2147483647, "%s: grid too large", who);
  const dim3 grid(static_cast<unsigned>(wgs));
  hipLaunchKernelGGL(backbone_gemm_kernel, grid, dim3(kBgThreads), 0, s, g);
  int rc = check_launch(who);
  if (rc || g.direct) return rc;
  return launch_backbone_reduce4(g.b, nproj, s, who, scatter, top_k, out_rows);
}

int launch_backbone(const uint16_t* x, int tokens, int in_features, const int64_t* row_index, const uint16_t* sv_a,
                    const uint16_t* sv_b, int rank, const uint16_t* in_scale_a, const uint16_t* in_scale_b,
                    uint16_t* out_a, uint16_t* out_b, void* workspace, int64_t workspace_bytes, void* stream,
                    const char* who, bool use_gemm = true, int32_t* deferred_slices = nullptr) {
  TRIS_REQUIRE(tokens >= 0 && in_features >= 0 && rank >= 0, "%s: negative shape", who);
  if (deferred_slices != nullptr) *deferred_slices = 1;
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
  BackboneArgs args;
  BackbonePlan pl;
  int rc = backbone_prepare(x, tokens, in_features, row_index, sv_a, sv_b, rank, in_scale_a, in_scale_b, out_a, out_b,
                            workspace, workspace_bytes, &args, &pl, who, use_gemm);
  if (rc) return rc;
  const bool gemm = use_gemm && backbone_gemm_fits(tokens, in_features, rank);
  TRIS_REQUIRE(deferred_slices == nullptr || !gemm,
               "%s: %d rows take the tiled GEMM, whose reduction cannot be deferred", who, tokens);
  if (gemm) return launch_backbone_gemm(args, nproj, s, who);
  const dim3 grid(pl.row_tiles, pl.token_groups * pl.slices, nproj);
  switch (pl.tt) {
    case 1: hipLaunchKernelGGL((backbone_kernel<1, 8>), grid, dim3(kBbThreads), 0, s, args); break;
    case 2: hipLaunchKernelGGL((backbone_kernel<2, 8>), grid, dim3(kBbThreads), 0, s, args); break;
    case 3: hipLaunchKernelGGL((backbone_kernel<3, 4>), grid, dim3(kBbThreads), 0, s, args); break;
    default: hipLaunchKernelGGL((backbone_kernel<4, 4>), grid, dim3(kBbThreads), 0, s, args); break;
  }
  rc = check_launch(who);
  if (rc || pl.slices == 1) return rc;
  if (deferred_slices != nullptr) {  // the consumer adds the slices
    *deferred_slices = pl.slices;
    return TRIS_OK;
  }
  return launch_backbone_reduce(args, nproj, s, who);
}

int launch_backbone_reduce(const BackboneArgs& args, int nproj, hipStream_t s, const char* who) {
  const int64_t count = static_cast<int64_t>(args.tokens) * args.rank;
  hipLaunchKernelGGL(backbone_reduce_kernel, dim3(static_cast<unsigned>((count + 255) / 256), nproj), dim3(256), 0, s,
                     args);
  return check_launch(who);
}

// ---------------------------------------------------------------------------------------------------------
// Down-projection backbone with the SwiGLU product fused into its operand staging:
// in[r][k] = fp16(fp16(silu(g[r][k])) * u[r][k]) (act_fn(gate) * up, modeling_mixtral.py:496, as swiglu_bits),
// times in_scale[k] as an fp16 product when given, and hidden = in . SV^T.  Workgroup (cg, slice) covers rank
// columns [128 cg, 128 cg + 128) over one K slice for every row (at most kSgMaxRowTiles 16-row tiles): it
// forms the slice's product once in LDS (each of the rank's column groups forms it: rank / 128 times in all,
// not once per 16-column tile), then wavefront w of kSgWaves multiplies it by columns [128 cg + 16 w, + 16)
// (one MFMA column tile).  A slice is at most kSgSteps K steps, whose SV loads are all issued before the
// product is formed.  Slices write fp32 partial tiles that backbone_reduce_kernel adds in slice order.
constexpr int kSgCols = 128;
constexpr int kSgWaves = kSgCols / 16;
constexpr int kSgThreads = kSgWaves * kWave;
constexpr int kSgMaxRowTiles = 8;                 // row tiles a workgroup stages (its row group)
constexpr int kSgMaxRowGroups = 4;                // row groups of one launch (blockIdx.z): at most 512 rows
constexpr int kSgSteps = 8;                       // K steps of 32 per slice at most
constexpr int kSgTargetWgs = 256;
constexpr int kSgVecIters = 4;                    // product vectors (8 columns) a thread forms per batch

struct SwigluBackboneArgs {
  const uint16_t* g;         // [rows, in_features]
  const uint16_t* u;         // [rows, in_features]
  const uint16_t* sv;        // [rank, in_features]
  const uint16_t* in_scale;  // [in_features] or null
  uint16_t* out;             // [rows, rank] (written directly when slices == 1), or [rows, split] with a split
  float* partials;           // [slices][rows][rank]
  int rows, in_features, rank, slices, slice_k;
  uint16_t* out_hi;          // with split > 0: columns [split, rank) as [rows, rank - split]
  int split;
};

template <int TT>
__global__ __launch_bounds__(kSgThreads) void backbone_swiglu_kernel(SwigluBackboneArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t sg_in[];  // [TT * 16][slice_k + 8]
  const int cg = blockIdx.x;
  const int slice = blockIdx.y;
  const int row0 = static_cast<int>(blockIdx.z) * TT * 16;  // the workgroup's row group
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int i16 = lane % 16;
  const int kg = lane / 16;
  const int stride = a.slice_k + 8;
  const int k0 = slice * a.slice_k;
  const int kn = (a.in_features - k0) < a.slice_k ? (a.in_features - k0) : a.slice_k;  // a multiple of 32
  const int steps = kn / 32;
  // SV operands of the whole slice (the wave's column tile), in flight while the product is formed
  const int col = cg * kSgCols + 16 * wave + i16;
  f16x8 bq[kSgSteps];
  {
    const bool cv = col < a.rank;
    const uint16_t* src = a.sv + static_cast<int64_t>(cv ? col : 0) * a.in_features + k0 + 8 * kg;
#pragma unroll
    for (int j = 0; j < kSgSteps; ++j) bq[j] = load8_vec(src, 32 * j, cv && j < steps);
  }
  // the product of the slice for every row (rows past a.rows are zero), kSgVecIters vectors a thread per batch
  const int v8 = kn / 8;
  const int nvec = TT * 16 * v8;
  for (int v0 = 0; v0 < nvec; v0 += kSgVecIters * kSgThreads) {
    uint4 gv[kSgVecIters], uv[kSgVecIters], sc[kSgVecIters];
#pragma unroll
    for (int i = 0; i < kSgVecIters; ++i) {
      const int v = v0 + i * kSgThreads + tid;
      const int r = v / v8;
      const int c = k0 + (v % v8) * 8;
      const bool ok = v < nvec && row0 + r < a.rows;
      const int64_t o = static_cast<int64_t>(ok ? row0 + r : 0) * a.in_features + (ok ? c : 0);
      gv[i] = ok ? *reinterpret_cast<const uint4*>(a.g + o) : make_uint4(0u, 0u, 0u, 0u);
      uv[i] = ok ? *reinterpret_cast<const uint4*>(a.u + o) : make_uint4(0u, 0u, 0u, 0u);
      sc[i] = (a.in_scale != nullptr && ok) ? *reinterpret_cast<const uint4*>(a.in_scale + c)
                                            : make_uint4(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u);
    }
#pragma unroll
    for (int i = 0; i < kSgVecIters; ++i) {
      const int v = v0 + i * kSgThreads + tid;
      if (v >= nvec) continue;
      const int r = v / v8;
      const int c = (v % v8) * 8;
      const uint32_t gw[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
      const uint32_t uw[4] = {uv[i].x, uv[i].y, uv[i].z, uv[i].w};
      const uint32_t sw[4] = {sc[i].x, sc[i].y, sc[i].z, sc[i].w};
      uint32_t pw[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t lo = swiglu_bits(static_cast<uint16_t>(gw[h]), static_cast<uint16_t>(uw[h]));
        const uint32_t hi = swiglu_bits(static_cast<uint16_t>(gw[h] >> 16), static_cast<uint16_t>(uw[h] >> 16));
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        // fp16 products with the input scale (1.0 without one), as the backbone's x * ns_col
        pw[h] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, lo | (hi << 16)) * __builtin_bit_cast(h2, sw[h]));
      }
      *reinterpret_cast<uint4*>(&sg_in[r * stride + c]) = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    }
  }
  __syncthreads();
  f32x4 acc[TT];
#pragma unroll
  for (int rt = 0; rt < TT; ++rt) acc[rt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < kSgSteps; ++j) {
    if (j < steps) {  // uniform
#pragma unroll
      for (int rt = 0; rt < TT; ++rt) {
        const f16x8 av = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&sg_in[(16 * rt + i16) * stride + 32 * j + 8 * kg]));
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bq[j], acc[rt], 0, 0, 0);
      }
    }
  }
  // acc[rt][v] = hidden[row0 + 16 rt + 4 kg + v][128 cg + 16 w + i16]
  if (col < a.rank) {
#pragma unroll
    for (int rt = 0; rt < TT; ++rt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = row0 + 16 * rt + 4 * kg + v;
        if (r >= a.rows) continue;
        if (a.slices == 1) {
          bb_store(BackboneProj{a.sv, a.out, a.in_scale, a.out_hi, a.split}, a.rank, r, col, f2h_bits(acc[rt][v]));
        } else {
          a.partials[(static_cast<int64_t>(slice) * a.rows + r) * a.rank + col] = acc[rt][v];
        }
      }
    }
  }
}

// Slices of backbone_swiglu_kernel: about kSgTargetWgs workgroups, at most kSgSteps K steps and
// kBbReduceMaxSlices slices; returns the slice width in columns (a multiple of 32) and sets *slices.
static int swiglu_backbone_slice_k(int in_features, int rank, int* slices) {
  const int groups = ceil_div(rank, kSgCols);
  int s = ceil_div(kSgTargetWgs, groups);
  s = s < kBbReduceMaxSlices ? s : kBbReduceMaxSlices;
  const int min_slices = ceil_div(in_features, kSgSteps * 32);
  s = s > min_slices ? s : min_slices;
  const int slice_k = ceil_div(ceil_div(in_features, s), 32) * 32;
  *slices = ceil_div(in_features, slice_k);
  return slice_k;
}

// ---------------------------------------------------------------------------------------------------------
// 4-bit packed backbone (PackedQuantMatrix4bit, qlinear_cuda.py:2637-2786): SV[r][c] =
// fp16((q[c][r] - z[g][r]) * s[g][r]) with q the nibble c % 8 of qweight[c / 8][r], z = nibble r % 8 of
// qzeros[g][r / 8] plus one, s = scales[g][r], g = g_idx[c] (the reference's dequantize, :2761-2786).

// Nibbles m of a qweight word (8 columns, natural order) to fp16 weights: (1024 + q) - (1024 + z) is exact,
// and the product with s is rounded once, as the reference's fp16 subtract and multiply.
__device__ __forceinline__ f16x8 p4_weights(uint32_t w, uint32_t z1024x2, uint32_t s2) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t lo = w & 0x0F0F0F0Fu;         // q0, q2, q4, q6 in bytes 0..3
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // q1, q3, q5, q7
  const h2 z = __builtin_bit_cast(h2, z1024x2);
  const h2 sc = __builtin_bit_cast(h2, s2);
  uint32_t out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // halves (q_2i, q_2i+1): byte i of lo, byte i of hi, each under 0x64 (fp16 1024 + q)
    const uint32_t sel = 0x0C000C00u | (static_cast<uint32_t>(4 + i) << 16) | static_cast<uint32_t>(i);
    const uint32_t pair = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
    out[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, pair) - z) * sc);
  }
  return __builtin_bit_cast(f16x8, make_uint4(out[0], out[1], out[2], out[3]));
}

struct Packed4Proj {
  const int32_t* qweight;
  const int32_t* qzeros;
  const uint16_t* scales;
  uint16_t* out;
};

struct Packed4Args {
  BackboneArgs base;  // x, row_index, in_scale, partials, shapes, slices (proj[].out for the reduce)
  Packed4Proj proj[2];
  int packed_cols;    // ceil(in / 8)
  int qzeros_cols;    // ceil(rank / 8)
  int group_size;     // a multiple of 8: the 8 columns of a word share a group
  int num_groups;
};

// The fp16 backbone kernel's tiling and split-K with the B operand built from packed words: lane (i, kg)
// of a K step holds the 8 weights of row r0 + i, columns k .. k + 7 (k = step + 8 kg), one qweight word.
__global__ __launch_bounds__(kBbThreads) void packed4_backbone_kernel(Packed4Args pa) {
  __shared__ f32x4 red[kBbWaves - 1][kWave];
  const BackboneArgs& a = pa.base;
  const int q = blockIdx.z;
  const Packed4Proj& pj = pa.proj[q];
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
  const int rr = r_valid ? r : 0;
  const uint16_t* in_scale = a.proj[q].in_scale;
  const bool scaled = in_scale != nullptr;
  const bool vec = (a.in_features % 8) == 0;
  const uint32_t zshift = 4u * static_cast<uint32_t>(rr & 7);

  auto weights = [&](int k) {  // k: a multiple of 8
    const int p = k >> 3;
    int g = k / pa.group_size;
    g = g < pa.num_groups ? g : pa.num_groups - 1;
    uint32_t w = 0u, zw = 0u;
    uint16_t sh = 0;
    if (r_valid && p < pa.packed_cols) {
      w = static_cast<uint32_t>(pj.qweight[static_cast<int64_t>(p) * a.rank + rr]);
      zw = static_cast<uint32_t>(pj.qzeros[static_cast<int64_t>(g) * pa.qzeros_cols + (rr >> 3)]);
      sh = pj.scales[static_cast<int64_t>(g) * a.rank + rr];
    }
    const uint32_t z = ((zw >> zshift) & 0xFu) + 1u;
    const uint32_t z2 = (0x6400u | z) * 0x00010001u;
    const uint32_t s2 = static_cast<uint32_t>(sh) * 0x00010001u;
    return p4_weights(w, z2, s2);
  };

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
        bv[u] = weights(k);
      }
      if (scaled) {
#pragma unroll
        for (int u = 0; u < kBbBatch; ++u) {
          av[u] = av[u] * load8_vec(in_scale, k0 + u * kBbKStep + kg * 8, true);  // fp16 products, as x * ns_col
        }
      }
#pragma unroll
      for (int u = 0; u < kBbBatch; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u], bv[u], acc, 0, 0, 0);
    }
  }
  for (; k0 < kend; k0 += kBbKStep) {
    const int k = k0 + kg * 8;
    f16x8 av;
    if (vec && k + 8 <= kend) {
      av = load8_vec(xsrc, k, t_valid);
      if (scaled) av = av * load8_vec(in_scale, k, true);
    } else {
      av = load8_tail(xsrc, k, kend, t_valid);  // columns past the end read 0, so their weights do not count
      if (scaled) av = av * load8_tail(in_scale, k, kend, true);
    }
    const f16x8 bv = k < kend ? weights(k) : f16x8{};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kBbWaves - 1; ++w) acc += red[w][lane];
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

// out[r][c] = the dequantised weight, any g_idx: one thread per (row, word), threads along the words of a row
// so that the 16-byte stores of a row are contiguous.
__global__ __launch_bounds__(256) void packed4_dequant_kernel(tris_packed4_matrix w, uint16_t* __restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int words = (w.cols + 7) / 8;
  if (idx >= static_cast<int64_t>(words) * w.rows) return;
  const int r = static_cast<int>(idx / words);
  const int p = static_cast<int>(idx % words);
  const int qzc = (w.rows + 7) / 8;
  const uint32_t word = static_cast<uint32_t>(w.qweight[static_cast<int64_t>(p) * w.rows + r]);
  uint16_t h[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int c = 8 * p + m;
    h[m] = 0;
    if (c < w.cols) {
      int g = w.g_idx[c];
      g = g < 0 ? 0 : (g >= w.num_groups ? w.num_groups - 1 : g);
      const uint32_t zw = static_cast<uint32_t>(w.qzeros[static_cast<int64_t>(g) * qzc + (r >> 3)]);
      const int z = static_cast<int>((zw >> (4 * (r & 7))) & 0xFu) + 1;
      const int qv = static_cast<int>((word >> (4 * m)) & 0xFu);
      // (q - z) is a small integer, so the fp32 product is exact and rounds once to fp16
      h[m] = f2h_bits(static_cast<float>(qv - z) * h2f(w.scales[static_cast<int64_t>(g) * w.rows + r]));
    }
  }
  uint16_t* dst = out + static_cast<int64_t>(r) * w.cols + 8 * p;
  if (w.cols % 8 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16),
                                                h[4] | (uint32_t(h[5]) << 16), h[6] | (uint32_t(h[7]) << 16));
  } else {
    for (int m = 0; m < 8 && 8 * p + m < w.cols; ++m) dst[m] = h[m];
  }
}

static int check_packed4(const tris_packed4_matrix* w, bool fused, const char* who) {
  TRIS_REQUIRE(w != nullptr, "%s: null matrix", who);
  TRIS_REQUIRE(w->rows >= 0 && w->cols >= 0 && w->num_groups >= 0, "%s: negative shape", who);
  if (w->rows == 0 || w->cols == 0) return TRIS_OK;
  TRIS_REQUIRE(w->num_groups > 0, "%s: no groups", who);
  TRIS_REQUIRE(w->qweight && w->qzeros && w->scales && (w->g_idx || fused), "%s: null tensor", who);
  TRIS_REQUIRE(static_cast<int64_t>((w->cols + 7) / 8) * w->rows < (int64_t{1} << 31),
               "%s: matrix too large", who);
  if (fused) {
    TRIS_REQUIRE(w->group_size > 0 && w->group_size % 8 == 0 &&
                     static_cast<int64_t>(w->group_size) * w->num_groups >= w->cols,
                 "%s: the fused kernel needs uniform groups of a multiple of 8 columns (g_idx[c] == c / group_size); "
                 "dequantize with tris_packed4_dequant and use tris_backbone_linear otherwise", who);
  }
  return TRIS_OK;
}

int launch_packed4_backbone(const uint16_t* x, int tokens, const int64_t* row_index, const tris_packed4_matrix* wa,
                            const tris_packed4_matrix* wb, const uint16_t* in_scale_a, const uint16_t* in_scale_b,
                            uint16_t* out_a, uint16_t* out_b, void* workspace, int64_t workspace_bytes, void* stream,
                            const char* who) {
  int rc = check_packed4(wa, true, who);
  if (rc) return rc;
  if (wb) {
    rc = check_packed4(wb, true, who);
    if (rc) return rc;
    TRIS_REQUIRE(wb->rows == wa->rows && wb->cols == wa->cols, "%s: pair shapes differ", who);
  }
  TRIS_REQUIRE(tokens >= 0, "%s: negative tokens", who);
  const int in_features = wa->cols;
  const int rank = wa->rows;
  if (tokens == 0 || rank == 0) return TRIS_OK;
  TRIS_REQUIRE(out_a != nullptr && (wb == nullptr || out_b != nullptr), "%s: null output", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nproj = wb != nullptr ? 2 : 1;
  if (in_features == 0) {
    const int64_t count = static_cast<int64_t>(tokens) * rank;
    for (int q = 0; q < nproj; ++q) {
      hipLaunchKernelGGL(fill_zero_u16_kernel, dim3(static_cast<unsigned>((count + 255) / 256)), dim3(256), 0, s,
                         q ? out_b : out_a, count);
    }
    return check_launch("fill_zero_u16_kernel");
  }
  TRIS_REQUIRE(x != nullptr, "%s: null input", who);
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(in_scale_a) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(in_scale_b) % 16 == 0,
               "%s: x and in_scale must be 16-byte aligned", who);
  const int slices = backbone_slices(tokens, in_features, rank, kBbPacked4TargetWgs);
  const int64_t need = backbone_workspace_bytes(tokens, in_features, rank, nproj, false, kBbPacked4TargetWgs);
  TRIS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
               "%s: workspace of %lld bytes needed, %lld given", who, static_cast<long long>(need),
               static_cast<long long>(workspace_bytes));
  const int token_tiles = ceil_div(tokens, 16);
  const int row_tiles = ceil_div(rank, 16);
  TRIS_REQUIRE(static_cast<int64_t>(token_tiles) * slices <= 65535, "%s: too many tokens", who);
  Packed4Args pa{};
  BackboneArgs& args = pa.base;
  args.x = x;
  args.row_index = row_index;
  args.proj[0] = BackboneProj{nullptr, out_a, in_scale_a};
  args.proj[1] = BackboneProj{nullptr, out_b, in_scale_b};
  args.partials = static_cast<float*>(workspace);
  args.tokens = tokens;
  args.in_features = in_features;
  args.rank = rank;
  args.slices = slices;
  args.slice_k = ceil_div(ceil_div(in_features, slices), kBbWaves * kBbKStep) * kBbWaves * kBbKStep;
  pa.proj[0] = Packed4Proj{wa->qweight, wa->qzeros, wa->scales, out_a};
  if (wb) pa.proj[1] = Packed4Proj{wb->qweight, wb->qzeros, wb->scales, out_b};
  pa.packed_cols = (in_features + 7) / 8;
  pa.qzeros_cols = (rank + 7) / 8;
  pa.group_size = wa->group_size;
  pa.num_groups = wa->num_groups;
  if (wb) {
    TRIS_REQUIRE(wb->group_size == wa->group_size && wb->num_groups == wa->num_groups, "%s: pair groups differ", who);
  }
  hipLaunchKernelGGL(packed4_backbone_kernel, dim3(row_tiles, token_tiles * slices, nproj), dim3(kBbThreads), 0, s,
                     pa);
  rc = check_launch(who);
  if (rc || slices == 1) return rc;
  const int64_t count = static_cast<int64_t>(tokens) * rank;
  hipLaunchKernelGGL(backbone_reduce_kernel, dim3(static_cast<unsigned>((count + 255) / 256), nproj), dim3(256), 0, s,
                     args);
  return check_launch(who);
}

}  // namespace tris

using namespace tris;

// Enough for tris_backbone_linear[_pair] and for tris_packed4_backbone_linear[_pair], whose plan keeps more slices.
static int64_t backbone_any_workspace_bytes(int tokens, int in_features, int rank, int nproj) {
  const int64_t a = backbone_workspace_bytes(tokens, in_features, rank, nproj);
  const int64_t b = backbone_workspace_bytes(tokens, in_features, rank, nproj, false, kBbPacked4TargetWgs);
  return a > b ? a : b;
}

extern "C" int64_t tris_backbone_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank) {
  return backbone_any_workspace_bytes(tokens, in_features, rank, 1);
}

extern "C" int64_t tris_backbone_pair_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank) {
  return backbone_any_workspace_bytes(tokens, in_features, rank, 2);
}

extern "C" int tris_backbone_linear(const uint16_t* x, int32_t tokens, int32_t in_features, const int64_t* row_index,
                                    const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  return launch_backbone(x, tokens, in_features, row_index, sv, nullptr, rank, in_scale, nullptr, out, nullptr,
                         workspace, workspace_bytes, stream, "tris_backbone_linear");
}

extern "C" int tris_backbone_linear_deferred(const uint16_t* x, int32_t tokens, int32_t in_features,
                                             const int64_t* row_index, const uint16_t* sv, int32_t rank,
                                             const uint16_t* in_scale, uint16_t* out, void* workspace,
                                             int64_t workspace_bytes, int32_t* slices, void* stream) {
  TRIS_REQUIRE(slices != nullptr, "tris_backbone_linear_deferred: null slice count");
  return launch_backbone(x, tokens, in_features, row_index, sv, nullptr, rank, in_scale, nullptr, out, nullptr,
                         workspace, workspace_bytes, stream, "tris_backbone_linear_deferred", true, slices);
}

// ---- tris_backbone_linear_noalloc: the split-K partial sums in a file-scope device array instead of a
// caller workspace, for callers that cannot allocate (code under HIP graph capture, tight serving loops).
// It runs the workspace entry's plan (the same kernel and slice count for every shape, so the same bits).
// The partial sums need slices * tokens * rank * 4 bytes.  On the decode-shaped kernel the slice count aims
// at kBbTargetWgs (256) workgroups of up to 64 x 16 outputs, which keeps that below 2 * 255 * 64 * 16 * 4 bytes
// (about 2 MiB) for every shape; the tiled GEMM of prefill-size batches (kBgMinRows rows on) can need
// more, and such shapes are rejected.  Every launch writes every partial sum it reads, so the array needs no
// clearing between calls.
constexpr int64_t kNoAllocScratchBytes = 4ll << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device (each GPU holds its own copy of the
// array at its own address; host code never passes the array's name itself to a kernel).
static int scratch_address(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("tris_backbone_linear_noalloc: hipGetDevice: %s", hipGetErrorString(err));
    return TRIS_ERR_HIP;
  }
  TRIS_REQUIRE(dev >= 0 && dev < kMaxDevices, "tris_backbone_linear_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error("tris_backbone_linear_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(err));
      return TRIS_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TRIS_OK;
}

extern "C" int64_t tris_backbone_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int tris_backbone_linear_noalloc(const uint16_t* x, int32_t tokens, int32_t in_features,
                                           const int64_t* row_index, const uint16_t* sv, int32_t rank,
                                           const uint16_t* in_scale, uint16_t* out, void* stream) {
  TRIS_REQUIRE(tokens >= 0 && in_features >= 0 && rank >= 0, "tris_backbone_linear_noalloc: negative shape");
  const int64_t need = backbone_workspace_bytes(tokens, in_features, rank, 1, true);
  TRIS_REQUIRE(need <= kNoAllocScratchBytes,
               "tris_backbone_linear_noalloc: %d tokens x %d in x %d rank need %lld bytes of scratch, the static "
               "buffer holds %lld (use tris_backbone_linear with a workspace)",
               tokens, in_features, rank, static_cast<long long>(need),
               static_cast<long long>(kNoAllocScratchBytes));
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc) return rc;
  }
  return launch_backbone(x, tokens, in_features, row_index, sv, nullptr, rank, in_scale, nullptr, out, nullptr, ws,
                         need, stream, "tris_backbone_linear_noalloc", true);
}

extern "C" int tris_backbone_linear_pair(const uint16_t* x, int32_t tokens, int32_t in_features,
                                         const int64_t* row_index, const uint16_t* sv_a, const uint16_t* sv_b,
                                         int32_t rank, const uint16_t* in_scale_a, const uint16_t* in_scale_b,
                                         uint16_t* out_a, uint16_t* out_b, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
  TRIS_REQUIRE(sv_b != nullptr, "tris_backbone_linear_pair: null sv_b");
  return launch_backbone(x, tokens, in_features, row_index, sv_a, sv_b, rank, in_scale_a, in_scale_b, out_a, out_b,
                         workspace, workspace_bytes, stream, "tris_backbone_linear_pair");
}

extern "C" int64_t tris_backbone_scatter_workspace_bytes(int32_t tokens, int32_t in_features, int32_t rank,
                                                         int32_t nproj) {
  if (tokens <= 0 || in_features <= 0 || rank <= 0 || nproj <= 0 || !backbone_gemm_fits(tokens, in_features, rank)) {
    return 0;
  }
  int slices = 1;
  backbone_gemm_slice_k(tokens, in_features, rank, &slices);
  return static_cast<int64_t>(slices) * nproj * tokens * rank * 4;
}

extern "C" int tris_backbone_linear_pair_scatter(const uint16_t* x, int32_t tokens, int32_t in_features,
                                                 const uint16_t* sv_a, const uint16_t* sv_b, int32_t rank,
                                                 const uint16_t* in_scale_a, const uint16_t* in_scale_b,
                                                 const int32_t* inverse_perm, int32_t top_k, int32_t out_rows,
                                                 uint16_t* out_a, uint16_t* out_b, void* workspace,
                                                 int64_t workspace_bytes, void* stream) {
  const char* who = "tris_backbone_linear_pair_scatter";
  TRIS_REQUIRE(tokens >= 0 && in_features >= 0 && rank >= 0 && top_k >= 0 && out_rows >= 0, "%s: negative shape",
               who);
  if (tokens == 0 || rank == 0 || top_k == 0 || out_rows == 0) return TRIS_OK;
  TRIS_REQUIRE(backbone_gemm_fits(tokens, in_features, rank),
               "%s: needs %d tokens or more, rank a multiple of %d and in_features a multiple of %d (got %d, %d, %d)",
               who, kBgMinRows, kBgN, kBgK, tokens, rank, in_features);
  TRIS_REQUIRE(x && sv_a && out_a && inverse_perm && (sv_b == nullptr || out_b != nullptr), "%s: null pointer", who);
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(sv_a) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(sv_b) % 16 == 0 && reinterpret_cast<uintptr_t>(in_scale_a) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(in_scale_b) % 16 == 0,
               "%s: x, sv and in_scale must be 16-byte aligned", who);
  const int nproj = sv_b != nullptr ? 2 : 1;
  const int64_t need = tris_backbone_scatter_workspace_bytes(tokens, in_features, rank, nproj);
  TRIS_REQUIRE(workspace != nullptr && workspace_bytes >= need, "%s: workspace of %lld bytes needed, %lld given", who,
               static_cast<long long>(need), static_cast<long long>(workspace_bytes));
  BackboneArgs ga{};
  ga.x = x;
  ga.proj[0] = BackboneProj{sv_a, out_a, in_scale_a};
  ga.proj[1] = BackboneProj{sv_b, out_b, in_scale_b};
  ga.partials = static_cast<float*>(workspace);
  ga.tokens = tokens;
  ga.in_features = in_features;
  ga.rank = rank;
  return launch_backbone_gemm(ga, nproj, static_cast<hipStream_t>(stream), who, inverse_perm, top_k, out_rows);
}

// More than kSgMaxRowTiles 16-row tiles take the tiled GEMM with the product formed in its operand staging.
// The tiled GEMM above one row group of the decode kernel, except for a rank that is not a multiple of 512 up to
// kSgMaxRowGroups row groups (its 512-column tiles would be partial): the decode kernel's row groups there.
static bool swiglu_backbone_gemm(int rows, int in_features, int rank) {
  if (rows <= kSgMaxRowTiles * 16) return false;
  if (rank % 512 != 0 && rows <= kSgMaxRowGroups * kSgMaxRowTiles * 16) return false;
  return rank % kBgN == 0 && in_features % kBgK == 0;
}

extern "C" int64_t tris_backbone_swiglu_workspace_bytes(int32_t rows, int32_t in_features, int32_t rank) {
  if (rows <= 0 || in_features <= 0 || rank <= 0) return 0;
  int slices = 1;
  if (swiglu_backbone_gemm(rows, in_features, rank)) {
    backbone_wide_slice_k(rows, in_features, rank, &slices);
  } else {
    swiglu_backbone_slice_k(in_features, rank, &slices);
  }
  return slices > 1 ? static_cast<int64_t>(slices) * rows * rank * 4 : 0;
}

static int swiglu_linear(const uint16_t* gate, const uint16_t* up, int32_t rows, int32_t in_features,
                         const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out, uint16_t* out_hi,
                         int32_t split, void* workspace, int64_t workspace_bytes, void* stream, const char* who) {
  TRIS_REQUIRE(rows >= 0 && in_features >= 0 && rank >= 0, "%s: negative shape", who);
  if (rows == 0 || rank == 0) return TRIS_OK;
  TRIS_REQUIRE(in_features > 0 && in_features % 32 == 0, "%s: in_features %d must be a positive multiple of 32", who,
               in_features);
  TRIS_REQUIRE(rows <= kSgMaxRowGroups * kSgMaxRowTiles * 16 || rank % kBgN == 0,
               "%s: %d rows need a rank that is a multiple of %d (rank %d)", who, rows, kBgN, rank);
  TRIS_REQUIRE(gate && up && sv && out, "%s: null pointer", who);
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(gate) % 16 == 0 && reinterpret_cast<uintptr_t>(up) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(sv) % 16 == 0 && reinterpret_cast<uintptr_t>(in_scale) % 16 == 0,
               "%s: gate, up, sv and in_scale must be 16-byte aligned", who);
  const int64_t need = tris_backbone_swiglu_workspace_bytes(rows, in_features, rank);
  TRIS_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
               "%s: workspace of %lld bytes needed, %lld given", who, static_cast<long long>(need),
               static_cast<long long>(workspace_bytes));
  hipStream_t s = static_cast<hipStream_t>(stream);
  TRIS_REQUIRE(split >= 0 && split < rank && (split == 0 || out_hi != nullptr), "%s: column split %d of %d columns",
               who, split, rank);
  TRIS_REQUIRE(split == 0 || !swiglu_backbone_gemm(rows, in_features, rank),
               "%s: a column split runs on the decode kernel, not on the tiled GEMM of %d rows", who, rows);
  if (swiglu_backbone_gemm(rows, in_features, rank)) {
    BackboneArgs ga{};
    ga.x = gate;
    ga.proj[0] = BackboneProj{sv, out, in_scale};
    ga.partials = static_cast<float*>(workspace);
    ga.tokens = rows;
    ga.in_features = in_features;
    ga.rank = rank;
    return launch_backbone_swiglu_gemm(ga, up, s, who);
  }
  int slices = 1;
  const int slice_k = swiglu_backbone_slice_k(in_features, rank, &slices);
  SwigluBackboneArgs a{gate, up, sv, in_scale, out, static_cast<float*>(workspace), rows, in_features, rank, slices,
                       slice_k, out_hi, split};
  // past kSgMaxRowTiles row tiles, row groups of that many (blockIdx.z), each staging its own rows' product and
  // reading the slice's SV again
  const int tt = ceil_div(rows, 16) < kSgMaxRowTiles ? ceil_div(rows, 16) : kSgMaxRowTiles;
  const size_t lds = static_cast<size_t>(tt) * 16 * (slice_k + 8) * 2;
  TRIS_REQUIRE(lds <= 64 * 1024, "%s: %zu bytes of LDS for a %d-column slice", who, lds, slice_k);
  const dim3 grid(ceil_div(rank, kSgCols), slices, ceil_div(rows, kSgMaxRowTiles * 16));
  switch (tt) {
    case 1: hipLaunchKernelGGL((backbone_swiglu_kernel<1>), grid, dim3(kSgThreads), lds, s, a); break;
    case 2: hipLaunchKernelGGL((backbone_swiglu_kernel<2>), grid, dim3(kSgThreads), lds, s, a); break;
    case 3: hipLaunchKernelGGL((backbone_swiglu_kernel<3>), grid, dim3(kSgThreads), lds, s, a); break;
    case 4: hipLaunchKernelGGL((backbone_swiglu_kernel<4>), grid, dim3(kSgThreads), lds, s, a); break;
    case 5: hipLaunchKernelGGL((backbone_swiglu_kernel<5>), grid, dim3(kSgThreads), lds, s, a); break;
    case 6: hipLaunchKernelGGL((backbone_swiglu_kernel<6>), grid, dim3(kSgThreads), lds, s, a); break;
    case 7: hipLaunchKernelGGL((backbone_swiglu_kernel<7>), grid, dim3(kSgThreads), lds, s, a); break;
    default: hipLaunchKernelGGL((backbone_swiglu_kernel<8>), grid, dim3(kSgThreads), lds, s, a); break;
  }
  int rc = check_launch(who);
  if (rc || slices == 1) return rc;
  BackboneArgs ra{};
  ra.proj[0].out = out;
  ra.proj[0].out_hi = out_hi;
  ra.proj[0].split = split;
  ra.partials = static_cast<float*>(workspace);
  ra.tokens = rows;
  ra.in_features = in_features;
  ra.rank = rank;
  ra.slices = slices;
  return launch_backbone_reduce(ra, 1, s, who);
}

extern "C" int tris_backbone_swiglu_linear(const uint16_t* gate, const uint16_t* up, int32_t rows, int32_t in_features,
                                           const uint16_t* sv, int32_t rank, const uint16_t* in_scale, uint16_t* out,
                                           void* workspace, int64_t workspace_bytes, void* stream) {
  return swiglu_linear(gate, up, rows, in_features, sv, rank, in_scale, out, nullptr, 0, workspace, workspace_bytes,
                       stream, "tris_backbone_swiglu_linear");
}

extern "C" int tris_backbone_swiglu_linear_split(const uint16_t* gate, const uint16_t* up, int32_t rows,
                                                 int32_t in_features, const uint16_t* sv, int32_t rank,
                                                 const uint16_t* in_scale, uint16_t* out, uint16_t* out_hi,
                                                 int32_t split, void* workspace, int64_t workspace_bytes,
                                                 void* stream) {
  TRIS_REQUIRE(split > 0, "tris_backbone_swiglu_linear_split: split %d must be positive", split);
  return swiglu_linear(gate, up, rows, in_features, sv, rank, in_scale, out, out_hi, split, workspace,
                       workspace_bytes, stream, "tris_backbone_swiglu_linear_split");
}

extern "C" int tris_packed4_dequant(const tris_packed4_matrix* w, uint16_t* out, void* stream) {
  int rc = check_packed4(w, false, "tris_packed4_dequant");
  if (rc) return rc;
  if (w->rows == 0 || w->cols == 0) return TRIS_OK;
  TRIS_REQUIRE(out != nullptr, "tris_packed4_dequant: null output");
  const int64_t n = static_cast<int64_t>((w->cols + 7) / 8) * w->rows;
  hipLaunchKernelGGL(packed4_dequant_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), *w, out);
  return check_launch("tris_packed4_dequant");
}

extern "C" int tris_packed4_backbone_linear(const uint16_t* x, int32_t tokens, const int64_t* row_index,
                                            const tris_packed4_matrix* w, const uint16_t* in_scale, uint16_t* out,
                                            void* workspace, int64_t workspace_bytes, void* stream) {
  return launch_packed4_backbone(x, tokens, row_index, w, nullptr, in_scale, nullptr, out, nullptr, workspace,
                                 workspace_bytes, stream, "tris_packed4_backbone_linear");
}

extern "C" int tris_packed4_backbone_linear_pair(const uint16_t* x, int32_t tokens, const int64_t* row_index,
                                                 const tris_packed4_matrix* wa, const tris_packed4_matrix* wb,
                                                 const uint16_t* in_scale_a, const uint16_t* in_scale_b,
                                                 uint16_t* out_a, uint16_t* out_b, void* workspace,
                                                 int64_t workspace_bytes, void* stream) {
  TRIS_REQUIRE(wb != nullptr, "tris_packed4_backbone_linear_pair: null second matrix");
  return launch_packed4_backbone(x, tokens, row_index, wa, wb, in_scale_a, in_scale_b, out_a, out_b, workspace,
                                 workspace_bytes, stream, "tris_packed4_backbone_linear_pair");
}
