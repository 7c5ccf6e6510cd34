// Grouped compact3 expert GEMM for gfx950 with the block-GR split bitmap
// decoded inside the kernel, plus the dense-dequant verification kernel.
//
// Reference kernels replaced: Compact3TriSMoEPrecomputedGroupedSegmentBlockGRKernel
// (TriSMoE_cuda_kernel.cu:4500-4681), ...DecodeBlockGRKernel (:5382-5586), their
// split-K and dual variants (:5628-7716) and the predecoded segment kernels
// (:4720-4885, :5094-5380).  Arithmetic per weight follows kernel.cu:665-774:
// exact fp16 weights (RNE __hmul/__hadd), accumulated in fp32.
//
// Work decomposition (one workgroup = 4 wavefronts):
//   * blockIdx.x = 64-output tile (one GR block column), blockIdx.y = a tile
//     of up to MT consecutive rows of one segment (one expert), blockIdx.z =
//     projection (0 or 1 for the gate/up pair).
//   * lane = output column; wave w owns the 64-column K blocks w, w+4, ...:
//     it decodes that block's split bitmap into its own LDS slot
//     (wavefront-parallel GR decode) and reconstructs the 64x64 weights in
//     registers, so decoded bits and weights never touch HBM.
//   * qweight1 rows are read as 256-byte coalesced wave loads ([e][k/32][n] is
//     n-contiguous); hidden rows are staged in LDS as fp32 and read as
//     broadcasts; the four per-wave partial sums are reduced through LDS.
//   * Every row of an expert's segment (up to MT) shares one decode of the
//     bitmap, unlike the reference's 4-row tiles that re-decode per tile.
#include "tris_gr_decode.h"

namespace tris {

constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = kGemmWaves * kWave;
constexpr int kGemmRows = 16;  // MT: rows per workgroup tile

// Where the kernel takes each packed row's split bits from.
constexpr int kGmapGr = 0;          // the payload's block-GR stream, decoded in the kernel
constexpr int kGmapPredecoded = 1;  // predecoded words [num_segments, nblk, 128]
constexpr int kGmapSparse = 2;      // the sparse form: non-salient columns only, compacted (SparseGmap)

// Split bitmap in the sparse form (TRIS_COMPACT3_BLOCK_GR=0 payloads): the j-th non-salient column of an expert
// (k order) is bit j % 32 of row j / 32 of words [E, rows, N]; prefix [E, packed_rows + 1] counts the
// non-salient columns before each packed row.
struct SparseGmap {
  const int32_t* words;
  const int32_t* prefix;
  int rows;
};

struct ProjArgs {
  const uint16_t* hidden;   // [batch, rank]
  uint16_t* out;            // [batch, N]
  const int32_t* decoded;   // predecoded words [num_segments, nblk, 128] (predecoded variant)
  tris_compact3_payload p;
  const uint16_t* input_scale;  // fp16 [rank] or NULL: the activation is fp16(hidden * input_scale) per column
  const float* addend;          // fp32 [batch, N] or NULL: added to the sum before the output scale
  SparseGmap sparse;            // the sparse variant's split bitmap
};

struct GroupedArgs {
  ProjArgs proj[2];
  const int32_t* expert_ids;
  const int32_t* segment_offsets;  // NULL: one segment of all batch rows, expert 0 (a non-expert linear)
  int num_segments;
  int row_tile;
  int batch;
};

// Map workgroup tile index -> (segment, first row, row count) with row_tile
// rows per tile; wave-uniform result.  Returns false past the last tile.
__device__ inline bool map_row_tile(const int32_t* __restrict__ seg, int nseg, int tile, int row_tile, int* s_out,
                                    int* row0_out, int* rc_out) {
  const int lane = static_cast<int>(__lane_id());
  int base = 0;
  for (int c = 0; c < nseg; c += kWave) {
    const int i = c + lane;
    int t = 0;
    if (i < nseg) {
      const int len = seg[i + 1] - seg[i];
      t = len > 0 ? (len + row_tile - 1) / row_tile : 0;
    }
    int incl = t;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    const int total = __shfl(incl, kWave - 1);
    if (tile < base + total) {
      const uint64_t hit = __ballot(i < nseg && tile < base + incl);
      const int L = __ffsll(static_cast<unsigned long long>(hit)) - 1;
      const int excl = __shfl(incl - t, L);
      const int s = c + L;
      const int local = tile - base - excl;
      const int row0 = seg[s] + local * row_tile;
      const int end = seg[s + 1];
      *s_out = s;
      *row0_out = row0;
      *rc_out = (end - row0) < row_tile ? (end - row0) : row_tile;
      return true;
    }
    base += total;
  }
  return false;
}

// One compact3 weight in exact fp16 (kernel.cu:665-774).  clo/chi: the column
// pack's halves (s_c1 | s_c2 << 16, ns_d_c1 | ns_nd_c1 << 16); rlo/rhi: the
// row pack's halves in the same order.
__device__ __forceinline__ uint16_t compact3_weight(bool salient, uint32_t sign1, uint32_t sign2, uint32_t large,
                                                    uint32_t clo, uint32_t chi, uint32_t rlo, uint32_t rhi) {
  if (salient) {
    uint16_t t1 = hmul_bits(static_cast<uint16_t>(clo), static_cast<uint16_t>(rlo));
    if (!sign1) t1 ^= 0x8000u;
    uint16_t t2 = hmul_bits(static_cast<uint16_t>(clo >> 16), static_cast<uint16_t>(rlo >> 16));
    if (!sign2) t2 ^= 0x8000u;
    return hadd_bits(t1, t2);
  }
  const uint32_t c = large ? chi : (chi >> 16);
  const uint32_t r = large ? rhi : (rhi >> 16);
  uint16_t w = hmul_bits(static_cast<uint16_t>(c), static_cast<uint16_t>(r));
  if (!sign1) w ^= 0x8000u;
  return w;
}

// Second-term signs of the salient columns of packed row pr, expanded to a
// dense 32-bit word (kernel.cu:599-663: sparse index = prefix[pr] + rank of
// the column among the row's salient columns).
__device__ __forceinline__ uint32_t dense_qweight2_word(const int32_t* __restrict__ q2, const int32_t* __restrict__ q2_prefix,
                                                        uint32_t cmap_word, int pr, int n, int N, bool nv) {
  uint32_t dense = 0u;
  if (cmap_word == 0u) return dense;
  const int sp = q2_prefix[pr];
  uint32_t pending = cmap_word;
  int j = 0;
  int cached_row = -1;
  uint32_t cached = 0u;
  while (pending != 0u) {
    const int b = __builtin_ctz(pending);
    const int idx = sp + j;
    const int row = idx >> 5;
    if (row != cached_row) {
      cached_row = row;
      cached = nv ? static_cast<uint32_t>(q2[static_cast<int64_t>(row) * N + n]) : 0u;
    }
    dense |= ((cached >> (idx & 31)) & 1u) << b;
    pending &= pending - 1u;
    ++j;
  }
  return dense;
}

// Split bits of packed row pr for column n from the sparse form (the reference looks each bit up,
// kernel.cu:619-637: index prefix[pr] + the column's rank among the row's non-salient columns).  The row's
// non-salient bits are one run of the column's sparse stream, read from at most two words; a zero is then
// inserted at each salient column (c_map is per row, so the loop is uniform across the wavefront).  Reads past
// the stream give zeros.
__device__ __forceinline__ uint32_t sparse_gmap_word(const int32_t* __restrict__ words,
                                                     const int32_t* __restrict__ prefix, int rows, uint32_t cmap_word,
                                                     int pr, int n, int N, bool nv) {
  const int j0 = prefix[pr];
  const int r0 = j0 >> 5;
  if (!nv || cmap_word == 0xFFFFFFFFu || j0 < 0 || r0 >= rows) return 0u;
  const uint32_t lo = static_cast<uint32_t>(words[static_cast<int64_t>(r0) * N + n]);
  const uint32_t hi = r0 + 1 < rows ? static_cast<uint32_t>(words[static_cast<int64_t>(r0 + 1) * N + n]) : 0u;
  const uint32_t sh = static_cast<uint32_t>(j0) & 31u;
  uint32_t d = sh == 0u ? lo : ((lo >> sh) | (hi << (32u - sh)));
  uint32_t pending = cmap_word;
  while (pending != 0u) {
    const uint32_t below = (1u << __builtin_ctz(pending)) - 1u;
    d = (d & below) | ((d & ~below) << 1);
    pending &= pending - 1u;
  }
  return d;
}

// kSrc: kGmapGr, kGmapPredecoded or kGmapSparse.  kNumProj (1 or 2) only separates the single and gate/up-pair
// launches in profiles; the pair selects its projection by blockIdx.z.
template <int kSrc, int kNumProj>
__global__ __launch_bounds__(kGemmThreads) void grouped_gemm_kernel(GroupedArgs a) {
  constexpr int MT = kGemmRows;
  __shared__ float xs[MT][kGemmWaves * kTileK];
  __shared__ uint32_t gm[kGemmWaves][kGrWords];
  __shared__ float red[kGemmWaves - 1][MT][kWave];

  const ProjArgs& pa = a.proj[kNumProj == 1 ? 0 : blockIdx.z];
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int n0 = blockIdx.x * kTileOut;
  if (n0 >= N) return;  // uniform over the workgroup, before any barrier

  int s = 0, row0 = 0, rc = 0;
  if (a.segment_offsets == nullptr) {  // uniform: every row in one segment of expert 0
    row0 = static_cast<int>(blockIdx.y) * a.row_tile;
    if (row0 >= a.batch) return;
    rc = (a.batch - row0) < a.row_tile ? (a.batch - row0) : a.row_tile;
  } else if (!map_row_tile(a.segment_offsets, a.num_segments, blockIdx.y, a.row_tile, &s, &row0, &rc)) {
    return;
  }

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int n = n0 + lane;
  const bool nv = n < N;
  const int e = a.segment_offsets == nullptr ? 0 : a.expert_ids[s];
  uint16_t* out = pa.out;

  // Negative slots give zero rows (the reference's expert_valid); ids past the
  // payload are treated the same way instead of being read out of bounds.
  if (e < 0 || e >= p.num_experts) {
    if (wave == 0 && nv) {
      for (int r = 0; r < rc; ++r) out[static_cast<int64_t>(row0 + r) * N + n] = 0;
    }
    return;
  }

  const int rank = p.rank;
  const int packed_rows = ceil_div(rank, 32);
  const int nkb = ceil_div(packed_rows, kGrPackedRows);
  const int nob = ceil_div(N, kTileOut);
  const int nblk = nkb * nob;
  const int ob = blockIdx.x;
  const int G = p.num_groups;

  const int32_t* q1_e = p.qweight1 + static_cast<int64_t>(e) * packed_rows * N;
  const int32_t* q2_e = p.qweight2_sparse + static_cast<int64_t>(e) * p.qweight2_sparse_rows * N;
  const int32_t* q2p_e = p.qweight2_sparse_prefix + static_cast<int64_t>(e) * (packed_rows + 1);
  const int32_t* cmap_e = p.c_map + static_cast<int64_t>(e) * packed_rows;
  const int32_t* gidx_e = p.g_idx + static_cast<int64_t>(e) * rank;
  const int64_t* col_e = p.col_pack3 + static_cast<int64_t>(e) * rank;
  const int64_t* row_e = p.row_pack3 + static_cast<int64_t>(e) * N * G;
  const int32_t* grw_e = nullptr;
  const int32_t* gro_e = nullptr;
  const int32_t* grm_e = nullptr;
  if (kSrc == kGmapGr && p.q_gmap_gr_offsets != nullptr) {
    grw_e = p.q_gmap_gr_words + static_cast<int64_t>(e) * p.gr_words_stride;
    gro_e = p.q_gmap_gr_offsets + static_cast<int64_t>(e) * (nblk + 1);
    grm_e = p.q_gmap_gr_meta + static_cast<int64_t>(e) * nblk;
  }
  const int32_t* dec_s = kSrc == kGmapPredecoded ? pa.decoded + static_cast<int64_t>(s) * nblk * kGrWords : nullptr;
  const int32_t* gs_e = nullptr;
  const int32_t* gsp_e = nullptr;
  if (kSrc == kGmapSparse) {
    gs_e = pa.sparse.words + static_cast<int64_t>(e) * pa.sparse.rows * N;
    gsp_e = pa.sparse.prefix + static_cast<int64_t>(e) * (packed_rows + 1);
  }
  const uint16_t* hid = pa.hidden;

  float acc[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r) acc[r] = 0.0f;

  for (int kc = 0; kc < nkb; kc += kGemmWaves) {
    __syncthreads();
    const int kchunk = kc * kTileK;
    for (int idx = tid; idx < rc * (kGemmWaves * kTileK); idx += kGemmThreads) {
      const int r = idx / (kGemmWaves * kTileK);
      const int j = idx % (kGemmWaves * kTileK);
      const int k = kchunk + j;
      float xv = k < rank ? h2f(hid[static_cast<int64_t>(row0 + r) * rank + k]) : 0.0f;
      if (pa.input_scale != nullptr && k < rank) xv = h2f(f2h_bits(xv * h2f(pa.input_scale[k])));  // __hmul
      xs[r][j] = xv;
    }
    __syncthreads();
    const int kb = kc + wave;
    if (kb >= nkb) continue;

    uint32_t gwords[kGrPackedRows];
    if (kSrc == kGmapPredecoded) {
      const int32_t* src = dec_s + static_cast<int64_t>(kb * nob + ob) * kGrWords;
      gwords[0] = static_cast<uint32_t>(src[lane]);
      gwords[1] = static_cast<uint32_t>(src[kWave + lane]);
    } else if (kSrc == kGmapSparse) {
#pragma unroll
      for (int lpr = 0; lpr < kGrPackedRows; ++lpr) {
        const int pr = kb * kGrPackedRows + lpr;
        gwords[lpr] = pr < packed_rows ? sparse_gmap_word(gs_e, gsp_e, pa.sparse.rows,
                                                          static_cast<uint32_t>(cmap_e[pr]), pr, n, N, nv)
                                       : 0u;
      }
    } else {
      gr_decode_block_wave(grw_e, gro_e, grm_e, kb * nob + ob, gm[wave]);
      gwords[0] = gm[wave][lane];
      gwords[1] = gm[wave][kWave + lane];
    }

    const int tile_group = gidx_e[kb * kTileK];
    int cur_group = -2;
    uint32_t rlo = 0u, rhi = 0u;
#pragma unroll
    for (int lpr = 0; lpr < kGrPackedRows; ++lpr) {
      const int pr = kb * kGrPackedRows + lpr;
      if (pr >= packed_rows) break;
      const int kbase = pr * 32;
      const int nbits = (rank - kbase) < 32 ? (rank - kbase) : 32;
      const uint32_t q1 = nv ? static_cast<uint32_t>(q1_e[static_cast<int64_t>(pr) * N + n]) : 0u;
      const uint32_t gw = gwords[lpr];
      const uint32_t cw = static_cast<uint32_t>(cmap_e[pr]) & low_mask(nbits);
      const uint32_t q2 = dense_qweight2_word(q2_e, q2p_e, cw, pr, n, N, nv);
      // Column packs of this packed row: lane l holds column kbase + l.
      const uint64_t cp = lane < nbits ? static_cast<uint64_t>(col_e[kbase + lane]) : 0ull;
      const uint32_t cp_lo = static_cast<uint32_t>(cp);
      const uint32_t cp_hi = static_cast<uint32_t>(cp >> 32);
      const int xoff = (kb - kc) * kTileK + lpr * 32;
#pragma unroll
      for (int b8 = 0; b8 < 32; b8 += 8) {
        if (b8 >= nbits) break;
        float wf[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int b = b8 + u;
          if (b < nbits) {
            const int g = p.use_uniform_k64_groups ? tile_group : gidx_e[kbase + b];
            if (g != cur_group) {
              cur_group = g;
              uint64_t rp = 0ull;
              if (nv && g >= 0 && g < G) rp = static_cast<uint64_t>(row_e[static_cast<int64_t>(n) * G + g]);
              rlo = static_cast<uint32_t>(rp);
              rhi = static_cast<uint32_t>(rp >> 32);
            }
            const uint32_t clo = __builtin_amdgcn_readlane(cp_lo, b);
            const uint32_t chi = __builtin_amdgcn_readlane(cp_hi, b);
            const uint16_t w = compact3_weight((cw >> b) & 1u, (q1 >> b) & 1u, (q2 >> b) & 1u, (gw >> b) & 1u,
                                               clo, chi, rlo, rhi);
            wf[u] = h2f(w);
          } else {
            wf[u] = 0.0f;
          }
        }
#pragma unroll
        for (int r = 0; r < MT; ++r) {
          if (r < rc) {
            const float4 x0 = *reinterpret_cast<const float4*>(&xs[r][xoff + b8]);
            const float4 x1 = *reinterpret_cast<const float4*>(&xs[r][xoff + b8 + 4]);
            float v = acc[r];
            v = fmaf(x0.x, wf[0], v);
            v = fmaf(x0.y, wf[1], v);
            v = fmaf(x0.z, wf[2], v);
            v = fmaf(x0.w, wf[3], v);
            v = fmaf(x1.x, wf[4], v);
            v = fmaf(x1.y, wf[5], v);
            v = fmaf(x1.z, wf[6], v);
            v = fmaf(x1.w, wf[7], v);
            acc[r] = v;
          }
        }
      }
    }
  }

  __syncthreads();
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < MT; ++r) red[wave - 1][r][lane] = acc[r];
  }
  __syncthreads();
  if (wave == 0 && nv) {
    const float scale = p.has_output_scale ? h2f(p.output_scale[static_cast<int64_t>(e) * N + n]) : 1.0f;
    const float bias = p.has_bias ? h2f(p.bias[static_cast<int64_t>(e) * N + n]) : 0.0f;
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      if (r < rc) {
        float v = acc[r] + red[0][r][lane] + red[1][r][lane] + red[2][r][lane];
        if (pa.addend != nullptr) v += pa.addend[static_cast<int64_t>(row0 + r) * N + n];
        if (p.has_output_scale) v = v * scale;
        if (p.has_bias) v = v + bias;
        out[static_cast<int64_t>(row0 + r) * N + n] = f2h_bits(v);
      }
    }
  }
}

// Dense fp16 weights [num, N, rank]; grid = (ceil(N/64), nkb, num), one wave.
__global__ __launch_bounds__(kWave) void compact3_dequant_kernel(tris_compact3_payload p, const int32_t* expert_ids,
                                                                 uint16_t* __restrict__ weights) {
  __shared__ uint32_t gm[kGrWords];
  const int lane = threadIdx.x;
  const int N = p.outfeatures;
  const int rank = p.rank;
  const int packed_rows = ceil_div(rank, 32);
  const int nkb = ceil_div(packed_rows, kGrPackedRows);
  const int nob = ceil_div(N, kTileOut);
  const int nblk = nkb * nob;
  const int ob = blockIdx.x;
  const int kb = blockIdx.y;
  const int item = blockIdx.z;
  const int e = expert_ids[item];
  const int n = ob * kTileOut + lane;
  const bool nv = n < N;
  const int G = p.num_groups;
  uint16_t* w_out = weights + static_cast<int64_t>(item) * N * rank;
  if (e < 0 || e >= p.num_experts) {
    if (nv) {
      for (int k = kb * kTileK; k < rank && k < (kb + 1) * kTileK; ++k) w_out[static_cast<int64_t>(n) * rank + k] = 0;
    }
    return;
  }
  const int32_t* q1_e = p.qweight1 + static_cast<int64_t>(e) * packed_rows * N;
  const int32_t* q2_e = p.qweight2_sparse + static_cast<int64_t>(e) * p.qweight2_sparse_rows * N;
  const int32_t* q2p_e = p.qweight2_sparse_prefix + static_cast<int64_t>(e) * (packed_rows + 1);
  const int32_t* cmap_e = p.c_map + static_cast<int64_t>(e) * packed_rows;
  const int32_t* gidx_e = p.g_idx + static_cast<int64_t>(e) * rank;
  const int64_t* col_e = p.col_pack3 + static_cast<int64_t>(e) * rank;
  const int64_t* row_e = p.row_pack3 + static_cast<int64_t>(e) * N * G;
  const int32_t* grw_e = p.q_gmap_gr_offsets ? p.q_gmap_gr_words + static_cast<int64_t>(e) * p.gr_words_stride : nullptr;
  const int32_t* gro_e = p.q_gmap_gr_offsets ? p.q_gmap_gr_offsets + static_cast<int64_t>(e) * (nblk + 1) : nullptr;
  const int32_t* grm_e = p.q_gmap_gr_offsets ? p.q_gmap_gr_meta + static_cast<int64_t>(e) * nblk : nullptr;
  gr_decode_block_wave(grw_e, gro_e, grm_e, kb * nob + ob, gm);
  const int tile_group = gidx_e[kb * kTileK];
  for (int lpr = 0; lpr < kGrPackedRows; ++lpr) {
    const int pr = kb * kGrPackedRows + lpr;
    if (pr >= packed_rows) break;
    const int kbase = pr * 32;
    const int nbits = (rank - kbase) < 32 ? (rank - kbase) : 32;
    const uint32_t q1 = nv ? static_cast<uint32_t>(q1_e[static_cast<int64_t>(pr) * N + n]) : 0u;
    const uint32_t gw = gm[lpr * kTileOut + lane];
    const uint32_t cw = static_cast<uint32_t>(cmap_e[pr]) & low_mask(nbits);
    const uint32_t q2 = dense_qweight2_word(q2_e, q2p_e, cw, pr, n, N, nv);
    for (int b = 0; b < nbits; ++b) {
      const int k = kbase + b;
      const int g = p.use_uniform_k64_groups ? tile_group : gidx_e[k];
      uint64_t rp = 0ull;
      if (nv && g >= 0 && g < G) rp = static_cast<uint64_t>(row_e[static_cast<int64_t>(n) * G + g]);
      const uint64_t cp = static_cast<uint64_t>(col_e[k]);
      const uint16_t w = compact3_weight((cw >> b) & 1u, (q1 >> b) & 1u, (q2 >> b) & 1u, (gw >> b) & 1u,
                                         static_cast<uint32_t>(cp), static_cast<uint32_t>(cp >> 32),
                                         static_cast<uint32_t>(rp), static_cast<uint32_t>(rp >> 32));
      if (nv) w_out[static_cast<int64_t>(n) * rank + k] = w;
    }
  }
}

// Host-side validation of one payload descriptor.
int check_payload(const tris_compact3_payload* p, bool need_gr, const char* who) {
  TRIS_REQUIRE(p != nullptr, "%s: null payload", who);
  TRIS_REQUIRE(p->num_experts >= 0 && p->rank >= 0 && p->outfeatures >= 0 && p->num_groups >= 0 &&
                   p->qweight2_sparse_rows >= 0 && p->gr_words_stride >= 0,
               "%s: negative payload dimension", who);
  if (p->num_experts == 0 || p->rank == 0 || p->outfeatures == 0) return TRIS_OK;
  TRIS_REQUIRE(p->qweight1 && p->qweight2_sparse_prefix && p->c_map && p->g_idx && p->col_pack3,
               "%s: null payload tensor", who);
  TRIS_REQUIRE(p->num_groups == 0 || p->row_pack3, "%s: null row_pack3", who);
  TRIS_REQUIRE(p->qweight2_sparse_rows == 0 || p->qweight2_sparse, "%s: null qweight2_sparse", who);
  TRIS_REQUIRE(!p->has_output_scale || p->output_scale, "%s: has_output_scale without output_scale", who);
  TRIS_REQUIRE(!p->has_bias || p->bias, "%s: has_bias without bias", who);
  if (need_gr) {
    TRIS_REQUIRE(p->q_gmap_gr_offsets && p->q_gmap_gr_meta, "%s: null q_gmap_gr_offsets/meta", who);
    TRIS_REQUIRE(p->gr_words_stride == 0 || p->q_gmap_gr_words, "%s: null q_gmap_gr_words", who);
  }
  return TRIS_OK;
}

// Upper bound on the number of row tiles of row_tile rows: every segment
// contributes ceil(len / row_tile) <= len / row_tile + 1, and the route's own
// count (m_tile 4) is also a bound.
int64_t row_tile_bound(int batch, int num_segments, int64_t total_problem_tiles, int row_tile) {
  const int64_t bound = static_cast<int64_t>(batch) / row_tile + num_segments;
  return total_problem_tiles < bound ? total_problem_tiles : bound;
}

// src: kGmapGr, kGmapPredecoded (decoded_a/b) or kGmapSparse (sparse: one projection).
int launch_grouped(const uint16_t* hidden_a, const uint16_t* hidden_b, int batch, const int32_t* expert_ids,
                   const int32_t* segment_offsets, int num_segments, int64_t total_problem_tiles,
                   const int32_t* decoded_a, const int32_t* decoded_b, const tris_compact3_payload* pa,
                   const tris_compact3_payload* pb, uint16_t* out_a, uint16_t* out_b, int src,
                   void* stream, const char* who, const SparseGmap* sparse = nullptr) {
  const int nproj = pb ? 2 : 1;
  const bool predecoded = src == kGmapPredecoded;
  TRIS_REQUIRE(batch >= 0 && num_segments >= 0, "%s: negative batch or segment count", who);
  TRIS_REQUIRE(src != kGmapSparse || (sparse != nullptr && pb == nullptr), "%s: sparse bitmaps for one projection",
               who);
  int rc = check_payload(pa, src == kGmapGr, who);
  if (rc) return rc;
  if (src == kGmapSparse && pa->num_experts > 0 && pa->rank > 0 && pa->outfeatures > 0) {
    TRIS_REQUIRE(sparse->rows >= 0, "%s: negative q_gmap_sparse row count", who);
    TRIS_REQUIRE(sparse->prefix != nullptr && (sparse->rows == 0 || sparse->words != nullptr),
                 "%s: null q_gmap_sparse / q_gmap_sparse_prefix", who);
  }
  if (pb) {
    rc = check_payload(pb, src == kGmapGr, who);
    if (rc) return rc;
    TRIS_REQUIRE(pa->num_experts == pb->num_experts, "%s: expert count mismatch between the pair", who);
  }
  if (batch == 0 || num_segments == 0 || total_problem_tiles <= 0) return TRIS_OK;
  TRIS_REQUIRE(hidden_a && out_a && expert_ids && segment_offsets, "%s: null pointer", who);
  TRIS_REQUIRE(!pb || (hidden_b && out_b), "%s: null pointer (second projection)", who);
  TRIS_REQUIRE(!predecoded || (decoded_a && (!pb || decoded_b)), "%s: null predecoded words", who);
  int max_n = 0;
  for (int i = 0; i < nproj; ++i) {
    const tris_compact3_payload* p = i ? pb : pa;
    if (p->num_experts == 0 || p->rank == 0 || p->outfeatures == 0) {
      TRIS_REQUIRE(false, "%s: empty payload with a non-empty route", who);
    }
    max_n = p->outfeatures > max_n ? p->outfeatures : max_n;
  }
  const int64_t tiles = row_tile_bound(batch, num_segments, total_problem_tiles, kGemmRows);
  TRIS_REQUIRE(tiles <= 2147483647LL, "%s: too many tiles", who);
  GroupedArgs args{};
  args.proj[0] = ProjArgs{hidden_a, out_a, decoded_a, *pa};
  if (sparse != nullptr) args.proj[0].sparse = *sparse;
  if (pb) args.proj[1] = ProjArgs{hidden_b, out_b, decoded_b, *pb};
  args.expert_ids = expert_ids;
  args.segment_offsets = segment_offsets;
  args.num_segments = num_segments;
  args.row_tile = kGemmRows;
  args.batch = batch;
  dim3 grid(ceil_div(max_n, kTileOut), static_cast<unsigned>(tiles), nproj);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (src == kGmapSparse) {
    hipLaunchKernelGGL((grouped_gemm_kernel<kGmapSparse, 1>), grid, dim3(kGemmThreads), 0, s, args);
  } else if (predecoded) {
    if (pb) {
      hipLaunchKernelGGL((grouped_gemm_kernel<kGmapPredecoded, 2>), grid, dim3(kGemmThreads), 0, s, args);
    } else {
      hipLaunchKernelGGL((grouped_gemm_kernel<kGmapPredecoded, 1>), grid, dim3(kGemmThreads), 0, s, args);
    }
  } else {
    if (pb) {
      hipLaunchKernelGGL((grouped_gemm_kernel<kGmapGr, 2>), grid, dim3(kGemmThreads), 0, s, args);
    } else {
      hipLaunchKernelGGL((grouped_gemm_kernel<kGmapGr, 1>), grid, dim3(kGemmThreads), 0, s, args);
    }
  }
  return check_launch(who);
}

// A non-expert linear (or two sharing the input): the exact kernel over one segment of all rows with each
// payload's single expert, an optional per-column input scale and fp32 addend per projection.
int launch_linear(const uint16_t* input, int batch, const tris_compact3_payload* pa, const tris_compact3_payload* pb,
                  const uint16_t* input_scale, const float* addend, uint16_t* out_a, uint16_t* out_b, void* stream,
                  const char* who) {
  const int nproj = pb ? 2 : 1;
  TRIS_REQUIRE(batch >= 0, "%s: negative batch", who);
  for (int i = 0; i < nproj; ++i) {
    const tris_compact3_payload* p = i ? pb : pa;
    int rc = check_payload(p, true, who);
    if (rc) return rc;
    TRIS_REQUIRE(p->num_experts == 1, "%s: a non-expert payload holds one matrix (num_experts %d)", who,
                 p->num_experts);
    TRIS_REQUIRE(p->q_gmap_gr_offsets != nullptr, "%s: block-GR split bitmaps required", who);
  }
  TRIS_REQUIRE(!pb || pb->rank == pa->rank, "%s: the pair's ranks differ", who);
  if (batch == 0 || pa->rank == 0) return TRIS_OK;
  TRIS_REQUIRE(input && out_a && (!pb || out_b), "%s: null pointer", who);
  int max_n = 0;
  for (int i = 0; i < nproj; ++i) {
    const tris_compact3_payload* p = i ? pb : pa;
    max_n = p->outfeatures > max_n ? p->outfeatures : max_n;
  }
  if (max_n == 0) return TRIS_OK;
  GroupedArgs args{};
  args.proj[0] = ProjArgs{input, out_a, nullptr, *pa, input_scale, addend};
  if (pb) args.proj[1] = ProjArgs{input, out_b, nullptr, *pb, nullptr, nullptr};
  args.segment_offsets = nullptr;
  args.num_segments = 1;
  args.row_tile = kGemmRows;
  args.batch = batch;
  dim3 grid(ceil_div(max_n, kTileOut), ceil_div(batch, kGemmRows), nproj);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pb) {
    hipLaunchKernelGGL((grouped_gemm_kernel<kGmapGr, 2>), grid, dim3(kGemmThreads), 0, s, args);
  } else {
    hipLaunchKernelGGL((grouped_gemm_kernel<kGmapGr, 1>), grid, dim3(kGemmThreads), 0, s, args);
  }
  return check_launch(who);
}

int launch_grouped_mfma(const uint16_t* hidden_a, const uint16_t* hidden_b, int batch, const int32_t* expert_ids,
                        const int32_t* segment_offsets, int num_segments, const int32_t* decoded_a,
                        const int32_t* decoded_b, const tris_compact3_payload* pa, const tris_compact3_payload* pb,
                        uint16_t* out_a, uint16_t* out_b, bool swiglu, void* stream, const char* who,
                        const int64_t* row_index = nullptr, int hidden_rows = 0, bool decoded_by_expert = false,
                        const float* partials = nullptr, int slices = 0, uint16_t* comb_out = nullptr,
                        const int32_t* comb_inv = nullptr, const uint16_t* comb_w = nullptr, bool comb_bf16 = false);
bool grouped_mfma_supported(const tris_compact3_payload* p, const uint16_t* hidden);

}  // namespace tris

using namespace tris;

extern "C" int tris_compact3_linear_forward(const uint16_t* input, int32_t batch, const tris_compact3_payload* payload,
                                            const uint16_t* input_scale, const float* addend, uint16_t* output,
                                            void* stream) {
  return launch_linear(input, batch, payload, nullptr, input_scale, addend, output, nullptr, stream,
                       "tris_compact3_linear_forward");
}

extern "C" int tris_compact3_dual_linear_forward(const uint16_t* input, int32_t batch,
                                                 const tris_compact3_payload* payload_a,
                                                 const tris_compact3_payload* payload_b, uint16_t* output_a,
                                                 uint16_t* output_b, void* stream) {
  return launch_linear(input, batch, payload_a, payload_b, nullptr, nullptr, output_a, output_b, stream,
                       "tris_compact3_dual_linear_forward");
}

extern "C" int tris_grouped_forward_block_gr(const uint16_t* hidden, int32_t batch, const int32_t* expert_ids,
                                             const int32_t* segment_offsets, const int32_t* problem_offsets,
                                             int32_t num_segments, int64_t total_problem_tiles,
                                             const tris_compact3_payload* payload, uint16_t* output, void* stream) {
  (void)problem_offsets;
  return launch_grouped(hidden, nullptr, batch, expert_ids, segment_offsets, num_segments, total_problem_tiles,
                        nullptr, nullptr, payload, nullptr, output, nullptr, kGmapGr, stream,
                        "tris_grouped_forward_block_gr");
}

extern "C" int tris_grouped_forward_sparse(const uint16_t* hidden, int32_t batch, const int32_t* expert_ids,
                                           const int32_t* segment_offsets, const int32_t* problem_offsets,
                                           int32_t num_segments, int64_t total_problem_tiles,
                                           const tris_compact3_payload* payload, const int32_t* q_gmap_sparse,
                                           const int32_t* q_gmap_sparse_prefix, int32_t q_gmap_sparse_rows,
                                           uint16_t* output, void* stream) {
  (void)problem_offsets;
  if (payload == nullptr) {
    set_error("tris_grouped_forward_sparse: null payload");
    return TRIS_ERR_INVALID;
  }
  tris_compact3_payload p = *payload;  // the reference's sparse kernels always apply the output scale
  p.has_output_scale = 1;
  p.q_gmap_gr_words = nullptr;
  p.q_gmap_gr_offsets = nullptr;
  p.q_gmap_gr_meta = nullptr;
  const SparseGmap sg{q_gmap_sparse, q_gmap_sparse_prefix, q_gmap_sparse_rows};
  return launch_grouped(hidden, nullptr, batch, expert_ids, segment_offsets, num_segments, total_problem_tiles,
                        nullptr, nullptr, &p, nullptr, output, nullptr, kGmapSparse, stream,
                        "tris_grouped_forward_sparse", &sg);
}

extern "C" int tris_grouped_dual_forward_block_gr(const uint16_t* hidden_a, const uint16_t* hidden_b, int32_t batch,
                                                  const int32_t* expert_ids, const int32_t* segment_offsets,
                                                  const int32_t* problem_offsets, int32_t num_segments,
                                                  int64_t total_problem_tiles, const tris_compact3_payload* payload_a,
                                                  const tris_compact3_payload* payload_b, uint16_t* output_a,
                                                  uint16_t* output_b, void* stream) {
  (void)problem_offsets;
  TRIS_REQUIRE(payload_b != nullptr, "tris_grouped_dual_forward_block_gr: null payload_b");
  return launch_grouped(hidden_a, hidden_b, batch, expert_ids, segment_offsets, num_segments, total_problem_tiles,
                        nullptr, nullptr, payload_a, payload_b, output_a, output_b, kGmapGr, stream,
                        "tris_grouped_dual_forward_block_gr");
}

extern "C" int tris_grouped_forward_block_gr_predecoded(const uint16_t* hidden, int32_t batch,
                                                        const int32_t* expert_ids, const int32_t* segment_offsets,
                                                        const int32_t* problem_offsets, int32_t num_segments,
                                                        int64_t total_problem_tiles, const int32_t* decoded,
                                                        const tris_compact3_payload* payload, uint16_t* output,
                                                        void* stream) {
  (void)problem_offsets;
  if (payload == nullptr) {
    set_error("tris_grouped_forward_block_gr_predecoded: null payload");
    return TRIS_ERR_INVALID;
  }
  tris_compact3_payload p = *payload;  // the predecoded kernels apply no scale or bias
  p.has_output_scale = 0;
  p.has_bias = 0;
  if (grouped_mfma_supported(&p, hidden)) {
    if (total_problem_tiles <= 0) return TRIS_OK;
    return launch_grouped_mfma(hidden, nullptr, batch, expert_ids, segment_offsets, num_segments, decoded, nullptr,
                               &p, nullptr, output, nullptr, false, stream, "tris_grouped_forward_block_gr_predecoded");
  }
  return launch_grouped(hidden, nullptr, batch, expert_ids, segment_offsets, num_segments, total_problem_tiles,
                        decoded, nullptr, &p, nullptr, output, nullptr, kGmapPredecoded, stream,
                        "tris_grouped_forward_block_gr_predecoded");
}

// The dual predecoded GEMM; row_index (or null) gathers the activation rows from hidden_rows rows.  The
// exact VALU kernel (payloads outside the MFMA kernel's conditions) reads ungathered rows only.
static int dual_predecoded(const uint16_t* hidden_a, const uint16_t* hidden_b, const int64_t* row_index,
                           int32_t hidden_rows, int32_t batch, const int32_t* expert_ids,
                           const int32_t* segment_offsets, int32_t num_segments, int64_t total_problem_tiles,
                           const int32_t* decoded_a, const int32_t* decoded_b, const tris_compact3_payload* payload_a,
                           const tris_compact3_payload* payload_b, uint16_t* output_a, uint16_t* output_b,
                           void* stream, const char* who) {
  if (payload_a == nullptr || payload_b == nullptr) {
    set_error("%s: null payload", who);
    return TRIS_ERR_INVALID;
  }
  tris_compact3_payload pa = *payload_a;
  tris_compact3_payload pb = *payload_b;
  pa.has_output_scale = pb.has_output_scale = 0;
  pa.has_bias = pb.has_bias = 0;
  if (grouped_mfma_supported(&pa, hidden_a) && grouped_mfma_supported(&pb, hidden_b)) {
    if (total_problem_tiles <= 0) return TRIS_OK;
    TRIS_REQUIRE(pa.num_experts == pb.num_experts, "%s: expert count mismatch", who);
    return launch_grouped_mfma(hidden_a, hidden_b, batch, expert_ids, segment_offsets, num_segments, decoded_a,
                               decoded_b, &pa, &pb, output_a, output_b, false, stream, who, row_index, hidden_rows);
  }
  TRIS_REQUIRE(row_index == nullptr, "%s: gathered rows need the MFMA kernel's payload conditions", who);
  return launch_grouped(hidden_a, hidden_b, batch, expert_ids, segment_offsets, num_segments, total_problem_tiles,
                        decoded_a, decoded_b, &pa, &pb, output_a, output_b, kGmapPredecoded, stream, who);
}

static int swiglu_predecoded(const uint16_t* hidden_gate, const uint16_t* hidden_up, const int64_t* row_index,
                             int32_t hidden_rows, int32_t batch, const int32_t* expert_ids,
                             const int32_t* segment_offsets, int32_t num_segments, int64_t total_problem_tiles,
                             const int32_t* decoded_gate, const int32_t* decoded_up,
                             const tris_compact3_payload* payload_gate, const tris_compact3_payload* payload_up,
                             uint16_t* output, void* stream, const char* who) {
  if (payload_gate == nullptr || payload_up == nullptr) {
    set_error("%s: null payload", who);
    return TRIS_ERR_INVALID;
  }
  tris_compact3_payload pg = *payload_gate;
  tris_compact3_payload pu = *payload_up;
  pg.has_output_scale = pu.has_output_scale = 0;
  pg.has_bias = pu.has_bias = 0;
  TRIS_REQUIRE(grouped_mfma_supported(&pg, hidden_gate) && grouped_mfma_supported(&pu, hidden_up),
               "%s: needs uniform 64-column groups, rank %% 64 == 0 and 16-byte aligned hidden rows", who);
  if (total_problem_tiles <= 0) return TRIS_OK;
  return launch_grouped_mfma(hidden_gate, hidden_up, batch, expert_ids, segment_offsets, num_segments, decoded_gate,
                             decoded_up, &pg, &pu, output, nullptr, true, stream, who, row_index, hidden_rows);
}

extern "C" int tris_grouped_dual_forward_block_gr_predecoded(
    const uint16_t* hidden_a, const uint16_t* hidden_b, int32_t batch, const int32_t* expert_ids,
    const int32_t* segment_offsets, const int32_t* problem_offsets, int32_t num_segments, int64_t total_problem_tiles,
    const int32_t* decoded_a, const int32_t* decoded_b, const tris_compact3_payload* payload_a,
    const tris_compact3_payload* payload_b, uint16_t* output_a, uint16_t* output_b, void* stream) {
  (void)problem_offsets;
  return dual_predecoded(hidden_a, hidden_b, nullptr, 0, batch, expert_ids, segment_offsets, num_segments,
                         total_problem_tiles, decoded_a, decoded_b, payload_a, payload_b, output_a, output_b, stream,
                         "tris_grouped_dual_forward_block_gr_predecoded");
}

extern "C" int tris_grouped_dual_forward_block_gr_predecoded_rows(
    const uint16_t* hidden_a, const uint16_t* hidden_b, const int64_t* row_index, int32_t hidden_rows, int32_t batch,
    const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments, int64_t total_problem_tiles,
    const int32_t* decoded_a, const int32_t* decoded_b, const tris_compact3_payload* payload_a,
    const tris_compact3_payload* payload_b, uint16_t* output_a, uint16_t* output_b, void* stream) {
  const char* who = "tris_grouped_dual_forward_block_gr_predecoded_rows";
  TRIS_REQUIRE(row_index != nullptr || batch == 0, "%s: null row_index", who);
  return dual_predecoded(hidden_a, hidden_b, row_index, hidden_rows, batch, expert_ids, segment_offsets, num_segments,
                         total_problem_tiles, decoded_a, decoded_b, payload_a, payload_b, output_a, output_b, stream,
                         who);
}

extern "C" int tris_grouped_swiglu_forward_block_gr_predecoded(
    const uint16_t* hidden_gate, const uint16_t* hidden_up, int32_t batch, const int32_t* expert_ids,
    const int32_t* segment_offsets, const int32_t* problem_offsets, int32_t num_segments, int64_t total_problem_tiles,
    const int32_t* decoded_gate, const int32_t* decoded_up, const tris_compact3_payload* payload_gate,
    const tris_compact3_payload* payload_up, uint16_t* output, void* stream) {
  (void)problem_offsets;
  return swiglu_predecoded(hidden_gate, hidden_up, nullptr, 0, batch, expert_ids, segment_offsets, num_segments,
                           total_problem_tiles, decoded_gate, decoded_up, payload_gate, payload_up, output, stream,
                           "tris_grouped_swiglu_forward_block_gr_predecoded");
}

extern "C" int tris_grouped_swiglu_forward_block_gr_predecoded_rows(
    const uint16_t* hidden_gate, const uint16_t* hidden_up, const int64_t* row_index, int32_t hidden_rows,
    int32_t batch, const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments,
    int64_t total_problem_tiles, const int32_t* decoded_gate, const int32_t* decoded_up,
    const tris_compact3_payload* payload_gate, const tris_compact3_payload* payload_up, uint16_t* output,
    void* stream) {
  const char* who = "tris_grouped_swiglu_forward_block_gr_predecoded_rows";
  TRIS_REQUIRE(row_index != nullptr || batch == 0, "%s: null row_index", who);
  return swiglu_predecoded(hidden_gate, hidden_up, row_index, hidden_rows, batch, expert_ids, segment_offsets,
                           num_segments, total_problem_tiles, decoded_gate, decoded_up, payload_gate, payload_up,
                           output, stream, who);
}

extern "C" int tris_grouped_forward_block_gr_predecoded_experts(
    const uint16_t* hidden_a, const uint16_t* hidden_b, const int64_t* row_index, int32_t hidden_rows, int32_t batch,
    const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments, int64_t total_problem_tiles,
    const int32_t* decoded_a, const int32_t* decoded_b, const tris_compact3_payload* payload_a,
    const tris_compact3_payload* payload_b, uint16_t* output_a, uint16_t* output_b, void* stream) {
  const char* who = "tris_grouped_forward_block_gr_predecoded_experts";
  TRIS_REQUIRE(payload_a != nullptr, "%s: null payload", who);
  TRIS_REQUIRE((payload_b == nullptr) == (hidden_b == nullptr), "%s: hidden_b and payload_b go together", who);
  tris_compact3_payload pa = *payload_a;
  tris_compact3_payload pb = payload_b != nullptr ? *payload_b : tris_compact3_payload{};
  pa.has_output_scale = pb.has_output_scale = 0;
  pa.has_bias = pb.has_bias = 0;
  TRIS_REQUIRE(grouped_mfma_supported(&pa, hidden_a) && (payload_b == nullptr || grouped_mfma_supported(&pb, hidden_b)),
               "%s: needs uniform 64-column groups, rank %% 64 == 0 and 16-byte aligned hidden rows", who);
  TRIS_REQUIRE(payload_b == nullptr || pa.num_experts == pb.num_experts, "%s: expert count mismatch", who);
  if (total_problem_tiles <= 0) return TRIS_OK;
  return launch_grouped_mfma(hidden_a, payload_b ? hidden_b : nullptr, batch, expert_ids, segment_offsets, num_segments,
                             decoded_a, payload_b ? decoded_b : nullptr, &pa, payload_b ? &pb : nullptr, output_a,
                             payload_b ? output_b : nullptr, false, stream, who, row_index, hidden_rows, true);
}

extern "C" int tris_grouped_forward_block_gr_predecoded_partials(
    const float* partials, int32_t slices, int32_t batch, const int32_t* expert_ids, const int32_t* segment_offsets,
    int32_t num_segments, int64_t total_problem_tiles, const int32_t* decoded, const tris_compact3_payload* payload,
    uint16_t* output, int32_t decoded_by_expert, void* stream) {
  const char* who = "tris_grouped_forward_block_gr_predecoded_partials";
  TRIS_REQUIRE(payload != nullptr && partials != nullptr, "%s: null payload or partial sums", who);
  TRIS_REQUIRE(batch >= 0 && slices >= 1, "%s: negative batch or no slices", who);
  tris_compact3_payload p = *payload;  // the predecoded kernels apply no scale or bias
  p.has_output_scale = 0;
  p.has_bias = 0;
  TRIS_REQUIRE(grouped_mfma_supported(&p, reinterpret_cast<const uint16_t*>(partials)),
               "%s: needs uniform 64-column groups, rank %% 64 == 0 and 16-byte aligned partial sums", who);
  if (total_problem_tiles <= 0 || batch == 0) return TRIS_OK;
  return launch_grouped_mfma(nullptr, nullptr, batch, expert_ids, segment_offsets, num_segments, decoded, nullptr, &p,
                             nullptr, output, nullptr, false, stream, who, nullptr, batch, decoded_by_expert != 0,
                             partials, slices);
}

extern "C" int tris_grouped_forward_block_gr_predecoded_partials_combine(
    const float* partials, int32_t slices, const int32_t* expert_ids, const int32_t* segment_offsets,
    int64_t total_problem_tiles, const int32_t* decoded, const tris_compact3_payload* payload,
    const int32_t* inverse_perm, const uint16_t* routing_weights_f16, int32_t out_bf16, uint16_t* out,
    int32_t decoded_by_expert, void* stream) {
  const char* who = "tris_grouped_forward_block_gr_predecoded_partials_combine";
  TRIS_REQUIRE(payload != nullptr && partials != nullptr && out != nullptr, "%s: null payload, partial sums or output",
               who);
  TRIS_REQUIRE(slices >= 1, "%s: no slices", who);
  tris_compact3_payload p = *payload;  // the predecoded kernels apply no scale or bias
  p.has_output_scale = 0;
  p.has_bias = 0;
  TRIS_REQUIRE(grouped_mfma_supported(&p, reinterpret_cast<const uint16_t*>(partials)),
               "%s: needs uniform 64-column groups, rank %% 64 == 0 and 16-byte aligned partial sums", who);
  if (total_problem_tiles <= 0) return TRIS_OK;
  return launch_grouped_mfma(nullptr, nullptr, 2, expert_ids, segment_offsets, 2, decoded, nullptr, &p, nullptr, out,
                             nullptr, false, stream, who, nullptr, 2, decoded_by_expert != 0, partials, slices, out,
                             inverse_perm, routing_weights_f16, out_bf16 != 0);
}

extern "C" int tris_compact3_dequant(const tris_compact3_payload* payload, const int32_t* expert_ids, int32_t num,
                                     uint16_t* weights, void* stream) {
  int rc = check_payload(payload, true, "tris_compact3_dequant");
  if (rc) return rc;
  TRIS_REQUIRE(num >= 0, "tris_compact3_dequant: negative count");
  if (num == 0 || payload->rank == 0 || payload->outfeatures == 0) return TRIS_OK;
  TRIS_REQUIRE(weights && expert_ids, "tris_compact3_dequant: null pointer");
  TRIS_REQUIRE(num <= 65535, "tris_compact3_dequant: too many experts");
  const int packed_rows = ceil_div(payload->rank, 32);
  dim3 grid(ceil_div(payload->outfeatures, kTileOut), ceil_div(packed_rows, kGrPackedRows), num);
  hipLaunchKernelGGL(compact3_dequant_kernel, grid, dim3(kWave), 0, static_cast<hipStream_t>(stream), *payload,
                     expert_ids, weights);
  return check_launch("compact3_dequant_kernel");
}
