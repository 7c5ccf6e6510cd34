// Grouped compact3 expert GEMM on MFMA for decode-sized segments, reading
// dense (predecoded) split bitmaps.
//
// Arithmetic.  Every non-salient weight is the reference's exact fp16 value
// w[n,k] = s1 * fp16(C_j[k] * R_j[n,g]) with j = d if the split bit is set,
// else nd, and s1 = +-1 from qweight1 (TriSMoE_cuda_kernel.cu:665-774); the
// products are formed with packed fp16 multiplies (round to nearest even, as
// __hmul).  The choice of j and the sign come from the bit planes as two
// selector pairs sd, sn in {0, +1, -1}: w = fma(sd, P_d, sn * P_nd), exact
// because one of the two terms is zero.  Salient columns (a few per cent,
// w = fp16(+-fp16(C0*R0) +- fp16(C1*R1))) are zero in that operand and get
// their own MFMA pass over an LDS table of their exact weights.  Products with the activations are
// exact in fp32 and accumulate in fp32, as in the reference's tensor-core
// kernel (TriSMoE_cuda_kernel.cu:4889-5093).
//
// Operand layout (v_mfma_f32_16x16x32_f16): A rows are up to 16 rows of one
// segment; lane group kg (lanes 16kg..16kg+15) supplies the 8 columns
// k = kg + 4i (i = 0..7) of each 32-column packed row, so after one shift the
// sign / split / salient bits of those columns sit at nibble positions 4i of a
// word.  OR-ing in the fp4 (e2m1) exponent pattern gives eight fp4 selectors
// (+-1.0 = 0b0010 / 0b1010, 0 = 0b0000) that v_cvt_scalef32_pk_f16_fp4
// expands two at a time to fp16 pairs.  Activations and the column factors are
// staged in LDS in the same permuted column order, so each lane reads its 8
// values with one 16-byte LDS load.
//
// Work decomposition: workgroup = 4 wavefronts = one 64-output tile x one
// tile of <= 16 rows of one segment x one projection (blockIdx.z).  The
// workgroup stages the rows' activations and the column factors of a 512-column
// chunk in LDS once; wavefront w then owns outputs [16w, 16w+16) over the whole
// chunk, issuing its weight loads (one column per lane, 16 packed rows) before
// computing, so no partial sums cross wavefronts.  Salient columns are zero in
// that pass; afterwards each lane writes the exact salient weights of its
// column (lane group kg takes the salient columns k = kg (mod 4)) into an LDS
// table, and one or two more MFMA steps multiply the activations gathered at
// the salient columns by it, into the same fp32 accumulator.  Requires each
// 64-column K tile to lie in a single group (the reference's UniformK64Groups
// case) and rank % 64 == 0.
#include "tris_common.h"

namespace tris {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfWaves = 4;
constexpr int kMfThreads = kMfWaves * kWave;
constexpr int kMfRows = 16;         // segment rows per workgroup tile
constexpr int kMfChunk = 512;       // K columns staged per pass
constexpr int kMfXStride = kMfChunk + 8;  // fp16 elements per staged row (pad breaks bank aliasing)
constexpr int kMfSalWin = 64;             // salient columns per MFMA pass
constexpr int kMfSalStride = kMfSalWin + 8;

struct MfmaProj {
  const uint16_t* hidden;  // [batch, rank]
  uint16_t* out;           // [batch, N]
  const int32_t* decoded;  // [num_segments, nblk, 128]
  tris_compact3_payload p;
};

struct MfmaArgs {
  MfmaProj proj[2];
  const int32_t* expert_ids;
  const int32_t* segment_offsets;
  int num_segments;
};

// Position of column k (0..31) of a packed row in the staged order: lane group
// k % 4, element k / 4.
__device__ __forceinline__ int mf_perm32(int k) { return 8 * (k & 3) + (k >> 2); }

// Nibbles 2i, 2i+1 (byte i) of eight fp4 values -> two fp16 (low nibble -> low half).
__device__ __forceinline__ f16x2 fp4x2_to_f16x2(uint32_t nib, int byte_sel) {
  switch (byte_sel) {
    case 0: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(nib, 1.0f, 0);
    case 1: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(nib, 1.0f, 1);
    case 2: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(nib, 1.0f, 2);
    default: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(nib, 1.0f, 3);
  }
}

__device__ __forceinline__ f16x2 u32_as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t f16x2_as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Same mapping as the in-kernel-decode GEMM (tris_grouped.hip).
__device__ inline bool mf_map_row_tile(const int32_t* __restrict__ seg, int nseg, int tile, int row_tile, int* s_out,
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

// LDS of one workgroup, shared by the projections it computes one after the other.
struct MfmaLds {
  uint16_t (*xs)[kMfXStride];          // activations, staged order
  uint16_t* cds;                        // C_d, staged order
  uint16_t* cns;                        // C_nd, staged order
  uint32_t* col_sal;                    // C0 | C1 << 16, natural order
  uint16_t* sal_col;                    // chunk column of the chunk's q-th salient column
  uint16_t (*ws)[16][kMfSalStride];    // per-wave salient weights
  uint32_t (*q1l)[kTileOut];           // qweight1 words of the tile's columns, per chunk packed row
  uint32_t (*r01)[kTileOut];           // R0 | R1 << 16 of the tile's columns, per chunk 64-column tile
};

constexpr uint32_t kBufferWord3 = 0x00020000;  // raw buffer resource, gfx9 family

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferWord3);
}
// Raw buffer loads: voffset at or past the buffer size returns 0 without a memory access.
__device__ __forceinline__ uint32_t bload32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ uint64_t bload64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
  return static_cast<uint64_t>(v[0]) | (static_cast<uint64_t>(v[1]) << 32);
}
__device__ __forceinline__ uint4 bload128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// One projection of one workgroup tile: rows [row0, row0 + rc) of segment s
// (expert e) x output columns [n0, n0 + 64).  Returns the lane's accumulator:
// rows 4*kg + v, column n0 + 16*wave + lane % 16.  Per-expert tensors are read
// through raw buffer resources (uniform base, 32-bit lane offsets; element
// offsets fit in 32 bits, which the host checks).
__device__ __forceinline__ f32x4 mfma_project(const MfmaProj& pa, int s, int row0, int rc, int e, int n0,
                                              const MfmaLds& L) {
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  uint16_t (*xs)[kMfXStride] = L.xs;
  uint16_t* cds = L.cds;
  uint16_t* cns = L.cns;
  uint32_t* col_sal = L.col_sal;
  uint16_t* sal_col = L.sal_col;
  uint16_t (*ws)[16][kMfSalStride] = L.ws;
  const int rank = p.rank;
  const int packed_rows = ceil_div(rank, 32);
  const int nkb = ceil_div(packed_rows, kGrPackedRows);
  const int nob = ceil_div(N, kTileOut);
  const int nblk = nkb * nob;
  const int ob = blockIdx.x;
  const int G = p.num_groups;
  const int32_t* q2p_e = p.qweight2_sparse_prefix + static_cast<int64_t>(e) * (packed_rows + 1);
  const int32_t* cmap_e = p.c_map + static_cast<int64_t>(e) * packed_rows;
  const int32_t* gidx_e = p.g_idx + static_cast<int64_t>(e) * rank;
  const uint32_t q1_bytes = static_cast<uint32_t>(packed_rows) * N * 4u;
  const uint32_t dec_bytes = static_cast<uint32_t>(nblk) * kGrWords * 4u;
  const uint32_t row_bytes = static_cast<uint32_t>(N) * G * 8u;
  const uint32_t q2_bytes = static_cast<uint32_t>(p.qweight2_sparse_rows) * N * 4u;
  const uint32_t col_bytes = static_cast<uint32_t>(rank) * 8u;
  const uint32_t hid_bytes = static_cast<uint32_t>(rc) * rank * 2u;
  const __amdgpu_buffer_rsrc_t r_q1 = make_rsrc(p.qweight1 + static_cast<int64_t>(e) * packed_rows * N, q1_bytes);
  const __amdgpu_buffer_rsrc_t r_dec = make_rsrc(pa.decoded + static_cast<int64_t>(s) * nblk * kGrWords, dec_bytes);
  const __amdgpu_buffer_rsrc_t r_row = make_rsrc(p.row_pack3 + static_cast<int64_t>(e) * N * G, row_bytes);
  const __amdgpu_buffer_rsrc_t r_q2 =
      make_rsrc(p.qweight2_sparse + static_cast<int64_t>(e) * p.qweight2_sparse_rows * N, q2_bytes);
  const __amdgpu_buffer_rsrc_t r_col = make_rsrc(p.col_pack3 + static_cast<int64_t>(e) * rank, col_bytes);
  const __amdgpu_buffer_rsrc_t r_hid = make_rsrc(pa.hidden + static_cast<int64_t>(row0) * rank, hid_bytes);

  const int i16 = lane % 16;   // MFMA column within the wave's 16 outputs / A row
  const int kg = lane / 16;    // MFMA k group: columns k = kg (mod 4) of every packed row
  const int tc = 16 * wave + i16;      // column within the tile
  const int n = n0 + tc;               // this lane's output column
  const bool nv = n < N;
  // lane offsets; an invalid column reads past its buffer, which returns 0
  const uint32_t v_q1 = nv ? static_cast<uint32_t>(n) * 4u : q1_bytes;
  const uint32_t v_dec = nv ? static_cast<uint32_t>(tc) * 4u : dec_bytes;
  const uint32_t v_row = nv ? static_cast<uint32_t>(n) * G * 8u : row_bytes;
  const uint32_t v_q2 = nv ? static_cast<uint32_t>(n) * 4u : q2_bytes;
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int kc = 0; kc < rank; kc += kMfChunk) {
    const int pr0 = kc / 32;
    const int npr = (packed_rows - pr0) < kMfChunk / 32 ? (packed_rows - pr0) : kMfChunk / 32;  // even
    const int pr_end = pr0 + npr;
    // ---- batch 1: the chunk's uniform metadata (group of each 64-column tile, salient words and
    // prefix per packed row), then the lane's weights, which do not depend on it.  Indices are
    // clamped so that every load is issued unconditionally; validity is applied afterwards.
    int gt[kMfChunk / kTileK];
    uint32_t cmw[kMfChunk / 32];
#pragma unroll
    for (int t = 0; t < kMfChunk / kTileK; ++t) {
      const int kt = kc + t * kTileK;
      gt[t] = gidx_e[kt < rank ? kt : rank - 1];
    }
#pragma unroll
    for (int j = 0; j < kMfChunk / 32; ++j) {
      cmw[j] = static_cast<uint32_t>(cmap_e[j < npr ? pr0 + j : packed_rows - 1]);
    }
    const int q2_first = q2p_e[pr0];
    const int q2_end = q2p_e[pr_end];
    // every load below is issued unconditionally (a branch around a load makes the compiler wait
    // for it at the join): an invalid row or group gets a lane offset past the buffer, which
    // reads 0, and an in-range uniform offset
    uint32_t qw[kMfChunk / 32], gw[kMfChunk / 32];
#pragma unroll
    for (int j = 0; j < kMfChunk / 32; ++j) {
      const bool jv = j < npr;  // uniform
      const uint32_t pr = static_cast<uint32_t>(jv ? pr0 + j : 0);
      qw[j] = bload32(r_q1, jv ? v_q1 : q1_bytes, pr * N * 4u);
      gw[j] = bload32(r_dec, jv ? v_dec : dec_bytes,
                      ((static_cast<uint32_t>(pr >> 1) * nob + ob) * kGrWords + (pr & 1u) * kTileOut) * 4u);
    }
#pragma unroll
    for (int t = 0; t < kMfChunk / kTileK; ++t) {
      // an invalid tile's group is made negative (uses the loaded value on every path, so the
      // compiler does not move its load behind the weight loads)
      gt[t] = __builtin_amdgcn_readfirstlane(gt[t] | ((kc + t * kTileK) < rank ? 0 : INT32_MIN));
    }
#pragma unroll
    for (int j = 0; j < kMfChunk / 32; ++j) {
      const int pr = pr0 + j;
      const int nbits = (rank - pr * 32) < 32 ? (rank - pr * 32) : 32;
      // uniform; readfirstlane keeps the load where it was issued
      cmw[j] = __builtin_amdgcn_readfirstlane(cmw[j]) & (j < npr ? low_mask(nbits) : 0u);
    }
    // ---- batch 2: row scales of each tile's group
    uint64_t rp[kMfChunk / kTileK];
#pragma unroll
    for (int t = 0; t < kMfChunk / kTileK; ++t) {
      const int g = gt[t];
      const bool gv = g >= 0 && g < G;
      rp[t] = bload64(r_row, gv ? v_row : row_bytes, static_cast<uint32_t>(gv ? g : 0) * 8u);
    }
    const int sbase0 = __builtin_amdgcn_readfirstlane(q2_first);  // qweight2_sparse index of the first salient column
    const int num_sal = __builtin_amdgcn_readfirstlane(q2_end) - sbase0;  // salient columns in the chunk
    // the first two qweight2_sparse rows of the chunk's salient columns (one window of salient
    // columns spans at most three)
    const int q2rows = p.qweight2_sparse_rows;
    const int q2row0 = sbase0 >> 5;
    uint32_t q2w01[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool rv = num_sal > 32 * h && q2row0 + h < q2rows;
      q2w01[h] = bload32(r_q2, rv ? v_q2 : q2_bytes, static_cast<uint32_t>(rv ? q2row0 + h : 0) * N * 4u);
    }
    // staging loads: activation runs (row idx / 64, 8-column run idx % 64; rank is a multiple
    // of 64, so a run is wholly inside or outside the matrix; rows >= rc read past the buffer)
    // and, for columns kc + tid and kc + tid + 256, the column factors, salient word and prefix
    constexpr int kRuns = kMfRows * (kMfChunk / 8) / kMfThreads;
    uint4 xv[kRuns];
#pragma unroll
    for (int h = 0; h < kRuns; ++h) {
      const int idx = tid + h * kMfThreads;
      const int r = idx / (kMfChunk / 8);
      const int c = (idx % (kMfChunk / 8)) * 8;
      const uint32_t voff = (kc + c < rank) ? static_cast<uint32_t>(r * rank + kc + c) * 2u : hid_bytes;
      xv[h] = bload128(r_hid, voff, 0u);
    }
    uint64_t cpv[2];
    uint32_t cmt[2];
    int q2t[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = kc + tid + h * kMfThreads;
      const bool kv = k < rank;
      const int pr = kv ? (k >> 5) : 0;
      cpv[h] = bload64(r_col, kv ? static_cast<uint32_t>(k) * 8u : col_bytes, 0u);
      cmt[h] = static_cast<uint32_t>(cmap_e[pr]);
      q2t[h] = q2p_e[pr];
    }
    __syncthreads();  // previous chunk's LDS readers are done
#pragma unroll
    for (int h = 0; h < kRuns; ++h) {
      const int idx = tid + h * kMfThreads;
      const int r = idx / (kMfChunk / 8);
      const int c = (idx % (kMfChunk / 8)) * 8;  // run start within the chunk (a multiple of 8)
      // columns c + b and c + b + 4 (b < 4) are neighbours in the staged order
      const uint32_t w[4] = {xv[h].x, xv[h].y, xv[h].z, xv[h].w};
      const int base = (c & ~31) + ((c & 31) >> 2);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t lo = (w[b >> 1] >> (16 * (b & 1))) & 0xFFFFu;
        const uint32_t hi = (w[2 + (b >> 1)] >> (16 * (b & 1))) & 0xFFFFu;
        *reinterpret_cast<uint32_t*>(&xs[r][base + 8 * b]) = lo | (hi << 16);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = tid + h * kMfThreads;
      const int k = kc + j;
      const int pj = (j & ~31) + mf_perm32(j & 31);
      cds[pj] = static_cast<uint16_t>(cpv[h] >> 32);
      cns[pj] = static_cast<uint16_t>(cpv[h] >> 48);
      col_sal[j] = static_cast<uint32_t>(cpv[h]);
      if (k < rank) {
        const int bit = k & 31;
        const int pr = k >> 5;
        const int nbits = (rank - pr * 32) < 32 ? (rank - pr * 32) : 32;
        const uint32_t cm = cmt[h] & low_mask(nbits);
        if ((cm >> bit) & 1u) sal_col[q2t[h] - sbase0 + __popc(cm & ((1u << bit) - 1u))] = static_cast<uint16_t>(j);
      }
    }
    // the lane's sign words and R0 | R1, for the salient pass (lane group kg writes every 4th)
    if (num_sal > 0) {
#pragma unroll
      for (int j = 0; j < kMfChunk / 32; j += 4) L.q1l[j + kg][tc] = qw[j + kg];
#pragma unroll
      for (int t = 0; t < kMfChunk / kTileK; t += 4) L.r01[t + kg][tc] = static_cast<uint32_t>(rp[t + kg]);
    }
    __syncthreads();

    // ---- MFMA over the chunk's packed rows (salient columns are zero here)
#pragma unroll
    for (int j = 0; j < kMfChunk / 32; ++j) {
      if (j < npr) {
        const int t = j / 2;
        const uint32_t d = static_cast<uint32_t>(rp[t] >> 32) & 0xFFFFu;
        const uint32_t nd = static_cast<uint32_t>(rp[t] >> 48);
        const f16x2 rd2 = u32_as_f16x2(d | (d << 16));
        const f16x2 rn2 = u32_as_f16x2(nd | (nd << 16));
        const int kl = j * 32 + 8 * kg;
        const f16x8 av = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&xs[i16][kl]));
        const uint4 cdv = *reinterpret_cast<const uint4*>(&cds[kl]);
        const uint4 cnv = *reinterpret_cast<const uint4*>(&cns[kl]);
        const uint32_t cd[4] = {cdv.x, cdv.y, cdv.z, cdv.w};
        const uint32_t cn[4] = {cnv.x, cnv.y, cnv.z, cnv.w};
        const uint32_t nsal = (~cmw[j] >> kg) & 0x11111111u;                       // 1 = non-salient
        const uint32_t neg = ((~qw[j]) >> kg) & 0x11111111u;                         // 1 = negative
        const uint32_t gd = (gw[j] >> kg) & nsal;                                    // 1 = d term
        const uint32_t gn = nsal ^ gd;                                               // 1 = nd term
        const uint32_t sd = (gd << 1) | ((gd & neg) << 3);                           // fp4 +-1.0 / 0
        const uint32_t sn = (gn << 1) | ((gn & neg) << 3);
        uint32_t b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f16x2 pd = u32_as_f16x2(cd[i]) * rd2;
          const f16x2 pn = u32_as_f16x2(cn[i]) * rn2;
          const f16x2 tn = fp4x2_to_f16x2(sn, i) * pn;
          b[i] = f16x2_as_u32(__builtin_elementwise_fma(fp4x2_to_f16x2(sd, i), pd, tn));
        }
        const f16x8 bv = __builtin_bit_cast(f16x8, make_uint4(b[0], b[1], b[2], b[3]));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
      }
    }

    // ---- salient columns, kMfSalWin at a time.  Lane group kg writes the exact fp16 weights of
    // its column for window slots kg, kg + 4, ... into ws (sign word and R0 | R1 from LDS), then
    // the wave multiplies the activations gathered at those columns by ws on MFMA.
    for (int w0 = 0; w0 < num_sal; w0 += kMfSalWin) {
      const int wn = (num_sal - w0) < kMfSalWin ? (num_sal - w0) : kMfSalWin;
#pragma unroll
      for (int i = 0; i < kMfSalWin / 4; ++i) {
        const int q = 4 * i + kg;
        uint16_t w = 0;
        if (q < wn) {
          const int c = sal_col[w0 + q];  // chunk column
          const int bit = c & 31;
          const uint32_t w1 = L.q1l[c >> 5][tc];
          const uint32_t rr = L.r01[c >> 6][tc];
          const uint32_t cp = col_sal[c];
          const int sidx = sbase0 + w0 + q;  // qweight2_sparse index
          const int q2r = (sidx >> 5) - q2row0;
          uint32_t q2w = q2r == 0 ? q2w01[0] : q2w01[1];
          if (q2r > 1) q2w = bload32(r_q2, v_q2, static_cast<uint32_t>(sidx >> 5) * N * 4u);
          uint16_t t1 = hmul_bits(static_cast<uint16_t>(cp), static_cast<uint16_t>(rr));
          if (!((w1 >> bit) & 1u)) t1 ^= 0x8000u;
          uint16_t t2 = hmul_bits(static_cast<uint16_t>(cp >> 16), static_cast<uint16_t>(rr >> 16));
          if (!((q2w >> (sidx & 31)) & 1u)) t2 ^= 0x8000u;
          w = hadd_bits(t1, t2);
        }
        ws[wave][i16][q] = w;
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int blk = 0; blk < kMfSalWin; blk += 32) {
        if (blk < wn) {
          uint32_t ap[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int q0 = blk + 8 * kg + 2 * i;
            uint32_t lo = 0u, hi = 0u;
            if (q0 < wn) {
              const int c = sal_col[w0 + q0];
              lo = xs[i16][(c & ~31) + mf_perm32(c & 31)];
            }
            if (q0 + 1 < wn) {
              const int c = sal_col[w0 + q0 + 1];
              hi = xs[i16][(c & ~31) + mf_perm32(c & 31)];
            }
            ap[i] = lo | (hi << 16);
          }
          const f16x8 av = __builtin_bit_cast(f16x8, make_uint4(ap[0], ap[1], ap[2], ap[3]));
          const f16x8 bv = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&ws[wave][i16][blk + 8 * kg]));
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
  }
  return acc;
}

// kMode 0: one projection; 1: two projections, blockIdx.z picks one; 2: both
// projections per workgroup (gate, up) and the output is fp16(silu(g) * u).
template <int kMode>
__global__ __launch_bounds__(kMfThreads) void grouped_mfma_kernel(MfmaArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kMfRows][kMfXStride];
  __shared__ __attribute__((aligned(16))) uint16_t cds[kMfChunk];
  __shared__ __attribute__((aligned(16))) uint16_t cns[kMfChunk];
  __shared__ uint32_t col_sal[kMfChunk];
  __shared__ uint16_t sal_col[kMfChunk];
  __shared__ __attribute__((aligned(16))) uint16_t ws[kMfWaves][16][kMfSalStride];
  __shared__ uint32_t q1l[kMfChunk / 32][kTileOut];
  __shared__ uint32_t r01[kMfChunk / kTileK][kTileOut];
  const MfmaLds L{xs, cds, cns, col_sal, sal_col, ws, q1l, r01};

  const MfmaProj& pa = a.proj[kMode == 1 ? blockIdx.z : 0];
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int n0 = blockIdx.x * kTileOut;
  if (n0 >= N) return;
  int s = 0, row0 = 0, rc = 0;
  if (!mf_map_row_tile(a.segment_offsets, a.num_segments, blockIdx.y, kMfRows, &s, &row0, &rc)) return;
  s = __builtin_amdgcn_readfirstlane(s);  // the mapping is the same in every lane
  row0 = __builtin_amdgcn_readfirstlane(row0);
  rc = __builtin_amdgcn_readfirstlane(rc);

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int e = __builtin_amdgcn_readfirstlane(a.expert_ids[s]);
  uint16_t* out = pa.out;
  if (e < 0 || e >= p.num_experts) {
    for (int idx = tid; idx < rc * kTileOut; idx += kMfThreads) {
      const int n = n0 + idx % kTileOut;
      if (n < N) out[static_cast<int64_t>(row0 + idx / kTileOut) * N + n] = 0;
    }
    return;
  }
  const f32x4 acc = mfma_project(pa, s, row0, rc, e, n0, L);
  f32x4 acc_up = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (kMode == 2) acc_up = mfma_project(a.proj[1], s, row0, rc, e, n0, L);

  const int kg = lane / 16;
  const int n = n0 + 16 * (tid / kWave) + lane % 16;
  const bool nv = n < N;
  const float scale = (nv && p.has_output_scale) ? h2f(p.output_scale[static_cast<int64_t>(e) * N + n]) : 1.0f;
  const float bias = (nv && p.has_bias) ? h2f(p.bias[static_cast<int64_t>(e) * N + n]) : 0.0f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * kg + v;
    if (!nv || r >= rc) continue;
    uint16_t y;
    if (kMode == 2) {
      // g and u rounded to fp16 as the two outputs would be, SiLU in fp32 rounded to fp16, then the
      // fp16 product (modeling_mixtral.py:496)
      const float g = h2f(f2h_bits(acc[v]));
      const float u = h2f(f2h_bits(acc_up[v]));
      const float sg = h2f(f2h_bits(g / (1.0f + expf(-g))));
      y = f2h_bits(sg * u);
    } else {
      float x = acc[v];
      if (p.has_output_scale) x = x * scale;
      if (p.has_bias) x = x + bias;
      y = f2h_bits(x);
    }
    out[static_cast<int64_t>(row0 + r) * N + n] = y;
  }
}

int check_payload(const tris_compact3_payload* p, bool need_gr, const char* who);

int launch_grouped_mfma(const uint16_t* hidden_a, const uint16_t* hidden_b, int batch, const int32_t* expert_ids,
                        const int32_t* segment_offsets, int num_segments, const int32_t* decoded_a,
                        const int32_t* decoded_b, const tris_compact3_payload* pa, const tris_compact3_payload* pb,
                        uint16_t* out_a, uint16_t* out_b, bool swiglu, void* stream, const char* who) {
  TRIS_REQUIRE(batch >= 0 && num_segments >= 0, "%s: negative batch or segment count", who);
  int rc = check_payload(pa, false, who);
  if (rc) return rc;
  if (pb) {
    rc = check_payload(pb, false, who);
    if (rc) return rc;
  }
  TRIS_REQUIRE(!swiglu || pb != nullptr, "%s: the fused SwiGLU needs two projections", who);
  if (batch == 0 || num_segments == 0) return TRIS_OK;
  TRIS_REQUIRE(hidden_a && out_a && expert_ids && segment_offsets && decoded_a, "%s: null pointer", who);
  TRIS_REQUIRE(!pb || (hidden_b && decoded_b && (swiglu || out_b)), "%s: null pointer (second projection)", who);
  int max_n = 0;
  for (int i = 0; i < (pb ? 2 : 1); ++i) {
    const tris_compact3_payload* p = i ? pb : pa;
    TRIS_REQUIRE(p->num_experts > 0 && p->rank > 0 && p->outfeatures > 0, "%s: empty payload", who);
    max_n = p->outfeatures > max_n ? p->outfeatures : max_n;
  }
  TRIS_REQUIRE(!swiglu || (pa->outfeatures == pb->outfeatures && pa->num_experts == pb->num_experts),
               "%s: gate and up projections differ in shape", who);
  const int64_t tiles = static_cast<int64_t>(batch) / kMfRows + num_segments;
  TRIS_REQUIRE(tiles <= 2147483647LL, "%s: too many tiles", who);
  MfmaArgs args{};
  args.proj[0] = MfmaProj{hidden_a, out_a, decoded_a, *pa};
  if (pb) args.proj[1] = MfmaProj{hidden_b, out_b, decoded_b, *pb};
  args.expert_ids = expert_ids;
  args.segment_offsets = segment_offsets;
  args.num_segments = num_segments;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (swiglu) {
    const dim3 grid(ceil_div(max_n, kTileOut), static_cast<unsigned>(tiles), 1);
    hipLaunchKernelGGL((grouped_mfma_kernel<2>), grid, dim3(kMfThreads), 0, s, args);
  } else if (pb) {
    const dim3 grid(ceil_div(max_n, kTileOut), static_cast<unsigned>(tiles), 2);
    hipLaunchKernelGGL((grouped_mfma_kernel<1>), grid, dim3(kMfThreads), 0, s, args);
  } else {
    const dim3 grid(ceil_div(max_n, kTileOut), static_cast<unsigned>(tiles), 1);
    hipLaunchKernelGGL((grouped_mfma_kernel<0>), grid, dim3(kMfThreads), 0, s, args);
  }
  return check_launch(who);
}

// True when the MFMA kernel can run this payload: uniform 64-column groups (so
// a 64-column K tile has one row scale) and a rank that is a whole number of
// 64-column tiles, with 16-byte aligned activations (8-column loads).
bool grouped_mfma_supported(const tris_compact3_payload* p, const uint16_t* hidden) {
  if (p == nullptr || !p->use_uniform_k64_groups || p->rank <= 0 || p->rank % kTileK != 0 ||
      reinterpret_cast<uintptr_t>(hidden) % 16 != 0) {
    return false;
  }
  // the kernel addresses each expert's tensors with 32-bit buffer offsets
  const int64_t limit = int64_t{1} << 31;
  const int64_t packed_rows = (p->rank + 31) / 32;
  const int64_t n = p->outfeatures;
  return packed_rows * n * 4 < limit && int64_t{p->qweight2_sparse_rows} * n * 4 < limit &&
         n * p->num_groups * 8 < limit && int64_t{kMfRows} * p->rank * 2 < limit &&
         ((packed_rows + 1) / 2) * ((n + kTileOut - 1) / kTileOut) * kGrWords * 4 < limit;
}

}  // namespace tris
