// Grouped compact3 expert GEMM on MFMA for decode-sized segments, reading
// dense (predecoded) split bitmaps.
//
// Arithmetic.  Every non-salient weight is the reference's exact fp16 value
// w[n,k] = s1 * fp16(C_j[k] * R_j[n,g]) with j = d if the split bit is set,
// else nd, and s1 = +-1 from qweight1 (TriSMoE_cuda_kernel.cu:665-774); the
// products are formed with packed fp16 multiplies (round to nearest even, as
// __hmul) on column factors staged negated (P_j = fp16(-C_j * R_j) = -fp16(C_j * R_j)
// exactly).  The choice of j and the sign come from the bit planes as two
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
constexpr int kMfSalWin = 32;             // salient columns per MFMA pass
constexpr int kMfSalStride = kMfSalWin + 8;

struct MfmaProj {
  const uint16_t* hidden;     // [batch, rank], or [hidden_rows, rank] read through row_index
  uint16_t* out;              // [batch, N]
  const int32_t* decoded;     // [num_segments, nblk, 128]
  tris_compact3_payload p;
  const int64_t* row_index;   // null, or [batch]: segment row r reads hidden row row_index[r]
  int hidden_rows;            // row_index's range, or with partials the rows of each slice
  // null, or [slices][hidden_rows][rank] fp32 split-K partial sums of the backbone that produced the activations:
  // hidden row r is then fp16(the slices' sum, added in slice order) and `hidden` is not read (rank <= kMfChunk)
  const float* partials;
  int slices;
};

struct MfmaArgs {
  MfmaProj proj[2];
  const int32_t* expert_ids;
  const int32_t* segment_offsets;
  int num_segments;
  int decoded_by_expert;  // 0: decoded holds one slot per segment; 1: one per expert id (every expert decoded)
  // One token's combine in the launch (two units, proj[1] == proj[0]; null: none): the token's two routed rows are
  // row tiles 0 and 1, one a unit, and unit 0 writes dt(fp16(out_r0 * w_r0) + fp16(out_r1 * w_r1)) to comb_out.
  uint16_t* comb_out;
  const int32_t* comb_inv;  // inverse_perm [2]: the row of each pick
  const uint16_t* comb_w;   // fp16 routing weights [2], by pick
  int comb_bf16;            // comb_out is bf16 (else fp16)
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

// Same mapping as the in-kernel-decode GEMM (tris_grouped.hip), plus the segment's expert id, loaded
// in the same round trip as the segment lengths.
__device__ inline bool mf_map_row_tile(const int32_t* __restrict__ seg, const int32_t* __restrict__ expert_ids,
                                       int nseg, int tile, int row_tile, int* s_out, int* row0_out, int* rc_out,
                                       int* e_out) {
  const int lane = static_cast<int>(__lane_id());
  int base = 0;
  for (int c = 0; c < nseg; c += kWave) {
    const int i = c + lane;
    const int ic = i < nseg ? i : nseg - 1;
    const int lo = seg[ic];
    const int hi = seg[ic + 1];
    const int ex = expert_ids[ic];
    int t = 0;
    if (i < nseg) {
      const int len = hi - lo;
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
      const int local = tile - base - excl;
      const int row0 = __shfl(lo, L) + local * row_tile;
      const int end = __shfl(hi, L);
      *s_out = c + L;
      *row0_out = row0;
      *rc_out = (end - row0) < row_tile ? (end - row0) : row_tile;
      *e_out = __shfl(ex, L);
      return true;
    }
    base += total;
  }
  return false;
}

// Row tiles of the segments (tiles of <= row_tile rows), scanned once: with at most 64 segments the
// scan stays in registers and mapping a row tile costs no memory access.
struct MfSegScan {
  int lo, hi, ex;  // this lane's segment (lane < nseg): row range and expert id
  int t, incl;     // its row tiles, inclusive prefix over lanes
  int total;       // row tiles of all segments (the same in every lane)
};

__device__ inline MfSegScan mf_scan_segments(const int32_t* __restrict__ seg, const int32_t* __restrict__ expert_ids,
                                             int nseg, int row_tile) {
  const int lane = static_cast<int>(__lane_id());
  MfSegScan r;
  r.total = 0;
  for (int c = 0; c < nseg; c += kWave) {
    const int i = c + lane;
    const int ic = i < nseg ? i : nseg - 1;
    const int lo = seg[ic];
    const int hi = seg[ic + 1];
    const int ex = expert_ids[ic];
    int t = 0;
    if (i < nseg) t = hi > lo ? (hi - lo + row_tile - 1) / row_tile : 0;
    int incl = t;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    if (c == 0) {
      r.lo = lo;
      r.hi = hi;
      r.ex = ex;
      r.t = t;
      r.incl = incl;
    }
    r.total += __shfl(incl, kWave - 1);
  }
  return r;
}

// Row tile `tile` (< sc.total) -> segment, first row, row count and expert id.
__device__ inline void mf_map_scanned(const MfSegScan& sc, const int32_t* __restrict__ seg,
                                      const int32_t* __restrict__ expert_ids, int nseg, int tile, int row_tile,
                                      int* s_out, int* row0_out, int* rc_out, int* e_out) {
  if (nseg <= kWave) {
    const int lane = static_cast<int>(__lane_id());
    const uint64_t hit = __ballot(lane < nseg && tile < sc.incl);
    const int L = __ffsll(static_cast<unsigned long long>(hit)) - 1;
    const int local = tile - __shfl(sc.incl - sc.t, L);
    const int row0 = __shfl(sc.lo, L) + local * row_tile;
    const int end = __shfl(sc.hi, L);
    *s_out = L;
    *row0_out = row0;
    *rc_out = (end - row0) < row_tile ? (end - row0) : row_tile;
    *e_out = __shfl(sc.ex, L);
    return;
  }
  mf_map_row_tile(seg, expert_ids, nseg, tile, row_tile, s_out, row0_out, rc_out, e_out);
}

constexpr int kMfPR = kMfChunk / 32;         // packed rows per chunk
constexpr int kMfTiles = kMfChunk / kTileK;  // 64-column K tiles per chunk
constexpr int kMfQ1Stride = kTileOut + 1;    // words per staged qweight1 row (odd, so per-lane row reads spread over banks)
constexpr int kMfMaxGroups = 8;              // the 64 columns x G row-scale block is staged whole
// One output tile's weight words in LDS: qweight1 [kMfPR][kMfQ1Stride], split words [kMfPR][64],
// row_pack3 [64][kMfMaxGroups][2] (32-bit words; every piece 16-byte aligned).
constexpr int kMfTbQ1 = 0;
constexpr int kMfTbGw = kMfPR * kMfQ1Stride;
constexpr int kMfTbRs = kMfTbGw + kMfPR * kTileOut;
constexpr int kMfTbWords = kMfTbRs + kTileOut * kMfMaxGroups * 2;
static_assert(kMfTbGw % 4 == 0 && kMfTbRs % 4 == 0, "tile buffer pieces must be 16-byte aligned");
constexpr int kMfCus = 256;  // MI355X compute units
// Decode kernel: row-scale groups and salient slots per chunk its LDS holds; the compact variant (at most 4
// groups and 64 salient columns per expert) fits four workgroups per CU.
constexpr int mf_groups_cap(bool compact) { return compact ? 4 : kMfMaxGroups; }
constexpr int mf_sal_slots(bool compact) { return compact ? 64 : kMfChunk; }
// per wavefront and copy buffer: qweight1 and split words of 16 columns, their row-scale block and a zero word
constexpr int mf_wave_alloc_bytes(bool compact) {
  return (2 * (kMfChunk / 32) * 16 + 16 * mf_groups_cap(compact) * 2 + 4) * 4;
}
constexpr int kMfRuns = kMfRows * (kMfChunk / 8) / kMfThreads;  // activation runs per thread of a unit

constexpr int kMfExchBytes = kMfThreads * 4 * 4;  // SwiGLU: the up unit's accumulators for the gate unit

// Bump allocation of 16-byte aligned pieces (byte offsets into dynamic LDS).
__host__ __device__ inline int mf_take(int* o, int b) {
  const int at = *o;
  *o += (b + 15) & ~15;
  return at;
}

// Static LDS of the decode kernel with `units` units and `rows` staged activation rows (as declared there).
constexpr int mf_static_lds_bytes(int units, int rows, bool compact) {
  return units * (rows * kMfXStride * 2 + kMfChunk * (2 + 2) + mf_sal_slots(compact) * (4 + 2 + 4) + 16 * 4 +
                  2 * kMfWaves * mf_wave_alloc_bytes(compact)) +
         (units == 2 ? kMfExchBytes : 16);
}

struct MfChunk {       // a unit's staged chunk
  uint16_t* xs;        // [rows][kMfXStride] activations, staged column order; column kMfChunk is zero (decode)
  uint16_t* cds;       // -C_d, staged column order (0 for salient columns)
  uint16_t* cns;       // -C_nd, staged column order (0 for salient columns)
  // Weight-stationary kernel (natural column order):
  uint32_t* col_sal;   // C0 | C1 << 16, natural order
  uint16_t* sal_col;   // chunk column of the chunk's q-th salient column
  // Decode kernel, per salient slot q (slots past the chunk's salient count, up to the next multiple of
  // kMfSalWin, read as zero weights and zero activations):
  uint32_t* sal_w;     // bits 0-4: (column - 15) mod 32, the right rotation that puts the column's qweight1 bit
                       // at bit 15; bits 8-15: byte offset of its group's R0 | R1 in a column's row-scale block;
                       // bits 16-31: byte offset of its packed row in a wavefront's qweight1 words
  uint16_t* sal_xo;    // byte offset of its activation in a staged row (the zero column for padding slots)
  uint32_t* sal_cp;    // C0 | C1 << 16 with both signs flipped (decode), or as stored (weight-stationary)
  uint16_t* sal_xi;    // weight-stationary: its position in the staged column order
  int32_t* meta;       // [t < 8] group of K tile t (-1: none); [8] first salient index; [9] end
};
struct MfTileBuf {     // one output tile's weight words
  uint32_t* q1;        // [kMfPR][kMfQ1Stride] qweight1 words of the tile's 64 columns
  uint32_t* gw;        // [kMfPR][64] predecoded split words
  uint32_t* rs;        // [64][G][2] row_pack3: R0 | R1 << 16, R_d | R_nd << 16
};

// Decode kernel: each wavefront copies only the weight words of its own 16 output columns, so no other
// wavefront waits for them.  Per wavefront and buffer: qweight1 [kMfPR][16], split words [kMfPR][16] and the
// row-scale block [16 columns][kMfMaxGroups][2]; every piece is a whole number of 64-lane copies, so a tile
// always takes kMfWDma copies (a fixed count lets each wavefront wait for exactly its own).
constexpr int kMfWCols = 16;
constexpr int kMfWq1 = 0;
constexpr int kMfWgw = kMfPR * kMfWCols;
constexpr int kMfWrs = 2 * kMfPR * kMfWCols;
template <bool kCompact>
struct MfWaveWords {
  static constexpr int kRsCopies = kMfWCols * mf_groups_cap(kCompact) * 2 / kWave;
  static constexpr int kWords = kMfWrs + kRsCopies * kWave;
  static constexpr int kDma = kWords / kWave;
  static constexpr int kAlloc = kWords + 4;  // + a zero word that no copy writes (read for K tiles without a group)
  static_assert(kMfWCols * mf_groups_cap(kCompact) * 2 % kWave == 0 && kMfWgw % kWave == 0 && kMfWrs % kWave == 0,
                "whole 64-lane copies");
  static_assert(kAlloc * 4 == mf_wave_alloc_bytes(kCompact), "LDS accounting");
};
struct MfWaveBuf {     // one wavefront's copy of its 16 columns' words
  uint32_t* q1;        // [kMfPR][16]
  uint32_t* gw;        // [kMfPR][16]
  uint32_t* rs;        // [16][G][2]
  uint32_t* zero;      // a word that holds 0
};

// Byte offset of 8 activation columns [c, c + 8) of segment row row0 + r (r < rc), or `oob` (an offset
// past the buffer: the load reads zeros) for rows outside the tile, columns past the rank and gathered
// rows whose index lies outside [0, hidden_rows).  With a row index the buffer resource covers all of
// hidden; without, it starts at row row0.  r is wave-uniform, so the index load is one scalar load.
__device__ __forceinline__ uint32_t mf_hidden_voff(const MfmaProj& pa, int row0, int r, int rc, int c, int rank,
                                                   uint32_t oob) {
  if (r >= rc || c >= rank) return oob;
  int64_t src = r;
  if (pa.row_index != nullptr) {
    src = pa.row_index[row0 + r];
    if (src < 0 || src >= pa.hidden_rows) return oob;
  }
  return static_cast<uint32_t>(src * rank + c) * 2u;
}

// The activation buffer resource of rows [row0, row0 + rc) and its size (the offset that reads zeros).  With
// partial sums the activations are staged from them (mf_partials_stage): an empty resource, whose loads read zeros
// without a memory access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mf_hidden_rsrc(const MfmaProj& pa, int row0, int rc, int rank,
                                                                 uint32_t* bytes, bool part = false) {
  if (part) {
    *bytes = 0u;
    return make_rsrc(pa.partials, 0u);
  }
  if (pa.row_index != nullptr) {
    *bytes = static_cast<uint32_t>(pa.hidden_rows) * rank * 2u;
    return make_rsrc(pa.hidden, *bytes);
  }
  *bytes = static_cast<uint32_t>(rc) * rank * 2u;
  return make_rsrc(pa.hidden + static_cast<int64_t>(row0) * rank, *bytes);
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
// Buffer loads straight into LDS: lane l's 4 (16) bytes land at dst + 4l (16l); dst is wave-uniform.
__device__ __forceinline__ void dma32(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma128(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

// s_waitcnt on the vector memory counter alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14; the export and LDS
// counters left at their maxima): wait until at most N vector memory operations are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Register-staged loads of a unit's chunk, held between issue and write.
struct MfRegs {
  uint4 xv[kMfRuns];  // activation runs: row 4h + wave, 8 columns at lane * 8
  uint64_t cpv[2];    // col_pack3 of columns kc + utid, kc + utid + 256
  uint32_t cmt[2];    // their salient words
  int q2t[2];         // their packed rows' salient prefix
  int gt[2];          // their groups (g_idx), -1 past the rank
  int sbase0;         // salient prefix at the chunk's first packed row
  int send;           // salient prefix at the chunk's end
  int32_t mv;         // metadata word (see mf_chunk_issue)
};

// Issue the register loads of chunk [kc, kc + 512) of one projection for rows [row0, row0 + rc) of
// expert e.  utid is the thread's index within its unit.  Every load is issued unconditionally (a
// branch around a load makes the compiler wait for it at the join); invalid lanes get an offset past
// their buffer, which reads 0.
__device__ __forceinline__ void mf_chunk_issue(const MfmaProj& pa, int e, int row0, int rc, int kc, int utid,
                                               MfRegs& R, bool part = false) {
  const tris_compact3_payload& p = pa.p;
  const int rank = p.rank;
  const int wave = __builtin_amdgcn_readfirstlane(utid / kWave);  // wave-uniform
  const int lane = utid % kWave;
  const int packed_rows = rank / 32;  // rank % 64 == 0
  const int pr0 = kc / 32;
  const int npr = (packed_rows - pr0) < kMfPR ? (packed_rows - pr0) : kMfPR;
  uint32_t hid_bytes;
  const __amdgpu_buffer_rsrc_t r_hid = mf_hidden_rsrc(pa, row0, rc, rank, &hid_bytes, part);
  const uint32_t col_bytes = static_cast<uint32_t>(rank) * 8u;
  const __amdgpu_buffer_rsrc_t r_col = make_rsrc(p.col_pack3 + static_cast<int64_t>(e) * rank, col_bytes);
  const int32_t* cmap_e = p.c_map + static_cast<int64_t>(e) * packed_rows;
  const int32_t* q2p_e = p.qweight2_sparse_prefix + static_cast<int64_t>(e) * (packed_rows + 1);
  const int32_t* gidx_e = p.g_idx + static_cast<int64_t>(e) * rank;
#pragma unroll
  for (int h = 0; h < kMfRuns; ++h) {
    const int r = 4 * h + wave;
    R.xv[h] = bload128(r_hid, mf_hidden_voff(pa, row0, r, rc, kc + lane * 8, rank, hid_bytes), 0u);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = kc + utid + h * kMfThreads;
    const bool kv = k < rank;
    const int pr = kv ? (k >> 5) : 0;
    R.cpv[h] = bload64(r_col, kv ? static_cast<uint32_t>(k) * 8u : col_bytes, 0u);
    R.cmt[h] = static_cast<uint32_t>(cmap_e[pr]);
    R.q2t[h] = q2p_e[pr];
    R.gt[h] = kv ? gidx_e[k] : -1;
  }
  R.sbase0 = q2p_e[pr0];
  R.send = q2p_e[pr0 + npr];
  // metadata: utid 64..71 -> group of K tile utid - 64; 72 / 73 -> salient prefix at the chunk's
  // start / end
  const int32_t* mp = q2p_e + pr0;
  if (utid >= 64 && utid < 72) {
    const int kt = kc + (utid - 64) * kTileK;
    mp = gidx_e + (kt < rank ? kt : rank - 1);
  } else if (utid == 73) {
    mp = q2p_e + pr0 + npr;
  }
  R.mv = *mp;
}

// Write a unit's register-staged chunk to LDS (waits for those loads).  Salient columns get zero
// C_d / C_nd, so the main pass gives them zero weights whatever their selector bits.
__device__ __forceinline__ void mf_chunk_write(const MfmaProj& pa, int rc, int kc, int utid, const MfChunk& ch,
                                               const MfRegs& R, bool natural = false, int sal_cap = kMfChunk,
                                               bool part = false) {
  const tris_compact3_payload& p = pa.p;
  const int rank = p.rank;
  const int G = p.num_groups;
  const int wave = __builtin_amdgcn_readfirstlane(utid / kWave);  // wave-uniform
  const int lane = utid % kWave;
#pragma unroll
  for (int h = 0; h < kMfRuns; ++h) {
    const int r = 4 * h + wave;
    if (r < rc && !part) {  // wave-uniform; partial sums are staged by mf_partials_stage
      const int c = lane * 8;  // run start within the chunk (a multiple of 8)
      // columns c + b and c + b + 4 (b < 4) are neighbours in the staged order
      const uint32_t w[4] = {R.xv[h].x, R.xv[h].y, R.xv[h].z, R.xv[h].w};
      const int base = (c & ~31) + ((c & 31) >> 2);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t lo = (w[b >> 1] >> (16 * (b & 1))) & 0xFFFFu;
        const uint32_t hi = (w[2 + (b >> 1)] >> (16 * (b & 1))) & 0xFFFFu;
        *reinterpret_cast<uint32_t*>(&ch.xs[r * kMfXStride + base + 8 * b]) = lo | (hi << 16);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int j = utid + h * kMfThreads;
    const int k = kc + j;
    const int pj = natural ? j : (j & ~31) + mf_perm32(j & 31);
    const int bit = k & 31;
    const uint32_t cm = R.cmt[h];
    const bool sal = k < rank && ((cm >> bit) & 1u);
    // staged negated (-C * R rounds to exactly -fp16(C * R)), so a set qweight1 bit is the selectors' sign bit
    ch.cds[pj] = sal ? static_cast<uint16_t>(0) : static_cast<uint16_t>((R.cpv[h] >> 32) ^ 0x8000u);
    ch.cns[pj] = sal ? static_cast<uint16_t>(0) : static_cast<uint16_t>((R.cpv[h] >> 48) ^ 0x8000u);
    if (natural) ch.col_sal[j] = static_cast<uint32_t>(R.cpv[h]);
    if (sal) {
      const int q = R.q2t[h] - R.sbase0 + __popc(cm & ((1u << bit) - 1u));
      if (natural) {
        ch.sal_col[q] = static_cast<uint16_t>(j);
        ch.sal_xi[q] = static_cast<uint16_t>((j & ~31) + mf_perm32(j & 31));
        ch.sal_cp[q] = static_cast<uint32_t>(R.cpv[h]);
      } else if (q >= 0 && q < sal_cap) {
        // the column's group as the main pass takes it (uniform 64-column groups); an invalid group gives
        // zero factors, as a K tile without a group does
        const bool gv = R.gt[h] >= 0 && R.gt[h] < G;
        ch.sal_w[q] = (static_cast<uint32_t>((j >> 5) * kMfWCols * 4) << 16) |
                      (static_cast<uint32_t>((gv ? R.gt[h] : 0) * 8) << 8) | (static_cast<uint32_t>(bit - 15) & 31u);
        ch.sal_xo[q] = static_cast<uint16_t>(pj * 2);
        ch.sal_cp[q] = (gv ? static_cast<uint32_t>(R.cpv[h]) : 0u) ^ 0x80008000u;
      }
    }
  }
  if (!natural) {
    // padding slots up to the last window's end read the zero activation column with zero factors
    const int nsal = R.send - R.sbase0;
    const int q = nsal + utid;
    if (utid < kMfSalWin && q >= 0 && q < sal_cap && q < ((nsal + kMfSalWin - 1) & ~(kMfSalWin - 1))) {
      ch.sal_w[q] = 0u;
      ch.sal_xo[q] = static_cast<uint16_t>(kMfChunk * 2);
      ch.sal_cp[q] = 0x80008000u;
    }
    // the zero column (and its neighbour, so that row 0 holds an aligned zero word)
    if (utid < rc) *reinterpret_cast<uint32_t*>(&ch.xs[utid * kMfXStride + kMfChunk]) = 0u;
  }
  if (utid >= 64 && utid < 72) {
    const bool tv = kc + (utid - 64) * kTileK < rank && R.mv >= 0 && R.mv < G;
    ch.meta[utid - 64] = tv ? R.mv : -1;
  } else if (utid >= 72 && utid < 74) {
    ch.meta[8 + (utid - 72)] = R.mv;
  }
}

// Activation rows [row0, row0 + rc) of the one chunk (rank <= kMfChunk) from the split-K partial sums of the backbone
// that produced them: fp16 of the slices' sum added in slice order, the bits the backbone's own reduction
// (backbone_reduce_at) writes.  Thread utid of the unit takes columns 2 utid and 2 utid + 1 of each row, with
// kMfPartialBatch slices' loads in flight.
constexpr int kMfPartialBatch = 16;
__device__ __forceinline__ void mf_partials_stage(const MfmaProj& pa, int row0, int rc, int utid, const MfChunk& ch) {
  const int rank = pa.p.rank;
  const int c = 2 * utid;
  const int slices = pa.slices;
  const int prow = pa.hidden_rows;
  const uint32_t bytes = static_cast<uint32_t>(slices) * static_cast<uint32_t>(prow) * rank * 4u;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(pa.partials, bytes);
  const int pos0 = (c & ~31) + mf_perm32(c & 31);
  const int pos1 = ((c + 1) & ~31) + mf_perm32((c + 1) & 31);
  for (int i = 0; i < rc; ++i) {  // uniform
    float a0 = 0.0f, a1 = 0.0f;
    for (int s0 = 0; s0 < slices; s0 += kMfPartialBatch) {
      uint64_t v[kMfPartialBatch];
#pragma unroll
      for (int j = 0; j < kMfPartialBatch; ++j) {
        const bool ok = s0 + j < slices && c < rank;
        v[j] = bload64(r, ok ? static_cast<uint32_t>(((s0 + j) * prow + row0 + i) * rank + c) * 4u : bytes, 0u);
      }
#pragma unroll
      for (int j = 0; j < kMfPartialBatch; ++j) {
        if (s0 + j < slices) {
          a0 += __uint_as_float(static_cast<uint32_t>(v[j]));
          a1 += __uint_as_float(static_cast<uint32_t>(v[j] >> 32));
        }
      }
    }
    if (c < rank) {
      ch.xs[i * kMfXStride + pos0] = f2h_bits(a0);
      ch.xs[i * kMfXStride + pos1] = f2h_bits(a1);
    }
  }
}

// LDS copies of one output tile's weight words for chunk kc: qweight1 and split words (wave w of the
// unit copies packed rows w, w + 4, ...) and the 64 x G row-scale block.  Wave-uniform conditions
// only; the caller waits (s_waitcnt) before reading.
__device__ __forceinline__ void mf_tile_issue(const MfmaProj& pa, int s, int e, int kc, int ob, int utid,
                                              const MfTileBuf& tb) {
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int rank = p.rank;
  const int G = p.num_groups;
  const int wave = __builtin_amdgcn_readfirstlane(utid / kWave);  // wave-uniform
  const int lane = utid % kWave;
  const int packed_rows = rank / 32;
  const int nob = ceil_div(N, kTileOut);
  const int nblk = (packed_rows / 2) * nob;
  const int pr0 = kc / 32;
  const int npr = (packed_rows - pr0) < kMfPR ? (packed_rows - pr0) : kMfPR;
  const int n0 = ob * kTileOut;
  const uint32_t q1_bytes = static_cast<uint32_t>(packed_rows) * N * 4u;
  const __amdgpu_buffer_rsrc_t r_q1 = make_rsrc(p.qweight1 + static_cast<int64_t>(e) * packed_rows * N, q1_bytes);
  const __amdgpu_buffer_rsrc_t r_dec =
      make_rsrc(pa.decoded + static_cast<int64_t>(s) * nblk * kGrWords, static_cast<uint32_t>(nblk) * kGrWords * 4u);
  const int n = n0 + lane;
  const uint32_t v_q1 = n < N ? static_cast<uint32_t>(n) * 4u : q1_bytes;
#pragma unroll
  for (int jj = 0; jj < kMfPR / kMfWaves; ++jj) {
    const int j = wave + kMfWaves * jj;
    if (j < npr) {
      const uint32_t pr = static_cast<uint32_t>(pr0 + j);
      dma32(r_q1, tb.q1 + j * kMfQ1Stride, v_q1, pr * N * 4u);
      dma32(r_dec, tb.gw + j * kTileOut, static_cast<uint32_t>(lane) * 4u,
            ((((pr >> 1) * nob) + ob) * kGrWords + (pr & 1u) * kTileOut) * 4u);
    }
  }
  // row_pack3[e][n0 .. n0 + 63][0 .. G - 1] is one contiguous block; columns >= N read 0
  const __amdgpu_buffer_rsrc_t r_rs =
      make_rsrc(p.row_pack3 + (static_cast<int64_t>(e) * N + n0) * G, static_cast<uint32_t>(N - n0) * G * 8u);
  const int kb = ceil_div(kTileOut * G * 8, 1024);  // <= 4 KiB (G <= kMfMaxGroups)
  for (int b = wave; b < kb; b += kMfWaves) {
    dma128(r_rs, reinterpret_cast<unsigned char*>(tb.rs) + b * 1024, static_cast<uint32_t>(b * 1024 + lane * 16), 0u);
  }
}

// Per-lane byte offsets of a wavefront's copies for chunk kc, output tile 0 (mf_wave_tile_issue adds the tile):
// lane l copies packed row pr0 + 4 i + l / 16 (copy i adds whole rows), column 16 wave + l % 16.
struct MfWaveOffsets {
  uint32_t q1;   // into the expert's qweight1 [packed rows][N]
  uint32_t dec;  // into the segment's predecoded blocks [packed rows / 2][tiles][128]
};
__device__ __forceinline__ MfWaveOffsets mf_wave_offsets(const MfmaProj& pa, int kc, int wave, int lane) {
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int nob = ceil_div(N, kTileOut);
  const uint32_t pr = static_cast<uint32_t>(kc / 32 + lane / kMfWCols);
  const uint32_t c = static_cast<uint32_t>(kMfWCols * wave + lane % kMfWCols);
  MfWaveOffsets o;
  o.q1 = (pr * N + c) * 4u;
  o.dec = ((pr >> 1) * nob * kGrWords + (pr & 1u) * kTileOut + c) * 4u;
  return o;
}

// The wavefront's LDS copies of its 16 columns of output tile ob for chunk kc: qweight1 and split words of the
// chunk's packed rows (lane l of copy i: packed row 4 i + l / 16, column l % 16) and the columns' row-scale block.
// Always MfWaveWords<kCompact>::kDma copies.  Nothing is masked: every offset is checked against its buffer's size (past it reads
// zeros), and what lies inside it but past the chunk's rows or past column N (the next row's words, the next
// tile's block) only feeds packed rows the compute skips or output columns that are not stored.  valid = false
// (a prefetch with no tile to fetch, wave-uniform) empties the buffer ranges, so every copy reads zeros without a
// memory access: a workgroup does not fetch the tile after its run, which another workgroup reads (likely through
// another XCD's L2).
template <bool kCompact>
__device__ __forceinline__ void mf_wave_tile_issue(const MfmaProj& pa, int s, int e, int ob, const MfWaveOffsets& o,
                                                   int lane, int wave, const MfWaveBuf& wb, bool valid = true) {
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int G = p.num_groups;
  const int packed_rows = p.rank / 32;
  const int nob = ceil_div(N, kTileOut);
  const int nblk = (packed_rows / 2) * nob;
  const uint32_t q1_bytes = static_cast<uint32_t>(packed_rows) * N * 4u;
  const uint32_t dec_bytes = static_cast<uint32_t>(nblk) * kGrWords * 4u;
  const __amdgpu_buffer_rsrc_t r_q1 =
      make_rsrc(p.qweight1 + static_cast<int64_t>(e) * packed_rows * N, valid ? q1_bytes : 0u);
  const __amdgpu_buffer_rsrc_t r_dec =
      make_rsrc(pa.decoded + static_cast<int64_t>(s) * nblk * kGrWords, valid ? dec_bytes : 0u);
#pragma unroll
  for (int i = 0; i < kMfPR / 4; ++i) {
    dma32(r_q1, wb.q1 + i * kWave, o.q1 + static_cast<uint32_t>(4 * i * N + ob * kTileOut) * 4u, 0u);
    dma32(r_dec, wb.gw + i * kWave, o.dec + static_cast<uint32_t>((2 * i * nob + ob) * kGrWords) * 4u, 0u);
  }
  // row_pack3[e][n0 .. n0 + 15][0 .. G - 1] is one contiguous run of 16 G pairs (32 G words); a lane past it reads
  // zeros without a memory access (an offset past the buffer), as do columns past the expert
  const int n0 = ob * kTileOut + kMfWCols * wave;
  const int ncols = valid ? N - n0 : 0;
  const uint32_t rs_bytes = ncols > 0 ? static_cast<uint32_t>(ncols) * G * 8u : 0u;
  const __amdgpu_buffer_rsrc_t r_rs =
      make_rsrc(p.row_pack3 + (static_cast<int64_t>(e) * N + (ncols > 0 ? n0 : 0)) * G, rs_bytes);
  const int rs_words = kMfWCols * 2 * G;
#pragma unroll
  for (int i = 0; i < MfWaveWords<kCompact>::kRsCopies; ++i) {
    const int w = i * kWave + lane;
    dma32(r_rs, wb.rs + i * kWave, w < rs_words ? static_cast<uint32_t>(w) * 4u : rs_bytes, 0u);
  }
}

// One projection over one staged chunk and output tile [n0, n0 + 64): accumulates rows 4 * kg + v,
// column n0 + 16 * wave + lane % 16 of x . W^T into acc.  xrow is the staged activation row this
// lane's A operand reads.
// Exact B operand of the lane's column for packed row j: the 8 weights k = kg + 4m.  Per packed row the
// lane builds nibble selectors: bit 1 = this term is used, bit 3 = the column's qweight1 bit (shared by both
// terms; the unused term is a signed zero); with the staged factors negated, w = fma(sd, fp16(-C_d * R_d),
// sn * fp16(-C_nd * R_nd)) is -fp16(C_j * R_j) where the bit is clear and +fp16(C_j * R_j) where it is set.
__device__ __forceinline__ f16x8 mf_row_b(uint32_t qw, uint32_t gw, const uint4& cdv, const uint4& cnv, uint32_t rs2,
                                          uint32_t shl, uint32_t rot) {
  const f16x2 rd2 = u32_as_f16x2(__builtin_amdgcn_perm(rs2, rs2, 0x01000100u));
  const f16x2 rn2 = u32_as_f16x2(__builtin_amdgcn_perm(rs2, rs2, 0x03020302u));
  const uint32_t cd[4] = {cdv.x, cdv.y, cdv.z, cdv.w};
  const uint32_t cn[4] = {cnv.x, cnv.y, cnv.z, cnv.w};
  const uint32_t sgn3 = (qw << shl) & 0x88888888u;  // fp4 -1.0 on a negated factor where the bit is set
  const uint32_t sd = (__builtin_rotateright32(gw, rot) & 0x22222222u) | sgn3;  // d term: fp4 +-1.0, else +-0
  const uint32_t sn = sd ^ 0x22222222u;                                        // nd term: the others
  uint32_t b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 pd = u32_as_f16x2(cd[i]) * rd2;
    const f16x2 pn = u32_as_f16x2(cn[i]) * rn2;
    const f16x2 tn = fp4x2_to_f16x2(sn, i) * pn;
    b[i] = f16x2_as_u32(__builtin_elementwise_fma(fp4x2_to_f16x2(sd, i), pd, tn));
  }
  return __builtin_bit_cast(f16x8, make_uint4(b[0], b[1], b[2], b[3]));
}

// Bit m of b (m < 8) to bit 4m.
__device__ __forceinline__ uint32_t spread8(uint32_t b) {
  b = (b | (b << 12)) & 0x000F000Fu;
  b = (b | (b << 6)) & 0x03030303u;
  return (b | (b << 3)) & 0x11111111u;
}

// mf_row_b for the natural column order: the lane's 8 weights are k = 8 kg + m (m < 8), so the A operand is 16
// contiguous bytes of an activation row.  The selector bits of those columns are byte kg of the packed words,
// spread to one nibble each.
__device__ __forceinline__ f16x8 mf_row_b_nat(uint32_t qw, uint32_t gw, const uint4& cdv, const uint4& cnv,
                                              uint32_t rs2, int kg) {
  const f16x2 rd2 = u32_as_f16x2(__builtin_amdgcn_perm(rs2, rs2, 0x01000100u));
  const f16x2 rn2 = u32_as_f16x2(__builtin_amdgcn_perm(rs2, rs2, 0x03020302u));
  const uint32_t cd[4] = {cdv.x, cdv.y, cdv.z, cdv.w};
  const uint32_t cn[4] = {cnv.x, cnv.y, cnv.z, cnv.w};
  const uint32_t q4 = spread8(__builtin_amdgcn_ubfe(qw, 8u * kg, 8u));
  const uint32_t g4 = spread8(__builtin_amdgcn_ubfe(gw, 8u * kg, 8u));
  const uint32_t sd = (g4 << 1) | (q4 << 3);  // d term: fp4 +-1.0, else +-0; bit 3 = qweight1 (negated factors)
  const uint32_t sn = sd ^ 0x22222222u;                        // nd term: the others
  uint32_t b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 pd = u32_as_f16x2(cd[i]) * rd2;
    const f16x2 pn = u32_as_f16x2(cn[i]) * rn2;
    const f16x2 tn = fp4x2_to_f16x2(sn, i) * pn;
    b[i] = f16x2_as_u32(__builtin_elementwise_fma(fp4x2_to_f16x2(sd, i), pd, tn));
  }
  return __builtin_bit_cast(f16x8, make_uint4(b[0], b[1], b[2], b[3]));
}

// Salient window [w0, w0 + wn) of the chunk (wn <= kMfSalWin): lane group kg writes the exact fp16 weights
// w = fp16(+-fp16(C0 * R0) +- fp16(C1 * R1)) of column tc for window slots kg, kg + 4, ... into its wave's
// ws row i16 (every slot, zero past wn, with no per-slot branch so the LDS reads overlap).  q2w holds the
// lane's qweight2_sparse words of rows q2b and q2b + 1 (a window spans at most two).
__device__ __forceinline__ void mf_salient_weights(const MfChunk& ch, const MfTileBuf& tb, const uint32_t* r01t,
                                                   int tc, int kg, int wave, int i16, int sbase0, int w0, int wn,
                                                   int q2b, const uint32_t q2w[2], uint16_t (*ws)[16][kMfSalStride]) {
  uint16_t wv[kMfSalWin / 4];
#pragma unroll
  for (int u = 0; u < kMfSalWin / 4; ++u) {
    const int q = 4 * u + kg;
    const bool qv = q < wn;
    const int c = ch.sal_col[w0 + (qv ? q : 0)];  // chunk column
    const uint32_t w1 = tb.q1[(c >> 5) * kMfQ1Stride + tc];
    const uint32_t rr = r01t[(c >> 6) * kTileOut + tc];
    const uint32_t cp = ch.col_sal[c];
    const int sidx = sbase0 + w0 + q;  // qweight2_sparse index
    const uint32_t q2 = ((sidx >> 5) - q2b) == 0 ? q2w[0] : q2w[1];
    // sign bits: positive where the qweight1 / qweight2 bit is set
    const uint32_t neg = ((~(w1 >> (c & 31)) & 1u) << 15) | ((~(q2 >> (sidx & 31)) & 1u) << 31);
    const f16x2 t = __builtin_bit_cast(f16x2, f16x2_as_u32(u32_as_f16x2(cp) * u32_as_f16x2(rr)) ^ neg);
    const _Float16 w = t[0] + t[1];
    wv[u] = qv ? __builtin_bit_cast(uint16_t, w) : static_cast<uint16_t>(0);
  }
#pragma unroll
  for (int u = 0; u < kMfSalWin / 4; ++u) ws[wave][i16][4 * u + kg] = wv[u];
}

// Both MFMA operands of the salient window starting at slot w0, built in registers: lane (i16, kg) takes window
// slots 8 kg .. 8 kg + 7.  bv holds the exact fp16 weights of its column, w = fp16(+-fp16(C0 * R0) +-
// fp16(C1 * R1)) (both products in one packed multiply), and av its activation row xr at those slots'
// columns.  The staged slot words carry every column-dependent offset, so a slot costs three LDS reads (its
// qweight1 word, its group's R0 | R1, its activation) and no masking: padding slots read zero factors and the
// zero activation column.  q1_lane / rs_lane: the byte offsets of the lane's column in the wavefront's qweight1
// rows and in its row-scale block; q2w: the lane's qweight2_sparse words of rows (sbase0 + w0) / 32 and the next
// (a window spans at most two), q2off = (sbase0 + w0) % 32 + 8 kg the bit of slot 0 in q2w[0] | q2w[1] << 32.
__device__ __forceinline__ void mf_salient_operands(const MfChunk& ch, const MfWaveBuf& tb, const uint16_t* xr,
                                                    uint32_t q1_lane, uint32_t rs_lane, int kg, int w0, int q2off,
                                                    const uint32_t q2w[2], f16x8& av, f16x8& bv) {
  const int s0 = w0 + 8 * kg;  // a multiple of 8: the slot vectors are 16-byte aligned
  const uint4 swa = *reinterpret_cast<const uint4*>(&ch.sal_w[s0]);
  const uint4 swb = *reinterpret_cast<const uint4*>(&ch.sal_w[s0 + 4]);
  const uint4 xov = *reinterpret_cast<const uint4*>(&ch.sal_xo[s0]);
  const uint32_t sw[8] = {swa.x, swa.y, swa.z, swa.w, swb.x, swb.y, swb.z, swb.w};
  const uint32_t xo[4] = {xov.x, xov.y, xov.z, xov.w};
  const unsigned char* q1b = reinterpret_cast<const unsigned char*>(tb.q1) + q1_lane;
  const unsigned char* rsb = reinterpret_cast<const unsigned char*>(tb.rs) + rs_lane;
  const unsigned char* xb = reinterpret_cast<const unsigned char*>(xr);
  uint32_t w1v[8], rrv[8], a16[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {  // all 24 reads issued before any is used
    w1v[u] = *reinterpret_cast<const uint32_t*>(q1b + (sw[u] >> 16));
    rrv[u] = *reinterpret_cast<const uint32_t*>(rsb + ((sw[u] >> 8) & 0xFFu));
    a16[u] = *reinterpret_cast<const uint16_t*>(xb + ((xo[u / 2] >> (16 * (u & 1))) & 0xFFFFu));
  }
  const uint4 cpa = *reinterpret_cast<const uint4*>(&ch.sal_cp[s0]);
  const uint4 cpb = *reinterpret_cast<const uint4*>(&ch.sal_cp[s0 + 4]);
  const uint32_t cp[8] = {cpa.x, cpa.y, cpa.z, cpa.w, cpb.x, cpb.y, cpb.z, cpb.w};
  // qweight2_sparse bits of the 8 slots: bit u of q2lo
  const uint32_t q2lo = static_cast<uint32_t>(((static_cast<uint64_t>(q2w[1]) << 32) | q2w[0]) >> q2off);
  uint32_t t[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    // staged factors have both signs flipped; flip back where the qweight1 (bit 15) / qweight2 (bit 31) bit is
    // set (the positive weights)
    const uint32_t rot = __builtin_amdgcn_alignbit(w1v[u], w1v[u], sw[u]);  // column's bit at bit 15
    const uint32_t pos = (rot & 0x8000u) | ((q2lo << (31 - u)) & 0x80000000u);
    t[u] = f16x2_as_u32(u32_as_f16x2(cp[u]) * u32_as_f16x2(rrv[u])) ^ pos;
  }
  uint32_t wb[4], ab[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = __builtin_amdgcn_perm(t[2 * i + 1], t[2 * i], 0x05040100u);  // the C0 R0 terms
    const uint32_t hi = __builtin_amdgcn_perm(t[2 * i + 1], t[2 * i], 0x07060302u);  // the C1 R1 terms
    wb[i] = f16x2_as_u32(u32_as_f16x2(lo) + u32_as_f16x2(hi));
    ab[i] = a16[2 * i] | (a16[2 * i + 1] << 16);
  }
  av = __builtin_bit_cast(f16x8, make_uint4(ab[0], ab[1], ab[2], ab[3]));
  bv = __builtin_bit_cast(f16x8, make_uint4(wb[0], wb[1], wb[2], wb[3]));
}

// The lane's qweight2_sparse words of the chunk's first salient window (a window of kMfSalWin salient
// columns spans at most two qweight2_sparse rows), for output column n.  Issued before the next tile's
// LDS copies so that waiting for them does not wait for the copies.
// A staged chunk's metadata in scalar registers: the group of each K tile (-1: none), the chunk's first
// salient index and its salient count.  One LDS round trip.
struct MfChunkMeta {
  int g[kMfTiles];
  int sbase0, num_sal;
};
__device__ __forceinline__ MfChunkMeta mf_chunk_meta(const MfChunk& ch) {
  const int4 m0 = *reinterpret_cast<const int4*>(&ch.meta[0]);
  const int4 m1 = *reinterpret_cast<const int4*>(&ch.meta[4]);
  const int4 m2 = *reinterpret_cast<const int4*>(&ch.meta[8]);
  const int gv[kMfTiles] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
  MfChunkMeta m;
#pragma unroll
  for (int t = 0; t < kMfTiles; ++t) m.g[t] = __builtin_amdgcn_readfirstlane(gv[t]);
  m.sbase0 = __builtin_amdgcn_readfirstlane(m2.x);
  m.num_sal = __builtin_amdgcn_readfirstlane(m2.y) - m.sbase0;
  return m;
}

__device__ __forceinline__ void mf_q2_issue(const MfmaProj& pa, int e, int n, const MfChunkMeta& cm,
                                            uint32_t q2w[2]) {
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int sbase0 = cm.sbase0;
  const int num_sal = cm.num_sal;
  const int q2rows = p.qweight2_sparse_rows;
  const uint32_t q2_bytes = static_cast<uint32_t>(q2rows) * N * 4u;
  const __amdgpu_buffer_rsrc_t r_q2 = make_rsrc(p.qweight2_sparse + static_cast<int64_t>(e) * q2rows * N, q2_bytes);
  const uint32_t v_q2 = n < N ? static_cast<uint32_t>(n) * 4u : q2_bytes;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = (sbase0 >> 5) + h;
    const bool rv = num_sal > 0 && row < q2rows;
    q2w[h] = bload32(r_q2, rv ? v_q2 : q2_bytes, static_cast<uint32_t>(rv ? row : 0) * N * 4u);
  }
}

__device__ __forceinline__ f32x4 mf_compute(const MfmaProj& pa, int e, int kc, int n0, int xrow, int utid,
                                            const MfChunk& ch, const MfChunkMeta& cm, const MfWaveBuf& tb,
                                            const uint32_t q2w0[2], f32x4 acc) {
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int rank = p.rank;
  const int G = p.num_groups;
  const int wave = __builtin_amdgcn_readfirstlane(utid / kWave);  // wave-uniform
  const int lane = utid % kWave;
  const int i16 = lane % 16;   // MFMA column within the wave's 16 outputs / A row
  const int kg = lane / 16;    // MFMA k group: columns k = kg (mod 4) of every packed row
  const int tc = 16 * wave + i16;
  const int n = n0 + tc;
  const int packed_rows = rank / 32;
  const int pr0 = kc / 32;
  const int npr = (packed_rows - pr0) < kMfPR ? (packed_rows - pr0) : kMfPR;
  const uint16_t* xr = ch.xs + xrow * kMfXStride;

  // salient columns of the chunk; the first window's qweight2_sparse words come in q2w0
  const int sbase0 = cm.sbase0;
  const int num_sal = cm.num_sal;
  const int q2rows = p.qweight2_sparse_rows;
  const uint32_t q2_bytes = static_cast<uint32_t>(q2rows) * N * 4u;
  const __amdgpu_buffer_rsrc_t r_q2 =
      make_rsrc(p.qweight2_sparse + static_cast<int64_t>(e) * q2rows * N, q2_bytes);
  const uint32_t v_q2 = n < N ? static_cast<uint32_t>(n) * 4u : q2_bytes;

  // ---- MFMA over the chunk's packed rows (salient columns have zero factors here).  Per packed row
  // the lane builds the nibble selectors of its 8 columns k = kg + 4m: bit 1 = this term is used,
  // bit 3 = negative (shared by both terms; the unused term is a signed zero).  The LDS reads of row
  // j + 1 are issued before row j is computed.
  const uint32_t rot = static_cast<uint32_t>(kg - 1) & 31u;  // rotate right: bit kg + 4m -> 4m + 1
  const uint32_t shl = static_cast<uint32_t>(3 - kg);        // shift left:   bit kg + 4m -> 4m + 3
  // the lane's column in the wavefront's row-scale block [16 columns][G][R0 | R1, R_d | R_nd]
  const uint32_t rs_lane = static_cast<uint32_t>(i16 * G * 8);
  // R_d | R_nd << 16 of each K tile's group for this column; a tile without a group reads the buffer's zero
  // word.  The offsets are selected, not the pointers, so every read is known to address this buffer and
  // need not wait for copies into the other.
  uint32_t rdn[kMfTiles];
  const uint32_t zero_off = static_cast<uint32_t>(reinterpret_cast<const unsigned char*>(tb.zero) -
                                                  reinterpret_cast<const unsigned char*>(tb.rs));
#pragma unroll
  for (int t = 0; t < kMfTiles; ++t) {
    const int g = cm.g[t];
    const uint32_t off = g >= 0 ? rs_lane + static_cast<uint32_t>(g) * 8u + 4u : zero_off;
    rdn[t] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const unsigned char*>(tb.rs) + off);
  }
  struct Row {
    uint32_t qw, gw;
    uint4 av, cd, cn;
  };
  auto load_row = [&](int j) {
    Row r;
    const int kl = j * 32 + 8 * kg;
    r.qw = tb.q1[j * kMfWCols + i16];
    r.gw = tb.gw[j * kMfWCols + i16];
    r.av = *reinterpret_cast<const uint4*>(&xr[kl]);
    r.cd = *reinterpret_cast<const uint4*>(&ch.cds[kl]);
    r.cn = *reinterpret_cast<const uint4*>(&ch.cns[kl]);
    return r;
  };
  auto row_mfma = [&](const Row& r, uint32_t rs2) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, r.av),
                                                 mf_row_b(r.qw, r.gw, r.cd, r.cn, rs2, shl, rot), acc, 0, 0, 0);
  };
  if (npr == kMfPR) {  // a full chunk
    Row cur = load_row(0);
#pragma unroll
    for (int j = 0; j < kMfPR; ++j) {
      Row nxt = cur;
      if (j + 1 < kMfPR) nxt = load_row(j + 1);  // compile-time condition
      row_mfma(cur, rdn[j / 2]);
      cur = nxt;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kMfPR; ++j) {
      if (j < npr) row_mfma(load_row(j), rdn[j / 2]);  // uniform
    }
  }

  // ---- salient columns, kMfSalWin at a time: both operands in registers (mf_salient_operands), one MFMA.
  // The first window uses the words loaded with the tile (no copy of them is made, so nothing waits for them
  // before the window); later windows load their own.
  if (num_sal > 0) {
    f16x8 av, bv;
    mf_salient_operands(ch, tb, xr, static_cast<uint32_t>(i16 * 4), rs_lane, kg, 0, (sbase0 & 31) + 8 * kg, q2w0, av,
                        bv);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
  }
  for (int w0 = kMfSalWin; w0 < num_sal; w0 += kMfSalWin) {
    const int q2b = (sbase0 + w0) >> 5;  // qweight2_sparse row of the window's first salient column
    uint32_t q2w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool rv = q2b + h < q2rows;
      q2w[h] = bload32(r_q2, rv ? v_q2 : q2_bytes, static_cast<uint32_t>(rv ? q2b + h : 0) * N * 4u);
    }
    f16x8 av, bv;
    mf_salient_operands(ch, tb, xr, static_cast<uint32_t>(i16 * 4), rs_lane, kg, w0,
                        ((sbase0 + w0) & 31) + 8 * kg, q2w, av, bv);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
  }
  return acc;
}

// Workgroup = kUnits units of 4 wavefronts.  The grid is sized to what the GPU holds at once, and the
// workgroups share the (row tile, output tile) pairs evenly: with R row tiles (tiles of <= 16 rows of one
// segment) and W = gridDim.x workgroups, each row tile gets W / R (or one more) workgroups that split its
// output tiles into runs; with R > W, workgroup w takes row tiles w, w + W, ... whole.
// kUnits == 1: one projection (blockIdx.z picks it when two are given, unfused).
// kUnits == 2: unit 0 computes the gate and unit 1 the up projection of the same tiles, side by side;
// the output is fp16(silu(g) * u).
// Along a run the units compute from one weight buffer while the next tile's weight words are copied into
// the other.  With more than one 512-column chunk (rank > 512) the chunk data is restaged per tile and
// nothing is prefetched.
// Registers are capped at what the LDS lets reside anyway: one unit with 4 staged rows fits four workgroups per CU
// (128 VGPRs), with 16 rows three.
// Every LDS array is a static object of its own (kRows activation rows staged: 4 when the batch has at most 4
// rows, else 16).  The compiler then tells the arrays apart from the copy buffers, and an LDS read waits only
// for copies into the buffer it reads; a read from dynamic LDS would wait for every copy in flight, the
// prefetch included.
template <int kUnits, int kRows, bool kCompact>
__global__ __launch_bounds__(kUnits * kMfThreads)
__attribute__((amdgpu_waves_per_eu(kUnits == 2 ? 2 : (kRows == kMfRows && !kCompact ? 3 : 4), 8)))
void grouped_mfma_kernel(MfmaArgs a) {
  using WW = MfWaveWords<kCompact>;
  constexpr int kSal = mf_sal_slots(kCompact);
  const int unit = kUnits == 2 ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kMfThreads) : 0;
  const int utid = static_cast<int>(threadIdx.x) % kMfThreads;
  const MfmaProj& pa = a.proj[kUnits == 2 ? unit : blockIdx.z];
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int nob = ceil_div(N, kTileOut);
  const MfSegScan sc = mf_scan_segments(a.segment_offsets, a.expert_ids, a.num_segments, kMfRows);
  const int R = __builtin_amdgcn_readfirstlane(sc.total);
  if (R == 0) return;  // no rows
  // the one-token combine: the two units take row tiles 0 and 1 of the same output tiles, so the workgroups share
  // out output tiles only
  const bool comb = kUnits == 2 && a.comb_out != nullptr;
  const int Rm = comb ? 1 : R;
  const int W = static_cast<int>(gridDim.x);
  const int w = static_cast<int>(blockIdx.x);
  int rt_first = w, rt_step = W, ob_lo = 0, ob_hi = nob;
  if (static_cast<int64_t>(Rm) * nob <= W) {
    // at least one workgroup per (row tile, output tile): workgroup w takes pair w, and the idle ones are the
    // last of the grid, so the busy ones are spread evenly over the CUs as the hardware deals them out
    if (w >= Rm * nob) return;
    rt_first = w / nob;
    ob_lo = w - rt_first * nob;
    ob_hi = ob_lo + 1;
    rt_step = Rm;  // one row tile
  } else if (Rm <= W) {
    const int per = W / Rm;
    const int extra = W % Rm;
    int sub, cnt;
    if (w < extra * (per + 1)) {
      rt_first = w / (per + 1);
      sub = w % (per + 1);
      cnt = per + 1;
    } else {
      rt_first = extra + (w - extra * (per + 1)) / per;
      sub = (w - extra * (per + 1)) % per;
      cnt = per;
    }
    cnt = cnt < nob ? cnt : nob;
    if (sub >= cnt) return;  // more workgroups than output tiles for this row tile
    ob_lo = static_cast<int>(static_cast<int64_t>(sub) * nob / cnt);
    ob_hi = static_cast<int>(static_cast<int64_t>(sub + 1) * nob / cnt);
    rt_step = Rm;  // one row tile
  }
  // the combine's weights by row (w_row[inverse_perm[s]] = w[s]); a route that is not one token on two experts,
  // one row each, gets zero outputs (before any barrier, the same in both units)
  uint16_t wr0 = 0, wr1 = 0;
  if (comb) {
    const int inv0 = a.comb_inv[0], inv1 = a.comb_inv[1];
    bool ok = R == 2 && ((inv0 == 0 && inv1 == 1) || (inv0 == 1 && inv1 == 0));
    for (int t = 0; t < 2 && ok; ++t) {
      int cs = 0, cr0 = 0, crc = 0, ce = -1;
      mf_map_scanned(sc, a.segment_offsets, a.expert_ids, a.num_segments, t, kMfRows, &cs, &cr0, &crc, &ce);
      ce = __builtin_amdgcn_readfirstlane(ce);
      ok = __builtin_amdgcn_readfirstlane(crc) == 1 && ce >= 0 && ce < p.num_experts;
    }
    if (!ok) {
      if (unit == 0) {
        for (int n = ob_lo * kTileOut + utid; n < ob_hi * kTileOut && n < N; n += kMfThreads) a.comb_out[n] = 0;
      }
      return;
    }
    wr0 = a.comb_w[inv0 == 0 ? 0 : 1];
    wr1 = a.comb_w[inv0 == 0 ? 1 : 0];
  }
  const int lane = utid % kWave;
  uint16_t* out = kUnits == 2 ? a.proj[0].out : pa.out;
  __shared__ __attribute__((aligned(16))) uint16_t mf_xs[kUnits][kRows * kMfXStride];
  __shared__ __attribute__((aligned(16))) uint16_t mf_cds[kUnits][kMfChunk];
  __shared__ __attribute__((aligned(16))) uint16_t mf_cns[kUnits][kMfChunk];
  __shared__ __attribute__((aligned(16))) uint32_t mf_salw[kUnits][kSal];
  __shared__ __attribute__((aligned(16))) uint16_t mf_salxo[kUnits][kSal];
  __shared__ __attribute__((aligned(16))) uint32_t mf_salcp[kUnits][kSal];
  __shared__ __attribute__((aligned(16))) int32_t mf_meta[kUnits][16];
  __shared__ __attribute__((aligned(16))) float mf_exch[kUnits == 2 ? kMfThreads * 4 : 4];
  MfChunk ch;
  ch.xs = &mf_xs[unit][0];
  ch.cds = &mf_cds[unit][0];
  ch.cns = &mf_cns[unit][0];
  ch.col_sal = nullptr;
  ch.sal_col = nullptr;
  ch.sal_xi = nullptr;
  ch.sal_w = &mf_salw[unit][0];
  ch.sal_xo = &mf_salxo[unit][0];
  ch.sal_cp = &mf_salcp[unit][0];
  ch.meta = &mf_meta[unit][0];
  // each wavefront's two copy buffers (two objects, so reads of one do not wait for copies into the other)
  __shared__ __attribute__((aligned(16))) uint32_t mf_wb0[kUnits * kMfWaves][WW::kAlloc];
  __shared__ __attribute__((aligned(16))) uint32_t mf_wb1[kUnits * kMfWaves][WW::kAlloc];
  const int wave = __builtin_amdgcn_readfirstlane(utid / kWave);
  const int wslot = unit * kMfWaves + wave;
  const MfWaveBuf tb0{&mf_wb0[wslot][kMfWq1], &mf_wb0[wslot][kMfWgw], &mf_wb0[wslot][kMfWrs],
                      &mf_wb0[wslot][WW::kWords]};
  const MfWaveBuf tb1{&mf_wb1[wslot][kMfWq1], &mf_wb1[wslot][kMfWgw], &mf_wb1[wslot][kMfWrs],
                      &mf_wb1[wslot][WW::kWords]};
  if (lane == 0) {  // the zero words (the first row tile's barrier orders these writes before any read)
    *tb0.zero = 0u;
    *tb1.zero = 0u;
  }
  float* exch = mf_exch;
  const int i16 = lane % 16;
  const int rank = p.rank;
  const bool one_chunk = rank <= kMfChunk;
  const int kg = lane / 16;

  for (int rt_i = rt_first; rt_i < Rm; rt_i += rt_step) {
  const int rt = comb ? unit : rt_i;  // the combine's units: row tiles 0 and 1
  int s = 0, row0 = 0, rc = 0, e = -1;
  mf_map_scanned(sc, a.segment_offsets, a.expert_ids, a.num_segments, rt, kMfRows, &s, &row0, &rc, &e);
  s = __builtin_amdgcn_readfirstlane(s);  // the mapping is the same in every lane
  row0 = __builtin_amdgcn_readfirstlane(row0);
  rc = __builtin_amdgcn_readfirstlane(rc);
  e = __builtin_amdgcn_readfirstlane(e);
  const int ds = a.decoded_by_expert ? e : s;  // the decoded bitmaps' slot
  // activations from partial sums: only the 4-row instances carry that staging (the host sends at most 4 rows),
  // so the others keep no register for it across their tile loop
  const bool part = kRows == 4 && pa.partials != nullptr;
  const int ob_begin = ob_lo;
  const int ob_end = ob_hi;
  if (e < 0 || e >= p.num_experts) {  // rows routed to no expert: zero output
    if (unit == 0) {
      const int span = (ob_end - ob_begin) * kTileOut;
      for (int idx = utid; idx < rc * span; idx += kMfThreads) {
        const int n = ob_begin * kTileOut + idx % span;
        if (n < N) out[static_cast<int64_t>(row0 + idx / span) * N + n] = 0;
      }
    }
    continue;
  }
  if (rt_i != rt_first) __syncthreads();  // the previous row tile's LDS readers are done
  // A operand row of this lane: rows past rc feed output rows that are not stored, so they read row 0 (the same
  // LDS words as lane 0's rows: broadcast reads instead of bank conflicts; T = 16 gate/up launch 33.2 -> 32.5 us)
  const int xrow = i16 < rc ? i16 : 0;
  const MfWaveOffsets wo = mf_wave_offsets(pa, 0, wave, lane);
  {  // chunk 0 and the first tile's weights
    MfRegs regs;
    mf_wave_tile_issue<kCompact>(pa, ds, e, ob_begin, wo, lane, wave, tb0);
    mf_chunk_issue(pa, e, row0, rc, 0, utid, regs, part);
    mf_chunk_write(pa, rc, 0, utid, ch, regs, false, kSal, part);
    if (part) mf_partials_stage(pa, row0, rc, utid, ch);  // one chunk (host-checked)
    __builtin_amdgcn_s_waitcnt(0);  // LDS copies landed (all counters zero)
    __syncthreads();
  }
  // One output tile, computed from `cur`; with one chunk each wavefront copies its columns of the next tile
  // into `nxt` meanwhile.  Called with the two buffers in alternation, so every instance knows which object it
  // reads and which it fills.  With one chunk and one unit the wavefronts do not wait for each other, and a
  // tile's four output stores are issued by the next tile (or after the last), once that tile has issued its
  // own loads and copies: nothing then waits for a store that has just been issued.  Each tile issues, after
  // the copies of `cur` (the previous tile's prefetch), at least its two qweight2_sparse loads, its prefetch
  // and the previous tile's stores, so waiting until no more than those are outstanding leaves `cur`'s copies
  // landed (vector memory operations complete in issue order).  The first tile of a row tile finds its copies
  // landed already.
  constexpr int kAfterCopies = 2 + WW::kDma + (kUnits == 1 ? 4 : 0);
  // the staged chunk's metadata, its salient count held to the slots staged (a payload whose prefix counts
  // disagree with its salient map reads no slot past them)
  const auto chunk_meta = [&]() {
    MfChunkMeta m = mf_chunk_meta(ch);
    m.num_sal = m.num_sal < 0 ? 0 : (m.num_sal < kSal ? m.num_sal : kSal);
    return m;
  };
  // one unit: the last tile's outputs (fp16 pairs of rows 4 kg .. 4 kg + 3) and the tile they belong to
  uint32_t held01 = 0u, held23 = 0u;
  int held_ob = -1;
  const uint32_t out_bytes = static_cast<uint32_t>(rc) * N * 2u;
  const __amdgpu_buffer_rsrc_t r_out = make_rsrc(out + static_cast<int64_t>(row0) * N, out_bytes);
  auto store_held = [&]() {
    const int hn = held_ob * kTileOut + 16 * wave + i16;
    const uint32_t hv[4] = {held01 & 0xFFFFu, held01 >> 16, held23 & 0xFFFFu, held23 >> 16};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * kg + v;
      __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(hv[v]), r_out,
                                            hn < N && r < rc ? static_cast<uint32_t>(r * N + hn) * 2u : out_bytes,
                                            0u, 0);
    }
  };
  auto tile = [&](int ob, const MfWaveBuf& cur, const MfWaveBuf& nxt) {
    const int n = ob * kTileOut + 16 * wave + i16;
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // (the two cases keep separate qweight2_sparse words: a variable shared by both would be copied at their join,
    // and the copy waits for the loads)
    if (one_chunk) {
      const MfChunkMeta cm = chunk_meta();
      uint32_t q2w[2];
      mf_q2_issue(pa, e, n, cm, q2w);
      mf_wave_tile_issue<kCompact>(pa, ds, e, ob + 1, wo, lane, wave, nxt, ob + 1 < ob_end);  // prefetch
      if (kUnits == 1 && held_ob >= 0) store_held();  // the previous tile's outputs (wave-uniform condition)
      wait_vmcnt<kAfterCopies>();  // this wavefront's copies into `cur` landed
      acc = mf_compute(pa, e, 0, ob * kTileOut, xrow, utid, ch, cm, cur, q2w, acc);
    } else {
      for (int kc = 0; kc < rank; kc += kMfChunk) {
        if (ob > ob_begin || kc > 0) {
          __syncthreads();  // the previous chunk's readers are done
          MfRegs regs;
          mf_wave_tile_issue<kCompact>(pa, ds, e, ob, mf_wave_offsets(pa, kc, wave, lane), lane, wave, cur);
          mf_chunk_issue(pa, e, row0, rc, kc, utid, regs);
          mf_chunk_write(pa, rc, kc, utid, ch, regs, false, kSal);
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
        }
        const MfChunkMeta cm = chunk_meta();
        uint32_t q2w[2];
        mf_q2_issue(pa, e, n, cm, q2w);
        acc = mf_compute(pa, e, kc, ob * kTileOut, xrow, utid, ch, cm, cur, q2w, acc);
      }
    }

    // stores through a buffer resource over the tile's rows: rows past rc and columns past N go past its end and
    // are dropped, so every lane issues all four
    const bool nv = n < N;
    if (kUnits == 2) {
      if (unit == 1) *reinterpret_cast<f32x4*>(&exch[utid * 4]) = acc;
      __syncthreads();
      if (unit == 0 && comb) {
        // row 0 of each unit's tile (one row a tile): the combine of the token's two rows at column n, the products
        // rounded to fp16 (the asm keeps them from being fused into the sum) and added in fp32 (two terms: the
        // pick order does not matter), rounded once to the output dtype
        if (kg == 0 && nv) {
          const float up0 = exch[utid * 4];
          uint16_t p0 = hmul_bits(f2h_bits(acc[0]), wr0);
          uint16_t p1 = hmul_bits(f2h_bits(up0), wr1);
          asm volatile("" : "+v"(p0), "+v"(p1));
          const float y = h2f(p0) + h2f(p1);
          a.comb_out[n] = a.comb_bf16 ? f32_to_bf16_rne(y) : f2h_bits(y);
        }
      } else if (unit == 0) {
        const f32x4 up = *reinterpret_cast<const f32x4*>(&exch[utid * 4]);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 4 * kg + v;
          // g and u rounded to fp16 as the two outputs would be
          __builtin_amdgcn_raw_buffer_store_b16(swiglu_bits(f2h_bits(acc[v]), f2h_bits(up[v])), r_out,
                                                nv && r < rc ? static_cast<uint32_t>(r * N + n) * 2u : out_bytes,
                                                0u, 0);
        }
      }
      __syncthreads();  // exch is rewritten by the next tile
    } else {
      // no output scale or bias here: the host sends none (launch_grouped_mfma rejects payloads with them)
      uint32_t hv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) hv[v] = f2h_bits(acc[v]);
      held01 = hv[0] | (hv[1] << 16);
      held23 = hv[2] | (hv[3] << 16);
      held_ob = ob;
      if (!one_chunk) {
        store_held();
        held_ob = -1;
      }
    }
  };
  for (int ob = ob_begin; ob < ob_end; ob += 2) {
    tile(ob, tb0, tb1);
    if (ob + 1 < ob_end) tile(ob + 1, tb1, tb0);
  }
  if (kUnits == 1 && held_ob >= 0) store_held();  // the row tile's last outputs
  }  // row tiles
}

// ----------------------------------------------------------------------------------------------------
// Weight-stationary variant for long segments (prefill).  A work item is (active segment, kSub 64-column
// output tiles): the unit copies the tiles' weight words, builds the exact B operands of its columns over the
// whole K (rank <= 512: 16 packed rows, 4 registers each per tile, plus at most two 32-column salient windows)
// once, and streams the segment's 16-row activation tiles through them: per row tile and output tile 16 + 1
// or 2 MFMAs per wavefront, with the next row tile's loads in flight meanwhile (two activation buffers).
// Each A-operand read from LDS feeds kSub MFMAs: one 16 x 16 x 32 MFMA per kilobyte read would need 256 B
// of LDS reads per clock on a CU (4 SIMDs), twice what the LDS delivers.  kUnits == 2 runs the gate and up
// projections of the same item side by side and writes fp16(silu(g) * u).
constexpr int kWsSalWindows = 2;  // salient columns per item <= 64
constexpr int kWsMinRows = 64;    // mean rows per active segment from which the host picks this kernel
#ifndef TRIS_WS_SUB
#define TRIS_WS_SUB 2
#endif
constexpr int kWsSub = TRIS_WS_SUB;  // output tiles per item (2: one activation read feeds two MFMAs)
#ifndef TRIS_WS_XSTRIDE
#define TRIS_WS_XSTRIDE 528
#endif
constexpr int kWsXStride = TRIS_WS_XSTRIDE;  // fp16 elements per staged activation row (kMfChunk + zero column + pad)
static_assert(kWsXStride > kMfChunk && kWsXStride % 8 == 0, "staged rows need the zero column and 16-byte runs");
#ifndef TRIS_WS_READ_AHEAD
#define TRIS_WS_READ_AHEAD 4
#endif
constexpr int kWsReadAhead = TRIS_WS_READ_AHEAD;  // A-operand LDS reads in flight ahead of the MFMAs
#ifndef TRIS_WS_XDEPTH
#define TRIS_WS_XDEPTH 1
#endif
constexpr int kWsXDepth = TRIS_WS_XDEPTH;  // row tiles of activations in flight in registers (1 or 2)
static_assert(kWsXDepth == 1 || kWsXDepth == 2, "activation prefetch depth is 1 or 2");

struct MfWsLayout {  // per unit, byte offsets into dynamic LDS
  int xs[2], cds, cns, col_sal, sal_col, sal_xi, sal_cp, meta, r01t, ws, bytes;
};

__host__ __device__ inline MfWsLayout mf_ws_layout() {
  MfWsLayout L;
  int o = 0;
  L.xs[0] = mf_take(&o, kMfRows * kWsXStride * 2);
  L.xs[1] = mf_take(&o, kMfRows * kWsXStride * 2);
  L.cds = mf_take(&o, kMfChunk * 2);
  L.cns = mf_take(&o, kMfChunk * 2);
  L.col_sal = mf_take(&o, kMfChunk * 4);
  L.sal_col = mf_take(&o, kMfChunk * 2);
  L.sal_xi = mf_take(&o, kMfChunk * 2);
  L.sal_cp = mf_take(&o, kMfChunk * 4);
  L.meta = mf_take(&o, 16 * 4);
  L.r01t = mf_take(&o, kMfTiles * kTileOut * 4);
  L.ws = mf_take(&o, kMfWaves * 16 * kMfSalStride * 2);
  L.bytes = o;
  return L;
}

__host__ __device__ inline int mf_ws_lds_bytes(int units, int sub) {
  return units * mf_ws_layout().bytes + (units == 2 ? sub * kMfExchBytes : 0);
}

// Activation rows [row0, row0 + rc) of the chunk: register loads (issued early) and the permuted LDS write.
struct WsX {
  uint4 xv[kMfRuns];
};

__device__ __forceinline__ void ws_x_issue(const MfmaProj& pa, int row0, int rc, int utid, WsX& X) {
  const int rank = pa.p.rank;
  const int wave = utid / kWave;
  const int lane = utid % kWave;
  uint32_t hid_bytes;
  const __amdgpu_buffer_rsrc_t r_hid = mf_hidden_rsrc(pa, row0, rc, rank, &hid_bytes);
#pragma unroll
  for (int h = 0; h < kMfRuns; ++h) {
    const int r = 4 * h + wave;
    X.xv[h] = bload128(r_hid, mf_hidden_voff(pa, row0, r, rc, lane * 8, rank, hid_bytes), 0u);
  }
}

// The same for materialised rows (no row_index): r_seg covers the segment's rows, rel0 is row0's row within
// it; rows past the segment read zeros through the resource's size, so no per-row test is needed.
__device__ __forceinline__ void ws_x_issue_seg(__amdgpu_buffer_rsrc_t r_seg, int rel0, int rank, int utid, WsX& X) {
  const int wave = utid / kWave;
  const int lane = utid % kWave;
  const uint32_t base = (static_cast<uint32_t>(rel0 + wave) * rank + lane * 8) * 2u;
#pragma unroll
  for (int h = 0; h < kMfRuns; ++h) X.xv[h] = bload128(r_seg, base + static_cast<uint32_t>(4 * h * rank) * 2u, 0u);
}

// Writes every staged row in natural column order (rows >= rc get the zeros their loads returned): one
// 16-byte LDS write per run, a wave's 64 runs one contiguous kilobyte.
__device__ __forceinline__ void ws_x_write(int utid, uint16_t* xs, const WsX& X) {
  const int wave = utid / kWave;
  const int lane = utid % kWave;
#pragma unroll
  for (int h = 0; h < kMfRuns; ++h) {
    const int r = 4 * h + wave;
    *reinterpret_cast<uint4*>(&xs[r * kWsXStride + lane * 8]) = X.xv[h];
  }
}

// Work split: item (segment a, kSub output tiles from tile kSub * i) costs t_a + kWsBuildCost row tiles (t_a:
// the segment's row tiles; building the B operands costs about kWsBuildCost of them).  Items are ordered
// segment-major, each item's build first and then its row tiles, and the workgroup of virtual index v takes
// the row tiles whose cost position lies in [v * total / W, (v + 1) * total / W), building the B operands of
// every item it touches: an item split between two workgroups is built twice, and every workgroup gets the
// same cost to within one item's build.  Each lane works out the item and row range of its segment, so no
// item list exists anywhere.  Virtual indices are XCD-major: the hardware places workgroup w on XCD w % 8, and each
// XCD gets a contiguous share of the items, so its L2 holds the activations of about one segment instead
// of every XCD streaming every segment.
constexpr int kWsBuildCost = 2;
constexpr int kXcds = 8;  // MI355X: 8 XCDs (32 CUs and one L2 each)

__device__ __forceinline__ int xcd_major_index(int w, int W) {
  const int x = w % kXcds;
  const int q = W / kXcds;
  const int r = W % kXcds;
  return x * q + (x < r ? x : r) + w / kXcds;
}

// kSub output tiles per item: wavefront w computes columns 16 w + (0..15) of each, so one activation read
// from LDS feeds kSub MFMAs (B operands: 16 packed rows x kSub x 4 registers).  Activations are staged in
// natural column order (a plain copy) and the B operands built for it (mf_row_b_nat).
template <int kUnits, int kSub>
__global__ __launch_bounds__(kUnits * kMfThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void grouped_mfma_ws_kernel(
    MfmaArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char mf_lds[];
  __shared__ __attribute__((aligned(16))) uint32_t ws_tb[kUnits][kSub][kMfTbWords];
  const int unit = kUnits == 2 ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kMfThreads) : 0;
  const int utid = static_cast<int>(threadIdx.x) % kMfThreads;
  const MfmaProj& pa = a.proj[kUnits == 2 ? unit : blockIdx.z];
  const tris_compact3_payload& p = pa.p;
  const int N = p.outfeatures;
  const int G = p.num_groups;
  const int nob = ceil_div(N, kTileOut);
  const int nit = ceil_div(nob, kSub);  // items per segment
  const int npr = p.rank / 32;          // <= kMfPR: rank <= kMfChunk (host-checked)
  const int wave = __builtin_amdgcn_readfirstlane(utid / kWave);
  const int lane = utid % kWave;
  const int i16 = lane % 16;
  const int kg = lane / 16;
  const int tc = 16 * wave + i16;
  uint16_t* out = kUnits == 2 ? a.proj[0].out : pa.out;

  // segments (<= 64, host-checked): lane i holds segment i
  const MfSegScan sc = mf_scan_segments(a.segment_offsets, a.expert_ids, a.num_segments, kMfRows);
  const bool act = static_cast<int>(__lane_id()) < a.num_segments && sc.t > 0;
  const int u = act ? sc.t + kWsBuildCost : 0;
  int incl = u;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int v = __shfl_up(incl, d);
    if (static_cast<int>(__lane_id()) >= d) incl += v;
  }
  const int64_t total = static_cast<int64_t>(nit) * __shfl(incl, kWave - 1);
  const int64_t W = gridDim.x;
  const int64_t vw = xcd_major_index(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int64_t lo_w = vw * total / W;
  const int64_t hi_w = (vw + 1) * total / W;
  const int64_t base = static_cast<int64_t>(nit) * (incl - u);
  // this workgroup's cost range relative to the segment's first item, clamped to the segment's cost; item it
  // covers [it * u, (it + 1) * u), its row tile r sits at it * u + kWsBuildCost + r
  int d0 = 0, d1 = 0, it_lo = 0, it_hi = 0;
  if (act) {
    const int64_t seg_cost = static_cast<int64_t>(nit) * u;
    const int64_t e0 = lo_w - base, e1 = hi_w - base;
    d0 = static_cast<int>(e0 < 0 ? 0 : (e0 > seg_cost ? seg_cost : e0));
    d1 = static_cast<int>(e1 < 0 ? 0 : (e1 > seg_cost ? seg_cost : e1));
    it_lo = d0 / u;  // first item with a row tile at or past d0
    it_hi = d1 > kWsBuildCost ? (d1 - kWsBuildCost + u - 1) / u : 0;  // first item whose row tiles start at or past d1
    it_hi = it_hi < nit ? it_hi : nit;
  }
  uint64_t todo = __ballot(act && it_hi > it_lo);

  const MfWsLayout L = mf_ws_layout();
  unsigned char* lbase = mf_lds + unit * L.bytes;
  MfChunk ch;
  ch.xs = nullptr;
  ch.cds = reinterpret_cast<uint16_t*>(lbase + L.cds);
  ch.cns = reinterpret_cast<uint16_t*>(lbase + L.cns);
  ch.col_sal = reinterpret_cast<uint32_t*>(lbase + L.col_sal);
  ch.sal_col = reinterpret_cast<uint16_t*>(lbase + L.sal_col);
  ch.sal_xi = reinterpret_cast<uint16_t*>(lbase + L.sal_xi);
  ch.sal_cp = reinterpret_cast<uint32_t*>(lbase + L.sal_cp);
  ch.sal_w = nullptr;
  ch.sal_xo = nullptr;
  ch.meta = reinterpret_cast<int32_t*>(lbase + L.meta);
  uint16_t* const xsb0 = reinterpret_cast<uint16_t*>(lbase + L.xs[0]);
  uint16_t* const xsb1 = reinterpret_cast<uint16_t*>(lbase + L.xs[1]);
  // column kMfChunk of every staged row stays zero (the activation writes cover columns 0 .. 511): the salient
  // gather's padding slots read it
  if (utid < 2 * kMfRows) (utid < kMfRows ? xsb0 : xsb1)[(utid % kMfRows) * kWsXStride + kMfChunk] = 0;
  uint32_t* r01t = reinterpret_cast<uint32_t*>(lbase + L.r01t);
  auto ws = reinterpret_cast<uint16_t (*)[16][kMfSalStride]>(lbase + L.ws);
  float* exch = reinterpret_cast<float*>(mf_lds + kUnits * L.bytes);
  MfTileBuf tb[kSub];
#pragma unroll
  for (int b = 0; b < kSub; ++b) {
    tb[b].q1 = &ws_tb[unit][b][kMfTbQ1];
    tb[b].gw = &ws_tb[unit][b][kMfTbGw];
    tb[b].rs = &ws_tb[unit][b][kMfTbRs];
  }
  while (todo != 0) {
    const int s = __ffsll(static_cast<unsigned long long>(todo)) - 1;  // wave-uniform
    todo &= todo - 1;
    const int seg_lo = __builtin_amdgcn_readfirstlane(__shfl(sc.lo, s));
    const int seg_hi = __builtin_amdgcn_readfirstlane(__shfl(sc.hi, s));
    const int e = __builtin_amdgcn_readfirstlane(__shfl(sc.ex, s));
    const int it0 = __builtin_amdgcn_readfirstlane(__shfl(it_lo, s));
    const int it1 = __builtin_amdgcn_readfirstlane(__shfl(it_hi, s));
    const int sd0 = __builtin_amdgcn_readfirstlane(__shfl(d0, s));
    const int sd1 = __builtin_amdgcn_readfirstlane(__shfl(d1, s));
    const int rows = seg_hi - seg_lo;
    const int nrt = ceil_div(rows, kMfRows);
    const int cu = nrt + kWsBuildCost;
    const bool dead = e < 0 || e >= p.num_experts;  // rows routed to no expert: zero output
    for (int it = it0; it < it1; ++it) {
      // this workgroup's row tiles of the item (never empty: see it_lo, it_hi)
      const int r_lo = max(0, min(nrt, sd0 - it * cu - kWsBuildCost));
      const int r_hi = max(0, min(nrt, sd1 - it * cu - kWsBuildCost));
      const int ob = it * kSub;
      if (dead) {
        if (unit == 0) {
          const int n_lo = ob * kTileOut;
          const int n_hi = ((ob + kSub) * kTileOut) < N ? (ob + kSub) * kTileOut : N;
          const int span = n_hi - n_lo;
          const int row_lo = seg_lo + r_lo * kMfRows;
          const int nrow = min(seg_hi, seg_lo + r_hi * kMfRows) - row_lo;
          for (int idx = utid; idx < nrow * span; idx += kMfThreads) {
            out[static_cast<int64_t>(row_lo + idx / span) * N + n_lo + idx % span] = 0;
          }
        }
        continue;
      }
      __syncthreads();  // the previous item's LDS readers are done
#pragma unroll
      for (int b = 0; b < kSub; ++b) {
        if (ob + b < nob) mf_tile_issue(pa, a.decoded_by_expert ? e : s, e, 0, ob + b, utid, tb[b]);  // uniform
      }
      if (it == it0) {  // the segment's column data
        MfRegs regs;
        mf_chunk_issue(pa, e, seg_lo, 0, 0, utid, regs);  // rc = 0: no activation rows
        mf_chunk_write(pa, 0, 0, utid, ch, regs, true);  // natural column order
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      int n[kSub];
      bool nv[kSub];
#pragma unroll
      for (int b = 0; b < kSub; ++b) {
        n[b] = (ob + b) * kTileOut + tc;
        nv[b] = n[b] < N;
      }
      const int sbase0 = __builtin_amdgcn_readfirstlane(ch.meta[8]);
      const int num_sal = __builtin_amdgcn_readfirstlane(ch.meta[9]) - sbase0;
      uint32_t q2w[kSub][kWsSalWindows + 1];  // qweight2_sparse words of the rows the windows span
      {
        const int q2rows = p.qweight2_sparse_rows;
        const uint32_t q2_bytes = static_cast<uint32_t>(q2rows) * N * 4u;
        const __amdgpu_buffer_rsrc_t r_q2 =
            make_rsrc(p.qweight2_sparse + static_cast<int64_t>(e) * q2rows * N, q2_bytes);
#pragma unroll
        for (int b = 0; b < kSub; ++b) {
          const uint32_t v_q2 = nv[b] ? static_cast<uint32_t>(n[b]) * 4u : q2_bytes;
#pragma unroll
          for (int h = 0; h <= kWsSalWindows; ++h) {
            const int row = (sbase0 >> 5) + h;
            const bool rv = num_sal > 0 && row < q2rows;
            q2w[b][h] = bload32(r_q2, rv ? v_q2 : q2_bytes, static_cast<uint32_t>(rv ? row : 0) * N * 4u);
          }
        }
      }
      // materialised rows: one buffer resource over the segment's activations and one over its outputs (rows
      // past the segment read zeros and drop their stores through the resources' sizes)
      const bool seg_rows = pa.row_index == nullptr;
      const __amdgpu_buffer_rsrc_t r_seg =
          make_rsrc(pa.hidden + static_cast<int64_t>(seg_lo) * p.rank, static_cast<uint32_t>(rows) * p.rank * 2u);
      const uint32_t out_bytes = static_cast<uint32_t>(rows) * N * 2u;
      const __amdgpu_buffer_rsrc_t r_out = make_rsrc(out + static_cast<int64_t>(seg_lo) * N, out_bytes);
      uint32_t ocol[kSub];  // byte offset of the lane's column in row 4 kg of the row tile, or past the outputs
#pragma unroll
      for (int b = 0; b < kSub; ++b) ocol[b] = nv[b] ? static_cast<uint32_t>(4 * kg * N + n[b]) * 2u : 0x80000000u;
      auto x_issue = [&](int rt, WsX& X) {
        const int r0 = seg_lo + rt * kMfRows;
        if (seg_rows) {
          ws_x_issue_seg(r_seg, rt * kMfRows, p.rank, utid, X);
        } else {
          ws_x_issue(pa, r0, min(seg_hi - r0, kMfRows), utid, X);
        }
      };
      // the first two row tiles' activations, in flight while the B operands are built; row tile rt's
      // registers are X[rt % 2], reloaded with row tile rt + 2 once staged
      WsX X0, X1;
      x_issue(r_lo, X0);
      if (kWsXDepth == 2 && r_lo + 1 < r_hi) x_issue(r_lo + 1, X1);

      // columns of the salient activations of each window, two 16-bit offsets a word, in the A operand's slot
      // order (padding slots point at the zero column kMfChunk)
      uint32_t soff[kWsSalWindows][4];
#pragma unroll
      for (int win = 0; win < kWsSalWindows; ++win) {
        const int w0 = win * kMfSalWin;
        const int wn = (num_sal - w0) < kMfSalWin ? (num_sal - w0) : kMfSalWin;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q0 = 8 * kg + 2 * i;
          uint32_t lo = kMfChunk, hi = kMfChunk;
          if (q0 < wn) {
            const int c = ch.sal_col[w0 + q0];
            lo = static_cast<uint32_t>(c);
          }
          if (q0 + 1 < wn) {
            const int c = ch.sal_col[w0 + q0 + 1];
            hi = static_cast<uint32_t>(c);
          }
          soff[win][i] = lo | (hi << 16);
        }
      }
      // ---- B operands over the whole K, per output tile: the packed rows, then the salient windows (the
      // row scales R0 | R1 << 16 go through r01t, rewritten per tile)
      f16x8 bmain[kSub][kMfPR];
      f16x8 bsal[kSub][kWsSalWindows];
#pragma unroll
      for (int b = 0; b < kSub; ++b) {
#pragma unroll
        for (int t = 0; t < kMfTiles; ++t) {
          const int g = __builtin_amdgcn_readfirstlane(ch.meta[t]);
          const int gi = (tc * G + (g >= 0 ? g : 0)) * 2;
          const uint32_t rdn = g >= 0 ? tb[b].rs[gi + 1] : 0u;
          if ((t & 3) == kg) r01t[t * kTileOut + tc] = g >= 0 ? tb[b].rs[gi] : 0u;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const int j = 2 * t + jj;
            bmain[b][j] = f16x8{};
            if (j < npr) {  // uniform
              const int kl = j * 32 + 8 * kg;
              bmain[b][j] = mf_row_b_nat(tb[b].q1[j * kMfQ1Stride + tc], tb[b].gw[j * kTileOut + tc],
                                         *reinterpret_cast<const uint4*>(&ch.cds[kl]),
                                         *reinterpret_cast<const uint4*>(&ch.cns[kl]), rdn, kg);
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();  // r01t written
#pragma unroll
        for (int win = 0; win < kWsSalWindows; ++win) {
          const int w0 = win * kMfSalWin;
          const int wn = (num_sal - w0) < kMfSalWin ? (num_sal - w0) : kMfSalWin;
          bsal[b][win] = f16x8{};
          if (wn > 0) {  // uniform
            const int q2b = (sbase0 + w0) >> 5;
            const uint32_t q2pair[2] = {q2w[b][win], q2w[b][win + 1]};
            mf_salient_weights(ch, tb[b], r01t, tc, kg, wave, i16, sbase0, w0, wn, q2b, q2pair, ws);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            bsal[b][win] = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&ws[wave][i16][8 * kg]));
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();  // ws (and, after the last window, r01t) are rewritten next
          }
        }
      }

      // ---- the segment's row tiles through the stationary B operands
      auto row_tile = [&](int rt, uint16_t* xs, WsX& X) {
        ws_x_write(utid, xs, X);
        __syncthreads();  // staged rows visible; the previous row tile's exch reads are done
        if (rt + kWsXDepth < r_hi) x_issue(rt + kWsXDepth, X);  // depth 1: X0 is the only register set
        const uint16_t* xr = xs + i16 * kWsXStride;
        f32x4 acc[kSub];
#pragma unroll
        for (int b = 0; b < kSub; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // activations at the salient columns of window win (their A operand)
        auto sal_gather = [&](int win) {
          uint32_t ap[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t lo = xr[soff[win][i] & 0xFFFFu];
            const uint32_t hi = xr[soff[win][i] >> 16];
            ap[i] = lo | (hi << 16);
          }
          return __builtin_bit_cast(f16x8, make_uint4(ap[0], ap[1], ap[2], ap[3]));
        };
        auto row_mfma = [&](int j) {
          const f16x8 av = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(&xr[j * 32 + 8 * kg]));
#pragma unroll
          for (int b = 0; b < kSub; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bmain[b][j], acc[b], 0, 0, 0);
        };
        // window 0 always runs (zero weights and the zero column when the chunk has no salient column), so it
        // joins the main block: its gathers are issued first and its MFMA comes last
        const f16x8 as0 = sal_gather(0);
        if (npr == kMfPR) {  // rank 512: no branch between the MFMAs, so the LDS reads run ahead of them
#pragma unroll
          for (int j = 0; j < kMfPR; ++j) row_mfma(j);
#pragma unroll
          for (int b = 0; b < kSub; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as0, bsal[b][0], acc[b], 0, 0, 0);
          // schedule: kWsReadAhead A reads, then one MFMA group per further read
          __builtin_amdgcn_sched_group_barrier(0x100, kWsReadAhead, 0);
#pragma unroll
          for (int j = kWsReadAhead; j < kMfPR; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x008, kSub, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, (kWsReadAhead + 1) * kSub, 0);
        } else {
#pragma unroll
          for (int j = 0; j < kMfPR; ++j) {
            if (j < npr) row_mfma(j);  // uniform
          }
#pragma unroll
          for (int b = 0; b < kSub; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as0, bsal[b][0], acc[b], 0, 0, 0);
        }
#pragma unroll
        for (int win = 1; win < kWsSalWindows; ++win) {
          if (win * kMfSalWin < num_sal) {  // uniform
            const f16x8 av = sal_gather(win);
#pragma unroll
            for (int b = 0; b < kSub; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bsal[b][win], acc[b], 0, 0, 0);
          }
        }
        if (kUnits == 2) {
          if (unit == 1) {
#pragma unroll
            for (int b = 0; b < kSub; ++b) *reinterpret_cast<f32x4*>(&exch[(b * kMfThreads + utid) * 4]) = acc[b];
          }
          __syncthreads();
          if (unit == 0) {
#pragma unroll
            for (int b = 0; b < kSub; ++b) {
              const f32x4 up = *reinterpret_cast<const f32x4*>(&exch[(b * kMfThreads + utid) * 4]);
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                __builtin_amdgcn_raw_buffer_store_b16(swiglu_bits(f2h_bits(acc[b][v]), f2h_bits(up[v])), r_out,
                                                      ocol[b] + static_cast<uint32_t>(rt * kMfRows + v) * N * 2u, 0u, 0);
              }
            }
          }
        } else {
#pragma unroll
          for (int b = 0; b < kSub; ++b) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              __builtin_amdgcn_raw_buffer_store_b16(f2h_bits(acc[b][v]), r_out,
                                                    ocol[b] + static_cast<uint32_t>(rt * kMfRows + v) * N * 2u, 0u, 0);
            }
          }
        }
      };
      // two activation buffers in alternation (distinct objects per call site)
      for (int rt = r_lo; rt < r_hi; rt += 2) {
        row_tile(rt, xsb0, X0);
        if (rt + 1 < r_hi) row_tile(rt + 1, xsb1, kWsXDepth == 2 ? X1 : X0);
      }
    }
  }
}

int check_payload(const tris_compact3_payload* p, bool need_gr, const char* who);

static bool allow_mfma_lds(const void* kernel, int bytes) {
  // dynamic LDS granted so far per kernel (the weight-stationary kernel's two instantiations)
  static const void* kernels[2] = {reinterpret_cast<const void*>(&grouped_mfma_ws_kernel<1, kWsSub>),
                                   reinterpret_cast<const void*>(&grouped_mfma_ws_kernel<2, kWsSub>)};
  static int granted[2] = {0, 0};
  int which = 0;
  while (which < 1 && kernels[which] != kernel) ++which;
  if (bytes <= granted[which]) return true;
  // Raising the dynamic LDS limit is not a stream operation, so it is safe while a caller captures a graph.
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  granted[which] = bytes;
  return true;
}

// Weight-stationary launch (long segments, one 512-column chunk, <= 64 salient columns per expert):
// workgroups as the GPU holds at once (the occupancy the compiled kernel allows with this LDS), no more
// than the items.
static int launch_grouped_mfma_ws(const MfmaArgs& args, int units, int nproj, int max_n, int batch,
                                  hipStream_t s, const char* who) {
  const int lds = mf_ws_lds_bytes(units, kWsSub);
  const int lds_total = lds + units * kWsSub * kMfTbWords * 4;
  TRIS_REQUIRE(lds_total <= 160 * 1024, "%s: LDS request %d exceeds a CU", who, lds_total);
  const void* kernel = units == 2 ? reinterpret_cast<const void*>(&grouped_mfma_ws_kernel<2, kWsSub>)
                                  : reinterpret_cast<const void*>(&grouped_mfma_ws_kernel<1, kWsSub>);
  TRIS_REQUIRE(allow_mfma_lds(kernel, lds), "%s: %s", who, "cannot raise the kernel's dynamic LDS limit");
  static int per_cu[2] = {0, 0};  // resident workgroups per CU, per kernel (queried once)
  int& wgs_per_cu = per_cu[units - 1];
  if (wgs_per_cu == 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, units * kMfThreads, lds) != hipSuccess) {
      (void)hipGetLastError();
      nb = 1;
    }
    wgs_per_cu = nb > 0 ? nb : 1;
  }
  int wgs = (kMfCus * wgs_per_cu) / nproj;
  // an upper bound of the work's cost in row tiles (each segment's last row tile may be partial, and every
  // item has its build): workgroups past it would find no row tile
  const int64_t items = static_cast<int64_t>(args.num_segments) * ceil_div(ceil_div(max_n, kTileOut), kWsSub);
  const int64_t cost = static_cast<int64_t>(ceil_div(ceil_div(max_n, kTileOut), kWsSub)) *
                           (ceil_div(batch, kMfRows) + args.num_segments) +
                       items * kWsBuildCost;
  if (cost < wgs) wgs = static_cast<int>(cost);
  const dim3 grid(wgs > 0 ? wgs : 1, 1, nproj);
  if (units == 2) {
    hipLaunchKernelGGL((grouped_mfma_ws_kernel<2, kWsSub>), grid, dim3(2 * kMfThreads), lds, s, args);
  } else {
    hipLaunchKernelGGL((grouped_mfma_ws_kernel<1, kWsSub>), grid, dim3(kMfThreads), lds, s, args);
  }
  return check_launch(who);
}

static bool ws_fits(const tris_compact3_payload* p) {
  return p->rank <= kMfChunk && p->qweight2_sparse_rows <= kWsSalWindows && !p->has_output_scale && !p->has_bias;
}

int launch_grouped_mfma(const uint16_t* hidden_a, const uint16_t* hidden_b, int batch, const int32_t* expert_ids,
                        const int32_t* segment_offsets, int num_segments, const int32_t* decoded_a,
                        const int32_t* decoded_b, const tris_compact3_payload* pa, const tris_compact3_payload* pb,
                        uint16_t* out_a, uint16_t* out_b, bool swiglu, void* stream, const char* who,
                        const int64_t* row_index, int hidden_rows, bool decoded_by_expert, const float* partials,
                        int slices, uint16_t* comb_out, const int32_t* comb_inv, const uint16_t* comb_w,
                        bool comb_bf16) {
  TRIS_REQUIRE(batch >= 0 && num_segments >= 0, "%s: negative batch or segment count", who);
  TRIS_REQUIRE(row_index == nullptr || hidden_rows >= 0, "%s: negative hidden row count", who);
  int rc = check_payload(pa, false, who);
  if (rc) return rc;
  if (pb) {
    rc = check_payload(pb, false, who);
    if (rc) return rc;
  }
  TRIS_REQUIRE(!swiglu || pb != nullptr, "%s: the fused SwiGLU needs two projections", who);
  TRIS_REQUIRE(!pa->has_output_scale && !pa->has_bias && (!pb || (!pb->has_output_scale && !pb->has_bias)),
               "%s: the MFMA GEMM applies no output scale or bias", who);
  if (batch == 0 || num_segments == 0) return TRIS_OK;
  TRIS_REQUIRE((hidden_a || partials) && out_a && expert_ids && segment_offsets && decoded_a, "%s: null pointer", who);
  if (comb_out != nullptr) {
    // one token routed to two experts: two rows, two segments, one projection
    TRIS_REQUIRE(pb == nullptr && !swiglu && row_index == nullptr && comb_inv && comb_w,
                 "%s: the one-token combine takes one projection and the route's picks", who);
    TRIS_REQUIRE(batch == 2 && num_segments == 2, "%s: the one-token combine takes 2 rows in 2 segments", who);
  }
  if (partials != nullptr) {
    // one projection, one chunk, every slice's rows addressed by 32-bit buffer offsets
    TRIS_REQUIRE(pb == nullptr && !swiglu && row_index == nullptr, "%s: partial sums feed one projection", who);
    TRIS_REQUIRE(pa->rank <= kMfChunk, "%s: partial sums need rank <= %d (one chunk)", who, kMfChunk);
    TRIS_REQUIRE(slices >= 1 && hidden_rows >= batch, "%s: bad partial-sum shape", who);
    TRIS_REQUIRE(batch <= 4, "%s: partial sums take at most 4 rows (%d given)", who, batch);
    TRIS_REQUIRE(static_cast<int64_t>(slices) * hidden_rows * pa->rank * 4 < (int64_t{1} << 31),
                 "%s: partial sums exceed the 2 GiB limit", who);
  }
  TRIS_REQUIRE(!pb || (hidden_b && decoded_b && (swiglu || out_b)), "%s: null pointer (second projection)", who);
  int max_n = 0;
  for (int i = 0; i < (pb ? 2 : 1); ++i) {
    const tris_compact3_payload* p = i ? pb : pa;
    TRIS_REQUIRE(p->num_experts > 0 && p->rank > 0 && p->outfeatures > 0, "%s: empty payload", who);
    max_n = p->outfeatures > max_n ? p->outfeatures : max_n;
  }
  TRIS_REQUIRE(!swiglu || (pa->outfeatures == pb->outfeatures && pa->num_experts == pb->num_experts &&
                           pa->rank == pb->rank),
               "%s: gate and up projections differ in shape", who);
  if (row_index != nullptr) {
    // gathered rows: one 32-bit buffer offset spans every hidden row
    const int64_t bytes = static_cast<int64_t>(hidden_rows) * (pb && pb->rank > pa->rank ? pb->rank : pa->rank) * 2;
    TRIS_REQUIRE(bytes < (int64_t{1} << 31), "%s: %d hidden rows exceed the 2 GiB activation limit", who,
                 hidden_rows);
  }
  MfmaArgs args{};
  args.proj[0] = MfmaProj{hidden_a, out_a, decoded_a, *pa, row_index, hidden_rows, partials, slices};
  if (pb) args.proj[1] = MfmaProj{hidden_b, out_b, decoded_b, *pb, row_index, hidden_rows};
  args.expert_ids = expert_ids;
  args.segment_offsets = segment_offsets;
  args.num_segments = num_segments;
  args.decoded_by_expert = decoded_by_expert ? 1 : 0;
  if (comb_out != nullptr) {  // both units run the one projection, on row tiles 0 and 1
    args.proj[1] = args.proj[0];
    args.comb_out = comb_out;
    args.comb_inv = comb_inv;
    args.comb_w = comb_w;
    args.comb_bf16 = comb_bf16 ? 1 : 0;
  }
  const int units = (swiglu || comb_out != nullptr) ? 2 : 1;
  const int nproj = (pb && !swiglu) ? 2 : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // long segments: keep each output tile's weights in registers and stream the segment's rows through them
  // (its buffer resources address a segment's rows in 32-bit byte offsets: the whole batch must stay below 2 GiB)
  if (partials == nullptr && num_segments <= kWave &&
      static_cast<int64_t>(batch) >= static_cast<int64_t>(kWsMinRows) * num_segments &&
      ws_fits(pa) && (!pb || ws_fits(pb)) && static_cast<int64_t>(batch) * max_n * 2 < (int64_t{1} << 31) &&
      static_cast<int64_t>(batch) * kMfChunk * 2 < (int64_t{1} << 31)) {
    return launch_grouped_mfma_ws(args, units, nproj, max_n, batch, s, who);
  }
  const int rows = batch <= 4 ? 4 : kMfRows;  // staged activation rows: a row tile has at most min(16, batch)
  // the compact LDS layout (four workgroups per CU): at most 4 row-scale groups and 64 salient columns per expert,
  // and rank <= 256, where a tile's work is short enough that the fourth workgroup's latency hiding pays (at
  // rank 512 the 128-register cap and the coarser tile split cost more: measured on MI355X, OLMoE T=16 77 -> 73 us,
  // Mixtral T=16 92.9 -> 95.5 us)
  const auto compact_ok = [](const tris_compact3_payload* p) {
    return p->num_groups <= mf_groups_cap(true) && p->qweight2_sparse_rows * kMfSalWin <= mf_sal_slots(true) &&
           p->rank <= kMfChunk / 2;
  };
  const bool compact = compact_ok(pa) && (!pb || compact_ok(pb));
  const int lds_total = mf_static_lds_bytes(units, rows, compact);
  TRIS_REQUIRE(lds_total <= 160 * 1024, "%s: LDS request %d exceeds a CU", who, lds_total);
  // Workgroups: as many as the GPU holds at once (LDS and the kernel's 128 VGPRs per lane, 4 wavefronts
  // per SIMD for one unit, bound them), shared by the projections of an unfused pair.
  int wgs_per_cu = (160 * 1024) / lds_total;
  const int by_regs = units == 1 ? 4 : 1;
  wgs_per_cu = wgs_per_cu < by_regs ? wgs_per_cu : by_regs;
  wgs_per_cu = wgs_per_cu > 0 ? wgs_per_cu : 1;
  int wgs = (kMfCus * wgs_per_cu) / nproj;
  // no more than the (row tile, output tile) pairs there can be: row tiles <= batch / 16 + min(segments, batch)
  const int64_t pairs =
      (static_cast<int64_t>(batch) / kMfRows + (num_segments < batch ? num_segments : batch)) * ceil_div(max_n, kTileOut);
  if (pairs < wgs) wgs = static_cast<int>(pairs);
  if (comb_out != nullptr && ceil_div(max_n, kTileOut) < wgs) wgs = ceil_div(max_n, kTileOut);  // output tiles only
  const dim3 grid(wgs > 0 ? wgs : 1, 1, nproj);
  const dim3 block(units * kMfThreads);
#define TRIS_MF_LAUNCH(U, ROWS, C) hipLaunchKernelGGL((grouped_mfma_kernel<U, ROWS, C>), grid, block, 0, s, args)
  if (units == 2) {
    if (rows == 4) {
      if (compact) TRIS_MF_LAUNCH(2, 4, true); else TRIS_MF_LAUNCH(2, 4, false);
    } else {
      if (compact) TRIS_MF_LAUNCH(2, kMfRows, true); else TRIS_MF_LAUNCH(2, kMfRows, false);
    }
  } else {
    if (rows == 4) {
      if (compact) TRIS_MF_LAUNCH(1, 4, true); else TRIS_MF_LAUNCH(1, 4, false);
    } else {
      if (compact) TRIS_MF_LAUNCH(1, kMfRows, true); else TRIS_MF_LAUNCH(1, kMfRows, false);
    }
  }
#undef TRIS_MF_LAUNCH
  return check_launch(who);
}

// True when the MFMA kernel can run this payload: uniform 64-column groups (so
// a 64-column K tile has one row scale) and a rank that is a whole number of
// 64-column tiles, with 16-byte aligned activations (8-column loads).
bool grouped_mfma_supported(const tris_compact3_payload* p, const uint16_t* hidden) {
  if (p == nullptr || !p->use_uniform_k64_groups || p->rank <= 0 || p->rank % kTileK != 0 ||
      p->num_groups < 1 || p->num_groups > kMfMaxGroups || reinterpret_cast<uintptr_t>(hidden) % 16 != 0) {
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
