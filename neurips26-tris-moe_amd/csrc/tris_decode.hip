// Grouped compact3 expert GEMM for decode-sized segments with the block-GR split bitmap decoded inside the
// kernel: the compressed words are read from HBM once per output tile and expanded in LDS, and no decoded
// bitmap or weight ever goes back to memory (TriSMoE_cuda_kernel.cu:5382-5586 and 6313-7716 decode inside
// the CTA as well, one thread per block).
//
// Arithmetic.  Every weight is the reference's exact fp16 value (kernel.cu:665-774): non-salient
// w = s1 * fp16(C_j[k] * R_j[n,g]) with j = d where the split bit is set, else nd; salient
// w = fp16(+-fp16(C0 * R0) +- fp16(C1 * R1)).  Products with the activations are exact in fp32 on MFMA
// (v_mfma_f32_16x16x32_f16) and accumulate in fp32; the epilogue applies the optional output scale and
// bias in fp32 and rounds once (kernel.cu:5588-5626).
//
// Decomposition.  A workgroup is two units of four wavefronts; an item is one row tile (<= 16 rows of one
// segment) and one 64-column output tile per unit.  In the SwiGLU and pair modes the two units are the gate
// and up projections of the same tile; in the single mode they are tiles ob and ob + 1 of one projection.
// Inside a unit the K dimension is split four ways: wavefront w owns packed rows [w*P, (w+1)*P) (P = rank /
// 128, so whole GR blocks) and
//   * decodes its own P / 2 GR blocks of the tile into a private LDS bitmap (the span decoder, 32 lanes per
//     block), so no other wavefront waits for them;
//   * keeps the column factors C_d, C_nd of its K slice in registers for as long as the expert stays the
//     same (salient columns zeroed);
//   * builds the B operand of each 16-column strip and packed row from lookup tables indexed by one byte of
//     the sign word and of the split word (lane group kg takes columns 8kg..8kg+7 of a packed row, the
//     natural order, so its A operand is 16 contiguous bytes of an activation row): per pair of weights
//     c = C_j, r = R_j selected by the split mask (v_bfi), one packed fp16 multiply, one sign xor;
//   * writes the exact weights of its salient columns (a few per slice) into an LDS table and adds them
//     with one more MFMA per strip and window of 32;
//   * hands its fp32 partial tiles to the unit through LDS, where they are added in wavefront order.
// Workgroups are persistent and take contiguous runs of items, so consecutive items share an expert.
#include "tris_common.h"
#include "tris_gr_span.h"

namespace tris {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kDcUnitWaves = 4;
constexpr int kDcWaves = 2 * kDcUnitWaves;
constexpr int kDcThreads = kDcWaves * kWave;
constexpr int kDcRows = 16;                     // rows per item (one MFMA row block)
constexpr int kDcMaxPrw = 4;                    // packed rows per wavefront: rank <= 512
constexpr int kDcMaxBlocks = kDcMaxPrw / 2;     // GR blocks per wavefront and item
constexpr int kDcSalWin = 32;                   // salient columns per MFMA window
constexpr int kDcSpan = 32;                     // span decoder lanes per block
constexpr int kDcStrips = kTileOut / 16;        // 16-column strips of an output tile
constexpr int kDcRedStride = kTileOut + 4;      // partial-tile row stride: the four row groups of an MFMA
                                                // result land in different LDS banks
constexpr int kDcWgsPerCu = 2;                  // <= 128 VGPRs and < 80 KB of LDS: two workgroups per CU

enum DcMode { kDcSingle = 0, kDcPair = 1, kDcSwiglu = 2 };

// Byte-indexed operand tables.  For byte b of a packed word (the 8 columns of one lane group), word i covers
// the columns 2i (low half) and 2i + 1 (high half):
//   sign[b][i]: 0x8000 in a half whose qweight1 bit is clear (negative weight);
//   gmask[b][i]: 0xFFFF in a half whose split bit is set (the d factors).
struct alignas(16) DcLuts {
  uint32_t sign[256][4];
  uint32_t gmask[256][4];
};

constexpr DcLuts dc_make_luts() {
  DcLuts t{};
  for (int b = 0; b < 256; ++b) {
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (static_cast<uint32_t>(b) >> (2 * i)) & 1u;
      const uint32_t hi = (static_cast<uint32_t>(b) >> (2 * i + 1)) & 1u;
      t.sign[b][i] = (lo ? 0u : 0x8000u) | (hi ? 0u : 0x80000000u);
      t.gmask[b][i] = (lo ? 0xFFFFu : 0u) | (hi ? 0xFFFF0000u : 0u);
    }
  }
  return t;
}

__constant__ DcLuts kDcLuts = dc_make_luts();

struct DcProj {
  const uint16_t* hidden;  // fp16 [hidden_rows, rank]
  uint16_t* out;           // fp16 [batch, N] (pair mode: this projection's output)
  tris_compact3_payload p;
};

struct DcArgs {
  DcProj proj[2];
  const int64_t* row_index;  // [batch]: hidden row of grouped row r (null: r itself)
  const int32_t* expert_ids;
  const int32_t* segment_offsets;
  int num_segments;
  int hidden_rows;
  int mode;
};

// A wavefront's per-item operands, loaded into LDS while its GR blocks are decoded: for every tile column,
// the sign words of the wavefront's packed rows, the row scales of each 64-column K tile's group (d | nd << 16
// and 0 | 1 << 16), and the two qweight2_sparse rows of the slice's first salient window.
struct DcStage {
  uint32_t qw[kDcMaxPrw][kTileOut];
  uint32_t rdn[kDcMaxBlocks][kTileOut];
  uint32_t r01[kDcMaxBlocks][kTileOut];
  uint32_t q2[2][kTileOut];
};

constexpr uint32_t kDcRsrcWord3 = 0x00020000;  // raw buffer resource, gfx9 family

// Every caller passes wave-uniform values; reading them back from the first lane lets the compiler keep the
// resource in scalar registers (a resource it cannot prove uniform costs a waterfall loop per load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dc_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32)));
  const int n = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  void* ub = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, n, kDcRsrcWord3);
}
// Raw buffer loads: an offset at or past the buffer's size reads 0 without touching memory.
__device__ __forceinline__ uint32_t dc_load32(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0u, 0);
}
__device__ __forceinline__ uint2 dc_load64(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0u, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint4 dc_load128(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0u, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Buffer loads straight into LDS: lane l's 4 (16) bytes land at dst + 4l (16l); dst is wave-uniform.  An
// offset past the buffer writes 0.  The wavefront waits for them (vmcnt) before reading dst.
__device__ __forceinline__ void dc_dma32(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, 0, 0, 0);
}
__device__ __forceinline__ void dc_dma128(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}
constexpr int kDcVmcnt0 = 0x0F70;  // s_waitcnt vmcnt(0), other counters untouched

__device__ __forceinline__ f16x2 dc_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t dc_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Row tiles (<= kDcRows rows of one segment) of every segment, scanned by one wavefront; the same values
// in every lane.  Segment s's tiles are [first(s), first(s) + tiles(s)).
struct DcScan {
  int total;
};

__device__ inline int dc_count_tiles(const int32_t* __restrict__ seg, int nseg) {
  const int lane = static_cast<int>(__lane_id());
  int total = 0;
  for (int c = 0; c < nseg; c += kWave) {
    const int i = c + lane;
    int t = 0;
    if (i < nseg) {
      const int len = seg[i + 1] - seg[i];
      t = len > 0 ? (len + kDcRows - 1) / kDcRows : 0;
    }
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) t += __shfl_xor(t, d);
    total += t;
  }
  return total;
}

// Row tile `tile` -> segment, first row, row count and expert id (wave-uniform results).
__device__ inline void dc_map_tile(const int32_t* __restrict__ seg, const int32_t* __restrict__ expert_ids, int nseg,
                                   int tile, int* s_out, int* row0_out, int* rc_out, int* e_out) {
  const int lane = static_cast<int>(__lane_id());
  int base = 0;
  for (int c = 0; c < nseg; c += kWave) {
    const int i = c + lane;
    const int ic = i < nseg ? i : nseg - 1;
    const int lo = seg[ic];
    const int hi = seg[ic + 1];
    const int ex = expert_ids[ic];
    int t = 0;
    if (i < nseg) t = hi > lo ? (hi - lo + kDcRows - 1) / kDcRows : 0;
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
      const int local = tile - base - __shfl(incl - t, L);
      const int row0 = __shfl(lo, L) + local * kDcRows;
      const int end = __shfl(hi, L);
      *s_out = c + L;
      *row0_out = row0;
      *rc_out = (end - row0) < kDcRows ? (end - row0) : kDcRows;
      *e_out = __shfl(ex, L);
      return;
    }
    base += total;
  }
  *s_out = 0;
  *row0_out = 0;
  *rc_out = 0;
  *e_out = -1;
}

// B operand of one packed row and strip: the 8 exact weights of column n, rows 8kg..8kg+7 of the packed row.
__device__ __forceinline__ f16x8 dc_b_operand(const DcLuts* __restrict__ lut, uint32_t qw, uint32_t gw, uint32_t kshift,
                                              const uint32_t cd[4], const uint32_t cn[4], uint32_t rd2, uint32_t rn2) {
  const uint32_t qb = (qw >> kshift) & 0xFFu;
  const uint32_t gb = (gw >> kshift) & 0xFFu;
  const uint4 sm = *reinterpret_cast<const uint4*>(lut->sign[qb]);
  const uint4 gm = *reinterpret_cast<const uint4*>(lut->gmask[gb]);
  const uint32_t s[4] = {sm.x, sm.y, sm.z, sm.w};
  const uint32_t g[4] = {gm.x, gm.y, gm.z, gm.w};
  uint32_t b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = (g[i] & cd[i]) | (~g[i] & cn[i]);
    const uint32_t r = (g[i] & rd2) | (~g[i] & rn2);
    b[i] = dc_u32(dc_h2(c) * dc_h2(r)) ^ s[i];
  }
  return __builtin_bit_cast(f16x8, make_uint4(b[0], b[1], b[2], b[3]));
}

// Per-wavefront state that depends only on the expert (and the wavefront's K slice).
struct DcExpert {
  int e;                           // expert whose data the registers hold (-1: none)
  int grp[kDcMaxBlocks];           // row-scale group of each of the slice's 64-column K tiles (-1: none)
  int sal_lane[2];                 // slice-relative column of salient slot lane / lane + 64 (-1: none)
  uint32_t sal_c01[2];             // C0 | C1 << 16 of those columns
  int nsal;                        // salient columns in the slice
  int sbase;                       // salient index (qweight2_sparse order) of the slice's first salient column
};

__device__ inline void dc_load_expert(const tris_compact3_payload& p, int e, int wu, int prw, DcExpert& X) {
  const int lane = static_cast<int>(__lane_id());
  const int rank = p.rank;
  const int packed_rows = rank / 32;
  const int pr0 = wu * prw;
  const int32_t* cmap = p.c_map + static_cast<int64_t>(e) * packed_rows;
  X.e = e;
  // groups of the slice's K tiles (one group per 64-column tile: the uniform-K64 case)
  const int32_t* gidx = p.g_idx + static_cast<int64_t>(e) * rank;
#pragma unroll
  for (int t = 0; t < kDcMaxBlocks; ++t) {
    int g = -1;
    if (2 * t < prw) {
      g = gidx[(pr0 + 2 * t) * 32];
      if (g < 0 || g >= p.num_groups) g = -1;
    }
    X.grp[t] = __builtin_amdgcn_readfirstlane(g);
  }
  // salient columns of the slice: lane q holds the q-th one (chunk-relative k)
  const int32_t* q2p = p.qweight2_sparse_prefix + static_cast<int64_t>(e) * (packed_rows + 1);
  X.sbase = __builtin_amdgcn_readfirstlane(q2p[pr0]);
  int before = 0;
  int mine[2] = {-1, -1};
  for (int j = 0; j < prw; ++j) {
    const uint32_t cm = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(cmap[pr0 + j]));
    const int cnt = __popc(cm);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int slot = lane + kWave * h;
      if (slot >= before && slot < before + cnt) {
        // the (slot - before)-th set bit of cm
        uint32_t m = cm;
        for (int q = 0; q < slot - before; ++q) m &= m - 1u;
        mine[h] = j * 32 + __builtin_ctz(m);
      }
    }
    before += cnt;
  }
  X.nsal = before;  // <= prw * 32 <= 128
  X.sal_lane[0] = mine[0];
  X.sal_lane[1] = mine[1];
  const __amdgpu_buffer_rsrc_t r_col =
      dc_rsrc(p.col_pack3 + static_cast<int64_t>(e) * rank, static_cast<uint32_t>(rank) * 8u);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    X.sal_c01[h] = dc_load64(r_col, mine[h] >= 0 ? static_cast<uint32_t>(pr0 * 32 + mine[h]) * 8u : 0xFFFFFFF0u).x;
  }
}

// Slice-relative column of salient slot q (any lane's q < 128).
__device__ __forceinline__ int dc_sal_col(const DcExpert& X, int q) {
  const int a = __shfl(X.sal_lane[0], q & 63);
  const int b = __shfl(X.sal_lane[1], q & 63);
  return q < kWave ? a : b;
}

// Salient A operand of window w: lane (row i16, kg) holds the activations of slots w*32 + 8kg .. + 8 of its row
// (zero past the slice's salient columns and for rows past the tile).  r_h covers the whole activation tensor;
// hoff is the byte offset of the lane's row (0xFFFFFFF0 past the tile: reads 0).
__device__ __forceinline__ f16x8 dc_sal_a(const DcExpert& X, __amdgpu_buffer_rsrc_t r_h, uint32_t hoff, int slice0,
                                          int w, int kg) {
  uint32_t h[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int slot0 = w * kDcSalWin + 8 * kg + 2 * q;
    const int k0 = dc_sal_col(X, slot0);
    const int k1 = dc_sal_col(X, slot0 + 1);
    const bool rv = hoff != 0xFFFFFFF0u;
    const uint32_t lo = slot0 < X.nsal && rv
                            ? dc_load32(r_h, (hoff + static_cast<uint32_t>(slice0 + k0) * 2u) & ~3u) >> (16 * (k0 & 1))
                            : 0u;
    const uint32_t hi = slot0 + 1 < X.nsal && rv
                            ? dc_load32(r_h, (hoff + static_cast<uint32_t>(slice0 + k1) * 2u) & ~3u) >> (16 * (k1 & 1))
                            : 0u;
    h[q] = (lo & 0xFFFFu) | (hi << 16);
  }
  return __builtin_bit_cast(f16x8, make_uint4(h[0], h[1], h[2], h[3]));
}

// The unit's column factors C_d, C_nd of expert e (fp16, natural column order; zero at salient columns, so the
// main pass gives those columns zero weights) into cd / cn [rank].  All threads of the unit; a barrier follows.
__device__ inline void dc_stage_columns(const tris_compact3_payload& p, int e, int utid, uint16_t* cd, uint16_t* cn) {
  const int rank = p.rank;
  const int packed_rows = rank / 32;
  const __amdgpu_buffer_rsrc_t r_col =
      dc_rsrc(p.col_pack3 + static_cast<int64_t>(e) * rank, static_cast<uint32_t>(rank) * 8u);
  const int32_t* cmap = p.c_map + static_cast<int64_t>(e) * packed_rows;
  for (int k = utid; k < rank; k += kDcUnitWaves * kWave) {
    const uint32_t hi = dc_load64(r_col, static_cast<uint32_t>(k) * 8u).y;  // C_d | C_nd << 16
    const bool sal = (static_cast<uint32_t>(cmap[k >> 5]) >> (k & 31)) & 1u;
    cd[k] = sal ? static_cast<uint16_t>(0) : static_cast<uint16_t>(hi & 0xFFFFu);
    cn[k] = sal ? static_cast<uint16_t>(0) : static_cast<uint16_t>(hi >> 16);
  }
}

static_assert(sizeof(DcStage) <= sizeof(float) * kDcRows * kDcRedStride &&
                  sizeof(uint16_t) * kTileOut * kDcSalWin <= sizeof(float) * kDcRows * kDcRedStride,
              "the stage and the salient table share a wavefront's partial-tile slot");

// Salient table [64 tile columns][kDcSalWin slots] of fp16 weights.  The four 16-byte chunks of column c's
// row are stored XOR-swizzled by c / 4, so a 16-lane phase of the MFMA operand read, and the zeroing of the
// rows, touch 16 different bank groups.
__device__ __forceinline__ int dc_sal_index(int c, int q) { return c * kDcSalWin + ((((q >> 3) ^ (c >> 2)) & 3) << 3) + (q & 7); }

// Zero output for the rows of an item routed to no expert.
__device__ inline void dc_zero_rows(uint16_t* out, int N, int row0, int rc, int n0, int utid) {
  for (int idx = utid; idx < rc * kTileOut; idx += kDcUnitWaves * kWave) {
    const int n = n0 + idx % kTileOut;
    if (n < N) out[static_cast<int64_t>(row0 + idx / kTileOut) * N + n] = 0;
  }
}

// Workgroup barrier ordering LDS only: outstanding global loads and stores stay in flight across it (a full
// __syncthreads waits for them).
__device__ __forceinline__ void dc_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ __launch_bounds__(kDcThreads) __attribute__((amdgpu_waves_per_eu(kDcWgsPerCu * kDcWaves / 4))) void
grouped_decode_kernel(DcArgs a) {
  __shared__ GrTables tab;
  __shared__ GrTables4 tab4;
  __shared__ DcLuts lut;
  __shared__ __attribute__((aligned(16))) uint32_t bitmap[kDcWaves][kDcMaxBlocks][kGrBlockStride];
  // per wavefront, in turn: the item's stage (decode to salient), its salient table, its partial tile
  __shared__ __attribute__((aligned(16))) float red[kDcWaves][kDcRows][kDcRedStride];
  __shared__ __attribute__((aligned(16))) uint16_t cols[2][2][kDcMaxPrw * kDcUnitWaves * 32];  // [unit][d / nd][k]

  gr_tables_to_lds(&tab);
  gr_tables4_to_lds(&tab4);
  {
    const uint4* src = reinterpret_cast<const uint4*>(&kDcLuts);
    uint4* dst = reinterpret_cast<uint4*>(&lut);
    for (int i = threadIdx.x; i < static_cast<int>(sizeof(DcLuts) / 16); i += kDcThreads) dst[i] = src[i];
  }
  __syncthreads();

  int tid = static_cast<int>(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int unit = wave / kDcUnitWaves;
  const int wu = wave % kDcUnitWaves;  // K slice of the wavefront within its unit
  // lane-derived values; recomputed from an opaque copy of the thread index at each item, so the compiler
  // rebuilds the addresses that derive from them inside the loop instead of holding them in registers
  int lane = tid % kWave;
  int i16 = lane % 16;
  int kg = lane / 16;
  int utid = tid % (kDcUnitWaves * kWave);
  const bool two_proj = a.mode != kDcSingle;
  const DcProj& pj = a.proj[two_proj ? unit : 0];
  const tris_compact3_payload& p = pj.p;
  const int N = p.outfeatures;
  const int rank = p.rank;
  const int packed_rows = rank / 32;
  const int prw = packed_rows / kDcUnitWaves;  // 2 or 4
  const int nblk_w = prw / 2;                  // GR blocks per wavefront and item
  const int nob = ceil_div(N, kTileOut);
  const int nob_items = two_proj ? nob : ceil_div(nob, 2);
  const int nblk = (packed_rows / 2) * nob;

  const int row_tiles = dc_count_tiles(a.segment_offsets, a.num_segments);
  const int64_t total = static_cast<int64_t>(row_tiles) * nob_items;
  const int W = static_cast<int>(gridDim.x);
  const int it0 = static_cast<int>(total * blockIdx.x / W);
  const int it1 = static_cast<int>(total * (blockIdx.x + 1) / W);

  DcExpert X;
  X.e = -1;
  uint32_t* bm = &bitmap[wave][0][0];
  DcStage& stg = *reinterpret_cast<DcStage*>(&red[wave][0][0]);
  uint32_t kshift = 8u * static_cast<uint32_t>(kg);
  int cur_rt = -1, s = 0, row0 = 0, rc = 0, e = -1;
  // the activations (wave-uniform resource); hoff: byte offset of the lane's row (0xFFFFFFF0: none)
  const __amdgpu_buffer_rsrc_t r_h =
      dc_rsrc(pj.hidden, static_cast<uint32_t>(static_cast<int64_t>(a.hidden_rows) * rank * 2));
  uint32_t hoff = 0xFFFFFFF0u;

  // GR blocks of the wavefront: block gb (lane group lane / 32) covers packed rows wu*prw + 2gb, + 1
  int gb = lane / kDcSpan;
  int gj = lane % kDcSpan;

  // An item's GR block as the span decoder sees it (header, then the lane's span words); the next item's is
  // loaded while this one is decoded and computed.
  struct ItemGr {
    int begin, word_count, meta, w0, nw;  // begin: the block's first word
    uint32_t w[GrSpan<kDcSpan>::kMaxWords];
  };
  // item index within its row tile -> the unit's output tile
  auto item_ob = [&](int obi) { return two_proj ? obi : 2 * obi + unit; };
  // GR header and span loads go through buffer resources over expert e's arrays and are issued whether or
  // not their item exists: an offset past the buffer reads 0 without touching memory, and no branch makes the
  // compiler wait for a load before its value is used.  The resources are rebuilt from the wave-uniform
  // expert id where they are used, so they stay in scalar registers.
  auto gr_header = [&](int obi, bool valid, ItemGr& G) {
    const __amdgpu_buffer_rsrc_t r_offs =
        dc_rsrc(p.q_gmap_gr_offsets + static_cast<int64_t>(e) * (nblk + 1), static_cast<uint32_t>(nblk + 1) * 4u);
    const __amdgpu_buffer_rsrc_t r_meta =
        dc_rsrc(p.q_gmap_gr_meta + static_cast<int64_t>(e) * nblk, static_cast<uint32_t>(nblk) * 4u);
    const int ob = item_ob(obi);
    const bool v = valid && ob < nob && gb < nblk_w;
    const uint32_t off = v ? static_cast<uint32_t>((wu * nblk_w + gb) * nob + ob) * 4u : 0xFFFFFFF0u;
    const int begin = static_cast<int>(dc_load32(r_offs, off));
    const int end = static_cast<int>(dc_load32(r_offs, off + 4u));
    G.begin = begin;
    G.word_count = end - begin;
    G.meta = static_cast<int>(dc_load32(r_meta, off));
  };
  auto gr_words = [&](ItemGr& G) {
    const __amdgpu_buffer_rsrc_t r_words = dc_rsrc(p.q_gmap_gr_words + static_cast<int64_t>(e) * p.gr_words_stride,
                                                   static_cast<uint32_t>(p.gr_words_stride) * 4u);
    const int wc = G.word_count;
    int w0 = 0, nw = 0;
    if (wc > 0 && wc <= kGrWords) {
      const int span = (wc + kDcSpan - 1) / kDcSpan;
      w0 = gj * span;
      const int rest = wc - w0;
      nw = rest < 0 ? 0 : (rest < span ? rest : span);
    }
    G.w0 = w0;
    G.nw = nw;
#pragma unroll
    for (int i = 0; i < GrSpan<kDcSpan>::kMaxWords; ++i) {
      G.w[i] = dc_load32(r_words, i < nw ? static_cast<uint32_t>(G.begin + w0 + i) * 4u : 0xFFFFFFF0u);
    }
  };

  ItemGr cur, nxt;
  bool have_next = false;
  // the current item's row tile and index within it, carried from item to item (no division per item)
  int rt = it0 / nob_items;
  int obi = it0 - rt * nob_items;
  const auto advance = [&]() {
    if (++obi == nob_items) {
      obi = 0;
      ++rt;
    }
  };
  for (int it = it0; it < it1; ++it, advance()) {
    asm volatile("" : "+v"(tid));
    lane = tid % kWave;
    i16 = lane % 16;
    kg = lane / 16;
    utid = tid % (kDcUnitWaves * kWave);
    kshift = 8u * static_cast<uint32_t>(kg);
    gb = lane / kDcSpan;
    gj = lane % kDcSpan;
    if (rt != cur_rt) {
      cur_rt = rt;
      have_next = false;
      dc_map_tile(a.segment_offsets, a.expert_ids, a.num_segments, rt, &s, &row0, &rc, &e);
      s = __builtin_amdgcn_readfirstlane(s);
      row0 = __builtin_amdgcn_readfirstlane(row0);
      rc = __builtin_amdgcn_readfirstlane(rc);
      e = __builtin_amdgcn_readfirstlane(e);
      if (e >= 0 && e < p.num_experts) {
        if (X.e != e) {
          dc_load_expert(p, e, wu, prw, X);
          dc_stage_columns(p, e, utid, cols[unit][0], cols[unit][1]);
          dc_lds_barrier();
        }
        // A operand rows of this row tile (rows past rc read zero)
        hoff = 0xFFFFFFF0u;
        if (i16 < rc) {
          int64_t hrow = a.row_index != nullptr ? a.row_index[row0 + i16] : row0 + i16;
          if (hrow < 0 || hrow >= a.hidden_rows) hrow = 0;
          hoff = static_cast<uint32_t>(hrow * rank * 2);
        }
      }
    }
    // wave-uniform tile state (loop-carried values the compiler cannot prove uniform otherwise)
    e = __builtin_amdgcn_readfirstlane(e);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    rc = __builtin_amdgcn_readfirstlane(rc);
    const int ob = item_ob(obi);
    const int n0 = ob * kTileOut;
    const bool unit_active = ob < nob;
    uint16_t* out = pj.out;
    if (e < 0 || e >= p.num_experts) {
      // rows routed to no expert: zero output (both outputs in pair mode, the unit's tile otherwise)
      if (unit_active && (a.mode != kDcSwiglu || unit == 0)) dc_zero_rows(out, N, row0, rc, n0, utid);
      continue;
    }
    if (have_next) {
      cur = nxt;
    } else {
      gr_header(obi, true, cur);
      gr_words(cur);
    }
    // the item's sign words, row scales and salient words into the wavefront's stage (landing during the decode)
    const int nsal = X.nsal;
    const int q2rows = p.qweight2_sparse_rows;
    {
      const __amdgpu_buffer_rsrc_t r_q1 =
          dc_rsrc(p.qweight1 + static_cast<int64_t>(e) * packed_rows * N, static_cast<uint32_t>(packed_rows) * N * 4u);
      const __amdgpu_buffer_rsrc_t r_rs = dc_rsrc(p.row_pack3 + static_cast<int64_t>(e) * N * p.num_groups,
                                                  static_cast<uint32_t>(N) * p.num_groups * 8u);
      const int nl = n0 + lane;
      const bool lv = unit_active && nl < N;
      if ((N & 3) == 0) {
        // lane (row lane / 16, columns 4 (lane % 16) ..): whole 16-byte chunks, none straddling N
        const int q = lane / 16;
        const int n = n0 + 4 * (lane % 16);
        dc_dma128(r_q1, &stg.qw[0][0],
                  unit_active && q < prw && n < N ? static_cast<uint32_t>((wu * prw + q) * N + n) * 4u : 0xFFFFFFF0u);
      } else {
#pragma unroll
        for (int j = 0; j < kDcMaxPrw; ++j) {
          dc_dma32(r_q1, &stg.qw[j][0], lv && j < prw ? static_cast<uint32_t>((wu * prw + j) * N + nl) * 4u : 0xFFFFFFF0u);
        }
      }
#pragma unroll
      for (int t = 0; t < kDcMaxBlocks; ++t) {
        const int g = X.grp[t];
        const uint32_t off = lv && g >= 0 ? static_cast<uint32_t>(nl * p.num_groups + g) * 8u : 0xFFFFFFF0u;
        dc_dma32(r_rs, &stg.rdn[t][0], off == 0xFFFFFFF0u ? off : off + 4u);
        if (nsal > 0) dc_dma32(r_rs, &stg.r01[t][0], off);
      }
      if (nsal > 0) {
        const __amdgpu_buffer_rsrc_t r_q2 = dc_rsrc(p.qweight2_sparse + static_cast<int64_t>(e) * q2rows * N,
                                                    static_cast<uint32_t>(q2rows) * N * 4u);
        const int sr0 = X.sbase >> 5;
        dc_dma32(r_q2, &stg.q2[0][0], lv && sr0 < q2rows ? static_cast<uint32_t>(sr0 * N + nl) * 4u : 0xFFFFFFF0u);
        dc_dma32(r_q2, &stg.q2[1][0], lv && sr0 + 1 < q2rows ? static_cast<uint32_t>((sr0 + 1) * N + nl) * 4u : 0xFFFFFFF0u);
      }
    }
    // the next item of the same row tile: its block header now, its words after this decode
    const int obi_next = obi + 1 < nob_items ? obi + 1 : 0;
    have_next = it + 1 < it1 && obi_next != 0;
    gr_header(obi_next, have_next, nxt);

    // ---- decode the wavefront's blocks into its LDS bitmap
    {
      GrSpan<kDcSpan> sp;
      const bool bvalid = unit_active && gb < nblk_w;
      sp.word_count = bvalid ? cur.word_count : 0;
      sp.payload = p.q_gmap_gr_words + static_cast<int64_t>(e) * p.gr_words_stride + cur.begin;
      sp.meta = cur.meta;
      sp.w0 = cur.w0;
      sp.nw = cur.nw;
#pragma unroll
      for (int i = 0; i < GrSpan<kDcSpan>::kMaxWords; ++i) sp.w[i] = cur.w[i];
      uint4* z = reinterpret_cast<uint4*>(bm);
      for (int q = lane; q < kDcMaxBlocks * kGrBlockStride / 4; q += kWave) z[q] = make_uint4(0u, 0u, 0u, 0u);
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      gr_decode_block_group<kDcSpan>(sp, &tab, bm + gb * kGrBlockStride + kGrPadFront, gj, &tab4);
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    // the stage has landed (and the next item's header, issued before the decode)
    __builtin_amdgcn_s_waitcnt(kDcVmcnt0);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    gr_words(nxt);

    // ---- main MFMA pass: per packed row of the slice, every strip.  A operand: row i16 of the row tile,
    // columns 32j + 8kg .. + 8 of the slice, read here each item (the row tile's activations stay in cache)
    f16x8 av[kDcMaxPrw];
#pragma unroll
    for (int j = 0; j < kDcMaxPrw; ++j) {
      const uint32_t off = hoff + static_cast<uint32_t>((wu * prw + j) * 32 + 8 * kg) * 2u;
      av[j] = __builtin_bit_cast(f16x8, dc_load128(r_h, j < prw && hoff != 0xFFFFFFF0u ? off : 0xFFFFFFF0u));
    }
    f32x4 acc[kDcStrips];
#pragma unroll
    for (int st = 0; st < kDcStrips; ++st) acc[st] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* ucd = cols[unit][0];
    const uint16_t* ucn = cols[unit][1];
#pragma unroll
    for (int j = 0; j < kDcMaxPrw; ++j) {
      if (j < prw) {
        const int kl = (wu * prw + j) * 32 + 8 * kg;
        const uint4 cdv = *reinterpret_cast<const uint4*>(&ucd[kl]);
        const uint4 cnv = *reinterpret_cast<const uint4*>(&ucn[kl]);
        const uint32_t cd[4] = {cdv.x, cdv.y, cdv.z, cdv.w};
        const uint32_t cn[4] = {cnv.x, cnv.y, cnv.z, cnv.w};
        const int t = j / 2;
#pragma unroll
        for (int st = 0; st < kDcStrips; ++st) {
          const uint32_t gw = bm[t * kGrBlockStride + kGrPadFront + (j & 1) * kTileOut + 16 * st + i16];
          const uint32_t r = stg.rdn[t][16 * st + i16];
          const uint32_t rd2 = (r & 0xFFFFu) * 0x00010001u;
          const uint32_t rn2 = (r >> 16) * 0x00010001u;
          const f16x8 bv = dc_b_operand(&lut, stg.qw[j][16 * st + i16], gw, kshift, cd, cn, rd2, rn2);
          acc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[j], bv, acc[st], 0, 0, 0);
        }
      }
    }

    // ---- salient columns: table of exact weights (lane = tile column), then one MFMA per strip and window
    if (nsal > 0) {
      uint16_t* sal_tab = reinterpret_cast<uint16_t*>(&red[wave][0][0]);  // [64 columns][kDcSalWin]
      const int nc = n0 + lane;
      const bool cv = unit_active && nc < N;
      const __amdgpu_buffer_rsrc_t r_q2 = dc_rsrc(p.qweight2_sparse + static_cast<int64_t>(e) * q2rows * N,
                                                  static_cast<uint32_t>(q2rows) * N * 4u);
      uint32_t q1c[kDcMaxPrw];
#pragma unroll
      for (int j = 0; j < kDcMaxPrw; ++j) q1c[j] = stg.qw[j][lane];
      const uint32_t r01[2] = {stg.r01[0][lane], stg.r01[kDcMaxBlocks - 1][lane]};
      uint32_t q2a = stg.q2[0][lane], q2b = stg.q2[1][lane];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the table overwrites the stage
      const int nwin = (nsal + kDcSalWin - 1) / kDcSalWin;
      uint4* trow = reinterpret_cast<uint4*>(&sal_tab[lane * kDcSalWin]);
      for (int w = 0; w < nwin; ++w) {
        const int wn = (nsal - w * kDcSalWin) < kDcSalWin ? (nsal - w * kDcSalWin) : kDcSalWin;
        const int r0 = (X.sbase + w * kDcSalWin) >> 5;
        if (w > 0) {
          q2a = dc_load32(r_q2, cv && r0 < q2rows ? static_cast<uint32_t>(r0 * N + nc) * 4u : 0xFFFFFFF0u);
          q2b = dc_load32(r_q2, cv && r0 + 1 < q2rows ? static_cast<uint32_t>((r0 + 1) * N + nc) * 4u : 0xFFFFFFF0u);
        }
#pragma unroll
        for (int z = 0; z < kDcSalWin / 8; ++z) trow[z] = make_uint4(0u, 0u, 0u, 0u);  // slots past wn stay zero
#pragma unroll 1
        for (int q = 0; q < wn; ++q) {
          const int slot = w * kDcSalWin + q;  // wave-uniform
          const int k = __builtin_amdgcn_readlane(slot < kWave ? X.sal_lane[0] : X.sal_lane[1], slot & 63);
          const uint32_t c01 = static_cast<uint32_t>(
              __builtin_amdgcn_readlane(static_cast<int>(slot < kWave ? X.sal_c01[0] : X.sal_c01[1]), slot & 63));
          const uint32_t rr = (k >> 6) == 0 ? r01[0] : r01[1];
          const int jr = k >> 5;
          const uint32_t w1 = jr == 0 ? q1c[0] : (jr == 1 ? q1c[1] : (jr == 2 ? q1c[2] : q1c[3]));
          const int sidx = X.sbase + slot;
          const uint32_t q2 = ((sidx >> 5) == r0) ? q2a : q2b;
          // signs: negative where the qweight1 / qweight2 bit is clear
          const uint32_t neg = ((~(w1 >> (k & 31)) & 1u) << 15) | ((~(q2 >> (sidx & 31)) & 1u) << 31);
          const f16x2 t = dc_h2(dc_u32(dc_h2(c01) * dc_h2(rr)) ^ neg);
          const _Float16 sum = t[0] + t[1];
          sal_tab[dc_sal_index(lane, q)] = __builtin_bit_cast(uint16_t, sum);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const f16x8 as = dc_sal_a(X, r_h, hoff, wu * prw * 32, w, kg);
#pragma unroll
        for (int st = 0; st < kDcStrips; ++st) {
          const f16x8 bs = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(
                                                          &sal_tab[dc_sal_index(16 * st + i16, 8 * kg)]));
          acc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as, bs, acc[st], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
      }
    }

    // ---- partial tiles to LDS (rows < rc), then the unit adds them in wavefront order
#pragma unroll
    for (int st = 0; st < kDcStrips; ++st) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = 4 * kg + v;
        if (r < rc) red[wave][r][16 * st + i16] = acc[st][v];
      }
    }
    dc_lds_barrier();
    if (a.mode == kDcSwiglu) {
      // both units' tile: out = fp16(silu(g) * u) with g, u each through its projection's epilogue
      const tris_compact3_payload& pg = a.proj[0].p;
      const tris_compact3_payload& pu = a.proj[1].p;
      for (int idx = tid; idx < rc * kTileOut; idx += kDcThreads) {
        const int r = idx / kTileOut;
        const int c = idx % kTileOut;
        const int n = n0 + c;
        if (n >= N) continue;
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int w = 0; w < kDcUnitWaves; ++w) {
          g += red[w][r][c];
          u += red[kDcUnitWaves + w][r][c];
        }
        const int64_t en = static_cast<int64_t>(e) * N + n;
        if (pg.has_output_scale) g *= h2f(pg.output_scale[en]);
        if (pg.has_bias) g += h2f(pg.bias[en]);
        if (pu.has_output_scale) u *= h2f(pu.output_scale[en]);
        if (pu.has_bias) u += h2f(pu.bias[en]);
        a.proj[0].out[static_cast<int64_t>(row0 + r) * N + n] = swiglu_bits(f2h_bits(g), f2h_bits(u));
      }
    } else if (unit_active) {
      // the unit's own tile (pair mode: its projection's output)
      for (int idx = utid; idx < rc * kTileOut; idx += kDcUnitWaves * kWave) {
        const int r = idx / kTileOut;
        const int c = idx % kTileOut;
        const int n = n0 + c;
        if (n >= N) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kDcUnitWaves; ++w) v += red[unit * kDcUnitWaves + w][r][c];
        const int64_t en = static_cast<int64_t>(e) * N + n;
        if (p.has_output_scale) v *= h2f(p.output_scale[en]);
        if (p.has_bias) v += h2f(p.bias[en]);
        out[static_cast<int64_t>(row0 + r) * N + n] = f2h_bits(v);
      }
    }
    dc_lds_barrier();  // the next item's stage overwrites the partial tiles
  }
}

}  // namespace tris

using namespace tris;

namespace {

constexpr int kDcCus = 256;          // MI355X compute units

// The decode kernel applies to one or two projections of one rank, rank a multiple of 256 up to 512 (whole GR
// blocks per wavefront), every 64-column K tile in one group, the GR stream present.
bool decode_supported(const tris_compact3_payload* p) {
  return p != nullptr && p->use_uniform_k64_groups && p->rank % 256 == 0 && p->rank <= 512 && p->rank > 0 &&
         p->q_gmap_gr_words != nullptr && p->q_gmap_gr_offsets != nullptr && p->q_gmap_gr_meta != nullptr &&
         p->num_groups > 0 && p->outfeatures > 0 && p->num_experts > 0;
}

int launch_decode(const uint16_t* hidden_a, const uint16_t* hidden_b, const int64_t* row_index, int32_t hidden_rows,
                  int32_t batch, const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments,
                  const tris_compact3_payload* pa, const tris_compact3_payload* pb, uint16_t* out_a, uint16_t* out_b,
                  int mode, void* stream, const char* who) {
  TRIS_REQUIRE(batch >= 0 && num_segments >= 0 && hidden_rows >= 0, "%s: negative shape", who);
  TRIS_REQUIRE(pa != nullptr && (mode == kDcSingle || pb != nullptr), "%s: null payload", who);
  TRIS_REQUIRE(decode_supported(pa) && (mode == kDcSingle || decode_supported(pb)),
               "%s: needs uniform 64-column groups, rank a multiple of 256 up to 512 and the GR stream", who);
  if (mode != kDcSingle) {
    TRIS_REQUIRE(pa->rank == pb->rank && pa->num_experts == pb->num_experts && pa->outfeatures == pb->outfeatures,
                 "%s: the two projections differ in shape", who);
  }
  if (batch == 0 || num_segments == 0) return TRIS_OK;
  TRIS_REQUIRE(hidden_a && out_a && expert_ids && segment_offsets && (mode == kDcSingle || hidden_b) &&
                   (mode != kDcPair || out_b),
               "%s: null pointer", who);
  TRIS_REQUIRE(reinterpret_cast<uintptr_t>(hidden_a) % 16 == 0 && reinterpret_cast<uintptr_t>(hidden_b) % 16 == 0,
               "%s: hidden rows must be 16-byte aligned", who);
  TRIS_REQUIRE(static_cast<int64_t>(hidden_rows) * pa->rank * 2 < 0xFFFFFFF0LL,
               "%s: activations too large for 32-bit offsets", who);
  TRIS_REQUIRE(static_cast<int64_t>(pa->num_experts) * ((pa->rank / 32) * pa->outfeatures) * 4 < (1LL << 32) &&
                   static_cast<int64_t>(pa->outfeatures) * pa->num_groups * 8 < (1LL << 32),
               "%s: payload too large for 32-bit offsets", who);
  DcArgs args{};
  args.proj[0] = DcProj{hidden_a, out_a, *pa};
  if (mode != kDcSingle) args.proj[1] = DcProj{hidden_b, mode == kDcPair ? out_b : out_a, *pb};
  args.row_index = row_index;
  args.expert_ids = expert_ids;
  args.segment_offsets = segment_offsets;
  args.num_segments = num_segments;
  args.hidden_rows = hidden_rows;
  args.mode = mode;
  // items: row tiles x output tiles; bound the row tiles by the rows and segments (no device sync)
  const int nob = ceil_div(pa->outfeatures, kTileOut);
  const int nob_items = mode == kDcSingle ? ceil_div(nob, 2) : nob;
  const int64_t tiles_bound = static_cast<int64_t>(batch) / kDcRows + (num_segments < batch ? num_segments : batch);
  int64_t grid = tiles_bound * nob_items;
  if (grid > kDcCus * kDcWgsPerCu) grid = kDcCus * kDcWgsPerCu;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(grouped_decode_kernel, dim3(static_cast<unsigned>(grid)), dim3(kDcThreads), 0,
                     static_cast<hipStream_t>(stream), args);
  return check_launch(who);
}

}  // namespace

extern "C" int tris_grouped_decode_forward_block_gr(const uint16_t* hidden, const int64_t* row_index,
                                                    int32_t hidden_rows, int32_t batch, const int32_t* expert_ids,
                                                    const int32_t* segment_offsets, int32_t num_segments,
                                                    const tris_compact3_payload* payload, uint16_t* output,
                                                    void* stream) {
  return launch_decode(hidden, nullptr, row_index, hidden_rows, batch, expert_ids, segment_offsets, num_segments,
                       payload, nullptr, output, nullptr, kDcSingle, stream, "tris_grouped_decode_forward_block_gr");
}

extern "C" int tris_grouped_decode_pair_forward_block_gr(
    const uint16_t* hidden_a, const uint16_t* hidden_b, const int64_t* row_index, int32_t hidden_rows, int32_t batch,
    const int32_t* expert_ids, const int32_t* segment_offsets, int32_t num_segments,
    const tris_compact3_payload* payload_a, const tris_compact3_payload* payload_b, uint16_t* output_a,
    uint16_t* output_b, int32_t swiglu, void* stream) {
  return launch_decode(hidden_a, hidden_b, row_index, hidden_rows, batch, expert_ids, segment_offsets, num_segments,
                       payload_a, payload_b, output_a, output_b, swiglu ? kDcSwiglu : kDcPair, stream,
                       "tris_grouped_decode_pair_forward_block_gr");
}
