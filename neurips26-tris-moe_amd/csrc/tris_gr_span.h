// Byte-table block-GR decoder: S lanes per block, each decoding a span of the
// block's codeword stream.
//
// Format (encoder qlinear_cuda.py:3763-3859, reference serial decoder
// TriSMoE_cuda_kernel.cu:403-479): each zero run before a one is Rice(k) coded
// as q = run >> k zero bits, a 1, then k remainder bits LSB first.  The flat
// position of the i-th one is F(end of codeword i) - 1, where F sums the
// contribution of every bit read so far: 2^k per unary zero, 1 per
// terminator, b * 2^j for remainder bit j.
//
// Decoding state at any bit is s in [0, k]: 0 = reading unary bits, s > 0 =
// s remainder bits still to read.  For k in {1, 2} two tables describe one
// byte of stream:
//   next[k][byte]       four bytes, byte s = the state after the byte from
//                       entry state s (identity above k).  A map of states in
//                       this form is a v_perm_b32 selector: composing maps,
//                       and stepping a state held in all four bytes, is one
//                       v_perm_b32;
//   entry[k][s][byte]   64 bits: the low word holds the completed ones' bit
//                       mask (bit i = a one at F(byte start) - 1 + i; a
//                       codeword entered mid-remainder whose last bits are
//                       zero ends at bit 0); the high word holds the F advance
//                       (bits 0..6) and the number of completed codewords
//                       (bits 12..15), so a lane's sum of high words holds its
//                       advance and count sums.
// Each lane of the block's group of S lanes:
//   A. reads next[] for every byte of its span (loads that do not wait on
//      each other) and composes them into its exit-state map;
//   B. learns its true entry state from a log-step scan that composes the
//      maps of the lanes before it;
//   C. walks its bytes from the true state with one v_perm_b32 per byte, so
//      every entry[] load is independent of the others, sums the F advances
//      and codeword counts (a packed segmented prefix sum gives its starting F
//      and the block's count), and ORs each byte's mask into the block's LDS
//      bitmap at its F.
// The bitmap has zero pad words before and after it: a one at a position
// past 4095 lands in the back pads (the reference stops there), and the
// decode falls back to the serial rules.  k = 0 streams are the bitmap itself
// (each codeword is run zeros then a one) and are copied.  Raw blocks are
// copied.
//
// For k in [3, 7] a codeword spans at least 4 bits, so a nibble completes at
// most one, and nibble tables (GrTables4, 2.9 KB; byte tables for these k
// would take 50 KB) describe the stream: per (k, nibble) the exit map over up
// to 8 states (two v_perm_b32 selector words, and the same map in 3-bit
// fields), per (k, s, nibble) the F advance, the completion and its F offset.
// The phases are those above, a nibble at a time: A composes the maps; C
// reads a word's packed maps, steps the state through them, reads the word's
// entries, and keeps each completion's F offset from the lane's start as a
// 16-bit half; after the group prefix sum the emission sets each completed
// codeword's bit with an LDS atomic OR.  Positions increase along the stream,
// so dropping those past 4095 is what the reference's early stop does.
// Callers without the nibble tables decode k in [3, 7] a word at a time with
// the word walks of tris_gr_decode.h: the word's exit map over the k + 1
// entry states, the same scan, then count-trailing-zeros walks from the true
// state.
//
// k > 7, streams longer than 128 words (the encoder stores those raw), and
// any stream whose completed codewords do not equal one_count (or, for
// k <= 2, reach past bit 4095) are decoded by the group's first lane with the
// reference's serial rules, so every input decodes as the reference decodes
// it.
#pragma once

#include "tris_common.h"
#include "tris_gr_decode.h"

namespace tris {

constexpr int kGrEntryStates = 2 + 3;                         // k = 1, 2; s in [0, k]
constexpr int kGrEntries = kGrEntryStates * 256 + 1;             // + one all-zero entry
constexpr uint32_t kGrZeroEntryOffset = kGrEntryStates * 256 * 8;  // byte offset of the zero entry
constexpr uint32_t kGrIdentityNext = 0x03020100u;               // byte s = s

// Decoded-block layout in LDS: four pad words, the 128 bitmap words, eight pad words.  The emission writes the
// word before the bitmap and up to three words after it.  Rows stay 16-byte aligned, and the 140-word stride
// puts the bitmaps of neighbouring blocks 12 banks apart.
constexpr int kGrPadFront = 4;
constexpr int kGrPadBack = 8;
constexpr int kGrBlockStride = kGrPadFront + kGrWords + kGrPadBack;

__host__ __device__ constexpr int gr_entry_base(int k) { return k == 1 ? 0 : 512; }

struct GrByteStep {
  uint32_t state;
  uint32_t count;
  uint32_t advance;
  uint64_t mask;
};

// Reading one byte (LSB first) of a Rice(k) stream from state st, 1 <= k <= 3 (the tables hold k <= 2).
// A completion needs k + 1 of the byte's bits after at most 7 - k zeros, so
// mask bits stay below (8 - k) * 2^k + 1 <= 41 and advance <= 8 * 2^k <= 64.
__host__ __device__ constexpr GrByteStep gr_byte_step(int k, int st, int byte) {
  uint32_t f = 0, n = 0;
  uint64_t mask = 0;
  for (int i = 0; i < 8; ++i) {
    const uint32_t b = (static_cast<uint32_t>(byte) >> i) & 1u;
    if (st == 0) {
      if (b == 0) {
        f += 1u << k;
      } else {
        f += 1u;
        st = k;
      }
    } else {
      f += b << (k - st);
      --st;
      if (st == 0) {
        mask |= 1ull << f;
        ++n;
      }
    }
  }
  return GrByteStep{static_cast<uint32_t>(st), n, f, mask};
}

struct alignas(16) GrTables {
  uint64_t entry[kGrEntries + 1];  // (k, s, byte); then the zero entry and one pad entry
  uint32_t next[2 * 256];          // (k, byte)
};

constexpr GrTables gr_make_tables() {
  GrTables t{};
  for (int k = 1; k <= 2; ++k) {
    for (int byte = 0; byte < 256; ++byte) {
      uint32_t fields = 0;
      for (int s = 0; s < 4; ++s) {
        uint32_t nx = static_cast<uint32_t>(s);
        if (s <= k) {
          const GrByteStep r = gr_byte_step(k, s, byte);
          nx = r.state;
          const uint32_t hi = r.advance | (r.count << 12) | (static_cast<uint32_t>(r.mask >> 32) << 23);
          t.entry[gr_entry_base(k) + s * 256 + byte] = (r.mask & 0xFFFFFFFFull) | (static_cast<uint64_t>(hi) << 32);
        }
        fields |= nx << (8 * s);
      }
      t.next[(k - 1) * 256 + byte] = fields;
    }
  }
  return t;
}

__constant__ GrTables kGrTables = gr_make_tables();
constexpr int kGrTableVec4 = static_cast<int>(sizeof(GrTables) / 16);
static_assert(sizeof(GrTables) % 16 == 0, "GrTables is copied as 16-byte vectors");

// Copy the tables into LDS (all threads of the workgroup; a barrier must follow).
__device__ inline void gr_tables_to_lds(GrTables* dst) {
  const uint4* src = reinterpret_cast<const uint4*>(&kGrTables);
  uint4* d = reinterpret_cast<uint4*>(dst);
  for (int i = threadIdx.x; i < kGrTableVec4; i += blockDim.x) d[i] = src[i];
}

// ---- Rice k in [3, 7], a nibble at a time.  A codeword spans at least 4 bits, so a nibble completes at most
// one: from an entry state s <= 4 at its bit s - 1, and the bits after it cannot hold a whole codeword (from state
// 0 only k = 3 completes, at bit 3).  Per (k, nibble) the exit map of the 8 states; per (k, s, nibble) the F
// advance (<= 4 * 2^7), the completion and its F offset from the nibble start (<= 2^k).
constexpr int kGrNibK0 = 3;
constexpr int kGrNibStates = 4 + 5 + 6 + 7 + 8;   // k = 3..7; s in [0, k]
constexpr int kGrNibZero = kGrNibStates * 16;      // index of the all-zero entry (nibbles past a span)

__host__ __device__ constexpr int gr_nib_entry_base(int k) {
  return k == 3 ? 0 : (k == 4 ? 64 : (k == 5 ? 144 : (k == 6 ? 240 : 352)));
}

struct GrNibStep {
  uint32_t state, advance, count, pos;
};

__host__ __device__ constexpr GrNibStep gr_nib_step(int k, int st, int nib) {
  uint32_t f = 0, n = 0, pos = 0;
  for (int i = 0; i < 4; ++i) {
    const uint32_t b = (static_cast<uint32_t>(nib) >> i) & 1u;
    if (st == 0) {
      if (b == 0) {
        f += 1u << k;
      } else {
        f += 1u;
        st = k;
      }
    } else {
      f += b << (k - st);
      --st;
      if (st == 0) {
        pos = f;
        ++n;
      }
    }
  }
  return GrNibStep{static_cast<uint32_t>(st), f, n, pos};
}

// Per (k - 3, nibble): next = the exit map as v_perm_b32 selectors {lo, hi} (byte s = image of s, states above k
// map to themselves), packed = the same map in 3-bit fields (bits 3s..3s+2).
struct GrNibNext {
  uint32_t lo, hi;
};

struct alignas(16) GrTables4 {
  GrNibNext next[5 * 16];
  uint32_t packed[5 * 16];
  uint32_t entry[kGrNibZero + 4];  // (k, s, nibble): advance | count << 16 | pos << 24; then zero entries
};

constexpr GrTables4 gr_make_tables4() {
  GrTables4 t{};
  for (int k = kGrNibK0; k <= 7; ++k) {
    for (int nib = 0; nib < 16; ++nib) {
      GrNibNext nx{0x03020100u, 0x07060504u};
      uint32_t packed = 0u;
      for (int s = 0; s <= k; ++s) {
        const GrNibStep r = gr_nib_step(k, s, nib);
        const uint32_t sh = 8u * static_cast<uint32_t>(s & 3);
        if (s < 4) {
          nx.lo = (nx.lo & ~(0xFFu << sh)) | (r.state << sh);
        } else {
          nx.hi = (nx.hi & ~(0xFFu << sh)) | (r.state << sh);
        }
        packed |= r.state << (3 * s);
        t.entry[gr_nib_entry_base(k) + s * 16 + nib] = r.advance | (r.count << 16) | (r.pos << 24);
      }
      t.next[(k - kGrNibK0) * 16 + nib] = nx;
      t.packed[(k - kGrNibK0) * 16 + nib] = packed;
    }
  }
  return t;
}

__constant__ GrTables4 kGrTables4 = gr_make_tables4();
constexpr int kGrTable4Vec4 = static_cast<int>(sizeof(GrTables4) / 16);
static_assert(sizeof(GrTables4) % 16 == 0, "GrTables4 is copied as 16-byte vectors");
static_assert(gr_nib_entry_base(7) + 8 * 16 == kGrNibZero, "nibble entry bases");

// Copy the nibble tables into LDS (all threads of the workgroup; a barrier must follow).
__device__ inline void gr_tables4_to_lds(GrTables4* dst) {
  const uint4* src = reinterpret_cast<const uint4*>(&kGrTables4);
  uint4* d = reinterpret_cast<uint4*>(dst);
  for (int i = threadIdx.x; i < kGrTable4Vec4; i += blockDim.x) d[i] = src[i];
}

// The reference's serial decode (general-k reader, TriSMoE_cuda_kernel.cu:403-479).
// out must be zero.
__device__ inline void gr_serial_decode(const int32_t* __restrict__ payload, int word_count, int k, int one_count,
                                        uint32_t* out) {
  const int total_bits = word_count * 32;
  gmem_i32* pl = as_gmem(payload);
  int bit_pos = 0;
  int flat_pos = 0;
  for (int one = 0; one < one_count; ++one) {
    int quotient = 0;
    while (bit_pos < total_bits) {
      const uint32_t bit = (static_cast<uint32_t>(pl[bit_pos >> 5]) >> (bit_pos & 31)) & 1u;
      ++bit_pos;
      if (bit != 0u) break;
      ++quotient;
    }
    int remainder = 0;
    for (int shift = 0; shift < k && bit_pos < total_bits; ++shift) {
      remainder |= static_cast<int>((static_cast<uint32_t>(pl[bit_pos >> 5]) >> (bit_pos & 31)) & 1u) << shift;
      ++bit_pos;
    }
    flat_pos += (quotient << k) | remainder;
    if (flat_pos >= kGrBits) break;
    out[flat_pos >> 5] |= 1u << (flat_pos & 31);
    ++flat_pos;
  }
}

// Group scans over S = 16 or 32 lanes (one or two DPP rows of a wavefront) with DPP row shifts and the
// row-15 broadcast (dpp_mov): register moves between lanes, no LDS round trips.  Every lane of a group must
// be active.

// Inclusive scan: op(own, earlier) combines a lane's value with the combined value of lanes before it.
template <int S, typename Op>
__device__ __forceinline__ uint32_t group_scan(uint32_t v, uint32_t identity, Op op) {
  static_assert(S == 16 || S == 32, "DPP group scans span one or two rows");
  v = op(v, dpp_mov<0x111, 0xF>(identity, v));  // row_shr:1
  v = op(v, dpp_mov<0x112, 0xF>(identity, v));  // row_shr:2
  v = op(v, dpp_mov<0x114, 0xF>(identity, v));  // row_shr:4
  v = op(v, dpp_mov<0x118, 0xF>(identity, v));  // row_shr:8
  if constexpr (S == 32) v = op(v, dpp_mov<0x142, 0xA>(identity, v));  // row_bcast:15 into rows 1 and 3
  return v;
}

template <int S>
__device__ __forceinline__ uint32_t group_incl_sum(uint32_t v) {
  return group_scan<S>(v, 0u, [](uint32_t own, uint32_t earlier) { return own + earlier; });
}

// The value of the group's last lane, in every lane of the group.
template <int S>
__device__ __forceinline__ uint32_t group_last(uint32_t v) {
  static_assert(S == 16 || S == 32, "groups of 16 or 32 lanes");
  const int g = static_cast<int>(__lane_id()) / S;
  if constexpr (S == 32) {
    const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 31));
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
    return g == 0 ? a : b;
  } else {
    const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 15));
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 31));
    const uint32_t c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 47));
    const uint32_t d = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
    return g == 0 ? a : (g == 1 ? b : (g == 2 ? c : d));
  }
}

// The largest span (in words) of the wavefront's groups: their first lanes hold the longest spans.  Read from
// those lanes whatever branch their groups took, so it is wave-uniform and only ever too large.
template <int S>
__device__ __forceinline__ int wave_max_words(int nw) {
  int m = __builtin_amdgcn_readlane(nw, 0);
#pragma unroll
  for (int g = 1; g < kWave / S; ++g) {
    const int v = __builtin_amdgcn_readlane(nw, g * S);
    m = v > m ? v : m;
  }
  return m;
}

// Composition of 4-state maps in the next[] byte encoding (byte s = image of s): first `earlier`, then `own`.
// Byte s of the result is byte earlier[s] of own, i.e. v_perm_b32 with `earlier` as the selector.
__device__ __forceinline__ uint32_t gr_map_compose(uint32_t own, uint32_t earlier) {
  return __builtin_amdgcn_perm(own, own, earlier);
}

// Maps of 8 states (Rice k in [4, 7]): byte s of {lo, hi} is the image of s; states above k are never reached.
struct GrMap8 {
  uint32_t lo, hi;
};

// First `earlier`, then `own`: selectors 0..3 pick own.lo's bytes, 4..7 own.hi's.
__device__ __forceinline__ GrMap8 gr_map8_compose(GrMap8 own, GrMap8 earlier) {
  return GrMap8{__builtin_amdgcn_perm(own.hi, own.lo, earlier.lo), __builtin_amdgcn_perm(own.hi, own.lo, earlier.hi)};
}

// A word's exit map (gr_exit_map: 3 bits per entry state) spread to one byte per state.
__device__ __forceinline__ GrMap8 gr_word_map8(uint32_t w, int k) {
  const uint32_t m = gr_exit_map(w, k);
  const auto spread = [](uint32_t x) {
    return (x & 7u) | ((x & 0x38u) << 5) | ((x & 0x1C0u) << 10) | ((x & 0xE00u) << 15);
  };
  return GrMap8{spread(m & 0xFFFu), spread(m >> 12)};
}

template <int S>
__device__ __forceinline__ GrMap8 group_scan_map8(GrMap8 v) {
  static_assert(S == 16 || S == 32, "DPP group scans span one or two rows");
  constexpr uint32_t kIdLo = 0x03020100u, kIdHi = 0x07060504u;
  v = gr_map8_compose(v, GrMap8{dpp_mov<0x111, 0xF>(kIdLo, v.lo), dpp_mov<0x111, 0xF>(kIdHi, v.hi)});
  v = gr_map8_compose(v, GrMap8{dpp_mov<0x112, 0xF>(kIdLo, v.lo), dpp_mov<0x112, 0xF>(kIdHi, v.hi)});
  v = gr_map8_compose(v, GrMap8{dpp_mov<0x114, 0xF>(kIdLo, v.lo), dpp_mov<0x114, 0xF>(kIdHi, v.hi)});
  v = gr_map8_compose(v, GrMap8{dpp_mov<0x118, 0xF>(kIdLo, v.lo), dpp_mov<0x118, 0xF>(kIdHi, v.hi)});
  if constexpr (S == 32) {
    v = gr_map8_compose(v, GrMap8{dpp_mov<0x142, 0xA>(kIdLo, v.lo), dpp_mov<0x142, 0xA>(kIdHi, v.hi)});
  }
  return v;
}

// One block's stream as seen by lane j of its group: the block header and the
// lane's span words [w0, w0 + nw) preloaded (when word_count <= 128).
template <int S>
struct GrSpan {
  static constexpr int kMaxWords = kGrWords / S;
  const int32_t* payload;  // null: absent or invalid block
  int word_count;
  int meta;
  int w0;
  int nw;
  uint32_t w[kMaxWords];
};

// The block header (stream start, word count, meta) of block_idx, or an empty block when !valid.  The loads are
// issued without a branch (an invalid block reads `dummy`, any readable word), so nothing waits for them until
// the header is used.
template <int S>
__device__ __forceinline__ void gr_span_header(GrSpan<S>& sp, const int32_t* __restrict__ words,
                                               const int32_t* __restrict__ offsets, const int32_t* __restrict__ meta,
                                               int block_idx, bool valid, const int32_t* __restrict__ dummy) {
  valid = valid && words != nullptr && offsets != nullptr && meta != nullptr;
  gmem_i32* o = as_gmem(valid ? offsets + block_idx : dummy);
  gmem_i32* m = as_gmem(valid ? meta + block_idx : dummy);
  const int begin = o[0];
  const int end = o[valid ? 1 : 0];
  const int mv = m[0];
  sp.payload = valid ? words + begin : nullptr;
  sp.word_count = valid ? end - begin : 0;
  sp.meta = valid ? mv : 0;
  sp.w0 = 0;
  sp.nw = 0;
}

// The lane's span words of a block whose header is loaded.
template <int S>
__device__ __forceinline__ void gr_span_words(GrSpan<S>& sp, int j) {
  const int wc = sp.word_count;
  if (wc > 0 && wc <= kGrWords) {
    const int span = (wc + S - 1) / S;
    sp.w0 = j * span;
    const int rest = wc - sp.w0;
    sp.nw = rest < 0 ? 0 : (rest < span ? rest : span);
  }
  gmem_i32* src = as_gmem(sp.payload);
#pragma unroll
  for (int i = 0; i < GrSpan<S>::kMaxWords; ++i) {
    sp.w[i] = i < sp.nw ? static_cast<uint32_t>(src[sp.w0 + i]) : 0u;
  }
}

// Decode one block by the S lanes of a group (j = lane within the group; all S
// lanes of the group call together, groups of a wave may decode different
// blocks).  out: the block's 128-word LDS bitmap with kGrPadFront words before
// it and kGrPadBack after it, all zero and visible to the wave.  A wave-level
// LDS sync must follow before out is read; the pads are left dirty.
template <int S>
__device__ inline void gr_decode_block_group(const GrSpan<S>& sp, const GrTables* __restrict__ tab, uint32_t* out,
                                             int j, const GrTables4* __restrict__ tab4 = nullptr) {
  static_assert(S == 16 || S == 32, "span decoder groups are 16 or 32 lanes");
  constexpr int kMaxWords = GrSpan<S>::kMaxWords;
  constexpr int kBytes = 4 * kMaxWords;
  const int wc = sp.word_count;
  if (wc <= 0) return;
  const int k = sp.meta & kMetaKMask;
  const int one_count = sp.meta >> kMetaOnesShift;
  if ((sp.meta & kMetaRaw) != 0) {
    if (wc <= kGrWords) {
#pragma unroll
      for (int i = 0; i < kMaxWords; ++i) {
        if (i < sp.nw) out[sp.w0 + i] = sp.w[i];
      }
    } else {
      for (int w = j; w < kGrWords; w += S) out[w] = static_cast<uint32_t>(as_gmem(sp.payload)[w]);
    }
    return;
  }
  if (one_count <= 0) return;
  bool serial = k > kMaxParallelK || wc > kGrWords;
  if (!serial && k == 0) {
    // The stream is the bitmap; it decodes as itself iff it holds exactly one_count ones.
    uint32_t ones = 0u;
#pragma unroll
    for (int i = 0; i < kMaxWords; ++i) ones += static_cast<uint32_t>(__popc(sp.w[i]));
    serial = static_cast<int>(group_last<S>(group_incl_sum<S>(ones))) != one_count;
    if (!serial) {
#pragma unroll
      for (int i = 0; i < kMaxWords; ++i) {
        if (i < sp.nw) out[sp.w0 + i] = sp.w[i];
      }
    }
  } else if (!serial && k <= 2) {
    const uint32_t* __restrict__ nxt = tab->next + (k - 1) * 256;
    const char* __restrict__ ent = reinterpret_cast<const char*>(tab->entry);
    const uint32_t kbase = static_cast<uint32_t>(gr_entry_base(k)) * 8u;  // byte offset of k's entries
    const int nbytes = 4 * sp.nw;
    // words any lane of the wavefront holds (a group's first lane holds the most): the walks stop there
    const int maxw = wave_max_words<S>(sp.nw);
    // Each phase walks the span a word at a time under a wave-uniform guard, and issues a word's four table
    // reads together before any is used: one LDS round trip per word, not per byte.
    // ---- A: next-state maps of every byte (kept for C), composed over the lane's words (the words past its
    // span leave the map as it is; C does not use their maps)
    uint32_t f[kBytes];
    uint32_t c = kGrIdentityNext;
#pragma unroll
    for (int wd = 0; wd < kMaxWords; ++wd) {
      if (wd < maxw) {
#pragma unroll
        for (int b = 0; b < 4; ++b) f[4 * wd + b] = nxt[(sp.w[wd] >> (8 * b)) & 0xFFu];
        uint32_t cw = c;
#pragma unroll
        for (int b = 0; b < 4; ++b) cw = gr_map_compose(f[4 * wd + b], cw);
        c = wd < sp.nw ? cw : c;
      }
    }
    // ---- B: the map of lanes 0..j, then the previous lane's (wave_shr:1) applied to state 0
    const uint32_t map = group_scan<S>(c, kGrIdentityNext, gr_map_compose);
    const uint32_t prev_map = dpp_mov<0x138, 0xF>(kGrIdentityNext, map);
    // the true entry state in all four bytes (a selector that steps it through a byte's map)
    uint32_t st = j == 0 ? 0u : __builtin_amdgcn_perm(prev_map, prev_map, 0u);
    // ---- C: entries along the true path (the state chain runs on A's maps); F advance and codeword count
    // sums from their high words, the masks read again for the emission
    uint32_t off[kBytes];
    uint32_t hisum = 0u;
#pragma unroll
    for (int wd = 0; wd < kMaxWords; ++wd) {
      if (wd < maxw) {
        uint32_t hi[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int i = 4 * wd + b;
          // entry index state * 256 + byte: the word's byte b into bits 0..7, the state into bits 8..15
          const uint32_t idx = __builtin_amdgcn_perm(st, sp.w[wd], 0x0C0C0400u | static_cast<uint32_t>(b));
          off[i] = i < nbytes ? (idx << 3) + kbase : kGrZeroEntryOffset;
          st = __builtin_amdgcn_perm(f[i], f[i], st);
          hi[b] = *reinterpret_cast<const uint32_t*>(ent + off[i] + 4);
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) hisum += hi[b];
      }
    }
    asm volatile("" ::: "memory");  // the emission reads the entries again rather than keeping 16 of them live
    // advance sum (< 2^12) and count sum (< 2^9) of the lane, repacked as adv | count << 16 for the group sums
    const uint32_t packed = (hisum & 0xFFFu) | (((hisum >> 12) & 0x1FFu) << 16);
    const uint32_t incl = group_incl_sum<S>(packed);
    const int total = static_cast<int>(group_last<S>(incl) >> 16);
    serial = total != one_count;
    if (!serial) {
      // bit position + 32 of the lane's first mask bit 0 (F at the span start - 1, biased past the front pad)
      uint32_t posb = ((incl - packed) & 0xFFFFu) + 31u;
      uint32_t* base = out - 1;
      // OR a mask (< 2^64) whose bit 0 is at posb - 32 into the bitmap; word 129 and up are the back pads,
      // where only positions past 4095 land
      const auto emit = [&](uint64_t m) {
        const uint32_t rel = posb & 31u;
        const uint32_t widx = (posb >> 5) < 129u ? (posb >> 5) : 129u;
        const uint64_t v = m << rel;
        atomicOr(&base[widx], static_cast<uint32_t>(v));
        atomicOr(&base[widx + 1], static_cast<uint32_t>(v >> 32));
        atomicOr(&base[widx + 2], static_cast<uint32_t>((m >> 32) << rel >> 32));
      };
      // k <= 2: a byte's mask is below 2^25 and its advance at most 32, so two bytes fit one 64-bit mask
#pragma unroll
      for (int wd = 0; wd < kMaxWords; ++wd) {
        if (wd < maxw) {
          uint2 e[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) e[b] = *reinterpret_cast<const uint2*>(ent + off[4 * wd + b]);
#pragma unroll
          for (int b = 0; b < 4; b += 2) {
            const uint32_t a0 = e[b].y & 0x7Fu;
            emit(static_cast<uint64_t>(e[b].x) | (static_cast<uint64_t>(e[b + 1].x) << a0));
            posb += a0 + (e[b + 1].y & 0x7Fu);
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      const uint32_t pad = j < 3 ? out[kGrWords + j] : 0u;
      const uint64_t hit = __ballot(pad != 0u);
      const uint64_t group_mask = (S == 64 ? ~0ull : ((1ull << S) - 1ull))
                                  << ((static_cast<int>(__lane_id()) / S) * S);
      serial = (hit & group_mask) != 0ull;
      if (serial) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        for (int w = j; w < kGrWords; w += S) out[w] = 0u;
      }
    }
  } else if (!serial && tab4 != nullptr) {
    // k in [3, 7]: nibble tables
    const GrNibNext* __restrict__ nxt = tab4->next + (k - kGrNibK0) * 16;
    const uint32_t* __restrict__ pkd = tab4->packed + (k - kGrNibK0) * 16;
    const uint32_t* __restrict__ ent = tab4->entry + gr_nib_entry_base(k);
    const uint32_t zrel = static_cast<uint32_t>(kGrNibZero - gr_nib_entry_base(k));
    const int maxw = wave_max_words<S>(sp.nw);
    // ---- A: every nibble's exit map, composed over the lane's words; a word's eight reads are issued together
    GrMap8 c{0x03020100u, 0x07060504u};
#pragma unroll
    for (int wd = 0; wd < kMaxWords; ++wd) {
      if (wd < maxw) {
        GrNibNext e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = nxt[(sp.w[wd] >> (4 * i)) & 15u];
        GrMap8 cw = c;
#pragma unroll
        for (int i = 0; i < 8; ++i) cw = gr_map8_compose(GrMap8{e[i].lo, e[i].hi}, cw);
        c = wd < sp.nw ? cw : c;
      }
    }
    // ---- B: the previous lanes' map applied to state 0
    const GrMap8 map = group_scan_map8<S>(c);
    const uint32_t prev_lo = dpp_mov<0x138, 0xF>(0u, map.lo);  // wave_shr:1
    uint32_t st = j == 0 ? 0u : (prev_lo & 0xFFu);
    // ---- C: the entries along the true path: a word's eight packed maps are read together, the state chain runs
    // on them, then its eight entry reads are issued together.  Sums of F advance and codeword count; per nibble
    // the F offset from the lane's start of the codeword it completes, + 1 (0: none), two to a register (a lane
    // advances at most 64 * 4 * 2^7, so offsets stay below 2^16)
    uint32_t loc[4 * kMaxWords];
    uint32_t adv = 0u, cnt = 0u;
    const int nnib = 8 * sp.nw;
#pragma unroll
    for (int wd = 0; wd < kMaxWords; ++wd) {
      if (wd < maxw) {
        uint32_t pm[8], e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pm[i] = pkd[(sp.w[wd] >> (4 * i)) & 15u];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t idx = 8 * wd + i < nnib ? st * 16u + ((sp.w[wd] >> (4 * i)) & 15u) : zrel;
          st = (pm[i] >> (3u * st)) & 7u;
          e[i] = ent[idx];
        }
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          const uint32_t h0 = (e[i] >> 16) & 1u;
          const uint32_t v0 = h0 != 0u ? adv + (e[i] >> 24) + 1u : 0u;
          adv += e[i] & 0xFFFFu;
          const uint32_t h1 = (e[i + 1] >> 16) & 1u;
          const uint32_t v1 = h1 != 0u ? adv + (e[i + 1] >> 24) + 1u : 0u;
          adv += e[i + 1] & 0xFFFFu;
          cnt += h0 + h1;
          loc[4 * wd + i / 2] = v0 | (v1 << 16);
        }
      }
    }
    // the count is below 2^7 per lane; an advance clamped at 8191 (already past the block) keeps the group sums
    // below 2^19 and every later position past 4095
    const uint32_t packed = (adv < 8191u ? adv : 8191u) | (cnt << 19);
    const uint32_t incl = group_incl_sum<S>(packed);
    serial = static_cast<int>(group_last<S>(incl) >> 19) != one_count;
    if (!serial) {
      // positions increase along the stream: those past 4095 are dropped, as the reference stops there
      const uint32_t run = ((incl - packed) & 0x7FFFFu) - 2u;  // F at the lane's start, less the two biases
#pragma unroll
      for (int wd = 0; wd < kMaxWords; ++wd) {
        if (wd < maxw) {
#pragma unroll
          for (int h = 0; h < 8; ++h) {
            const uint32_t v = (loc[4 * wd + h / 2] >> (16 * (h & 1))) & 0xFFFFu;
            const uint32_t pos = run + v;
            if (v != 0u && pos < static_cast<uint32_t>(kGrBits)) atomicOr(&out[pos >> 5], 1u << (pos & 31u));
          }
        }
      }
    }
  } else if (!serial) {
    // k in [3, 7] without the nibble tables: word walks
    const int maxw = wave_max_words<S>(sp.nw);
    // ---- A: the lane's exit map over its words
    GrMap8 c{0x03020100u, 0x07060504u};
#pragma unroll
    for (int wd = 0; wd < kMaxWords; ++wd) {
      if (wd < maxw && wd < sp.nw) c = gr_map8_compose(gr_word_map8(sp.w[wd], k), c);
    }
    // ---- B: the previous lanes' map applied to state 0
    const GrMap8 map = group_scan_map8<S>(c);
    const uint32_t prev_lo = dpp_mov<0x138, 0xF>(0u, map.lo);  // wave_shr:1
    const int st = j == 0 ? 0 : static_cast<int>(prev_lo & 0xFFu);
    // ---- C: F advance and codeword count along the true path
    int s = st;
    uint32_t dsum = 0u, osum = 0u;
#pragma unroll
    for (int wd = 0; wd < kMaxWords; ++wd) {
      if (wd < maxw && wd < sp.nw) {
        int d = 0, o = 0;
        s = gr_walk_word<false>(sp.w[wd], k, s, &d, &o, 0, 0, 0, nullptr);
        dsum += static_cast<uint32_t>(d);
        osum += static_cast<uint32_t>(o);
      }
    }
    // a lane advances at most 8 words * 32 << 7 and completes under 8 * 8 codewords; an advance clamped at
    // 8191 (already past the block) keeps the group sums below 2^19 and every later position past 4095
    const uint32_t packed = (dsum < 8191u ? dsum : 8191u) | (osum << 19);
    const uint32_t incl = group_incl_sum<S>(packed);
    serial = static_cast<int>(group_last<S>(incl) >> 19) != one_count;
    if (!serial) {
      int run = static_cast<int>((incl - packed) & 0x7FFFFu);
      s = st;
#pragma unroll
      for (int wd = 0; wd < kMaxWords; ++wd) {
        if (wd < maxw && wd < sp.nw) {
          int d = 0, o = 0;
          s = gr_walk_word<true>(sp.w[wd], k, s, &d, &o, run, 0, 0x7FFFFFFF, out);
          run += d;
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (serial && j == 0) gr_serial_decode(sp.payload, wc, k, one_count, out);
}

}  // namespace tris
