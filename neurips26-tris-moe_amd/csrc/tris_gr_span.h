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
// s remainder bits still to read.  For k in {1, 2, 3} two tables describe one
// byte of stream:
//   next[k][byte]       four bytes, byte s = the state after the byte from
//                       entry state s (identity above k).  A map of states in
//                       this form is a v_perm_b32 selector: composing maps,
//                       and stepping a state held in all four bytes, is one
//                       v_perm_b32;
//   entry[k][s][byte]   64 bits: the low word holds bits 0..31 of the
//                       completed ones' bit mask (bit i = a one at
//                       F(byte start) - 1 + i; a codeword entered
//                       mid-remainder whose last bits are zero ends at bit 0);
//                       the high word holds the F advance (bits 0..6), the
//                       number of completed codewords (bits 12..15) and mask
//                       bits 32..40 (bits 23..31), so a lane's sum of high
//                       words holds its advance and count sums in bits 0..20.
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
// The bitmap has zero pad words before and after it: a one at a
// position past 4095 lands in the back pads (the reference stops there), and
// the decode falls back to the serial rules.  k = 0 streams are the bitmap
// itself (each codeword is run zeros then a one) and are copied.  Raw blocks
// are copied.  k >= 4, streams longer than 128 words (the encoder stores
// those raw), and any stream whose completed codewords do not equal one_count
// or reach past bit 4095, are decoded by the group's first lane with the
// reference's serial rules, so every input decodes as the reference decodes
// it.
#pragma once

#include "tris_common.h"

namespace tris {

constexpr int kGrEntryStates = 2 + 3 + 4;                     // k = 1, 2, 3; s in [0, k]
constexpr int kGrEntries = kGrEntryStates * 256 + 1;             // + one all-zero entry
constexpr uint32_t kGrZeroEntryOffset = kGrEntryStates * 256 * 8;  // byte offset of the zero entry
constexpr uint32_t kGrIdentityNext = 0x03020100u;               // byte s = s

// Decoded-block layout in LDS: four pad words, the 128 bitmap words, eight pad words.  The emission writes the
// word before the bitmap and up to three words after it.  Rows stay 16-byte aligned, and the 140-word stride
// puts the bitmaps of neighbouring blocks 12 banks apart.
constexpr int kGrPadFront = 4;
constexpr int kGrPadBack = 8;
constexpr int kGrBlockStride = kGrPadFront + kGrWords + kGrPadBack;

__host__ __device__ constexpr int gr_entry_base(int k) { return k == 1 ? 0 : (k == 2 ? 512 : 1280); }

struct GrByteStep {
  uint32_t state;
  uint32_t count;
  uint32_t advance;
  uint64_t mask;
};

// Reading one byte (LSB first) of a Rice(k) stream from state st, 1 <= k <= 3.
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
  uint32_t next[3 * 256];          // (k, byte)
};

constexpr GrTables gr_make_tables() {
  GrTables t{};
  for (int k = 1; k <= 3; ++k) {
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

// The reference's serial decode (general-k reader, TriSMoE_cuda_kernel.cu:403-479).
// out must be zero.
__device__ inline void gr_serial_decode(const int32_t* __restrict__ payload, int word_count, int k, int one_count,
                                        uint32_t* out) {
  const int total_bits = word_count * 32;
  int bit_pos = 0;
  int flat_pos = 0;
  for (int one = 0; one < one_count; ++one) {
    int quotient = 0;
    while (bit_pos < total_bits) {
      const uint32_t bit = (static_cast<uint32_t>(payload[bit_pos >> 5]) >> (bit_pos & 31)) & 1u;
      ++bit_pos;
      if (bit != 0u) break;
      ++quotient;
    }
    int remainder = 0;
    for (int shift = 0; shift < k && bit_pos < total_bits; ++shift) {
      remainder |= static_cast<int>((static_cast<uint32_t>(payload[bit_pos >> 5]) >> (bit_pos & 31)) & 1u) << shift;
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
  const int32_t* o = valid ? offsets + block_idx : dummy;
  const int32_t* m = valid ? meta + block_idx : dummy;
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
#pragma unroll
  for (int i = 0; i < GrSpan<S>::kMaxWords; ++i) {
    sp.w[i] = i < sp.nw ? static_cast<uint32_t>(sp.payload[sp.w0 + i]) : 0u;
  }
}

// Decode one block by the S lanes of a group (j = lane within the group; all S
// lanes of the group call together, groups of a wave may decode different
// blocks).  out: the block's 128-word LDS bitmap with kGrPadFront words before
// it and kGrPadBack after it, all zero and visible to the wave.  A wave-level
// LDS sync must follow before out is read; the pads are left dirty.
template <int S>
__device__ inline void gr_decode_block_group(const GrSpan<S>& sp, const GrTables* __restrict__ tab, uint32_t* out,
                                             int j) {
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
      for (int w = j; w < kGrWords; w += S) out[w] = static_cast<uint32_t>(sp.payload[w]);
    }
    return;
  }
  if (one_count <= 0) return;
  bool serial = k > 3 || wc > kGrWords;
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
  } else if (!serial) {
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
      if (k <= 2) {
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
      } else {
#pragma unroll
        for (int wd = 0; wd < kMaxWords; ++wd) {
          if (wd < maxw) {
            uint2 e[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) e[b] = *reinterpret_cast<const uint2*>(ent + off[4 * wd + b]);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              emit(static_cast<uint64_t>(e[b].y >> 23) << 32 | e[b].x);
              posb += e[b].y & 0x7Fu;
            }
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
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (serial && j == 0) gr_serial_decode(sp.payload, wc, k, one_count, out);
}

}  // namespace tris
