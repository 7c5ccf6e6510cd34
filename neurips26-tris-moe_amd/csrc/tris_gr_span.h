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
//   step[k][byte]    four 16-bit slots, slot s = the transition from entry
//                    state s: s' | n << 2 | dF << 6 (n codewords completed,
//                    dF added to F); slots above k are the identity;
//   mask[k][s][byte] the completed ones as a bit mask, bit i = a one at
//                    F(byte start) - 1 + i (a codeword entered mid-remainder
//                    whose last bits are zero ends at bit 0).
// Because step is indexed by the byte alone, following all k + 1 entry states
// through a span costs table reads that do not wait on each other.  Each lane
// of the block's group of S lanes:
//   A. runs its span from every entry state, giving per entry state the exit
//      state, the F advance and the completed-codeword count;
//   B. learns its true entry state by chaining the exit states of the lanes
//      before it, and its starting F by a segmented prefix sum;
//   C. runs its span again from the true state, OR-ing the decoded ones into
//      the block's 128-word LDS bitmap.
// k = 0 streams are the bitmap itself (each codeword is run zeros then a one)
// and are copied.  Raw blocks are copied.  k >= 4, streams longer than 128
// words (the encoder stores those raw), and any stream whose completed
// codewords do not equal one_count or reach past bit 4095, are decoded by the
// group's first lane with the reference's serial rules, so every input
// decodes as the reference decodes it.
#pragma once

#include "tris_common.h"

namespace tris {

constexpr int kGrStepEntries = 3 * 256;            // k = 1, 2, 3; byte
constexpr int kGrMaskEntries = (2 + 3 + 4) * 256;  // k = 1, 2, 3; s in [0, k]; byte

__host__ __device__ constexpr int gr_mask_base(int k) { return k == 1 ? 0 : (k == 2 ? 512 : 1280); }

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
  uint64_t step[kGrStepEntries];
  uint64_t mask[kGrMaskEntries];
};

constexpr GrTables gr_make_tables() {
  GrTables t{};
  for (int k = 1; k <= 3; ++k) {
    for (int byte = 0; byte < 256; ++byte) {
      uint64_t packed = 0;
      for (int s = 0; s < 4; ++s) {
        uint64_t slot = static_cast<uint64_t>(s);
        if (s <= k) {
          const GrByteStep r = gr_byte_step(k, s, byte);
          slot = r.state | (r.count << 2) | (r.advance << 6);
          t.mask[gr_mask_base(k) + s * 256 + byte] = r.mask;
        }
        packed |= slot << (16 * s);
      }
      t.step[(k - 1) * 256 + byte] = packed;
    }
  }
  return t;
}

__constant__ GrTables kGrTables = gr_make_tables();
constexpr int kGrTableVec4 = static_cast<int>(sizeof(GrTables) / 16);

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

// Segmented (groups of S lanes) inclusive prefix sum.
template <int S>
__device__ __forceinline__ int group_incl_sum(int v, int j) {
#pragma unroll
  for (int d = 1; d < S; d <<= 1) {
    const int u = __shfl_up(v, d);
    if (j >= d) v += u;
  }
  return v;
}

template <int S>
__device__ __forceinline__ int group_last(int v) {
  return __shfl(v, (static_cast<int>(__lane_id()) / S) * S + S - 1);
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

// Read the block header and the lane's span words.  Loads are issued together
// so their latencies overlap.
template <int S>
__device__ __forceinline__ void gr_span_load(GrSpan<S>& sp, const int32_t* __restrict__ words,
                                             const int32_t* __restrict__ offsets, const int32_t* __restrict__ meta,
                                             int block_idx, bool valid, int j) {
  sp.payload = nullptr;
  sp.word_count = 0;
  sp.meta = 0;
  sp.w0 = 0;
  sp.nw = 0;
  if (valid && words != nullptr && offsets != nullptr && meta != nullptr) {
    const int begin = offsets[block_idx];
    sp.word_count = offsets[block_idx + 1] - begin;
    sp.meta = meta[block_idx];
    sp.payload = words + begin;
  }
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
// blocks).  out: the block's 128-word LDS bitmap, already zero and visible to
// the wave.  A wave-level LDS sync must follow before out is read.
template <int S>
__device__ inline void gr_decode_block_group(const GrSpan<S>& sp, const GrTables* __restrict__ tab, uint32_t* out,
                                             int j) {
  constexpr int kMaxWords = GrSpan<S>::kMaxWords;
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
    int ones = 0;
#pragma unroll
    for (int i = 0; i < kMaxWords; ++i) ones += __popc(sp.w[i]);
    serial = group_last<S>(group_incl_sum<S>(ones, j)) != one_count;
    if (!serial) {
#pragma unroll
      for (int i = 0; i < kMaxWords; ++i) {
        if (i < sp.nw) out[sp.w0 + i] = sp.w[i];
      }
    }
  } else if (!serial) {
    const uint64_t* step = tab->step + (k - 1) * 256;
    const uint64_t* mtab = tab->mask + gr_mask_base(k);
    // ---- A: every entry state through the span
    uint32_t cur[4] = {0u, 1u, 2u, 3u};
    int df[4] = {0, 0, 0, 0};
    int nc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < kMaxWords; ++i) {
      if (i < sp.nw) {
        const uint32_t word = sp.w[i];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint64_t t = step[(word >> (8 * b)) & 0xFFu];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const uint32_t slot = static_cast<uint32_t>(t >> (cur[s] << 4));
            cur[s] = slot & 3u;
            nc[s] += static_cast<int>((slot >> 2) & 15u);
            df[s] += static_cast<int>((slot >> 6) & 127u);
          }
        }
      }
    }
    const int exit_map = static_cast<int>(cur[0] | (cur[1] << 2) | (cur[2] << 4) | (cur[3] << 6));
    // ---- B: true entry state (chain over the group), then prefix sums
    int entry = 0;
#pragma unroll
    for (int t = 1; t < S; ++t) {
      const int prev_entry = __shfl_up(entry, 1);
      const int prev_map = __shfl_up(exit_map, 1);
      if (j == t) entry = (prev_map >> (2 * prev_entry)) & 3;
    }
    int my_df = df[0], my_nc = nc[0];
#pragma unroll
    for (int s = 1; s < 4; ++s) {
      if (entry == s) {
        my_df = df[s];
        my_nc = nc[s];
      }
    }
    const int incl_df = group_incl_sum<S>(my_df, j);
    const int total_nc = group_last<S>(group_incl_sum<S>(my_nc, j));
    // Completed codewords must number one_count: then they are exactly the
    // reference's first one_count codewords, and whatever follows is padding.
    serial = total_nc != one_count;
    if (!serial) {
      // ---- C: emission from the true entry state
      int pos = incl_df - my_df - 1;  // F at the span start, minus 1: mask bit 0's position
      uint32_t state = static_cast<uint32_t>(entry);
      uint32_t acc0 = 0u, acc1 = 0u, acc2 = 0u;  // bitmap words [aw, aw + 3)
      int aw = pos >> 5;                         // -1 only at the block start
      bool overflow = false;
#pragma unroll
      for (int i = 0; i < kMaxWords; ++i) {
        if (i < sp.nw) {
          const uint32_t word = sp.w[i];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const uint32_t byte = (word >> (8 * b)) & 0xFFu;
            const uint64_t mask = mtab[(state << 8) | byte];
            const uint32_t slot = static_cast<uint32_t>(step[byte] >> (state << 4));
            state = slot & 3u;
            // 0 <= rel < 32 and mask bits < 41 keep every bit inside the 3-word window
            const int rel = pos - (aw << 5);
            const uint64_t lo = mask << rel;
            const uint32_t hi = rel == 0 ? 0u : static_cast<uint32_t>(mask >> (64 - rel));
            acc0 |= static_cast<uint32_t>(lo);
            acc1 |= static_cast<uint32_t>(lo >> 32);
            acc2 |= hi;
            pos += static_cast<int>((slot >> 6) & 127u);
            // advance <= 64 moves pos by at most two words; words below pos are final
#pragma unroll
            for (int f = 0; f < 2; ++f) {
              if (pos - (aw << 5) >= 32) {
                if (acc0 != 0u) {
                  if (aw >= 0 && aw < kGrWords) {
                    atomicOr(&out[aw], acc0);
                  } else {
                    overflow = true;
                  }
                }
                acc0 = acc1;
                acc1 = acc2;
                acc2 = 0u;
                ++aw;
              }
            }
          }
        }
      }
      const uint32_t rest[3] = {acc0, acc1, acc2};
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        if (rest[i] != 0u) {
          if (aw + i >= 0 && aw + i < kGrWords) {
            atomicOr(&out[aw + i], rest[i]);
          } else {
            overflow = true;
          }
        }
      }
      // A one at position >= 4096: the reference stops there (and drops later
      // ones); fall back to its serial rules.
      const uint64_t any_overflow = __ballot(overflow);
      const uint64_t group_mask = (S == 64 ? ~0ull : ((1ull << S) - 1ull))
                                  << ((static_cast<int>(__lane_id()) / S) * S);
      serial = (any_overflow & group_mask) != 0ull;
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
