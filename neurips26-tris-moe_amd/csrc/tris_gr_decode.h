// Wavefront-parallel decoder for one block-GR coded split-bitmap block.
//
// Bitstream (encoder qlinear_cuda.py:3763-3859; reference decoder
// TriSMoE_cuda_kernel.cu:321-479, which decodes a block serially on one
// thread): the zero run before each one is Rice(k) coded as q = run >> k zero
// bits, a terminating 1 bit, then k remainder bits LSB first, packed LSB first
// into 32-bit words.  meta = k | (one_count << 8), or the raw flag 1 << 4 for
// a block stored as its 128 dense words.
//
// Parallel scheme (one 64-lane wavefront per block, lane i owns word i of the
// stream, 64 words per round):
//   * The decoder is a finite-state transducer over bits with k+1 states:
//     0 = reading unary zeros, j = j remainder bits still to read.
//   * Pass 1: each lane computes its word's exit state for every entry
//     state.  The walk from state 0 records where it is in unary mode; a walk
//     from j > 0 is finished as soon as it reaches a codeword start at such a
//     position (both walks read the same bits from there on), which usually
//     takes one or two codewords.
//   * The true entry state of every lane is the fixed point of
//     entry[l] = exit_map[l-1](entry[l-1]) with entry[0] = carry; iterating
//     it with lane shuffles converges in a few steps because most exit maps
//     are constant, and is bounded by 64 steps.
//   * Pass 2: each lane walks its word from its true entry state, counting
//     completed codewords and the advance of the flat bit position (each
//     unary zero adds 2^k, a terminator 1, remainder bit j adds 2^j).  A
//     wave prefix sum gives every lane its starting flat position and one
//     index.
//   * Pass 3: the walk is repeated and each completed codeword sets bit
//     (flat position - 1) in the LDS bitmap with an LDS atomic OR, subject to
//     the reference's limits: only the first one_count ones, only positions
//     below 4096.
//   * If the stream holds fewer complete codewords than one_count (never true
//     for encoder output) or k > 7, the block is decoded serially by lane 0
//     with the reference's exact rules, so every input decodes as the
//     reference decodes it.
#pragma once

#include "tris_common.h"

namespace tris {

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Mask with bits [lo, hi] set (0 <= lo <= hi <= 31).
__device__ __forceinline__ uint32_t bit_range(int lo, int hi) {
  const uint32_t upto_hi = hi >= 31 ? 0xFFFFFFFFu : ((2u << hi) - 1u);
  return upto_hi & ~((1u << lo) - 1u);
}

// Pass 2 / 3 walk over the 32 bits of w from entry state s.
// Returns the exit state; *delta and *ones receive the flat-position advance
// and the number of completed codewords.  With kEmit, completed codewords are
// written to out (LDS) at base + running delta - 1, for global index
// idx0 + local count < one_count and position < 4096.
template <bool kEmit>
__device__ __forceinline__ int gr_walk_word(uint32_t w, int k, int s, int* delta_out, int* ones_out, int base,
                                            int idx0, int one_count, uint32_t* out) {
  int p = 0;
  int delta = 0;
  int ones = 0;
  if (s > 0) {
    // Finish the pending remainder bits of a codeword begun in an earlier word.
    const int r = s;  // s <= 7 < 32
    const uint32_t b = w & ((1u << r) - 1u);
    delta += static_cast<int>(b << (k - s));
    p = r;
    s = 0;
    if (kEmit) {
      const int pos = base + delta - 1;
      if (idx0 + ones < one_count && pos < kGrBits) atomicOr(&out[pos >> 5], 1u << (pos & 31));
    }
    ++ones;
  }
  while (p < 32) {
    const uint32_t m = w >> p;
    if (m == 0u) {
      delta += (32 - p) << k;
      p = 32;
      break;
    }
    const int z = __builtin_ctz(m);
    delta += (z << k) + 1;
    p += z + 1;
    const int avail = 32 - p;
    const int r = k < avail ? k : avail;
    if (r > 0) {
      const uint32_t b = (w >> p) & ((1u << r) - 1u);
      delta += static_cast<int>(b);
      p += r;
    }
    s = k - r;
    if (s == 0) {
      if (kEmit) {
        const int pos = base + delta - 1;
        if (idx0 + ones < one_count && pos < kGrBits) atomicOr(&out[pos >> 5], 1u << (pos & 31));
      }
      ++ones;
    }
  }
  *delta_out = delta;
  *ones_out = ones;
  return s;
}

// Pass 1: exit state for every entry state 0..k, packed 3 bits per state.
__device__ __forceinline__ uint32_t gr_exit_map(uint32_t w, int k) {
  // Walk from state 0, recording the positions where it reads unary bits.
  uint32_t unary = 0u;
  int p = 0;
  int exit0 = 0;
  while (p < 32) {
    const uint32_t m = w >> p;
    if (m == 0u) {
      unary |= bit_range(p, 31);
      exit0 = 0;
      p = 32;
      break;
    }
    const int t = p + __builtin_ctz(m);
    unary |= bit_range(p, t);
    p = t + 1 + k;
    exit0 = p > 32 ? p - 32 : 0;
  }
  uint32_t map = static_cast<uint32_t>(exit0);
  for (int j = 1; j <= k; ++j) {
    int q = j;
    int ex = 0;
    for (;;) {
      if (q >= 32) {
        ex = q - 32;
        break;
      }
      if ((unary >> q) & 1u) {
        ex = exit0;
        break;
      }
      const uint32_t m = w >> q;
      if (m == 0u) {
        ex = 0;
        break;
      }
      q += __builtin_ctz(m) + 1 + k;
    }
    map |= static_cast<uint32_t>(ex) << (3 * j);
  }
  return map;
}

// The reference's serial decode of one block (TriSMoE_cuda_kernel.cu:403-479,
// general-k reader; its k == 3 fast path decodes identically).  out must be zero.
__device__ inline void gr_decode_block_serial(const int32_t* __restrict__ payload, int word_count, int k,
                                              int one_count, uint32_t* out) {
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

// Decode block `block_idx` of one expert's GR stream into out[128] (LDS,
// owned by the calling wavefront).  Must be called by all 64 lanes of a wave
// with wave-uniform arguments.  A null `words` (absent payload) yields zeros.
__device__ inline void gr_decode_block_wave(const int32_t* __restrict__ words, const int32_t* __restrict__ offsets,
                                            const int32_t* __restrict__ meta, int block_idx, uint32_t* out) {
  const int lane = static_cast<int>(__lane_id());
  out[lane] = 0u;
  out[lane + kWave] = 0u;
  if (words == nullptr || offsets == nullptr || meta == nullptr) {
    wave_sync_lds();
    return;
  }
  const int meta_word = meta[block_idx];
  const int word_begin = offsets[block_idx];
  const int word_count = offsets[block_idx + 1] - word_begin;
  wave_sync_lds();
  if (word_count <= 0) return;
  const int32_t* payload = words + word_begin;
  if ((meta_word & kMetaRaw) != 0) {
    const int n = word_count < kGrWords ? word_count : kGrWords;
    for (int i = lane; i < n; i += kWave) out[i] = static_cast<uint32_t>(payload[i]);
    wave_sync_lds();
    return;
  }
  const int k = meta_word & kMetaKMask;
  const int one_count = meta_word >> kMetaOnesShift;
  if (one_count <= 0) return;
  bool serial = k > kMaxParallelK;
  if (!serial) {
    int carry_state = 0;
    int carry_delta = 0;
    int carry_ones = 0;
    for (int round = 0; round < word_count; round += kWave) {
      const int idx = round + lane;
      const bool active = idx < word_count;
      const int count = (word_count - round) < kWave ? (word_count - round) : kWave;
      const uint32_t w = active ? static_cast<uint32_t>(payload[idx]) : 0u;
      const uint32_t map = gr_exit_map(w, k);
      // Fixed point of entry[l] = map[l-1](entry[l-1]), entry[0] = carry_state.
      const uint32_t prev_map = static_cast<uint32_t>(__shfl_up(static_cast<int>(map), 1));
      int entry = lane == 0 ? carry_state : static_cast<int>(prev_map & 7u);
      for (int it = 0; it < kWave; ++it) {
        const int prev_entry = __shfl_up(entry, 1);
        const int next = lane == 0 ? carry_state : static_cast<int>((prev_map >> (3 * prev_entry)) & 7u);
        const bool changed = __any(next != entry);
        entry = next;
        if (!changed) break;
      }
      int delta = 0;
      int ones = 0;
      const int exit_state = gr_walk_word<false>(w, k, entry, &delta, &ones, 0, 0, 0, nullptr);
      // Inclusive wave prefix sum of (delta | ones << 19): delta per word <= 32*128,
      // so 64 words sum to at most 2^18; ones per word <= 32, at most 2^11 per round.
      const int packed = active ? (delta | (ones << 19)) : 0;
      int incl = packed;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
      }
      const int excl = incl - packed;
      const int base = carry_delta + (excl & 0x7FFFF);
      const int idx0 = carry_ones + (excl >> 19);
      if (active) {
        int d2 = 0;
        int o2 = 0;
        gr_walk_word<true>(w, k, entry, &d2, &o2, base, idx0, one_count, out);
      }
      const int last_incl = __shfl(incl, count - 1);
      carry_state = __shfl(exit_state, count - 1);
      carry_delta += last_incl & 0x7FFFF;
      carry_ones += last_incl >> 19;
    }
    serial = carry_ones < one_count;
    if (serial) {
      out[lane] = 0u;
      out[lane + kWave] = 0u;
    }
  }
  wave_sync_lds();
  if (serial) {
    if (lane == 0) gr_decode_block_serial(payload, word_count, k, one_count, out);
    wave_sync_lds();
  }
}

}  // namespace tris
