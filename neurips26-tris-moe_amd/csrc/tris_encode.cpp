// Offline block-GR encoder for split bitmaps (host code).
//
// Produces the bitstream of QuantLinear._pack_block_gr_gmap_tensor
// (qlinear_cuda.py:3793-3859) and of the export tool's
// pack_block_gr_gmap_tensor (tools/rewrite_runtime_min_checkpoint.py:252-347):
// per 64x64 block, the zero runs between ones are Rice(k) coded with the k in
// [k_min, k_max] that first minimises the coded length; blocks whose code
// needs >= 128 words (or all blocks with force_raw) are stored raw.
//
// The coded length for every k comes from one pass over the runs:
// bits(k) = sum_i (run_i >> k) + n * (1 + k).  The writer keeps a 64-bit
// accumulator and emits long unary runs a word at a time.
#include <cstdint>
#include <cstring>
#include <vector>

#include "tris_common_host.h"

namespace {

constexpr int kTileOut = 64;
constexpr int kPackedRows = 2;
constexpr int kWords = 128;
constexpr int kBits = kWords * 32;
constexpr int kMaxK = 7;

struct BitWriter {
  uint32_t* out;
  int64_t nwords = 0;
  uint64_t acc = 0;
  int fill = 0;  // bits pending in acc (< 32 between calls)

  void put(uint32_t value, int nbits) {  // nbits <= 32, value < 2^nbits
    acc |= static_cast<uint64_t>(value) << fill;
    fill += nbits;
    if (fill >= 32) {
      out[nwords++] = static_cast<uint32_t>(acc);
      acc >>= 32;
      fill -= 32;
    }
  }
  void zeros(int64_t count) {
    while (count > 0) {
      const int take = count > 32 ? 32 : static_cast<int>(count);
      put(0u, take);
      count -= take;
    }
  }
  void flush() {
    if (fill > 0) {
      out[nwords++] = static_cast<uint32_t>(acc);
      acc = 0;
      fill = 0;
    }
  }
};

}  // namespace

extern "C" int64_t tris_gr_encode(const int32_t* packed, int32_t packed_rows, int32_t outfeatures, int32_t k_min,
                                  int32_t k_max, int32_t force_raw, int32_t* words_out, int64_t words_capacity,
                                  int32_t* offsets_out, int32_t* meta_out) {
  if (packed_rows < 0 || outfeatures < 0) {
    tris::set_error("tris_gr_encode: negative shape");
    return TRIS_ERR_INVALID;
  }
  if (k_min < 0 || k_max > kMaxK || k_min > k_max) {
    tris::set_error("tris_gr_encode: k bounds must satisfy 0 <= k_min <= k_max <= %d (got %d, %d)", kMaxK, k_min,
                    k_max);
    return TRIS_ERR_INVALID;
  }
  const int nkb = (packed_rows + kPackedRows - 1) / kPackedRows;
  const int nob = (outfeatures + kTileOut - 1) / kTileOut;
  const int64_t nblk = static_cast<int64_t>(nkb) * nob;
  if (nblk > 0 && (packed == nullptr || words_out == nullptr || offsets_out == nullptr || meta_out == nullptr)) {
    tris::set_error("tris_gr_encode: null pointer");
    return TRIS_ERR_INVALID;
  }
  if (words_capacity < nblk * kWords) {
    tris::set_error("tris_gr_encode: words_capacity %lld < %lld", static_cast<long long>(words_capacity),
                    static_cast<long long>(nblk * kWords));
    return TRIS_ERR_INVALID;
  }
  uint32_t block[kWords];
  std::vector<int32_t> runs(kBits);
  int64_t total = 0;
  if (nblk > 0) offsets_out[0] = 0;
  for (int kb = 0; kb < nkb; ++kb) {
    for (int ob = 0; ob < nob; ++ob) {
      const int64_t bi = static_cast<int64_t>(kb) * nob + ob;
      // Block words in order lpr*64 + lo, zero past the matrix edges.
      for (int lpr = 0; lpr < kPackedRows; ++lpr) {
        const int row = kb * kPackedRows + lpr;
        for (int lo = 0; lo < kTileOut; ++lo) {
          const int col = ob * kTileOut + lo;
          block[lpr * kTileOut + lo] = (row < packed_rows && col < outfeatures)
                                           ? static_cast<uint32_t>(packed[static_cast<int64_t>(row) * outfeatures + col])
                                           : 0u;
        }
      }
      int n = 0;
      int prev = -1;
      int64_t shifted[kMaxK + 1] = {0};
      for (int w = 0; w < kWords; ++w) {
        uint32_t v = block[w];
        while (v != 0u) {
          const int pos = w * 32 + __builtin_ctz(v);
          const int run = pos - prev - 1;
          runs[n++] = run;
          for (int k = k_min; k <= k_max; ++k) shifted[k] += run >> k;
          prev = pos;
          v &= v - 1u;
        }
      }
      int64_t best_bits = static_cast<int64_t>(kBits) + 1;
      int best_k = k_min;
      for (int k = k_min; k <= k_max; ++k) {
        const int64_t bits = shifted[k] + static_cast<int64_t>(n) * (1 + k);
        if (bits < best_bits) {
          best_bits = bits;
          best_k = k;
        }
      }
      const int64_t coded_words = (best_bits + 31) / 32;
      uint32_t* dst = reinterpret_cast<uint32_t*>(words_out) + total;
      if (force_raw || coded_words >= kWords) {
        std::memcpy(dst, block, sizeof(block));
        total += kWords;
        meta_out[bi] = 1 << 4;
      } else {
        BitWriter bw{dst};
        const uint32_t rmask = (1u << best_k) - 1u;
        for (int i = 0; i < n; ++i) {
          bw.zeros(runs[i] >> best_k);
          // terminator 1 followed by the k remainder bits, LSB first
          bw.put(1u | ((static_cast<uint32_t>(runs[i]) & rmask) << 1), 1 + best_k);
        }
        bw.flush();
        total += bw.nwords;
        meta_out[bi] = best_k | (n << 8);
      }
      offsets_out[bi + 1] = static_cast<int32_t>(total);
    }
  }
  return total;
}
