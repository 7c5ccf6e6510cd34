/*
 * CPU restatement of the TriS-MoE block Golomb-Rice (GR) bitmap codec.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * product path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  Nothing in the product links against it.
 *
 * What it restates (all paths relative to the reference checkout):
 *   encoder  AutoGPTQ/auto_gptq/nn_modules/qlinear/qlinear_cuda.py:3763-3859
 *            (QuantLinear._encode_block_gr_zero_runs / _pack_block_gr_gmap_tensor)
 *            and tools/rewrite_runtime_min_checkpoint.py:170-347 (export tool,
 *            same bitstream; closed-form bit count :221-225, k bounds :228-249)
 *   decoder  AutoGPTQ/autogptq_extension/TriSMoE/TriSMoE_cuda_kernel.cu:321-502
 *            (read_block_gr_bit, decode_block_gr_zero_run[_k3],
 *             decode_block_gr_block, decode_block_gr_tile)
 *
 * Block format: a block covers packed rows 2*kb, 2*kb+1 of the dense packed
 * bitmap [packed_rows, N] and outputs 64*ob .. 64*ob+63 (zero padded past the
 * edges); block index kb*ceil(N/64)+ob; the 128 words of a block are in order
 * w = local_packed_row*64 + local_out; flat bit position p = w*32 + bit.
 * Zero runs between successive ones are Rice(k) coded: q = run>>k zero bits,
 * one 1 bit, then k remainder bits LSB first, packed LSB first into 32-bit
 * words.  k is the first minimiser of the coded length over [kmin, kmax];
 * a block whose coded length needs >= 128 words is stored raw (meta 1<<4).
 * Otherwise meta = k | (one_count << 8).
 */
#include <stdint.h>
#include <string.h>

#define GR_TILE_OUT 64
#define GR_PACKED_ROWS 2
#define GR_WORDS 128
#define GR_BITS (GR_WORDS * 32)
#define GR_META_K_MASK 0xF
#define GR_META_RAW 16
#define GR_META_ONES_SHIFT 8

static int ceil_div(int a, int b) { return (a + b - 1) / b; }

/* Gather the 128 dense words of block (kb, ob): qlinear_cuda.py:3810-3822. */
static void gather_block(const int32_t* packed, int packed_rows, int n, int kb, int ob, uint32_t* out) {
  for (int lpr = 0; lpr < GR_PACKED_ROWS; ++lpr) {
    const int row = kb * GR_PACKED_ROWS + lpr;
    for (int lo = 0; lo < GR_TILE_OUT; ++lo) {
      const int col = ob * GR_TILE_OUT + lo;
      out[lpr * GR_TILE_OUT + lo] =
          (row < packed_rows && col < n) ? (uint32_t)packed[(int64_t)row * n + col] : 0u;
    }
  }
}

/* Zero runs before each one, in flat order (qlinear_cuda.py:3823-3838). */
static int block_zero_runs(const uint32_t* block, int32_t* runs) {
  int count = 0;
  int prev = -1;
  for (int w = 0; w < GR_WORDS; ++w) {
    for (int b = 0; b < 32; ++b) {
      if ((block[w] >> b) & 1u) {
        const int pos = w * 32 + b;
        runs[count++] = pos - prev - 1;
        prev = pos;
      }
    }
  }
  return count;
}

/* Closed-form Rice length: rewrite_runtime_min_checkpoint.py:221-225. */
int64_t orc_rice_bits(const int32_t* runs, int nruns, int k) {
  int64_t bits = 0;
  for (int i = 0; i < nruns; ++i) bits += (int64_t)(runs[i] >> k) + 1 + k;
  return bits;
}

/* Bit-serial Rice encoder: qlinear_cuda.py:3763-3791.  Returns words written. */
int orc_rice_encode(const int32_t* runs, int nruns, int k, uint32_t* out, int cap_words) {
  int nwords = 0;
  uint32_t cur = 0;
  int off = 0;
#define PUSH_BIT(bit)                                   \
  do {                                                  \
    if (bit) cur |= 1u << off;                          \
    if (++off == 32) {                                  \
      if (nwords < cap_words) out[nwords] = cur;        \
      ++nwords;                                         \
      cur = 0;                                          \
      off = 0;                                          \
    }                                                   \
  } while (0)
  for (int i = 0; i < nruns; ++i) {
    const int run = runs[i];
    const int q = run >> k;
    const int rem = k > 0 ? (run & ((1 << k) - 1)) : 0;
    for (int z = 0; z < q; ++z) PUSH_BIT(0);
    PUSH_BIT(1);
    for (int s = 0; s < k; ++s) PUSH_BIT((rem >> s) & 1);
  }
  if (off != 0) {
    if (nwords < cap_words) out[nwords] = cur;
    ++nwords;
  }
#undef PUSH_BIT
  return nwords;
}

/*
 * Encode a dense packed bitmap [packed_rows, n] (int32 words, bit k&31 of row
 * k/32) into (words, offsets[nblk+1], meta[nblk]).  words_out must hold
 * nblk*128 words.  Returns the total word count.
 */
int64_t orc_gr_encode(const int32_t* packed, int packed_rows, int n, int kmin, int kmax, int force_raw,
                      int32_t* words_out, int32_t* offsets_out, int32_t* meta_out) {
  const int nkb = ceil_div(packed_rows, GR_PACKED_ROWS);
  const int nob = ceil_div(n, GR_TILE_OUT);
  uint32_t block[GR_WORDS];
  int32_t runs[GR_BITS];
  uint32_t coded[GR_WORDS + 1];
  int64_t total = 0;
  offsets_out[0] = 0;
  for (int kb = 0; kb < nkb; ++kb) {
    for (int ob = 0; ob < nob; ++ob) {
      const int bi = kb * nob + ob;
      gather_block(packed, packed_rows, n, kb, ob, block);
      const int nruns = block_zero_runs(block, runs);
      int64_t best_bits = (int64_t)GR_BITS + 1;
      int best_k = kmin;
      for (int k = kmin; k <= kmax; ++k) {
        const int64_t bits = orc_rice_bits(runs, nruns, k);
        if (bits < best_bits) {
          best_bits = bits;
          best_k = k;
        }
      }
      const int64_t coded_words = (best_bits + 31) / 32;
      if (force_raw || coded_words >= GR_WORDS) {
        for (int w = 0; w < GR_WORDS; ++w) words_out[total + w] = (int32_t)block[w];
        total += GR_WORDS;
        meta_out[bi] = GR_META_RAW;
      } else {
        const int nw = orc_rice_encode(runs, nruns, best_k, coded, GR_WORDS + 1);
        for (int w = 0; w < nw; ++w) words_out[total + w] = (int32_t)coded[w];
        total += nw;
        meta_out[bi] = best_k | (nruns << GR_META_ONES_SHIFT);
      }
      offsets_out[bi + 1] = (int32_t)total;
    }
  }
  return total;
}

/* ---------------------------------------------------------------- decoder */

/* read_block_gr_bit: TriSMoE_cuda_kernel.cu:321-323 */
static unsigned read_bit(const int32_t* words, int bit_idx) {
  return ((uint32_t)words[bit_idx >> 5] >> (bit_idx & 31)) & 1u;
}

/* read_block_gr_bits_upto_32: TriSMoE_cuda_kernel.cu:325-345 */
static unsigned read_bits_upto_32(const int32_t* words, int total_bits, int bit_pos, int count) {
  if (count <= 0 || bit_pos >= total_bits) return 0u;
  const int total_words = (total_bits + 31) >> 5;
  const int word_idx = bit_pos >> 5;
  const int bit_idx = bit_pos & 31;
  unsigned bits = (uint32_t)words[word_idx] >> bit_idx;
  const int bits_in_word = 32 - bit_idx;
  if (bits_in_word < count && word_idx + 1 < total_words) bits |= (uint32_t)words[word_idx + 1] << bits_in_word;
  if (count < 32) bits &= (1u << count) - 1u;
  return bits;
}

/* decode_block_gr_zero_run (general k): TriSMoE_cuda_kernel.cu:403-424 */
static int zero_run_general(const int32_t* words, int total_bits, int* bit_pos, int k) {
  int quotient = 0;
  while (*bit_pos < total_bits) {
    const unsigned bit = read_bit(words, *bit_pos);
    ++(*bit_pos);
    if (bit != 0u) break;
    ++quotient;
  }
  int remainder = 0;
  for (int shift = 0; shift < k && *bit_pos < total_bits; ++shift) {
    remainder |= (int)read_bit(words, *bit_pos) << shift;
    ++(*bit_pos);
  }
  return (quotient << k) | remainder;
}

static int ffs32(unsigned v) { return v ? __builtin_ctz(v) + 1 : 0; }

/* decode_block_gr_zero_run_k3 (k == 3 fast path): TriSMoE_cuda_kernel.cu:347-401 */
static int zero_run_k3(const int32_t* words, int total_bits, int* bit_pos) {
  if (*bit_pos >= total_bits) return 0;
  const int total_words = (total_bits + 31) >> 5;
  int quotient = 0;
  int word_idx = *bit_pos >> 5;
  int bit_idx = *bit_pos & 31;
  unsigned word = (uint32_t)words[word_idx];
  if (bit_idx != 0) word >>= bit_idx;
  for (;;) {
    if (word != 0u) {
      const int first_one = ffs32(word) - 1;
      quotient += first_one;
      *bit_pos += first_one + 1;
      word = (first_one + 1) >= 32 ? 0u : (word >> (first_one + 1));
      const int bits_left_in_word = 32 - bit_idx - (first_one + 1);
      const int remainder_bits = total_bits - *bit_pos;
      const int take = remainder_bits < 3 ? remainder_bits : 3;
      unsigned remainder = 0u;
      if (take > 0) {
        if (bits_left_in_word >= take) {
          remainder = word & ((1u << take) - 1u);
        } else {
          remainder = read_bits_upto_32(words, total_bits, *bit_pos, take) & 0x7u;
        }
      }
      *bit_pos += take;
      return (quotient << 3) | (int)remainder;
    }
    const int remaining = total_bits - *bit_pos;
    const int available = remaining < (32 - bit_idx) ? remaining : (32 - bit_idx);
    quotient += available;
    *bit_pos += available;
    if (*bit_pos >= total_bits) return quotient << 3;
    ++word_idx;
    bit_idx = 0;
    if (word_idx >= total_words) return quotient << 3;
    word = (uint32_t)words[word_idx];
  }
}

/*
 * decode_block_gr_block: TriSMoE_cuda_kernel.cu:426-479.
 * use_k3_fast_path selects the reference's k==3 specialisation (as the CUDA
 * code does); passing 0 decodes every k with the general bit-serial reader,
 * which lets the tests check that both reference paths agree.
 */
void orc_gr_decode_block_impl(const int32_t* words, const int32_t* offsets, const int32_t* meta, int block_idx,
                              int use_k3_fast_path, uint32_t* out) {
  memset(out, 0, GR_WORDS * sizeof(uint32_t));
  const int meta_word = meta[block_idx];
  const int word_begin = offsets[block_idx];
  const int word_end = offsets[block_idx + 1];
  const int word_count = word_end - word_begin;
  if (word_count <= 0) return;
  const int32_t* payload = words + word_begin;
  if ((meta_word & GR_META_RAW) != 0) {
    for (int w = 0; w < GR_WORDS && w < word_count; ++w) out[w] = (uint32_t)payload[w];
    return;
  }
  const int k = meta_word & GR_META_K_MASK;
  const int one_count = meta_word >> GR_META_ONES_SHIFT;
  const int total_bits = word_count * 32;
  int bit_pos = 0;
  int flat_pos = 0;
  for (int one = 0; one < one_count; ++one) {
    if (k == 3 && use_k3_fast_path) {
      flat_pos += zero_run_k3(payload, total_bits, &bit_pos);
    } else {
      flat_pos += zero_run_general(payload, total_bits, &bit_pos, k);
    }
    if (flat_pos >= GR_BITS) break;
    out[flat_pos >> 5] |= 1u << (flat_pos & 31);
    ++flat_pos;
  }
}

void orc_gr_decode_block(const int32_t* words, const int32_t* offsets, const int32_t* meta, int block_idx,
                         uint32_t* out) {
  orc_gr_decode_block_impl(words, offsets, meta, block_idx, 1, out);
}

/*
 * Decode every block of one expert back into the dense packed bitmap
 * [packed_rows, n] (the inverse of gather_block; decode_block_gr_tile,
 * TriSMoE_cuda_kernel.cu:481-502, addresses blocks the same way).
 */
void orc_gr_decode_dense(const int32_t* words, const int32_t* offsets, const int32_t* meta, int packed_rows, int n,
                         int32_t* dense) {
  const int nkb = ceil_div(packed_rows, GR_PACKED_ROWS);
  const int nob = ceil_div(n, GR_TILE_OUT);
  uint32_t block[GR_WORDS];
  for (int kb = 0; kb < nkb; ++kb) {
    for (int ob = 0; ob < nob; ++ob) {
      orc_gr_decode_block(words, offsets, meta, kb * nob + ob, block);
      for (int lpr = 0; lpr < GR_PACKED_ROWS; ++lpr) {
        const int row = kb * GR_PACKED_ROWS + lpr;
        if (row >= packed_rows) continue;
        for (int lo = 0; lo < GR_TILE_OUT; ++lo) {
          const int col = ob * GR_TILE_OUT + lo;
          if (col < n) dense[(int64_t)row * n + col] = (int32_t)block[lpr * GR_TILE_OUT + lo];
        }
      }
    }
  }
}

/* Predecode layout of the reference (TriSMoE_cuda_kernel.cu:4683-4718):
 * out[active][block][128] for the listed expert slots (negative slot => zeros). */
void orc_gr_predecode(const int32_t* words, const int32_t* offsets, const int32_t* meta, int words_stride,
                      int nblk, const int32_t* expert_ids, int num_active, int32_t* out) {
  for (int a = 0; a < num_active; ++a) {
    const int e = expert_ids[a];
    for (int b = 0; b < nblk; ++b) {
      uint32_t* dst = (uint32_t*)out + ((int64_t)a * nblk + b) * GR_WORDS;
      if (e < 0) {
        memset(dst, 0, GR_WORDS * sizeof(uint32_t));
        continue;
      }
      orc_gr_decode_block(words + (int64_t)e * words_stride, offsets + (int64_t)e * (nblk + 1),
                          meta + (int64_t)e * nblk, b, dst);
    }
  }
}
