// Block-GR predecode and dense-decode kernels.
//
// Predecode replaces Compact3TriSMoEGroupedBlockGRPredecodeKernel
// (TriSMoE_cuda_kernel.cu:4683-4718), which decodes each block serially on
// thread 0.  Here a workgroup builds the byte decode table in LDS once, then
// every group of S lanes decodes one block (tris_gr_span.h), so a 256-lane
// workgroup decodes 256/S blocks at once; the decoded words leave LDS as
// coalesced stores.  Work per block does not depend on S; more lanes per block
// shorten each lane's serial span (latency), fewer cut the shuffle steps, so S
// is chosen from the block count.
#include "tris_gr_span.h"

namespace tris {

constexpr int kSpanThreads = 256;

template <int S>
__global__ __launch_bounds__(kSpanThreads) void gr_decode_span_kernel(
    int32_t* __restrict__ decoded, const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ num_active_dev,
    const int32_t* __restrict__ words, const int32_t* __restrict__ offsets, const int32_t* __restrict__ meta,
    int words_stride, int nblk, int num_experts, int dense_rows, int dense_cols, int num_out_blocks) {
  constexpr int kBlocksPerWg = kSpanThreads / S;
  __shared__ GrTables tab;
  __shared__ uint32_t outb[kBlocksPerWg][kGrWords];
  const int slot = blockIdx.y;
  if (num_active_dev != nullptr && slot >= *num_active_dev) return;  // uniform over the workgroup
  const int tid = threadIdx.x;
  const int g = tid / S;
  const int j = tid % S;
  const int block0 = blockIdx.x * kBlocksPerWg;
  const int block = block0 + g;
  const int expert = expert_ids[slot];
  const bool evalid = expert >= 0 && expert < num_experts;
  GrSpan<S> sp;
  gr_span_load<S>(sp, evalid ? words + static_cast<int64_t>(expert) * words_stride : nullptr,
                  evalid ? offsets + static_cast<int64_t>(expert) * (nblk + 1) : nullptr,
                  evalid ? meta + static_cast<int64_t>(expert) * nblk : nullptr, block, evalid && block < nblk, j);
  gr_tables_to_lds(&tab);
  for (int idx = tid; idx < kBlocksPerWg * kGrWords; idx += kSpanThreads) outb[idx / kGrWords][idx % kGrWords] = 0u;
  __syncthreads();
  gr_decode_block_group<S>(sp, &tab, outb[g], j);
  __syncthreads();
  if (dense_rows == 0) {
    // predecode layout [slot][block][128]
    int32_t* dst = decoded + (static_cast<int64_t>(slot) * nblk + block0) * kGrWords;
    for (int idx = tid; idx < kBlocksPerWg * kGrWords; idx += kSpanThreads) {
      if (block0 + idx / kGrWords < nblk) dst[idx] = static_cast<int32_t>(outb[idx / kGrWords][idx % kGrWords]);
    }
  } else {
    // dense layout [slot][packed_rows][N]
    int32_t* dst = decoded + static_cast<int64_t>(slot) * dense_rows * dense_cols;
    for (int idx = tid; idx < kBlocksPerWg * kGrWords; idx += kSpanThreads) {
      const int b = block0 + idx / kGrWords;
      if (b >= nblk) continue;
      const int w = idx % kGrWords;
      const int row = (b / num_out_blocks) * kGrPackedRows + w / kTileOut;
      const int col = (b % num_out_blocks) * kTileOut + w % kTileOut;
      if (row < dense_rows && col < dense_cols) {
        dst[static_cast<int64_t>(row) * dense_cols + col] = static_cast<int32_t>(outb[idx / kGrWords][w]);
      }
    }
  }
}

int launch_gr_decode(int32_t* out, const int32_t* expert_ids, const int32_t* num_active_dev, int num_slots,
                     const int32_t* words, const int32_t* offsets, const int32_t* meta, int num_experts,
                     int words_stride, int packed_rows, int outfeatures, bool dense, void* stream, const char* who) {
  const int nob = ceil_div(outfeatures, kTileOut);
  const int nblk = ceil_div(packed_rows, kGrPackedRows) * nob;
  if (num_slots == 0 || nblk == 0) return TRIS_OK;
  TRIS_REQUIRE(out && expert_ids && offsets && meta && words, "%s: null pointer", who);
  TRIS_REQUIRE(num_slots <= 65535, "%s: too many experts (%d)", who, num_slots);
  const int64_t total = static_cast<int64_t>(nblk) * num_slots;
  const int S = total >= 8192 ? 8 : (total >= 2048 ? 16 : 32);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int dr = dense ? packed_rows : 0;
  const int dc = dense ? outfeatures : 0;
  if (S == 8) {
    hipLaunchKernelGGL((gr_decode_span_kernel<8>), dim3(ceil_div(nblk, kSpanThreads / 8), num_slots),
                       dim3(kSpanThreads), 0, s, out, expert_ids, num_active_dev, words, offsets, meta, words_stride,
                       nblk, num_experts, dr, dc, nob);
  } else if (S == 16) {
    hipLaunchKernelGGL((gr_decode_span_kernel<16>), dim3(ceil_div(nblk, kSpanThreads / 16), num_slots),
                       dim3(kSpanThreads), 0, s, out, expert_ids, num_active_dev, words, offsets, meta, words_stride,
                       nblk, num_experts, dr, dc, nob);
  } else {
    hipLaunchKernelGGL((gr_decode_span_kernel<32>), dim3(ceil_div(nblk, kSpanThreads / 32), num_slots),
                       dim3(kSpanThreads), 0, s, out, expert_ids, num_active_dev, words, offsets, meta, words_stride,
                       nblk, num_experts, dr, dc, nob);
  }
  return check_launch(who);
}

}  // namespace tris

using namespace tris;

extern "C" int tris_grouped_block_gr_predecode(int32_t* decoded, const int32_t* expert_ids, int32_t num_active,
                                               const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                                               const int32_t* q_gmap_gr_meta, int32_t num_experts,
                                               int32_t words_stride, int32_t packed_rows, int32_t outfeatures,
                                               void* stream) {
  TRIS_REQUIRE(num_active >= 0 && packed_rows >= 0 && outfeatures >= 0 && words_stride >= 0 && num_experts >= 0,
               "predecode: negative size");
  return launch_gr_decode(decoded, expert_ids, nullptr, num_active, q_gmap_gr_words, q_gmap_gr_offsets,
                          q_gmap_gr_meta, num_experts, words_stride, packed_rows, outfeatures, false, stream,
                          "tris_grouped_block_gr_predecode");
}

extern "C" int tris_gr_decode_dense(const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                                    const int32_t* q_gmap_gr_meta, int32_t num_experts, int32_t words_stride,
                                    const int32_t* expert_ids, int32_t num, int32_t packed_rows,
                                    int32_t outfeatures, int32_t* dense, void* stream) {
  TRIS_REQUIRE(num >= 0 && packed_rows >= 0 && outfeatures >= 0 && words_stride >= 0 && num_experts >= 0,
               "decode_dense: negative size");
  return launch_gr_decode(dense, expert_ids, nullptr, num, q_gmap_gr_words, q_gmap_gr_offsets, q_gmap_gr_meta,
                          num_experts, words_stride, packed_rows, outfeatures, true, stream, "tris_gr_decode_dense");
}
