// Block-GR predecode and dense-decode kernels (one wavefront per GR block).
//
// Predecode replaces Compact3TriSMoEGroupedBlockGRPredecodeKernel
// (TriSMoE_cuda_kernel.cu:4683-4718), which decodes each block serially on
// thread 0; here a whole wavefront decodes a block (tris_gr_decode.h) and
// the 128 decoded words leave LDS as two coalesced 256-byte stores.
#include "tris_gr_decode.h"

namespace tris {

constexpr int kDecodeWavesPerBlock = 4;

// decoded[a][b][128] for b < nblk; grid = (ceil(nblk / 4), num_active).
__global__ __launch_bounds__(kWave * kDecodeWavesPerBlock) void gr_predecode_kernel(
    int32_t* __restrict__ decoded, const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ words,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ meta, int words_stride, int nblk,
    int num_experts) {
  __shared__ uint32_t lds[kDecodeWavesPerBlock][kGrWords];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int block = blockIdx.x * kDecodeWavesPerBlock + wave;
  const int active = blockIdx.y;
  if (block >= nblk) return;  // whole wave exits; no block-wide barrier follows
  const int expert = expert_ids[active];
  uint32_t* out = lds[wave];
  if (expert >= 0 && expert < num_experts) {
    gr_decode_block_wave(words + static_cast<int64_t>(expert) * words_stride,
                         offsets + static_cast<int64_t>(expert) * (nblk + 1),
                         meta + static_cast<int64_t>(expert) * nblk, block, out);
  } else {
    out[lane] = 0u;
    out[lane + kWave] = 0u;
    wave_sync_lds();
  }
  int32_t* dst = decoded + (static_cast<int64_t>(active) * nblk + block) * kGrWords;
  dst[lane] = static_cast<int32_t>(out[lane]);
  dst[lane + kWave] = static_cast<int32_t>(out[lane + kWave]);
}

// dense[i][packed_rows][N] for expert expert_ids[i]; grid = (ceil(nblk / 4), num).
__global__ __launch_bounds__(kWave * kDecodeWavesPerBlock) void gr_decode_dense_kernel(
    int32_t* __restrict__ dense, const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ words,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ meta, int words_stride, int packed_rows,
    int outfeatures, int nblk, int num_out_blocks, int num_experts) {
  __shared__ uint32_t lds[kDecodeWavesPerBlock][kGrWords];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int block = blockIdx.x * kDecodeWavesPerBlock + wave;
  const int item = blockIdx.y;
  if (block >= nblk) return;
  const int expert = expert_ids[item];
  uint32_t* out = lds[wave];
  if (expert >= 0 && expert < num_experts) {
    gr_decode_block_wave(words + static_cast<int64_t>(expert) * words_stride,
                         offsets + static_cast<int64_t>(expert) * (nblk + 1),
                         meta + static_cast<int64_t>(expert) * nblk, block, out);
  } else {
    out[lane] = 0u;
    out[lane + kWave] = 0u;
    wave_sync_lds();
  }
  const int kb = block / num_out_blocks;
  const int ob = block % num_out_blocks;
  const int col = ob * kTileOut + lane;
  int32_t* dst = dense + static_cast<int64_t>(item) * packed_rows * outfeatures;
#pragma unroll
  for (int lpr = 0; lpr < kGrPackedRows; ++lpr) {
    const int row = kb * kGrPackedRows + lpr;
    if (row < packed_rows && col < outfeatures) {
      dst[static_cast<int64_t>(row) * outfeatures + col] = static_cast<int32_t>(out[lpr * kTileOut + lane]);
    }
  }
}

}  // namespace tris

using namespace tris;

extern "C" int tris_grouped_block_gr_predecode(int32_t* decoded, const int32_t* expert_ids, int32_t num_active,
                                               const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                                               const int32_t* q_gmap_gr_meta, int32_t num_experts,
                                               int32_t words_stride, int32_t packed_rows, int32_t outfeatures,
                                               void* stream) {
  TRIS_REQUIRE(num_active >= 0 && packed_rows >= 0 && outfeatures >= 0 && words_stride >= 0,
               "predecode: negative size");
  const int nblk = ceil_div(packed_rows, kGrPackedRows) * ceil_div(outfeatures, kTileOut);
  if (num_active == 0 || nblk == 0) return TRIS_OK;
  TRIS_REQUIRE(decoded && expert_ids && q_gmap_gr_offsets && q_gmap_gr_meta && q_gmap_gr_words,
               "predecode: null pointer");
  TRIS_REQUIRE(num_active <= 65535, "predecode: too many active experts (%d)", num_active);
  dim3 grid(ceil_div(nblk, kDecodeWavesPerBlock), num_active);
  hipLaunchKernelGGL(gr_predecode_kernel, grid, dim3(kWave * kDecodeWavesPerBlock), 0,
                     static_cast<hipStream_t>(stream), decoded, expert_ids, q_gmap_gr_words, q_gmap_gr_offsets,
                     q_gmap_gr_meta, words_stride, nblk, num_experts);
  return check_launch("gr_predecode_kernel");
}

extern "C" int tris_gr_decode_dense(const int32_t* q_gmap_gr_words, const int32_t* q_gmap_gr_offsets,
                                    const int32_t* q_gmap_gr_meta, int32_t num_experts, int32_t words_stride,
                                    const int32_t* expert_ids, int32_t num, int32_t packed_rows,
                                    int32_t outfeatures, int32_t* dense, void* stream) {
  TRIS_REQUIRE(num >= 0 && packed_rows >= 0 && outfeatures >= 0 && words_stride >= 0, "decode_dense: negative size");
  const int nob = ceil_div(outfeatures, kTileOut);
  const int nblk = ceil_div(packed_rows, kGrPackedRows) * nob;
  if (num == 0 || nblk == 0) return TRIS_OK;
  TRIS_REQUIRE(dense && expert_ids && q_gmap_gr_offsets && q_gmap_gr_meta && q_gmap_gr_words,
               "decode_dense: null pointer");
  TRIS_REQUIRE(num <= 65535, "decode_dense: too many experts (%d)", num);
  dim3 grid(ceil_div(nblk, kDecodeWavesPerBlock), num);
  hipLaunchKernelGGL(gr_decode_dense_kernel, grid, dim3(kWave * kDecodeWavesPerBlock), 0,
                     static_cast<hipStream_t>(stream), dense, expert_ids, q_gmap_gr_words, q_gmap_gr_offsets,
                     q_gmap_gr_meta, words_stride, packed_rows, outfeatures, nblk, nob, num_experts);
  return check_launch("gr_decode_dense_kernel");
}
