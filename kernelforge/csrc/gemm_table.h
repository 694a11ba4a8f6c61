// Registry entry for one compiled GEMM tile configuration.
#pragma once

#include <stdint.h>

namespace kf {
namespace gemm {

// Kernel argument block (passed by value).
struct Args {
  const void* A;
  const void* B;
  const void* bias;
  void* C;
  int64_t M, N, K;
  int64_t lda_m, lda_k, ldb_k, ldb_n, ldc_m, ldc_n;
  int epilogue;
  int group_m;
  // Split-K (DMA pipeline only). With split_k > 1, tiles [0, full_tiles) run
  // one program each and the (tile, k-slice) iterations of the other tiles
  // are cut into tail_programs contiguous ranges, one program each; ws holds
  // two fp32 partial tiles per such program and tickets one counter per split
  // tile (zero between launches). split_k == 1 leaves the rest unused.
  int split_k;
  int64_t full_tiles;
  int64_t tail_programs;
  float* ws;
  unsigned* tickets;
};

struct Entry {
  int bm, bn, bk, waves, stages;
  int lds_bytes;
  const void* kernel;  // __global__ gemm_kernel<...> for this tile and loader pair
};

using TableFn = const Entry* (*)(int*);

}  // namespace gemm
}  // namespace kf
