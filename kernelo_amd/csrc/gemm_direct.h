// Direct-to-LDS MFMA GEMM for 16-bit inputs on gfx950 (the fast path).
//
// Differences from the register-staged kernel in gemm_impl.h:
//   * Global -> LDS with global_load_lds_dwordx4: each lane's 16 bytes land at
//     (wave base + 16*lane) in LDS without passing through VGPRs, so the
//     staging registers and the ds_write instructions disappear and the
//     accumulators get the register file.
//   * No padding: LDS rows are dense and 16-byte chunks are XOR-swizzled by
//     row, which is what keeps both the DMA writes (a wave fills 1 KiB of
//     consecutive LDS) and the fragment reads bank-conflict free.
//   * Row-major B stays n-contiguous in LDS and is read with
//     ds_read_b64_tr_b16: within a 16-lane group, lane i addressing
//     (row0 + i/4, col0 + 4*(i%4)) receives column col0+i of rows
//     row0..row0+3, which is the MFMA B-operand layout. Two such reads give
//     the 8 consecutive k a v_mfma_f32_16x16x32 lane needs.
//
// Requirements (checked on the host): 16-bit dtype, A k-contiguous with a
// 16-byte aligned base and row pitch, B either n-contiguous (BLAYOUT 0) or
// k-contiguous (BLAYOUT 1) with the same alignment, N (BLAYOUT 0) and K
// multiples of 8. BK is 64: one A row of a k-slice is exactly 128 bytes.
// M/N edges clamp rows/columns (results discarded); a partial last k-slice
// has its chunks past K zeroed in LDS after the DMA lands.
#pragma once

#include "gemm_impl.h"

namespace kf {
namespace gemm {

#define KF_LDS __attribute__((address_space(3)))

typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __bf16 bf16x4_t __attribute__((__vector_size__(4 * sizeof(__bf16))));

constexpr int kDirectBK = 64;

// 4 k-rows of one column from an n-contiguous LDS tile (see header comment).
template <typename T>
__device__ __forceinline__ uint64_t ds_read_tr4(const char* p);
template <>
__device__ __forceinline__ uint64_t ds_read_tr4<f16>(const char* p) {
  fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((KF_LDS fp16x4_t*)(p));
  return __builtin_bit_cast(uint64_t, v);
}
template <>
__device__ __forceinline__ uint64_t ds_read_tr4<bf16>(const char* p) {
  bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((KF_LDS bf16x4_t*)(p));
  return __builtin_bit_cast(uint64_t, v);
}

// DMA 16 bytes per lane into LDS at lds_wave_base + 16*lane.
__device__ __forceinline__ void dma16(const void* gptr, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(gptr, (KF_LDS void*)(lds_wave_base), 16, 0, 0);
}

__device__ __forceinline__ void wait_dma() {
  // s_waitcnt vmcnt(0), leaving expcnt/lgkmcnt unconstrained (gfx9 encoding).
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

template <int BM, int BN, int WAVES, int BLAYOUT>
struct DirectTile {
  static constexpr int BK = kDirectBK;
  static constexpr int NT = WAVES * kWave;
  static constexpr int WM = WaveGrid<WAVES, BM, BN>::WM;
  static constexpr int WN = WaveGrid<WAVES, BM, BN>::WN;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int FM = TM / 16;
  static constexpr int FN = TN / 16;
  // Byte sizes of one stage.
  static constexpr int kABytes = BM * BK * 2;
  static constexpr int kBBytes = BN * BK * 2;
  static constexpr int kStageBytes = kABytes + kBBytes;
  static constexpr int kLdsBytes = 2 * kStageBytes;  // static LDS (two stage objects)
  // 16-byte chunks per stage and DMA instructions per lane.
  static constexpr int kAChunks = BM * BK / 8;
  static constexpr int kBChunks = BN * BK / 8;
  static constexpr int kAIters = kAChunks / NT;
  static constexpr int kBIters = kBChunks / NT;
  // B row (BLAYOUT 0: one k-row of BN elements) in chunks.
  static constexpr int kBRowChunks = BN / 8;
  static_assert(kAChunks % NT == 0 && kBChunks % NT == 0, "DMA must tile the stage exactly");
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be whole 16x16 fragments");
  static_assert(BLAYOUT == 1 || BN >= 64, "n-contiguous B swizzle needs >= 8 chunks per row");
};

// Swizzled chunk position within a row.
__device__ __forceinline__ int swz_k(int chunk, int row) { return chunk ^ (row & 7); }   // k-contig rows
__device__ __forceinline__ int swz_n(int chunk, int row) { return chunk ^ ((row & 3) << 1); }  // n-contig rows

template <typename T, int BM, int BN, int WAVES, int BLAYOUT>
__global__ __launch_bounds__(WAVES * 64) void gemm_direct_kernel(Args args) {
  using Tl = DirectTile<BM, BN, WAVES, BLAYOUT>;
  constexpr int BK = Tl::BK;
  constexpr int NT = Tl::NT;
  constexpr int FM = Tl::FM, FN = Tl::FN;

  // One LDS object per stage: with distinct objects the compiler can prove
  // that the DMA into one stage does not alias fragment reads of the other,
  // so it does not wait for the DMA before the reads.
  __shared__ __attribute__((aligned(16))) char stage0[Tl::kStageBytes];
  __shared__ __attribute__((aligned(16))) char stage1[Tl::kStageBytes];

  const T* __restrict__ A = static_cast<const T*>(args.A);
  const T* __restrict__ B = static_cast<const T*>(args.B);
  const int64_t M = args.M, N = args.N, K = args.K;

  // ---- tile order: regroup per XCD, then GROUP_M bands (as gemm_kernel) ----
  const int64_t tiles_m = ceil_div(M, BM);
  const int64_t tiles_n = ceil_div(N, BN);
  const int64_t ntiles = tiles_m * tiles_n;
  int64_t pid = blockIdx.x;
  if (ntiles % kNumXcd == 0) pid = (pid % kNumXcd) * (ntiles / kNumXcd) + pid / kNumXcd;
  const int64_t gm = args.group_m;
  const int64_t in_group = gm * tiles_n;
  const int64_t group = pid / in_group;
  const int64_t first_m = group * gm;
  const int64_t size_m = (tiles_m - first_m < gm) ? (tiles_m - first_m) : gm;
  const int64_t m0 = (first_m + (pid % in_group) % size_m) * BM;
  const int64_t n0 = ((pid % in_group) / size_m) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / Tl::WN;
  const int wn = wave % Tl::WN;

  // ---- DMA sources ------------------------------------------------------------
  // Each lane owns fixed chunks of a stage: a row pointer plus the chunk's k
  // offset within the slice (A and k-contiguous B), or a column pointer plus
  // the slice-relative k row (n-contiguous B). Chunk q = j*NT + tid is
  // written to LDS slot q; its logical chunk is the slot position XOR the
  // row's swizzle.
  const T* a_row[Tl::kAIters];
  int a_k[Tl::kAIters];
#pragma unroll
  for (int j = 0; j < Tl::kAIters; ++j) {
    const int q = j * NT + tid;
    const int r = q >> 3;
    int64_t row = m0 + r;
    row = row < M ? row : M - 1;
    a_row[j] = A + row * args.lda_m;
    a_k[j] = swz_k(q & 7, r) * 8;
  }
  const T* b_ptr[Tl::kBIters];
  int b_k[Tl::kBIters];
#pragma unroll
  for (int j = 0; j < Tl::kBIters; ++j) {
    const int q = j * NT + tid;
    if constexpr (BLAYOUT == 0) {
      const int r = q / Tl::kBRowChunks;  // k row within the slice
      int64_t col = n0 + swz_n(q % Tl::kBRowChunks, r) * 8;
      col = col < N ? col : N - 8;
      b_ptr[j] = B + col;
      b_k[j] = r;
    } else {
      const int r = q >> 3;  // n row
      int64_t row = n0 + r;
      row = row < N ? row : N - 1;
      b_ptr[j] = B + row * args.ldb_n;
      b_k[j] = swz_k(q & 7, r) * 8;
    }
  }

  // Enqueue the DMA of k-slice kt into the stage at `base`. Sources past K
  // (only in a partial last slice) are clamped to the last valid k so every
  // address stays inside the operand; zero_tail() later overwrites them.
  auto issue = [&](char* base, int64_t kt) {
    const int64_t k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < Tl::kAIters; ++j) {
      int64_t k = k0 + a_k[j];
      k = k < K ? k : K - 8;
      dma16(a_row[j] + k, base + (j * NT + wave * 64) * 16);
    }
#pragma unroll
    for (int j = 0; j < Tl::kBIters; ++j) {
      int64_t k = k0 + b_k[j];
      if constexpr (BLAYOUT == 0) {
        k = k < K ? k : K - 1;
        dma16(b_ptr[j] + k * args.ldb_k, base + Tl::kABytes + (j * NT + wave * 64) * 16);
      } else {
        k = k < K ? k : K - 8;
        dma16(b_ptr[j] + k, base + Tl::kABytes + (j * NT + wave * 64) * 16);
      }
    }
  };

  // Zero the chunks of a partial k-slice that lie past K (after its DMA landed).
  auto zero_tail = [&](char* base, int64_t k0) {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < Tl::kAIters; ++j) {
      const int q = j * NT + tid;
      const int c = swz_k(q & 7, q >> 3);
      if (k0 + c * 8 >= K) *reinterpret_cast<u32x4*>(base + q * 16) = z;
    }
#pragma unroll
    for (int j = 0; j < Tl::kBIters; ++j) {
      const int q = j * NT + tid;
      int kk;
      if constexpr (BLAYOUT == 0)
        kk = q / Tl::kBRowChunks;
      else
        kk = swz_k(q & 7, q >> 3) * 8;
      if (k0 + kk >= K) *reinterpret_cast<u32x4*>(base + Tl::kABytes + q * 16) = z;
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int g = lane >> 4;   // lane group: k offset 8*g within a 32-wide step
  const int li = lane & 15;  // row (A) / column (B) within a fragment

  auto compute = [&](const char* As) {
    const char* Bs = As + Tl::kABytes;
#pragma unroll
    for (int kc = 0; kc < BK / 32; ++kc) {
      u32x4 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * Tl::TM + i * 16 + li;
        af[i] = *reinterpret_cast<const u32x4*>(As + r * 128 + swz_k(kc * 4 + g, r) * 16);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (BLAYOUT == 0) {
          // Two transposing reads: k rows kc*32 + 8g + {0..3, 4..7} of column li.
          const int col = wn * Tl::TN + j * 16 + (li & 3) * 4;
          uint64_t lo, hi;
          {
            const int r = kc * 32 + 8 * g + (li >> 2);
            const int c = col >> 3;
            lo = ds_read_tr4<T>(Bs + r * (BN * 2) + swz_n(c, r) * 16 + (col & 7) * 2);
          }
          {
            const int r = kc * 32 + 8 * g + 4 + (li >> 2);
            const int c = col >> 3;
            hi = ds_read_tr4<T>(Bs + r * (BN * 2) + swz_n(c, r) * 16 + (col & 7) * 2);
          }
          bfr[j] = u32x4{static_cast<uint32_t>(lo), static_cast<uint32_t>(lo >> 32),
                         static_cast<uint32_t>(hi), static_cast<uint32_t>(hi >> 32)};
        } else {
          const int r = wn * Tl::TN + j * 16 + li;
          bfr[j] = *reinterpret_cast<const u32x4*>(Bs + r * 128 + swz_k(kc * 4 + g, r) * 16);
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Mma<T>::run(af[i], bfr[j], acc[i][j]);
    }
  };

  // ---- main loop: DMA of slice t+1 overlaps the MFMAs of slice t -----------
  // Unrolled by two so that each half names its stage objects at compile time.
  const int64_t nk = ceil_div(K, BK);
  auto step = [&](char* cur, char* nxt, int64_t kt) {
    const bool more = kt + 1 < nk;
    if (more) issue(nxt, kt + 1);
    compute(cur);
    if (more) {
      wait_dma();
      if ((kt + 2) * BK > K) zero_tail(nxt, (kt + 1) * BK);
    }
    __syncthreads();
  };
  if (nk > 0) {
    issue(stage0, 0);
    wait_dma();
    if (BK > K) zero_tail(stage0, 0);
    __syncthreads();
    for (int64_t kt = 0; kt < nk; kt += 2) {
      step(stage0, stage1, kt);
      if (kt + 1 < nk) step(stage1, stage0, kt + 1);
    }
  }

  // ---- epilogue -------------------------------------------------------------
  T* __restrict__ C = static_cast<T*>(args.C);
  const T* __restrict__ bias = static_cast<const T*>(args.bias);
  const bool gelu = args.epilogue == KF_EPILOGUE_BIAS_GELU;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * Tl::TN + j * 16 + li;
    if (col >= N) continue;
    const float bcol = gelu ? to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm * Tl::TM + i * 16 + g * 4 + r;
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (gelu) v = gelu_tanh(v + bcol);
        C[row * args.ldc_m + col * args.ldc_n] = from_f32<T>(v);
      }
    }
  }
}

}  // namespace gemm
}  // namespace kf
