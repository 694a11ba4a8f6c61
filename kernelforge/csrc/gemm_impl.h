// Tiled MFMA GEMM for gfx950, C = A @ B (+ bias, tanh-GELU), fp32 accumulation.
//
// Counterpart of the reference's matmul_kernel (kernels/matmul.py:54-113) and
// fused_linear_gelu_kernel (kernels/fused_linear.py:49-104): same contract
// (any strides, masked M/N/K tails, output rounded once to the input dtype),
// different machine.
//
// Structure of one workgroup (WAVES wavefronts of 64 lanes):
//   * The BM x BN output tile is split over a WM x WN grid of waves; each
//     wave owns (BM/WM) x (BN/WN) outputs as 16x16 MFMA fragments.
//   * A and B k-slices of depth BK are staged in LDS, both k-contiguous
//     ([row][BK + pad]), double buffered: global loads for slice t+1 are in
//     flight while slice t is multiplied, one barrier per slice.
//   * The pad (16 bytes per row) makes the 16-byte fragment reads
//     bank-conflict free.
//   * MFMA: v_mfma_f32_16x16x32_{f16,bf16} for 16-bit inputs (8 elements per
//     lane), v_mfma_f32_16x16x4_f32 x4 for fp32. Which k each lane carries
//     does not matter as long as A and B agree, so both read the same
//     16-byte chunk of their k-contiguous LDS row.
//   * Row-major B (n-contiguous, the common case) is transposed in registers
//     on its way to LDS: a lane loads R consecutive k-rows of 16 bytes and
//     writes 4-byte (k, k+1) pairs per column.
//   * Launch order: workgroups are dealt round-robin to the 8 XCDs, each with
//     its own L2, so consecutive tile indices are first regrouped per XCD and
//     then walked in GROUP_M-row bands, keeping A and B strips that share
//     rows/columns inside one L2.
#pragma once

#include <math.h>

#include "common.h"
#include "gemm_table.h"

namespace kf {
namespace gemm {

enum Loader : int {
  kLoadVecK = 0,   // 16-byte loads along k (k-contiguous rows)
  kLoadVecN = 1,   // 16-byte loads along n (row-major B), transposed into LDS
  kLoadScalar = 2  // element loads with arbitrary strides
};

constexpr int kNumXcd = 8;
constexpr float kGeluC = 1.5957691216057308f;  // 2*sqrt(2/pi)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float gelu_tanh(float a) {
  // 0.5a(1 + tanh(z)) with tanh(z) = 2/(1+exp(-2z)) - 1  =>  a / (1 + exp(-2z)).
  // The quotient uses the hardware reciprocal (v_rcp_f32, 1 ulp) rather than
  // the IEEE division sequence: the result is rounded to the output dtype and
  // gated at 5e-3 (16-bit) or 1e-5 (fp32), and rcp(inf) = 0 keeps the
  // saturated negative tail at -0.
  const float inner = kGeluC * (a + 0.044715f * a * a * a);
  return a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-inner * kLog2e));
}

template <typename T>
struct Mma;

template <>
struct Mma<f16> {
  static constexpr int KC = 32;  // k per MFMA step: 4 lane groups x 8
  __device__ __forceinline__ static void run(const u32x4& a, const u32x4& b, f32x4& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mma<bf16> {
  static constexpr int KC = 32;
  __device__ __forceinline__ static void run(const u32x4& a, const u32x4& b, f32x4& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mma<float> {
  static constexpr int KC = 16;  // 4 lane groups x 4, issued as four 16x16x4 steps
  __device__ __forceinline__ static void run(const u32x4& a, const u32x4& b, f32x4& c) {
    // Cast the whole vector, then take elements: element-wise bit casts of
    // an ext-vector subscript were folded to element 0 by this compiler.
    const f32x4 af = __builtin_bit_cast(f32x4, a);
    const f32x4 bf = __builtin_bit_cast(f32x4, b);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], c, 0, 0, 0);
  }
};

template <int WAVES, int BM, int BN>
struct WaveGrid {
  // 4 waves: 2x2. 8 waves: 4x2 when the tile is at least as tall as wide, else 2x4.
  static constexpr int WM = (WAVES == 4) ? 2 : ((WAVES == 8) ? (BM >= BN ? 4 : 2) : 1);
  static constexpr int WN = WAVES / WM;
};

template <typename T, int BM, int BN, int BK, int WAVES>
struct Tile {
  static constexpr int V = Vec<T>::N;          // elements per 16 bytes
  static constexpr int NT = WAVES * kWave;     // lanes per workgroup
  static constexpr int LDK = BK + V;           // padded LDS row, elements
  static constexpr int WM = WaveGrid<WAVES, BM, BN>::WM;
  static constexpr int WN = WaveGrid<WAVES, BM, BN>::WN;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int FM = TM / 16;
  static constexpr int FN = TN / 16;
  static constexpr int KC = Mma<T>::KC;
  static constexpr int R = 4 / sizeof(T);      // k-rows per transposed dword (VecN loader)
  static constexpr int kLdsA = BM * LDK;       // elements per stage
  static constexpr int kLdsB = BN * LDK;
  static constexpr int kLdsBytes = 2 * (kLdsA + kLdsB) * sizeof(T);
  // Global->LDS work items per lane, rounded up (guarded).
  static constexpr int kVecItemsA = (BM * BK / V + NT - 1) / NT;
  static constexpr int kVecItemsBk = (BN * BK / V + NT - 1) / NT;
  static constexpr int kVecItemsBn = ((BK / R) * (BN / V) + NT - 1) / NT;
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be whole 16x16 fragments");
  static_assert(BK % KC == 0, "BK must be a multiple of the MFMA k step");
  static_assert(BK % (R * 1) == 0 && BN % V == 0, "vector loaders need whole vectors");
};

// ---------------------------------------------------------------------------
// Global -> register staging. Each loader fills `regs` for k-slice k0 and
// later writes them to one LDS stage. Rows past M/N are clamped (their
// results are never stored); k past K is zero-filled.
// ---------------------------------------------------------------------------

// A or B with 16-byte vectors along k. `rows` = BM (A) or BN (B).
template <typename T, int ROWS, int BK, int NT>
struct VecKLoader {
  static constexpr int V = Vec<T>::N;
  static constexpr int PER_ROW = BK / V;
  static constexpr int ITEMS = (ROWS * PER_ROW + NT - 1) / NT;
  u32x4 regs[ITEMS];

  // FULL: the whole k-slice lies inside K (no masking in the steady state).
  template <bool FULL>
  __device__ __forceinline__ void load(const T* base, int64_t ld_row, int64_t row0, int64_t nrows,
                                       int64_t k0, int64_t K, int tid) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int item = tid + j * NT;
      if ((ROWS * PER_ROW) % NT != 0 && item >= ROWS * PER_ROW) break;
      const int r = item / PER_ROW;
      const int kv = item % PER_ROW;
      int64_t row = row0 + r;
      row = row < nrows ? row : nrows - 1;
      const T* p = base + row * ld_row + k0 + kv * V;
      if constexpr (FULL) {
        regs[j] = *reinterpret_cast<const u32x4*>(p);
      } else {
        T tmp[V];
#pragma unroll
        for (int e = 0; e < V; ++e)
          tmp[e] = (k0 + kv * V + e < K) ? p[e] : static_cast<T>(0.f);
        __builtin_memcpy(&regs[j], tmp, 16);
      }
    }
  }

  __device__ __forceinline__ void store(T* lds, int tid) const {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int item = tid + j * NT;
      if ((ROWS * PER_ROW) % NT != 0 && item >= ROWS * PER_ROW) break;
      const int r = item / PER_ROW;
      const int kv = item % PER_ROW;
      *reinterpret_cast<u32x4*>(lds + r * (BK + V) + kv * V) = regs[j];
    }
  }
};

// A or B with element loads at arbitrary strides (misaligned rows, views).
// Element (row, k) lives at base + row*ld_row + k*ld_k. The layouts it serves
// are the slow fallback, so it trades overlap for registers: load_to_lds()
// writes each 16-byte LDS chunk as soon as its elements arrive (the next
// stage is free while the current one is multiplied) and keeps nothing live
// across the compute.
template <typename T, int ROWS, int BK, int NT>
struct ScalarLoader {
  static constexpr int V = Vec<T>::N;
  static constexpr int PER_ROW = BK / V;
  static constexpr int ITEMS = (ROWS * PER_ROW + NT - 1) / NT;

  template <bool FULL>
  __device__ __forceinline__ void load_to_lds(T* lds, const T* base, int64_t ld_row, int64_t ld_k,
                                              int64_t row0, int64_t nrows, int64_t k0, int64_t K,
                                              int tid) const {
#pragma unroll 1
    for (int j = 0; j < ITEMS; ++j) {
      const int item = tid + j * NT;
      if (item >= ROWS * PER_ROW) break;
      const int r = item / PER_ROW;
      const int kv = item % PER_ROW;
      int64_t row = row0 + r;
      row = row < nrows ? row : nrows - 1;
      const int64_t kb = k0 + kv * V;
      const T* p = base + row * ld_row + kb * ld_k;
      T tmp[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        tmp[e] = (FULL || kb + e < K) ? *p : static_cast<T>(0.f);
        p += ld_k;
      }
      u32x4 raw;
      __builtin_memcpy(&raw, tmp, 16);
      *reinterpret_cast<u32x4*>(lds + r * (BK + V) + kv * V) = raw;
    }
  }
};

// Row-major B: 16-byte vectors along n from R consecutive k-rows, transposed
// in registers into one dword per column holding R consecutive k. Lanes walk
// k fastest so each LDS write instruction covers consecutive dwords of a row.
template <typename T, int BN, int BK, int NT>
struct VecNLoader {
  static constexpr int V = Vec<T>::N;
  static constexpr int R = 4 / sizeof(T);
  static constexpr int KR = BK / R;           // dword columns per LDS row
  static constexpr int SUBS = KR * (BN / V);  // R x V sub-blocks per slice
  static constexpr int ITEMS = (SUBS + NT - 1) / NT;
  u32x4 regs[ITEMS][R];

  template <bool FULL>
  __device__ __forceinline__ void load(const T* base, int64_t ldb_k, int64_t n0, int64_t N,
                                       int64_t k0, int64_t K, int tid) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int item = tid + j * NT;
      if (SUBS % NT != 0 && item >= SUBS) break;
      const int kr = item % KR;
      const int nv = item / KR;
      int64_t col = n0 + nv * V;
      // Clamp a whole vector that starts past N; a vector straddling N reads
      // only valid columns (N is a multiple of V whenever this loader is chosen).
      col = col < N ? col : N - V;
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int64_t k = k0 + kr * R + q;
        if (FULL || k < K)
          regs[j][q] = *reinterpret_cast<const u32x4*>(base + k * ldb_k + col);
        else
          regs[j][q] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  __device__ __forceinline__ void store(T* lds, int tid) const {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int item = tid + j * NT;
      if (SUBS % NT != 0 && item >= SUBS) break;
      const int kr = item % KR;
      const int nv = item / KR;
      uint32_t* dst = reinterpret_cast<uint32_t*>(lds + (nv * V) * (BK + V)) + kr;
      constexpr int ROW_DW = (BK + V) * sizeof(T) / 4;
      if constexpr (R == 2) {
        // Column e of the vector = halfword e of rows q=0,1; pack (k, k+1).
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t r0 = regs[j][0][d];
          const uint32_t r1 = regs[j][1][d];
          dst[(2 * d) * ROW_DW] = __builtin_amdgcn_perm(r1, r0, 0x05040100u);
          dst[(2 * d + 1) * ROW_DW] = __builtin_amdgcn_perm(r1, r0, 0x07060302u);
        }
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) dst[d * ROW_DW] = regs[j][0][d];
      }
    }
  }
};

template <typename T, int BM, int BN, int BK, int WAVES, int ALOAD, int BLOAD>
__global__ __launch_bounds__(WAVES * 64) void gemm_kernel(Args args) {
  using Tl = Tile<T, BM, BN, BK, WAVES>;
  constexpr int NT = Tl::NT;
  constexpr int LDK = Tl::LDK;
  constexpr int V = Tl::V;
  constexpr int FM = Tl::FM, FN = Tl::FN, KC = Tl::KC;

  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  T* smem = reinterpret_cast<T*>(smem_raw);

  const T* __restrict__ A = static_cast<const T*>(args.A);
  const T* __restrict__ B = static_cast<const T*>(args.B);
  const int64_t M = args.M, N = args.N, K = args.K;

  // ---- tile order: regroup per XCD, then GROUP_M bands -------------------
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
  const int64_t tm = first_m + (pid % in_group) % size_m;
  const int64_t tn = (pid % in_group) / size_m;
  const int64_t m0 = tm * BM;
  const int64_t n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / Tl::WN;
  const int wn = wave % Tl::WN;

  // ---- loaders ------------------------------------------------------------
  using ALd = std::conditional_t<ALOAD == kLoadScalar, ScalarLoader<T, BM, BK, NT>,
                                 VecKLoader<T, BM, BK, NT>>;
  using BLd = std::conditional_t<
      BLOAD == kLoadScalar, ScalarLoader<T, BN, BK, NT>,
      std::conditional_t<BLOAD == kLoadVecN, VecNLoader<T, BN, BK, NT>, VecKLoader<T, BN, BK, NT>>>;
  ALd aload;
  BLd bload;

  // Fetch k-slice k0 for LDS stage `stage`: vector loaders stage it in
  // registers (written by sstore after the compute), the scalar loader writes
  // the stage directly.
  auto gload = [&](int64_t k0, auto full_tag, int stage) {
    constexpr bool F = decltype(full_tag)::value;
    T* As = smem + stage * (Tl::kLdsA + Tl::kLdsB);
    T* Bs = As + Tl::kLdsA;
    if constexpr (ALOAD == kLoadScalar)
      aload.template load_to_lds<F>(As, A, args.lda_m, args.lda_k, m0, M, k0, K, tid);
    else
      aload.template load<F>(A, args.lda_m, m0, M, k0, K, tid);
    if constexpr (BLOAD == kLoadScalar)
      bload.template load_to_lds<F>(Bs, B, args.ldb_n, args.ldb_k, n0, N, k0, K, tid);
    else if constexpr (BLOAD == kLoadVecN)
      bload.template load<F>(B, args.ldb_k, n0, N, k0, K, tid);
    else
      bload.template load<F>(B, args.ldb_n, n0, N, k0, K, tid);
    (void)As;
    (void)Bs;
  };
  using Full = std::true_type;
  using Part = std::false_type;
  auto sstore = [&](int stage) {
    T* As = smem + stage * (Tl::kLdsA + Tl::kLdsB);
    T* Bs = As + Tl::kLdsA;
    if constexpr (ALOAD != kLoadScalar) aload.store(As, tid);
    if constexpr (BLOAD != kLoadScalar) bload.store(Bs, tid);
    (void)As;
    (void)Bs;
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Fragment addressing: lane reads 16 bytes at row (lane%16) of its
  // fragment, k offset 4*V*chunk + V*(lane/16).
  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * V;

  auto compute = [&](int stage) {
    const T* As = smem + stage * (Tl::kLdsA + Tl::kLdsB);
    const T* Bs = As + Tl::kLdsA;
    const T* a_base = As + (wm * Tl::TM + frag_row) * LDK + frag_k;
    const T* b_base = Bs + (wn * Tl::TN + frag_row) * LDK + frag_k;
#pragma unroll
    for (int kc = 0; kc < BK / KC; ++kc) {
      u32x4 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(a_base + i * 16 * LDK + kc * KC);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const u32x4*>(b_base + j * 16 * LDK + kc * KC);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Mma<T>::run(af[i], bfr[j], acc[i][j]);
    }
  };

  // ---- main loop: double-buffered LDS, one barrier per k-slice ----------
  // The steady state only ever loads whole k-slices, so it has no masking and
  // no data-dependent branches; the (at most one) partial slice at the end
  // of K is peeled into the short loop after it.
  const int64_t nk = ceil_div(K, BK);
  const int64_t nfull = K / BK;
  if (nk > 0) {
    if (nfull > 0)
      gload(0, Full{}, 0);
    else
      gload(0, Part{}, 0);
    sstore(0);
    __syncthreads();
    int64_t kt = 0;
    for (; kt + 1 < nfull; ++kt) {
      gload((kt + 1) * BK, Full{}, static_cast<int>((kt + 1) & 1));
      compute(static_cast<int>(kt & 1));
      sstore(static_cast<int>((kt + 1) & 1));
      __syncthreads();
    }
    for (; kt < nk; ++kt) {
      if (kt + 1 < nk) gload((kt + 1) * BK, Part{}, static_cast<int>((kt + 1) & 1));
      compute(static_cast<int>(kt & 1));
      if (kt + 1 < nk) sstore(static_cast<int>((kt + 1) & 1));
      __syncthreads();
    }
  }

  // ---- epilogue -------------------------------------------------------------
  T* __restrict__ C = static_cast<T*>(args.C);
  const T* __restrict__ bias = static_cast<const T*>(args.bias);
  const bool gelu = args.epilogue == KF_EPILOGUE_BIAS_GELU;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * Tl::TN + j * 16 + (lane & 15);
    if (col >= N) continue;
    const float bcol = gelu ? to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm * Tl::TM + i * 16 + (lane >> 4) * 4 + r;
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
