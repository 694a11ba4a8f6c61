// Single-pass row kernels for gfx950: softmax and RMSNorm.
//
// One workgroup owns `rows_per_program` whole rows; each row is read from HBM
// exactly once into registers (16-byte loads, EPT fp32 values per lane),
// reduced with wave64 shuffles plus one LDS exchange across waves, and
// written once. These are the HBM-bound counterparts of the reference's
// softmax_kernel (kernels/softmax.py:31-58) and rmsnorm_kernel
// (kernels/rmsnorm.py:41-72).
#include <math.h>

#include "common.h"

namespace kf {

namespace {

constexpr int kMaxWaves = 16;  // 1024 lanes, the workgroup limit
// A workgroup keeps at most 16384 fp32 row values in registers (64 KiB): the
// single-pass limit. EPT values per lane therefore allow 16384/EPT lanes, and
// the launch bound tells the compiler that, so it can give each lane the
// registers EPT (and RMSNorm's gamma copy) need without spilling.
constexpr int kMaxRowValues = 16384;
template <int EPT>
constexpr int max_lanes() { return (kMaxRowValues / EPT < 1024) ? kMaxRowValues / EPT : 1024; }
constexpr float kLog2e = 1.4426950408889634f;
// Rows of at most four 16-byte vectors per lane keep the next row's raw
// loads in flight during the current row's reductions (16 extra registers
// at most); wider rows already hold enough loads per lane.
template <typename T, int EPT>
constexpr bool prefetch_rows() {
  return EPT >= 16 / static_cast<int>(sizeof(T)) && EPT * static_cast<int>(sizeof(T)) <= 64;
}

// Lane `t` of a `nt`-lane workgroup owns vector slots t, t+nt, t+2nt, ... of
// the row; slot s covers columns [s*V, s*V+V). `vec` says whether the row is
// 16-byte aligned, so a full slot can be one load.
template <typename T, int EPT>
struct RowTile {
  static constexpr int V = (EPT < Vec<T>::N) ? EPT : Vec<T>::N;
  static constexpr int NV = EPT / V;
  static constexpr bool kVector = (V == Vec<T>::N);
  float v[EPT];

  // Vector path: aligned rows whose width is a multiple of V. Then every
  // lane's slot is wholly inside the row or wholly past it; lanes past the
  // row load a clamped valid vector and substitute `fill`, so all loads
  // issue back to back with no per-lane branches.
  __device__ __forceinline__ static bool vector_ok(bool vec, int64_t cols) {
    return kVector && vec && cols >= V && cols % V == 0;
  }

  __device__ __forceinline__ void load(const T* row, int64_t cols, int t, int nt, bool vec,
                                       float fill) {
    if constexpr (kVector) {
      if (vector_ok(vec, cols)) {
        load_vector(row, cols, t, nt, fill);
        return;
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t c0 = (static_cast<int64_t>(j) * nt + t) * V;
#pragma unroll
      for (int e = 0; e < V; ++e) v[j * V + e] = (c0 + e < cols) ? to_f32(row[c0 + e]) : fill;
    }
  }

  __device__ __forceinline__ void load_vector(const T* row, int64_t cols, int t, int nt,
                                              float fill) {
    {
      u32x4 raw[NV];
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int64_t c0 = (static_cast<int64_t>(j) * nt + t) * V;
        raw[j] = *reinterpret_cast<const u32x4*>(row + ((c0 < cols) ? c0 : cols - V));
      }
      // Convert only after every load has been issued.
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int64_t c0 = (static_cast<int64_t>(j) * nt + t) * V;
        T tmp[V];
        __builtin_memcpy(tmp, &raw[j], 16);
#pragma unroll
        for (int e = 0; e < V; ++e) v[j * V + e] = (c0 < cols) ? to_f32(tmp[e]) : fill;
      }
    }
  }

  // The vector path split in two, so that the next row's loads can be in
  // flight while this row is reduced: issue the raw 16-byte loads, convert
  // later. Valid only where vector_ok() holds.
  struct Raw {
    u32x4 raw[NV];
  };
  __device__ __forceinline__ static void load_raw(Raw& r, const T* row, int64_t cols, int t,
                                                  int nt) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t c0 = (static_cast<int64_t>(j) * nt + t) * V;
      r.raw[j] = *reinterpret_cast<const u32x4*>(row + ((c0 < cols) ? c0 : cols - V));
    }
  }
  __device__ __forceinline__ void convert(const Raw& r, int64_t cols, int t, int nt, float fill) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t c0 = (static_cast<int64_t>(j) * nt + t) * V;
      T tmp[V];
      __builtin_memcpy(tmp, &r.raw[j], 16);
#pragma unroll
      for (int e = 0; e < V; ++e) v[j * V + e] = (c0 < cols) ? to_f32(tmp[e]) : fill;
    }
  }

  template <typename F>
  __device__ __forceinline__ void store(T* row, int64_t cols, int t, int nt, bool vec, F f) const {
    const bool vpath = vector_ok(vec, cols);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t c0 = (static_cast<int64_t>(j) * nt + t) * V;
      T tmp[V];
#pragma unroll
      for (int e = 0; e < V; ++e) tmp[e] = from_f32<T>(f(v[j * V + e], j * V + e));
      if constexpr (kVector) {
        if (vpath) {
          if (c0 < cols) {
            u32x4 raw;
            __builtin_memcpy(&raw, tmp, 16);
            *reinterpret_cast<u32x4*>(row + c0) = raw;
          }
          continue;
        }
      }
      {
#pragma unroll
        for (int e = 0; e < V; ++e)
          if (c0 + e < cols) row[c0 + e] = tmp[e];
      }
    }
  }
};

// Barrier for the LDS exchange only: this wave's LDS accesses are complete
// (lgkmcnt(0)) and the compiler may not move memory operations across it. It
// does not wait for outstanding global stores (the fences of __syncthreads()
// would): the previous row's stores stay in flight across the reductions.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt unconstrained
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroup reduction: wave64 butterfly, then one LDS exchange. `slot`
// alternates between two buffers so a reduction needs a single barrier: the
// buffer reused two reductions later cannot be overwritten before every wave
// has passed the barrier of the reduction in between.
template <bool IsMax>
__device__ __forceinline__ float block_reduce(float x, float (*part)[kMaxWaves], int& slot,
                                              int nwaves) {
  x = IsMax ? wave_max(x) : wave_sum(x);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (nwaves == 1) return x;
  if (lane == 0) part[slot][wave] = x;
  lds_sync();
  float r = part[slot][0];
  for (int w = 1; w < nwaves; ++w) r = IsMax ? fmaxf(r, part[slot][w]) : r + part[slot][w];
  slot ^= 1;
  return r;
}

template <typename T, int EPT>
__global__ __launch_bounds__(max_lanes<EPT>()) void softmax_rows(const T* __restrict__ x, T* __restrict__ y,
                                                     int64_t xrs, int64_t yrs, int64_t rows,
                                                     int64_t cols, int rpp, int vec) {
  __shared__ float part[2][kMaxWaves];
  int slot = 0;
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  const int nwaves = nt / kWave;
  using Tile = RowTile<T, EPT>;
  auto process = [&](Tile& tile, int64_t r) {
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < EPT; ++e) m = fmaxf(m, tile.v[e]);
    m = block_reduce<true>(m, part, slot, nwaves);
    // exp(x - m) = exp2((x - m) * log2(e)); v_exp_f32 is the hardware exp2.
    const float ms = m * kLog2e;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      tile.v[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(tile.v[e], kLog2e, -ms));
      s += tile.v[e];
    }
    s = block_reduce<false>(s, part, slot, nwaves);
    const float inv = 1.0f / s;
    tile.store(y + r * yrs, cols, t, nt, vec, [inv](float v, int) { return v * inv; });
  };
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rpp;
  // Out-of-row lanes hold -inf: they lose the max and add exp(-inf)=0.
  if constexpr (prefetch_rows<T, EPT>()) {
    if (Tile::vector_ok(vec, cols)) {
      typename Tile::Raw cur, nxt;
      if (r0 < rows) Tile::load_raw(cur, x + r0 * xrs, cols, t, nt);
      for (int i = 0; i < rpp; ++i) {
        const int64_t r = r0 + i;
        if (r >= rows) break;
        if (i + 1 < rpp && r + 1 < rows) Tile::load_raw(nxt, x + (r + 1) * xrs, cols, t, nt);
        Tile tile;
        tile.convert(cur, cols, t, nt, -INFINITY);
        process(tile, r);
        cur = nxt;
      }
      return;
    }
  }
  for (int i = 0; i < rpp; ++i) {
    const int64_t r = r0 + i;
    if (r >= rows) break;
    Tile tile;
    tile.load(x + r * xrs, cols, t, nt, vec, -INFINITY);
    process(tile, r);
  }
}

template <typename T, int EPT>
__global__ __launch_bounds__(max_lanes<EPT>()) void rmsnorm_rows(const T* __restrict__ x,
                                                     const T* __restrict__ gamma,
                                                     T* __restrict__ y, int64_t xrs, int64_t yrs,
                                                     int64_t rows, int64_t cols, float eps,
                                                     int rpp, int vec) {
  __shared__ float part[2][kMaxWaves];
  int slot = 0;
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  const int nwaves = nt / kWave;
  const float inv_cols = 1.0f / static_cast<float>(cols);
  using Tile = RowTile<T, EPT>;
  // gamma is shared by all rows of the program and read once. On the vector
  // path its loads are issued after the first row's and converted only when
  // the first row is stored, so the two latencies overlap instead of adding
  // up at the start of every workgroup.
  auto process = [&](Tile& tile, int64_t r, const Tile& g) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) ss = __builtin_fmaf(tile.v[e], tile.v[e], ss);
    ss = block_reduce<false>(ss, part, slot, nwaves);
    const float inv_rms = rsqrtf(ss * inv_cols + eps);
    tile.store(y + r * yrs, cols, t, nt, vec,
               [inv_rms, &g](float v, int e) { return (v * inv_rms) * g.v[e]; });
  };
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rpp;
  if (r0 >= rows) return;
  // Out-of-row lanes hold 0, which adds nothing to the sum of squares.
  if constexpr (Tile::kVector) {
  if (Tile::vector_ok(vec, cols)) {
    typename Tile::Raw cur, graw;
    Tile::load_raw(cur, x + r0 * xrs, cols, t, nt);
    Tile::load_raw(graw, gamma, cols, t, nt);
    Tile g;
    bool have_gamma = false;
    for (int i = 0; i < rpp; ++i) {
      const int64_t r = r0 + i;
      if (r >= rows) break;
      typename Tile::Raw nxt;
      // Rows of at most four vectors per lane keep the next row in flight
      // during this row's reduction.
      if constexpr (prefetch_rows<T, EPT>()) {
        if (i + 1 < rpp && r + 1 < rows) Tile::load_raw(nxt, x + (r + 1) * xrs, cols, t, nt);
      }
      Tile tile;
      tile.convert(cur, cols, t, nt, 0.f);
      if (!have_gamma) {
        g.convert(graw, cols, t, nt, 0.f);
        have_gamma = true;
      }
      process(tile, r, g);
      if constexpr (prefetch_rows<T, EPT>()) {
        cur = nxt;
      } else if (i + 1 < rpp && r + 1 < rows) {
        Tile::load_raw(cur, x + (r + 1) * xrs, cols, t, nt);
      }
    }
    return;
  }
  }
  Tile g;
  g.load(gamma, cols, t, nt, vec, 0.f);
  for (int i = 0; i < rpp; ++i) {
    const int64_t r = r0 + i;
    if (r >= rows) break;
    Tile tile;
    tile.load(x + r * xrs, cols, t, nt, vec, 0.f);
    process(tile, r, g);
  }
}

// Elements-per-lane dispatch: EPT = block_size / (waves*64) must be one of
// the instantiated powers of two.
template <typename T, typename Launch>
int dispatch_ept(int ept, Launch&& launch) {
  switch (ept) {
    case 1: return launch(std::integral_constant<int, 1>{});
    case 2: return launch(std::integral_constant<int, 2>{});
    case 4: return launch(std::integral_constant<int, 4>{});
    case 8: return launch(std::integral_constant<int, 8>{});
    case 16: return launch(std::integral_constant<int, 16>{});
    case 32: return launch(std::integral_constant<int, 32>{});
    case 64: return launch(std::integral_constant<int, 64>{});
    default:
      set_error("no row-kernel instantiation holds %d elements per lane (1..64, powers of two)",
                ept);
      return KF_ERR_NOT_BUILT;
  }
}

int check_row_config(int64_t rows, int64_t cols, int64_t xrs, int64_t yrs, int block_size,
                     int rpp, int waves, int* ept) {
  if (rows < 0 || cols < 0) {
    set_error("negative shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (waves < 1 || waves > kMaxWaves) {
    set_error("waves=%d outside 1..%d (workgroup limit of 1024 lanes)", waves, kMaxWaves);
    return KF_ERR_OUT_OF_RESOURCES;
  }
  if (rpp < 1) {
    set_error("rows_per_program=%d must be positive", rpp);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (block_size < 1 || (block_size & (block_size - 1)) != 0) {
    set_error("block_size=%d is not a power of two", block_size);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (block_size < cols) {
    set_error("block_size=%d cannot hold a row of %lld", block_size, (long long)cols);
    return KF_ERR_INVALID_ARGUMENT;
  }
  // A row narrower than the workgroup leaves lanes idle (one element each,
  // masked); the search space rejects that for tuning, the kernel accepts it.
  if (block_size >= waves * kWave && block_size % (waves * kWave) != 0) {
    set_error("block_size=%d is not a whole number of elements per lane at waves=%d",
              block_size, waves);
    return KF_ERR_OUT_OF_RESOURCES;
  }
  if (xrs < cols || yrs < cols) {
    set_error("row strides (%lld, %lld) shorter than the row (%lld)", (long long)xrs,
              (long long)yrs, (long long)cols);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (block_size > kMaxRowValues) {
    set_error("row of %lld exceeds the single-pass limit of %d values per workgroup",
              (long long)cols, kMaxRowValues);
    return KF_ERR_INVALID_ARGUMENT;
  }
  *ept = block_size >= waves * kWave ? block_size / (waves * kWave) : 1;
  return KF_OK;
}

template <typename T>
int launch_softmax(const void* x, void* y, int64_t rows, int64_t cols, int64_t xrs, int64_t yrs,
                   int ept, int rpp, int waves, hipStream_t s) {
  const bool vec = aligned16(x) && aligned16(y) && (xrs * sizeof(T)) % 16 == 0 &&
                   (yrs * sizeof(T)) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, rpp)));
  const dim3 block(waves * kWave);
  return dispatch_ept<T>(ept, [&](auto e) -> int {
    constexpr int E = decltype(e)::value;
    hipLaunchKernelGGL((softmax_rows<T, E>), grid, block, 0, s, static_cast<const T*>(x),
                       static_cast<T*>(y), xrs, yrs, rows, cols, rpp, vec ? 1 : 0);
    return launch_status("softmax");
  });
}

template <typename T>
int launch_rmsnorm(const void* x, const void* g, void* y, int64_t rows, int64_t cols,
                   int64_t xrs, int64_t yrs, float eps, int ept, int rpp, int waves,
                   hipStream_t s) {
  const bool vec = aligned16(x) && aligned16(y) && aligned16(g) &&
                   (xrs * sizeof(T)) % 16 == 0 && (yrs * sizeof(T)) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, rpp)));
  const dim3 block(waves * kWave);
  return dispatch_ept<T>(ept, [&](auto e) -> int {
    constexpr int E = decltype(e)::value;
    hipLaunchKernelGGL((rmsnorm_rows<T, E>), grid, block, 0, s, static_cast<const T*>(x),
                       static_cast<const T*>(g), static_cast<T*>(y), xrs, yrs, rows, cols, eps,
                       rpp, vec ? 1 : 0);
    return launch_status("rmsnorm");
  });
}

}  // namespace
}  // namespace kf

extern "C" int kf_softmax(int dtype, const void* x, void* y, int64_t rows, int64_t cols,
                          int64_t x_row_stride, int64_t y_row_stride, int block_size,
                          int rows_per_program, int waves, void* stream) {
  using namespace kf;
  int ept = 0;
  int rc = check_row_config(rows, cols, x_row_stride, y_row_stride, block_size, rows_per_program,
                            waves, &ept);
  if (rc != KF_OK) return rc;
  if (rows == 0 || cols == 0) return KF_OK;
  if (!x || !y) {
    set_error("softmax: null pointer");
    return KF_ERR_INVALID_ARGUMENT;
  }
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case KF_DTYPE_F32:
      return launch_softmax<float>(x, y, rows, cols, x_row_stride, y_row_stride, ept,
                                   rows_per_program, waves, s);
    case KF_DTYPE_F16:
      return launch_softmax<f16>(x, y, rows, cols, x_row_stride, y_row_stride, ept,
                                 rows_per_program, waves, s);
    case KF_DTYPE_BF16:
      return launch_softmax<bf16>(x, y, rows, cols, x_row_stride, y_row_stride, ept,
                                  rows_per_program, waves, s);
    default:
      set_error("softmax: unsupported dtype code %d", dtype);
      return KF_ERR_UNSUPPORTED_DTYPE;
  }
}

extern "C" int kf_rmsnorm(int dtype, const void* x, const void* gamma, void* y, int64_t rows,
                          int64_t cols, int64_t x_row_stride, int64_t y_row_stride, float eps,
                          int block_size, int rows_per_program, int waves, void* stream) {
  using namespace kf;
  int ept = 0;
  int rc = check_row_config(rows, cols, x_row_stride, y_row_stride, block_size, rows_per_program,
                            waves, &ept);
  if (rc != KF_OK) return rc;
  if (!(eps >= 0.f)) {
    set_error("rmsnorm: eps must be non-negative");
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (rows == 0 || cols == 0) return KF_OK;
  if (!x || !gamma || !y) {
    set_error("rmsnorm: null pointer");
    return KF_ERR_INVALID_ARGUMENT;
  }
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case KF_DTYPE_F32:
      return launch_rmsnorm<float>(x, gamma, y, rows, cols, x_row_stride, y_row_stride, eps, ept,
                                   rows_per_program, waves, s);
    case KF_DTYPE_F16:
      return launch_rmsnorm<f16>(x, gamma, y, rows, cols, x_row_stride, y_row_stride, eps, ept,
                                 rows_per_program, waves, s);
    case KF_DTYPE_BF16:
      return launch_rmsnorm<bf16>(x, gamma, y, rows, cols, x_row_stride, y_row_stride, eps, ept,
                                  rows_per_program, waves, s);
    default:
      set_error("rmsnorm: unsupported dtype code %d", dtype);
      return KF_ERR_UNSUPPORTED_DTYPE;
  }
}
