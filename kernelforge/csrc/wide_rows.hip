// Two-pass RMSNorm for rows of any width (the single-pass kernel in rows.hip
// holds a row in registers and stops at 16384 values).
//
// The reference names this kernel as its first future improvement
// (README.md:656-660): lift the single-pass cap at the cost of a second look
// at the row. A workgroup walks its row in trips of `block_size` columns:
//
//   pass 1: U 16-byte loads per lane per trip, all issued before the first
//           use, accumulate x^2 in V independent fp32 lanes of a vector;
//           one workgroup reduction gives rsqrt(mean(x^2) + eps);
//   pass 2: the row again, times inv_rms times gamma, rounded once.
//
// With STAGE the row is parked in LDS during pass 1 (up to 159 KiB of the
// 160 KiB a gfx950 workgroup may hold), so HBM sees one read and one write
// per element, like the single-pass kernel. Without STAGE pass 2 reads x
// again; it is then served by L2 or the Infinity Cache when the rows in
// flight fit, else by HBM.
#include <math.h>

#include <type_traits>

#include "common.h"

namespace kf {

namespace {

constexpr int kWideMaxWaves = 16;
// Dynamic LDS a staged row may use: 160 KiB minus room for the reduction
// buffer and the allocation granule.
constexpr int64_t kMaxStagedBytes = 159 * 1024;
// Eight vectors of x and eight of gamma per lane need more than the 128
// registers a lane gets at 1024 lanes: that unroll runs at up to 512.
constexpr int two_pass_max_lanes(int unroll) { return unroll >= 8 ? 512 : 1024; }

__device__ __forceinline__ void wide_lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt unconstrained
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float wide_block_sum(float x, float (*part)[kWideMaxWaves], int& slot,
                                                int nwaves) {
  x = wave_sum(x);
  if (nwaves == 1) return x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane == 0) part[slot][wave] = x;
  wide_lds_sync();
  float r = part[slot][0];
  for (int w = 1; w < nwaves; ++w) r += part[slot][w];
  slot ^= 1;
  return r;
}

// U vectors of V elements per lane for the trip starting at column c0:
// vector u of lane t covers columns c0 + (u*nt + t)*V ... + V - 1, so each of
// the U loads is one contiguous, coalesced sweep of the workgroup.
template <typename T, int U>
struct Trip {
  static constexpr int V = Vec<T>::N;
  T v[U][V];

  __device__ __forceinline__ static int64_t col(int64_t c0, int u, int t, int nt) {
    return c0 + (static_cast<int64_t>(u) * nt + t) * V;
  }

  // Out-of-row elements read as zero. `vec`: 16-byte aligned rows whose width
  // is a multiple of V, so a vector is wholly inside the row or wholly past
  // it; past-the-end lanes load a clamped valid vector and then discard it,
  // which keeps the U loads back to back without branches.
  __device__ __forceinline__ void load(const T* row, int64_t cols, int64_t c0, int t, int nt,
                                       bool vec) {
    if (vec) {
      u32x4 raw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = col(c0, u, t, nt);
        raw[u] = *reinterpret_cast<const u32x4*>(row + ((c < cols) ? c : cols - V));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        __builtin_memcpy(v[u], &raw[u], 16);
        if (col(c0, u, t, nt) >= cols) {
#pragma unroll
          for (int e = 0; e < V; ++e) v[u][e] = from_f32<T>(0.f);
        }
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = col(c0, u, t, nt);
#pragma unroll
      for (int e = 0; e < V; ++e) v[u][e] = (c + e < cols) ? row[c + e] : from_f32<T>(0.f);
    }
  }

  // The same positions in an LDS copy of the row (element index = column).
  __device__ __forceinline__ void park(T* lds, int64_t cols, int64_t c0, int t, int nt,
                                       bool vec) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = col(c0, u, t, nt);
      if (vec) {
        if (c < cols) {
          u32x4 raw;
          __builtin_memcpy(&raw, v[u], 16);
          *reinterpret_cast<u32x4*>(lds + c) = raw;
        }
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e)
          if (c + e < cols) lds[c + e] = v[u][e];
      }
    }
  }

  __device__ __forceinline__ void unpark(const T* lds, int64_t cols, int64_t c0, int t, int nt,
                                         bool vec) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = col(c0, u, t, nt);
      if (vec) {
        if (c < cols) {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(lds + c);
          __builtin_memcpy(v[u], &raw, 16);
        }
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e)
          if (c + e < cols) v[u][e] = lds[c + e];
      }
    }
  }
};

template <typename T, int U, bool STAGE>
__global__ __launch_bounds__(two_pass_max_lanes(U)) void rmsnorm_two_pass(const T* __restrict__ x,
                                                         const T* __restrict__ gamma,
                                                         T* __restrict__ y, int64_t xrs,
                                                         int64_t yrs, int64_t rows, int64_t cols,
                                                         float eps, int rpp, int vec) {
  using Tr = Trip<T, U>;
  constexpr int V = Tr::V;
  extern __shared__ __align__(16) char row_lds[];
  __shared__ float part[2][kWideMaxWaves];
  int slot = 0;
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  const int nwaves = nt / kWave;
  const int64_t trip = static_cast<int64_t>(nt) * U * V;
  const float inv_cols = 1.0f / static_cast<float>(cols);
  T* staged = reinterpret_cast<T*>(row_lds);
  for (int i = 0; i < rpp; ++i) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * rpp + i;
    if (r >= rows) break;
    const T* xr = x + r * xrs;
    T* yr = y + r * yrs;
    // The previous row's pass 2 must be done reading the staged copy.
    if (STAGE && i > 0) wide_lds_sync();

    float ss[V];
#pragma unroll
    for (int e = 0; e < V; ++e) ss[e] = 0.f;
    for (int64_t c0 = 0; c0 < cols; c0 += trip) {
      Tr tr;
      tr.load(xr, cols, c0, t, nt, vec != 0);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float f = to_f32(tr.v[u][e]);
          ss[e] = __builtin_fmaf(f, f, ss[e]);
        }
      if (STAGE) tr.park(staged, cols, c0, t, nt, vec != 0);
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < V; ++e) s += ss[e];
    s = wide_block_sum(s, part, slot, nwaves);
    // Staged elements were written by other lanes: publish them.
    if (STAGE) wide_lds_sync();
    const float inv_rms = rsqrtf(s * inv_cols + eps);

    for (int64_t c0 = 0; c0 < cols; c0 += trip) {
      Tr xv, gv;
      if (STAGE)
        xv.unpark(staged, cols, c0, t, nt, vec != 0);
      else
        xv.load(xr, cols, c0, t, nt, vec != 0);
      gv.load(gamma, cols, c0, t, nt, vec != 0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = Tr::col(c0, u, t, nt);
        T out[V];
#pragma unroll
        for (int e = 0; e < V; ++e)
          out[e] = from_f32<T>((to_f32(xv.v[u][e]) * inv_rms) * to_f32(gv.v[u][e]));
        if (vec) {
          if (c < cols) {
            u32x4 raw;
            __builtin_memcpy(&raw, out, 16);
            *reinterpret_cast<u32x4*>(yr + c) = raw;
          }
        } else {
#pragma unroll
          for (int e = 0; e < V; ++e)
            if (c + e < cols) yr[c + e] = out[e];
        }
      }
    }
  }
}

template <typename F>
int dispatch_unroll(int u, F&& f) {
  switch (u) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default:
      set_error("two-pass rmsnorm: %d vectors per lane per trip is not built (1, 2, 4, 8)", u);
      return KF_ERR_NOT_BUILT;
  }
}

// Dynamic LDS above the default must be granted once per kernel.
int grant_lds(const void* kernel, int64_t bytes) {
  static thread_local const void* granted[64];
  static thread_local int64_t granted_bytes[64];
  static thread_local int count = 0;
  for (int i = 0; i < count; ++i)
    if (granted[i] == kernel && granted_bytes[i] >= bytes) return KF_OK;
  const hipError_t err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(kMaxStagedBytes));
  if (err != hipSuccess) {
    set_error("two-pass rmsnorm: granting %lld B of LDS failed: %s", (long long)kMaxStagedBytes,
              hipGetErrorString(err));
    return KF_ERR_OUT_OF_RESOURCES;
  }
  if (count < 64) {
    granted[count] = kernel;
    granted_bytes[count] = kMaxStagedBytes;
    ++count;
  }
  return KF_OK;
}

template <typename T>
int launch_two_pass(const void* x, const void* g, void* y, int64_t rows, int64_t cols,
                    int64_t xrs, int64_t yrs, float eps, int unroll, int rpp, int waves,
                    int stage, hipStream_t s) {
  constexpr int V = Vec<T>::N;
  const bool vec = aligned16(x) && aligned16(y) && aligned16(g) && cols % V == 0 &&
                   (xrs * static_cast<int64_t>(sizeof(T))) % 16 == 0 &&
                   (yrs * static_cast<int64_t>(sizeof(T))) % 16 == 0;
  const int64_t lds = stage ? ((cols * static_cast<int64_t>(sizeof(T)) + 15) / 16) * 16 : 0;
  if (lds > kMaxStagedBytes) {
    set_error("two-pass rmsnorm: a staged row of %lld B exceeds the %lld B of LDS available",
              (long long)(cols * static_cast<int64_t>(sizeof(T))), (long long)kMaxStagedBytes);
    return KF_ERR_OUT_OF_RESOURCES;
  }
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, rpp)));
  const dim3 block(waves * kWave);
  return dispatch_unroll(unroll, [&](auto uc) -> int {
    constexpr int U = decltype(uc)::value;
    auto run = [&](auto st) -> int {
      constexpr bool S = decltype(st)::value;
      if (lds > 0) {
        const int rc = grant_lds(reinterpret_cast<const void*>(&rmsnorm_two_pass<T, U, S>), lds);
        if (rc != KF_OK) return rc;
      }
      hipLaunchKernelGGL((rmsnorm_two_pass<T, U, S>), grid, block, static_cast<unsigned>(lds), s,
                         static_cast<const T*>(x), static_cast<const T*>(g), static_cast<T*>(y),
                         xrs, yrs, rows, cols, eps, rpp, vec ? 1 : 0);
      return launch_status("rmsnorm_two_pass");
    };
    return stage ? run(std::true_type{}) : run(std::false_type{});
  });
}

int elem_size(int dtype) {
  switch (dtype) {
    case KF_DTYPE_F32: return 4;
    case KF_DTYPE_F16:
    case KF_DTYPE_BF16: return 2;
    default: return 0;
  }
}

}  // namespace
}  // namespace kf

extern "C" int kf_rmsnorm_two_pass(int dtype, const void* x, const void* gamma, void* y,
                                   int64_t rows, int64_t cols, int64_t x_row_stride,
                                   int64_t y_row_stride, float eps, int block_size,
                                   int rows_per_program, int waves, int stage_row,
                                   void* stream) {
  using namespace kf;
  const int es = elem_size(dtype);
  if (es == 0) {
    set_error("rmsnorm_two_pass: unsupported dtype code %d", dtype);
    return KF_ERR_UNSUPPORTED_DTYPE;
  }
  if (rows < 0 || cols < 0) {
    set_error("negative shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (waves < 1 || waves > kWideMaxWaves) {
    set_error("waves=%d outside 1..%d (workgroup limit of 1024 lanes)", waves, kWideMaxWaves);
    return KF_ERR_OUT_OF_RESOURCES;
  }
  if (rows_per_program < 1) {
    set_error("rows_per_program=%d must be positive", rows_per_program);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (stage_row != 0 && stage_row != 1) {
    set_error("stage_row=%d must be 0 or 1", stage_row);
    return KF_ERR_INVALID_ARGUMENT;
  }
  const int vec_elems = 16 / es;
  const int64_t lane_cols = static_cast<int64_t>(waves) * kWave * vec_elems;
  if (block_size < lane_cols || block_size % lane_cols != 0) {
    set_error("block_size=%d is not a whole number of 16-byte vectors per lane at waves=%d "
              "(multiples of %lld)",
              block_size, waves, (long long)lane_cols);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (!(eps >= 0.f)) {
    set_error("rmsnorm_two_pass: eps must be non-negative");
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (x_row_stride < cols || y_row_stride < cols) {
    set_error("row strides (%lld, %lld) shorter than the row (%lld)", (long long)x_row_stride,
              (long long)y_row_stride, (long long)cols);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (rows == 0 || cols == 0) return KF_OK;
  if (!x || !gamma || !y) {
    set_error("rmsnorm_two_pass: null pointer");
    return KF_ERR_INVALID_ARGUMENT;
  }
  const int unroll = static_cast<int>(block_size / lane_cols);
  if (waves * kWave > two_pass_max_lanes(unroll)) {
    set_error("register pressure: %d vectors per lane per trip allow at most %d waves, got %d",
              unroll, two_pass_max_lanes(unroll) / kWave, waves);
    return KF_ERR_OUT_OF_RESOURCES;
  }
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case KF_DTYPE_F32:
      return launch_two_pass<float>(x, gamma, y, rows, cols, x_row_stride, y_row_stride, eps,
                                    unroll, rows_per_program, waves, stage_row, s);
    case KF_DTYPE_F16:
      return launch_two_pass<f16>(x, gamma, y, rows, cols, x_row_stride, y_row_stride, eps,
                                  unroll, rows_per_program, waves, stage_row, s);
    default:
      return launch_two_pass<bf16>(x, gamma, y, rows, cols, x_row_stride, y_row_stride, eps,
                                   unroll, rows_per_program, waves, stage_row, s);
  }
}

extern "C" int64_t kf_rmsnorm_two_pass_max_staged_cols(int dtype) {
  const int es = kf::elem_size(dtype);
  return es ? kf::kMaxStagedBytes / es : 0;
}
