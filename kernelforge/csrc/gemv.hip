// Split-K GEMV for decode-shaped products, y[M,N] = x[M,K] @ W[K,N], M <= 8.
//
// HBM-bound: every byte of W is read exactly once. A workgroup owns a strip
// of LPR*V columns (LPR lanes of 16-byte vectors, V = 16/sizeof(T)) and one
// of `split_k` slices of K. A wave load covers 64/LPR rows of the strip, so
// the workgroup's waves hold nwaves*64/LPR row groups that stride through the
// slice with U rows in flight per lane. Narrow strips give many workgroups
// (hundreds for a decode-sized W) with few slices, so the cross-slice tail
// stays short while every CU streams.
//
// Reduction, all in fixed order so results are bitwise reproducible run to
// run: the row groups of a wave by lane shuffles, the waves through LDS, the
// slices through an fp32 workspace -- the last workgroup to finish a strip
// (atomic ticket) sums the slices in ascending order.
//
// W laid out k-contiguous (nn.Linear's weight, passed as weight.t(), so
// ldw_k == 1) takes gemv_dot instead: LPR lanes split one column's k-run into
// 16-byte vectors (a wave load covers 64/LPR columns), x is read the same
// way, and the LPR partial sums of a column meet in a butterfly. Both
// kernels end in the same cross-slice tail.
//
// The reference has no GEMV: decode runs through matmul_kernel with
// BLOCK_M=16 (kernels/matmul.py:54-113, tuning/search.py:377-386).
#include <math.h>

#include <mutex>
#include <type_traits>

#include "common.h"

namespace kf {

namespace {

constexpr int kGemvMaxWaves = 16;
constexpr size_t kGemvMaxLds = 64 * 1024;  // dynamic LDS without an opt-in attribute

// One x row of a 16-bit type takes the packed-dot trip (U = 8 rows, even).
template <typename T, int MR>
constexpr bool kPackedDot = MR == 1 && sizeof(T) == 2;

// a.lo*b.lo + a.hi*b.hi + c over two packed 16-bit values, in fp32.
template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  typedef T pair __attribute__((ext_vector_type(2)));
  if constexpr (std::is_same<T, bf16>::value)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(pair, a), __builtin_bit_cast(pair, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(pair, a), __builtin_bit_cast(pair, b), c, false);
}

// A wave-uniform 64-bit value held in scalar registers.
__device__ __forceinline__ int64_t wave_uniform(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi =
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// B bytes loaded as one vector (B = 4, 8, 16) or two 16-byte vectors (32).
template <int B> struct XChunkT;
template <> struct XChunkT<4> { using type = uint32_t; };
template <> struct XChunkT<8> { using type = uint32_t __attribute__((ext_vector_type(2))); };
template <> struct XChunkT<16> { using type = u32x4; };
struct U32x8 { u32x4 lo, hi; };
template <> struct XChunkT<32> { using type = U32x8; };
template <int B>
using XChunk = typename XChunkT<B>::type;
constexpr float kGeluC = 1.5957691216057308f;  // 2*sqrt(2/pi)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float gelu_tanh(float a) {
  // gelu(a) = 0.5a(1+tanh(sqrt(2/pi)(a+0.044715a^3))) = a / (1 + exp(-2sqrt(2/pi)(...)))
  const float inner = kGeluC * (a + 0.044715f * a * a * a);
  return a / (1.0f + __builtin_amdgcn_exp2f(-inner * kLog2e));
}

// Registers per lane: trips are double buffered, so one x row keeps 2 x 8
// rows of W (64 registers) in flight, two keep 2 x 4, more keep 2 x 2; eight
// x rows need 8x the accumulators and x values. Only four rows fit 128
// registers (a 1024-lane workgroup); the others cap it at 512 lanes (256
// registers each).
template <int MR>
constexpr int gemv_max_lanes() { return MR == 4 ? 1024 : 512; }
template <int MR>
constexpr int gemv_unroll() { return MR <= 1 ? 8 : (MR <= 2 ? 4 : 2); }

// The end both kernels share. red[(w*MR + m)*BN + c] holds red_waves partial
// sums per (row m, column c of the block); each thread owns columns t,
// t + nthreads, ... and combines the partials in ascending order. With split_k
// slices, the slice publishes its sums to the fp32 workspace and the last
// slice of the block to arrive (atomic ticket) adds them in slice order and
// writes y; otherwise y is written directly. Callers synchronise the
// workgroup after filling red.
template <typename T, int MR>
__device__ __forceinline__ void finish_block(const float* red, int red_waves, int BN, int64_t nb,
                                             int64_t M, int64_t N, int s, int split_k,
                                             int epilogue, const T* __restrict__ bias,
                                             T* __restrict__ y, int64_t ldy_m, int64_t ldy_n,
                                             float* __restrict__ ws,
                                             unsigned* __restrict__ tickets) {
  const int t = threadIdx.x;
  const int nthreads = blockDim.x;
  auto wave_sum = [&](int m, int c) {
    float r = 0.f;
    for (int w = 0; w < red_waves; ++w) r += red[(w * MR + m) * BN + c];
    return r;
  };
  if (split_k > 1) {
    // Publish this slice's partial sums, then take a ticket for the block.
    // The partials move through agent-scope relaxed atomic stores/loads,
    // which are coherent across XCDs without writing back or invalidating
    // whole L2s (what a device-scope fence costs here); the only ordering
    // needed is that every thread's stores have completed before the
    // workgroup's ticket is taken.
    for (int c = t; c < BN; c += nthreads) {
      const int64_t col = nb * BN + c;
      if (col >= N) continue;
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m >= M) break;
        __hip_atomic_store(ws + (static_cast<int64_t>(s) * M + m) * N + col, wave_sum(m, c),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores are done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __shared__ unsigned ticket;
    __syncthreads();  // every thread's stores are done
    if (t == 0)
      ticket = __hip_atomic_fetch_add(&tickets[nb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != static_cast<unsigned>(split_k - 1)) return;
    // Sum the slices in ascending order (deterministic). kSliceBatch slices'
    // loads are issued before any is added, so they are in flight together.
    constexpr int kSliceBatch = 4;
    for (int c = t; c < BN; c += nthreads) {
      const int64_t col = nb * BN + c;
      const int64_t cl = (col < N) ? col : N - 1;  // threads past N read a valid column
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m >= M) break;
        const float* src = ws + static_cast<int64_t>(m) * N + cl;
        float r = 0.f;
        for (int q0 = 0; q0 < split_k; q0 += kSliceBatch) {
          float part[kSliceBatch];
#pragma unroll
          for (int b = 0; b < kSliceBatch; ++b) {
            const int q = (q0 + b < split_k) ? q0 + b : split_k - 1;
            part[b] = __hip_atomic_load(src + static_cast<int64_t>(q) * M * N, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
          }
#pragma unroll
          for (int b = 0; b < kSliceBatch; ++b)
            if (q0 + b < split_k) r += part[b];
        }
        if (col >= N) continue;
        if (epilogue == KF_EPILOGUE_BIAS_GELU) r = gelu_tanh(r + to_f32(bias[col]));
        y[m * ldy_m + col * ldy_n] = from_f32<T>(r);
      }
    }
    if (t == 0) __hip_atomic_store(&tickets[nb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  for (int c = t; c < BN; c += nthreads) {
    const int64_t col = nb * BN + c;
    if (col >= N) continue;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= M) break;
      float r = wave_sum(m, c);
      if (epilogue == KF_EPILOGUE_BIAS_GELU) r = gelu_tanh(r + to_f32(bias[col]));
      y[m * ldy_m + col * ldy_n] = from_f32<T>(r);
    }
  }
}

template <typename T, int MR, int LPR>
__global__ __launch_bounds__(gemv_max_lanes<MR>()) void gemv_splitk(
    const T* __restrict__ x, const T* __restrict__ W, const T* __restrict__ bias,
    T* __restrict__ y, int64_t M, int64_t N, int64_t K, int64_t ldx_m, int64_t ldx_k,
    int64_t ldw_k, int64_t ldw_n, int64_t ldy_m, int64_t ldy_n, int epilogue, int split_k,
    int vec, float* __restrict__ ws, unsigned* __restrict__ tickets) {
  constexpr int V = Vec<T>::N;
  constexpr int RPW = kWave / LPR;  // rows per wave load
  constexpr int BN = LPR * V;       // columns per strip
  constexpr int U = gemv_unroll<MR>();
  // red[wave][m][column]: nwaves*MR*BN floats of dynamic LDS.
  extern __shared__ float red[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int sub = lane / LPR;                 // row of the wave load
  const int cv = (lane % LPR) * V;            // column of the lane's vector within the strip
  const int64_t nb = blockIdx.x;
  const int64_t col0 = nb * BN + cv;
  const int s = blockIdx.y;
  const int64_t step = static_cast<int64_t>(nwaves) * RPW;  // row groups
  // Slices are cut on whole trips of U*step rows, shared out as evenly as
  // whole trips allow: every slice starts on a trip (so x is read as vectors)
  // and only the last one can end in a partial trip. Slices past the last
  // trip are empty and publish zeros.
  const int64_t trip_rows = static_cast<int64_t>(U) * step;
  const int64_t ntr = ceil_div(K, trip_rows);
  const int64_t tb = static_cast<int64_t>(s) * ntr / split_k;
  const int64_t te = static_cast<int64_t>(s + 1) * ntr / split_k;
  const int64_t kbeg = wave_uniform((tb * trip_rows < K) ? tb * trip_rows : K);
  const int64_t kend = wave_uniform((te * trip_rows < K) ? te * trip_rows : K);
  // With aligned rows and N a multiple of V every lane's vector is either
  // wholly inside [0, N) or wholly past it. Lanes past N load a clamped,
  // valid vector whose sums are never stored, so one branch-free loop serves
  // every strip, including the last.
  const bool vec_path = vec && (N % V == 0);
  const int64_t col_ld = (col0 < N) ? col0 : N - V;

  float acc[MR][V];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[m][e] = 0.f;

  // x rows past M read row M-1: their accumulators are never stored, and
  // clamping keeps the loads unconditional.
  const T* xrow[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) xrow[m] = x + ((m < M) ? m : M - 1) * ldx_m;

  auto fma_row = [&](const float (&xv)[MR], const T (&w)[V]) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int e = 0; e < V; ++e) acc[m][e] = __builtin_fmaf(xv[m], to_f32(w[e]), acc[m][e]);
  };

  int64_t k = kbeg + wave * RPW + sub;
  if (vec_path) {
    const T* wcol = W + col_ld;
    // A trip covers U*step rows; the lane owns U adjacent ones at lane_row,
    // so its x values of a trip are U adjacent elements of each x row: one
    // vector load per row when x is k-contiguous and aligned, instead of U
    // element loads beside the U W loads. Every lane runs the same number of
    // whole trips; the rows after them take the per-row loop below.
    // The x values go first so that the wait for them does not also wait for
    // the W rows behind them; then all W loads issue back to back and are
    // consumed in order. Trips are double buffered: the next trip's loads are
    // in flight while this one is multiplied, so a wave streams without a
    // latency gap between trips.
    const int64_t trip = U * step;
    const int64_t ntrips = (kend - kbeg) / trip;
    const int64_t lane_row = kbeg + static_cast<int64_t>(wave * RPW + sub) * U;
    constexpr int kXBytes = U * static_cast<int>(sizeof(T));
    bool xvec = ldx_k == 1 && kbeg % U == 0;
#pragma unroll
    for (int m = 0; m < MR; ++m)
      xvec = xvec && reinterpret_cast<uintptr_t>(xrow[m]) % kXBytes == 0;
    auto run_trips = [&](auto xvec_tag) {
      constexpr bool XV = decltype(xvec_tag)::value;
      auto load_trip = [&](int64_t kk, T (&xt)[U][MR], u32x4 (&raw)[U]) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          if constexpr (XV) {
            XChunk<kXBytes> c = *reinterpret_cast<const XChunk<kXBytes>*>(xrow[m] + kk);
            T e[U];
            __builtin_memcpy(e, &c, kXBytes);
#pragma unroll
            for (int u = 0; u < U; ++u) xt[u][m] = e[u];
          } else {
#pragma unroll
            for (int u = 0; u < U; ++u) xt[u][m] = xrow[m][(kk + u) * ldx_k];
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          raw[u] = load_once(reinterpret_cast<const u32x4*>(wcol + (kk + u) * ldw_k));
      };
      auto use_trip = [&](const T (&xt)[U][MR], const u32x4 (&raw)[U]) {
        if constexpr (kPackedDot<T, MR>) {
          // Rows u and u+1 in pairs: for each 32-bit word of the two W
          // vectors, v_perm_b32 gathers each column's two rows into one
          // register and v_dot2 multiplies the pair by the x pair in fp32.
          // Two instructions per two elements instead of two conversions
          // and two FMAs.
#pragma unroll
          for (int u = 0; u < U; u += 2) {
            const uint32_t xp = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, xt[u][0])) |
                                (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, xt[u + 1][0])) << 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t w0 = raw[u][j], w1 = raw[u + 1][j];
              acc[0][2 * j] = dot2<T>(__builtin_amdgcn_perm(w1, w0, 0x05040100u), xp, acc[0][2 * j]);
              acc[0][2 * j + 1] =
                  dot2<T>(__builtin_amdgcn_perm(w1, w0, 0x07060302u), xp, acc[0][2 * j + 1]);
            }
          }
          return;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float xv[MR];
#pragma unroll
          for (int m = 0; m < MR; ++m) xv[m] = to_f32(xt[u][m]);
          T w[V];
          __builtin_memcpy(w, &raw[u], 16);
          fma_row(xv, w);
        }
      };
      T xa[U][MR], xb[U][MR];
      u32x4 ra[U], rb[U];
      if (ntrips > 0) load_trip(lane_row, xa, ra);
      int64_t t = 0;
      // One x row with eight or more waves per CU: one trip in flight per
      // wave is enough and measured faster (bf16 1x11008x4096 at 32-lane
      // strips: 17.45 against 17.63 us kernel-only; 4 waves need the second
      // trip: 18.25 against 19.08 us). The sum order is the same either way.
      if (MR == 1 && nwaves >= 8) {
        for (; t < ntrips; ++t) {
          if (t > 0) load_trip(lane_row + t * trip, xa, ra);
          __builtin_amdgcn_sched_barrier(0);
          use_trip(xa, ra);
        }
      }
      // The scheduling barriers keep each trip's loads ahead of the previous
      // trip's multiplies: without them the scheduler converts each value
      // right after its load and waits for it, serialising the memory
      // latencies.
      for (; t + 1 < ntrips; t += 2) {
        load_trip(lane_row + (t + 1) * trip, xb, rb);
        __builtin_amdgcn_sched_barrier(0);
        use_trip(xa, ra);
        if (t + 2 < ntrips) load_trip(lane_row + (t + 2) * trip, xa, ra);
        __builtin_amdgcn_sched_barrier(0);
        use_trip(xb, rb);
      }
      if (t < ntrips) {
        __builtin_amdgcn_sched_barrier(0);
        use_trip(xa, ra);
      }
    };
    if constexpr (gemv_max_lanes<MR>() < 1024) {
      if (xvec)
        run_trips(std::true_type{});
      else
        run_trips(std::false_type{});
    } else {
      // 1024-lane workgroups have 128 registers per lane: one loop body only.
      (void)xvec;
      run_trips(std::false_type{});
    }
    k += ntrips * trip;
    for (; k < kend; k += step) {
      float xv[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) xv[m] = to_f32(xrow[m][k * ldx_k]);
      const u32x4 raw = load_once(reinterpret_cast<const u32x4*>(wcol + k * ldw_k));
      T w[V];
      __builtin_memcpy(w, &raw, 16);
      fma_row(xv, w);
    }
  } else {
    for (; k < kend; k += step) {
      float xv[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) xv[m] = to_f32(xrow[m][k * ldx_k]);
      T w[V];
#pragma unroll
      for (int e = 0; e < V; ++e)
        w[e] = (col0 + e < N) ? W[k * ldw_k + (col0 + e) * ldw_n] : from_f32<T>(0.f);
      fma_row(xv, w);
    }
  }

  // Rows of one wave load: lanes LPR apart hold the same columns. Butterfly
  // over those lane bits, so every lane ends with the wave's sum.
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int e = 0; e < V; ++e) acc[m][e] += __shfl_xor(acc[m][e], off, kWave);
  if (sub == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int e = 0; e < V; ++e) red[(wave * MR + m) * BN + cv + e] = acc[m][e];
  }
  __syncthreads();

  finish_block<T, MR>(red, nwaves, BN, nb, M, N, s, split_k, epilogue, bias, y, ldy_m, ldy_n, ws,
                      tickets);
}

// k-contiguous W (ldw_k == 1, ldw_n = row pitch of nn.Linear's weight).
// A wave load covers G = 64/LPR columns: lane l reads the 16-byte vector at
// k = kbeg + (j*LPR + l%LPR)*V of column l/LPR, and the matching vector of
// each x row, U vectors per lane in flight. The workgroup's waves take
// adjacent column groups, so a block is nwaves*G columns of one K slice.
template <int MR>
constexpr int gemv_dot_unroll() { return MR <= 2 ? 8 : (MR <= 4 ? 4 : 2); }

template <typename T, int MR, int LPR>
__global__ __launch_bounds__(gemv_max_lanes<MR>()) void gemv_dot(
    const T* __restrict__ x, const T* __restrict__ W, const T* __restrict__ bias,
    T* __restrict__ y, int64_t M, int64_t N, int64_t K, int64_t ldx_m, int64_t ldw_n,
    int64_t ldy_m, int64_t ldy_n, int epilogue, int split_k, float* __restrict__ ws,
    unsigned* __restrict__ tickets) {
  constexpr int V = Vec<T>::N;
  constexpr int G = kWave / LPR;  // columns per wave load
  constexpr int U = gemv_dot_unroll<MR>();
  extern __shared__ float red[];  // red[m][column of the block]

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int BN = nwaves * G;
  const int64_t nb = blockIdx.x;
  const int cw = wave * G + lane / LPR;  // this lane's column within the block
  const int64_t col = nb * BN + cw;
  const int64_t col_ld = (col < N) ? col : N - 1;  // past N: a valid column, never stored
  const int s = blockIdx.y;
  // Slices are whole vectors so every load is one aligned 16-byte access.
  const int64_t kc = ceil_div(ceil_div(K, split_k), V) * V;
  const int64_t kbeg = static_cast<int64_t>(s) * kc;
  const int64_t kend = (kbeg + kc < K) ? kbeg + kc : K;
  constexpr int64_t kStep = static_cast<int64_t>(LPR) * V;  // k per wave load and column
  const T* wcol = W + col_ld * ldw_n;

  const T* xrow[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) xrow[m] = x + ((m < M) ? m : M - 1) * ldx_m;

  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
  auto dot8 = [&](const u32x4 (&xr)[MR], const u32x4& wr) {
    T w[V];
    __builtin_memcpy(w, &wr, 16);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      T xv[V];
      __builtin_memcpy(xv, &xr[m], 16);
#pragma unroll
      for (int e = 0; e < V; ++e) acc[m] = __builtin_fmaf(to_f32(xv[e]), to_f32(w[e]), acc[m]);
    }
  };

  int64_t k = kbeg + (lane % LPR) * V;
  for (; k + (U - 1) * kStep < kend; k += U * kStep) {
    u32x4 wr[U];
    u32x4 xr[U][MR];
#pragma unroll
    for (int u = 0; u < U; ++u) wr[u] = load_once(reinterpret_cast<const u32x4*>(wcol + k + u * kStep));
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        xr[u][m] = *reinterpret_cast<const u32x4*>(xrow[m] + k + u * kStep);
    // All of the trip's loads issue before the first use.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) dot8(xr[u], wr[u]);
  }
  for (; k < kend; k += kStep) {
    u32x4 xr[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xr[m] = *reinterpret_cast<const u32x4*>(xrow[m] + k);
    dot8(xr, load_once(reinterpret_cast<const u32x4*>(wcol + k)));
  }

  // The LPR lanes of a column: butterfly over the low lane bits.
#pragma unroll
  for (int off = 1; off < LPR; off <<= 1)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] += __shfl_xor(acc[m], off, kWave);
  if (lane % LPR == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[m * BN + cw] = acc[m];
  }
  __syncthreads();
  finish_block<T, MR>(red, 1, BN, nb, M, N, s, split_k, epilogue, bias, y, ldy_m, ldy_n, ws,
                      tickets);
}


template <typename T>
int launch_gemv(const void* x, const void* W, const void* bias, void* y, int64_t M, int64_t N,
                int64_t K, int64_t ldx_m, int64_t ldx_k, int64_t ldw_k, int64_t ldw_n,
                int64_t ldy_m, int64_t ldy_n, int epilogue, int split_k, int waves, int lpr,
                void* ws, hipStream_t s) {
  constexpr int V = Vec<T>::N;
  const bool vec = ldw_n == 1 && aligned16(W) && (ldw_k * sizeof(T)) % 16 == 0;
  const int64_t es = static_cast<int64_t>(sizeof(T));
  // k-contiguous W and x, 16-byte aligned rows, whole vectors of k.
  const bool dot = ldw_k == 1 && ldx_k == 1 && K % V == 0 && aligned16(W) && aligned16(x) &&
                   (ldw_n * es) % 16 == 0 && (M == 1 || (ldx_m * es) % 16 == 0);
  const dim3 block(waves * kWave);
  unsigned* tickets = static_cast<unsigned*>(ws);
  float* partial = ws ? reinterpret_cast<float*>(static_cast<char*>(ws) + KF_WORKSPACE_COUNTER_BYTES)
                      : nullptr;
  auto go = [&](auto mr, auto lanes) -> int {
    constexpr int MR = decltype(mr)::value;
    constexpr int LPR = decltype(lanes)::value;
    if (waves * kWave > gemv_max_lanes<MR>()) {
      set_error("gemv: register pressure: %d rows allow at most %d waves, got %d", MR,
                gemv_max_lanes<MR>() / kWave, waves);
      return KF_ERR_OUT_OF_RESOURCES;
    }
    if (dot) {
      const int64_t bn = static_cast<int64_t>(waves) * (kWave / LPR);
      const dim3 grid(static_cast<unsigned>(ceil_div(N, bn)), static_cast<unsigned>(split_k));
      const size_t lds = static_cast<size_t>(MR) * bn * sizeof(float);
      hipLaunchKernelGGL((gemv_dot<T, MR, LPR>), grid, block, lds, s, static_cast<const T*>(x),
                         static_cast<const T*>(W), static_cast<const T*>(bias), static_cast<T*>(y),
                         M, N, K, ldx_m, ldw_n, ldy_m, ldy_n, epilogue, split_k, partial, tickets);
      return launch_status("gemv");
    }
    const dim3 grid(static_cast<unsigned>(ceil_div(N, static_cast<int64_t>(lpr) * V)),
                    static_cast<unsigned>(split_k));
    const size_t lds = static_cast<size_t>(waves) * MR * LPR * V * sizeof(float);
    if (lds > kGemvMaxLds) {
      set_error("gemv: waves=%d x %d rows needs %zu B of LDS for the wave reduction (limit %zu)",
                waves, MR, lds, kGemvMaxLds);
      return KF_ERR_OUT_OF_RESOURCES;
    }
    hipLaunchKernelGGL((gemv_splitk<T, MR, LPR>), grid, block, lds, s, static_cast<const T*>(x),
                       static_cast<const T*>(W), static_cast<const T*>(bias), static_cast<T*>(y),
                       M, N, K, ldx_m, ldx_k, ldw_k, ldw_n, ldy_m, ldy_n, epilogue, split_k,
                       vec ? 1 : 0, partial, tickets);
    return launch_status("gemv");
  };
  auto with_rows = [&](auto lanes) -> int {
    if (M <= 1) return go(std::integral_constant<int, 1>{}, lanes);
    if (M <= 2) return go(std::integral_constant<int, 2>{}, lanes);
    if (M <= 4) return go(std::integral_constant<int, 4>{}, lanes);
    return go(std::integral_constant<int, 8>{}, lanes);
  };
  switch (lpr) {
    case 8: return with_rows(std::integral_constant<int, 8>{});
    case 16: return with_rows(std::integral_constant<int, 16>{});
    case 32: return with_rows(std::integral_constant<int, 32>{});
    default: return with_rows(std::integral_constant<int, 64>{});
  }
}

}  // namespace
}  // namespace kf

extern "C" size_t kf_gemv_workspace_bytes(int64_t M, int64_t N, int split_k) {
  if (M <= 0 || N <= 0 || split_k <= 1) return 0;
  return static_cast<size_t>(KF_WORKSPACE_COUNTER_BYTES) +
         static_cast<size_t>(split_k) * M * N * sizeof(float);
}

namespace kf {
namespace {

// Argument checks, workspace check and dispatch shared by kf_gemv and
// kf_gemv_no_alloc; they differ only in where the workspace comes from.
int gemv_entry(int dtype, const void* x, const void* W, const void* bias, void* y, int64_t M,
               int64_t N, int64_t K, int64_t ldx_m, int64_t ldx_k, int64_t ldw_k, int64_t ldw_n,
               int64_t ldy_m, int64_t ldy_n, int epilogue, int split_k, int waves,
               int lanes_per_row, void* workspace, size_t workspace_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 0) {
    set_error("gemv: negative shape");
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (M > 8) {
    set_error("gemv: M=%lld exceeds the decode limit of 8 rows", (long long)M);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (epilogue != KF_EPILOGUE_NONE && epilogue != KF_EPILOGUE_BIAS_GELU) {
    set_error("gemv: unknown epilogue %d", epilogue);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (waves < 1 || waves > kGemvMaxWaves) {
    set_error("gemv: waves=%d outside 1..%d", waves, kGemvMaxWaves);
    return KF_ERR_OUT_OF_RESOURCES;
  }
  if (lanes_per_row != 8 && lanes_per_row != 16 && lanes_per_row != 32 && lanes_per_row != 64) {
    set_error("gemv: lanes_per_row=%d must be 8, 16, 32 or 64", lanes_per_row);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (split_k < 1 || split_k > 65535) {
    set_error("gemv: split_k=%d outside 1..65535", split_k);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (M == 0 || N == 0) return KF_OK;
  if (!x && K > 0) {
    set_error("gemv: null x");
    return KF_ERR_INVALID_ARGUMENT;
  }
  if ((!W && K > 0) || !y || (epilogue == KF_EPILOGUE_BIAS_GELU && !bias)) {
    set_error("gemv: null pointer");
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (split_k > 1) {
    // One counter per column block, and a block holds at least one column.
    if (N > KF_WORKSPACE_COUNTERS) {
      set_error("gemv: split_k=%d needs one counter per column block; N=%lld exceeds the %d "
                "counters of a workspace", split_k, (long long)N, KF_WORKSPACE_COUNTERS);
      return KF_ERR_INVALID_ARGUMENT;
    }
    const size_t need = kf_gemv_workspace_bytes(M, N, split_k);
    if (!workspace || workspace_bytes < need || !aligned16(workspace)) {
      set_error("gemv: split_k=%d needs a 16-byte aligned workspace of %zu bytes, got %zu",
                split_k, need, workspace ? workspace_bytes : (size_t)0);
      return KF_ERR_WORKSPACE;
    }
  }
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case KF_DTYPE_F32:
      return launch_gemv<float>(x, W, bias, y, M, N, K, ldx_m, ldx_k, ldw_k, ldw_n, ldy_m, ldy_n,
                                epilogue, split_k, waves, lanes_per_row, workspace, s);
    case KF_DTYPE_F16:
      return launch_gemv<f16>(x, W, bias, y, M, N, K, ldx_m, ldx_k, ldw_k, ldw_n, ldy_m, ldy_n,
                              epilogue, split_k, waves, lanes_per_row, workspace, s);
    case KF_DTYPE_BF16:
      return launch_gemv<bf16>(x, W, bias, y, M, N, K, ldx_m, ldx_k, ldw_k, ldw_n, ldy_m, ldy_n,
                               epilogue, split_k, waves, lanes_per_row, workspace, s);
    default:
      set_error("gemv: unsupported dtype code %d", dtype);
      return KF_ERR_UNSUPPORTED_DTYPE;
  }
}

// ---------------------------------------------------------------------------
// The no-allocation variant's workspace: one file-scope device array per GPU,
// laid out like every split-K workspace (counters, then fp32 partials). In
// host code `gemv_scratch` names a host-side stand-in, not device memory, so
// it is only ever used through the address hipGetSymbolAddress returns for
// the current device.
static __device__ __align__(256) unsigned char gemv_scratch[KF_GEMV_NO_ALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  void* ptr = nullptr;   // device address of gemv_scratch on this GPU
  bool cleared = false;  // its counters were zeroed by an executed (not captured) launch
};
std::mutex g_scratch_mu;
DeviceScratch g_scratch[kMaxDevices];

// Zero the counter region: one 16-byte store per lane.
__global__ __launch_bounds__(256) void clear_counters(u32x4* __restrict__ counters, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) counters[i] = u32x4{0u, 0u, 0u, 0u};
}

// Device address of the current GPU's scratch array. On the first call per
// device the counters are zeroed by a kernel on `s` (a fill kernel, not a
// memset, so a call under graph capture records an ordinary kernel node);
// until such a launch has run outside a capture, every call enqueues it again.
int gemv_scratch_for_current_device(hipStream_t s, void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("gemv_no_alloc: no usable current device (%s, device %d)", hipGetErrorName(err), dev);
    return KF_ERR_LAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  DeviceScratch& d = g_scratch[dev];
  if (d.ptr == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(gemv_scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error("gemv_no_alloc: hipGetSymbolAddress of the scratch array failed on device %d: %s",
                dev, hipGetErrorName(err));
      return KF_ERR_LAUNCH;
    }
    d.ptr = ptr;
  }
  if (!d.cleared) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(s, &capture);
    if (err != hipSuccess) {
      set_error("gemv_no_alloc: hipStreamIsCapturing failed: %s", hipGetErrorName(err));
      return KF_ERR_LAUNCH;
    }
    constexpr int n = KF_WORKSPACE_COUNTER_BYTES / 16;
    hipLaunchKernelGGL(clear_counters, dim3(n / 256), dim3(256), 0, s,
                       static_cast<u32x4*>(d.ptr), n);
    const int rc = launch_status("gemv_no_alloc: counter clear");
    if (rc != KF_OK) return rc;
    if (capture == hipStreamCaptureStatusNone) d.cleared = true;
  }
  *out = d.ptr;
  return KF_OK;
}

}  // namespace
}  // namespace kf

extern "C" int kf_gemv(int dtype, const void* x, const void* W, const void* bias, void* y,
                       int64_t M, int64_t N, int64_t K, int64_t ldx_m, int64_t ldx_k,
                       int64_t ldw_k, int64_t ldw_n, int64_t ldy_m, int64_t ldy_n, int epilogue,
                       int split_k, int waves, int lanes_per_row, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return kf::gemv_entry(dtype, x, W, bias, y, M, N, K, ldx_m, ldx_k, ldw_k, ldw_n, ldy_m, ldy_n,
                        epilogue, split_k, waves, lanes_per_row, workspace, workspace_bytes,
                        stream);
}

extern "C" int kf_gemv_no_alloc(int dtype, const void* x, const void* W, const void* bias,
                                void* y, int64_t M, int64_t N, int64_t K, int64_t ldx_m,
                                int64_t ldx_k, int64_t ldw_k, int64_t ldw_n, int64_t ldy_m,
                                int64_t ldy_n, int epilogue, int split_k, int waves,
                                int lanes_per_row, void* stream) {
  using namespace kf;
  // Shapes kf_gemv rejects, and zero-size calls, go straight to its checks
  // without touching the scratch array.
  const bool needs_scratch = split_k > 1 && split_k <= 65535 && M >= 1 && M <= 8 && N >= 1 &&
                             K >= 0;
  if (!needs_scratch)
    return gemv_entry(dtype, x, W, bias, y, M, N, K, ldx_m, ldx_k, ldw_k, ldw_n, ldy_m, ldy_n,
                      epilogue, split_k, waves, lanes_per_row, nullptr, 0, stream);
  // Only the size is checked here; shapes kf_gemv refuses for other reasons
  // (more column blocks than counters) get its own error from gemv_entry.
  const size_t need = kf_gemv_workspace_bytes(M, N, split_k);
  if (need > static_cast<size_t>(KF_GEMV_NO_ALLOC_SCRATCH_BYTES)) {
    set_error("gemv_no_alloc: split_k=%d over %lldx%lld outputs needs %zu bytes of workspace, "
              "more than the %d bytes of static scratch; use kf_gemv with a workspace",
              split_k, (long long)M, (long long)N, need, KF_GEMV_NO_ALLOC_SCRATCH_BYTES);
    return KF_ERR_WORKSPACE;
  }
  void* scratch = nullptr;
  const int rc = gemv_scratch_for_current_device(static_cast<hipStream_t>(stream), &scratch);
  if (rc != KF_OK) return rc;
  return gemv_entry(dtype, x, W, bias, y, M, N, K, ldx_m, ldx_k, ldw_k, ldw_n, ldy_m, ldy_n,
                    epilogue, split_k, waves, lanes_per_row, scratch,
                    static_cast<size_t>(KF_GEMV_NO_ALLOC_SCRATCH_BYTES), stream);
}
