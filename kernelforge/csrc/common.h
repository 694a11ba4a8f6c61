// Shared device/host helpers for the gfx950 kernels behind the kernelforge C-ABI.
//
// Everything here is CDNA4-specific: wave64, 16-byte vector global loads,
// fp32 math on fp16/bf16 storage. There is one code path per op.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernelforge_hip.h"

namespace kf {

// Storage types. _Float16 and __bf16 are the clang-native 16-bit floats; the
// MFMA builtins take vectors of exactly these.
using f16 = _Float16;
using bf16 = __bf16;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// 16 bytes: the widest global load a lane issues (global_load_dwordx4).
template <typename T>
struct Vec {
  static constexpr int N = 16 / sizeof(T);
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(bf16 v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return static_cast<bf16>(v); }

// Load / store N contiguous elements as one 16-byte transaction. The caller
// guarantees 16-byte alignment (checked on the host before a vector variant
// is chosen).
template <typename T>
__device__ __forceinline__ void load16(const T* p, T (&out)[Vec<T>::N]) {
  u32x4 raw = *reinterpret_cast<const u32x4*>(p);
  __builtin_memcpy(out, &raw, 16);
}
template <typename T>
__device__ __forceinline__ void store16(T* p, const T (&in)[Vec<T>::N]) {
  u32x4 raw;
  __builtin_memcpy(&raw, in, 16);
  *reinterpret_cast<u32x4*>(p) = raw;
}

// Streaming load (non-temporal cache policy) for data a kernel reads once.
// Measured on MI355X with flushed caches: the decode GEMV's weight stream
// 27.4 -> 26.3 us and vector_add of 2^26 fp32 132 -> 121 us; the row
// kernels got slower with it (RMSNorm fp32 4096x4096 25.7 -> 30.8 us) and
// non-temporal stores gained nothing, so only those two loads use it.
template <typename R>
__device__ __forceinline__ R load_once(const R* p) {
  return __builtin_nontemporal_load(p);
}

// Wave64 butterfly reductions. Every lane ends with the full result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Thread-local error text for kf_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Map the result of a launch onto a C-ABI status code, recording the message.
int launch_status(const char* what);

}  // namespace kf
