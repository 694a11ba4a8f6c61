// Elementwise add c[i] = a[i] + b[i] for gfx950: the pure HBM stream.
//
// The rebuild of the reference's vector_add (kernels/vector_add.py:24-40).
// A workgroup owns `block_size` consecutive elements; each lane holds
// E = block_size / lanes of them as E/W loads of W elements, W = 16 bytes'
// worth (or all E when E is smaller), placed so that load j of every lane is
// one contiguous sweep of the workgroup. All loads of a and b are issued
// before the first add. The sum is formed in fp32 and rounded once: for
// fp16 and bf16 that is the correctly rounded 16-bit sum, since fp32 carries
// more than twice their precision plus two bits.
#include <type_traits>

#include "common.h"

namespace kf {

namespace {

// Raw storage of one load of `Bytes` bytes.
template <int Bytes>
struct Raw;
template <>
struct Raw<2> { using type = uint16_t; };
template <>
struct Raw<4> { using type = uint32_t; };
template <>
struct Raw<8> { using type = uint32_t __attribute__((ext_vector_type(2))); };
template <>
struct Raw<16> { using type = u32x4; };

template <typename T, int E>
__global__ __launch_bounds__(1024) void vector_add_kernel(const T* __restrict__ a,
                                                          const T* __restrict__ b,
                                                          T* __restrict__ c, int64_t n, int vec) {
  constexpr int V = Vec<T>::N;
  constexpr int W = (E < V) ? E : V;  // elements per load
  constexpr int NL = E / W;           // loads per lane per operand
  using R = typename Raw<W * static_cast<int>(sizeof(T))>::type;
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * nt * E;
  auto at = [&](int j) { return base + (static_cast<int64_t>(j) * nt + t) * W; };

  if (vec && base + static_cast<int64_t>(nt) * E <= n) {
    // A whole block: every load is in range.
    R ra[NL], rb[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      ra[j] = load_once(reinterpret_cast<const R*>(a + at(j)));
      rb[j] = load_once(reinterpret_cast<const R*>(b + at(j)));
    }
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      T va[W], vb[W], vc[W];
      __builtin_memcpy(va, &ra[j], sizeof(R));
      __builtin_memcpy(vb, &rb[j], sizeof(R));
#pragma unroll
      for (int e = 0; e < W; ++e) vc[e] = from_f32<T>(to_f32(va[e]) + to_f32(vb[e]));
      R rc;
      __builtin_memcpy(&rc, vc, sizeof(R));
      *reinterpret_cast<R*>(c + at(j)) = rc;
    }
    return;
  }
  // The partial last block, or operands not aligned for W-element loads.
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int64_t i0 = at(j);
#pragma unroll
    for (int e = 0; e < W; ++e)
      if (i0 + e < n) c[i0 + e] = from_f32<T>(to_f32(a[i0 + e]) + to_f32(b[i0 + e]));
  }
}

template <typename F>
int dispatch_elems(int e, F&& f) {
  switch (e) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, 64>{});
    default:
      set_error("vector_add: %d elements per lane is not built (1..64, powers of two)", e);
      return KF_ERR_NOT_BUILT;
  }
}

template <typename T>
int launch_vector_add(const void* a, const void* b, void* c, int64_t n, int block_size,
                      int waves, hipStream_t s) {
  const int lanes = waves * kWave;
  const int e = block_size / lanes;
  const int64_t blocks = ceil_div(n, block_size);
  if (blocks > 0x7fffffffLL) {
    set_error("vector_add: %lld workgroups exceed the grid limit; use a larger block_size",
              (long long)blocks);
    return KF_ERR_INVALID_ARGUMENT;
  }
  return dispatch_elems(e, [&](auto ec) -> int {
    constexpr int E = decltype(ec)::value;
    constexpr int W = (E < Vec<T>::N) ? E : Vec<T>::N;
    const uintptr_t mask = W * sizeof(T) - 1;
    const bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                       reinterpret_cast<uintptr_t>(c)) & mask) == 0;
    hipLaunchKernelGGL((vector_add_kernel<T, E>), dim3(static_cast<unsigned>(blocks)),
                       dim3(lanes), 0, s, static_cast<const T*>(a), static_cast<const T*>(b),
                       static_cast<T*>(c), n, vec ? 1 : 0);
    return launch_status("vector_add");
  });
}

}  // namespace
}  // namespace kf

extern "C" int kf_vector_add(int dtype, const void* a, const void* b, void* c, int64_t n,
                             int block_size, int waves, void* stream) {
  using namespace kf;
  if (n < 0) {
    set_error("vector_add: negative element count %lld", (long long)n);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (waves < 1 || waves > 16) {
    set_error("waves=%d outside 1..16 (workgroup limit of 1024 lanes)", waves);
    return KF_ERR_OUT_OF_RESOURCES;
  }
  const int lanes = waves * kWave;
  if (block_size < lanes || block_size % lanes != 0) {
    set_error("vector_add: block_size=%d is not a whole number of elements per lane at "
              "waves=%d",
              block_size, waves);
    return KF_ERR_INVALID_ARGUMENT;
  }
  if (dtype != KF_DTYPE_F32 && dtype != KF_DTYPE_F16 && dtype != KF_DTYPE_BF16) {
    set_error("vector_add: unsupported dtype code %d", dtype);
    return KF_ERR_UNSUPPORTED_DTYPE;
  }
  if (n == 0) return KF_OK;
  if (!a || !b || !c) {
    set_error("vector_add: null pointer");
    return KF_ERR_INVALID_ARGUMENT;
  }
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case KF_DTYPE_F32: return launch_vector_add<float>(a, b, c, n, block_size, waves, s);
    case KF_DTYPE_F16: return launch_vector_add<f16>(a, b, c, n, block_size, waves, s);
    default: return launch_vector_add<bf16>(a, b, c, n, block_size, waves, s);
  }
}
