// Direct-to-LDS MFMA GEMM for 16-bit and fp32 inputs on gfx950 (the fast path).
//
// Differences from the register-staged kernel in gemm_impl.h:
//   * Global -> LDS with global_load_lds_dwordx4: each lane's 16 bytes land at
//     (M0 + 16*lane) in LDS without passing through VGPRs. The loads use the
//     scalar-base form: one wave-uniform SGPR base per operand and k-slice and
//     one 32-bit per-lane byte offset per chunk that is fixed for the whole
//     K loop, so the DMA costs almost no VGPRs.
//   * STAGES (2 or 3) LDS buffers; with 3, slices t+1 and t+2 are in flight
//     while slice t is multiplied. Each wave waits (vmcnt) for exactly its own
//     loads of the next slice, then a plain s_barrier publishes them: the
//     fences of __syncthreads() would wait for every outstanding load,
//     including the prefetch of slice t+2.
//   * The DMA is issued from inline assembly so the compiler's wait-count
//     pass does not track it; every wait for it is explicit. (Untracked
//     in-order loads can only make the compiler's own waits longer.)
//   * No padding: LDS rows are dense and 16-byte chunks are XOR-swizzled by
//     row (swz_k, swz_n below). The swizzles keep the fragment reads at the
//     conflict-free rate of gfx950's LDS and leave the per-lane offsets
//     invariant under the row steps the code adds as immediates.
//   * Row-major B stays n-contiguous in LDS and is read with
//     ds_read_b64_tr_b16: within a 16-lane group, lane i addressing
//     (row0 + i/4, col0 + 4*(i%4)) receives column col0+i of rows
//     row0..row0+3, which is the MFMA B-operand layout. Two such reads give
//     the 8 consecutive k a v_mfma_f32_16x16x32 lane needs.
//   * Scheduling groups interleave the fragment reads of a slice's second
//     32-wide k step with the MFMAs of its first, so LDS latency is spent
//     under MFMAs and the reads are done by the slice's barrier.
//
// fp32 runs the same pipeline: a k-slice is 32 elements, so every row of it
// is still 128 bytes and the A side (DMA, k swizzle, 16-byte fragment reads)
// is byte for byte the 16-bit one. Each 16x16 fragment step is four
// v_mfma_f32_16x16x4_f32 over 16 k; n-contiguous B, which has no transposing
// read for 32-bit elements, is read four bytes per lane per MFMA under its
// own swizzle (swz_n4).
//
// Requirements (checked on the host): 16-bit or fp32 dtype, A k-contiguous
// with a 16-byte aligned base and row pitch, B either n-contiguous (BLAYOUT
// 0) or k-contiguous (BLAYOUT 1) with the same alignment, N (BLAYOUT 0) and
// K multiples of a 16-byte chunk (8 or 4 elements), and per-lane byte
// offsets (BM rows of A, BK k-rows or BN rows of B) below 4 GiB. BK is 128
// bytes of elements: one A row of a k-slice is 128 bytes.
// M/N edges clamp rows/columns (results discarded); the partial last k-slice
// clamps k into range and zeroes its chunks past K after the DMA lands.
//
// Split-K (stream-K over the split tiles): with args.split_k > 1, tiles
// [0, args.full_tiles) run one program each and the remaining T tiles are
// shared out over P = args.tail_programs programs. Their T*slices (tile,
// k-slice) iterations, tile-major, are cut into P contiguous ranges; program p
// walks its range segment by segment (a range may end inside one tile and go
// on in the next), moving its operand bases to each segment's first slice and
// running the ordinary loop over a K of its own. A segment that is a whole
// tile writes C directly. Any other segment publishes its fp32 accumulators to
// one of the program's two partial slots (its first segment, its last), in
// fragment order so the stores coalesce, and takes the tile's ticket; the
// last of the tile's programs adds the tile's segments in ascending k -- the
// same order whichever program is last, so results are deterministic --
// applies the epilogue, writes C and returns the ticket to zero. With T*S <=
// P and S dividing the slice count this is the classic split-K into S equal
// k-ranges per tile.
#pragma once

#include <type_traits>

#include "gemm_impl.h"

namespace kf {
namespace gemm {

#define KF_LDS __attribute__((address_space(3)))

typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __bf16 bf16x4_t __attribute__((__vector_size__(4 * sizeof(__bf16))));

// Every operand row of a k-slice is 128 bytes: 64 elements of a 16-bit type,
// 32 of fp32.
constexpr int kSliceRowBytes = 128;

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16 on 16-bit inputs. Lane l holds A row l%32 (B column
// l%32) at k 8*(l/32)..+7 of a 16-wide k step, and accumulator element v of
// C row 8*(v/4) + 4*(l/32) + v%4, column l%32.
template <typename T>
struct Mma32;
template <>
struct Mma32<f16> {
  __device__ __forceinline__ static void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mma32<bf16> {
  __device__ __forceinline__ static void run(const u32x4& a, const u32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

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

__device__ __forceinline__ uint32_t lds_offset(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((KF_LDS const char*)(p)));
}

// A wave-uniform pointer, moved into SGPRs for the scalar-base load form.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// A wave-uniform 64-bit integer, moved into SGPRs. Values the compiler
// computes with vector instructions (64-bit division) would otherwise occupy
// VGPRs for the whole K loop.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// 16 bytes per lane from (sbase + voff) into LDS at lds + 16*lane; sbase and
// lds are wave-uniform. M0 holds the LDS address for the instruction.
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(uniform_ptr(sbase)), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Split-K partial tiles move through raw buffer stores and loads of 16 bytes
// with the cache policy of the compiler's agent-scope atomic dword store/load
// (sc1): coherent across XCDs without writing back or invalidating whole
// L2s. The buffer resource covers one partial tile (bytes in num_records;
// the third dword selects 32-bit data, as raw buffer access on gfx9 needs).
constexpr int kBufferWord3 = 0x00020000;
constexpr int kCachePolicySc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(float* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, bytes, kBufferWord3);
}

// Workgroup barrier for the DMA pipeline: this wave's LDS reads and writes
// are complete (lgkmcnt(0)); its DMA was waited for explicitly before.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt unconstrained
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Swizzled 16-byte chunk of a k-contiguous row (8 chunks per 128-byte row)
// and of an n-contiguous B row of ROW_CHUNKS chunks.
//
// gfx950's LDS serves a ds_read_b128 in 4.4 clocks and a ds_read_b64 (or
// ds_read_b64_tr_b16) in 2.5 clocks when no two lanes of one pass share a
// bank with different addresses; the 8-byte reads pass lanes 0-31, then
// 32-63, each over 32 eight-byte bank pairs. The swizzles below were chosen
// against that rule and measured at those rates, eight waves per CU, for the
// fragment reads of both MFMA shapes this library uses (16x16x32: 16 rows x
// 4 lane groups; 32x32x16: 32 rows x 2 lane groups), where the earlier forms
// took 8.0 (A, one of the two shapes) and 4.0 clocks (B, 32x32x16).
//
// k-contiguous: chunk ^ ((row >> 1) & 7) -- row bits 1..3, so rows 16 and 32
// apart (the fragment steps added as immediates) share it.
// n-contiguous: row bits 0, 1 and 3 only, so rows r and r + 4 (a fragment's
// second transposing read) and rows 16 apart share it.
__device__ __forceinline__ int swz_k(int chunk, int row) {
  return chunk ^ ((row >> 1) & 7);
}
template <int ROW_CHUNKS>
__device__ __forceinline__ int swz_n(int chunk, int row) {
  if constexpr (ROW_CHUNKS >= 16) return chunk ^ (((row & 3) << 2) ^ (((row >> 3) & 1) << 1));
  return chunk ^ ((row & 3) << 1);
}
// n-contiguous fp32 B rows. Its fragments are read 4 bytes per lane: for one
// MFMA, lane group g reads 16 columns (64 bytes) of k-row 4g + e, so the four
// groups read rows 4 apart, whose rows (a multiple of 256 bytes long) fall on
// the same banks unswizzled. XOR-ing the chunk with row bits 2..3 puts the
// groups' 64-byte runs in four different quarters of the 256-byte bank
// window; rows differing in bits 0, 1 and 4 (the MFMAs of a step, the two
// steps of a slice) share the swizzle, so their offsets differ by immediates.
template <int ROW_CHUNKS>
__device__ __forceinline__ int swz_n4(int chunk, int row) {
  static_assert(ROW_CHUNKS >= 16, "fp32 n-contiguous B needs 16 or more chunks per row");
  return chunk ^ (((row >> 2) & 3) << 2);
}
template <int ES, int ROW_CHUNKS>
__device__ __forceinline__ int swz_nb(int chunk, int row) {
  if constexpr (ES == 4) return swz_n4<ROW_CHUNKS>(chunk, row);
  else return swz_n<ROW_CHUNKS>(chunk, row);
}

template <int BM, int BN, int WAVES, int STAGES, int ES = 2>
struct DirectTile {
  static constexpr int V = 16 / ES;                   // elements per 16-byte chunk
  static constexpr int BK = kSliceRowBytes / ES;      // elements per k-slice
  static constexpr int NT = WAVES * kWave;
  static constexpr int WM = WaveGrid<WAVES, BM, BN>::WM;
  static constexpr int WN = WaveGrid<WAVES, BM, BN>::WN;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  // Fragment edge: 32x32x16 MFMAs for the 256x256 tile, whose 64x128 wave
  // tiles hold 128 accumulators per lane either way but need half the
  // fragment registers of 16x16 pieces; 16x16x32 everywhere else.
  static constexpr int MF = (BM == 256 && BN == 256 && ES == 2) ? 32 : 16;
  static constexpr int FM = TM / MF;
  static constexpr int FN = TN / MF;
  // MFMA k steps per slice: 64 bytes of a row each for 16x16 fragments (32
  // 16-bit k, or 16 fp32 k as four 16x16x4 MFMAs), 32 bytes for 32x32x16.
  static constexpr int kSteps = MF == 32 ? 4 : 2;
  // Byte sizes of one stage.
  static constexpr int kABytes = BM * kSliceRowBytes;
  static constexpr int kBBytes = BN * kSliceRowBytes;
  static constexpr int kStageBytes = kABytes + kBBytes;
  // Static LDS: the stages, or the staged C tile of the 32x32 path if larger.
  static constexpr int kCStageBytes = BM * (BN + 8) * ES;
  static constexpr int kLdsBytes = (MF == 32 && kCStageBytes > STAGES * kStageBytes)
                                       ? kCStageBytes
                                       : STAGES * kStageBytes;
  // 16-byte chunks per stage and DMA instructions per lane.
  static constexpr int kAIters = BM * (kSliceRowBytes / 16) / NT;
  static constexpr int kBIters = BN * (kSliceRowBytes / 16) / NT;
  static constexpr int kPer = kAIters + kBIters;  // vector-memory instructions per slice
  static constexpr int kBRowChunks = BN / V;      // BLAYOUT 0: chunks per k-row of B
  static_assert(STAGES == 2 || STAGES == 3, "two or three LDS stages");
  static_assert((BM * 8) % NT == 0 && (BN * 8) % NT == 0, "DMA must tile the stage");
  static_assert(ES == 2 || ES == 4, "16-bit or fp32 operands");
  static_assert(TM % MF == 0 && TN % MF == 0, "wave tile must be whole MFMA fragments");
  static_assert(MF == 16 || STAGES == 2, "the 256x256 tile runs two stages");
  static_assert(2 * kPer < 64, "outstanding DMA must fit the vmcnt counter");
};

template <typename T, int BM, int BN, int WAVES, int BLAYOUT, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void gemm_direct_kernel(Args args) {
  using Tl = DirectTile<BM, BN, WAVES, STAGES, static_cast<int>(sizeof(T))>;
  constexpr int ES = static_cast<int>(sizeof(T));  // bytes per element
  constexpr int V = Tl::V;                         // elements per 16-byte chunk
  constexpr int BK = Tl::BK;
  constexpr int NT = Tl::NT;
  constexpr int FM = Tl::FM, FN = Tl::FN;
  constexpr int kPer = Tl::kPer;
  static_assert(BLAYOUT == 1 || BN >= 64, "n-contiguous B needs >= 8 chunks per k-row");

  __shared__ __attribute__((aligned(16))) char lds[Tl::kLdsBytes];
  char* const s0 = lds;
  char* const s1 = lds + Tl::kStageBytes;
  char* const s2 = lds + (STAGES == 3 ? 2 * Tl::kStageBytes : 0);

  const int64_t M = args.M, N = args.N;

  // ---- work: whole tiles, then ranges of k-slices over the split tiles -----
  // Tiles [0, full) run one program each (every tile when split_k is 1),
  // regrouped per XCD and into GROUP_M bands. The other T = tiles - full
  // tiles are shared out over P = args.tail_programs programs: their T*nk
  // (tile, k-slice) iterations, tile-major, are cut into P contiguous ranges,
  // program p taking [floor(p*I/P), floor((p+1)*I/P)) with P <= I, so no
  // range is empty. A range may end inside one tile and go on in the next, so
  // a program works through one or more segments; a segment that is a whole
  // tile writes C itself, the others publish an fp32 partial tile for the
  // tile's last-arriving program.
  const int64_t tiles_m = ceil_div(M, BM);
  const int64_t tiles_n = ceil_div(N, BN);
  const int64_t ntiles = tiles_m * tiles_n;
  const int64_t nk_all = ceil_div(args.K, static_cast<int64_t>(BK));
  const int64_t full = args.split_k > 1 ? args.full_tiles : ntiles;
  const int64_t P = args.split_k > 1 ? args.tail_programs : 1;
  const int64_t I = (ntiles - full) * nk_all;
  const bool streamed = static_cast<int64_t>(blockIdx.x) >= full;
  const int64_t prog = streamed ? static_cast<int64_t>(blockIdx.x) - full : 0;
  const int64_t it_first = uniform64(streamed ? prog * I / P : 0);
  const int64_t it_end = uniform64(streamed ? (prog + 1) * I / P : 1);  // unsplit: one pass
  auto owner = [&](int64_t i) { return ((i + 1) * P - 1) / I; };  // program holding iteration i

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Tl::WN;
  const int wn = wave % Tl::WN;

  for (int64_t it = it_first; it < it_end;) {
  int64_t pid, kb, ke;
  if (!streamed) {
    pid = blockIdx.x;
    if (full % kNumXcd == 0) pid = (pid % kNumXcd) * (full / kNumXcd) + pid / kNumXcd;
    kb = 0;
    ke = nk_all;
    it = it_end;
  } else {
    const int64_t t = uniform64(it / nk_all);
    kb = it - t * nk_all;
    ke = kb + (it_end - it) < nk_all ? kb + (it_end - it) : nk_all;
    pid = full + t;
    it += ke - kb;
  }
  pid = uniform64(pid);
  const int64_t tile = pid;
  // This segment's k-range: slices [kb, ke), as a K of its own.
  const int64_t kt0 = kb;
  int64_t K = args.K - kt0 * BK;
  K = K < (ke - kb) * BK ? K : (ke - kb) * BK;
  const int64_t gm = args.group_m;
  const int64_t in_group = gm * tiles_n;
  const int64_t group = pid / in_group;
  const int64_t first_m = group * gm;
  const int64_t size_m = (tiles_m - first_m < gm) ? (tiles_m - first_m) : gm;
  const int64_t m0 = uniform64((first_m + (pid % in_group) % size_m) * BM);
  const int64_t n0 = uniform64(((pid % in_group) / size_m) * BN);

  // ---- DMA sources: tile bases + per-lane byte offsets -----------------------
  // Chunk q = j*NT + tid is written to LDS slot q; its source is the chunk at
  // the slot's position XOR the row's swizzle. Rows past M (and columns or
  // rows of B past N) are clamped to the last valid one.
  const char* const a_tile = static_cast<const char*>(args.A) + m0 * args.lda_m * ES + kt0 * BK * ES;
  const int64_t lda_b = args.lda_m * ES;
  const int64_t ldb_b = (BLAYOUT == 0 ? args.ldb_k : args.ldb_n) * ES;  // bytes per B row
  const char* const b_tile = static_cast<const char*>(args.B) +
                             (BLAYOUT == 0 ? n0 * ES + kt0 * BK * ldb_b : n0 * ldb_b + kt0 * BK * ES);
  // The 256x256 tile computes its per-lane offsets from an opaque copy of the
  // lane id, so the compiler cannot hoist the 64-bit row products out of the
  // segment loop, where they would not fit its registers and spill.
  int dtid = tid;
  if constexpr (Tl::MF == 32) asm volatile("" : "+v"(dtid));
  constexpr int kRowsPerIter = NT / 8;  // k-contiguous rows (A, BLAYOUT 1) per DMA instruction
  // Chunk j of a lane reuses the k swizzle of its row kr for row kr + j*kRowsPerIter;
  // swz_k reads row bits 1..3, so the row step must be a multiple of 16.
  static_assert(kRowsPerIter % 16 == 0, "the DMA row step (lanes / 8) must keep the k swizzle: two or more waves");
  const int kr = dtid >> 3;             // this lane's row within an instruction's rows
  const int kc = swz_k(dtid & 7, kr) * V;  // its k within the slice; same for every j
  uint32_t a_off[Tl::kAIters];
#pragma unroll
  for (int j = 0; j < Tl::kAIters; ++j) {
    int64_t r = j * kRowsPerIter + kr;
    r = (m0 + r < M) ? r : (M - 1 - m0);
    a_off[j] = static_cast<uint32_t>(r * lda_b + kc * ES);
  }
  uint32_t b_off[Tl::kBIters];
  // BLAYOUT 0: k-row of chunk j within the slice. Recomputed where the
  // partial last slice needs it rather than held through the K loop.
  auto b_row = [&](int j) { return (j * NT + tid) / Tl::kBRowChunks; };
#pragma unroll
  for (int j = 0; j < Tl::kBIters; ++j) {
    const int q = j * NT + dtid;
    if constexpr (BLAYOUT == 0) {
      const int r = q / Tl::kBRowChunks;
      int64_t col = swz_nb<ES, Tl::kBRowChunks>(q % Tl::kBRowChunks, r) * V;
      // The last whole chunk of the row; N % V == 0 (kf_gemm admits n-contiguous
      // B on this pipeline only then), so it lies at or right of n0.
      col = (n0 + col < N) ? col : (N - V - n0);
      b_off[j] = static_cast<uint32_t>(r * ldb_b + col * ES);
    } else {
      int64_t r = j * kRowsPerIter + kr;
      r = (n0 + r < N) ? r : (N - 1 - n0);
      b_off[j] = static_cast<uint32_t>(r * ldb_b + kc * ES);
    }
  }
  const uint32_t lds_lane0 = static_cast<uint32_t>(wave * 64 * 16);

  const int64_t nk = ceil_div(K, BK);
  const bool ktail = (K % BK) != 0;

  // Enqueue the DMA of k-slice kt into `stage`.
  auto issue_full = [&](const char* stage, int64_t kt) {
    const uint32_t la = lds_offset(stage) + lds_lane0;
    const char* ab = a_tile + kt * BK * ES;
    const char* bb = b_tile + (BLAYOUT == 0 ? kt * BK * ldb_b : kt * BK * ES);
#pragma unroll
    for (int j = 0; j < Tl::kAIters; ++j) dma16(ab, a_off[j], la + j * NT * 16);
#pragma unroll
    for (int j = 0; j < Tl::kBIters; ++j) dma16(bb, b_off[j], la + Tl::kABytes + j * NT * 16);
  };
  // The partial last slice: k is clamped into range per lane so every source
  // stays inside its operand (K % V == 0, so K - V >= k0); the chunks past K
  // are zeroed by fix() once the DMA has landed.
  // Offsets within the slice are 32-bit: `rem` (1..BK-1, a multiple of V) is
  // the number of valid k of the partial slice.
  auto issue_last = [&](const char* stage, int64_t kt) {
    const uint32_t la = lds_offset(stage) + lds_lane0;
    const int64_t k0 = kt * BK;
    const int rem = static_cast<int>(K - k0);
    const int k = kc < rem ? kc : rem - V;
    const uint32_t dk = static_cast<uint32_t>(k * ES) - static_cast<uint32_t>(kc * ES);
    const char* ab = a_tile + k0 * ES;
#pragma unroll
    for (int j = 0; j < Tl::kAIters; ++j) dma16(ab, a_off[j] + dk, la + j * NT * 16);
    if constexpr (BLAYOUT == 0) {
      const char* bb = b_tile + k0 * ldb_b;
#pragma unroll
      for (int j = 0; j < Tl::kBIters; ++j) {
        const int kb = b_row(j) < rem ? b_row(j) : rem - 1;
        const uint32_t off = b_off[j] - static_cast<uint32_t>(b_row(j) * ldb_b) +
                             static_cast<uint32_t>(kb * ldb_b);
        dma16(bb, off, la + Tl::kABytes + j * NT * 16);
      }
    } else {
      const char* bb = b_tile + k0 * ES;
#pragma unroll
      for (int j = 0; j < Tl::kBIters; ++j) dma16(bb, b_off[j] + dk, la + Tl::kABytes + j * NT * 16);
    }
  };
  auto issue = [&](const char* stage, int64_t kt) {
    if (ktail && kt == nk - 1)
      issue_last(stage, kt);
    else
      issue_full(stage, kt);
  };
  // Zero the chunks of slice kt that lie past K (after its DMA landed).
  auto fix = [&](char* stage, int64_t kt) {
    if (!(ktail && kt == nk - 1)) return;
    const int rem = static_cast<int>(K - kt * BK);
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < Tl::kAIters; ++j)
      if (kc >= rem) *reinterpret_cast<u32x4*>(stage + (j * NT + tid) * 16) = z;
#pragma unroll
    for (int j = 0; j < Tl::kBIters; ++j) {
      const int kk = BLAYOUT == 0 ? b_row(j) : kc;
      if (kk >= rem) *reinterpret_cast<u32x4*>(stage + Tl::kABytes + (j * NT + tid) * 16) = z;
    }
  };

  // ---- fragments ----------------------------------------------------------------
  // Tiles with 128 or more accumulator registers per lane (4 waves over 256x128
  // or 128x256) run one wave per SIMD, whose 512 registers exceed the 256
  // VGPRs: an operand in an AGPR lets the compiler put accumulators there.
  // The 16x16x32 tiles (the 32x32x16 one holds its accumulators in VGPRs:
  // the hint made the compiler split them 128/128 between the files and spill).
  constexpr int MF = Tl::MF;
  constexpr int kSteps = Tl::kSteps;
  using AccT = std::conditional_t<MF == 32, f32x16, f32x4>;
  if constexpr (MF == 16 && FM * FN * 4 >= 128) asm volatile("" ::"a"(0.0f));
  AccT acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = AccT{};

  const int g = lane >> 4;   // 16x16x32: lane group, k offset 8*g within a 32-wide step
  const int li = lane & 15;  // 16x16x32: row (A) / column (B) within a fragment
  const int fr = MF == 32 ? (lane & 31) : li;  // the lane's row (A) / column (B) in a fragment
  // Stage-relative byte offsets of this lane's fragments for k step c. Rows
  // MF apart share the swizzle, so fragment i adds i*MF rows as an immediate.
  const int ar = wm * Tl::TM + fr;
  int a_frag[kSteps];
  int b_frag[kSteps][FN];
#pragma unroll
  for (int c = 0; c < kSteps; ++c) {
    // 16-byte k chunk of the 64-wide slice: 16x16x32 lane groups take chunks
    // 4c..4c+3, 32x32x16 lane halves chunks 2c and 2c+1.
    const int kch = MF == 32 ? 2 * c + (lane >> 5) : c * 4 + g;
    a_frag[c] = ar * 128 + swz_k(kch, ar) * 16;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (BLAYOUT == 0 && ES == 4) {
        // fp32: lane (g, li) holds column li of k-rows 16c + 4g + e for the
        // step's four 16x16x4 MFMAs e = 0..3 -- the k of its A chunk 4c + g,
        // element e. Four 4-byte reads, the rows e apart (same swizzle).
        const int col = wn * Tl::TN + j * 16 + li;
        const int r0 = c * 16 + 4 * g;
        b_frag[c][j] = Tl::kABytes + r0 * (BN * 4) + swz_n4<Tl::kBRowChunks>(col >> 2, r0) * 16 + (col & 3) * 4;
      } else if constexpr (BLAYOUT == 0) {
        // Transposing reads: a 16-lane group covers 16 columns and 4 k-rows
        // per read; 32x32x16 groups alternate column halves, then k halves.
        const int col = MF == 32 ? wn * Tl::TN + j * 32 + 16 * (g & 1) + (li & 3) * 4
                                 : wn * Tl::TN + j * 16 + (li & 3) * 4;
        const int r0 = MF == 32 ? c * 16 + 8 * (g >> 1) + (li >> 2)
                                : c * 32 + 8 * g + (li >> 2);  // rows r0 and r0 + 4 share the swizzle
        b_frag[c][j] = Tl::kABytes + r0 * (BN * 2) + swz_n<Tl::kBRowChunks>(col >> 3, r0) * 16 + (col & 7) * 2;
      } else {
        const int br = wn * Tl::TN + j * MF + fr;
        b_frag[c][j] = Tl::kABytes + br * 128 + swz_k(kch, br) * 16;
      }
    }
  }
  // B offset of fragment j at k step c. On the 32x32 path the swizzles make
  // the steps constant: n-contiguous rows 16 apart share the n-swizzle (the
  // k steps differ by 16 rows), k-contiguous rows 32 apart the k one (the
  // fragments differ by 32 rows), so one offset register serves each.
  auto bfrag_off = [&](int c, int j) -> int {
    if constexpr (MF == 32 && BLAYOUT == 0) return b_frag[0][j] + c * 16 * BN * 2;
    else if constexpr (MF == 32) return b_frag[c][0] + j * 32 * 128;
    else return b_frag[c][j];
  };
  auto load_frags = [&](const char* S, int c, u32x4 (&af)[FM], u32x4 (&bf)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const u32x4*>(S + a_frag[c] + i * MF * 128);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (BLAYOUT == 0 && ES == 4) {
        const char* p = S + bfrag_off(c, j);
        bf[j] = u32x4{*reinterpret_cast<const uint32_t*>(p),
                      *reinterpret_cast<const uint32_t*>(p + BN * 4),
                      *reinterpret_cast<const uint32_t*>(p + 2 * BN * 4),
                      *reinterpret_cast<const uint32_t*>(p + 3 * BN * 4)};
      } else if constexpr (BLAYOUT == 0) {
        const uint64_t lo = ds_read_tr4<T>(S + bfrag_off(c, j));
        const uint64_t hi = ds_read_tr4<T>(S + bfrag_off(c, j) + 4 * BN * 2);
        bf[j] = u32x4{static_cast<uint32_t>(lo), static_cast<uint32_t>(lo >> 32),
                      static_cast<uint32_t>(hi), static_cast<uint32_t>(hi >> 32)};
      } else {
        bf[j] = *reinterpret_cast<const u32x4*>(S + bfrag_off(c, j));
      }
    }
  };
  // Snake order: odd fragment rows walk the columns backwards, so every MFMA
  // after the first changes one operand, never both. Random operands hold the
  // board at its power limit and fewer operand changes buy clock: 0.4-0.8%
  // on 2048x4096x4096 (fp16, bf16) and 0.2-0.3% on the fused 4096x11008x4096,
  // interleaved flushed medians, bit-identical outputs (each accumulator
  // keeps its k order).
  auto mma_all = [&](const u32x4 (&af)[FM], const u32x4 (&bf)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int jj = 0; jj < FN; ++jj) {
        const int j = (i & 1) ? FN - 1 - jj : jj;
        if constexpr (MF == 32)
          Mma32<T>::run(af[i], bf[j], acc[i][j]);
        else
          Mma<T>::run(af[i], bf[j], acc[i][j]);
      }
  };
  // Both 32-wide k steps of a slice are read and multiplied before its
  // barrier. The scheduling groups pin the order: step 0's reads, then step
  // 1's reads alternating one for one with step 0's MFMAs, then step 1's
  // MFMAs, so each wave's reads run under its own (and the SIMD's other
  // wave's) MFMAs and the barrier's lgkmcnt(0) finds them done. Left to
  // itself the scheduler issues step 1's reads late and waits for them at
  // the barrier with most MFMAs still to issue. (Carrying step 1's MFMAs
  // over the barrier instead measured slower: it keeps a third fragment set
  // live.)
  // LDS reads per k step: an A fragment is one 16-byte read; a B fragment one
  // (k-contiguous), two transposing (16-bit n-contiguous) or four 4-byte reads
  // (fp32 n-contiguous). MFMA instructions per k step: fp32 fragments take
  // four 16x16x4 MFMAs each.
  constexpr int kBReads = BLAYOUT == 1 ? 1 : (ES == 4 ? 4 : 2);
  constexpr int kReads = FM + kBReads * FN;
  constexpr int kMfma = FM * FN * (ES == 4 ? 4 : 1);
  constexpr int kPairs = kReads < kMfma ? kReads : kMfma;
  // The 32x32x16 tile runs four 16-wide k steps per slice the same way:
  // step s+1's reads alternate with step s's MFMAs.
  auto compute = [&](const char* S) {
    u32x4 fa[kSteps][FM], fb[kSteps][FN];
#pragma unroll
    for (int c = 0; c < kSteps; ++c) load_frags(S, c, fa[c], fb[c]);
#pragma unroll
    for (int c = 0; c < kSteps; ++c) mma_all(fa[c], fb[c]);
    __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // step 0 reads
#pragma unroll
    for (int c = 0; c + 1 < kSteps; ++c) {
#pragma unroll
      for (int q = 0; q < kPairs; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one read of step c+1
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA of step c
      }
      if constexpr (kMfma > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kPairs, 0);
      if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPairs, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);  // the last step's MFMAs
  };

  // ---- main loop ------------------------------------------------------------------
  // Steps whose prefetch is known to exist run unconditionally with their
  // stages named at compile time; the first and last steps are generic.
  if (nk > 0) {
    if constexpr (STAGES == 2) {
      issue(s0, 0);
      wait_vm<0>();
      fix(s0, 0);
      lds_barrier();
      auto step = [&](char* cur, char* nxt, int64_t t) {
        if (t < nk) {
          if (t + 1 < nk) issue(nxt, t + 1);
          compute(cur);
          wait_vm<0>();
          if (t + 1 < nk) fix(nxt, t + 1);
          lds_barrier();
        }
      };
      step(s0, s1, 0);
      int64_t kt = 1;
      for (; kt + 3 <= nk; kt += 2) {  // slices kt (s1) and kt+1 (s0)
        issue(s0, kt + 1);             // kt+1 <= nk-2: never the partial slice
        compute(s1);
        wait_vm<0>();
        lds_barrier();
        issue(s1, kt + 2);             // kt+2 may be the partial last slice
        compute(s0);
        wait_vm<0>();
        fix(s1, kt + 2);
        lds_barrier();
      }
      step(s1, s0, kt);
      step(s0, s1, kt + 1);
    } else {
      issue(s0, 0);
      if (nk > 1) {
        issue(s1, 1);
        wait_vm<kPer>();
      } else {
        wait_vm<0>();
      }
      fix(s0, 0);
      lds_barrier();
      auto step = [&](char* cur, char* nxt, char* pre, int64_t t) {
        if (t < nk) {
          if (t + 2 < nk) issue(pre, t + 2);
          compute(cur);
          if (t + 2 < nk)
            wait_vm<kPer>();
          else
            wait_vm<0>();
          if (t + 1 < nk) fix(nxt, t + 1);
          lds_barrier();
        }
      };
      step(s0, s1, s2, 0);
      int64_t kt = 1;
      // Slices kt (s1), kt+1 (s2), kt+2 (s0). The slices waited for here
      // (kt+1..kt+3 <= nk-2) are never the partial one; kt+4 may be, and the
      // step that waits for it (t = kt+3, below or in the next trip) zeroes it.
      for (; kt + 5 <= nk; kt += 3) {
        issue(s0, kt + 2);
        compute(s1);
        wait_vm<kPer>();
        lds_barrier();
        issue(s1, kt + 3);
        compute(s2);
        wait_vm<kPer>();
        lds_barrier();
        issue(s2, kt + 4);
        compute(s0);
        wait_vm<kPer>();
        lds_barrier();
      }
      step(s1, s2, s0, kt);
      step(s2, s0, s1, kt + 1);
      step(s0, s1, s2, kt + 2);
      step(s1, s2, s0, kt + 3);
    }
  }

  // ---- partial segments: publish; the tile's last program sums them -------
  if (!(kb == 0 && ke == nk_all)) {
    // Partials move through agent-scope (sc1) stores and loads, which are
    // coherent across XCDs without writing back or invalidating whole L2s;
    // the only ordering needed is that every lane's stores have completed
    // (vmcnt(0), then the workgroup barrier) before the ticket is taken.
    // Program q keeps two partial slots: 2q for its first segment, 2q + 1
    // for its last (middle segments are whole tiles). Part p (16 bytes) of
    // fragment (i, j) of lane tid is at (((i*FN + j)*kParts + p)*NT + tid)*16
    // of a slot; a fragment is one part (16x16) or four (32x32).
    constexpr int kTileFloats = BM * BN;
    constexpr int kParts = static_cast<int>(sizeof(AccT)) / 16;
    const int64_t st = tile - full;  // index among the split tiles
    auto slot = [&](int64_t q, bool first) {
      return tile_rsrc(args.ws + (2 * q + (first ? 0 : 1)) * kTileFloats, kTileFloats * 4);
    };
    const __amdgpu_buffer_rsrc_t mine = slot(prog, st * nk_all + kb == it_first);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int pp = 0; pp < kParts; ++pp) {
          const f32x4 part = {acc[i][j][4 * pp], acc[i][j][4 * pp + 1], acc[i][j][4 * pp + 2],
                              acc[i][j][4 * pp + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, part), mine,
                                                 (((i * FN + j) * kParts + pp) * NT + tid) * 16, 0,
                                                 kCachePolicySc1);
        }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    wait_vm<0>();  // this lane's partial stores are done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // The K loop ended on a barrier, so the stage buffers are free: the
    // ticket is broadcast through the first word of LDS, and every wave has
    // read it before any starts the next segment's DMA.
    unsigned* const ticket = reinterpret_cast<unsigned*>(lds);
    __syncthreads();
    if (tid == 0)
      *ticket = __hip_atomic_fetch_add(&args.tickets[st], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const unsigned arrived = *ticket;
    __syncthreads();
    const int64_t q0 = owner(st * nk_all);
    const int64_t q1 = owner((st + 1) * nk_all - 1);
    if (arrived != static_cast<unsigned>(q1 - q0)) continue;
    // Last of the tile's programs: add the segments in ascending k.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = AccT{};
    for (int64_t q = q0; q <= q1; ++q) {
      const __amdgpu_buffer_rsrc_t src = slot(q, (q * I / P) / nk_all == st);
      // A segment's loads are in flight together before the first add: all of
      // them for 16x16 fragments, one fragment row at a time for 32x32 ones
      // (all at once would need another 128 registers per lane).
      constexpr int kRowsInFlight = kParts == 1 ? FM : 1;
#pragma unroll
      for (int i0 = 0; i0 < FM; i0 += kRowsInFlight) {
        u32x4 pv[kRowsInFlight][FN][kParts];
#pragma unroll
        for (int di = 0; di < kRowsInFlight; ++di)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int pp = 0; pp < kParts; ++pp)
              pv[di][j][pp] = __builtin_amdgcn_raw_buffer_load_b128(
                  src, ((((i0 + di) * FN + j) * kParts + pp) * NT + tid) * 16, 0, kCachePolicySc1);
#pragma unroll
        for (int di = 0; di < kRowsInFlight; ++di)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int pp = 0; pp < kParts; ++pp) {
              const f32x4 part = __builtin_bit_cast(f32x4, pv[di][j][pp]);
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[i0 + di][j][4 * pp + e] += part[e];
            }
      }
    }
    if (tid == 0) __hip_atomic_store(&args.tickets[st], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- epilogue -------------------------------------------------------------
  // Opaque copies of the tile origin: no epilogue address can be computed
  // ahead of the K loop, where it would hold registers for the whole loop.
  int64_t em0 = m0, en0 = n0;
  // The lane's column in a fragment and its row group: accumulator element e
  // is fragment row 4*eg + e (16x16) or 8*(e/4) + 4*eg + e%4 (32x32).
  int eli = fr, eg = MF == 32 ? (lane >> 5) : g, etid = tid;
  constexpr int kAccN = MF == 32 ? 16 : 4;
  auto frag_row = [&](int e) { return MF == 32 ? 8 * (e >> 2) + 4 * eg + (e & 3) : 4 * eg + e; };
  asm volatile("" : "+s"(em0), "+s"(en0), "+v"(eli), "+v"(eg), "+v"(etid));
  T* __restrict__ C = static_cast<T*>(args.C);
  const T* __restrict__ bias = static_cast<const T*>(args.bias);
  const bool gelu = args.epilogue == KF_EPILOGUE_BIAS_GELU;
  // A row-contiguous C with 16-byte aligned rows is staged through LDS (the
  // stage buffers are free after the K loop) and written as 16-byte row
  // pieces: 8 stores per lane for a 256x128 tile instead of 64 two-byte
  // ones, whose per-lane addressing held the tile's last round back
  // (4096x11008x4096: 387 -> 354 us). Other layouts store element by element.
  // The row pieces are stored with the non-temporal policy: C is written once
  // and not read back by this launch. Measured against plain stores, same
  // outputs (flushed event medians): 2048x4096x4096 at 256x128 68.8 against
  // 70.6 us, 4096x11008x4096 unsplit 360.7 against 371.4 us, 2048x11008x4096
  // 187.8 against 190.9 us; level at 128x256 on 2048x4096x4096.
  constexpr int kPitch = BN + V;  // elements per LDS row of the staged C: 16 bytes of padding
  constexpr bool kCFits = BM * kPitch * ES <= Tl::kLdsBytes;
  const bool stage_c = kCFits && args.ldc_n == 1 && (args.ldc_m * ES) % 16 == 0 &&
                       (reinterpret_cast<uintptr_t>(C) & 15u) == 0;
  if (stage_c) {
    T* const ct = reinterpret_cast<T*>(lds);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int cl = wn * Tl::TN + j * MF + eli;
      const int64_t col = en0 + cl;
      const float bcol = (gelu && col < N) ? to_f32(bias[col]) : 0.f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < kAccN; ++r) {
          float v = acc[i][j][r];
          if (gelu) v = gelu_tanh(v + bcol);
          ct[(wm * Tl::TM + i * MF + frag_row(r)) * kPitch + cl] = from_f32<T>(v);
        }
    }
    __syncthreads();
    constexpr int kRowChunks = BN / V;
    for (int idx = etid; idx < BM * kRowChunks; idx += NT) {
      const int rl = idx / kRowChunks, cl = (idx % kRowChunks) * V;
      const int64_t row = em0 + rl, col = en0 + cl;
      if (row >= M || col >= N) continue;
      const T* src = ct + rl * kPitch + cl;
      T* dst = C + row * args.ldc_m + col;
      if (col + V <= N) {
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(src), reinterpret_cast<u32x4*>(dst));
      } else {
        for (int e = 0; e < V && col + e < N; ++e) dst[e] = src[e];
      }
    }
    __syncthreads();  // the next segment's DMA reuses the stage buffers
    continue;
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = en0 + wn * Tl::TN + j * MF + eli;
    if (col >= N) continue;
    const float bcol = gelu ? to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < kAccN; ++r) {
        const int64_t row = em0 + wm * Tl::TM + i * MF + frag_row(r);
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (gelu) v = gelu_tanh(v + bcol);
        C[row * args.ldc_m + col * args.ldc_n] = from_f32<T>(v);
      }
    }
  }
  }  // segments
}

}  // namespace gemm
}  // namespace kf
