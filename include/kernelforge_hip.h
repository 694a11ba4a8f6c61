/*
 * kernelforge C-ABI: the drop-in device boundary for KernelForge's tunable
 * kernel set, rebuilt as hand-written HIP kernels for gfx950 (MI355X).
 *
 * In the reference every kernel is launched from Python with raw pointers,
 * dimensions, strides and compile-time tile parameters:
 *   matmul_kernel[grid](a, b, c, M, N, K, strides..., BLOCK_*, GROUP_M,
 *                       num_warps, num_stages)   kernelforge/kernels/matmul.py:132-155
 *   fused_linear_gelu_kernel[grid](...)           kernelforge/kernels/fused_linear.py:112-157
 *   softmax_kernel[grid](...)                     kernelforge/kernels/softmax.py:70-104
 *   rmsnorm_kernel[grid](...)                     kernelforge/kernels/rmsnorm.py:81-127
 *   rmsnorm_forward_cuda(x, gamma, eps)           kernelforge/csrc/rmsnorm.cu:19-57
 * These entry points take exactly that information, plus the HIP stream the
 * launch is enqueued on (torch's current stream; the reference launches on
 * the current CUDA stream, csrc/rmsnorm.cu:41).
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers; strides are in elements, not bytes.
 *   - Nothing is allocated or freed; outputs are caller-owned.
 *   - Launches are asynchronous on `stream`; nothing synchronises.
 *   - A zero-sized problem returns KF_OK without launching
 *     (csrc/rmsnorm.cu:27-29).
 *   - The return value is KF_OK or a negative KF_ERR_* code; the message for
 *     the last failure on the calling thread is kf_last_error().
 */
#ifndef KERNELFORGE_HIP_H_
#define KERNELFORGE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. Double is refused, as in csrc/rmsnorm.cpp:23-30. */
enum {
  KF_DTYPE_F32 = 0,
  KF_DTYPE_F16 = 1,
  KF_DTYPE_BF16 = 2
};

/* Status codes. The Python loader maps them onto exception classes whose
 * names drive the tuner's failure classification (kernelforge/tuning/tuner.py:60-71). */
enum {
  KF_OK = 0,
  KF_ERR_INVALID_ARGUMENT = -1, /* bad shape, stride, pointer or parameter   */
  KF_ERR_NOT_BUILT = -2,        /* no instantiation for this tile config      */
  KF_ERR_OUT_OF_RESOURCES = -3, /* config exceeds LDS / register / block caps */
  KF_ERR_LAUNCH = -4,           /* the HIP runtime rejected the launch        */
  KF_ERR_UNSUPPORTED_DTYPE = -5,
  KF_ERR_WORKSPACE = -6,        /* caller workspace missing or too small      */
  KF_ERR_OUT_OF_MEMORY = -7     /* hipErrorOutOfMemory from the runtime       */
};

/* GEMM main-loop pipelines. */
enum {
  KF_PIPELINE_STAGED = 0, /* global -> VGPR -> LDS (padded rows), any layout      */
  KF_PIPELINE_DIRECT = 1  /* global -> LDS DMA (swizzled rows), 16-bit aligned
                             operands with K (and N for row-major B) % 8 == 0;
                             other layouts fall back to the staged twin tile   */
};

/* GEMM epilogues. */
enum {
  KF_EPILOGUE_NONE = 0,      /* C = A @ B                                     */
  KF_EPILOGUE_BIAS_GELU = 1  /* C = gelu_tanh(A @ B + bias), fused_linear.py:94-104 */
};

/*
 * Split-K workspaces (kf_gemv, kf_gemm_split_k) are laid out the same way
 * for every shape: KF_WORKSPACE_COUNTER_BYTES of 32-bit arrival counters,
 * one per output block (at most KF_WORKSPACE_COUNTERS blocks), then the fp32
 * partial sums. The counters must be zero before a workspace's first use and
 * every completed call leaves them zero; because their region never moves,
 * partial sums of one call can never land where a later call expects a zero
 * counter, so one workspace can serve any sequence of calls on one stream.
 */
enum {
  KF_WORKSPACE_COUNTERS = 1 << 18,
  KF_WORKSPACE_COUNTER_BYTES = 4 << 18
};

/* Library identification: ABI version and the offload target it was built for. */
int kf_abi_version(void);
const char* kf_build_target(void);
/* First 16 hex digits of SHA-256 over the sources, tile lists and flags the
 * library was built from (kernelforge/build.py source_digest): profiles and
 * measurements record it to name the code they ran. No counterpart in the
 * reference (Triton compiles from the Python source it ships). */
const char* kf_source_digest(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* kf_last_error(void);

/* The id of the graph capture `stream` is in (0 when it is not capturing),
 * from hipStreamGetCaptureInfo. Support for callers that keep split-K
 * workspaces per capture; no counterpart in the reference (Triton launches are
 * never captured there). */
int kf_stream_capture_id(void* stream, unsigned long long* id);

/*
 * Tiled MFMA GEMM, optionally with the fused bias + tanh-GELU epilogue.
 * Replaces matmul() (kernels/matmul.py:132-155) and fused_linear_gelu()
 * (kernels/fused_linear.py:112-157).
 *
 *   C[M,N] = A[M,K] @ B[K,N]                    (epilogue KF_EPILOGUE_NONE)
 *   C[M,N] = gelu_tanh(A @ B + bias[N])         (epilogue KF_EPILOGUE_BIAS_GELU)
 *
 * fp32 accumulation; C is written in the input dtype. Any strides are
 * accepted (e.g. nn.Linear weight.t()), as in the reference; 16-byte vector
 * loads are used where pointers and strides allow them, scalar loads
 * otherwise. Tile parameters select one ahead-of-time instantiation:
 *   block_m, block_n, block_k : macro tile
 *   waves                     : wavefronts (64 lanes) per workgroup
 *   stages                    : LDS buffers (2 = double buffered)
 *   group_m                   : rows of tiles per launch-order group
 *   pipeline                  : KF_PIPELINE_STAGED or KF_PIPELINE_DIRECT
 * Returns KF_ERR_NOT_BUILT for a tile config that was not instantiated.
 */
int kf_gemm(int dtype, const void* A, const void* B, const void* bias, void* C,
            int64_t M, int64_t N, int64_t K,
            int64_t lda_m, int64_t lda_k, int64_t ldb_k, int64_t ldb_n,
            int64_t ldc_m, int64_t ldc_n, int epilogue,
            int block_m, int block_n, int block_k, int waves, int stages, int group_m,
            int pipeline, void* stream);

/*
 * kf_gemm with the K dimension split over `split_k` (1..64) programs per
 * output tile, for shapes whose tile count leaves CUs idle: few rows (e.g.
 * M = 16..128 of a prefill or batched decode), or a last round of tiles that
 * fills only part of the GPU. When there are at least as many tiles as
 * workgroups the device runs at once (kf_gemm_concurrent_tiles), only the
 * tiles of the last, partial round are split (none when every round is
 * full). The reference has no split-K
 * GEMM: it launches matmul_kernel (kernels/matmul.py:132-155) with one
 * program per tile at every M, and this is that call with the K loop shared
 * out. Runs on the direct pipeline (pipeline argument implied); a layout the
 * direct pipeline cannot take runs unsplit on the register-staged fallback,
 * as kf_gemm does. Each program adds its k-range in fp32 and publishes the
 * partial tile to `workspace`; the last of a tile's programs to arrive sums
 * the partials in ascending order, so results are deterministic. The
 * workspace (kf_gemm_workspace_bytes, 16-byte aligned, laid out as described
 * at KF_WORKSPACE_COUNTERS: one counter per tile) may be shared with kf_gemv;
 * launches sharing a workspace must not overlap.
 */
int kf_gemm_split_k(int dtype, const void* A, const void* B, const void* bias, void* C,
                    int64_t M, int64_t N, int64_t K,
                    int64_t lda_m, int64_t lda_k, int64_t ldb_k, int64_t ldb_n,
                    int64_t ldc_m, int64_t ldc_n, int epilogue,
                    int block_m, int block_n, int block_k, int waves, int stages, int group_m,
                    int split_k, void* workspace, size_t workspace_bytes, void* stream);
/* Workgroups of one GEMM variant the current device runs at once (CUs x the
 * workgroups a CU holds by LDS, wave slots and registers): one round, the
 * size that decides which tiles kf_gemm_split_k splits. A negative KF_ERR_*
 * code on failure. No counterpart in the reference (Triton sizes nothing). */
int64_t kf_gemm_concurrent_tiles(int dtype, int block_m, int block_n, int block_k, int waves,
                                 int stages, int pipeline);
/* Workspace bytes kf_gemm_split_k needs (0 when split_k <= 1). */
size_t kf_gemm_workspace_bytes(int64_t M, int64_t N, int block_m, int block_n, int split_k);

/* 1 if (dtype, tile config, pipeline) has an instantiation in this build, else 0. */
int kf_gemm_has_variant(int dtype, int block_m, int block_n, int block_k, int waves, int stages,
                        int pipeline);

/* Number of GEMM instantiations (one per tile and pipeline), and the config of
 * instantiation `index`. Returns KF_OK or an error. */
int kf_gemm_variant_count(void);
int kf_gemm_variant_info(int index, int* dtype, int* block_m, int* block_n, int* block_k,
                         int* waves, int* stages, int* pipeline);

/*
 * Split-K GEMV for decode shapes: y[M,N] = x[M,K] @ W[K,N], M <= 8.
 * The reference runs decode through the same matmul at M=1
 * (kernels/matmul.py:132-155, tuning/search.py:377-386); this is its
 * HBM-bound replacement. A workgroup of `waves` wavefronts owns a strip of
 * lanes_per_row (8, 16, 32 or 64) 16-byte vectors of columns and one of
 * `split_k` slices of K. For n-contiguous W the slices are cut on whole
 * trips (the rows a workgroup reads in one double-buffered step:
 * U*64/lanes_per_row per wave, U = 8 for one x row, 4 for two, 2 for three
 * to eight) and shared out as evenly as whole trips allow, so a split_k above
 * the number of trips leaves some slices empty. When W is k-contiguous (ldw_k == 1, e.g.
 * nn.Linear's weight passed as weight.t()) with x k-contiguous, 16-byte
 * aligned rows and K a multiple of 16 bytes' worth of elements, the
 * lanes_per_row lanes split one column's k-run instead, 64/lanes_per_row
 * columns per wave load. Partial sums over the slices are reduced
 * deterministically (fixed order) by the last workgroup of each column block,
 * using a caller-provided workspace of kf_gemv_workspace_bytes() bytes laid
 * out as described at KF_WORKSPACE_COUNTERS (one counter per column block).
 * epilogue as for kf_gemm.
 */
int kf_gemv(int dtype, const void* x, const void* W, const void* bias, void* y,
            int64_t M, int64_t N, int64_t K,
            int64_t ldx_m, int64_t ldx_k, int64_t ldw_k, int64_t ldw_n,
            int64_t ldy_m, int64_t ldy_n, int epilogue,
            int split_k, int waves, int lanes_per_row, void* workspace, size_t workspace_bytes,
            void* stream);
size_t kf_gemv_workspace_bytes(int64_t M, int64_t N, int split_k);

/* Size of the static scratch behind kf_gemv_no_alloc, per GPU: the
 * KF_WORKSPACE_COUNTER_BYTES counter region plus 15 MiB of fp32 partials, so
 * split_k * M * N <= 3,932,160 (e.g. M=8, N=11008, split_k=44). */
enum { KF_GEMV_NO_ALLOC_SCRATCH_BYTES = 16 << 20 };

/*
 * kf_gemv without a workspace argument and without allocating: no hipMalloc,
 * hipFree or allocating library call. No counterpart in the reference; it is
 * for callers that cannot allocate (code under HIP graph capture, tight
 * decode-serving loops, harnesses that forbid allocation). Same arguments,
 * kernels, results and error codes as kf_gemv; the split-K workspace is a
 * file-scope device array of KF_GEMV_NO_ALLOC_SCRATCH_BYTES that each GPU
 * holds from its first call until the process ends. A split that needs more
 * (kf_gemv_workspace_bytes(M, N, split_k) > KF_GEMV_NO_ALLOC_SCRATCH_BYTES)
 * returns KF_ERR_WORKSPACE. The first call on a device also enqueues a
 * kernel that zeroes the counters. Every call on one GPU shares its array:
 * calls that overlap on one GPU (different streams, concurrent graph
 * replays) race and must be serialised by the caller.
 */
int kf_gemv_no_alloc(int dtype, const void* x, const void* W, const void* bias, void* y,
                     int64_t M, int64_t N, int64_t K,
                     int64_t ldx_m, int64_t ldx_k, int64_t ldw_k, int64_t ldw_n,
                     int64_t ldy_m, int64_t ldy_n, int epilogue,
                     int split_k, int waves, int lanes_per_row, void* stream);

/*
 * Single-pass row softmax over the last dimension, fp32 internal.
 * Replaces softmax() (kernels/softmax.py:70-104). Rows must have unit column
 * stride. block_size (a power of two >= cols) / (waves*64) is the number of
 * elements each lane holds; rows_per_program rows are handled per workgroup.
 */
int kf_softmax(int dtype, const void* x, void* y, int64_t rows, int64_t cols,
               int64_t x_row_stride, int64_t y_row_stride,
               int block_size, int rows_per_program, int waves, void* stream);

/*
 * Single-pass RMSNorm: y = x * rsqrt(mean(x^2) + eps) * gamma, fp32 math.
 * Replaces rmsnorm() (kernels/rmsnorm.py:81-127) and rmsnorm_forward_cuda()
 * (csrc/rmsnorm.cu:19-57). Same tile parameters as kf_softmax.
 */
int kf_rmsnorm(int dtype, const void* x, const void* gamma, void* y, int64_t rows,
               int64_t cols, int64_t x_row_stride, int64_t y_row_stride, float eps,
               int block_size, int rows_per_program, int waves, void* stream);

/*
 * Two-pass RMSNorm for rows of any width: the reference's first listed future
 * improvement (README.md:656-660), which lifts the single-pass cap of
 * kf_rmsnorm. Same math, rounding and argument meaning as kf_rmsnorm except:
 *   block_size : columns per trip of the workgroup over its row, a multiple
 *                of waves*64*(16 / element size) -- 1, 2, 4 or 8 16-byte
 *                vectors per lane per trip;
 *   stage_row  : 1 keeps the row in LDS between the passes (one HBM read),
 *                which needs cols*element size <= the value
 *                kf_rmsnorm_two_pass_max_staged_cols() reports; 0 reads the
 *                row twice.
 */
int kf_rmsnorm_two_pass(int dtype, const void* x, const void* gamma, void* y, int64_t rows,
                        int64_t cols, int64_t x_row_stride, int64_t y_row_stride, float eps,
                        int block_size, int rows_per_program, int waves, int stage_row,
                        void* stream);
/* Widest row (in elements of `dtype`) that kf_rmsnorm_two_pass can stage in LDS. */
int64_t kf_rmsnorm_two_pass_max_staged_cols(int dtype);

/*
 * Elementwise c[i] = a[i] + b[i] over n contiguous elements, fp32 sum rounded
 * once. Replaces vector_add() (kernels/vector_add.py:43-57): a workgroup of
 * `waves` wavefronts owns block_size elements (block_size / (waves*64) per
 * lane, a power of two from 1 to 64).
 */
int kf_vector_add(int dtype, const void* a, const void* b, void* c, int64_t n, int block_size,
                  int waves, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KERNELFORGE_HIP_H_ */
