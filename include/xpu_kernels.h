/*
 * xpu_kernels.h - C-ABI entry points of the GEMV / GEMM hot path on gfx950.
 *
 * Kernel ABI kept from the reference (row-major, contiguous unless an lda is
 * given, element type bf16 or fp16 as raw 16-bit codes, FP32 accumulation):
 *   GEMV (A, x, y, m, k)      gemv_kernel.hpp:21-26, level_zero/gem_spv_entry.cpp:11-27,
 *                             level_zero/peak_l0.cpp:840-842
 *   GEMM (a, b, c, m, n, k)   gemm_kernel.hpp:28-33, level_zero/gem_spv_entry.cpp:28-60,
 *                             level_zero/peak_l0.cpp:920-922
 * Unlike the reference (gemv.cpp:79-80, gemm.cpp:75-85 pad on the host), any
 * M, N, K >= 1 is handled inside the kernels; no padding is needed.
 *
 * All launches are asynchronous on the runtime's stream; rt may be NULL for
 * none of these functions. Return 0 on success, an XPU_ERR_* code otherwise
 * (xpu_last_error() has the message).
 */
#ifndef XPU_KERNELS_H
#define XPU_KERNELS_H

#include "xpu_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

#define XPU_DTYPE_BF16 0
#define XPU_DTYPE_FP16 1

/* y[M] = A[M x K] . x[K]; lda >= K is the row pitch in elements (K for a
 * packed matrix). Replaces gemv::Kernel<T> (gemv_kernel.hpp:21-63) launched
 * by gemv.cpp:105-108 / peak_l0.cpp:849-856. Each y[r] is the canonical-order
 * FP32 sum rounded to the storage type. */
int xpu_gemv(xpu_runtime *rt, int dtype, const void *A, const void *x, void *y,
             uint32_t M, uint32_t K, uint64_t lda);

/* C[M x N] = A[M x K] . B[K x N], row-major, FP32 accumulation on MFMA.
 * Replaces gemm::Kernel<T, Large> (gemm_kernel.hpp:25-143) launched by
 * gemm.cpp:98-101 / peak_l0.cpp:929-934, and the choice between its large
 * and small tile (gemm.cpp:145): the block tile (256x256, 224x256, 128x256
 * or 128x128) is the one with the least estimated time at this shape on this
 * GPU's compute units (xpu_gemm_tile). Any M, N, K and 2-byte aligned
 * pointers: the operands are read in place (the reference pads them on the
 * host, gemm.cpp:75-85). Outputs that leave most compute units idle even
 * with 128 x 128 tiles, with 8 or more 64-deep K-slices, split K over the
 * idle units (FP32 partials in the runtime's workspace, added in split
 * order). Asynchronous on the runtime's stream. */
int xpu_gemm(xpu_runtime *rt, int dtype, const void *A, const void *B, void *C,
             uint32_t M, uint32_t N, uint32_t K);

/* The block tile xpu_gemm uses for an M x N output on this runtime's GPU:
 * *rows x *cols. No device work. The reference's counterpart is the
 * large_tile expression of gemm.cpp:145. */
int xpu_gemm_tile(const xpu_runtime *rt, uint32_t M, uint32_t N, uint32_t *rows, uint32_t *cols);

/* Size of the scratch array behind xpu_gemm_noalloc: 16 MiB per GPU. */
#define XPU_GEMM_NOALLOC_SCRATCH_BYTES (16ull << 20)

/* xpu_gemm without allocation. No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same kernels and results
 * as xpu_gemm, bit for bit. Where xpu_gemm splits K (outputs that leave most
 * compute units idle, with 8 or more 64-deep K-slices), its FP32 partials
 * (splits x M x round_up(N, 4) x 4 bytes) go into a fixed device array of
 * XPU_GEMM_NOALLOC_SCRATCH_BYTES per GPU, set up when the first runtime on
 * that GPU is created and held until the process ends, instead of the
 * runtime's workspace; other shapes use no scratch. Needs above the array
 * fail with XPU_ERR_INVALID before any launch. Calls no hipMalloc/hipFree.
 * All calls on one GPU share the array: calls that overlap on one GPU (other
 * streams or runtimes) race. */
int xpu_gemm_noalloc(xpu_runtime *rt, int dtype, const void *A, const void *B, void *C,
                     uint32_t M, uint32_t N, uint32_t K);

/* Seeded U[-1,1) synthetic data written on the device: element i is
 * encode(dtype, (2u - 2^24) / 2^24) with u the top 24 bits of
 * splitmix64(splitmix64(seed) + (i + 1) * 0x9e3779b97f4a7c15). The same
 * values the CPU oracle's generator produces. */
int xpu_fill_uniform(xpu_runtime *rt, int dtype, void *dst, uint64_t count, uint64_t seed);

/* The reference's hash initialisation (gemv.cpp:91-103) on the device: the
 * matrix (m rows, pitch ld) and the vector (k entries). */
int xpu_fill_reference_gemv(xpu_runtime *rt, int dtype, void *matrix, void *vector,
                            uint32_t m, uint32_t k, uint32_t ld);

/* Command-line programs with the reference's flags and output lines:
 * run_gemv: gemv.cpp:157-170 (--size N | --m M --k K, --type bf16|fp16,
 *           --iterations N (50), --warmups N (5); default 16384 x 16384 bf16)
 * run_gemm: gemm.cpp:135-155 (--size N | --m M --n N --k K, --type,
 *           --iterations N (20), --warmups N (5); default 4096^3 bf16)
 * Both return 0 after "Verification: PASS", 1 on any error, a failed
 * verification included ("Error: GEMV verification failed" /
 * "Error: GEMM verification failed: ..." on stderr, as gemv.cpp:135-136,
 * gemm.cpp:117-123 throw into the catch of run_gemv / run_gemm). */
int run_gemv(int argc, char **argv);
int run_gemm(int argc, char **argv);

/* Peak-rate microbenchmarks, the measured ceilings of the rooflines.
 * xpu_peak_mfma: `blocks` x 256 threads, each wavefront running `rounds`
 * batches of 8 independent v_mfma_f32_32x32x16_bf16 on the 8 bf16 codes at
 * `operand` (replaces peak_compute_dpas_kernel.cpp:10-68); sink receives one
 * float per thread (28 + 32 * rounds for operands of 0.5) and clock four
 * uint64 (shader clock and constant-rate clock before / after the loop of
 * block 0). xpu_peak_read: streaming 16-byte reads of `bytes` (replaces
 * peak_mem_2d_kernel.cpp:13-52); sink needs blocks * 1024 bytes. */
int xpu_peak_mfma(xpu_runtime *rt, const void *operand, void *sink, void *clock, uint32_t blocks,
                  uint32_t rounds);
int xpu_peak_read(xpu_runtime *rt, const void *input, uint64_t bytes, void *sink, uint32_t blocks);

/* run_peak_compute: peak_compute_dpas.cpp (--waves-per-simd N (2),
 *   --rounds N (8192), --iterations N (100)); prints median / best TFLOP/s
 *   against 2500 TFLOP/s, the shader clock during the loop, checksum.
 * run_peak_mem: peak_mem_2d.cpp (--size-mib N (4096), --iterations N (100));
 *   prints median / best read GB/s against 8000 GB/s.
 * 0 on success, 1 on error. */
int run_peak_compute(int argc, char **argv);
int run_peak_mem(int argc, char **argv);


#ifdef __cplusplus
}
#endif
#endif
