// GEMV entry kernels: y[M] = A[M x K] . x[K], bf16 or fp16 storage, FP32
// accumulation (reference: gemv_kernel.hpp:21-63, entries
// level_zero/gem_spv_entry.cpp:11-27 with argument order (A, x, y, m, k)).
//
// Launch: 256 threads (4 wavefronts, fixed at compile time); dynamic LDS = round_up(K, 512) * 2
// bytes for the staged vector; the grid walks tiles of 4*R rows with a
// grid-stride loop so each block stages the vector once. Any M, K >= 1 and
// any leading dimension lda >= K are accepted; the _vec variants need A, x
// 16-byte aligned and K, lda multiples of 8 (the host checks), the others
// use 16-bit loads. The _vecg variants read the vector from global memory
// when it does not fit in LDS.
#include "gemv_core.hpp"

namespace xpu {

// XG: read the vector from global memory (cached loads) instead of LDS, for
// vectors longer than the LDS holds; needs the _vec alignment conditions.
template <int DT, int R, int U, bool VEC, bool XG = false>
XPU_DEVICE void gemv_entry(const uint16_t *__restrict__ A, const uint16_t *__restrict__ x,
                           uint16_t *__restrict__ y, uint32_t M, uint32_t K, uint64_t lda) {
  extern __shared__ __align__(16) uint16_t lds_x[];
  const uint16_t *xs = x;
  constexpr uint32_t kBlock = 256;  // launched with 256 threads (gemv_api.cpp)
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t rows_per_block = (kBlock >> 6) * R;
  if constexpr (!XG) {
    const uint32_t kpad = (K + 511u) & ~511u;
    stage_vector<VEC, kBlock>(lds_x, x, K, kpad);
    __syncthreads();
    xs = lds_x;
  }
  for (uint32_t base = blockIdx.x * rows_per_block; base < M; base += gridDim.x * rows_per_block) {
    const uint32_t row0 = base + wave * R;
    if (row0 >= M) continue;
    float out[R];
    gemv_rows<DT, R, U, VEC>(A, lda, K, M, xs, row0, out);
    const uint32_t lane = lane_id();
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (lane == static_cast<uint32_t>(r) && row0 + r < M)
        y[row0 + r] = static_cast<uint16_t>(encode<DT>(out[r]));
  }
}

}  // namespace xpu

#define XPU_GEMV_VARIANT(NAME, DT, R, U, VEC, XG)                                          \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                  \
      const uint16_t *__restrict__ A, const uint16_t *__restrict__ x,                      \
      uint16_t *__restrict__ y, uint32_t M, uint32_t K, uint64_t lda) {                    \
    XPU_STAMP(xpu::kStampGemv);                                                            \
    xpu::gemv_entry<DT, R, U, VEC, XG>(A, x, y, M, K, lda);                                \
  }

// name: xpu_gemv_<type>_r<R>u<U>_<vec|any|vecg>; R rows per wavefront, U
// 512-column chunks per pipelined load batch
#define XPU_GEMV_TYPES(R, U)                                                         \
  XPU_GEMV_VARIANT(xpu_gemv_bf16_r##R##u##U##_vec, xpu::kBf16, R, U, true, false)   \
  XPU_GEMV_VARIANT(xpu_gemv_fp16_r##R##u##U##_vec, xpu::kFp16, R, U, true, false)

XPU_GEMV_TYPES(1, 4)
XPU_GEMV_TYPES(2, 2)
XPU_GEMV_VARIANT(xpu_gemv_bf16_r1u2_any, xpu::kBf16, 1, 2, false, false)
XPU_GEMV_VARIANT(xpu_gemv_fp16_r1u2_any, xpu::kFp16, 1, 2, false, false)
XPU_GEMV_VARIANT(xpu_gemv_bf16_r1u8_vecg, xpu::kBf16, 1, 8, true, true)
XPU_GEMV_VARIANT(xpu_gemv_fp16_r1u8_vecg, xpu::kFp16, 1, 8, true, true)
