// GEMM C[M x N] = A[M x K] . B[K x N] on gfx950 MFMA, bf16 or fp16 storage,
// FP32 accumulation (reference: gemm_kernel.hpp:25-143 with argument order
// (a, b, c, m, n, k), level_zero/gem_spv_entry.cpp:28-60).
//
// Block tile 256 x 256 x 64 with 256 threads: four wavefronts in a 2 x 2
// arrangement, each owning 128 x 128 of C as 4 x 4 tiles of
// v_mfma_f32_32x32x16_{bf16,f16} (256 FP32 accumulators per lane).
// A and B tiles are staged through LDS, double buffered: while the MFMAs
// consume one buffer the next K-slice is in flight from global memory and is
// written to the other buffer afterwards (one barrier per K-slice). A is
// stored row-major [m][k]; B is transposed in registers (8 x 8 blocks of
// 16-bit values via v_perm_b32) and stored [n][k], so both MFMA operands
// are single 16-byte LDS reads. Rows are padded by 8 elements so the 32 rows
// read by one ds_read_b128 fall in distinct banks.
//
// Any M, N, K >= 1: out-of-range rows, columns and K are zero-filled on load
// and masked on store (the reference pads on the host instead, gemm.cpp:75-85).
// The _vec variants need A, B 16-byte aligned and K, N multiples of 8; the
// _any variants load 16-bit elements.
//
// Tile order: blocks are dealt round-robin to the 8 XCDs, so when the tile
// count is a multiple of 8 block b is renumbered to a contiguous range per
// XCD; tiles are then walked in groups of 4 tile-rows so the blocks of one
// XCD share A and B panels in that XCD's L2 (the reference snakes the
// tile order, gemm_kernel.hpp:79-83, for its L3).
#include "device_common.hpp"

namespace xpu {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kBM = 256, kBN = 256, kBK = 64;
constexpr uint32_t kLdsPitch = kBK + 8;  // elements per staged row
constexpr uint32_t kTileElems = kBM * kLdsPitch;

template <int DT>
XPU_DEVICE f32x16 mfma(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
  if constexpr (DT == kFp16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 8 consecutive elements of a row starting at column col (< cols), zero
// beyond cols; VEC loads them as one 16-byte access.
template <bool VEC>
XPU_DEVICE u32x4 load8(const uint16_t *__restrict__ row, uint32_t col, uint32_t cols, bool row_ok) {
  if (!row_ok || col >= cols) return u32x4{0, 0, 0, 0};
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4 *>(row + col);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = (col + e < cols) ? row[col + e] : 0u;
    return u32x4{w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16), w[6] | (w[7] << 16)};
  }
}

struct TileCoord {
  uint32_t tm, tn;
};

XPU_DEVICE TileCoord tile_of_block(uint32_t b, uint32_t tiles_m, uint32_t tiles_n) {
  const uint32_t total = tiles_m * tiles_n;
  uint32_t logical = b;
  if (total % 8u == 0) logical = (b % 8u) * (total / 8u) + b / 8u;
  constexpr uint32_t kGroup = 4;
  const uint32_t per_group = kGroup * tiles_n;
  const uint32_t group = logical / per_group;
  const uint32_t first_m = group * kGroup;
  const uint32_t rows = min(kGroup, tiles_m - first_m);
  const uint32_t in_group = logical % per_group;
  return {first_m + in_group % rows, in_group / rows};
}

template <int DT, bool VEC>
XPU_DEVICE void gemm_body(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                          uint16_t *__restrict__ C, uint32_t M, uint32_t N, uint32_t K) {
  __shared__ __align__(16) uint16_t lds[2][2][kTileElems];  // [buffer][A | Bt][...]
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const TileCoord tc = tile_of_block(blockIdx.x, tiles_m, tiles_n);
  const uint32_t m0 = tc.tm * kBM, n0 = tc.tn * kBN;

  // global -> register assignment
  // A: thread loads chunk (tid % 8) of rows tid/8 + 32 i, i = 0..7
  const uint32_t a_chunk = tid & 7u, a_row = tid >> 3;
  // B: thread loads an 8 x 8 block: k rows kb*8..+7, n columns nb*8..+7
  const uint32_t b_nb = tid & 31u, b_kb = tid >> 5;

  u32x4 ra[8], rb[8];
  auto load_tiles = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t row = m0 + a_row + 32u * i;
      ra[i] = load8<VEC>(A + static_cast<uint64_t>(min(row, M - 1)) * K, k0 + a_chunk * 8u, K, row < M);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t k = k0 + b_kb * 8u + i;
      rb[i] = load8<VEC>(B + static_cast<uint64_t>(min(k, K - 1)) * N, n0 + b_nb * 8u, N, k < K);
    }
  };
  auto store_tiles = [&](uint32_t buf) {
    uint16_t *la = lds[buf][0];
    uint16_t *lb = lds[buf][1];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<u32x4 *>(la + (a_row + 32u * i) * kLdsPitch + a_chunk * 8u) = ra[i];
    // transpose the 8 x 8 block: column j of rb -> row n = nb*8 + j of Bt
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo = rb[2 * q][j >> 1], hi = rb[2 * q + 1][j >> 1];
        w[q] = __builtin_amdgcn_perm(hi, lo, sel);
      }
      *reinterpret_cast<u32x4 *>(lb + (b_nb * 8u + j) * kLdsPitch + b_kb * 8u) = u32x4{w[0], w[1], w[2], w[3]};
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const uint32_t wm = wave >> 1, wn = wave & 1u;
  const uint32_t frag_row = lane & 31u, frag_k = (lane >> 5) * 8u;
  const uint32_t nk = (K + kBK - 1) / kBK;

  load_tiles(0);
  store_tiles(0);
  __syncthreads();
  for (uint32_t it = 0; it < nk; ++it) {
    const uint32_t buf = it & 1u;
    if (it + 1 < nk) load_tiles((it + 1) * kBK);
    const uint16_t *la = lds[buf][0] + (wm * 128u + frag_row) * kLdsPitch + frag_k;
    const uint16_t *lb = lds[buf][1] + (wn * 128u + frag_row) * kLdsPitch + frag_k;
#pragma unroll
    for (uint32_t kk = 0; kk < kBK; kk += 16u) {
      u32x4 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = *reinterpret_cast<const u32x4 *>(la + i * 32u * kLdsPitch + kk);
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const u32x4 *>(lb + j * 32u * kLdsPitch + kk);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma<DT>(fa[i], fb[j], acc[i][j]);
    }
    if (it + 1 < nk) store_tiles(buf ^ 1u);
    __syncthreads();
  }

  // D layout of v_mfma_f32_32x32x16: lane l holds column l % 32 and rows
  // 8 (v / 4) + 4 (l / 32) + v % 4 for v = 0..15
  const uint32_t col_in = lane & 31u, row_in = (lane >> 5) * 4u;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t col = n0 + wn * 128u + j * 32u + col_in;
      if (col >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t row = m0 + wm * 128u + i * 32u + (v / 4) * 8u + row_in + (v % 4);
        if (row < M) C[static_cast<uint64_t>(row) * N + col] = static_cast<uint16_t>(encode<DT>(acc[i][j][v]));
      }
    }
}

}  // namespace xpu

#define XPU_GEMM_VARIANT(NAME, DT, VEC)                                                        \
  extern "C" __global__ __launch_bounds__(256, 1) void NAME(                                  \
      const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, uint16_t *__restrict__ C, \
      uint32_t M, uint32_t N, uint32_t K) {                                                    \
    xpu::gemm_body<DT, VEC>(A, B, C, M, N, K);                                                 \
  }

XPU_GEMM_VARIANT(xpu_gemm_bf16_vec, xpu::kBf16, true)
XPU_GEMM_VARIANT(xpu_gemm_fp16_vec, xpu::kFp16, true)
XPU_GEMM_VARIANT(xpu_gemm_bf16_any, xpu::kBf16, false)
XPU_GEMM_VARIANT(xpu_gemm_fp16_any, xpu::kFp16, false)
