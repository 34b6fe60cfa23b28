// Row-major GEMV core for gfx950: one wavefront computes R rows, each lane
// streams 16-byte slices of the rows with non-temporal loads, the vector is
// read from LDS, and every row ends in the canonical reduction (lane slots
// folded 8 -> 1, then a 64-lane xor-butterfly).
//
// Reference semantics: gemv_kernel.hpp:33-60 (y = A.x, FP32 accumulation,
// result converted to the storage type). The reference's lane order
// (k mod 32) is replaced by the canonical order described in
// device_common.hpp; FP32 rounding of each product is exact for 16-bit
// inputs, so only the order of the additions differs.
#pragma once

#include "device_common.hpp"

namespace xpu {

// Copy x[0..K) into LDS zero-padded to kpad (a multiple of 512 codes).
// BLOCK: the launch's block size when fixed at compile time (0: read
// blockDim.x, a load from the dispatch packet that the first loads would
// wait for). VEC (K % 8 == 0, x 16-byte aligned): four 16-byte loads per
// thread are issued before their LDS writes (a chunk past K, or past kpad,
// reads the last chunk of x; past K it writes zeros, past kpad nothing).
template <bool VEC, uint32_t BLOCK = 0>
XPU_DEVICE void stage_vector(uint16_t *xs, const uint16_t *__restrict__ x, uint32_t K, uint32_t kpad) {
  const uint32_t threads = BLOCK ? BLOCK : blockDim.x;
  if constexpr (VEC) {
    const uint32_t step = threads * 8u;
    for (uint32_t i0 = threadIdx.x * 8u; i0 < kpad; i0 += 4u * step) {
      u32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t i = i0 + u * step;
        v[u] = *reinterpret_cast<const u32x4 *>(x + (i < K ? i : K - 8u));  // branch-free
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t i = i0 + u * step;
        if (i < kpad) *reinterpret_cast<u32x4 *>(xs + i) = i < K ? v[u] : u32x4{0, 0, 0, 0};
      }
    }
    return;
  }
  for (uint32_t i = threadIdx.x * 8u; i < kpad; i += threads * 8u) {
    u32x4 v;
    if (VEC && i + 8u <= K) {
      v = *reinterpret_cast<const u32x4 *>(x + i);
    } else {
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = (i + e < K) ? x[i + e] : 0u;
      v = u32x4{w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16),
                w[6] | (w[7] << 16)};
    }
    *reinterpret_cast<u32x4 *>(xs + i) = v;
  }
}

// 8 codes of row starting at p, columns col..col+7 of a row of length K.
template <bool VEC>
XPU_DEVICE u32x4 load_row8(const uint16_t *__restrict__ p, uint32_t col, uint32_t K) {
  if constexpr (VEC) {
    return load_nt16(p);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = (col + e < K) ? __builtin_nontemporal_load(p + e) : 0u;
    return u32x4{w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16),
                 w[6] | (w[7] << 16)};
  }
}

template <int DT, int R>
XPU_DEVICE void fma_chunk(float (&acc)[R][8], const u32x4 (&a)[R], const u32x4 &xv) {
  float xf[8];
  unpack8<DT>(xv, xf);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float af[8];
    unpack8<DT>(a[r], af);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(af[e], xf[e], acc[r][e]);
  }
}

// Canonical dot products of rows row0 .. row0+R-1 (indices clamped to M-1,
// so rows past the end re-read the last row and are discarded by the
// caller) with the LDS-staged vector xs. All lanes must be active.
// Row pointers (lane offset included) of the R rows a wavefront computes.
// PAIRED: rows r < R/2 are row0 + r and rows r >= R/2 are
// row0 + pair_offset + r - R/2 (gate and up halves of a [gate; up] matrix).
// Indices past M are clamped to M - 1 (re-read and discarded by the caller).
template <int R, bool PAIRED = false>
XPU_DEVICE void gemv_row_ptrs(const uint16_t *__restrict__ A, uint64_t lda, uint32_t M, uint32_t row0,
                              uint32_t pair_offset, const uint16_t *(&rows)[R]) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t want = PAIRED ? (r < R / 2 ? row0 + r : row0 + pair_offset + (r - R / 2)) : row0 + r;
    const uint32_t row = want < M ? want : M - 1;
    rows[r] = A + static_cast<uint64_t>(row) * lda + lane * 8u;
  }
}

template <int R, int U, bool VEC>
XPU_DEVICE void gemv_load_batch(u32x4 (&buf)[U][R], const uint16_t *const (&rows)[R], uint32_t j0,
                                uint32_t K) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int r = 0; r < R; ++r)
      buf[u][r] = load_row8<VEC>(rows[r] + (j0 + u) * 512u, (j0 + u) * 512u + lane * 8u, K);
}

// Canonical dot products of R rows (see gemv_row_ptrs) with the staged
// vector xs. All lanes must be active. When use_first is set (wave-uniform),
// `first` holds the rows' first batch (chunks 0..U-1), loaded earlier by the
// caller with gemv_load_batch so that its latency overlaps other work; it is
// only used when K has at least U full chunks.
template <int DT, int R, int U, bool VEC, bool PAIRED = false>
XPU_DEVICE void gemv_rows_first(const uint16_t *__restrict__ A, uint64_t lda, uint32_t K,
                                uint32_t M, const uint16_t *xs, uint32_t row0, float (&out)[R],
                                uint32_t pair_offset, const u32x4 (&first)[U][R], bool use_first) {
  const uint32_t lane = lane_id();
  float acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;
  const uint16_t *rows[R];
  gemv_row_ptrs<R, PAIRED>(A, lda, M, row0, pair_offset, rows);
  const uint16_t *xl = xs + lane * 8u;
  const uint32_t nfull = K / 512u;
  // Batches of U chunks (U x R 16-byte loads per lane) are software
  // pipelined: the loads of batch j + U are issued before the FMAs of batch
  // j, and a scheduling barrier keeps the compiler from interleaving each
  // load with its use (which would leave one load in flight per wave).
  auto load_batch = [&](u32x4 (&buf)[U][R], uint32_t j0) { gemv_load_batch<R, U, VEC>(buf, rows, j0, K); };
  auto fma_batch = [&](const u32x4 (&buf)[U][R], uint32_t j0) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      fma_chunk<DT, R>(acc, buf[u], *reinterpret_cast<const u32x4 *>(xl + (j0 + u) * 512u));
  };
  uint32_t j = 0;
  if (nfull >= static_cast<uint32_t>(U)) {
    u32x4 b0[U][R], b1[U][R];
    if (use_first) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r) b0[u][r] = first[u][r];
    } else {
      load_batch(b0, 0);
    }
    while (true) {
      if (j + 2 * U > nfull) { fma_batch(b0, j); j += U; break; }
      load_batch(b1, j + U);
      __builtin_amdgcn_sched_barrier(0);
      fma_batch(b0, j);
      j += U;
      if (j + 2 * U > nfull) { fma_batch(b1, j); j += U; break; }
      load_batch(b0, j + U);
      __builtin_amdgcn_sched_barrier(0);
      fma_batch(b1, j);
      j += U;
    }
  }
  for (; j < nfull; ++j) {
    u32x4 a[R];
#pragma unroll
    for (int r = 0; r < R; ++r) a[r] = load_row8<VEC>(rows[r] + j * 512u, j * 512u + lane * 8u, K);
    fma_chunk<DT, R>(acc, a, *reinterpret_cast<const u32x4 *>(xl + j * 512u));
  }
  if (K % 512u) {
    const uint32_t col = nfull * 512u + lane * 8u;
    if (col < K) {
      u32x4 a[R];
#pragma unroll
      for (int r = 0; r < R; ++r) a[r] = load_row8<VEC>(rows[r] + nfull * 512u, col, K);
      fma_chunk<DT, R>(acc, a, *reinterpret_cast<const u32x4 *>(xl + nfull * 512u));
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = wave_butterfly(fold8(acc[r]));
}

template <int DT, int R, int U, bool VEC, bool PAIRED = false>
XPU_DEVICE void gemv_rows(const uint16_t *__restrict__ A, uint64_t lda, uint32_t K, uint32_t M,
                          const uint16_t *xs, uint32_t row0, float (&out)[R], uint32_t pair_offset = 0) {
  u32x4 unused[U][R];
  gemv_rows_first<DT, R, U, VEC, PAIRED>(A, lda, K, M, xs, row0, out, pair_offset, unused, false);
}

}  // namespace xpu
