// GEMM C[M x N] = A[M x K] . B[K x N] on gfx950 MFMA, bf16 or fp16 storage,
// FP32 accumulation (reference: gemm_kernel.hpp:25-143 with argument order
// (a, b, c, m, n, k), level_zero/gem_spv_entry.cpp:28-60).
//
// Block tile 256 x 256 x 64 with 256 threads: four wavefronts in a 2 x 2
// arrangement, each owning 128 x 128 of C as 4 x 4 tiles of
// v_mfma_f32_32x32x16_{bf16,f16} (256 FP32 accumulators per lane, in AGPRs).
// A and B K-slices are loaded with buffer instructions into registers two
// slices ahead and stored to LDS, double buffered, one barrier per slice. A
// is stored row-major [m][k]; B is transposed in registers (8 x 8 blocks of
// 16-bit values via v_perm_b32) and stored [n][k], so both MFMA operands are
// single 16-byte LDS reads. Rows are padded by 8 elements so the 32 rows read
// by one ds_read_b128 fall in distinct banks.
//
// The kernels need A and B rows 16-byte aligned (K and N multiples of 8);
// the host pads other shapes into a workspace first (xpu_pad_rows below, the
// device counterpart of the reference's host padding, gemm.cpp:75-85). Rows
// past M, columns past N and the K tail are handled in the kernel: loads
// past the end of A or B read zero through the buffer range check, stores
// are masked.
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
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// ------------------------------------------------------------------ main path
//
// Rows of A and B 16-byte aligned (K, N multiples of 8): every 8-element
// chunk is wholly inside or wholly outside the matrix. Loads go through
// buffer descriptors rebased per K-slice, so rows past M (A) and past K (B)
// read as zero from the hardware range check, and chunks past K (A) or N (B)
// are sent to an offset beyond the descriptor's range (no branches in the
// main loop; slices past the end load zeros).
//
// Schedule per K-slice it (two register sets, two LDS buffers):
//   issue global loads of slice it + 2 into register set it % 2
//   MFMAs of slice it from LDS buffer it % 2
//   transpose + store slice it + 1 (register set (it + 1) % 2) to buffer (it + 1) % 2
//   barrier
// The loop is unrolled by two so register sets and LDS buffers are
// compile-time indices.
namespace vec {

constexpr uint32_t kOob = 0x80000000u;  // any offset >= the descriptor range reads 0

XPU_DEVICE __amdgpu_buffer_rsrc_t rsrc(const uint16_t *base, int64_t records) {
  records = records < 0 ? 0 : (records > 0x7fffffff ? 0x7fffffff : records);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(base), static_cast<short>(0),
                                           static_cast<int>(records), 0x00020000);
}

// Two FP32 values to packed 16-bit codes with the hardware conversion
// (round to nearest even, as the reference's esimd::convert<T> store,
// gemm_kernel.hpp:40-48); branch-free, unlike the integer codec.
template <int DT> XPU_DEVICE uint32_t cvt_pack(float lo, float hi) {
  if constexpr (DT == kFp16)
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(lo))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
  else
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(lo))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(hi))) << 16);
}

XPU_DEVICE u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
}

struct Ctx {
  const uint16_t *A, *B;
  uint32_t M, N, K, kb, m0, n0;
  uint32_t a_off;     // byte offset of this thread's first A chunk within a slice
  uint32_t b_off;     // byte offset of this thread's first B chunk (kOob + ... past N)
  uint32_t a_stride;  // bytes between the A chunks of one thread (32 rows)
  uint32_t b_stride;  // bytes between the B chunks of one thread (1 row)
  uint32_t a_col;     // first column of this thread's A chunk within a slice
};

// Loads of K-slice s: A rows a_row + 32 i, columns s*64 + a_chunk*8 .. +7;
// B rows s*64 + b_kb*8 + i, columns n0 + b_nb*8 .. +7.
XPU_DEVICE void issue(const Ctx &c, uint32_t s, u32x4 (&ra)[8], u32x4 (&rb)[8]) {
  const uint64_t k0 = static_cast<uint64_t>(s) * kBK;
  const __amdgpu_buffer_rsrc_t r_a =
      rsrc(c.A + static_cast<uint64_t>(c.m0) * c.K + k0,
           (static_cast<int64_t>(c.M - c.m0) * c.K - static_cast<int64_t>(k0)) * 2);
  const __amdgpu_buffer_rsrc_t r_b =
      rsrc(c.B + k0 * c.N + c.n0, (static_cast<int64_t>(c.kb) - static_cast<int64_t>(k0)) * c.N * 2 -
                                      static_cast<int64_t>(c.n0) * 2);
  const uint32_t a_base = k0 + c.a_col < c.K ? c.a_off : kOob;
#pragma unroll
  for (int i = 0; i < 8; ++i) ra[i] = load16(r_a, a_base + i * c.a_stride);
#pragma unroll
  for (int i = 0; i < 8; ++i) rb[i] = load16(r_b, c.b_off + i * c.b_stride);
}

// A chunks as loaded ([m][k] rows); B 8 x 8 blocks transposed to [n][k].
XPU_DEVICE void commit(uint16_t *__restrict__ la, uint16_t *__restrict__ lb, uint32_t tid,
                       const u32x4 (&ra)[8], const u32x4 (&rb)[8]) {
  const uint32_t a_chunk = tid & 7u, a_row = tid >> 3;
  const uint32_t b_kb = tid & 7u, b_nb = tid >> 3;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<u32x4 *>(la + (a_row + 32u * i) * kLdsPitch + a_chunk * 8u) = ra[i];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = __builtin_amdgcn_perm(rb[2 * q + 1][j >> 1], rb[2 * q][j >> 1], sel);
    *reinterpret_cast<u32x4 *>(lb + (b_nb * 8u + j) * kLdsPitch + b_kb * 8u) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// 4 k-steps of 16 MFMAs over one LDS buffer; fragments of the next k-step
// are read before the MFMAs of the current one.
template <int DT>
XPU_DEVICE void compute(const uint16_t *__restrict__ la, const uint16_t *__restrict__ lb, f32x16 (&acc)[4][4]) {
  u32x4 fa[2][4], fb[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    fa[0][i] = *reinterpret_cast<const u32x4 *>(la + i * 32u * kLdsPitch);
    fb[0][i] = *reinterpret_cast<const u32x4 *>(lb + i * 32u * kLdsPitch);
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fa[cur ^ 1][i] = *reinterpret_cast<const u32x4 *>(la + i * 32u * kLdsPitch + (ks + 1) * 16);
        fb[cur ^ 1][i] = *reinterpret_cast<const u32x4 *>(lb + i * 32u * kLdsPitch + (ks + 1) * 16);
      }
    }
    // operands swapped (B^T fragment first): the accumulator tile is C^T,
    // so each lane ends up with 4 consecutive columns of one row of C
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma<DT>(fb[cur][j], fa[cur][i], acc[i][j]);
  }
}

// Instruction order of one K-slice step (issue + compute + commit, one
// basic block): after the first k-step's 8 fragment reads, every MFMA is
// paired with one other instruction - the next k-step's fragment reads,
// the 16 global loads of slice it + 2, the 8 A-tile LDS stores and the
// 8 transposed B stores with their v_perm_b32 - so the matrix pipe never
// waits on an LDS round trip that could have been issued earlier.
XPU_DEVICE void schedule_step() {
  constexpr int kMfma = 0x008, kValu = 0x002, kVmemRead = 0x020, kDsRead = 0x100, kDsWrite = 0x200;
  __builtin_amdgcn_sched_group_barrier(kDsRead, 8, 0);
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // k-step 0: k-step 1 fragments, then loads 0..7
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kVmemRead, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // k-step 1: k-step 2 fragments, then loads 8..15
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kVmemRead, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // k-step 2: k-step 3 fragments, then A stores
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kDsWrite, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // k-step 3: B transposes and stores
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kValu, 4, 0);
    __builtin_amdgcn_sched_group_barrier(kDsWrite, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(kMfma, 8, 0);
}

// K: reduction length (columns of A); kb: rows of B (<= K; rows kb..K-1
// read as zero); N: columns of B; C has row stride ldc and n_out <= N valid
// columns. C16: C rows 16-byte aligned and n_out % 8 == 0 (16-byte stores).
template <int DT, bool C16>
XPU_DEVICE void body(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, uint16_t *__restrict__ C,
                     uint32_t M, uint32_t N, uint32_t K, uint32_t kb, uint32_t ldc, uint32_t n_out) {
  __shared__ __align__(16) uint16_t lds[2][2][kTileElems];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const TileCoord tc = tile_of_block(blockIdx.x, tiles_m, tiles_n);
  Ctx c;
  c.A = A;
  c.B = B;
  c.M = M;
  c.N = N;
  c.K = K;
  c.kb = kb;
  c.m0 = tc.tm * kBM;
  c.n0 = tc.tn * kBN;
  {
    const uint32_t a_chunk = tid & 7u, a_row = tid >> 3;
    const uint32_t b_kb = tid & 7u, b_nb = tid >> 3;
    c.a_col = a_chunk * 8u;
    // kOob + i * stride stays at or above the descriptor range limit
    // (< 2^31) and below 2^32 for the sizes the host admits
    c.a_off = (a_row * K + a_chunk * 8u) * 2u;
    c.b_off = c.n0 + b_nb * 8u < N ? (b_kb * 8u * N + b_nb * 8u) * 2u : kOob;
    c.a_stride = 64u * K;
    c.b_stride = 2u * N;
  }

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const uint32_t wm = wave >> 1, wn = wave & 1u;
  const uint32_t frag = (lane & 31u) * kLdsPitch + (lane >> 5) * 8u;
  const uint32_t fa_off = wm * 128u * kLdsPitch + frag, fb_off = wn * 128u * kLdsPitch + frag;
  const uint32_t nk = (K + kBK - 1) / kBK;

  u32x4 ra0[8], rb0[8], ra1[8], rb1[8];
  issue(c, 0, ra0, rb0);
  issue(c, 1, ra1, rb1);
  commit(lds[0][0], lds[0][1], tid, ra0, rb0);
  __syncthreads();
  uint32_t it = 0;
  do {  // nk >= 1 (K >= 1)
    issue(c, it + 2, ra0, rb0);
    compute<DT>(lds[0][0] + fa_off, lds[0][1] + fb_off, acc);
    commit(lds[1][0], lds[1][1], tid, ra1, rb1);
    schedule_step();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    // for odd nk this step runs slice nk, which loaded as zeros
    issue(c, it + 3, ra1, rb1);
    compute<DT>(lds[1][0] + fa_off, lds[1][1] + fb_off, acc);
    commit(lds[0][0], lds[0][1], tid, ra0, rb0);
    schedule_step();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    it += 2;
  } while (it < nk);

  // Epilogue through LDS (free after the loop's last barrier), one 64-row
  // band per round: each wave writes its 64 x 128 FP32 band (D layout of
  // v_mfma_f32_32x32x16 with C^T tiles: lane l holds row l % 32, columns
  // 8 g + 4 (l / 32) + 0..3 in accumulators 4 g..4 g + 3) as 16-byte rows
  // into its own region (pitch 132 floats: the 8 rows written by 8
  // consecutive lanes fall in distinct banks), then reads it back 8
  // consecutive columns per lane and stores 16 bytes of C per lane.
  constexpr uint32_t kEpPitch = 132;
  float *ep = reinterpret_cast<float *>(&lds[0][0][0]) + wave * 64u * kEpPitch;
  const uint32_t m_lane = lane & 31u, n_lane = (lane >> 5) * 4u;
  const uint32_t r_lane = lane >> 4, c_lane = (lane & 15u) * 8u;
#pragma unroll
  for (int band = 0; band < 2; ++band) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int i = band * 2 + ii;
          *reinterpret_cast<f32x4 *>(ep + (ii * 32u + m_lane) * kEpPitch + j * 32u + 8u * g + n_lane) =
              f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const uint32_t r = rr * 4u + r_lane;
      const f32x4 lo = *reinterpret_cast<const f32x4 *>(ep + r * kEpPitch + c_lane);
      const f32x4 hi = *reinterpret_cast<const f32x4 *>(ep + r * kEpPitch + c_lane + 4u);
      const uint32_t m = c.m0 + wm * 128u + band * 64u + r, n = c.n0 + wn * 128u + c_lane;
      if (m >= M || n >= n_out) continue;
      const u32x4 packed{cvt_pack<DT>(lo.x, lo.y), cvt_pack<DT>(lo.z, lo.w), cvt_pack<DT>(hi.x, hi.y),
                         cvt_pack<DT>(hi.z, hi.w)};
      uint16_t *dst = C + static_cast<uint64_t>(m) * ldc + n;
      if constexpr (C16) {
        *reinterpret_cast<u32x4 *>(dst) = packed;  // n_out % 8 == 0: n + 7 < n_out
      } else {
        const uint32_t w[4] = {packed.x, packed.y, packed.z, packed.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < n_out) dst[e] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

}  // namespace vec

}  // namespace xpu

#define XPU_GEMM_VEC_VARIANT(NAME, DT, C16)                                                    \
  extern "C" __global__ __launch_bounds__(256, 1) void NAME(                                  \
      const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, uint16_t *__restrict__ C, \
      uint32_t M, uint32_t N, uint32_t K, uint32_t kb, uint32_t ldc, uint32_t n_out) {         \
    xpu::vec::body<DT, C16>(A, B, C, M, N, K, kb, ldc, n_out);                                 \
  }

XPU_GEMM_VEC_VARIANT(xpu_gemm_bf16_vec, xpu::kBf16, true)
XPU_GEMM_VEC_VARIANT(xpu_gemm_fp16_vec, xpu::kFp16, true)
XPU_GEMM_VEC_VARIANT(xpu_gemm_bf16_vecu, xpu::kBf16, false)
XPU_GEMM_VEC_VARIANT(xpu_gemm_fp16_vecu, xpu::kFp16, false)

// dst[r][c] = src[r * src_ld + c] for c < cols, 0 for cols <= c < dst_cols
// (dst_cols % 8 == 0, dst 16-byte aligned): the zero padding of the
// reference's host GEMM setup (gemm.cpp:75-85) done on the device, so rows
// of the copy are 16-byte aligned. One thread per 8 destination elements.
// src only needs 2-byte alignment: a chunk that starts on a 4-byte boundary
// is one 16-byte load; one that starts 2 bytes past it is the 16-byte load
// one element earlier plus the chunk's last element, shifted into place.
// The chunk holding the row's end is read element by element, so no load
// reaches past the last element of a row.
extern "C" __global__ __launch_bounds__(256) void xpu_pad_rows(const uint16_t *__restrict__ src, uint64_t src_ld,
                                                               uint32_t rows, uint32_t cols,
                                                               uint16_t *__restrict__ dst, uint32_t dst_cols) {
  const uint64_t chunks_per_row = dst_cols / 8u;
  const uint64_t total = static_cast<uint64_t>(rows) * chunks_per_row;
  for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t r = idx / chunks_per_row;
    const uint32_t c0 = static_cast<uint32_t>(idx % chunks_per_row) * 8u;
    const uint16_t *p = src + r * src_ld + c0;
    xpu::u32x4 v;
    if (c0 + 8u <= cols) {
      if ((reinterpret_cast<uintptr_t>(p) & 3u) == 0) {
        v = *reinterpret_cast<const xpu::u32x4 *>(p);
      } else {
        const xpu::u32x4 d = *reinterpret_cast<const xpu::u32x4 *>(p - 1);  // elements -1..6
        const uint32_t last = p[7];
        v = xpu::u32x4{__builtin_amdgcn_alignbit(d.y, d.x, 16), __builtin_amdgcn_alignbit(d.z, d.y, 16),
                       __builtin_amdgcn_alignbit(d.w, d.z, 16), __builtin_amdgcn_alignbit(last, d.w, 16)};
      }
    } else {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo = c0 + 2 * q < cols ? p[2 * q] : 0u;
        const uint32_t hi = c0 + 2 * q + 1 < cols ? p[2 * q + 1] : 0u;
        w[q] = lo | (hi << 16);
      }
      v = xpu::u32x4{w[0], w[1], w[2], w[3]};
    }
    *reinterpret_cast<xpu::u32x4 *>(dst + r * dst_cols + c0) = v;
  }
}
