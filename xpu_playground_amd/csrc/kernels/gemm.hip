// GEMM C[M x N] = A[M x K] . B[K x N] on gfx950 MFMA with LDS-DMA operand
// staging, bf16 or fp16 storage, FP32 accumulation (reference:
// gemm_kernel.hpp:25-143, argument order (a, b, c, m, n, k) of
// level_zero/gem_spv_entry.cpp:28-60).
//
// Block tile (64 MI) x (64 NJ), K-slice BK (64 or 32), two LDS stages, 256
// threads: four wavefronts in a 2 x 2 arrangement, each owning 32 MI x 32 NJ
// of C as MI x NJ tiles of v_mfma_f32_32x32x16_{bf16,f16}. The large tile is
// 256 x 256 (MI = NJ = 4, 256 FP32 accumulators per lane). The small tiles,
// 128 x 256 (the reference's small tile, gemm_kernel.hpp:26-27) and
// 128 x 128, cut shapes that fill few compute units with the large tile
// into more blocks. The 224 x 256 tile puts the four wavefronts side by
// side along N (1 x 4, MI = 7, NJ = 2): outputs whose 256 x 256 tiles leave
// compute units idle but whose 224-row tiles still fit one per unit
// (3000 x 4097: 204 of 256 units busy with 256 x 256, 238 with 224 x 256)
// run 7/8 of the work per unit. The host picks the tile by compute-unit
// fill.
//
// Operands go from global memory straight into LDS with buffer_load_dwordx4
// ... lds (the LDS-DMA form: lane t's 16 bytes land at M0 + 16 t), so no
// VGPR staging and no LDS store instructions. Both tiles keep the global
// row-major orientation: A as [m][k] (2 BK bytes per row), B as [k][n]
// (512 bytes per row). 16-byte chunks are XOR-swizzled within a row so the
// fragment reads hit distinct banks. A fragments are single ds_read_b128
// (lane l: row l % 32, 8 consecutive k); B fragments are two
// ds_read_b64_tr_b16 (the gfx950 transposing read: within each 16-lane
// group, lane j receives element (j & 3) of the 4-element rows addressed by
// lanes (j >> 2) + 4 e, e = 0..3), which hand each lane 8 consecutive k of
// one column n - the MFMA operand layout - out of the [k][n] tile.
//
// Pipeline (slice s in stage s % 2): the DMA of slice s + 2 is issued right
// after the barrier that publishes slice s + 1, into the stage slice s just
// vacated; that barrier sits in slice s's last k-step after the first P of
// its MFMAs and is preceded by a wait for the DMA of slice s + 1. A slice's
// DMA is spread over the D k-steps from its barrier on (D = 2 leaves the last
// of it more than two k-steps to land). Fragments of the next k-step are read
// while the current one's MFMAs run. Slices go in pairs; the _odd kernels
// (an odd slice count of 3 or more) run the last slice on its own, only its
// k-steps below K.
//
// Edges, for any M, N, K and operands at any 2-byte alignment (the
// reference pads on the host instead, gemm.cpp:75-85):
// - The LDS-DMA moves 16 bytes from any byte address (checked on gfx950 at
//   every offset 0..15), so rows of A and B that are not 16-byte aligned
//   (K or N not a multiple of 8, or an unaligned base) are staged in place.
// - Loads past row M of A and past row K of B read zero through the buffer
//   range check; 16-byte chunks that start at or past column K of A or N of
//   B are sent beyond the descriptor range.
// - The chunk of A that straddles column K holds the next row's first
//   elements: in the last K-slice each wavefront zeroes them in the rows it
//   staged, after its DMA has landed and before the barrier that publishes
//   the slice (fix_tail). B rows past K are zero, and B columns past N only
//   reach C columns that are not stored.
// - The range check zeroes whole dwords (any dword whose end passes the
//   range reads 0), so with K odd the last element of A, A[M-1][K-1], shares
//   a dword with the byte past A's end and reads 0, and with N odd so does
//   B[K-1][N-1]. fix_tail puts each back from a plain 2-byte load. Nothing
//   is read past either operand.
// Stores are masked to M x n_out; the _dmau variants take C rows that are
// only 2-byte aligned.
#include "device_common.hpp"

#include <type_traits>

namespace xpu {
namespace dma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr uint32_t kOob = 0x80000000u;  // any offset >= the descriptor range reads 0

template <int DT>
XPU_DEVICE f32x16 mfma(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
  if constexpr (DT == kFp16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// XOR swizzles of 16-byte chunks. A: row r of the tile (2 BK bytes), B:
// row k (512 bytes). With them the rows read by one ds_read_b128 (32 rows,
// one chunk column) and the 4 x 4 (row, chunk) blocks read by one
// ds_read_b64_tr_b16 group pair fall into distinct 16-byte bank groups
// whether the LDS serves 128 or 256 bytes per clock.
template <int BK> XPU_DEVICE uint32_t a_swz(uint32_t r) {
  if constexpr (BK == 64) return (r & 7u) ^ ((r >> 3) & 1u);
  else return ((r >> 1) & 3u) ^ ((r >> 3) & 1u);
}
XPU_DEVICE uint32_t b_swz(uint32_t k) { return ((k & 1u) ? 10u : 0u) ^ ((k & 2u) ? 4u : 0u); }

struct TileCoord {
  uint32_t tm, tn;
};

// Blocks are dealt round-robin to the 8 XCDs; when the tile count is a
// multiple of 8, block b is renumbered to a contiguous range per XCD, and
// tiles are walked in groups of 4 tile-rows so the blocks of one XCD share
// A and B panels in that XCD's L2.
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

// Two FP32 values to two RNE-rounded 16-bit codes in one register (lo in
// bits 0-15): one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <int DT> XPU_DEVICE uint32_t cvt_pack(float lo, float hi) {
  if constexpr (DT == kFp16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// MI, NJ: 32 x 32 MFMA tiles per wavefront along M and N (wavefront tile
// 32 MI x 32 NJ); WN: wavefronts along N (2: a 2 x 2 arrangement, block tile
// 64 MI x 64 NJ; 4: 1 x 4, block tile 32 MI x 128 NJ); BK: K-slice; S: LDS
// stages.
template <int MI, int NJ, int BK, int S, bool BT = false, int WN = 2> struct Cfg {
  static_assert(WN == 2 || WN == 4, "2 x 2 or 1 x 4 wavefronts");
  static constexpr uint32_t kBMW = 32u * MI;                 // rows per wavefront
  static constexpr uint32_t kBM = (4u / WN) * kBMW;          // block tile rows
  static constexpr uint32_t kBNW = 32u * NJ;                 // columns per wavefront
  static constexpr uint32_t kBN = WN * kBNW;                 // block tile columns
  static constexpr uint32_t kKs = BK / 16;                   // k-steps per slice
  static constexpr uint32_t kABytes = kBM * 2u * BK;         // kBM rows x 2 BK bytes
  static constexpr uint32_t kBRow = 2u * kBN;                // bytes per B row in LDS
  static constexpr uint32_t kStage = kABytes + BK * kBRow;   // A then B
  static constexpr uint32_t kCpr = BK / 8;                   // 16-byte chunks per A row
  static constexpr uint32_t kRpi = 64 / kCpr;                // A rows per DMA instruction
  static constexpr uint32_t kBCpr = kBN / 8;                 // 16-byte chunks per B row
  static constexpr uint32_t kBRpi = 64 / kBCpr;              // B rows per DMA instruction
  static constexpr uint32_t kDmaA = kBM / kRpi / 4;          // A DMA instructions per wave per slice
  // B DMA instructions per wave per slice ([n][k] tiles: as A, kBN rows)
  static constexpr uint32_t kDmaB = BT ? kBN / kRpi / 4 : BK / kBRpi / 4;
  static constexpr uint32_t kDma = kDmaA + kDmaB;
  static constexpr uint32_t kMf = MI * NJ;                   // MFMAs per k-step
  // fragment reads per k-step ([n][k] B fragments are one read each)
  static constexpr uint32_t kReads = BT ? MI + NJ : MI + 2u * NJ;
  static constexpr uint32_t kEpPitch = kBNW + 4;             // epilogue staging pitch (floats)
  static constexpr uint32_t kEpBytes = 4u * 64u * kEpPitch * 4u;
  static constexpr uint32_t kLds = S * kStage > kEpBytes ? S * kStage : kEpBytes;
  static_assert(kLds <= 160u * 1024u, "LDS");
  static_assert(BT || kBCpr == 16 || kBCpr == 32, "[k][n] B rows of 16 or 32 chunks (the swizzle permutes 16)");
  static_assert(kBM % (4u * kRpi) == 0 && kDmaA >= 1, "every wave issues the same A DMA, at least one");
};

// ODD: the slice count nk is odd and at least 3 (the host's choice; other
// counts would sum a slice twice); the last slice runs on its own after the
// pairs, and only its k-steps that start below K (otherwise the last pair's
// second slice would add a slice of zeros, and a slice that ends past K its
// dead k-steps).
// BT: B is given as its transpose, [N][K] row-major (the rows of a weight
// matrix W for C = X W^T); its tile is staged and read like A's. RES: C is
// updated in place, C = bf16(C + bf16(A B)) (a residual add), C16 only.
// PART: split K. Block b computes tile b % tiles over slices split * kb ..
// split * kb + kb - 1, split = b / tiles (kb, a multiple of S, is the slices
// per split here), and stores its FP32 partial tile into ((float *)
// C)[split][M][ldc] (ldc >= N, a multiple of 4: whole 16-byte groups of
// columns are stored); xpu_gemm_splitk_reduce[_any] adds the splits.
template <int DT, int MI, int NJ, int BK, int S, int P, int D, bool C16, bool ODD, bool BT = false,
          bool RES = false, bool PART = false, bool EDGE = false, int WN = 2>
XPU_DEVICE void body(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, uint16_t *__restrict__ C,
                     uint32_t M, uint32_t N, uint32_t K, uint32_t kb, uint32_t ldc, uint32_t n_out) {
  using G = Cfg<MI, NJ, BK, S, BT, WN>;
  const uint32_t K_ = K, M_ = M, N_ = N;  // for fix_tail, which shadows them
  static_assert(!RES || C16, "the residual epilogue stores 16-byte chunks");
  static_assert(!PART || (!RES && !ODD), "split K: the reduction applies any residual");
  static_assert(!EDGE || !BT, "the [n][k] kernels take K % 8 == 0");
  __shared__ __align__(1024) uint8_t lds[G::kLds];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t tiles_m = (M + G::kBM - 1) / G::kBM, tiles_n = (N + G::kBN - 1) / G::kBN;
  const uint32_t split = PART ? blockIdx.x / (tiles_m * tiles_n) : 0u;
  const uint32_t s_base = PART ? split * kb : 0u;  // first slice of this block
  const TileCoord tc = tile_of_block(PART ? blockIdx.x % (tiles_m * tiles_n) : blockIdx.x, tiles_m, tiles_n);
  const uint32_t m0 = tc.tm * G::kBM, n0 = tc.tn * G::kBN;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));

  // DMA lane maps. A: instruction i of this wave fills tile rows
  // (wave + 4 i) * kRpi .. + kRpi - 1; lane t lands in physical chunk
  // t % kCpr of row t / kCpr and fetches the logical chunk that the swizzle
  // puts there. B: instruction i fills rows kBRpi (wave + 4 i) .. + kBRpi - 1.
  const uint32_t a_row = wave * G::kRpi + lane / G::kCpr;
  const uint32_t a_chunk = (lane % G::kCpr) ^ a_swz<BK>(a_row & 15u);
  const uint32_t a_voff = (a_row * K + a_chunk * 8u) * 2u;
  const uint32_t a_istride = 4u * G::kRpi * K * 2u;
  // B as [k][n]: instruction i fills rows kBRpi (wave + 4 i) .. + kBRpi - 1;
  // B as [n][k] (BT): the A map over its kBN rows
  const uint32_t b_row = BT ? a_row : G::kBRpi * wave + lane / G::kBCpr;
  const uint32_t b_chunk = BT ? a_chunk : (lane % G::kBCpr) ^ b_swz(b_row & 3u);
  const uint32_t b_voff = BT ? (b_row * K + b_chunk * 8u) * 2u
                             : (n0 + b_chunk * 8u < N ? (b_row * N + b_chunk * 8u) * 2u : kOob);
  const uint32_t b_istride = BT ? a_istride : 4u * G::kBRpi * N * 2u;

  // Each lane's buffer offset of every DMA instruction, computed once: the
  // slices differ only in their descriptors, so the K loop issues its DMA
  // with scalar work only (vector ALU instructions between the MFMAs cost
  // the MFMA pipe their issue cycles).
  // a_cur / b_cur: the offsets the next slice's DMA uses (a_off / b_off
  // with the chunks at or past column K sent out of range, from the first
  // slice that is not live on)
  uint32_t a_off[G::kDmaA], b_off[G::kDmaB], a_cur[G::kDmaA], b_cur[G::kDmaB];
#pragma unroll
  for (uint32_t op = 0; op < G::kDmaA; ++op) a_cur[op] = a_off[op] = a_voff + op * a_istride;
#pragma unroll
  for (uint32_t op = 0; op < G::kDmaB; ++op) b_cur[op] = b_off[op] = b_voff + op * b_istride;

  // DMA instruction d (0 .. kDma-1) of slice s into stage st: A rows first,
  // then B rows. Per slice the descriptors are rebased to the slice's first
  // column (A) and row (B); from the slice that holds column K on (the last
  // one, and the zero slices that complete a group), the chunks at or past
  // column K of A (and of an [n][k] B) go past the descriptor range and read
  // zeros. Slices are set up in ascending order, so a_cur / b_cur only ever
  // lose lanes.
  struct Slice {
    i32x4 r_a, r_b;
    uint32_t st_base;
  };
  auto slice_of = [&](uint32_t s, uint32_t stage) {
    const uint32_t k0_32 = (s_base + s) * BK;
    const uint64_t k0 = k0_32;
    Slice d;
    d.r_a = rsrc(A + static_cast<uint64_t>(m0) * K + k0,
                 (static_cast<int64_t>(M - m0) * K - static_cast<int64_t>(k0)) * 2);
    if constexpr (BT)
      d.r_b = rsrc(B + static_cast<uint64_t>(n0) * K + k0,
                   (static_cast<int64_t>(N - n0) * K - static_cast<int64_t>(k0)) * 2);
    else
      d.r_b = rsrc(B + k0 * N + n0,
                   (static_cast<int64_t>(K) - static_cast<int64_t>(k0)) * N * 2 - static_cast<int64_t>(n0) * 2);
    d.st_base = lds0 + stage * G::kStage;
    if (k0_32 + BK > K) {  // the last slice of A's columns, or one past them (a uniform branch)
#pragma unroll
      for (uint32_t op = 0; op < G::kDmaA; ++op) a_cur[op] = k0_32 + a_chunk * 8u < K ? a_off[op] : kOob;
      if constexpr (BT) {
#pragma unroll
        for (uint32_t op = 0; op < G::kDmaB; ++op) b_cur[op] = k0_32 + b_chunk * 8u < K ? b_off[op] : kOob;
      }
    }
    return d;
  };
  auto dma = [&](const Slice &d, uint32_t op) {
    if (op < G::kDmaA)
      dma16(d.st_base + (wave + 4u * op) * 1024u, d.r_a, a_cur[op]);
    else
      dma16(d.st_base + G::kABytes + (wave + 4u * (op - G::kDmaA)) * 1024u, d.r_b, b_cur[op - G::kDmaA]);
  };

  // Fragment addresses (bytes within a stage). A: row wm*kBMW + 32 i + l%32,
  // logical chunk 2 ks + l/32. B: k-row 16 ks + 8 (l/32) + 4 h + (l%16)/4,
  // column wn*kBNW + 32 j + 16 ((l/16) % 2) + 4 (l % 4): the 4-element row
  // that lane l contributes to its group's transposing read.
  const uint32_t wm = wave / WN, wn = wave % WN;
  // The ds_read offset field holds 16 bits, so the stages are addressed from
  // one base per 64 KiB group; the bases are made opaque to the compiler so
  // that it keeps them in registers instead of materialising one register per
  // (stage, k-step, tile) combination.
  constexpr uint32_t kGroups = (S * G::kStage + 65535u) / 65536u;
  constexpr uint32_t kFb = BT ? G::kKs : NJ;  // B bases: per k-step ([n][k]) or per column tile ([k][n])
  uint32_t fa_base[kGroups][G::kKs], fb_base[kGroups][kFb];
  {
    const uint32_t krow = 8u * (lane >> 5) + ((lane & 15u) >> 2);
    const uint32_t x = 2u * ((lane >> 4) & 1u) + ((lane & 3u) >> 1);
#pragma unroll
    for (uint32_t g = 0; g < kGroups; ++g) {
#pragma unroll
      for (uint32_t ks = 0; ks < G::kKs; ++ks) {
        fa_base[g][ks] = lds0 + g * 65536u + (wm * G::kBMW + (lane & 31u)) * (2u * BK) +
                         16u * ((2u * ks + (lane >> 5)) ^ a_swz<BK>(lane & 15u));
        asm volatile("" : "+v"(fa_base[g][ks]));
      }
#pragma unroll
      for (uint32_t j = 0; j < kFb; ++j) {
        if constexpr (BT)  // row wn*kBNW + 32 jj + l%32, logical chunk 2 ks + l/32 (ks = j here)
          fb_base[g][j] = lds0 + g * 65536u + G::kABytes + (wn * G::kBNW + (lane & 31u)) * (2u * BK) +
                          16u * ((2u * j + (lane >> 5)) ^ a_swz<BK>(lane & 15u));
        else
          fb_base[g][j] = lds0 + g * 65536u + G::kABytes + krow * G::kBRow +
                          16u * ((wn * (G::kBNW / 8u) + 4u * j + x) ^ b_swz(krow & 3u)) + 8u * (lane & 1u);
        asm volatile("" : "+v"(fb_base[g][j]));
      }
    }
  }

  struct Frags {
    u32x4 a[MI], b[NJ];
  };
  // Read r (0 .. kReads-1) of the fragments of k-step ks in a stage, in the
  // order the MFMAs consume them: A0, B0 .. B(NJ-1) (two halves each), A1 ..
  // A(MI-1).
  auto read = [&](uint32_t stage, uint32_t ks, Frags &f, uint32_t r) {
    const uint32_t g = stage * G::kStage / 65536u, in_group = stage * G::kStage % 65536u;
    if constexpr (BT) {
      // A0, B0 .. B(NJ-1), A1 .. A(MI-1), one ds_read_b128 each
      if (r == 0 || r > NJ) {
        const uint32_t i = r == 0 ? 0 : r - NJ;
        f.a[i] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(
            fa_base[g][ks] + in_group + i * 32u * 2u * BK);
      } else {
        f.b[r - 1] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(
            fb_base[g][ks] + in_group + (r - 1) * 32u * 2u * BK);
      }
      return;
    }
    if (r == 0 || r > 2u * NJ) {
      const uint32_t i = r == 0 ? 0 : r - 2u * NJ;
      const uint32_t addr = fa_base[g][ks] + in_group + i * 32u * 2u * BK;
      f.a[i] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(addr);
    } else {
      const uint32_t j = (r - 1) >> 1, h = (r - 1) & 1;
      const uint32_t addr = fb_base[g][j] + in_group + (16u * ks + 4u * h) * G::kBRow;
      const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(addr)));
      if (h == 0) {
        f.b[j].x = v.x;
        f.b[j].y = v.y;
      } else {
        f.b[j].z = v.x;
        f.b[j].w = v.y;
      }
    }
  };

  f32x16 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // MFMA q = NJ i + j. Operands swapped (B^T fragment first): the
  // accumulator tile is C^T, so each lane ends up with 4 consecutive
  // columns of one row of C.
  auto mfma_q = [&](const Frags &f, uint32_t q) {
    acc[q / NJ][q % NJ] = mfma<DT>(f.b[q % NJ], f.a[q / NJ], acc[q / NJ][q % NJ]);
  };

  const uint32_t nk = PART ? kb : (K + BK - 1) / BK;
  static_assert(D >= 1 && D <= G::kKs, "a slice's DMA is issued within the k-steps before the next barrier");
  static_assert(P < G::kMf, "k-step schedule: MFMAs after the barrier carry the next slice's first reads");
  // fragment reads of the next k-step issued after MFMA q of an ordinary
  // k-step: one after each of the first kReads MFMAs, or spread evenly when
  // there are more reads than MFMAs
  auto reads_after = [](uint32_t q, uint32_t &lo, uint32_t &hi) {
    if constexpr (G::kReads <= G::kMf) {
      lo = q;
      hi = q < G::kReads ? q + 1 : q;
    } else {
      lo = q * G::kReads / G::kMf;
      hi = (q + 1) * G::kReads / G::kMf;
    }
  };
  // DMA ops of one slice issued during the e-th k-step after its barrier
  auto dma_part = [&](const Slice &d, uint32_t e, uint32_t x, uint32_t nx) {
    const uint32_t lo = e * G::kDma / D, hi = (e + 1) * G::kDma / D;
#pragma unroll
    for (uint32_t op = lo + x * (hi - lo) / nx; op < lo + (x + 1) * (hi - lo) / nx; ++op) dma(d, op);
  };
  // The last K-slice's edges (EDGE kernels: K % 8 != 0 or N odd), in stage
  // `stage`, after this wavefront's DMA of the slice has landed and before
  // the barrier that publishes it. A: lane l owns tile row (wave + 4 (l /
  // kRpi)) kRpi + l % kRpi (the rows this wave staged) and zeroes the
  // elements of the chunk holding column K at and past K; the lane holding
  // row M - 1 restores A[M-1][K-1] (K odd). B: the wave that staged tile row
  // K - 1 restores B[K-1][N-1] (N odd). The shapes are passed through an
  // empty asm first, so that the compiler derives the addresses here, once,
  // instead of holding them in scalar registers across the K loop.
  // (split K: the last slice of the whole product, in the last split's
  // blocks; last_local is its index among this block's slices)
  const uint32_t nk_total = (K + BK - 1) / BK;
  const uint32_t last_local = nk_total - 1u - s_base;  // wraps past any slice of a block before it
  auto fix_tail = [&](uint32_t stage) {
    if constexpr (EDGE) {
      uint32_t K = K_, M = M_, N = N_;
      asm volatile("" : "+s"(K), "+s"(M), "+s"(N));
      const uint32_t kc = K - (nk_total - 1u) * BK;  // live columns of the last slice, 1 .. BK
      const uint32_t st_base = lds0 + stage * G::kStage;
      typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
      typedef __attribute__((address_space(3))) uint16_t lds_u16;
      constexpr uint32_t kRowsW = G::kDmaA * G::kRpi;  // A rows staged per wave (kBM / 4)
      const uint32_t keep = kc % 8u;
      if (keep != 0 && lane < kRowsW) {
        const uint32_t r = (wave + 4u * (lane / G::kRpi)) * G::kRpi + lane % G::kRpi;
        const uint32_t addr = st_base + r * (2u * BK) + 16u * ((kc / 8u) ^ a_swz<BK>(r & 15u));
        const u32x4 v = *reinterpret_cast<const lds_u32x4 *>(addr);
        // element keep - 1 (even when K is odd) is the low half of dword keep / 2
        const bool restore = (K & 1u) && m0 + r == M - 1u;
        const uint32_t e = restore ? A[static_cast<uint64_t>(M - 1u) * K + (K - 1u)] : 0u;
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (uint32_t d = 0; d < 4; ++d) {
          if (restore && d == keep / 2u) w[d] = (w[d] & 0xffff0000u) | e;
          if (2u * d >= keep) w[d] = 0u;
          else if (2u * d + 1u >= keep) w[d] &= 0xffffu;
        }
        *reinterpret_cast<lds_u32x4 *>(addr) = u32x4{w[0], w[1], w[2], w[3]};
      }
      if (N & 1u) {
        const uint32_t kt = kc - 1u, nt = N - 1u - n0;
        if (nt < G::kBN && (kt / G::kBRpi) % 4u == wave && lane == 0) {
          const uint32_t addr =
              st_base + G::kABytes + kt * G::kBRow + 16u * ((nt / 8u) ^ b_swz(kt & 3u)) + 2u * (nt % 8u);
          *reinterpret_cast<lds_u16 *>(addr) = B[static_cast<uint64_t>(K - 1u) * N + (N - 1u)];
        }
      }
    }
  };

  Frags frag[2];
  static_assert(S == 2 || (S >= 3 && S <= 6 && !ODD), "groups of 2 to 6 slices; the odd tail follows a pair");
  // Slice s lives in LDS stage s % S. Prologue: slices 0 .. S - 2 whole, and
  // the first part of slice S - 1 as if its barrier had just passed; the
  // rest of slice S - 1 follows during slice 0 like any slice's DMA.
#pragma unroll
  for (uint32_t s = 0; s + 1 < S; ++s) {
    const Slice d = slice_of(s, s);
#pragma unroll
    for (uint32_t op = 0; op < G::kDma; ++op) dma(d, op);
  }
  Slice pend = slice_of(S - 1, S - 1);
  dma_part(pend, 0, 0, 1);
  wait_vmcnt<(S - 2) * G::kDma + G::kDma / D>();  // slice 0 landed
  if (EDGE && last_local == 0) fix_tail(0);
  __syncthreads();
#pragma unroll
  for (uint32_t r = 0; r < G::kReads; ++r) read(0, 0, frag[0], r);
  XPU_PHASE(0);  // (stamps build) prologue done: slice 0 published, its first fragments read

  // Instruction order is fixed with sched_barrier. Ordinary k-step: each of
  // the first kReads MFMAs is followed by one fragment read of the next
  // k-step, and the pending slice's DMA share of this k-step is spread over
  // the kMf MFMAs. Last k-step of a slice: P MFMAs, the wait and the
  // barrier, then the remaining MFMAs with the next slice's first fragment
  // reads and the first share of the new slice's DMA (the DMA of a slice is
  // spread over the D k-steps from its barrier on).
  // One slice: s0 + st, in stage st (st a compile-time constant).
  auto slice_step = [&](auto stc, uint32_t s0) {
    constexpr uint32_t st = decltype(stc)::value;
#pragma unroll
      for (uint32_t ks = 0; ks < G::kKs; ++ks) {
        const int cur = (st * G::kKs + ks) & 1;
        if (ks + 1 < G::kKs) {
          const uint32_t e = ks + 1;  // k-steps since the pending slice's barrier
#pragma unroll
          for (uint32_t q = 0; q < G::kMf; ++q) {
            mfma_q(frag[cur], q);
            uint32_t lo, hi;
            reads_after(q, lo, hi);
#pragma unroll
            for (uint32_t r = lo; r < hi; ++r) read(st, ks + 1, frag[cur ^ 1], r);
            if (e < D) dma_part(pend, e, q, G::kMf);
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
#pragma unroll
          for (uint32_t q = 0; q < P; ++q) {
            mfma_q(frag[cur], q);
            __builtin_amdgcn_sched_barrier(0);
          }
          wait_vmcnt<(S - 2) * G::kDma>();
          if (EDGE && s0 + st + 1u == last_local) fix_tail((st + 1) % S);  // publishes the last slice
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
          pend = slice_of(s0 + st + S, st);
          constexpr uint32_t kAfter = G::kMf - P;
#pragma unroll
          for (uint32_t q = P; q < G::kMf; ++q) {
            mfma_q(frag[cur], q);
            const uint32_t x = q - P;
            dma_part(pend, 0, x, kAfter);
#pragma unroll
            for (uint32_t r = x * G::kReads / kAfter; r < (x + 1) * G::kReads / kAfter; ++r)
              read((st + 1) % S, 0, frag[cur ^ 1], r);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
  };
  // Whole groups of S slices (one exit keeps the accumulators in place); a
  // group's slices past nk read zeros and add nothing. With ODD the pairs
  // stop before the last slice, which follows on its own (stage 0, its DMA
  // and barrier already done by the last pair): the MFMAs of its k-steps
  // that start below K, with the next k-step's fragment reads.
  // stage constants 0 .. S - 1 (a stage index past S - 1 is never run)
  auto step_if = [&](auto stc, uint32_t s) {
    if constexpr (decltype(stc)::value < S) slice_step(stc, s);
  };
  // (at least one pair: ODD kernels take nk >= 3)
  uint32_t s0 = 0;
  do {
    step_if(std::integral_constant<uint32_t, 0>{}, s0);
    step_if(std::integral_constant<uint32_t, 1>{}, s0);
    step_if(std::integral_constant<uint32_t, 2>{}, s0);
    step_if(std::integral_constant<uint32_t, 3>{}, s0);
    step_if(std::integral_constant<uint32_t, 4>{}, s0);
    step_if(std::integral_constant<uint32_t, 5>{}, s0);
    s0 += S;
  } while (s0 < (ODD ? nk - 1 : nk));
  if constexpr (ODD) {
    const uint32_t live = (K - (nk - 1) * BK + 15) / 16;  // 1 .. kKs
    // k-steps past the live ones are skipped by a uniform branch; the reads
    // of k-step ks + 1 only where it is live
#pragma unroll
    for (uint32_t ks = 0; ks < G::kKs; ++ks) {
      if (ks == 0 || ks < live) {
        const int cur = ks & 1;
#pragma unroll
        for (uint32_t q = 0; q < G::kMf; ++q) {
          mfma_q(frag[cur], q);
          uint32_t lo, hi;
          reads_after(q, lo, hi);
          if (ks + 1 < G::kKs && ks + 1 < live) {
#pragma unroll
            for (uint32_t r = lo; r < hi; ++r) read(0, ks + 1, frag[cur ^ 1], r);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
  XPU_PHASE(1);  // (stamps build) the K loop's last MFMA issued
  // drain the DMA of slices past the end (they read zeros) before the
  // epilogue reuses the LDS
  wait_vmcnt<0>();
  __syncthreads();
  XPU_PHASE(2);  // (stamps build) the epilogue starts

  // Epilogue through LDS, one 64-row band per round ((MI + 1) / 2 rounds; with
  // MI odd the last band has 32 rows): each wave writes its
  // 64 x kBNW FP32 band (D layout of v_mfma_f32_32x32x16 with C^T tiles: lane
  // l holds row l % 32, columns 8 g + 4 (l / 32) + 0..3 in accumulators
  // 4 g..4 g + 3) as 16-byte rows into its own region (pitch kBNW + 4
  // floats), then reads it back 8 consecutive columns per lane and stores 16
  // bytes of C per lane.
  if constexpr (PART) {
    // FP32 partials straight from the accumulators: lane l holds columns
    // 32 j + 8 g + 4 (l / 32) .. + 3 of row 32 i + l % 32 of its wave tile
    float *part = reinterpret_cast<float *>(C) + static_cast<uint64_t>(split) * M * ldc;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t m = m0 + wm * G::kBMW + 32u * i + (lane & 31u);
          const uint32_t n = n0 + wn * G::kBNW + 32u * j + 8u * g + 4u * (lane >> 5);
          if (m < M && n < N)
            *reinterpret_cast<f32x4 *>(part + static_cast<uint64_t>(m) * ldc + n) =
                f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        }
    return;
  }
  constexpr uint32_t kEpPitch = G::kEpPitch;
  constexpr uint32_t kLpr = G::kBNW / 8u;  // lanes per staged row on the way out
  constexpr uint32_t kRpr = 64u / kLpr;    // rows per read instruction
  float *ep = reinterpret_cast<float *>(lds) + wave * 64u * kEpPitch;
  const uint32_t m_lane = lane & 31u, n_lane = (lane >> 5) * 4u;
  const uint32_t r_lane = lane / kLpr, c_lane = (lane % kLpr) * 8u;
#pragma unroll
  for (int band = 0; band < (MI + 1) / 2; ++band) {
    const uint32_t band_rows = 2 * band + 1 < MI ? 64u : 32u;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int i = band * 2 + ii;
          if (i >= MI) continue;
          *reinterpret_cast<f32x4 *>(ep + (ii * 32u + m_lane) * kEpPitch + j * 32u + 8u * g + n_lane) =
              f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Rows of the band in batches of kBatch read-back rows: every LDS read of
    // a batch is issued before the first conversion. Bands inside M x n_out
    // skip the per-row bounds checks.
    constexpr uint32_t kBatch = 4;
    static_assert((64u / kRpr) % kBatch == 0 && (MI % 2 == 0 || (32u / kRpr) % kBatch == 0),
                  "whole batches in every band");
    const uint32_t iters = band_rows / kRpr;
    const uint32_t mb = m0 + wm * G::kBMW + band * 64u, nb0 = n0 + wn * G::kBNW;
    const bool inside = mb + band_rows <= M && nb0 + G::kBNW <= n_out;
#pragma unroll
    for (uint32_t rr0 = 0; rr0 < iters; rr0 += kBatch) {
      f32x4 lo[kBatch], hi[kBatch];
#pragma unroll
      for (uint32_t b = 0; b < kBatch; ++b) {
        const uint32_t r = (rr0 + b) * kRpr + r_lane;
        lo[b] = *reinterpret_cast<const f32x4 *>(ep + r * kEpPitch + c_lane);
        hi[b] = *reinterpret_cast<const f32x4 *>(ep + r * kEpPitch + c_lane + 4u);
      }
#pragma unroll
      for (uint32_t b = 0; b < kBatch; ++b) {
        const uint32_t r = (rr0 + b) * kRpr + r_lane;
        const uint32_t m = mb + r, n = nb0 + c_lane;
        // whole 16-byte chunks; the edge chunk below
        if (!inside && (m >= M || n + 8u > n_out)) continue;
        const u32x4 packed{cvt_pack<DT>(lo[b].x, lo[b].y), cvt_pack<DT>(lo[b].z, lo[b].w),
                           cvt_pack<DT>(hi[b].x, hi[b].y), cvt_pack<DT>(hi[b].z, hi[b].w)};
        uint16_t *dst = C + static_cast<uint64_t>(m) * ldc + n;
        if constexpr (RES) {
          // C = bf16(C + bf16(product)), element by element
          const u32x4 old = *reinterpret_cast<const u32x4 *>(dst);
          const float pr[8] = {lo[b].x, lo[b].y, lo[b].z, lo[b].w, hi[b].x, hi[b].y, hi[b].z, hi[b].w};
          const uint32_t ow[4] = {old.x, old.y, old.z, old.w};
          uint32_t nw[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            nw[q] = f32_to_bf16(bf16_to_f32(ow[q] & 0xffffu) + round_bf16(pr[2 * q])) |
                    (f32_to_bf16(bf16_to_f32(ow[q] >> 16) + round_bf16(pr[2 * q + 1])) << 16);
          *reinterpret_cast<u32x4 *>(dst) = u32x4{nw[0], nw[1], nw[2], nw[3]};
        } else if constexpr (C16)
          *reinterpret_cast<u32x4 *>(dst) = packed;
        else  // C rows 2-byte aligned: global memory runs in unaligned access mode on gfx950
          __builtin_memcpy(dst, &packed, 16);
      }
    }
    if constexpr (!C16) {
      // The partial chunk at C's right edge (n_out % 8 columns), once per
      // band by the wave whose columns hold it: lane = row of the band.
      const uint32_t nb = n0 + wn * G::kBNW, edge = n_out & ~7u, cnt = n_out & 7u;
      const uint32_t m = m0 + wm * G::kBMW + band * 64u + lane;
      if (cnt != 0 && edge >= nb && edge < nb + G::kBNW && lane < band_rows && m < M) {
        const float *src = ep + lane * kEpPitch + (edge - nb);
        uint16_t *dst = C + static_cast<uint64_t>(m) * ldc + edge;
#pragma unroll
        for (uint32_t e = 0; e < 7; ++e)
          if (e < cnt) dst[e] = static_cast<uint16_t>(cvt_pack<DT>(src[e], 0.0f));
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

}  // namespace dma
}  // namespace xpu

// Each [k][n] kernel also comes in an _edge form (EDGE: the last slice's
// fix-up for K % 8 != 0 or odd N), so that aligned shapes run code without it.
#define XPU_GEMM_DMA_VARIANT1(NAME, DT, MI, NJ, BK, S, P, D, MINB, C16, ODD, EDGE, WN)                      \
  extern "C" __global__ __launch_bounds__(256, MINB) void NAME(                                             \
      const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, uint16_t *__restrict__ C,               \
      uint32_t M, uint32_t N, uint32_t K, uint32_t kb, uint32_t ldc, uint32_t n_out) {                       \
    XPU_STAMP(xpu::kStampGemm);                                                                               \
    xpu::dma::body<DT, MI, NJ, BK, S, P, D, C16, ODD, false, false, false, EDGE, WN>(A, B, C, M, N, K, kb,   \
                                                                                      ldc, n_out);           \
  }
#define XPU_GEMM_DMA_VARIANT(NAME, DT, MI, NJ, BK, S, P, D, MINB, C16, ODD)        \
  XPU_GEMM_DMA_VARIANT1(NAME, DT, MI, NJ, BK, S, P, D, MINB, C16, ODD, false, 2) \
  XPU_GEMM_DMA_VARIANT1(NAME##_edge, DT, MI, NJ, BK, S, P, D, MINB, C16, ODD, true, 2)
// 1 x 4 wavefronts
#define XPU_GEMM_DMA_VARIANT_W4(NAME, DT, MI, NJ, BK, S, P, D, MINB, C16, ODD)     \
  XPU_GEMM_DMA_VARIANT1(NAME, DT, MI, NJ, BK, S, P, D, MINB, C16, ODD, false, 4) \
  XPU_GEMM_DMA_VARIANT1(NAME##_edge, DT, MI, NJ, BK, S, P, D, MINB, C16, ODD, true, 4)

// C = A W^T with W given [N][K] (BT) for the batched prompt projections, bf16,
// 16-byte aligned C; _res adds into C (residual)
#define XPU_GEMM_NT_VARIANT(NAME, MI, NJ, S, P, MINB, ODD, RES)                                   \
  extern "C" __global__ __launch_bounds__(256, MINB) void NAME(                               \
      const uint16_t *__restrict__ A, const uint16_t *__restrict__ W, uint16_t *__restrict__ C, \
      uint32_t M, uint32_t N, uint32_t K, uint32_t kb, uint32_t ldc, uint32_t n_out) {         \
    XPU_STAMP(xpu::kStampGemm);                                                                 \
    xpu::dma::body<xpu::kBf16, MI, NJ, 64, S, P, 2, true, ODD, true, RES>(A, W, C, M, N, K, kb, ldc, n_out); \
  }
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_nt_dma, 4, 4, 2, 4, 1, false, false)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_nt_res_dma, 4, 4, 2, 4, 1, false, true)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_odd_nt_dma, 4, 4, 2, 4, 1, true, false)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_odd_nt_res_dma, 4, 4, 2, 4, 1, true, true)
// 128 x 256 with three stages (two slices in flight)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_m128_nt_dma, 2, 4, 3, 4, 1, false, false)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_m128_nt_res_dma, 2, 4, 3, 4, 1, false, true)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_t128_nt_dma, 2, 2, 2, 2, 2, false, false)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_t128_nt_res_dma, 2, 2, 2, 2, 2, false, true)
// 128 x 64 ([n][k] weights only): outputs that leave compute units idle even
// with 128 x 128 tiles (a 1024-wide projection of a few thousand tokens).
// Its slices are short (8 MFMAs per wavefront), so four stages keep three
// slices in flight to cover the memory latency; groups of 4 slices (K past
// the last whole group reads zeros). 96 KiB of LDS: one block per CU.
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_n64_nt_dma, 2, 1, 4, 1, 1, false, false)
XPU_GEMM_NT_VARIANT(xpu_gemm_bf16_n64_nt_res_dma, 2, 1, 4, 1, 1, false, true)
// split K for outputs that leave most compute units idle even at 128 x 64
// (a short prompt's o_proj and down): FP32 partials of each K range (kb
// slices, a multiple of 4), added by xpu_gemm_splitk_reduce
extern "C" __global__ __launch_bounds__(256, 1) void xpu_gemm_bf16_n64_nt_part_dma(
    const uint16_t *__restrict__ A, const uint16_t *__restrict__ W, uint16_t *__restrict__ C, uint32_t M,
    uint32_t N, uint32_t K, uint32_t kb, uint32_t ldc, uint32_t n_out) {
  XPU_STAMP(xpu::kStampGemm);
  xpu::dma::body<xpu::kBf16, 2, 1, 64, 4, 1, 2, true, false, true, false, true>(A, W, C, M, N, K, kb, ldc, n_out);
}

// C (M x N bf16) from the FP32 partials P[splits][M][N] of the split-K GEMM,
// added in split order: C = bf16(y) or, with residual, bf16(C + bf16(y));
// N a multiple of 8, 8 outputs per thread, grid-stride.
extern "C" __global__ __launch_bounds__(256) void xpu_gemm_splitk_reduce(const float *__restrict__ P,
                                                                         uint16_t *__restrict__ C, uint32_t M,
                                                                         uint32_t N, uint32_t splits,
                                                                         uint32_t residual) {
  const uint64_t mn = static_cast<uint64_t>(M) * N, total = mn / 8u;
  for (uint64_t c = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < total;
       c += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const float4 *p = reinterpret_cast<const float4 *>(P + c * 8u);
    float4 lo = p[0], hi = p[1];
    for (uint32_t s = 1; s < splits; ++s) {
      const float4 a = p[s * (mn / 4u)], b = p[s * (mn / 4u) + 1];
      lo = float4{lo.x + a.x, lo.y + a.y, lo.z + a.z, lo.w + a.w};
      hi = float4{hi.x + b.x, hi.y + b.y, hi.z + b.z, hi.w + b.w};
    }
    const float y[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    uint16_t *dst = C + c * 8u;
    const xpu::u32x4 old = residual ? *reinterpret_cast<const xpu::u32x4 *>(dst) : xpu::u32x4{0, 0, 0, 0};
    const uint32_t ow[4] = {old.x, old.y, old.z, old.w};
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = y[2 * q + e];
        h[e] = residual ? xpu::f32_to_bf16(xpu::bf16_to_f32((ow[q] >> (16 * e)) & 0xffffu) + xpu::round_bf16(v))
                        : xpu::f32_to_bf16(v);
      }
      w[q] = h[0] | (h[1] << 16);
    }
    *reinterpret_cast<xpu::u32x4 *>(dst) = xpu::u32x4{w[0], w[1], w[2], w[3]};
  }
}

// C (M x N, bf16 or fp16, row stride ldc, any alignment) from the FP32
// partials P[splits][M][pitch] of the [k][n] split-K GEMM (pitch >= N, a
// multiple of 4), added in split order and rounded to nearest even; each
// thread takes 4 consecutive columns of one row, grid-stride.
extern "C" __global__ __launch_bounds__(256) void xpu_gemm_splitk_reduce_any(
    const float *__restrict__ P, uint16_t *__restrict__ C, uint32_t M, uint32_t N, uint32_t pitch, uint32_t ldc,
    uint32_t splits, uint32_t dtype) {
  const uint32_t groups = (N + 3u) / 4u;
  const uint64_t total = static_cast<uint64_t>(M) * groups, split4 = static_cast<uint64_t>(M) * pitch / 4u;
  for (uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < total;
       g += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint32_t m = static_cast<uint32_t>(g / groups), n = static_cast<uint32_t>(g % groups) * 4u;
    const float4 *p = reinterpret_cast<const float4 *>(P + static_cast<uint64_t>(m) * pitch + n);
    float4 acc = p[0];
    for (uint32_t s = 1; s < splits; ++s) {
      const float4 v = p[s * split4];
      acc = float4{acc.x + v.x, acc.y + v.y, acc.z + v.z, acc.w + v.w};
    }
    const float y[4] = {acc.x, acc.y, acc.z, acc.w};
    uint16_t *dst = C + static_cast<uint64_t>(m) * ldc + n;
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e)
      if (n + e < N) dst[e] = static_cast<uint16_t>(dtype ? xpu::f32_to_fp16(y[e]) : xpu::f32_to_bf16(y[e]));
  }
}

// The same reduction fused with the RMSNorm of the rows it completes (the
// next kernel's input in the Qwen3 prompt): one wavefront per row, lane l
// holding columns 512 c + 8 l .. + 7 (N = 512 or 1024); row = bf16(C +
// bf16(y)) (or bf16(y)) as xpu_gemm_splitk_reduce writes it, then Xn =
// bf16(w * bf16(row * (1 / sqrt(sum(row^2) / N + eps)))) with the sum of
// squares in the order of xpu_q3_pf_rmsnorm (per-lane slots over the
// chunks, fold8, 64-lane butterfly). The partials of up to 4 splits, both
// chunks and the residual are loaded before any addition; the splits are
// still added in order. Grid ceil(M / 4) blocks of 256.
extern "C" __global__ __launch_bounds__(256) void xpu_gemm_splitk_reduce_norm(
    const float *__restrict__ P, uint16_t *__restrict__ C, uint32_t M, uint32_t N, uint32_t splits,
    uint32_t residual, const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ Xn, float eps) {
  constexpr uint32_t kChunks = 2, kBatch = 4;  // N <= 1024; splits loaded 4 at a time
  const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
  if (row >= M) return;  // whole wavefronts
  const uint32_t nc = N / 512u;
  const uint64_t mn4 = static_cast<uint64_t>(M) * N / 4u;  // one split, in float4
  const float4 *p[kChunks];
  xpu::u32x4 old[kChunks];
  float4 lo[kChunks], hi[kChunks];
#pragma unroll
  for (uint32_t c = 0; c < kChunks; ++c) {
    const uint32_t cc = c < nc ? c : 0u;  // a chunk past N re-reads chunk 0 (not used)
    const uint64_t off = static_cast<uint64_t>(row) * N + cc * 512u + lane * 8u;
    p[c] = reinterpret_cast<const float4 *>(P + off);
    old[c] = residual ? *reinterpret_cast<const xpu::u32x4 *>(C + off) : xpu::u32x4{0, 0, 0, 0};
    lo[c] = p[c][0];
    hi[c] = p[c][1];
  }
  for (uint32_t s0 = 1; s0 < splits; s0 += kBatch) {
    float4 a[kBatch][kChunks], b[kBatch][kChunks];
#pragma unroll
    for (uint32_t k = 0; k < kBatch; ++k) {
      const uint64_t s = min(s0 + k, splits - 1u);  // past the last split: re-read it (not added)
#pragma unroll
      for (uint32_t c = 0; c < kChunks; ++c) {
        a[k][c] = p[c][s * mn4];
        b[k][c] = p[c][s * mn4 + 1];
      }
    }
#pragma unroll
    for (uint32_t k = 0; k < kBatch; ++k) {
      if (s0 + k >= splits) break;  // uniform
#pragma unroll
      for (uint32_t c = 0; c < kChunks; ++c) {
        lo[c] = float4{lo[c].x + a[k][c].x, lo[c].y + a[k][c].y, lo[c].z + a[k][c].z, lo[c].w + a[k][c].w};
        hi[c] = float4{hi[c].x + b[k][c].x, hi[c].y + b[k][c].y, hi[c].z + b[k][c].z, hi[c].w + b[k][c].w};
      }
    }
  }
  xpu::u32x4 xc[kChunks];
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (uint32_t c = 0; c < kChunks; ++c) {
    if (c >= nc) break;  // uniform
    const float y[8] = {lo[c].x, lo[c].y, lo[c].z, lo[c].w, hi[c].x, hi[c].y, hi[c].z, hi[c].w};
    const uint32_t ow[4] = {old[c].x, old[c].y, old[c].z, old[c].w};
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = y[2 * q + e];
        h[e] = residual ? xpu::f32_to_bf16(xpu::bf16_to_f32((ow[q] >> (16 * e)) & 0xffffu) + xpu::round_bf16(v))
                        : xpu::f32_to_bf16(v);
      }
      w[q] = h[0] | (h[1] << 16);
    }
    xc[c] = xpu::u32x4{w[0], w[1], w[2], w[3]};
    *reinterpret_cast<xpu::u32x4 *>(C + static_cast<uint64_t>(row) * N + c * 512u + lane * 8u) = xc[c];
    float f[8];
    xpu::unpack8<xpu::kBf16>(xc[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(f[e], f[e], acc[e]);
  }
  const float ss = xpu::wave_butterfly(xpu::fold8(acc));
  const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(N) + eps);
#pragma unroll
  for (uint32_t c = 0; c < kChunks; ++c) {
    if (c >= nc) break;
    const uint64_t off = static_cast<uint64_t>(row) * N + c * 512u + lane * 8u;
    float xf[8], wf[8];
    xpu::unpack8<xpu::kBf16>(xc[c], xf);
    xpu::unpack8<xpu::kBf16>(*reinterpret_cast<const xpu::u32x4 *>(norm_w + c * 512u + lane * 8u), wf);
    uint32_t code[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) code[e] = xpu::f32_to_bf16(wf[e] * xpu::round_bf16(xf[e] * scale));
    *reinterpret_cast<xpu::u32x4 *>(Xn + off) = xpu::u32x4{code[0] | (code[1] << 16), code[2] | (code[3] << 16),
                                                         code[4] | (code[5] << 16), code[6] | (code[7] << 16)};
  }
}

// 256 x 256: BK = 64, two stages, barrier after 4 MFMAs of a slice's last
// k-step, each slice's DMA spread over two k-steps; _odd for an odd number
// of 64-deep slices
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_dma, xpu::kBf16, 4, 4, 64, 2, 4, 2, 1, true, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_dma, xpu::kFp16, 4, 4, 64, 2, 4, 2, 1, true, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_dmau, xpu::kBf16, 4, 4, 64, 2, 4, 2, 1, false, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_dmau, xpu::kFp16, 4, 4, 64, 2, 4, 2, 1, false, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_odd_dma, xpu::kBf16, 4, 4, 64, 2, 4, 2, 1, true, true)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_odd_dma, xpu::kFp16, 4, 4, 64, 2, 4, 2, 1, true, true)
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_odd_dmau, xpu::kBf16, 4, 4, 64, 2, 4, 2, 1, false, true)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_odd_dmau, xpu::kFp16, 4, 4, 64, 2, 4, 2, 1, false, true)
// 128 x 256 (one block per compute unit: 96 KiB of stages, 132 KiB of
// epilogue staging)
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_m128_dma, xpu::kBf16, 2, 4, 64, 2, 4, 2, 1, true, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_m128_dma, xpu::kFp16, 2, 4, 64, 2, 4, 2, 1, true, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_m128_dmau, xpu::kBf16, 2, 4, 64, 2, 4, 2, 1, false, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_m128_dmau, xpu::kFp16, 2, 4, 64, 2, 4, 2, 1, false, false)

// 224 x 256 (1 x 4 wavefronts of 224 x 64), with odd-slice forms as the 256 x 256 tile
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_bf16_m224_dma, xpu::kBf16, 7, 2, 64, 2, 4, 2, 1, true, false)
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_fp16_m224_dma, xpu::kFp16, 7, 2, 64, 2, 4, 2, 1, true, false)
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_bf16_m224_dmau, xpu::kBf16, 7, 2, 64, 2, 4, 2, 1, false, false)
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_fp16_m224_dmau, xpu::kFp16, 7, 2, 64, 2, 4, 2, 1, false, false)
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_bf16_m224_odd_dma, xpu::kBf16, 7, 2, 64, 2, 4, 2, 1, true, true)
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_fp16_m224_odd_dma, xpu::kFp16, 7, 2, 64, 2, 4, 2, 1, true, true)
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_bf16_m224_odd_dmau, xpu::kBf16, 7, 2, 64, 2, 4, 2, 1, false, true)
XPU_GEMM_DMA_VARIANT_W4(xpu_gemm_fp16_m224_odd_dmau, xpu::kFp16, 7, 2, 64, 2, 4, 2, 1, false, true)
// 128 x 128 (two blocks per compute unit: 64 KiB of stages, 68 KiB of
// epilogue staging); the barrier after 2 of the k-step's 4 MFMAs
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_t128_dma, xpu::kBf16, 2, 2, 64, 2, 2, 2, 2, true, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_t128_dma, xpu::kFp16, 2, 2, 64, 2, 2, 2, 2, true, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_bf16_t128_dmau, xpu::kBf16, 2, 2, 64, 2, 2, 2, 2, false, false)
XPU_GEMM_DMA_VARIANT(xpu_gemm_fp16_t128_dmau, xpu::kFp16, 2, 2, 64, 2, 2, 2, 2, false, false)

// Split K for [k][n] products that leave most compute units idle even with
// 128 x 128 tiles (a small output with a long reduction): FP32 partials of
// each K range (kb slices, a multiple of 2), added by
// xpu_gemm_splitk_reduce_any; _edge as for the whole-K kernels.
#define XPU_GEMM_PART_KN(NAME, DT, EDGE)                                                                   \
  extern "C" __global__ __launch_bounds__(256, 2) void NAME(                                               \
      const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, uint16_t *__restrict__ C, uint32_t M, \
      uint32_t N, uint32_t K, uint32_t kb, uint32_t ldc, uint32_t n_out) {                                  \
    XPU_STAMP(xpu::kStampGemm);                                                                             \
    xpu::dma::body<DT, 2, 2, 64, 2, 2, 2, true, false, false, false, true, EDGE>(A, B, C, M, N, K, kb, ldc, \
                                                                                n_out);                    \
  }
XPU_GEMM_PART_KN(xpu_gemm_bf16_t128_part_dma, xpu::kBf16, false)
XPU_GEMM_PART_KN(xpu_gemm_bf16_t128_part_dma_edge, xpu::kBf16, true)
XPU_GEMM_PART_KN(xpu_gemm_fp16_t128_part_dma, xpu::kFp16, false)
XPU_GEMM_PART_KN(xpu_gemm_fp16_t128_part_dma_edge, xpu::kFp16, true)

// dst[r][c] = src[r * src_ld + c] for c < cols, 0 for cols <= c < dst_cols
// (dst_cols % 8 == 0, dst 16-byte aligned): the zero padding of the
// reference's host GEMM setup (gemm.cpp:75-85) done on the device, so rows
// of the copy are 16-byte aligned. xpu_gemm does not use it (its kernels
// read unpadded operands); it prepares operands for a measurement of the
// reference's own method (pad once at setup, then time the GEMM). One thread per 8 destination elements.
// src only needs 2-byte alignment: a whole chunk is one 16-byte load at a
// 2-byte aligned address (global memory runs in unaligned access mode on
// gfx950). The chunk holding the row's end is read element by element, so
// no load reaches past the last element of a row.
namespace xpu {
// One 16-byte destination chunk (8 elements from column c0 of src row p).
XPU_DEVICE xpu::u32x4 pad_chunk(const uint16_t *__restrict__ p, uint32_t c0, uint32_t cols) {
  if (c0 + 8u <= cols) {
    xpu::u32x4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
  }
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = c0 + 2 * q < cols ? p[2 * q] : 0u;
    const uint32_t hi = c0 + 2 * q + 1 < cols ? p[2 * q + 1] : 0u;
    w[q] = lo | (hi << 16);
  }
  return xpu::u32x4{w[0], w[1], w[2], w[3]};
}

// Blocks block0 .. block0 + nblocks - 1 of the grid copy one matrix; each
// thread takes kPadUnroll chunks a grid stride apart per step, all loads
// issued before the stores.
constexpr int kPadUnroll = 4;
XPU_DEVICE void pad_rows(const uint16_t *__restrict__ src, uint64_t src_ld, uint32_t rows, uint32_t cols,
                         uint16_t *__restrict__ dst, uint32_t dst_cols, uint32_t block0, uint32_t nblocks) {
  const uint64_t chunks_per_row = dst_cols / 8u;
  const uint64_t total = static_cast<uint64_t>(rows) * chunks_per_row;
  const uint64_t stride = static_cast<uint64_t>(nblocks) * blockDim.x;
  for (uint64_t idx = static_cast<uint64_t>(blockIdx.x - block0) * blockDim.x + threadIdx.x; idx < total;
       idx += kPadUnroll * stride) {
    xpu::u32x4 v[kPadUnroll];
#pragma unroll
    for (int u = 0; u < kPadUnroll; ++u) {
      const uint64_t i = idx + u * stride;
      if (i < total) {
        const uint64_t r = i / chunks_per_row;
        const uint32_t c0 = static_cast<uint32_t>(i % chunks_per_row) * 8u;
        v[u] = pad_chunk(src + r * src_ld + c0, c0, cols);
      }
    }
#pragma unroll
    for (int u = 0; u < kPadUnroll; ++u) {
      const uint64_t i = idx + u * stride;
      if (i < total) *reinterpret_cast<xpu::u32x4 *>(dst + (i / chunks_per_row) * dst_cols + (i % chunks_per_row) * 8u) = v[u];
    }
  }
}
}  // namespace xpu

extern "C" __global__ __launch_bounds__(256) void xpu_pad_rows(const uint16_t *__restrict__ src, uint64_t src_ld,
                                                               uint32_t rows, uint32_t cols,
                                                               uint16_t *__restrict__ dst, uint32_t dst_cols) {
  xpu::pad_rows(src, src_ld, rows, cols, dst, dst_cols, 0, gridDim.x);
}
