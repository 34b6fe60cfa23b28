// Causal attention of a prompt chunk on MFMA (the GEMM prompt mode of the
// Qwen3 engine): queries p0 .. p0 + T - 1 of every query head against cache
// positions 0 .. own position, K and V read from the chunk-major caches
// [kv_head][16][max_seq][8] that xpu_q3_pf_rope_cache filled.
//
// Rounding: s = bf16(bf16(q . k) * scale) as in the decode attention
// (qwen3/kernels.hpp:157-192 as restated by the oracle), then an online
// softmax in one sweep over the key tiles, as the reference's own kernel
// runs it (FP32 running max and sum, kernels.hpp:174-190): per query a
// reference max m, p = bf16(exp(s - m)) as the P.V MFMA operand, the FP32
// sum of exp(s - m) and the FP32 output rescaled by exp(m_old - m_new) when
// a score passes m by more than 8 ln 2 (so p <= 256 and rescales are rare),
// and out = bf16(O / sum) at the end. The decode path (bit-exact
// against the CPU oracle) instead rounds p = bf16(exp(s - M) / sum) with
// the final max M; the exponential here is the hardware's exp2 (v_exp_f32
// of s log2 e - m log2 e; the reference's kernel uses the device exp too),
// and the FP32 sums run in the MFMA's order. So results agree with the
// decode path to rounding (about half the output codes equal, the rest one
// bf16 step away), not bitwise.
//
// Block: one kv head, 4 wavefronts of 32 query rows each: G query heads x
// U query sub-tiles x H key halves (G U H = 4; QT = 32 U queries). Key
// tiles of 64 positions: half h takes tiles h, h + H, ..., so the causal
// work of a block is spread over its waves, and the halves merge their
// (max, sum, FP32 partial output) through LDS after the sweep, in half
// order. Tiles are staged by LDS-DMA, two stages
// of H tile slots of K [16 chunks][64 keys][8] and V [64 keys][16 chunks,
// XOR-swizzled][8]. Per wave and tile:
// S^T = K Q^T as two 32 x 32 MFMA tiles (A: K rows from LDS, B: the wave's Q
// rows held in registers), so each lane holds 32 scores of one query; O^T
// += V^T P^T with the lane's own bf16 p as the B operand and V^T fragments
// from two ds_read_b64_tr_b16 whose row blocks follow the accumulator's key
// order (4 keys of each half-wave, then 4 more 8 keys on). Keys past the
// block's last query read as zero (out-of-range DMA offsets); keys past a
// query's own position are masked before the max, the sum and p.
#include "device_common.hpp"

#include <type_traits>

namespace xpu {
namespace pfa {

using dma::bf16x8;
using dma::f32x16;
using dma::lds_s16x4;

constexpr uint32_t kKeys = 64;          // keys per tile
constexpr uint32_t kStage = 32768;      // K (16 KiB) then V (16 KiB)
constexpr uint32_t kOob = dma::kOob;

XPU_DEVICE f32x16 mfma_bf16(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

template <int G, int H>
XPU_DEVICE void prefill_attention(const uint16_t *__restrict__ Q, const uint16_t *__restrict__ kcache,
                                  const uint16_t *__restrict__ vcache, uint16_t *__restrict__ out, uint32_t p0,
                                  uint32_t T, uint32_t heads, uint32_t kv_heads, uint32_t max_seq, float scale) {
  static_assert((G == 1 || G == 2 || G == 4) && (H == 1 || H == 2) && 4 % (G * H) == 0,
                "4 wavefronts: G query heads x U query sub-tiles x H key halves");
  constexpr uint32_t U = 4u / (G * H), QT = 32u * U, kSlots = G * U;  // waves per half
  __shared__ __align__(1024) uint8_t lds[2 * H * kStage];
  __shared__ float merge[H][kSlots][2][64];  // (max, sum) of each half's waves
  const uint32_t tid = threadIdx.x, lane = tid & 63u, hh = lane >> 5;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t half = wave / kSlots, slot = wave % kSlots;
  // heaviest query tiles first: block b takes tile n_qt - 1 - b / kv_heads
  const uint32_t n_qt = (T + QT - 1) / QT;
  const uint32_t qt = n_qt - 1u - blockIdx.x / kv_heads, kvh = blockIdx.x % kv_heads;
  const uint32_t head = kvh * G + slot % G;
  const uint32_t t0 = qt * QT + 32u * (slot / G);  // the wave's first query
  const uint32_t t = t0 + (lane & 31u);
  const uint32_t qpos = p0 + t;
  const uint32_t n_valid = p0 + min(qt * QT + QT, T);  // keys of the block: 0 .. n_valid - 1
  const uint32_t n_tiles = (n_valid + kKeys - 1) / kKeys;
  const uint32_t wave_tiles = t0 < T ? (p0 + min(t0 + 31u, T - 1u)) / kKeys + 1u : 0u;

  // the lane's Q row (B operand of S^T): dims 16 ks + 8 hh .. + 7
  u32x4 qf[8];
  {
    const uint16_t *qrow = Q + (static_cast<uint64_t>(min(t, T - 1u)) * heads + head) * kHeadDim;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const u32x4 *>(qrow + (2u * ks + hh) * 8u);
  }

  const uint64_t head_base = static_cast<uint64_t>(kvh) * max_seq * kHeadDim;
  const i32x4 rk = rsrc(kcache + head_base, static_cast<int64_t>(max_seq) * kHeadDim * 2);
  const i32x4 rv = rsrc(vcache + head_base, static_cast<int64_t>(max_seq) * kHeadDim * 2);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));

  // DMA of key tile `tile` into slot `slot_of` of a stage: K chunk c (wave
  // 4 j) = 64 keys x 16 bytes; V rows 4 i .. 4 i + 3, lane -> (key 4 i +
  // lane / 16, physical chunk lane % 16 = logical chunk ^ b_swz(key))
  auto issue_tile = [&](uint32_t tile, uint32_t sb, bool with_v) {
    const uint32_t k0 = tile * kKeys;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t c = wave * 4u + j, key = k0 + lane;
      dma16(sb + c * 1024u, rk, key < n_valid ? (c * max_seq + key) * 16u : kOob);
    }
    if (with_v) {
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t i = wave * 4u + j, key = k0 + 4u * i + (lane >> 4);
        const uint32_t c = (lane & 15u) ^ dma::b_swz(lane >> 4);
        dma16(sb + 16384u + i * 1024u, rv, key < n_valid ? (c * max_seq + key) * 16u : kOob);
      }
    }
  };
  // step i of a sweep: tiles H i .. H i + H - 1 into stage i % 2
  const uint32_t n_steps = (n_tiles + H - 1) / H;
  auto issue = [&](uint32_t step, bool with_v) {
#pragma unroll
    for (uint32_t h = 0; h < H; ++h)
      if (H * step + h < n_tiles) issue_tile(H * step + h, lds0 + ((step & 1u) * H + h) * kStage, with_v);
  };

  // S^T of a tile: s[kt] holds keys 32 kt + 8 (r / 4) + 4 hh + r % 4 of the
  // lane's query (r = register), scaled and rounded as the decode path does
  auto scores = [&](uint32_t kb, f32x16 (&s)[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
#pragma unroll
    for (uint32_t ks = 0; ks < 8; ++ks)
#pragma unroll
      for (uint32_t kt = 0; kt < 2; ++kt) {
        const u32x4 kf = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(
            kb + ((2u * ks + hh) * kKeys + 32u * kt + (lane & 31u)) * 16u);
        s[kt] = mfma_bf16(kf, qf[ks], s[kt]);
      }
    // bf16(bf16(q . k) * scale), the roundings by v_cvt_pk_bf16_f32 (RNE,
    // the bits of f32_to_bf16 for finite values)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const uint32_t w = dma::cvt_pack<kBf16>(s[kt][r], s[kt][r + 1]);
        const uint32_t w2 = dma::cvt_pack<kBf16>(lo16<kBf16>(w) * scale, hi16<kBf16>(w) * scale);
        s[kt][r] = lo16<kBf16>(w2);
        s[kt][r + 1] = hi16<kBf16>(w2);
      }
  };
  // Masks: key 32 kt + 8 (r / 4) + 4 hh + r % 4 of the tile is valid for the
  // lane's query when that offset <= qpos - (first key + 4 hh). Only the
  // tiles that reach past the wave's first query position (the diagonal
  // ones) have invalid keys; there the invalid scores become -inf, which
  // leaves the max alone and whose exponentials are 0.
  const float ninf = -__builtin_inff();
  auto mask_scores = [&](uint32_t tile, f32x16 (&s)[2]) {
    if (__builtin_expect(tile * kKeys + kKeys - 1u <= p0 + t0, 1)) return;  // wave-uniform
    const int32_t lim = static_cast<int32_t>(qpos) - static_cast<int32_t>(tile * kKeys + 4u * hh);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (32 * kt + 8 * (r / 4) + (r % 4) > lim) s[kt][r] = ninf;
  };

  // body(tile, stage byte address of the tile) for the wave's tiles:
  // H step + half
  auto sweep = [&](bool with_v, auto &&body) {
    issue(0, with_v);
    for (uint32_t i = 0; i < n_steps; ++i) {
      wait_vmcnt<0>();
      __syncthreads();
      if (i + 1 < n_steps) issue(i + 1, with_v);
      const uint32_t tile = H * i + half, sb = lds0 + ((i & 1u) * H + half) * kStage;
      if (tile < wave_tiles) body(tile, sb);
    }
    __syncthreads();  // the next sweep's first DMA reuses stage 0
  };

  // One sweep, online softmax: per lane (query) a reference max m, the FP32
  // sum of exp(s - m) and the FP32 O^T columns, both rescaled by
  // exp(m_old - m_new) when m moves; p = bf16(exp(s - m)) feeds the P.V
  // MFMA, and the output is divided by the sum at the end. The two
  // half-waves of a query (lanes l and l ^ 32) merge each tile's max, so
  // they share m.
  constexpr float kLog2e = 1.44269504088896340736f;
  constexpr float kLazy = 5.54517744447956247533f;  // 8 ln 2
  auto exp_hw = [&](float x) { return __builtin_amdgcn_exp2f(x * kLog2e); };
  // exp(s - m) as exp2(s log2 e - m log2 e), one FMA per score with
  // neg_ml = -m log2 e formed once per tile
  auto exp_shift = [&](float sc, float neg_ml) {
    return __builtin_amdgcn_exp2f(__builtin_fmaf(sc, kLog2e, neg_ml));
  };
  float mx = ninf, sum = 0.0f;
  // O^T tile dt: dims 32 dt + 8 (r / 4) + 4 hh + r % 4 of the lane's query
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
  // tr-read address pieces: lane i of a 16-lane group gives row (i & 15) / 4
  // of the group's 4-row block, dims 16 ((lane / 16) % 2) + 4 (lane % 4)
  const uint32_t tr_row = (lane & 15u) >> 2;
  const uint32_t tr_chunk = 2u * ((lane >> 4) & 1u) + ((lane & 3u) >> 1);
  const uint32_t tr_half = 8u * (lane & 1u);
  sweep(true, [&](uint32_t tile, uint32_t sb) {
    f32x16 s[2];
    scores(sb, s);
    mask_scores(tile, s);
    float tmax = ninf;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[kt][r]);
    // the reference max m moves only when a score exceeds it by more than
    // 8 ln 2, so exp(s - m) <= 256 (exact in scale for bf16 p and the FP32
    // sums) and the rescale of o and sum is rare after the first tiles
    const float m_tile = fmaxf(tmax, xor32_f(tmax));
    const bool grow = m_tile > mx + kLazy;  // mx = -inf: any valid key
    if (__builtin_amdgcn_ballot_w64(grow)) {  // wave-uniform: some query's reference moves
      const float m_new = grow ? m_tile : mx;
      // no valid key before (mx = -inf): o and sum are still 0
      const float a = mx == ninf ? 0.0f : exp_hw(mx - m_new);
      sum *= a;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= a;
      mx = m_new;
    }
    // no valid key yet (m = -inf): every score is -inf and gives p = 0
    const float neg_ml = mx == ninf ? 0.0f : -mx * kLog2e;
    // p = bf16(exp(s - m)): the packing conversion is the rounding; masked
    // scores give 0
    uint32_t pk[2][8];
    float part = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float e0 = exp_shift(s[kt][r], neg_ml), e1 = exp_shift(s[kt][r + 1], neg_ml);
        part = part + e0 + e1;
        pk[kt][r / 2] = dma::cvt_pack<kBf16>(e0, e1);
      }
    sum += part;
    const uint32_t vb = sb + 16384u;
#pragma unroll
    for (uint32_t ks = 0; ks < 4; ++ks) {
      const uint32_t kt = ks / 2, rb = 4u * (ks % 2);
      const u32x4 pf = {pk[kt][rb], pk[kt][rb + 1], pk[kt][rb + 2], pk[kt][rb + 3]};
#pragma unroll
      for (uint32_t dt = 0; dt < 4; ++dt) {
        u32x4 vf;
#pragma unroll
        for (uint32_t h2 = 0; h2 < 2; ++h2) {
          const uint32_t row = 16u * ks + 4u * hh + 8u * h2 + tr_row;
          const uint32_t addr = vb + row * 256u + 16u * ((4u * dt + tr_chunk) ^ dma::b_swz(tr_row)) + tr_half;
          const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(addr)));
          if (h2 == 0) {
            vf.x = v.x;
            vf.y = v.y;
          } else {
            vf.z = v.x;
            vf.w = v.y;
          }
        }
        o[dt] = mfma_bf16(vf, pf, o[dt]);
      }
    }
  });
  sum = sum + xor32_f(sum);  // the query's two half-waves (same m)

  if constexpr (H > 1) {
    // half h > 0 leaves (m, sum) and its partial O^T in LDS (the stage
    // memory is idle after the sweep); half 0 merges them in half order
    float *po = reinterpret_cast<float *>(lds);
    if (half > 0) {
      merge[half][slot][0][lane] = mx;
      merge[half][slot][1][lane] = sum;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) po[(((half - 1) * kSlots + slot) * 64 + dt * 16 + r) * 64 + lane] = o[dt][r];
    }
    __syncthreads();
    if (half > 0) return;
#pragma unroll
    for (uint32_t h = 1; h < H; ++h) {
      const float m2 = merge[h][slot][0][lane], s2 = merge[h][slot][1][lane];
      const float m_row = fmaxf(mx, m2);
      const float a = mx == ninf ? 0.0f : exp_hw(mx - m_row);
      const float b = m2 == ninf ? 0.0f : exp_hw(m2 - m_row);
      sum = sum * a + s2 * b;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          o[dt][r] = o[dt][r] * a + po[(((h - 1) * kSlots + slot) * 64 + dt * 16 + r) * 64 + lane] * b;
      mx = m_row;
    }
  }
  // position 0 is a key of every query, so sum >= 1 for a query in range
  const float inv = 1.0f / sum;
  if (t < T && t0 < T) {
    uint16_t *orow = out + (static_cast<uint64_t>(t) * heads + head) * kHeadDim;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x2 w = {dma::cvt_pack<kBf16>(o[dt][4 * q] * inv, o[dt][4 * q + 1] * inv),
                         dma::cvt_pack<kBf16>(o[dt][4 * q + 2] * inv, o[dt][4 * q + 3] * inv)};
        *reinterpret_cast<u32x2 *>(orow + 32u * dt + 8u * q + 4u * hh) = w;
      }
  }
}

}  // namespace pfa
}  // namespace xpu

// grid: ceil(T / QT) * kv_heads blocks of 256 threads (QT = 64 for G = 1,
// 32 for G = 2 and 4); heads = G kv_heads; A: [T][heads][128]
#define XPU_PF_ATTN_MFMA(G, H)                                                                                \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_attention_mfma_g##G(                           \
      const uint16_t *__restrict__ Q, const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache, \
      uint16_t *__restrict__ A, uint32_t p0, uint32_t T, uint32_t heads, uint32_t kv_heads, uint32_t max_seq,  \
      float scale) {                                                                                          \
    xpu::pfa::prefill_attention<G, H>(Q, kcache, vcache, A, p0, T, heads, kv_heads, max_seq, scale);         \
  }
XPU_PF_ATTN_MFMA(1, 2)
XPU_PF_ATTN_MFMA(2, 2)
XPU_PF_ATTN_MFMA(4, 1)
