// Qwen3 decode building blocks for gfx950 (head_dim 128): block RMSNorm,
// per-head QK-norm + RoPE, single-query attention, argmax reduction.
//
// Rounding points follow transformers' eager bf16 Qwen3 (the arithmetic
// behind the reference oracle qwen3/reference.py); operations follow the
// reference kernels qwen3/kernels.hpp:36-246. Summation orders are the
// canonical ones also evaluated by the CPU oracle (oracle/oracle.c).
#pragma once

#include "gemv_core.hpp"

namespace xpu {

constexpr uint32_t kHeadDim = 128;
constexpr uint32_t kAttnChunk = 4096;  // positions per softmax / P.V chunk

// Block-cooperative RMSNorm of x[0..W) into LDS buffer xs (bf16 codes,
// zero-padded to a multiple of 512). red is one float of LDS.
// qwen3/kernels.hpp:43-54 with transformers rounding:
// out = bf16(w * bf16(x * (1 / sqrt(sum(x^2) / W + eps)))).
// Generic form: any width, any alignment.
XPU_DEVICE void block_rmsnorm(uint16_t *xs, const uint16_t *__restrict__ x,
                              const uint16_t *__restrict__ w, uint32_t W, float eps, float *red) {
  const uint32_t wpad = (W + 511u) & ~511u;
  stage_vector<false>(xs, x, W, wpad);
  __syncthreads();
  if (threadIdx.x < 64) {
    const uint32_t lane = threadIdx.x;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t j = 0; j < wpad; j += 512u) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(xs + j + lane * 8u);
      float f[8];
      unpack8<kBf16>(v, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(f[e], f[e], acc[e]);
    }
    const float ss = wave_butterfly(fold8(acc));
    if (lane == 0) red[0] = 1.0f / __builtin_sqrtf(ss / static_cast<float>(W) + eps);
  }
  __syncthreads();
  const float scale = red[0];
  for (uint32_t i = threadIdx.x; i < W; i += blockDim.x)
    xs[i] = static_cast<uint16_t>(
        f32_to_bf16(bf16_to_f32(w[i]) * round_bf16(bf16_to_f32(xs[i]) * scale)));
  __syncthreads();
}

// Same result for 16-byte aligned x, w with W a multiple of 8 and
// W <= 8 * 8 * blockDim: x and the gains are fetched together with 16-byte
// loads (one memory round trip) and kept in registers.
XPU_DEVICE void block_rmsnorm_vec(uint16_t *xs, const uint16_t *__restrict__ x,
                                  const uint16_t *__restrict__ w, uint32_t W, float eps, float *red) {
  constexpr int kGroups = 8;
  const uint32_t wpad = (W + 511u) & ~511u;
  u32x4 xv[kGroups], wv[kGroups];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const uint32_t i = (threadIdx.x + q * blockDim.x) * 8u;
    if (i < W) {
      xv[q] = *reinterpret_cast<const u32x4 *>(x + i);
      wv[q] = *reinterpret_cast<const u32x4 *>(w + i);
    } else {
      xv[q] = u32x4{0, 0, 0, 0};
      wv[q] = u32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const uint32_t i = (threadIdx.x + q * blockDim.x) * 8u;
    if (i < wpad) *reinterpret_cast<u32x4 *>(xs + i) = xv[q];
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const uint32_t lane = threadIdx.x;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t j = 0; j < wpad; j += 512u) {
      float f[8];
      unpack8<kBf16>(*reinterpret_cast<const u32x4 *>(xs + j + lane * 8u), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(f[e], f[e], acc[e]);
    }
    const float ss = wave_butterfly(fold8(acc));
    if (lane == 0) red[0] = 1.0f / __builtin_sqrtf(ss / static_cast<float>(W) + eps);
  }
  __syncthreads();
  const float scale = red[0];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const uint32_t i = (threadIdx.x + q * blockDim.x) * 8u;
    if (i < W) {
      float xf[8], wf[8];
      unpack8<kBf16>(xv[q], xf);
      unpack8<kBf16>(wv[q], wf);
      uint32_t c[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) c[e] = f32_to_bf16(wf[e] * round_bf16(xf[e] * scale));
      *reinterpret_cast<u32x4 *>(xs + i) =
          u32x4{c[0] | (c[1] << 16), c[2] | (c[3] << 16), c[4] | (c[5] << 16), c[6] | (c[7] << 16)};
    }
  }
  __syncthreads();
}

// One wavefront: RMSNorm over a 128-wide head then rotate-half RoPE
// (qwen3/kernels.hpp:76-124 with transformers rounding:
// out[i] = bf16(bf16(n[i] * cos[i]) + bf16(rot[i] * sin[i])), rot = (-n[64:], n[:64])).
// Lanes 0..15 hold 8 consecutive entries each; lanes 16..63 contribute
// zeros to the sum. normed_out (optional) receives the normed, un-rotated
// codes; roped_out the rotated ones.
XPU_DEVICE void head_norm_rope(const uint16_t *src, const uint16_t *__restrict__ w,
                               const uint16_t *__restrict__ cos_row,
                               const uint16_t *__restrict__ sin_row, float eps,
                               uint16_t *normed_out, uint16_t *roped_out) {
  const uint32_t lane = lane_id();
  const bool active = lane < 16;
  float x[8];
  if (active) {
    unpack8<kBf16>(*reinterpret_cast<const u32x4 *>(src + lane * 8u), x);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
  }
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(x[e], x[e], 0.0f);
  const float ss = wave_butterfly(fold8(acc));
  const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(kHeadDim) + eps);
  float n[8], p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t i = (lane & 15u) * 8u + e;
    n[e] = active ? round_bf16(bf16_to_f32(w[i]) * round_bf16(x[e] * scale)) : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = xor8_f(n[e]);
  if (active) {
    uint32_t codes[8], ncodes[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t i = lane * 8u + e;
      const float rot = lane < 8 ? -p[e] : p[e];
      const float a = round_bf16(n[e] * bf16_to_f32(cos_row[i]));
      const float b = round_bf16(rot * bf16_to_f32(sin_row[i]));
      codes[e] = f32_to_bf16(a + b);
      ncodes[e] = f32_to_bf16(n[e]);
    }
    *reinterpret_cast<u32x4 *>(roped_out + lane * 8u) =
        u32x4{codes[0] | (codes[1] << 16), codes[2] | (codes[3] << 16),
              codes[4] | (codes[5] << 16), codes[6] | (codes[7] << 16)};
    if (normed_out)
      *reinterpret_cast<u32x4 *>(normed_out + lane * 8u) =
          u32x4{ncodes[0] | (ncodes[1] << 16), ncodes[2] | (ncodes[3] << 16),
                ncodes[4] | (ncodes[5] << 16), ncodes[6] | (ncodes[7] << 16)};
  }
}

// head_norm_rope with the lane's operands already loaded (lanes 0..15:
// elements 8 l..8 l + 7 of the head row, the norm weight, cos and sin rows;
// other lanes ignored), so the caller can issue those loads early. Same
// operations in the same order; writes the roped row only, lane l's eight
// codes at roped_out + l * out_chunk.
XPU_DEVICE void head_norm_rope_vec(const u32x4 &xv, const u32x4 &wv, const u32x4 &cv, const u32x4 &sv,
                                   float eps, uint16_t *roped_out, uint64_t out_chunk = 8) {
  const uint32_t lane = lane_id();
  const bool active = lane < 16;
  float x[8], wf[8];
  unpack8<kBf16>(xv, x);
  unpack8<kBf16>(wv, wf);
  if (!active) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
  }
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(x[e], x[e], 0.0f);
  const float ss = wave_butterfly(fold8(acc));
  const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(kHeadDim) + eps);
  float n[8], p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = active ? round_bf16(wf[e] * round_bf16(x[e] * scale)) : 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = xor8_f(n[e]);
  if (active) {
    float cf[8], sf[8];
    unpack8<kBf16>(cv, cf);
    unpack8<kBf16>(sv, sf);
    uint32_t codes[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float rot = lane < 8 ? -p[e] : p[e];
      const float a = round_bf16(n[e] * cf[e]);
      const float b = round_bf16(rot * sf[e]);
      codes[e] = f32_to_bf16(a + b);
    }
    *reinterpret_cast<u32x4 *>(roped_out + lane * out_chunk) =
        u32x4{codes[0] | (codes[1] << 16), codes[2] | (codes[3] << 16), codes[4] | (codes[5] << 16),
              codes[6] | (codes[7] << 16)};
  }
}

// head_norm_rope_vec for four head rows per wavefront, one per 16-lane row
// (local lane l = lane % 16 holds elements 8 l..8 l + 7; every lane
// active). The sum of squares folds each lane's 8 slots and then runs the
// butterfly's l ^ 8, 4, 2, 1 steps within the row: the single-row form's
// l ^ 32 and l ^ 16 steps only add the idle lanes' zeros to a sum of
// squares (x + 0 = x), so the result is the same bits.
XPU_DEVICE void head_norm_rope_rows16(const u32x4 &xv, const u32x4 &wv, const u32x4 &cv, const u32x4 &sv,
                                      float eps, uint16_t *roped_out, uint64_t out_chunk = 8) {
  const uint32_t l16 = lane_id() & 15u;
  float x[8], wf[8];
  unpack8<kBf16>(xv, x);
  unpack8<kBf16>(wv, wf);
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(x[e], x[e], 0.0f);
  float ss = fold8(acc);
  ss = ss + xor8_f(ss);
  ss = ss + dpp_f<0x124>(ss);  // row_ror:4 (the values depend on l % 8 only)
  ss = ss + dpp_f<0x4E>(ss);   // quad_perm [2,3,0,1]
  ss = ss + dpp_f<0xB1>(ss);   // quad_perm [1,0,3,2]
  const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(kHeadDim) + eps);
  float n[8], p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = round_bf16(wf[e] * round_bf16(x[e] * scale));
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = xor8_f(n[e]);
  float cf[8], sf[8];
  unpack8<kBf16>(cv, cf);
  unpack8<kBf16>(sv, sf);
  uint32_t codes[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float rot = l16 < 8 ? -p[e] : p[e];
    const float a = round_bf16(n[e] * cf[e]);
    const float b = round_bf16(rot * sf[e]);
    codes[e] = f32_to_bf16(a + b);
  }
  *reinterpret_cast<u32x4 *>(roped_out + l16 * out_chunk) =
      u32x4{codes[0] | (codes[1] << 16), codes[2] | (codes[3] << 16), codes[4] | (codes[5] << 16),
            codes[6] | (codes[7] << 16)};
}

XPU_DEVICE float block_max(float v, float *red) {
  v = wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
  const uint32_t wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  __syncthreads();
  if (lane_id() == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (uint32_t i = 1; i < nwaves; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

// Attention score of query qs (LDS, roped bf16) against key row krow:
// bf16(bf16(lane-local 8-slot dot) * scale) (transformers eager: bf16 matmul
// then bf16 * scaling). The 16 row loads are independent and issued
// together.
XPU_DEVICE float attention_score_regs(const uint16_t *qs, const u32x4 (&kv)[16], float scale) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float q[8], k[8];
    unpack8<kBf16>(*reinterpret_cast<const u32x4 *>(qs + j * 8), q);
    unpack8<kBf16>(kv[j], k);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(q[e], k[e], acc[e]);
  }
  return round_bf16(round_bf16(fold8(acc)) * scale);
}

// The 16 eight-element chunks of a 128-wide head row; chunk j at row + j * chunk
// (8 for a contiguous row).
XPU_DEVICE void load_head_row(const uint16_t *row, u32x4 (&r)[16], uint64_t chunk = 8) {
#pragma unroll
  for (int j = 0; j < 16; ++j) r[j] = *reinterpret_cast<const u32x4 *>(row + j * chunk);
}

XPU_DEVICE float attention_score(const uint16_t *qs, const uint16_t *krow, float scale, uint64_t chunk = 8) {
  u32x4 kv[16];
  load_head_row(krow, kv, chunk);
  return attention_score_regs(qs, kv, scale);
}

// Cache addressing of one kv head: K row t chunk j (8 codes) at kbase +
// t * kstride + j * kchunk, V row t chunk j at vbase + t * vstride +
// j * vchunk. The reference layout [position][kv_head][128] has kstride =
// vstride = kv_heads * 128, kchunk = vchunk = 8; the engine's K and V caches
// are chunk-major [kv_head][16][max_seq][8] (stride 8, chunk max_seq * 8:
// chunk j of consecutive positions is contiguous, so a lane-per-position K
// read is coalesced and a block that owns a few dims of V reads whole lines).
struct KvLayout {
  uint64_t kstride, kchunk, vstride, vchunk;
};

constexpr uint32_t kAttnTile = 256;             // positions per V tile in LDS
constexpr uint32_t kVPitch = kHeadDim + 8;      // LDS row pitch of the V tile (bank spread)

// Single-query attention of one head with a 256-thread block
// (qwen3/kernels.hpp:157-192): positions 0..n-1, rows of K/V addressed by
// kbase/vbase and the layout lay, except that when HAS_CURRENT the last
// position reads kcur/vcur (the new token, contiguous rows not yet visible in
// the cache).
// p_t = bf16(exp(s_t - max) * (1 / sum_t exp)), out = bf16(sum_t p_t v_t).
// sbuf: kAttnChunk floats of LDS; vtile: VT * kVPitch codes of LDS (VT V
// rows per tile, a multiple of 64 up to 256: the tiles only stage the rows,
// the chains run over them in the same order whatever VT is); red: >= 4*128
// floats of LDS. Position t is handled by thread t % 256 in the score pass;
// V rows go through vtile so that the P.V pass reads LDS.
template <bool HAS_CURRENT, uint32_t VT = kAttnTile>
XPU_DEVICE void attention_tail(const uint16_t *qs, const uint16_t *kbase, const uint16_t *vbase,
                               KvLayout lay, uint32_t n, const uint16_t *kcur,
                               const uint16_t *vcur, float scale, uint16_t *out, float *sbuf,
                               uint16_t *vtile, float *red, float local_max);

// KPF: the score pass loads each thread's next K row while it scores the
// current one (64 more VGPRs; off where two blocks share a CU instead).
template <bool HAS_CURRENT, uint32_t VT = kAttnTile, bool KPF = true>
XPU_DEVICE void attention_head(const uint16_t *qs, const uint16_t *kbase, const uint16_t *vbase,
                               KvLayout lay, uint32_t n, const uint16_t *kcur,
                               const uint16_t *vcur, float scale, uint16_t *out, float *sbuf,
                               uint16_t *vtile, float *red) {
  static_assert(VT % 64 == 0 && VT <= kAttnTile, "V tiles of whole 64-row steps, at most one row per thread");
  const uint32_t tid = threadIdx.x;
  const bool single_tile = n <= VT;
  // V row t: chunk j at vrow_of(t) + j * vchunk_of(t) (the new token's row,
  // kept contiguous in vcur, when HAS_CURRENT and t is the last position)
  auto vrow_of = [&](uint32_t t) -> const uint16_t * {
    return (HAS_CURRENT && t + 1 == n) ? vcur : vbase + static_cast<uint64_t>(t) * lay.vstride;
  };
  auto vchunk_of = [&](uint32_t t) -> uint64_t { return (HAS_CURRENT && t + 1 == n) ? 8u : lay.vchunk; };
  auto stage_v_row = [&](uint32_t t, uint32_t slot) {
    const uint16_t *src = vrow_of(t);
    const uint64_t vc = vchunk_of(t);
    u32x4 vv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) vv[j] = *reinterpret_cast<const u32x4 *>(src + j * vc);
#pragma unroll
    for (int j = 0; j < 16; ++j) *reinterpret_cast<u32x4 *>(vtile + slot * kVPitch + j * 8) = vv[j];
  };
  // pass 1: scores (kept in sbuf when one chunk holds them all) and the max;
  // a single-tile context also stages its V rows here. Thread tid takes
  // positions tid, tid + 256, ... (kAttnChunk is a multiple of 256); the K
  // row of its next position is loaded before the current score is computed.
  static_assert(kAttnChunk % kAttnTile == 0, "chunks hold whole tiles");
  float local_max = -__builtin_inff();
  u32x4 knext[16];  // (unused without KPF)
  if constexpr (KPF)
    if (tid < n) load_head_row(kbase + static_cast<uint64_t>(tid) * lay.kstride, knext, lay.kchunk);
  for (uint32_t t = tid; t < n; t += kAttnTile) {
    u32x4 kcur_row[16];
    if constexpr (KPF) {
#pragma unroll
      for (int j = 0; j < 16; ++j) kcur_row[j] = knext[j];
      if (t + kAttnTile < n)
        load_head_row(kbase + static_cast<uint64_t>(t + kAttnTile) * lay.kstride, knext, lay.kchunk);
    } else {
      load_head_row(kbase + static_cast<uint64_t>(t) * lay.kstride, kcur_row, lay.kchunk);
    }
    const float s = (HAS_CURRENT && t + 1 == n) ? attention_score(qs, kcur, scale)
                                                 : attention_score_regs(qs, kcur_row, scale);
    if (single_tile) stage_v_row(t, t);
    sbuf[t % kAttnChunk] = s;
    local_max = fmaxf(local_max, s);
  }
  attention_tail<HAS_CURRENT, VT>(qs, kbase, vbase, lay, n, kcur, vcur, scale, out, sbuf, vtile, red, local_max);
}

// Passes 2 and 3 of attention_head, after the scores (sbuf, when one chunk
// holds them), the V rows (vtile, when one tile holds them) and each
// thread's running max are in place.
template <bool HAS_CURRENT, uint32_t VT>
XPU_DEVICE void attention_tail(const uint16_t *qs, const uint16_t *kbase, const uint16_t *vbase,
                               KvLayout lay, uint32_t n, const uint16_t *kcur,
                               const uint16_t *vcur, float scale, uint16_t *out, float *sbuf,
                               uint16_t *vtile, float *red, float local_max) {
  constexpr int kVJ = static_cast<int>(VT / 16);  // V rows per thread and tile
  const uint32_t tid = threadIdx.x;
  const uint32_t nchunks = (n + kAttnChunk - 1) / kAttnChunk;
  const bool single_tile = n <= VT;
  auto score_of = [&](uint32_t t) -> float {
    if (HAS_CURRENT && t + 1 == n) return attention_score(qs, kcur, scale);
    return attention_score(qs, kbase + static_cast<uint64_t>(t) * lay.kstride, scale, lay.kchunk);
  };
  auto vrow_of = [&](uint32_t t) -> const uint16_t * {
    return (HAS_CURRENT && t + 1 == n) ? vcur : vbase + static_cast<uint64_t>(t) * lay.vstride;
  };
  auto vchunk_of = [&](uint32_t t) -> uint64_t { return (HAS_CURRENT && t + 1 == n) ? 8u : lay.vchunk; };
  // a tile of tlen V rows from position t0: thread tid holds chunk tid / 16
  // of rows 16 j + tid % 16 (in the chunk-major cache a load instruction
  // reads 16 consecutive rows of each of 4 chunks, 256 contiguous bytes
  // each)
  const uint32_t v_chunk = tid >> 4, v_row0 = tid & 15u;
  auto load_v_tile = [&](uint32_t t0, uint32_t tlen, u32x4 (&vv)[kVJ]) {
#pragma unroll
    for (int j = 0; j < kVJ; ++j) {
      const uint32_t r = j * 16u + v_row0;
      if (r < tlen) vv[j] = *reinterpret_cast<const u32x4 *>(vrow_of(t0 + r) + v_chunk * vchunk_of(t0 + r));
    }
  };
  auto store_v_tile = [&](uint32_t tlen, const u32x4 (&vv)[kVJ]) {
#pragma unroll
    for (int j = 0; j < kVJ; ++j) {
      const uint32_t r = j * 16u + v_row0;
      if (r < tlen) *reinterpret_cast<u32x4 *>(vtile + r * kVPitch + v_chunk * 8u) = vv[j];
    }
  };
  const float mx = block_max(local_max, red);
  // pass 2: exponentials and the chunked canonical sum
  float total = 0.0f;
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t base = c * kAttnChunk;
    const uint32_t len = min(kAttnChunk, n - base);
    for (uint32_t i = tid; i < len; i += blockDim.x) {
      const float s = nchunks == 1 ? sbuf[i] : score_of(base + i);
      sbuf[i] = canonical_exp(s - mx);
    }
    __syncthreads();
    if (tid < 64) {
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (uint32_t j = 0; j < len; j += 512u)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t k = j + tid * 8u + e;
          if (k < len) acc[e] = acc[e] + sbuf[k];
        }
      const float chunk_sum = wave_butterfly(fold8(acc));
      total = total + chunk_sum;
    }
    __syncthreads();
  }
  if (tid == 0) red[0] = 1.0f / total;
  __syncthreads();
  const float inv = red[0];
  __syncthreads();
  // pass 3: probabilities and P.V in 16 residue classes (wave w owns
  // residues 4w..4w+3, lane l owns dims 2l and 2l+1), V read from LDS
  const uint32_t wave = tid >> 6, lane = lane_id();
  float tot[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t base = c * kAttnChunk;
    const uint32_t len = min(kAttnChunk, n - base);
    for (uint32_t i = tid; i < len; i += blockDim.x) {
      const float e = nchunks == 1 ? sbuf[i]
                                   : canonical_exp(score_of(base + i) - mx);
      sbuf[i] = round_bf16(e * inv);
    }
    __syncthreads();
    float part[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};
    // V tiles of VT rows go through vtile; the next tile's rows of this
    // thread are loaded into registers while the current tile is used
    u32x4 vnext[kVJ];
    if (!single_tile) load_v_tile(base, min(VT, len), vnext);
    for (uint32_t i0 = 0; i0 < len; i0 += VT) {
      const uint32_t tile_len = min(VT, len - i0);
      if (!single_tile) {
        store_v_tile(tile_len, vnext);
        __syncthreads();
        const uint32_t next_len = i0 + VT < len ? min(VT, len - i0 - VT) : 0u;
        if (next_len) load_v_tile(base + i0 + VT, next_len, vnext);
      }
      // 64 rows per step: the operands of 4 groups of 16 rows are read
      // (index clamped into the tile) before their FMAs, each chain in
      // ascending row order
      for (uint32_t ii0 = 0; ii0 < tile_len; ii0 += 64u) {
        float pt[4][4];
        uint32_t vv[4][4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const uint32_t i = min(ii0 + 16u * q + wave * 4u + rr, tile_len - 1);
            pt[q][rr] = sbuf[i0 + i];
            vv[q][rr] = *reinterpret_cast<const uint32_t *>(vtile + i * kVPitch + lane * 2u);
          }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            if (ii0 + 16u * q + wave * 4u + rr < tile_len) {
              part[rr][0] = __builtin_fmaf(pt[q][rr], lo16<kBf16>(vv[q][rr]), part[rr][0]);
              part[rr][1] = __builtin_fmaf(pt[q][rr], hi16<kBf16>(vv[q][rr]), part[rr][1]);
            }
          }
      }
      if (!single_tile) __syncthreads();
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      tot[rr][0] = tot[rr][0] + part[rr][0];
      tot[rr][1] = tot[rr][1] + part[rr][1];
    }
    __syncthreads();
  }
  red[wave * kHeadDim + lane * 2u] = (tot[0][0] + tot[1][0]) + (tot[2][0] + tot[3][0]);
  red[wave * kHeadDim + lane * 2u + 1] = (tot[0][1] + tot[1][1]) + (tot[2][1] + tot[3][1]);
  __syncthreads();
  if (tid < kHeadDim) {
    const float r = (red[tid] + red[kHeadDim + tid]) + (red[2 * kHeadDim + tid] + red[3 * kHeadDim + tid]);
    out[tid] = static_cast<uint16_t>(f32_to_bf16(r));
  }
  __syncthreads();
}

// Passes 2 and 3 of attention_head for n <= kAttnTile positions (one
// softmax chunk), from the scores in sbuf[0..n) and each thread's running
// max. The V operands come preloaded in the P.V layout: lane l of wave w
// owns residue class c = 4 w + l / 16 and dims 8 (l % 16) .. + 7, and
// vpv[it] holds V[t][those dims] for t = 16 it + c. Same operations in the
// same order as attention_tail (each class is one ascending FMA chain per
// dim; classes combine as ((c0 + c1) + (c2 + c3)) within a wave, then
// across waves).
XPU_DEVICE void attention_tail_short(uint32_t n, uint16_t *out, float *sbuf, float *red, float local_max,
                                     const u32x4 (&vpv)[kAttnTile / 16]) {
  const uint32_t tid = threadIdx.x;
  const float mx = block_max(local_max, red);
  if (tid < n) sbuf[tid] = canonical_exp(sbuf[tid] - mx);
  __syncthreads();
  if (tid < 64) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t k = tid * 8u + e;
      if (k < n) acc[e] = acc[e] + sbuf[k];
    }
    const float total = 0.0f + wave_butterfly(fold8(acc));
    if (tid == 0) red[0] = 1.0f / total;
  }
  __syncthreads();
  const float inv = red[0];
  const uint32_t wave = tid >> 6, lane = lane_id(), cls = wave * 4u + (lane >> 4);
  float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int it = 0; it < static_cast<int>(kAttnTile / 16); ++it) {
    const uint32_t t = it * 16u + cls;
    if (t < n) {
      const float pt = round_bf16(sbuf[t] * inv);
      float v[8];
      unpack8<kBf16>(vpv[it], v);
#pragma unroll
      for (int e = 0; e < 8; ++e) part[e] = __builtin_fmaf(pt, v[e], part[e]);
    }
  }
  float sum[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float tot = 0.0f + part[e];
    const float pair = tot + xor16_f(tot);   // (c0 + c1), (c2 + c3)
    sum[e] = pair + xor32_f(pair);           // (c0 + c1) + (c2 + c3)
  }
  __syncthreads();  // everyone has read red[0]
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wave * kHeadDim + lane * 8u + e] = sum[e];
  }
  __syncthreads();
  if (tid < kHeadDim) {
    const float r = (red[tid] + red[kHeadDim + tid]) + (red[2 * kHeadDim + tid] + red[3 * kHeadDim + tid]);
    out[tid] = static_cast<uint16_t>(f32_to_bf16(r));
  }
}

// (value, index) argmax step with the reference's tie rule (strict >, so the
// lowest index wins among equal values; kernels.hpp:238-242).
XPU_DEVICE void argmax_merge(float &v, uint32_t &i, float ov, uint32_t oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

XPU_DEVICE bool finite_f(float v) { return v == v && v != __builtin_inff() && v != -__builtin_inff(); }

// Block-wide argmax of (v, i) pairs plus an OR of bad flags; result valid in
// thread 0. red needs 3 * (blockDim/64) words of LDS.
XPU_DEVICE void block_argmax(float &v, uint32_t &i, uint32_t &bad, float *redv, uint32_t *redi,
                             uint32_t *redb) {
  // partners l ^ 32, 16, 8, then lanes with equal l % 8 hold equal pairs, so
  // row_ror:4 and the quad permutations complete the butterfly (the merge
  // is symmetric)
  auto step = [&](float ov, uint32_t oi, uint32_t ob) {
    bad |= ob;
    argmax_merge(v, i, ov, oi);
  };
  step(xor32_f(v), xor32_u(i), xor32_u(bad));
  step(xor16_f(v), xor16_u(i), xor16_u(bad));
  step(xor8_f(v), dpp_u<0x128>(i), dpp_u<0x128>(bad));
  step(dpp_f<0x124>(v), dpp_u<0x124>(i), dpp_u<0x124>(bad));
  step(dpp_f<0x4E>(v), dpp_u<0x4E>(i), dpp_u<0x4E>(bad));
  step(dpp_f<0xB1>(v), dpp_u<0xB1>(i), dpp_u<0xB1>(bad));
  const uint32_t wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  __syncthreads();
  if (lane_id() == 0) {
    redv[wave] = v;
    redi[wave] = i;
    redb[wave] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (uint32_t w = 1; w < nwaves; ++w) {
      argmax_merge(v, i, redv[w], redi[w]);
      bad |= redb[w];
    }
  }
}

}  // namespace xpu
