// Test-only probe of two decode fusions that the shipped decode does not
// use (Qwen3-0.6B shape: hidden 1024, 16 query heads, 8 kv heads, head
// dim 128; contexts of at most 256 positions). Built with the product
// kernels and their timestamps (-DXPU_STAMPS) into one code object, which
// tests/fusion_probe/fusion_probe.py loads to time whole-layer sequences.
//
//   o_proj folded into the attention: block (head, slice) of
//   probe_attn_fold<S> runs its head's attention (the short-context path
//   of xpu_q3_attention, the same operations) and then that head's o_proj
//   partial for output rows [slice * 1024 / S, +1024 / S): the 128
//   columns of the head, 8 per lane, folded over 16 lanes. The partials
//   [16][1024] (FP32) replace the o_proj kernel; probe_swiglu_partials sums
//   them in head order, rounds, adds the residual, and runs the [gate; up]
//   GEMV of xpu_q3_norm_gemv_swiglu_r2_v2 on the result. The o_proj sum is
//   re-associated (per head, then across heads), so this is a different
//   rounding of the same layer, not a bit-exact one.
//
//   probe_attn_ctrl: the same attention without the fold (one block per
//   head, spare blocks prefetching), the control for the fold's cost.
#include "../../xpu_playground_amd/csrc/kernels/module.hip"

// Blocks past heads * S prefetch [prefetch, + prefetch_bytes) as
// xpu_q3_attention's spare blocks do.
template <uint32_t S, bool FOLD>
XPU_DEVICE void probe_attention(const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ qnorm_w,
                                const uint16_t *__restrict__ knorm_w, const uint16_t *__restrict__ cos_row,
                                const uint16_t *__restrict__ sin_row, uint16_t *__restrict__ kcache,
                                uint16_t *__restrict__ vcache, uint16_t *__restrict__ out,
                                const uint32_t *__restrict__ state, uint32_t heads, uint32_t kv_heads,
                                uint32_t max_seq, float eps, float scale, const uint16_t *__restrict__ prefetch,
                                uint64_t prefetch_bytes, const uint16_t *__restrict__ Wo,
                                float *__restrict__ partials, uint32_t hidden) {
  XPU_STAMP(xpu::kStampQ3Attention);
  constexpr uint32_t kRowsPerLane = FOLD ? 1024u / S / 16u : 1u;  // hidden = 1024
  __shared__ float red[4 * xpu::kHeadDim];
  __shared__ __align__(16) uint16_t qs[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t ks[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t junk[2 * xpu::kHeadDim];
  __shared__ __align__(16) uint16_t ob[xpu::kHeadDim];
  __shared__ float sbuf[xpu::kAttnTile];
  const uint32_t nattn = heads * S;
  if (blockIdx.x >= nattn) {
    __builtin_amdgcn_s_sleep(8);
    constexpr int kUnroll = 8;
    const uint64_t n16 = prefetch_bytes / 16u;
    if (n16 == 0) return;
    const u32x4 *p = reinterpret_cast<const u32x4 *>(prefetch);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x - nattn) * blockDim.x;
    uint32_t acc = 0;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x - nattn) * blockDim.x + threadIdx.x; i < n16;
         i += kUnroll * stride) {
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = p[min(i + u * stride, n16 - 1)];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].w;
    }
    asm volatile("" : : "v"(acc));
    return;
  }
  const uint32_t head = blockIdx.x / S, slice = blockIdx.x % S;
  const uint32_t group = heads / kv_heads;
  const uint32_t kv = head / group;
  const uint16_t *qsrc = qkv + head * xpu::kHeadDim;
  const uint16_t *ksrc = qkv + (heads + kv) * xpu::kHeadDim;
  const uint16_t *vsrc = qkv + (heads + kv_heads + kv) * xpu::kHeadDim;
  const uint32_t tid = threadIdx.x, lane = xpu::lane_id();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint64_t head_base = static_cast<uint64_t>(kv) * max_seq * xpu::kHeadDim;
  const uint64_t kchunk = static_cast<uint64_t>(max_seq) * 8u;
  const uint32_t l16 = lane & 15u;
  const u32x4 hx = *reinterpret_cast<const u32x4 *>((wave == 0 ? qsrc : ksrc) + l16 * 8u);
  const u32x4 hw = *reinterpret_cast<const u32x4 *>((wave == 0 ? qnorm_w : knorm_w) + l16 * 8u);
  const u32x4 hc = *reinterpret_cast<const u32x4 *>(cos_row + l16 * 8u);
  const u32x4 hs = *reinterpret_cast<const u32x4 *>(sin_row + l16 * 8u);
  const u32x4 hv = *reinterpret_cast<const u32x4 *>(vsrc + l16 * 8u);
  // the o_proj slice: row slice * R0 + wave * R0 / 4 + 4 j + lane / 16,
  // columns head * 128 + 8 (lane % 16) .. + 7
  u32x4 wrow[kRowsPerLane];
  const uint32_t r0 = slice * (1024u / S) + wave * (1024u / S / 4u);
  if constexpr (FOLD) {
#pragma unroll
    for (uint32_t j = 0; j < kRowsPerLane; ++j)
      wrow[j] = *reinterpret_cast<const u32x4 *>(Wo + static_cast<uint64_t>(r0 + 4u * j + (lane >> 4)) * (heads * 128u) +
                                                 head * 128u + l16 * 8u);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 krow[16];
  xpu::load_head_row(kcache + head_base + static_cast<uint64_t>(min(tid, max_seq - 1)) * 8u, krow, kchunk);
  {
    const bool active = lane < 16;
    const u32x4 zero{0, 0, 0, 0};
    xpu::head_norm_rope_vec(active ? hx : zero, active ? hw : zero, hc, hs, eps,
                            wave == 0 ? qs : wave == 1 ? ks : junk + (wave - 2) * xpu::kHeadDim);
  }
  __syncthreads();
  const uint32_t pos = state[0];
  if (pos >= max_seq) return;
  const uint32_t n = pos + 1;
  if (n > xpu::kAttnTile) return;  // short contexts only (the host checks)
  if (head % group == 0 && slice == 0 && tid < 16) {
    *reinterpret_cast<u32x4 *>(kcache + head_base + tid * kchunk + static_cast<uint64_t>(pos) * 8u) =
        *reinterpret_cast<const u32x4 *>(ks + tid * 8u);
    *reinterpret_cast<u32x4 *>(vcache + head_base + tid * kchunk + static_cast<uint64_t>(pos) * 8u) = hv;
  }
  if (tid == pos) xpu::load_head_row(ks, krow);
  const float sc = tid < n ? xpu::attention_score_regs(qs, krow, scale) : -__builtin_inff();
  u32x4 vpv[xpu::kAttnTile / 16];
  const uint32_t cls = l16, vch = wave * 4u + (lane >> 4);
#pragma unroll
  for (int it = 0; it < static_cast<int>(xpu::kAttnTile / 16); ++it) {
    const uint32_t t = it * 16u + cls;
    const uint16_t *src = t < pos ? vcache + head_base + vch * kchunk + static_cast<uint64_t>(t) * 8u : vsrc + vch * 8u;
    vpv[it] = *reinterpret_cast<const u32x4 *>(src);
  }
  const float wmax = xpu::wave_reduce(sc, [](float x, float y) { return fmaxf(x, y); });
  if (lane == 0) red[wave] = wmax;
  __syncthreads();
  const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float ex = tid < n ? xpu::canonical_exp(sc - mx) : 0.0f;
  sbuf[tid] = ex;
  float f = ex + xpu::dpp_f<0xB1>(ex);
  f = f + xpu::dpp_f<0x4E>(f);
  f = f + xpu::dpp_f<0x141>(f);
  float *lane_sum = red + 4;
  if ((tid & 7u) == 0) lane_sum[tid >> 3] = f;
  __syncthreads();
  const float total = xpu::wave_butterfly(lane < 32 ? lane_sum[lane] : 0.0f);
  const float inv = 1.0f / total;
  float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int it = 0; it < static_cast<int>(xpu::kAttnTile / 16); ++it) {
    const uint32_t t = it * 16u + cls;
    if (t < n) {
      const float pt = xpu::round_bf16(sbuf[t] * inv);
      float v[8];
      xpu::unpack8<xpu::kBf16>(vpv[it], v);
#pragma unroll
      for (int e = 0; e < 8; ++e) part[e] = __builtin_fmaf(pt, v[e], part[e]);
    }
  }
  uint32_t code[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float v = part[e];
    v = v + xpu::dpp_f<0xB1>(v);
    v = v + xpu::dpp_f<0x4E>(v);
    v = v + xpu::dpp_f<0x141>(v);
    v = v + xpu::xor8_f(v);
    code[e] = xpu::f32_to_bf16(v);
  }
  const u32x4 packed{code[0] | (code[1] << 16), code[2] | (code[3] << 16), code[4] | (code[5] << 16),
                     code[6] | (code[7] << 16)};
  if constexpr (!FOLD) {
    if (cls == 0) *reinterpret_cast<u32x4 *>(out + head * xpu::kHeadDim + vch * 8u) = packed;
    return;
  } else {
    if (cls == 0) *reinterpret_cast<u32x4 *>(ob + vch * 8u) = packed;
    __syncthreads();
    float ov[8];
    xpu::unpack8<xpu::kBf16>(*reinterpret_cast<const u32x4 *>(ob + l16 * 8u), ov);
#pragma unroll
    for (uint32_t j = 0; j < kRowsPerLane; ++j) {
      float w[8];
      xpu::unpack8<xpu::kBf16>(wrow[j], w);
      float a = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) a = __builtin_fmaf(w[e], ov[e], a);
      a = a + __shfl_xor(a, 8);
      a = a + __shfl_xor(a, 4);
      a = a + __shfl_xor(a, 2);
      a = a + __shfl_xor(a, 1);
      if (l16 == 0) partials[head * hidden + r0 + 4u * j + (lane >> 4)] = a;
    }
  }
}

#define PROBE_ATTN(NAME, S, FOLD)                                                                         \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                                       \
      const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ qnorm_w, const uint16_t *__restrict__ knorm_w, \
      const uint16_t *__restrict__ cos_row, const uint16_t *__restrict__ sin_row, uint16_t *__restrict__ kcache,   \
      uint16_t *__restrict__ vcache, uint16_t *__restrict__ out, const uint32_t *__restrict__ state,            \
      uint32_t heads, uint32_t kv_heads, uint32_t max_seq, float eps, float scale,                               \
      const uint16_t *__restrict__ prefetch, uint64_t prefetch_bytes, const uint16_t *__restrict__ Wo,          \
      float *__restrict__ partials, uint32_t hidden) {                                                           \
    probe_attention<S, FOLD>(qkv, qnorm_w, knorm_w, cos_row, sin_row, kcache, vcache, out, state, heads, \
                                   kv_heads, max_seq, eps, scale, prefetch, prefetch_bytes, Wo, partials, hidden); \
  }
PROBE_ATTN(probe_attn_fold16, 16, true)
PROBE_ATTN(probe_attn_fold8, 8, true)
PROBE_ATTN(probe_attn_fold4, 4, true)
PROBE_ATTN(probe_attn_ctrl, 1, false)

// [gate; up] + SiLU whose input is the sum of `parts` FP32 partials
// [parts][1024] (in part order) rounded to bf16 plus the residual x (bf16);
// block 0 writes the new residual to x_out (a buffer other than x: the
// other blocks still read x). K = 1024, NC = 2, R = 2.
extern "C" __global__ __launch_bounds__(256) void probe_swiglu_partials(
    const uint16_t *__restrict__ Wgu, const uint16_t *__restrict__ x, const float *__restrict__ partials,
    uint32_t parts, uint16_t *__restrict__ x_out, const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ h,
    uint32_t I, uint32_t K, float eps) {
  XPU_STAMP(xpu::kStampQ3Swiglu);
  __shared__ __align__(16) uint16_t xs[1024];
  const uint32_t tid = threadIdx.x;  // elements 4 tid .. 4 tid + 3
  {
    float4 acc = {0, 0, 0, 0};
    for (uint32_t p = 0; p < parts; ++p) {
      const float4 v = *reinterpret_cast<const float4 *>(partials + p * 1024u + 4u * tid);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    const uint2 xr = *reinterpret_cast<const uint2 *>(x + 4u * tid);
    const float o[4] = {acc.x, acc.y, acc.z, acc.w};
    const uint32_t xin[4] = {xr.x & 0xffffu, xr.x >> 16, xr.y & 0xffffu, xr.y >> 16};
    uint32_t c[4];
    for (int e = 0; e < 4; ++e) c[e] = xpu::f32_to_bf16(xpu::bf16_to_f32(xin[e]) + xpu::round_bf16(o[e]));
    const uint2 packed{c[0] | (c[1] << 16), c[2] | (c[3] << 16)};
    *reinterpret_cast<uint2 *>(xs + 4u * tid) = packed;
    if (blockIdx.x == 0) *reinterpret_cast<uint2 *>(x_out + 4u * tid) = packed;
  }
  __syncthreads();
  q3_norm_gemv_swiglu_reg<2, 2>(Wgu, xs, norm_w, h, I, K, eps);
}
