// Qwen3 decode kernels for gfx950.
//
// Part 1: the reference's eight entries with the reference's names and
// argument order (qwen3/kernels_entry.cpp:8-72), launchable through the
// runtime's work-item convention (xpu_rt_launch). The reference hard-codes
// the 8B shape (kernels.hpp:20-22, hidden 4096 at :32); the shape is passed
// as trailing arguments instead. KV caches use the reference layout
// [position][kv_head][128] (kernels.hpp:128-131).
//
// Part 2: the fused decode path the engine runs (one hipGraph per token):
//   xpu_q3_norm_gemv        RMSNorm + QKV projection (layer 0: + embedding)
//   xpu_q3_attention        QK-norm + RoPE + KV-cache write + attention
//   xpu_q3_gemv_residual    o_proj / down_proj + residual add
//   xpu_q3_norm_gemv_swiglu RMSNorm + gate/up projection + SiLU * up
//                           (gate/up stored as one [gate; up] matrix)
//   xpu_q3_norm_gemv_logits final RMSNorm + tied lm_head + per-block argmax
//   xpu_q3_argmax_finish    argmax, next token, position advance
// The decode position and token live in device memory (state[0], state[1])
// so one captured graph serves every step. Engine caches: K and V
// chunk-major [kv_head][16][max_seq][8] (eight-element chunk j of every
// position contiguous).
#include "qwen3_core.hpp"

using xpu::u32x4;

// ------------------------------------------------------------ reference entries

// kernels.hpp:24-34: out[i] = table[token * hidden + i]
extern "C" __global__ __launch_bounds__(256) void QwenEmbedding(
    const uint16_t *__restrict__ table, uint16_t *__restrict__ out, uint32_t token, uint32_t hidden) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < hidden) out[i] = table[static_cast<uint64_t>(token) * hidden + i];
}

// kernels.hpp:36-56 (one block; the reference uses one work-item)
extern "C" __global__ __launch_bounds__(256) void QwenRmsNorm(
    const uint16_t *__restrict__ input, const uint16_t *__restrict__ weight,
    uint16_t *__restrict__ output, uint32_t width, float epsilon) {
  extern __shared__ __align__(16) uint16_t xs[];
  __shared__ float red[1];
  xpu::block_rmsnorm(xs, input, weight, width, epsilon, red);
  for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) output[i] = xs[i];
}

// kernels_entry.cpp:23-29: bf16 GEMV with lda = columns
extern "C" __global__ __launch_bounds__(256) void QwenGemv(
    const uint16_t *__restrict__ matrix, const uint16_t *__restrict__ vector,
    uint16_t *__restrict__ output, uint32_t rows, uint32_t columns) {
  extern __shared__ __align__(16) uint16_t xs[];
  const bool vec = (reinterpret_cast<uintptr_t>(matrix) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(vector) % 16 == 0) && columns % 8 == 0;
  const uint32_t kpad = (columns + 511u) & ~511u;
  if (vec) xpu::stage_vector<true>(xs, vector, columns, kpad);
  else xpu::stage_vector<false>(xs, vector, columns, kpad);
  __syncthreads();
  const uint32_t wave = threadIdx.x >> 6, lane = xpu::lane_id();
  for (uint32_t base = blockIdx.x * 8u; base < rows; base += gridDim.x * 8u) {
    for (uint32_t half = 0; half < 2; ++half) {
      const uint32_t row0 = base + half * 4u + wave;
      if (row0 >= rows) continue;
      float out[1];
      if (vec) xpu::gemv_rows<xpu::kBf16, 1, 4, true>(matrix, columns, columns, rows, xs, row0, out);
      else xpu::gemv_rows<xpu::kBf16, 1, 2, false>(matrix, columns, columns, rows, xs, row0, out);
      if (lane == 0) output[row0] = static_cast<uint16_t>(xpu::f32_to_bf16(out[0]));
    }
  }
}

// kernels.hpp:58-155, one wavefront per query head: q normed + roped in
// place; heads < kv_heads also norm k in place, write roped k and v to the
// cache slot (position * kv_heads + head) * 128. Skipped when position >=
// maximum_sequence (:74-75).
extern "C" __global__ __launch_bounds__(64) void QwenQkvRopeCache(
    uint16_t *query, uint16_t *key, const uint16_t *__restrict__ value,
    const uint16_t *__restrict__ query_norm, const uint16_t *__restrict__ key_norm,
    const uint16_t *__restrict__ rope_cos, const uint16_t *__restrict__ rope_sin,
    uint16_t *__restrict__ key_cache, uint16_t *__restrict__ value_cache, uint32_t position,
    uint32_t maximum_sequence, uint32_t heads, uint32_t kv_heads) {
  const uint32_t head = blockIdx.x;
  if (position >= maximum_sequence || head >= heads) return;
  const uint16_t *cos_row = rope_cos + static_cast<uint64_t>(position) * xpu::kHeadDim;
  const uint16_t *sin_row = rope_sin + static_cast<uint64_t>(position) * xpu::kHeadDim;
  __shared__ __align__(16) uint16_t roped[xpu::kHeadDim];
  uint16_t *q = query + head * xpu::kHeadDim;
  xpu::head_norm_rope(q, query_norm, cos_row, sin_row, 1.0e-6f, nullptr, roped);
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < xpu::kHeadDim; i += 64) q[i] = roped[i];
  __syncthreads();
  if (head < kv_heads) {
    uint16_t *k = key + head * xpu::kHeadDim;
    const uint64_t slot = (static_cast<uint64_t>(position) * kv_heads + head) * xpu::kHeadDim;
    xpu::head_norm_rope(k, key_norm, cos_row, sin_row, 1.0e-6f, k, key_cache + slot);
    for (uint32_t i = threadIdx.x; i < xpu::kHeadDim; i += 64)
      value_cache[slot + i] = value[head * xpu::kHeadDim + i];
  }
}

// kernels.hpp:157-192: one block per query head over cache positions
// 0..position, kv head = head / (heads / kv_heads).
extern "C" __global__ __launch_bounds__(256) void QwenAttention(
    const uint16_t *__restrict__ query, const uint16_t *__restrict__ key_cache,
    const uint16_t *__restrict__ value_cache, uint16_t *__restrict__ output, uint32_t position,
    uint32_t heads, uint32_t kv_heads) {
  __shared__ float sbuf[xpu::kAttnChunk];
  __shared__ float red[4 * xpu::kHeadDim];
  __shared__ __align__(16) uint16_t qs[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t vtile[xpu::kAttnTile * xpu::kVPitch];
  const uint32_t head = blockIdx.x;
  if (head >= heads) return;
  const uint32_t kv = head / (heads / kv_heads);
  if (threadIdx.x < xpu::kHeadDim) qs[threadIdx.x] = query[head * xpu::kHeadDim + threadIdx.x];
  __syncthreads();
  const uint64_t stride = static_cast<uint64_t>(kv_heads) * xpu::kHeadDim;
  xpu::attention_head<false>(qs, key_cache + kv * xpu::kHeadDim, value_cache + kv * xpu::kHeadDim,
                             xpu::KvLayout{stride, 8, stride, 8}, position + 1, nullptr, nullptr, 0.08838834764831845f,
                             output + head * xpu::kHeadDim, sbuf, vtile, red);
}

// kernels.hpp:194-207: left = bf16(left + right)
extern "C" __global__ __launch_bounds__(256) void QwenAdd(uint16_t *left, const uint16_t *right,
                                                          uint32_t width) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < width)
    left[i] = static_cast<uint16_t>(
        xpu::f32_to_bf16(xpu::bf16_to_f32(left[i]) + xpu::bf16_to_f32(right[i])));
}

// kernels.hpp:209-223 with transformers rounding: bf16(bf16(silu(g)) * u)
XPU_DEVICE uint32_t silu_mul_code(float g, float u) {
  const float act = xpu::round_bf16(g / (1.0f + xpu::canonical_exp(-g)));
  return xpu::f32_to_bf16(act * u);
}

extern "C" __global__ __launch_bounds__(256) void QwenSiluMultiply(uint16_t *gate, const uint16_t *up,
                                                                   uint32_t width) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < width)
    gate[i] = static_cast<uint16_t>(silu_mul_code(xpu::bf16_to_f32(gate[i]), xpu::bf16_to_f32(up[i])));
}

// kernels.hpp:225-246 (one block): first maximum, NaN/Inf -> 0xffffffff
extern "C" __global__ __launch_bounds__(1024) void QwenArgmax(const uint16_t *__restrict__ values,
                                                              uint32_t *token, uint32_t width) {
  __shared__ float redv[16];
  __shared__ uint32_t redi[16], redb[16];
  float best = -__builtin_inff();
  uint32_t best_index = 0xffffffffu, bad = 0;
  for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) {
    const float v = xpu::bf16_to_f32(values[i]);
    if (!xpu::finite_f(v)) bad = 1;
    xpu::argmax_merge(best, best_index, v, i);
  }
  xpu::block_argmax(best, best_index, bad, redv, redi, redb);
  if (threadIdx.x == 0) *token = bad ? 0xffffffffu : (best_index == 0xffffffffu ? 0u : best_index);
}

// ------------------------------------------------------------ fused decode path

namespace {

// Grid-stride loop of a fused GEMV kernel over output units (rows, or row
// pairs when PAIRED) in tiles of 4 wavefronts; each wavefront computes R
// rows. The first tile's first load batch is issued before the prologue
// (which stages the input vector in LDS) so that the weight stream's latency
// overlaps it. body(unit0, out[R]).
template <int R, int U, bool PAIRED, typename Prologue, typename Body>
XPU_DEVICE void fused_gemv(const uint16_t *__restrict__ W, uint32_t units, uint32_t K, const uint16_t *xs,
                           Prologue prologue, Body body) {
  constexpr uint32_t per_wave = PAIRED ? R / 2 : R;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t per_block = (blockDim.x >> 6) * per_wave;
  const uint32_t rows_total = PAIRED ? 2 * units : units;
  const uint32_t pair_offset = PAIRED ? units : 0;
  xpu::u32x4 first[U][R];
  bool have_first = false;
  uint32_t base = blockIdx.x * per_block;
  if (base + wave * per_wave < units && K / 512u >= static_cast<uint32_t>(U)) {
    const uint16_t *rows[R];
    xpu::gemv_row_ptrs<R, PAIRED>(W, K, rows_total, base + wave * per_wave, pair_offset, rows);
    xpu::gemv_load_batch<R, U, true>(first, rows, 0, K);
    have_first = true;
  }
  prologue();
  for (; base < units; base += gridDim.x * per_block) {
    const uint32_t u0 = base + wave * per_wave;
    if (u0 >= units) continue;
    float out[R];
    xpu::gemv_rows_first<xpu::kBf16, R, U, true, PAIRED>(W, K, K, rows_total, xs, u0, out, pair_offset,
                                                         first, have_first);
    have_first = false;
    body(u0, out);
  }
}

}  // namespace

// out[M] = W[M x K] . rmsnorm(x). When embed is non-null (first layer) the
// source row is embed[state[1]] and block 0 also stores it into x.
template <int R, int U>
XPU_DEVICE void q3_norm_gemv(const uint16_t *__restrict__ W, uint16_t *x,
                             const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ out,
                             uint32_t M, uint32_t K, float eps, const uint16_t *__restrict__ embed,
                             const uint32_t *__restrict__ state, uint32_t vocab) {
  extern __shared__ __align__(16) uint16_t xs[];
  __shared__ float red[1];
  const uint16_t *src = x;
  if (embed) {
    uint32_t token = state[1];
    if (token >= vocab) token = 0;
    src = embed + static_cast<uint64_t>(token) * K;
    if (blockIdx.x == 0)
      for (uint32_t i = threadIdx.x; i < K; i += blockDim.x) x[i] = src[i];
  }
  const uint32_t lane = xpu::lane_id();
  fused_gemv<R, U, false>(
      W, M, K, xs, [&] { xpu::block_rmsnorm_vec(xs, src, norm_w, K, eps, red); },
      [&](uint32_t row0, const float (&o)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (lane == static_cast<uint32_t>(r) && row0 + r < M)
            out[row0 + r] = static_cast<uint16_t>(xpu::f32_to_bf16(o[r]));
      });
}

// x[M] = bf16(x + bf16(W[M x K] . v))
template <int R, int U>
XPU_DEVICE void q3_gemv_residual(const uint16_t *__restrict__ W, const uint16_t *__restrict__ v,
                                 uint16_t *x, uint32_t M, uint32_t K) {
  extern __shared__ __align__(16) uint16_t xs[];
  const uint32_t lane = xpu::lane_id();
  fused_gemv<R, U, false>(
      W, M, K, xs,
      [&] {
        xpu::stage_vector<true>(xs, v, K, (K + 511u) & ~511u);
        __syncthreads();
      },
      [&](uint32_t row0, const float (&o)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (lane == static_cast<uint32_t>(r) && row0 + r < M) {
            const float sum = xpu::bf16_to_f32(x[row0 + r]) + xpu::round_bf16(o[r]);
            x[row0 + r] = static_cast<uint16_t>(xpu::f32_to_bf16(sum));
          }
      });
}

// h[i] = bf16(bf16(silu(g_i)) * u_i) for i < I, with g = gate . rmsnorm(x)
// and u = up . rmsnorm(x) from the [gate; up] matrix (2I x K); a wavefront
// computes P = R/2 consecutive outputs (rows i.. of each half).
template <int R, int U>
XPU_DEVICE void q3_norm_gemv_swiglu(const uint16_t *__restrict__ Wgu, const uint16_t *__restrict__ x,
                                    const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ h,
                                    uint32_t I, uint32_t K, float eps) {
  static_assert(R % 2 == 0, "gate/up rows come in pairs");
  constexpr int P = R / 2;
  extern __shared__ __align__(16) uint16_t xs[];
  __shared__ float red[1];
  const uint32_t lane = xpu::lane_id();
  fused_gemv<R, U, true>(
      Wgu, I, K, xs, [&] { xpu::block_rmsnorm_vec(xs, x, norm_w, K, eps, red); },
      [&](uint32_t i0, const float (&o)[R]) {
#pragma unroll
        for (int p = 0; p < P; ++p)
          if (lane == static_cast<uint32_t>(p) && i0 + p < I)
            h[i0 + p] = static_cast<uint16_t>(silu_mul_code(xpu::round_bf16(o[p]), xpu::round_bf16(o[P + p])));
      });
}

// logits[V] = E[V x K] . rmsnorm(x); block b also writes its (max, index,
// non-finite flag) to part_*[b]
template <int R, int U>
XPU_DEVICE void q3_norm_gemv_logits(const uint16_t *__restrict__ E, const uint16_t *__restrict__ x,
                                    const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ logits,
                                    uint32_t V, uint32_t K, float eps, float *__restrict__ part_val,
                                    uint32_t *__restrict__ part_idx, uint32_t *__restrict__ part_bad) {
  extern __shared__ __align__(16) uint16_t xs[];
  __shared__ float red[1];
  __shared__ float redv[4];
  __shared__ uint32_t redi[4], redb[4];
  const uint32_t lane = xpu::lane_id();
  float best = -__builtin_inff();
  uint32_t best_index = 0xffffffffu, bad = 0;
  fused_gemv<R, U, false>(
      E, V, K, xs, [&] { xpu::block_rmsnorm_vec(xs, x, norm_w, K, eps, red); },
      [&](uint32_t row0, const float (&o)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (row0 + r >= V) break;
          const uint32_t code = xpu::f32_to_bf16(o[r]);
          if (lane == static_cast<uint32_t>(r)) logits[row0 + r] = static_cast<uint16_t>(code);
          const float v = xpu::bf16_to_f32(code);
          if (!xpu::finite_f(v)) bad = 1;
          xpu::argmax_merge(best, best_index, v, row0 + r);
        }
      });
  xpu::block_argmax(best, best_index, bad, redv, redi, redb);
  if (threadIdx.x == 0) {
    part_val[blockIdx.x] = best;
    part_idx[blockIdx.x] = best_index;
    part_bad[blockIdx.x] = bad;
  }
}

#define XPU_Q3_NORM_GEMV(SUFFIX, R, U)                                                          \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_norm_gemv##SUFFIX(                   \
      const uint16_t *__restrict__ W, uint16_t *x, const uint16_t *__restrict__ norm_w,         \
      uint16_t *__restrict__ out, uint32_t M, uint32_t K, float eps,                            \
      const uint16_t *__restrict__ embed, const uint32_t *__restrict__ state, uint32_t vocab) { \
    XPU_STAMP(xpu::kStampQ3Qkv);                                                                \
    q3_norm_gemv<R, U>(W, x, norm_w, out, M, K, eps, embed, state, vocab);                      \
  }
#define XPU_Q3_GEMV_RESIDUAL(SUFFIX, R, U)                                                      \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_gemv_residual##SUFFIX(               \
      const uint16_t *__restrict__ W, const uint16_t *__restrict__ v, uint16_t *x, uint32_t M,  \
      uint32_t K) {                                                                             \
    XPU_STAMP(xpu::kStampQ3Residual);                                                           \
    q3_gemv_residual<R, U>(W, v, x, M, K);                                                      \
  }
#define XPU_Q3_SWIGLU(SUFFIX, R, U)                                                             \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_norm_gemv_swiglu##SUFFIX(            \
      const uint16_t *__restrict__ Wgu, const uint16_t *__restrict__ x,                         \
      const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ h, uint32_t I, uint32_t K,    \
      float eps) {                                                                              \
    XPU_STAMP(xpu::kStampQ3Swiglu);                                                             \
    q3_norm_gemv_swiglu<R, U>(Wgu, x, norm_w, h, I, K, eps);                                    \
  }
#define XPU_Q3_LOGITS(SUFFIX, R, U)                                                             \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_norm_gemv_logits##SUFFIX(            \
      const uint16_t *__restrict__ E, const uint16_t *__restrict__ x,                           \
      const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ logits, uint32_t V,           \
      uint32_t K, float eps, float *__restrict__ part_val, uint32_t *__restrict__ part_idx,     \
      uint32_t *__restrict__ part_bad) {                                                        \
    XPU_STAMP(xpu::kStampQ3Logits);                                                             \
    q3_norm_gemv_logits<R, U>(E, x, norm_w, logits, V, K, eps, part_val, part_idx, part_bad);   \
  }

XPU_Q3_NORM_GEMV(_r2, 2, 2)
XPU_Q3_GEMV_RESIDUAL(_r1, 1, 2)
XPU_Q3_SWIGLU(_r2, 2, 2)
XPU_Q3_LOGITS(_r2, 2, 2)

// ---- register-vector forms of the four fused GEMVs
//
// For K <= 512 NC: lane l of every wavefront holds elements 512 c + 8 l ..
// 512 c + 8 l + 7 of the input vector in xv[c] (zeros past K), which are
// exactly the elements it multiplies in the canonical GEMV order, and which
// are also the canonical (lane, slot, chunk) layout of the RMSNorm sum of
// squares. So each wavefront loads its vector slices from global memory
// (the same addresses in every wavefront, served by the caches) and, for
// the norm kernels, computes the RMSNorm scale and the normed codes in
// registers: no LDS staging and no block barriers. Same operations in the
// same order as block_rmsnorm_vec and gemv_rows_first. The vector loads are
// issued first, then the first batch of weight rows (rows past the end are
// clamped and discarded), so the weight latency overlaps the norm.
namespace {

constexpr uint32_t kRegBlock = 256;  // block size of the register-vector kernels

// Branch-free masked loads (K % 8 == 0, K >= 8): a slice past K reads the
// last in-range slice and is replaced by zeros, so every load is issued
// unconditionally and the wait counts stay exact.
XPU_DEVICE u32x4 masked16(const uint16_t *__restrict__ base, uint32_t col, uint32_t K, bool nt) {
  const uint32_t c = col < K ? col : K - 8u;
  const u32x4 v = nt ? xpu::load_nt16(base + c) : *reinterpret_cast<const u32x4 *>(base + c);
  return col < K ? v : u32x4{0, 0, 0, 0};
}

template <int NC>
XPU_DEVICE void load_slices(const uint16_t *__restrict__ v, uint32_t K, u32x4 (&xv)[NC]) {
  const uint32_t lane = xpu::lane_id();
#pragma unroll
  for (int c = 0; c < NC; ++c) xv[c] = masked16(v, c * 512u + lane * 8u, K, false);
}

// xv <- codes of bf16(w * bf16(x * (1 / sqrt(sum(x^2) / K + eps))))
template <int NC>
XPU_DEVICE void rmsnorm_slices(u32x4 (&xv)[NC], const u32x4 (&wv)[NC], uint32_t K, float eps) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float f[8];
    xpu::unpack8<xpu::kBf16>(xv[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(f[e], f[e], acc[e]);
  }
  const float ss = xpu::wave_butterfly(xpu::fold8(acc));
  const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(K) + eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float xf[8], wf[8];
    xpu::unpack8<xpu::kBf16>(xv[c], xf);
    xpu::unpack8<xpu::kBf16>(wv[c], wf);
    uint32_t code[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) code[e] = xpu::f32_to_bf16(wf[e] * xpu::round_bf16(xf[e] * scale));
    // slices past K stay zero (their x and w loads were zero, and so are
    // their codes: bf16(0 * ...) = +0)
    xv[c] = u32x4{code[0] | (code[1] << 16), code[2] | (code[3] << 16), code[4] | (code[5] << 16),
                  code[6] | (code[7] << 16)};
  }
}

template <int R, int NC, bool PAIRED>
XPU_DEVICE void load_rows(const uint16_t *__restrict__ W, uint32_t K, uint32_t rows_total, uint32_t u0,
                          uint32_t pair_offset, u32x4 (&a)[NC][R]) {
  const uint32_t lane = xpu::lane_id();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t want = PAIRED ? (r < R / 2 ? u0 + r : u0 + pair_offset + (r - R / 2)) : u0 + r;
    const uint16_t *row = W + static_cast<uint64_t>(want < rows_total ? want : rows_total - 1) * K;
#pragma unroll
    for (int c = 0; c < NC; ++c) a[c][r] = masked16(row, c * 512u + lane * 8u, K, true);
  }
}

template <int R, int NC>
XPU_DEVICE void dot_rows(const u32x4 (&a)[NC][R], const u32x4 (&xv)[NC], float (&out)[R]) {
  float acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) xpu::fma_chunk<xpu::kBf16, R>(acc, a[c], xv[c]);
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = xpu::wave_butterfly(xpu::fold8(acc[r]));
}

// Grid-stride loop over output units (rows, or row pairs when PAIRED), one
// unit group of R rows per wavefront per step. vec_load(first unit) issues
// the vector loads (and any other early load), vec_finish turns them into
// xv; body(unit0, out[R]).
template <int R, int NC, bool PAIRED, typename VecLoad, typename VecFinish, typename Body>
XPU_DEVICE void reg_gemv(const uint16_t *__restrict__ W, uint32_t units, uint32_t K, VecLoad vec_load,
                         VecFinish vec_finish, Body body) {
  constexpr uint32_t per_wave = PAIRED ? R / 2 : R;
  constexpr uint32_t waves = kRegBlock / 64;  // launched with kRegBlock threads
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t rows_total = PAIRED ? 2 * units : units;
  const uint32_t pair_offset = PAIRED ? units : 0;
  const uint32_t stride = gridDim.x * waves * per_wave;
  uint32_t u0 = (blockIdx.x * waves + wave) * per_wave;
  vec_load(u0);
  u32x4 a[NC][R];
  load_rows<R, NC, PAIRED>(W, K, rows_total, u0 < units ? u0 : 0, pair_offset, a);
  u32x4 xv[NC];
  vec_finish(xv);
  for (; u0 < units; u0 += stride) {
    float out[R];
    dot_rows<R, NC>(a, xv, out);
    body(u0, out);
    if (u0 + stride < units) load_rows<R, NC, PAIRED>(W, K, rows_total, u0 + stride, pair_offset, a);
  }
}

}  // namespace

template <int R, int NC>
XPU_DEVICE void q3_norm_gemv_reg(const uint16_t *__restrict__ W, uint16_t *x, const uint16_t *__restrict__ norm_w,
                                 uint16_t *__restrict__ out, uint32_t M, uint32_t K, float eps,
                                 const uint16_t *__restrict__ embed, const uint32_t *__restrict__ state,
                                 uint32_t vocab) {
  const uint16_t *src = x;
  if (embed) {
    uint32_t token = state[1];
    if (token >= vocab) token = 0;
    src = embed + static_cast<uint64_t>(token) * K;
  }
  const uint32_t lane = xpu::lane_id();
  u32x4 xr[NC], wr[NC];
  reg_gemv<R, NC, false>(
      W, M, K,
      [&](uint32_t) {
        load_slices<NC>(src, K, xr);
        load_slices<NC>(norm_w, K, wr);
      },
      [&](u32x4 (&xv)[NC]) {
        if (embed && blockIdx.x == 0 && threadIdx.x < 64) {  // the residual stream starts as the embedding row
#pragma unroll
          for (int c = 0; c < NC; ++c)
            if (c * 512u + lane * 8u < K) *reinterpret_cast<u32x4 *>(x + c * 512u + lane * 8u) = xr[c];
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) xv[c] = xr[c];
        rmsnorm_slices<NC>(xv, wr, K, eps);
      },
      [&](uint32_t row0, const float (&o)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (lane == static_cast<uint32_t>(r) && row0 + r < M)
            out[row0 + r] = static_cast<uint16_t>(xpu::f32_to_bf16(o[r]));
      });
}

template <int R, int NC>
XPU_DEVICE void q3_gemv_residual_reg(const uint16_t *__restrict__ W, const uint16_t *__restrict__ v, uint16_t *x,
                                     uint32_t M, uint32_t K) {
  const uint32_t lane = xpu::lane_id();
  u32x4 vr[NC];
  // residual input of the first unit's rows (lane r: row u0 + r), loaded
  // with the vector so the read-modify-write does not wait on memory
  uint32_t first = 0xffffffffu, xres = 0;
  reg_gemv<R, NC, false>(
      W, M, K,
      [&](uint32_t u0) {
        load_slices<NC>(v, K, vr);
        first = u0;
        if (lane < static_cast<uint32_t>(R) && u0 + lane < M) xres = x[u0 + lane];
      },
      [&](u32x4 (&xv)[NC]) {
#pragma unroll
        for (int c = 0; c < NC; ++c) xv[c] = vr[c];
      },
      [&](uint32_t row0, const float (&o)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (lane == static_cast<uint32_t>(r) && row0 + r < M) {
            const uint32_t old = row0 == first ? xres : x[row0 + r];
            const float sum = xpu::bf16_to_f32(old) + xpu::round_bf16(o[r]);
            x[row0 + r] = static_cast<uint16_t>(xpu::f32_to_bf16(sum));
          }
      });
}

template <int R, int NC>
XPU_DEVICE void q3_norm_gemv_swiglu_reg(const uint16_t *__restrict__ Wgu, const uint16_t *__restrict__ x,
                                        const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ h, uint32_t I,
                                        uint32_t K, float eps) {
  static_assert(R % 2 == 0, "gate/up rows come in pairs");
  constexpr int P = R / 2;
  const uint32_t lane = xpu::lane_id();
  u32x4 xr[NC], wr[NC];
  reg_gemv<R, NC, true>(
      Wgu, I, K,
      [&](uint32_t) {
        load_slices<NC>(x, K, xr);
        load_slices<NC>(norm_w, K, wr);
      },
      [&](u32x4 (&xv)[NC]) {
#pragma unroll
        for (int c = 0; c < NC; ++c) xv[c] = xr[c];
        rmsnorm_slices<NC>(xv, wr, K, eps);
      },
      [&](uint32_t i0, const float (&o)[R]) {
#pragma unroll
        for (int p = 0; p < P; ++p)
          if (lane == static_cast<uint32_t>(p) && i0 + p < I)
            h[i0 + p] = static_cast<uint16_t>(silu_mul_code(xpu::round_bf16(o[p]), xpu::round_bf16(o[P + p])));
      });
}

template <int R, int NC>
XPU_DEVICE void q3_norm_gemv_logits_reg(const uint16_t *__restrict__ E, const uint16_t *__restrict__ x,
                                        const uint16_t *__restrict__ norm_w, uint16_t *__restrict__ logits,
                                        uint32_t V, uint32_t K, float eps, float *__restrict__ part_val,
                                        uint32_t *__restrict__ part_idx, uint32_t *__restrict__ part_bad) {
  __shared__ float redv[4];
  __shared__ uint32_t redi[4], redb[4];
  const uint32_t lane = xpu::lane_id();
  float best = -__builtin_inff();
  uint32_t best_index = 0xffffffffu, bad = 0;
  u32x4 xr[NC], wr[NC];
  reg_gemv<R, NC, false>(
      E, V, K,
      [&](uint32_t) {
        load_slices<NC>(x, K, xr);
        load_slices<NC>(norm_w, K, wr);
      },
      [&](u32x4 (&xv)[NC]) {
#pragma unroll
        for (int c = 0; c < NC; ++c) xv[c] = xr[c];
        rmsnorm_slices<NC>(xv, wr, K, eps);
      },
      [&](uint32_t row0, const float (&o)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (row0 + r >= V) break;
          const uint32_t code = xpu::f32_to_bf16(o[r]);
          if (lane == static_cast<uint32_t>(r)) logits[row0 + r] = static_cast<uint16_t>(code);
          const float v = xpu::bf16_to_f32(code);
          if (!xpu::finite_f(v)) bad = 1;
          xpu::argmax_merge(best, best_index, v, row0 + r);
        }
      });
  xpu::block_argmax(best, best_index, bad, redv, redi, redb);
  if (threadIdx.x == 0) {
    part_val[blockIdx.x] = best;
    part_idx[blockIdx.x] = best_index;
    part_bad[blockIdx.x] = bad;
  }
}

#define XPU_Q3_REG_SET(NC)                                                                                     \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_norm_gemv_r2_v##NC(                                \
      const uint16_t *__restrict__ W, uint16_t *x, const uint16_t *__restrict__ norm_w,                       \
      uint16_t *__restrict__ out, uint32_t M, uint32_t K, float eps, const uint16_t *__restrict__ embed,      \
      const uint32_t *__restrict__ state, uint32_t vocab) {                                                   \
    XPU_STAMP(xpu::kStampQ3Qkv);                                                                              \
    q3_norm_gemv_reg<2, NC>(W, x, norm_w, out, M, K, eps, embed, state, vocab);                               \
  }                                                                                                           \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_gemv_residual_r1_v##NC(                            \
      const uint16_t *__restrict__ W, const uint16_t *__restrict__ v, uint16_t *x, uint32_t M, uint32_t K) {  \
    XPU_STAMP(xpu::kStampQ3Residual);                                                                         \
    q3_gemv_residual_reg<1, NC>(W, v, x, M, K);                                                               \
  }                                                                                                           \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_norm_gemv_swiglu_r2_v##NC(                         \
      const uint16_t *__restrict__ Wgu, const uint16_t *__restrict__ x, const uint16_t *__restrict__ norm_w,  \
      uint16_t *__restrict__ h, uint32_t I, uint32_t K, float eps) {                                          \
    XPU_STAMP(xpu::kStampQ3Swiglu);                                                                           \
    q3_norm_gemv_swiglu_reg<2, NC>(Wgu, x, norm_w, h, I, K, eps);                                             \
  }                                                                                                           \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_norm_gemv_logits_r2_v##NC(                         \
      const uint16_t *__restrict__ E, const uint16_t *__restrict__ x, const uint16_t *__restrict__ norm_w,    \
      uint16_t *__restrict__ logits, uint32_t V, uint32_t K, float eps, float *__restrict__ part_val,         \
      uint32_t *__restrict__ part_idx, uint32_t *__restrict__ part_bad) {                                     \
    XPU_STAMP(xpu::kStampQ3Logits);                                                                           \
    q3_norm_gemv_logits_reg<2, NC>(E, x, norm_w, logits, V, K, eps, part_val, part_idx, part_bad);            \
  }

XPU_Q3_REG_SET(1)
XPU_Q3_REG_SET(2)
XPU_Q3_REG_SET(4)
XPU_Q3_REG_SET(6)
XPU_Q3_REG_SET(8)

// One block per query head: QK-norm + RoPE of q and of its kv head's k,
// attention over positions 0..state[0] (position state[0] itself from the
// roped k and the qkv row), then the first query head of each group writes k
// and v into the engine caches at position state[0].
// cos_row / sin_row are the RoPE table rows of position state[0] (the engine
// keeps them in a fixed buffer, rewritten whenever the position changes), so
// that no load before the QK-norm depends on the position.
//
// Contexts of up to kAttnTile positions (thread t <-> position t) take three
// block barriers: the loads that do not depend on the position are issued at
// entry without branches (q/k rows, norm gains and cos/sin first, so the
// QK-norm / RoPE of waves 0 and 1 only waits for those; then the thread's K
// row from the chunk-major cache), the position is first used after barrier
// 1; the V pieces in the P.V layout are loaded after the scores, so that they
// do not queue ahead of the K rows; the softmax maximum goes through one LDS
// exchange; the canonical denominator is folded in registers (the 8 slots
// of canonical lane L are the exponentials of positions 8 L .. 8 L + 7,
// held by 8 consecutive lanes, folded with quad permutations and a half-row
// mirror) and its 64-lane butterfly is evaluated by every wave from LDS;
// then P.V (lane <-> residue class, wave <-> four cache chunks) and the fixed
// class tree across the 16 lanes of a chunk. Same operations in the same
// order as attention_tail_short. Longer contexts use attention_head, or the
// split kernels below.
extern "C" __global__ __launch_bounds__(256) void xpu_q3_attention(
    const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ qnorm_w,
    const uint16_t *__restrict__ knorm_w, const uint16_t *__restrict__ cos_row,
    const uint16_t *__restrict__ sin_row, uint16_t *__restrict__ kcache,
    uint16_t *__restrict__ vcache, uint16_t *__restrict__ out, const uint32_t *__restrict__ state,
    uint32_t heads, uint32_t kv_heads, uint32_t max_seq, float eps, float scale,
    const uint16_t *__restrict__ prefetch, uint64_t prefetch_bytes, uint32_t prefetch_delay) {
  XPU_STAMP(xpu::kStampQ3Attention);
  __shared__ float sbuf[xpu::kAttnChunk];
  __shared__ float red[4 * xpu::kHeadDim];
  __shared__ __align__(16) uint16_t qs[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t ks[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t junk[2 * xpu::kHeadDim];
  __shared__ __align__(16) uint16_t vtile[xpu::kAttnTile * xpu::kVPitch];
  const uint32_t head = blockIdx.x;
  if (head >= heads) {
    // Blocks past the query heads read [prefetch, prefetch + prefetch_bytes)
    // (the weights of the kernels that follow) so that they come from the
    // Infinity Cache, not HBM, when those kernels run; the attention itself
    // occupies only `heads` compute units for its latency-bound duration.
    // start after prefetch_delay x 64 x 8 cycles, behind the attention's
    // own loads
    for (uint32_t d = 0; d < prefetch_delay; ++d) __builtin_amdgcn_s_sleep(8);
    // 8 16-byte loads in flight per thread, branch-free (indices past the
    // range re-read its last word): the prefetch then ends before the query
    // heads (4 loads in flight outlasted them by ~1 us, 16 slowed them)
    constexpr int kUnroll = 8;
    const uint64_t n16 = prefetch_bytes / 16u;
    if (n16 == 0) return;
    const u32x4 *p = reinterpret_cast<const u32x4 *>(prefetch);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x - heads) * blockDim.x;
    uint32_t acc = 0;
    for (uint64_t i = static_cast<uint64_t>(head - heads) * blockDim.x + threadIdx.x; i < n16; i += kUnroll * stride) {
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = p[min(i + u * stride, n16 - 1)];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].w;
    }
    asm volatile("" : : "v"(acc));  // keeps the loads
    return;
  }
  // the position: a scalar load issued early, so that its latency overlaps
  // the operand loads and the QK-norm instead of following barrier 1
  uint32_t pos = state[0];
  const uint32_t group = heads / kv_heads;
  const uint32_t kv = head / group;
  const uint16_t *qsrc = qkv + head * xpu::kHeadDim;
  const uint16_t *ksrc = qkv + (heads + kv) * xpu::kHeadDim;
  const uint16_t *vsrc = qkv + (heads + kv_heads + kv) * xpu::kHeadDim;
  const uint32_t tid = threadIdx.x, lane = xpu::lane_id();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint64_t head_base = static_cast<uint64_t>(kv) * max_seq * xpu::kHeadDim;
  const uint64_t kchunk = static_cast<uint64_t>(max_seq) * 8u;  // chunk-major K cache
  // QK-norm / RoPE operands (waves 0: q, 1: k; lanes 0..15 used)
  const uint32_t l16 = lane & 15u;
  const u32x4 hx = *reinterpret_cast<const u32x4 *>((wave == 0 ? qsrc : ksrc) + l16 * 8u);
  const u32x4 hw = *reinterpret_cast<const u32x4 *>((wave == 0 ? qnorm_w : knorm_w) + l16 * 8u);
  const u32x4 hc = *reinterpret_cast<const u32x4 *>(cos_row + l16 * 8u);
  const u32x4 hs = *reinterpret_cast<const u32x4 *>(sin_row + l16 * 8u);
  const u32x4 hv = *reinterpret_cast<const u32x4 *>(vsrc + l16 * 8u);  // the new v row
  __builtin_amdgcn_sched_barrier(0);  // these five loads go out first
  // K row of position tid (clamped into the cache; positions >= pos are
  // replaced below)
  u32x4 krow[16];
  xpu::load_head_row(kcache + head_base + static_cast<uint64_t>(min(tid, max_seq - 1)) * 8u, krow, kchunk);
  // the position in a register here, while the vector loads are in flight
  // (otherwise the compiler issues its load next to its first use)
  asm volatile("" : "+s"(pos));
  {
    // every wave evaluates a QK-norm / RoPE (waves 2 and 3 into scratch) so
    // that the four operand loads stay ahead of the K loads
    const bool active = lane < 16;
    const u32x4 zero{0, 0, 0, 0};
    xpu::head_norm_rope_vec(active ? hx : zero, active ? hw : zero, hc, hs, eps,
                            wave == 0 ? qs : wave == 1 ? ks : junk + (wave - 2) * xpu::kHeadDim);
  }
  __syncthreads();  // 1: qs, ks
  XPU_PHASE(0);     // (stamps build) operand loads, QK-norm and RoPE done
  if (pos >= max_seq) return;  // the reference skips the step (kernels.hpp:74-75)
  const uint32_t n = pos + 1;
  const bool short_ctx = n <= xpu::kAttnTile;
  // The new k and v (chunk-major) at position pos, stored by the first query
  // head of each group after its output: this kernel reads position pos from
  // ks / the qkv row, never from the caches, so the stores stay off the
  // wait for the K rows (on gfx950 stores count in vmcnt like loads).
  auto store_kv = [&]() {
    if (head % group == 0 && tid < 16) {
      *reinterpret_cast<u32x4 *>(kcache + head_base + tid * kchunk + static_cast<uint64_t>(pos) * 8u) =
          *reinterpret_cast<const u32x4 *>(ks + tid * 8u);
      *reinterpret_cast<u32x4 *>(vcache + head_base + tid * kchunk + static_cast<uint64_t>(pos) * 8u) = hv;
    }
  };
  if (!short_ctx) {
    xpu::attention_head<true>(qs, kcache + head_base, vcache + head_base,
                              xpu::KvLayout{8u, kchunk, 8u, kchunk}, n, ks, vsrc, scale,
                              out + head * xpu::kHeadDim, sbuf, vtile, red);
    store_kv();
    return;
  }
  // scores (the current position from ks) and the block maximum
  if (tid == pos) xpu::load_head_row(ks, krow);
  const float sc = tid < n ? xpu::attention_score_regs(qs, krow, scale) : -__builtin_inff();
  // V pieces: lane l of wave w owns residue class cls = l % 16 and cache
  // chunk vch = 4 w + l / 16 (dims 8 vch .. + 7); vpv[it] = V[16 it + cls]
  // (the current position's v from qkv; entries past pos are not used), so
  // a load instruction reads 256 contiguous bytes of each of 4 chunks
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
  __syncthreads();  // 2: wave maxima
  XPU_PHASE(1);     // (stamps build) scores and their maximum done
  const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // exponentials; canonical lane L = tid / 8 folds its 8 slots
  const float ex = tid < n ? xpu::canonical_exp(sc - mx) : 0.0f;
  sbuf[tid] = ex;
  float f = ex + xpu::dpp_f<0xB1>(ex);  // (a0 + a1), (a2 + a3), ...
  f = f + xpu::dpp_f<0x4E>(f);          // (a0 + a1) + (a2 + a3)
  f = f + xpu::dpp_f<0x141>(f);         // row_half_mirror: the other quad of the eight
  float *lane_sum = red + 4;            // 32 canonical lane sums (n <= 256)
  if ((tid & 7u) == 0) lane_sum[tid >> 3] = f;
  __syncthreads();  // 3: exponentials and lane sums
  XPU_PHASE(2);     // (stamps build) exponentials and the denominator's lane sums done
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
  // the class tree over the 16 lanes of a chunk: (c0 + c1), then
  // ((c0 + c1) + (c2 + c3)), then the two quads of eight (half-row mirror:
  // the values are uniform within a quad), then the two eights
  uint32_t code[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float v = part[e];
    v = v + xpu::dpp_f<0xB1>(v);   // xor 1
    v = v + xpu::dpp_f<0x4E>(v);   // xor 2
    v = v + xpu::dpp_f<0x141>(v);  // row_half_mirror
    v = v + xpu::xor8_f(v);
    code[e] = xpu::f32_to_bf16(v);
  }
  if (cls == 0)
    *reinterpret_cast<u32x4 *>(out + head * xpu::kHeadDim + vch * 8u) =
        u32x4{code[0] | (code[1] << 16), code[2] | (code[3] << 16), code[4] | (code[5] << 16), code[6] | (code[7] << 16)};
  store_kv();
}

// Attention split over compute units (two kernels, for long contexts): the
// operations and their order are those of xpu_q3_attention /
// attention_head (qwen3/kernels.hpp:157-192 with transformers rounding), so
// results are bit-identical; the work of one head is spread over many
// blocks because one compute unit's load path bounds a block that reads a
// long K/V history.
//
// Block b of both kernels serves kv head b % kv_heads, query head
// kv_head * group + (b / kv_heads) % group and part (b / kv_heads) / group,
// so with 8 kv heads and round-robin dispatch over 8 XCDs all blocks of a
// kv head share one L2.
XPU_DEVICE void split_block(uint32_t b, uint32_t heads, uint32_t kv_heads, uint32_t &kv, uint32_t &head,
                            uint32_t &part) {
  const uint32_t group = heads / kv_heads, rest = b / kv_heads;
  kv = b % kv_heads;
  head = kv * group + rest % group;
  part = rest / group;
}

// Part 1: QK-norm + RoPE of q and of its kv head's k (every block; after
// its scores the first query head of each group with part 0 writes k and v
// into the caches at position state[0]), then the scores of the 256-position tiles
// part, part + parts, ... (thread t <-> position tile * 256 + t, the current
// position from the freshly roped k) into scores[head * spitch + t], and the
// block's maximum into maxima[head * parts + part] (-inf without a tile).
// grid = heads * parts; cos_row / sin_row as for xpu_q3_attention.
extern "C" __global__ __launch_bounds__(256) void xpu_q3_attn_scores(
    const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ qnorm_w,
    const uint16_t *__restrict__ knorm_w, const uint16_t *__restrict__ cos_row,
    const uint16_t *__restrict__ sin_row, uint16_t *__restrict__ kcache,
    uint16_t *__restrict__ vcache, float *__restrict__ scores, float *__restrict__ maxima,
    const uint32_t *__restrict__ state, uint32_t heads, uint32_t kv_heads, uint32_t max_seq,
    uint32_t spitch, uint32_t parts, float eps, float scale) {
  XPU_STAMP(xpu::kStampQ3Scores);
  __shared__ float red[4];
  __shared__ __align__(16) uint16_t qs[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t ks[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t junk[2 * xpu::kHeadDim];
  uint32_t pos = state[0];  // issued early (see xpu_q3_attention)
  uint32_t kv, head, part;
  split_block(blockIdx.x, heads, kv_heads, kv, head, part);
  const uint32_t group = heads / kv_heads;
  const uint16_t *qsrc = qkv + head * xpu::kHeadDim;
  const uint16_t *ksrc = qkv + (heads + kv) * xpu::kHeadDim;
  const uint16_t *vsrc = qkv + (heads + kv_heads + kv) * xpu::kHeadDim;
  const uint32_t tid = threadIdx.x, lane = xpu::lane_id();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint64_t head_base = static_cast<uint64_t>(kv) * max_seq * xpu::kHeadDim;
  const uint64_t kchunk = static_cast<uint64_t>(max_seq) * 8u;  // chunk-major K cache
  const uint32_t l16 = lane & 15u;
  const u32x4 hx = *reinterpret_cast<const u32x4 *>((wave == 0 ? qsrc : ksrc) + l16 * 8u);
  const u32x4 hw = *reinterpret_cast<const u32x4 *>((wave == 0 ? qnorm_w : knorm_w) + l16 * 8u);
  const u32x4 hc = *reinterpret_cast<const u32x4 *>(cos_row + l16 * 8u);
  const u32x4 hs = *reinterpret_cast<const u32x4 *>(sin_row + l16 * 8u);
  const u32x4 hv = *reinterpret_cast<const u32x4 *>(vsrc + l16 * 8u);
  __builtin_amdgcn_sched_barrier(0);  // these five loads go out first
  // K row of this thread's position in the block's first tile (clamped into
  // the cache; positions past the context are not used)
  u32x4 knext[16];
  xpu::load_head_row(kcache + head_base + static_cast<uint64_t>(min(part * 256u + tid, max_seq - 1)) * 8u, knext,
                     kchunk);
  asm volatile("" : "+s"(pos));  // the position in a register while the vector loads are in flight
  {
    const bool active = lane < 16;
    const u32x4 zero{0, 0, 0, 0};
    xpu::head_norm_rope_vec(active ? hx : zero, active ? hw : zero, hc, hs, eps,
                            wave == 0 ? qs : wave == 1 ? ks : junk + (wave - 2) * xpu::kHeadDim);
  }
  __syncthreads();  // qs, ks
  if (pos >= max_seq) return;  // the reference skips the step (kernels.hpp:74-75)
  const uint32_t n = pos + 1, ntiles = (n + 255u) / 256u;
  float *srow = scores + static_cast<uint64_t>(head) * spitch;
  float local_max = -__builtin_inff();
  for (uint32_t tile = part; tile < ntiles; tile += parts) {
    u32x4 kcur[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) kcur[j] = knext[j];
    if (tile + parts < ntiles)  // the next tile's row, loaded while this one is scored
      xpu::load_head_row(kcache + head_base + static_cast<uint64_t>(min((tile + parts) * 256u + tid, max_seq - 1)) * 8u,
                         knext, kchunk);
    const uint32_t t = tile * 256u + tid;
    if (t < n) {
      const float s = t == pos ? xpu::attention_score(qs, ks, scale) : xpu::attention_score_regs(qs, kcur, scale);
      srow[t] = s;
      local_max = fmaxf(local_max, s);
    }
  }
  // the new k and v at position pos, after the scores (which take position
  // pos from ks): xpu_q3_attn_pv, the next kernel, reads them from the caches
  if (head % group == 0 && part == 0 && tid < 16) {
    *reinterpret_cast<u32x4 *>(kcache + head_base + tid * kchunk + static_cast<uint64_t>(pos) * 8u) =
        *reinterpret_cast<const u32x4 *>(ks + tid * 8u);
    *reinterpret_cast<u32x4 *>(vcache + head_base + tid * kchunk + static_cast<uint64_t>(pos) * 8u) = hv;
  }
  const float wmax = xpu::wave_reduce(local_max, [](float x, float y) { return fmaxf(x, y); });
  if (lane == 0) red[wave] = wmax;
  __syncthreads();
  if (tid == 0) maxima[head * parts + part] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Part 2: block (kv head, query head, dim group g) of grid heads * 8 owns
// dims 16 g .. 16 g + 15 of its head's output. Every block rebuilds the
// softmax maximum (from the parts' maxima) and the canonical denominator
// (chunks of kAttnChunk positions: lane L adds the exponentials of
// positions 512 j + 8 L + e of the chunk into slot e, the chunk sum is the
// 8 -> 1 fold and 64-lane butterfly, chunk sums are added in order), then
// p_t = bf16(exp(s_t - max) * (1 / sum)) and, for each of its 16 dims, the
// 16 residue-class FMA chains over ascending t (one chain per chunk, chunks
// added in order), combined by the fixed class tree ((c0 + c1) + (c2 + c3))
// ... as attention_tail does. The exponentials of a chunk are computed once
// by all threads into LDS; the block's 32-byte slice of the V rows goes
// through registers into LDS in 1024-row tiles, each tile loaded while the
// previous one's chains run; the chains take their operands 16 steps at a
// time from LDS. spitch: a multiple of 512.
extern "C" __global__ __launch_bounds__(256) void xpu_q3_attn_pv(
    const float *__restrict__ scores, const float *__restrict__ maxima, const uint16_t *__restrict__ vcache,
    uint16_t *__restrict__ out, const uint32_t *__restrict__ state, uint32_t heads, uint32_t kv_heads,
    uint32_t max_seq, uint32_t spitch, uint32_t parts) {
  XPU_STAMP(xpu::kStampQ3Pv);
  constexpr uint32_t kDims = 16, kChunk = xpu::kAttnChunk, kTile = 1024, kRows = kTile / 128, kMaxChunks = 64;
  constexpr uint32_t kPer = kChunk / 256, kBatch = 16;
  extern __shared__ __align__(16) uint8_t pv_lds[];
  float *pbuf = reinterpret_cast<float *>(pv_lds);                           // kChunk floats
  uint16_t *vt = reinterpret_cast<uint16_t *>(pv_lds + kChunk * 4);         // kChunk x 16 codes
  float *csum = reinterpret_cast<float *>(pv_lds + kChunk * 4 + kChunk * kDims * 2);
  float *wsum = csum + kMaxChunks;                                           // 4 x 16
  uint32_t kv, head, g;
  split_block(blockIdx.x, heads, kv_heads, kv, head, g);
  const uint32_t tid = threadIdx.x, lane = xpu::lane_id();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float pm = maxima[head * parts + min(lane, parts - 1)];
  const uint32_t pos = state[0];
  if (pos >= max_seq) return;
  const uint32_t n = pos + 1, nchunks = (n + kChunk - 1) / kChunk;
  const float *srow = scores + static_cast<uint64_t>(head) * spitch;
  // the chunk's scores (16 per thread, positions tid + 256 k, index clamped)
  auto load_s = [&](uint32_t base, uint32_t len, float (&sv)[kPer]) {
#pragma unroll
    for (int k = 0; k < static_cast<int>(kPer); ++k) sv[k] = srow[base + min(tid + 256u * k, len - 1)];
  };
  // V rows from the chunk-major cache (dims 16 g .. 16 g + 15 are cache
  // chunks 2 g and 2 g + 1): waves 0, 1 read chunk 2 g and waves 2, 3 chunk
  // 2 g + 1, lane l of wave w rows 128 k + 64 (w % 2) + l of a tile, so a
  // load instruction reads 1 KiB contiguous. The loads go through a buffer
  // descriptor that ends at the context: rows past it read zeros without a
  // memory access, and no load is behind a branch (which would make the
  // compiler wait for all earlier loads before each one).
  const uint32_t vr = (wave & 1u) * 64u + lane, vh = (wave >> 1) * 8u;
  const uint16_t *vb = vcache + static_cast<uint64_t>(kv) * max_seq * xpu::kHeadDim +
                       static_cast<uint64_t>(2u * g + (wave >> 1)) * max_seq * 8u;
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(vb), static_cast<short>(0), static_cast<int>(n * 16u),
                                        0x00020000);
  auto load_tile = [&](uint32_t t0, u32x4 (&vv)[kRows]) {  // rows t0 .. t0 + 1023 of the context
#pragma unroll
    for (int k = 0; k < static_cast<int>(kRows); ++k)
      vv[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, (t0 + k * 128u + vr) * 16u, 0, 0));
  };
  auto store_tile = [&](uint32_t r0, const u32x4 (&vv)[kRows]) {  // into chunk rows r0 .. r0 + 1023
#pragma unroll
    for (int k = 0; k < static_cast<int>(kRows); ++k)
      *reinterpret_cast<u32x4 *>(vt + (r0 + k * 128u + vr) * kDims + vh) = vv[k];
  };
  float sv[kPer];
  u32x4 vv[kRows];
  load_s(0, min(kChunk, n), sv);
  load_tile(0, vv);
  const float mx = xpu::wave_reduce(pm, [](float x, float y) { return fmaxf(x, y); });
  XPU_PHASE(0);  // (stamps build) the softmax maximum
  auto exps = [&](uint32_t len, const float (&s)[kPer], bool scaled, float sinv) {
#pragma unroll
    for (int k = 0; k < static_cast<int>(kPer); ++k) {
      const uint32_t i = tid + 256u * k;
      if (i < len) {
        const float e = xpu::canonical_exp(s[k] - mx);
        pbuf[i] = scaled ? xpu::round_bf16(e * sinv) : e;
      }
    }
  };
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t base = c * kChunk, len = min(kChunk, n - base);
    if (c) {
      float sc[kPer];
      load_s(base, len, sc);
      exps(len, sc, false, 0.0f);
    } else {
      exps(len, sv, false, 0.0f);
    }
    __syncthreads();
    if (wave == 0) {
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (uint32_t j = 0; j < len; j += 512u) {
        const float4 a = *reinterpret_cast<const float4 *>(pbuf + j + lane * 8u);
        const float4 b = *reinterpret_cast<const float4 *>(pbuf + j + lane * 8u + 4u);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (j + lane * 8u + e < len) acc[e] = acc[e] + x[e];
      }
      const float cs = xpu::wave_butterfly(xpu::fold8(acc));
      if (lane == 0) csum[c] = cs;
    }
    __syncthreads();
  }
  XPU_PHASE(1);  // (stamps build) exponentials and the denominator's chunk sums
  float total = 0.0f;
  for (uint32_t c = 0; c < nchunks; ++c) total = total + csum[c];
  const float inv = 1.0f / total;
  // P.V: lane l of wave w owns residue class 4 w + l / 16 and dim l % 16
  const uint32_t cls = wave * 4u + (lane >> 4), d = lane & 15u;
  float tot = 0.0f;
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t base = c * kChunk, len = min(kChunk, n - base);
    if (c) {
      __syncthreads();  // the previous chunk's probabilities and rows are no longer read
      float sc[kPer];
      load_s(base, len, sc);
      exps(len, sc, true, inv);
    } else if (nchunks == 1) {
      for (uint32_t i = tid; i < len; i += 256u) pbuf[i] = xpu::round_bf16(pbuf[i] * inv);
    } else {
      exps(len, sv, true, inv);
    }
    XPU_PHASE(2);  // (stamps build) the (last) chunk's probabilities
    float part = 0.0f;
    for (uint32_t i0 = 0; i0 < len; i0 += kTile) {
      store_tile(i0, vv);  // a region of the chunk's rows that no chain reads yet
      load_tile(base + i0 + kTile, vv);  // the next tile (zeros past the context)
      __syncthreads();  // the tile (and the chunk's probabilities) in LDS
      // rows i0 + cls, i0 + cls + 16, ... of the tile, 16 at a time: the
      // operands of a batch are read before its FMAs
      const uint32_t tend = min(i0 + kTile, len);
      uint32_t t0 = i0 + cls;
      for (; t0 + 16u * (kBatch - 1) < tend; t0 += 16u * kBatch) {
        float pp[kBatch];
        uint32_t v[kBatch];
#pragma unroll
        for (int u = 0; u < static_cast<int>(kBatch); ++u) {
          pp[u] = pbuf[t0 + 16u * u];
          v[u] = vt[(t0 + 16u * u) * kDims + d];
        }
#pragma unroll
        for (int u = 0; u < static_cast<int>(kBatch); ++u) part = __builtin_fmaf(pp[u], xpu::bf16_to_f32(v[u]), part);
      }
      for (; t0 < tend; t0 += 16u) part = __builtin_fmaf(pbuf[t0], xpu::bf16_to_f32(vt[t0 * kDims + d]), part);
    }
    tot = tot + part;
  }
  XPU_PHASE(3);  // (stamps build) the V tiles and their chains
  const float pair = tot + xpu::xor16_f(tot);  // (c0 + c1), (c2 + c3)
  const float sum = pair + xpu::xor32_f(pair); // (c0 + c1) + (c2 + c3)
  if (lane < 16) wsum[wave * kDims + lane] = sum;
  __syncthreads();
  if (tid < kDims) {
    const float r = (wsum[tid] + wsum[kDims + tid]) + (wsum[2 * kDims + tid] + wsum[3 * kDims + tid]);
    out[head * xpu::kHeadDim + g * kDims + tid] = static_cast<uint16_t>(xpu::f32_to_bf16(r));
  }
}

// Reduce the per-block argmax partials; token = 0xffffffff if any logit was
// non-finite. Then advance: position + 1, next token = next prompt id while
// the prompt lasts (state[3] = prompt length), else the argmax; the argmax
// after position p >= prompt length - 1 is stored at gen[p + 1 - length].
// state: [0] position, [1] input token, [2] last argmax, [3] prompt length.
extern "C" __global__ __launch_bounds__(1024) void xpu_q3_argmax_finish(
    const float *__restrict__ part_val, const uint32_t *__restrict__ part_idx,
    const uint32_t *__restrict__ part_bad, uint32_t nparts, uint32_t *state,
    const uint32_t *__restrict__ prompt, uint32_t *__restrict__ gen, uint32_t gen_capacity,
    const uint16_t *__restrict__ rope_cos, const uint16_t *__restrict__ rope_sin,
    uint16_t *__restrict__ rope_row, uint32_t max_seq) {
  XPU_STAMP(xpu::kStampQ3Finish);
  constexpr uint32_t kBlock = 1024;  // launched with 1024 threads
  __shared__ float redv[16];
  __shared__ uint32_t redi[16], redb[16];
  float best = -__builtin_inff();
  uint32_t best_index = 0xffffffffu, bad = 0;
  for (uint32_t i = threadIdx.x; i < nparts; i += kBlock) {
    bad |= part_bad[i];
    xpu::argmax_merge(best, best_index, part_val[i], part_idx[i]);
  }
  {
    // the RoPE rows of the next position into rope_row (cos, then sin), read
    // by the next step's attention kernels; state[0] is read here, before the
    // barriers of block_argmax, and advanced by thread 0 after them
    const uint32_t next_pos = state[0] + 1;
    const uint32_t i = threadIdx.x;
    if (next_pos < max_seq && i < 2 * xpu::kHeadDim)
      rope_row[i] = i < xpu::kHeadDim ? rope_cos[static_cast<uint64_t>(next_pos) * xpu::kHeadDim + i]
                                      : rope_sin[static_cast<uint64_t>(next_pos) * xpu::kHeadDim + i - xpu::kHeadDim];
  }
  xpu::block_argmax(best, best_index, bad, redv, redi, redb);
  if (threadIdx.x == 0) {
    const uint32_t token = bad ? 0xffffffffu : (best_index == 0xffffffffu ? 0u : best_index);
    const uint32_t pos = state[0], n_prompt = state[3];
    const uint32_t next_pos = pos + 1;
    state[2] = token;
    state[1] = next_pos < n_prompt ? prompt[next_pos] : token;
    state[0] = next_pos;
    if (next_pos >= n_prompt) {
      const uint32_t g = next_pos - n_prompt;
      if (g < gen_capacity) gen[g] = token;
    }
  }
}

// ------------------------------------------------------------ batched prefill
//
// Part 3: the prompt positions go through the model as one batch per layer
// (the K/V cache entries of every position; the engine finishes the last
// position's last layer and head with the decode step's kernels, which
// produce the first generated token). Every value is computed with the same
// operations in the same order as the decode kernels, so the cache contents
// and that token's logits are bit-identical to decoding the prompt one
// position at a time (qwen3/main.cpp:343-344).
// Buffers hold T tokens of a chunk: X, Xn [T][H], QKV [T][(Hq+2Hkv)*128],
// Q and A [T][Hq*128], Hb [T][I].

// X[t] = embed[prompt[p0 + t]]
extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_embed(const uint16_t *__restrict__ embed,
                                                                  const uint32_t *__restrict__ prompt, uint32_t p0,
                                                                  uint16_t *__restrict__ X, uint32_t H, uint32_t vocab) {
  const uint32_t t = blockIdx.x;
  uint32_t token = prompt[p0 + t];
  if (token >= vocab) token = 0;
  const uint16_t *src = embed + static_cast<uint64_t>(token) * H;
  for (uint32_t i = threadIdx.x; i < H; i += blockDim.x) X[static_cast<uint64_t>(t) * H + i] = src[i];
}

// Xn[t] = rmsnorm(X[t]) * w, one wavefront per token (4 per 256-thread
// block, grid ceil(T / 4)); H a multiple of 8, X, w, Xn 16-byte aligned.
// The operations of block_rmsnorm_vec in the same order: lane l accumulates
// the squares of elements 512 c + 8 l + slot over chunks c in order (a
// missing tail reads as zeros, as that kernel's zero padding), then fold8
// and the 64-lane butterfly; out = bf16(w * bf16(x * scale)). The first
// kRegChunks chunks of x and w are loaded once, up front, and kept in
// registers; wider rows re-read the rest.
extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_rmsnorm(const uint16_t *__restrict__ X,
                                                                    const uint16_t *__restrict__ w,
                                                                    uint16_t *__restrict__ Xn, uint32_t H, float eps,
                                                                    uint32_t T) {
  constexpr uint32_t kRegChunks = 8;
  const uint32_t t = blockIdx.x * 4u + (threadIdx.x >> 6), lane = xpu::lane_id();
  if (t >= T) return;  // whole wavefronts
  const uint16_t *x = X + static_cast<uint64_t>(t) * H;
  u32x4 xv[kRegChunks], wv[kRegChunks];
#pragma unroll
  for (uint32_t c = 0; c < kRegChunks; ++c) {
    const uint32_t j = c * 512u + lane * 8u;
    xv[c] = j < H ? *reinterpret_cast<const u32x4 *>(x + j) : u32x4{0, 0, 0, 0};
    wv[c] = j < H ? *reinterpret_cast<const u32x4 *>(w + j) : u32x4{0, 0, 0, 0};
  }
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (uint32_t c = 0; c < kRegChunks; ++c) {
    if (c * 512u >= H) break;  // uniform
    float f[8];
    xpu::unpack8<xpu::kBf16>(xv[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(f[e], f[e], acc[e]);
  }
  for (uint32_t j = kRegChunks * 512u + lane * 8u; j < H; j += 512u) {
    float f[8];
    xpu::unpack8<xpu::kBf16>(*reinterpret_cast<const u32x4 *>(x + j), f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(f[e], f[e], acc[e]);
  }
  const float ss = xpu::wave_butterfly(xpu::fold8(acc));
  const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(H) + eps);
  uint16_t *out = Xn + static_cast<uint64_t>(t) * H;
  auto emit = [&](const u32x4 &xq, const u32x4 &wq, uint32_t j) {
    float xf[8], wf[8];
    xpu::unpack8<xpu::kBf16>(xq, xf);
    xpu::unpack8<xpu::kBf16>(wq, wf);
    uint32_t c[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) c[e] = xpu::f32_to_bf16(wf[e] * xpu::round_bf16(xf[e] * scale));
    *reinterpret_cast<u32x4 *>(out + j) =
        u32x4{c[0] | (c[1] << 16), c[2] | (c[3] << 16), c[4] | (c[5] << 16), c[6] | (c[7] << 16)};
  };
#pragma unroll
  for (uint32_t c = 0; c < kRegChunks; ++c) {
    const uint32_t j = c * 512u + lane * 8u;
    if (j < H) emit(xv[c], wv[c], j);
  }
  for (uint32_t j = kRegChunks * 512u + lane * 8u; j < H; j += 512u)
    emit(*reinterpret_cast<const u32x4 *>(x + j), *reinterpret_cast<const u32x4 *>(w + j), j);
}

// Hb[t][i] = bf16(bf16(silu(g)) u) for g = GU[t][i], u = GU[t][I + i]: the
// SiLU-multiply after the MFMA form of the prompt's [gate; up] projection
// (GU [T][2I], its gate and up halves side by side). The rounding points
// are silu_mul_code's; silu(g) = g * rcp(1 + exp2(-g log2 e)) takes the
// hardware exp2 and reciprocal (a few FP32 ulps from the canonical exp and
// the IEEE division; this prompt form is checked by tolerance). Block
// (x, y): 8 outputs per thread at columns 8 (256 x + thread) of tokens
// kPfSiluTok y .. + kPfSiluTok - 1, all loads issued before the math
// (grid ceil(I / 2048) x ceil(T / kPfSiluTok); I % 8 == 0).
constexpr uint32_t kPfSiluTok = 4;
extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_silu_mul(const uint16_t *__restrict__ GU,
                                                                     uint16_t *__restrict__ Hb, uint32_t I,
                                                                     uint32_t T) {
  const uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 8u, t0 = blockIdx.y * kPfSiluTok;
  if (i >= I) return;
  constexpr float kLog2e = 1.44269504088896340736f;
  u32x4 g[kPfSiluTok], u[kPfSiluTok];
#pragma unroll
  for (uint32_t k = 0; k < kPfSiluTok; ++k) {
    const uint64_t t = min(t0 + k, T - 1u);  // tokens past the last re-read it (not stored)
    g[k] = *reinterpret_cast<const u32x4 *>(GU + t * 2u * I + i);
    u[k] = *reinterpret_cast<const u32x4 *>(GU + t * 2u * I + I + i);
  }
#pragma unroll
  for (uint32_t k = 0; k < kPfSiluTok; ++k) {
    if (t0 + k >= T) break;
    const uint32_t gw[4] = {g[k].x, g[k].y, g[k].z, g[k].w}, uw[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
    uint32_t hw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float gv = xpu::bf16_to_f32((gw[q] >> (16 * e)) & 0xffffu);
        const float uv = xpu::bf16_to_f32((uw[q] >> (16 * e)) & 0xffffu);
        // g -> -inf: exp2 = inf, rcp = 0, act = -0; g -> +inf: act = g
        const float act =
            xpu::round_bf16(gv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gv * kLog2e)));
        h[e] = xpu::f32_to_bf16(act * uv);
      }
      hw[q] = h[0] | (h[1] << 16);
    }
    *reinterpret_cast<u32x4 *>(Hb + static_cast<uint64_t>(t0 + k) * I + i) = u32x4{hw[0], hw[1], hw[2], hw[3]};
  }
}

namespace {

// Batched canonical GEMV: Out[t][row] for rows of W (M x K, K = 512 NC) and
// token rows In[t] (T x K). A wavefront holds R rows (PAIRED: rows i and
// I + i of a [gate; up] matrix, M = I) in registers for the whole token
// loop; the block stages TT token rows at a time in LDS, for token group
// blockIdx.y of gridDim.y (whole tiles; more rows per wavefront share each
// staged token's unpacking among more FMAs, and the token groups keep the
// block count up). Each (row, token)
// dot product is the decode GEMV's: lane l, slot s accumulate elements
// c*512 + 8 l + s over chunks c in order (FMA), then fold8 and the xor
// butterfly. EPI 0: Out = bf16(y); 1: Out = bf16(Out + bf16(y)) (residual);
// 2 (PAIRED): Out[t][i] = bf16(bf16(silu(bf16(g))) * bf16(u)).
//
// The 64-lane butterflies of the TT = 8 tokens of a tile are evaluated by
// recursive halving: at the l ^ 32, l ^ 16 and l ^ 8 steps each lane keeps
// half of its tokens (chosen by that lane bit) and adds the partner's value
// of the same token, own + partner, as the butterfly does; the l ^ 4, l ^ 2
// and l ^ 1 steps run on the one token left (4 b5 + 2 b4 + b3 of the lane
// index). Every sum is the butterfly's, with 10 exchanges instead of 48.
XPU_DEVICE float xor4_f(float v) {  // ds_swizzle, bit mode: and 0x1f, xor 4
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x101F));
}

template <int N>
XPU_DEVICE void halve_tokens(float (&v)[2 * N], float (&w)[N], bool upper, float (*xchg)(float)) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float keep = upper ? v[N + j] : v[j];
    const float send = upper ? v[j] : v[N + j];
    w[j] = keep + xchg(send);
  }
}

// the 64-lane sums of v[t] for t < 8, token 4 b5 + 2 b4 + b3 of this lane
XPU_DEVICE float token_butterfly8(float (&v)[8]) {
  const uint32_t lane = xpu::lane_id();
  float w4[4], w2[2], w1[1];
  halve_tokens<4>(v, w4, (lane & 32u) != 0, xpu::xor32_f);
  halve_tokens<2>(w4, w2, (lane & 16u) != 0, xpu::xor16_f);
  halve_tokens<1>(w2, w1, (lane & 8u) != 0, xpu::xor8_f);
  float s = w1[0];
  s = s + xor4_f(s);
  s = s + xpu::dpp_f<0x4E>(s);  // quad_perm [2,3,0,1]
  s = s + xpu::dpp_f<0xB1>(s);  // quad_perm [1,0,3,2]
  return s;
}

template <int R, int NC, int TT, int EPI, bool HOIST = (R * NC <= 12)>
XPU_DEVICE void pf_gemv(const uint16_t *__restrict__ W, const uint16_t *__restrict__ In, uint16_t *Out, uint32_t M,
                        uint32_t T) {
  constexpr uint32_t K = 512u * NC;
  constexpr bool kPaired = EPI == 2;
  constexpr int kOuts = kPaired ? R / 2 : R;         // outputs per wavefront
  constexpr uint32_t kTile = TT * K;                 // codes per token tile
  constexpr int kLoads = kTile / (256 * 8);          // 16-byte staging loads per thread
  static_assert(kTile % (256 * 8) == 0, "tile must split evenly over the block");
  // two tiles for K <= 2048; one past that (48 KiB at K = 3072, so up to
  // three blocks share a compute unit), its next tile stored after a barrier
  constexpr bool kDouble = NC <= 4;
  extern __shared__ __align__(16) uint16_t xt[];
  const uint32_t wave = threadIdx.x >> 6, lane = xpu::lane_id();
  const uint32_t o0 = (blockIdx.x * 4u + wave) * kOuts;  // first output of this wavefront
  const uint32_t rows_total = kPaired ? 2u * M : M;
  // the wavefront's rows, chunk c at columns c*512 + 8 lane
  u32x4 a[R][NC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t want = kPaired ? (r < R / 2 ? o0 + r : M + o0 + (r - R / 2)) : o0 + r;
    const uint32_t row = want < rows_total ? want : rows_total - 1;
    const uint16_t *p = W + static_cast<uint64_t>(row) * K + lane * 8u;
#pragma unroll
    for (int c = 0; c < NC; ++c) a[r][c] = xpu::load_nt16(p + c * 512u);
  }
  // the rows unpacked to FP32 once, when that fits the registers
  constexpr bool kHoist = HOIST;
  float af[kHoist ? R : 1][kHoist ? NC : 1][8];
  if constexpr (kHoist) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int c = 0; c < NC; ++c) xpu::unpack8<xpu::kBf16>(a[r][c], af[r][c]);
  }
  // token tiles are double buffered: the loads of tile i + 1 are issued
  // before the FMAs of tile i and stored to the other buffer after them
  u32x4 stage[kLoads];
  auto load_tile = [&](uint32_t t0) {
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
      const uint32_t i = (threadIdx.x + q * 256u) * 8u, tt = i / K, col = i % K;
      stage[q] = t0 + tt < T ? *reinterpret_cast<const u32x4 *>(In + static_cast<uint64_t>(t0 + tt) * K + col)
                             : u32x4{0, 0, 0, 0};
    }
  };
  auto store_tile = [&](uint16_t *buf) {
#pragma unroll
    for (int q = 0; q < kLoads; ++q) *reinterpret_cast<u32x4 *>(buf + (threadIdx.x + q * 256u) * 8u) = stage[q];
  };
  // token group blockIdx.y of gridDim.y: tokens [t_beg, t_end), whole tiles
  const uint32_t per_group = ((T + gridDim.y - 1) / gridDim.y + TT - 1) / TT * TT;
  const uint32_t t_beg = blockIdx.y * per_group, t_end = min(T, t_beg + per_group);
  if (t_beg >= t_end) return;  // whole block
  load_tile(t_beg);
  store_tile(xt);
  __syncthreads();
  uint32_t cur = 0;
  for (uint32_t t0 = t_beg; t0 < t_end; t0 += TT) {
    const bool more = t0 + TT < t_end;
    if (more) load_tile(t0 + TT);
    const uint16_t *tile = xt + (kDouble ? cur * kTile : 0u);
    static_assert(TT == 8, "token_butterfly8 reduces 8 tokens");
    // token by token: each slot's FMA chain over the chunks, then its fold,
    // so only one token's accumulators are live
    float v[R][TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      float acc[R][8];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float xf[8];
        xpu::unpack8<xpu::kBf16>(*reinterpret_cast<const u32x4 *>(tile + tt * K + c * 512u + lane * 8u), xf);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float aw[8];
          if constexpr (kHoist) {
#pragma unroll
            for (int e = 0; e < 8; ++e) aw[e] = af[r][c][e];
          } else {
            xpu::unpack8<xpu::kBf16>(a[r][c], aw);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(aw[e], xf[e], acc[r][e]);
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) v[r][tt] = xpu::fold8(acc[r]);
    }
    {
      // row r's sum for token tt_l = 4 b5 + 2 b4 + b3 of the lane; lane
      // 8 tt_l + o writes output o of that token
      float y[R];
#pragma unroll
      for (int r = 0; r < R; ++r) y[r] = token_butterfly8(v[r]);
      const uint32_t tt_l = ((lane >> 5) & 1u) * 4u + ((lane >> 4) & 1u) * 2u + ((lane >> 3) & 1u);
      const uint32_t t = t0 + tt_l;
      uint16_t *orow = Out + static_cast<uint64_t>(t) * M;
#pragma unroll
      for (int o = 0; o < kOuts; ++o) {
        if ((lane & 7u) != static_cast<uint32_t>(o) || t >= T || o0 + o >= M) continue;
        if constexpr (EPI == 0) {
          orow[o0 + o] = static_cast<uint16_t>(xpu::f32_to_bf16(y[o]));
        } else if constexpr (EPI == 1) {
          const float sum = xpu::bf16_to_f32(orow[o0 + o]) + xpu::round_bf16(y[o]);
          orow[o0 + o] = static_cast<uint16_t>(xpu::f32_to_bf16(sum));
        } else {
          orow[o0 + o] =
              static_cast<uint16_t>(silu_mul_code(xpu::round_bf16(y[o]), xpu::round_bf16(y[kOuts + o])));
        }
      }
    }
    if (more) {
      if constexpr (!kDouble) __syncthreads();  // every wavefront is done with the tile
      store_tile(xt + (kDouble ? (cur ^ 1u) * kTile : 0u));
      __syncthreads();
      cur ^= 1u;
    }
  }
}

}  // namespace

// xpu_q3_pf_gemv_e<EPI>_c<NC>_r<R>: R as large as fits the registers
// without spills (the engine takes the largest R the module has); _H: the
// rows held unpacked regardless of size
#define XPU_Q3_PF_GEMV(EPI, R, NC)                                                                  \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_gemv_e##EPI##_c##NC##_r##R(          \
      const uint16_t *__restrict__ W, const uint16_t *__restrict__ In, uint16_t *Out, uint32_t M,  \
      uint32_t T) {                                                                                 \
    pf_gemv<R, NC, 8, EPI>(W, In, Out, M, T);                                                       \
  }
#define XPU_Q3_PF_GEMV_H(EPI, R, NC)                                                                \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_gemv_e##EPI##_c##NC##_r##R(          \
      const uint16_t *__restrict__ W, const uint16_t *__restrict__ In, uint16_t *Out, uint32_t M,  \
      uint32_t T) {                                                                                 \
    pf_gemv<R, NC, 8, EPI, true>(W, In, Out, M, T);                                                 \
  }
XPU_Q3_PF_GEMV(0, 4, 2)
XPU_Q3_PF_GEMV(0, 4, 4)
XPU_Q3_PF_GEMV(0, 2, 8)
XPU_Q3_PF_GEMV(1, 2, 2)
XPU_Q3_PF_GEMV(1, 2, 4)
XPU_Q3_PF_GEMV_H(1, 4, 4)
XPU_Q3_PF_GEMV(1, 2, 6)
XPU_Q3_PF_GEMV(1, 1, 8)
XPU_Q3_PF_GEMV(2, 4, 2)
XPU_Q3_PF_GEMV(2, 4, 4)
XPU_Q3_PF_GEMV(2, 2, 8)

// QK-norm + RoPE of every token of the chunk: 32 head rows per 256-thread
// block, two per 16 lanes: head h of tokens 32 b .. 32 b + 31 for block
// (b, h) (grid ceil(T / 32) x (heads + kv_heads)), lanes of row r taking
// tokens 32 b + r and 32 b + 16 + r, both rows' loads issued before either
// row's math; a chunk's cache writes of a wavefront are 64 contiguous
// bytes. h < heads: roped q of head h into Q[t]; else kv head h - heads:
// roped k and the v row into the engine caches at position p0 + t.
constexpr uint32_t kPfRopeRows = 2;  // token rows per 16 lanes
extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_rope_cache(
    const uint16_t *__restrict__ QKV, const uint16_t *__restrict__ qnorm_w, const uint16_t *__restrict__ knorm_w,
    const uint16_t *__restrict__ rope_cos, const uint16_t *__restrict__ rope_sin, uint16_t *__restrict__ kcache,
    uint16_t *__restrict__ vcache, uint16_t *__restrict__ Q, uint32_t p0, uint32_t T, uint32_t heads,
    uint32_t kv_heads, uint32_t max_seq, float eps) {
  const uint32_t l16 = threadIdx.x & 15u, h = blockIdx.y;
  const uint32_t row_len = (heads + 2 * kv_heads) * xpu::kHeadDim;
  const bool is_q = h < heads;
  const uint32_t kvh = is_q ? 0 : h - heads;
  const u32x4 hw = *reinterpret_cast<const u32x4 *>((is_q ? qnorm_w : knorm_w) + l16 * 8u);
  uint32_t t[kPfRopeRows];
  u32x4 hx[kPfRopeRows], hc[kPfRopeRows], hs[kPfRopeRows], hv[kPfRopeRows];
#pragma unroll
  for (uint32_t r = 0; r < kPfRopeRows; ++r) {
    // tokens past the last are clamped onto it (recomputed, stored identically)
    t[r] = min(blockIdx.x * 16u * kPfRopeRows + 16u * r + (threadIdx.x >> 4), T - 1u);
    const uint16_t *row = QKV + static_cast<uint64_t>(t[r]) * row_len;
    const uint64_t pos = p0 + t[r];
    hx[r] = *reinterpret_cast<const u32x4 *>(row + h * xpu::kHeadDim + l16 * 8u);  // q heads, then k heads
    hc[r] = *reinterpret_cast<const u32x4 *>(rope_cos + pos * xpu::kHeadDim + l16 * 8u);
    hs[r] = *reinterpret_cast<const u32x4 *>(rope_sin + pos * xpu::kHeadDim + l16 * 8u);
    // the v row (kv heads only; q heads re-read their own row, unused)
    hv[r] = *reinterpret_cast<const u32x4 *>(row + (is_q ? h : heads + kv_heads + kvh) * xpu::kHeadDim + l16 * 8u);
  }
#pragma unroll
  for (uint32_t r = 0; r < kPfRopeRows; ++r) {
    const uint32_t pos = p0 + t[r];
    // K and V: chunk-major [kv_head][16][max_seq][8]
    const uint64_t kslot = static_cast<uint64_t>(kvh) * max_seq * xpu::kHeadDim + static_cast<uint64_t>(pos) * 8u;
    uint16_t *dst = is_q ? Q + static_cast<uint64_t>(t[r]) * heads * xpu::kHeadDim + h * xpu::kHeadDim : kcache + kslot;
    xpu::head_norm_rope_rows16(hx[r], hw, hc[r], hs[r], eps, dst, is_q ? 8u : static_cast<uint64_t>(max_seq) * 8u);
    if (!is_q) *reinterpret_cast<u32x4 *>(vcache + kslot + l16 * static_cast<uint64_t>(max_seq) * 8u) = hv[r];
  }
}

// Attention of every token of the chunk: block (head, t) over cache
// positions 0..p0 + t (all written by xpu_q3_pf_rope_cache and earlier
// steps), the general attention_head of the decode path with V tiles of
// kPfVTile rows (same operations in the same order): 53 KiB of LDS, so two
// of these latency-bound blocks share a compute unit.
constexpr uint32_t kPfVTile = 128;
extern "C" __global__ __launch_bounds__(256, 2) void xpu_q3_pf_attention(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache,
    uint16_t *__restrict__ A, uint32_t p0, uint32_t heads, uint32_t kv_heads, uint32_t max_seq, float scale) {
  __shared__ float sbuf[xpu::kAttnChunk];
  __shared__ float red[4 * xpu::kHeadDim];
  __shared__ __align__(16) uint16_t qs[xpu::kHeadDim];
  __shared__ __align__(16) uint16_t vtile[kPfVTile * xpu::kVPitch];
  const uint32_t head = blockIdx.x, t = blockIdx.y;
  const uint32_t kv = head / (heads / kv_heads);
  const uint64_t qoff = (static_cast<uint64_t>(t) * heads + head) * xpu::kHeadDim;
  if (threadIdx.x < xpu::kHeadDim) qs[threadIdx.x] = Q[qoff + threadIdx.x];
  __syncthreads();
  const uint64_t head_base = static_cast<uint64_t>(kv) * max_seq * xpu::kHeadDim;
  xpu::attention_head<false, kPfVTile, false>(qs, kcache + head_base, vcache + head_base,
                             xpu::KvLayout{8u, static_cast<uint64_t>(max_seq) * 8u, 8u, static_cast<uint64_t>(max_seq) * 8u},
                             p0 + t + 1, nullptr,
                             nullptr, scale, A + qoff, sbuf, vtile, red);
}

// xpu_q3_pf_attention for chunks whose contexts stay within kAttnTile
// positions (p0 + gridDim.y <= 256): the decode kernel's short path with
// every position read from the caches (thread t <-> position t, the V
// pieces in registers in the P.V layout, three block barriers), the same
// operations in the same order.
extern "C" __global__ __launch_bounds__(256) void xpu_q3_pf_attention_short(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache,
    uint16_t *__restrict__ A, uint32_t p0, uint32_t heads, uint32_t kv_heads, uint32_t max_seq, float scale) {
  __shared__ float sbuf[xpu::kAttnTile];
  __shared__ float red[4 + 32];
  __shared__ __align__(16) uint16_t qs[xpu::kHeadDim];
  const uint32_t head = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = xpu::lane_id();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t kv = head / (heads / kv_heads);
  const uint64_t qoff = (static_cast<uint64_t>(t) * heads + head) * xpu::kHeadDim;
  const uint64_t head_base = static_cast<uint64_t>(kv) * max_seq * xpu::kHeadDim;
  const uint64_t kchunk = static_cast<uint64_t>(max_seq) * 8u;
  const uint32_t n = p0 + t + 1;
  if (tid < 16) *reinterpret_cast<u32x4 *>(qs + tid * 8u) = *reinterpret_cast<const u32x4 *>(Q + qoff + tid * 8u);
  u32x4 krow[16];
  xpu::load_head_row(kcache + head_base + static_cast<uint64_t>(min(tid, n - 1)) * 8u, krow, kchunk);
  __syncthreads();  // 1: qs
  const float sc = tid < n ? xpu::attention_score_regs(qs, krow, scale) : -__builtin_inff();
  // V pieces: lane l of wave w owns residue class l % 16 and cache chunk
  // 4 w + l / 16; vpv[it] = V[16 it + cls] (rows past the context re-read
  // the last row and are not used)
  u32x4 vpv[xpu::kAttnTile / 16];
  const uint32_t cls = lane & 15u, vch = wave * 4u + (lane >> 4);
#pragma unroll
  for (int it = 0; it < static_cast<int>(xpu::kAttnTile / 16); ++it) {
    const uint32_t tv = min(it * 16u + cls, n - 1);
    vpv[it] = *reinterpret_cast<const u32x4 *>(vcache + head_base + vch * kchunk + static_cast<uint64_t>(tv) * 8u);
  }
  const float wmax = xpu::wave_reduce(sc, [](float x, float y) { return fmaxf(x, y); });
  if (lane == 0) red[wave] = wmax;
  __syncthreads();  // 2: wave maxima
  XPU_PHASE(1);     // (stamps build) scores and their maximum done
  const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float ex = tid < n ? xpu::canonical_exp(sc - mx) : 0.0f;
  sbuf[tid] = ex;
  float f = ex + xpu::dpp_f<0xB1>(ex);  // (a0 + a1), (a2 + a3), ...
  f = f + xpu::dpp_f<0x4E>(f);          // (a0 + a1) + (a2 + a3)
  f = f + xpu::dpp_f<0x141>(f);         // row_half_mirror: the other quad of the eight
  float *lane_sum = red + 4;            // 32 canonical lane sums
  if ((tid & 7u) == 0) lane_sum[tid >> 3] = f;
  __syncthreads();  // 3: exponentials and lane sums
  XPU_PHASE(2);     // (stamps build) exponentials and the denominator's lane sums done
  const float total = xpu::wave_butterfly(lane < 32 ? lane_sum[lane] : 0.0f);
  const float inv = 1.0f / total;
  float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int it = 0; it < static_cast<int>(xpu::kAttnTile / 16); ++it) {
    const uint32_t tp = it * 16u + cls;
    if (tp < n) {
      const float pt = xpu::round_bf16(sbuf[tp] * inv);
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
    v = v + xpu::dpp_f<0xB1>(v);   // xor 1
    v = v + xpu::dpp_f<0x4E>(v);   // xor 2
    v = v + xpu::dpp_f<0x141>(v);  // row_half_mirror
    v = v + xpu::xor8_f(v);
    code[e] = xpu::f32_to_bf16(v);
  }
  if (cls == 0)
    *reinterpret_cast<u32x4 *>(A + qoff + vch * 8u) =
        u32x4{code[0] | (code[1] << 16), code[2] | (code[3] << 16), code[4] | (code[5] << 16), code[6] | (code[7] << 16)};
}
