// Device helpers shared by the gfx950 kernels: 16-bit codecs, the canonical
// FP32 reduction order, and the exp used by softmax and SiLU.
//
// Canonical order (all GEMV/RMSNorm sums): element k of a length-n sum goes
// to lane (k / 8) % 64, slot k % 8, chunk k / 512; each of the 512 (lane,
// slot) accumulators starts at +0 and adds its terms in ascending chunk
// order; a lane then folds its 8 slots as ((0+1)+(2+3))+((4+5)+(6+7)) and
// the wave folds lanes with xor-butterflies 32,16,8,4,2,1. The CPU oracle
// (oracle/oracle.c) evaluates the same sequence, so results agree bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define XPU_DEVICE __device__ __forceinline__

namespace xpu {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum : int { kBf16 = 0, kFp16 = 1 };

XPU_DEVICE float bf16_to_f32(uint32_t code) { return __uint_as_float(code << 16); }

// qwen3/model.cpp:497-502: +0x7fff+lsb then truncate (no NaN special case).
XPU_DEVICE uint32_t f32_to_bf16(float v) {
  const uint32_t bits = __float_as_uint(v);
  return (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
}

XPU_DEVICE float fp16_to_f32(uint32_t code) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(code)));
}

// level_zero/peak_l0.cpp:740-761: RNE with subnormals, overflow/NaN -> Inf.
XPU_DEVICE uint32_t f32_to_fp16(float v) {
  const uint32_t bits = __float_as_uint(v);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  int exponent = static_cast<int>((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mantissa = bits & 0x7fffffu;
  if (exponent <= 0) {
    if (exponent < -10) return sign;
    mantissa = (mantissa | 0x800000u) >> (1 - exponent);
    return sign | ((mantissa + 0xfffu + ((mantissa >> 13) & 1u)) >> 13);
  }
  if (exponent >= 31) return sign | 0x7c00u;
  mantissa += 0xfffu + ((mantissa >> 13) & 1u);
  if (mantissa & 0x800000u) {
    mantissa = 0;
    if (++exponent >= 31) return sign | 0x7c00u;
  }
  return sign | (static_cast<uint32_t>(exponent) << 10) | (mantissa >> 13);
}

template <int DT> XPU_DEVICE float decode(uint32_t code) {
  if constexpr (DT == kFp16) return fp16_to_f32(code);
  else return bf16_to_f32(code);
}
template <int DT> XPU_DEVICE uint32_t encode(float v) {
  if constexpr (DT == kFp16) return f32_to_fp16(v);
  else return f32_to_bf16(v);
}

XPU_DEVICE float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Low and high 16-bit halves of a 32-bit word of packed codes.
template <int DT> XPU_DEVICE float lo16(uint32_t w) {
  if constexpr (DT == kFp16) return fp16_to_f32(w & 0xffffu);
  else return __uint_as_float(w << 16);
}
template <int DT> XPU_DEVICE float hi16(uint32_t w) {
  if constexpr (DT == kFp16) return fp16_to_f32(w >> 16);
  else return __uint_as_float(w & 0xffff0000u);
}

// 8 packed codes (16 bytes) -> 8 floats
template <int DT> XPU_DEVICE void unpack8(const u32x4 &v, float (&f)[8]) {
  f[0] = lo16<DT>(v.x); f[1] = hi16<DT>(v.x);
  f[2] = lo16<DT>(v.y); f[3] = hi16<DT>(v.y);
  f[4] = lo16<DT>(v.z); f[5] = hi16<DT>(v.z);
  f[6] = lo16<DT>(v.w); f[7] = hi16<DT>(v.w);
}

XPU_DEVICE float fold8(const float (&a)[8]) {
  return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

XPU_DEVICE uint32_t lane_id() { return threadIdx.x & 63u; }

// Cross-lane exchanges for a full wavefront (all 64 lanes active), without
// LDS round trips. DPP row_ror:8 moves the value of lane l ^ 8 (rotation by
// 8 within each 16-lane row); quad_perm [2,3,0,1] and [1,0,3,2] move lanes
// l ^ 2 and l ^ 1. gfx950 v_permlane32_swap / v_permlane16_swap of a value
// with itself return (own, partner of lane l ^ 32) in the lower half and
// (partner, own) in the upper half (likewise for rows of 16 with l ^ 16).
template <int CTRL> XPU_DEVICE uint32_t dpp_u(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL> XPU_DEVICE float dpp_f(float v) {
  return __builtin_bit_cast(float, dpp_u<CTRL>(__builtin_bit_cast(uint32_t, v)));
}
XPU_DEVICE uint32_t xor32_u(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (lane_id() & 32u) ? r[0] : r[1];
}
XPU_DEVICE uint32_t xor16_u(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (lane_id() & 16u) ? r[0] : r[1];
}
XPU_DEVICE float xor32_f(float v) { return __builtin_bit_cast(float, xor32_u(__builtin_bit_cast(uint32_t, v))); }
XPU_DEVICE float xor16_f(float v) { return __builtin_bit_cast(float, xor16_u(__builtin_bit_cast(uint32_t, v))); }
XPU_DEVICE float xor8_f(float v) { return dpp_f<0x128>(v); }  // row_ror:8

// Butterfly reduction op(own, partner) with partners l ^ 32, 16, 8, 4, 2, 1
// in that order; every lane ends with the same value. At the l ^ 4 step the
// values depend on l % 8 only, so row_ror:4 (lane (l + 4) % 16 of the row)
// supplies the l ^ 4 value.
template <typename Op> XPU_DEVICE float wave_reduce(float s, Op op) {
  s = op(s, xor32_f(s));
  s = op(s, xor16_f(s));
  s = op(s, xor8_f(s));
  s = op(s, dpp_f<0x124>(s));  // row_ror:4
  s = op(s, dpp_f<0x4E>(s));   // quad_perm [2,3,0,1]
  s = op(s, dpp_f<0xB1>(s));   // quad_perm [1,0,3,2]
  return s;
}

// xor-butterfly sum over the 64 lanes of a wavefront (s + partner for
// partners l ^ 32, 16, 8, 4, 2, 1); every lane ends with the same value.
XPU_DEVICE float wave_butterfly(float s) {
  return wave_reduce(s, [](float a, float b) { return a + b; });
}

// exp: Cody-Waite reduction and degree-7 Taylor polynomial, the same
// operation sequence as orc_exp in the oracle.
XPU_DEVICE float pow2i(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }

// Written without branches: every case is computed and the result picked by
// selects in the oracle's order of tests (NaN, overflow, underflow, the
// subnormal scaling, then the ordinary result), so a wavefront with mixed
// cases (or masked lanes) runs one straight sequence; the results are the
// oracle's bit for bit. n is clamped before the integer conversion so that
// out-of-range inputs convert to a defined value (their results are
// replaced by the selects).
XPU_DEVICE float canonical_exp(float x) {
  const float n = __builtin_rintf(x * 1.44269502162933349609f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860676533018704504e-06f, r);
  float p = 1.98412698412698412526e-04f;
  p = __builtin_fmaf(p, r, 1.38888888888888894189e-03f);
  p = __builtin_fmaf(p, r, 8.33333333333333321769e-03f);
  p = __builtin_fmaf(p, r, 4.16666666666666643537e-02f);
  p = __builtin_fmaf(p, r, 1.66666666666666657415e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int e = static_cast<int>(__builtin_fminf(__builtin_fmaxf(n, -200.0f), 200.0f));
  const bool top = e > 127;
  p = top ? p * 2.0f : p;
  e = top ? e - 1 : e;
  const float normal = p * pow2i(e < -126 ? 0 : e);
  const float sub = (p * pow2i(e < -126 ? e + 64 : 0)) * 0x1p-64f;
  float res = e < -126 ? sub : normal;
  res = x < -103.972084045410156f ? 0.0f : res;
  res = x > 88.72283935546875f ? __builtin_inff() : res;
  return x != x ? x : res;
}

// canonical_exp for x <= 0 (a softmax's s - max), the same bits with fewer
// operations: NaN, overflow and the e > 127 adjustment cannot occur, and
// the result is always formed as (p * 2^(e + 64)) * 2^-64, which is the
// subnormal path itself and, for a normal result, equal to p * 2^e (both
// products are exact power-of-two scalings). Inputs above 0 give
// unspecified finite-or-infinite values.
XPU_DEVICE float canonical_exp_nonpos(float x) {
  const float n = __builtin_rintf(x * 1.44269502162933349609f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860676533018704504e-06f, r);
  float p = 1.98412698412698412526e-04f;
  p = __builtin_fmaf(p, r, 1.38888888888888894189e-03f);
  p = __builtin_fmaf(p, r, 8.33333333333333321769e-03f);
  p = __builtin_fmaf(p, r, 4.16666666666666643537e-02f);
  p = __builtin_fmaf(p, r, 1.66666666666666657415e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  // -151 <= n <= 0 wherever the result is used; the clamp keeps the
  // conversion and the exponent arithmetic defined for the rest
  const int e = static_cast<int>(__builtin_fminf(__builtin_fmaxf(n, -160.0f), 60.0f));
  const float res = (p * pow2i(e + 64)) * 0x1p-64f;
  return x < -103.972084045410156f ? 0.0f : res;
}

XPU_DEVICE u32x4 load_nt16(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// ------------------------------------------------ global -> LDS DMA (gfx950)

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer descriptor: 48-bit base, stride 0, num_records bytes, 32-bit
// data format. Offsets at or past num_records read as zero.
XPU_DEVICE i32x4 rsrc(const void *base, int64_t records) {
  // clamp to [0, 2^31 - 1] on the two 32-bit halves (scalar compares; a
  // 64-bit signed compare would run on the vector ALU)
  int32_t hi = static_cast<int32_t>(static_cast<uint64_t>(records) >> 32);
  uint32_t lo = static_cast<uint32_t>(records);
  asm("" : "+s"(hi), "+s"(lo));  // keeps the halves apart (no 64-bit compare)
  const uint32_t n = hi < 0 ? 0u : (hi > 0 || lo > 0x7fffffffu ? 0x7fffffffu : lo);
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4{static_cast<int>(a & 0xffffffffu), static_cast<int>((a >> 32) & 0xffffu), static_cast<int>(n),
               0x00020000};
}

// 16 bytes per lane from the buffer at voff into LDS at m0 + 16 * lane (m0
// wave-uniform). Written as asm so that the compiler's wait-count pass,
// which does not track these writes, does not wait for every DMA before each
// LDS read; callers issue the waits themselves (wait_vmcnt, then a barrier
// before other wavefronts read the data).
XPU_DEVICE void dma16(uint32_t m0, const i32x4 &r, uint32_t voff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(r), "{m0}"(m0)
               : "memory");
}

template <int N> XPU_DEVICE void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // gfx9 s_waitcnt: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14; expcnt and
  // lgkmcnt at their maxima (no wait)
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS byte address of a __shared__ object
XPU_DEVICE uint32_t lds_addr(const void *p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)p));
}

}  // namespace xpu

// ---- Opt-in per-wave timestamps (code object built with -DXPU_STAMPS:
// build/xpu_kernels_stamps.hsaco). A kernel that starts with
// XPU_STAMP(id) has lane 0 of each wave record, when the wave leaves the
// kernel, the constant 100 MHz clock (s_memrealtime) at entry, the elapsed
// constant-clock and shader-clock (s_memtime) ticks, the kernel id, the
// block and the XCD. Records go to a ring per (block, wave) slot, indexed by
// that slot's own sequence counter: only one wave occupies a slot at a time
// (launches on a stream do not overlap), so no atomics perturb the timing.
// xpu_playground_amd/timeline.py reads and groups them. XPU_PHASE(i)
// (i < 4) marks a point inside such a kernel: lane 0 of the wave writes the
// shader clock into a wave-indexed LDS array (no memory traffic), and the
// exit record of the first kPhaseSlots (block, wave) slots carries each
// mark as shader-clock ticks since entry (0 where the wave did not pass
// it). Without XPU_STAMPS both macros are empty.
#ifdef XPU_STAMPS
namespace xpu {
// (block, wave) slots: up to 1024 blocks of 4 waves (the decode GEMVs' grid
// cap); 2048 records each (a decode token launches 142 kernels); phase
// marks for the first 1024 slots
constexpr uint32_t kStampSlots = 4096, kStampRing = 2048, kPhaseSlots = 1024, kPhases = 4;
struct StampRecord {
  uint32_t start_lo;     // s_memrealtime at entry, low 32 bits (100 MHz)
  uint32_t real_ticks;   // constant-clock ticks from entry to exit
  uint32_t clock_ticks;  // shader-clock ticks (s_memtime) from entry to exit
  uint32_t tag;          // kernel id << 24 | XCD << 20 | wave << 16 | block
};
}  // namespace xpu
extern "C" __device__ uint32_t xpu_stamp_seq[xpu::kStampSlots];
extern "C" __device__ xpu::StampRecord xpu_stamp_ring[xpu::kStampSlots * xpu::kStampRing];
extern "C" __device__ uint32_t xpu_stamp_phase[xpu::kPhaseSlots * xpu::kStampRing * xpu::kPhases];
__shared__ uint32_t xpu_phase_marks[16 * xpu::kPhases];  // [wave][phase], shader clock, low 32 bits
namespace xpu {
struct StampGuard {
  uint64_t r0, c0;
  uint32_t id;
  XPU_DEVICE explicit StampGuard(uint32_t kernel_id) : id(kernel_id) {
    r0 = __builtin_amdgcn_s_memrealtime();
    c0 = __builtin_amdgcn_s_memtime();
    if ((threadIdx.x & 63u) == 0)
      for (uint32_t i = 0; i < kPhases; ++i) xpu_phase_marks[(threadIdx.x >> 6) * kPhases + i] = 0;
  }
  XPU_DEVICE ~StampGuard() {
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if ((threadIdx.x & 63u) != 0) return;
    const uint32_t wave = threadIdx.x >> 6, slot = blockIdx.x * (blockDim.x >> 6) + wave;
    if (slot >= kStampSlots) return;
    // HW_REG_XCC_ID (hwreg 20), bits [3:0]
    const uint32_t xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u;
    const uint32_t seq = xpu_stamp_seq[slot];
    xpu_stamp_seq[slot] = seq + 1;
    StampRecord rec;
    rec.start_lo = static_cast<uint32_t>(r0);
    rec.real_ticks = static_cast<uint32_t>(r1 - r0);
    rec.clock_ticks = static_cast<uint32_t>(c1 - c0);
    rec.tag = (id << 24) | (xcc << 20) | ((wave & 15u) << 16) | (blockIdx.x & 0xffffu);
    xpu_stamp_ring[slot * kStampRing + seq % kStampRing] = rec;
    if (slot < kPhaseSlots)
      for (uint32_t i = 0; i < kPhases; ++i) {
        const uint32_t mark = xpu_phase_marks[wave * kPhases + i];
        xpu_stamp_phase[(slot * kStampRing + seq % kStampRing) * kPhases + i] =
            mark ? mark - static_cast<uint32_t>(c0) : 0u;
      }
  }
};
XPU_DEVICE void phase_mark(uint32_t i) {
  const uint32_t t = static_cast<uint32_t>(__builtin_amdgcn_s_memtime());
  if ((threadIdx.x & 63u) == 0) xpu_phase_marks[(threadIdx.x >> 6) * kPhases + i] = t | 1u;
}
}  // namespace xpu
#define XPU_STAMP(id) const ::xpu::StampGuard xpu_stamp_guard_(id)
#define XPU_PHASE(i) ::xpu::phase_mark(i)
#else
#define XPU_STAMP(id) \
  do {                \
  } while (0)
#define XPU_PHASE(i) \
  do {               \
  } while (0)
#endif

namespace xpu {
// kernel ids of the stamps (xpu_playground_amd/timeline.py names them)
enum : uint32_t {
  kStampGemv = 1, kStampGemm = 2, kStampQ3Qkv = 10, kStampQ3Attention = 11, kStampQ3Scores = 12, kStampQ3Pv = 13,
  kStampQ3Residual = 14, kStampQ3Swiglu = 15, kStampQ3Logits = 16, kStampQ3Finish = 17
};
}  // namespace xpu
