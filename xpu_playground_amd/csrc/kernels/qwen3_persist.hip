// Persistent Qwen3 decode: a range of decode steps in one cooperative launch
// of one 256-thread block per compute unit, with the kernel boundaries of the
// fused step (RMSNorm + QKV, attention, o_proj + residual, RMSNorm + gate/up
// + SiLU, down + residual per layer, then final norm + lm_head + argmax)
// replaced by flags in device memory.
//
// Every block takes its share of each stage's rows (the same per-row
// arithmetic as the per-stage kernels, so tokens, logits and hidden states
// are bit-identical to them), publishes the stage with a flag word of its
// own, and waits for the flags of the blocks whose outputs the next stage
// reads. A flag holds a tick that increases with every stage instance of the
// engine's lifetime, so flags are never cleared. The weight rows of a stage
// are loaded before its wait, so they arrive while the producers finish.
// The argmax over the logits blocks' partials is computed by every block
// (no broadcast needed), so the next step's first stage waits on nothing.
//
// Handoff: the producer's waves each execute an agent-scope release fence,
// the block barrier follows, then thread 0 stores the flag; the consumer's
// wave 0 polls the flags (agent-scope loads), the block barrier follows,
// then every wave executes an agent-scope acquire fence before its loads.
// Every wait is bounded: past args.spin_limit polls the waiter sets *error,
// every waiter also stops when it sees *error set, and the whole grid then
// returns (the host reports the failure).
//
// Attention: one block per query head at the decode position (contexts up
// to kAttnTile positions take the short path of attention_decode_head).

#include "persist_abi.h"

namespace xpu {

using PersistLayer = ::xpu_persist_layer;
using PersistArgs = ::xpu_persist_args;

enum : uint32_t { kPfQkv = 0, kPfAtt, kPfO, kPfGu, kPfDown, kPfLogits, kPersistStages };

XPU_DEVICE uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m)));
  return v;
}

// Wait until flags[0..count) all hold >= target. False when the grid stops:
// *error set by another block, or spin_limit polls (~1 us each) passed.
XPU_DEVICE bool persist_wait(const uint32_t *flags, uint32_t count, uint32_t target, uint32_t *error,
                             uint32_t spin_limit) {
  __shared__ uint32_t status;
  if (threadIdx.x < 64) {
    const uint32_t lane = threadIdx.x;
    uint32_t st = 0;
    for (uint32_t spin = 0;; ++spin) {
      uint32_t low = 0xffffffffu;
      for (uint32_t i = lane; i < count; i += 64)
        low = min(low, __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      low = wave_min_u32(low);
      const uint32_t err = __hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (low >= target) {
        st = 1;
        break;
      }
      if (err) {
        st = 2;
        break;
      }
      if (spin >= spin_limit) {
        if (lane == 0) __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        st = 2;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) status = st;
  }
  __syncthreads();
  const bool ok = status == 1;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return ok;
}

// Publish this block's outputs of a stage: flag = value.
XPU_DEVICE void persist_signal(uint32_t *flag, uint32_t value) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

#ifdef XPU_STAMPS
// stage completion records (wave 0 of each block, its stamp slot): the
// elapsed time since the block's previous stage record
struct StageStamps {
  uint64_t last_real, last_clock;
  XPU_DEVICE StageStamps() : last_real(__builtin_amdgcn_s_memrealtime()), last_clock(__builtin_amdgcn_s_memtime()) {}
  XPU_DEVICE void mark(uint32_t id) {
    const uint64_t c = __builtin_amdgcn_s_memtime(), r = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
      const uint32_t slot = blockIdx.x * (blockDim.x >> 6);
      if (slot < kStampSlots) {
        const uint32_t xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u;
        const uint32_t seq = xpu_stamp_seq[slot];
        xpu_stamp_seq[slot] = seq + 1;
        StampRecord rec;
        rec.start_lo = static_cast<uint32_t>(last_real);
        rec.real_ticks = static_cast<uint32_t>(r - last_real);
        rec.clock_ticks = static_cast<uint32_t>(c - last_clock);
        rec.tag = (id << 24) | (xcc << 20) | (blockIdx.x & 0xffffu);
        xpu_stamp_ring[slot * kStampRing + seq % kStampRing] = rec;
      }
    }
    last_real = r;
    last_clock = c;
  }
};
#define XPU_STAGE_STAMPS StageStamps stage_stamps_
#define XPU_STAGE_MARK(id) stage_stamps_.mark(id)
#else
#define XPU_STAGE_STAMPS \
  do {                   \
  } while (0)
#define XPU_STAGE_MARK(id) \
  do {                     \
  } while (0)
#endif

// stage ids of the stamp records (kernel ids 20..26)
enum : uint32_t {
  kStampPfQkv = 20, kStampPfAtt, kStampPfO, kStampPfGu, kStampPfDown, kStampPfLogits, kStampPfArgmax
};

// NCH, NCQ, NCI: 512-element chunks per lane of hidden, heads * 128 and
// intermediate (the register-vector GEMV width of each stage).
template <int NCH, int NCQ, int NCI>
XPU_DEVICE void persist_decode(const PersistArgs &a, uint32_t p_begin, uint32_t p_end, uint32_t tick_base) {
  XPU_STAGE_STAMPS;
  const uint32_t nb = gridDim.x, bid = blockIdx.x;
  const GridSpan g{bid, nb};
  const uint32_t L = a.layers_n, H = a.hidden, I = a.inter, V = a.vocab;
  const uint32_t qd = a.heads * kHeadDim, qkv_rows = (a.heads + 2 * a.kv_heads) * kHeadDim;
  uint32_t *const F = a.flags;
  auto flags = [&](uint32_t stage) { return F + stage * nb; };
  const uint32_t n_prompt = a.state[3];
  uint32_t token = a.state[1];
  __shared__ float redv[4];
  __shared__ uint32_t redi[4], redb[4], next_token;
  for (uint32_t p = p_begin, t = 0; p < p_end; ++p, ++t) {
    const uint32_t tick0 = tick_base + t * (L + 1);
    for (uint32_t l = 0; l < L; ++l) {
      const PersistLayer ly = a.layers[l];
      const uint32_t T = tick0 + l + 1, Tprev = tick0 + l;
      bool ok = true;
      // RMSNorm + [q; k; v] (layer 0: of the embedding row of `token`)
      if (l == 0)
        q3_norm_gemv_reg<2, NCH>(ly.qkv, a.x, ly.in_norm, a.qkv, qkv_rows, H, a.eps, a.embed, a.state, V, g,
                                 NoWait(), token < V ? token : 0u);
      else
        q3_norm_gemv_reg<2, NCH>(ly.qkv, a.x, ly.in_norm, a.qkv, qkv_rows, H, a.eps, nullptr, a.state, V, g,
                                 [&] { ok = persist_wait(flags(kPfDown), nb, Tprev, a.error, a.spin_limit); });
      if (!ok) return;
      persist_signal(flags(kPfQkv) + bid, T);
      XPU_STAGE_MARK(kStampPfQkv);
      // attention, one block per query head
      if (bid < a.heads) {
        if (!persist_wait(flags(kPfQkv), nb, T, a.error, a.spin_limit)) return;
        const uint64_t rope = static_cast<uint64_t>(p) * kHeadDim;
        attention_decode_head(bid, a.qkv, ly.q_norm, ly.k_norm, a.cos_t + rope, a.sin_t + rope, ly.kc, ly.vc, a.attn,
                              [&] { return p; }, a.heads, a.kv_heads, a.max_seq, a.eps, a.scale);
        persist_signal(flags(kPfAtt) + bid, T);
        XPU_STAGE_MARK(kStampPfAtt);
      }
      // o_proj + residual
      q3_gemv_residual_reg<1, NCQ>(ly.o, a.attn, a.x, H, qd, g,
                                   [&] { ok = persist_wait(flags(kPfAtt), a.heads, T, a.error, a.spin_limit); });
      if (!ok) return;
      persist_signal(flags(kPfO) + bid, T);
      XPU_STAGE_MARK(kStampPfO);
      // RMSNorm + [gate; up] + SiLU * up
      q3_norm_gemv_swiglu_reg<2, NCH>(ly.gu, a.x, ly.post_norm, a.h, I, H, a.eps, g,
                                      [&] { ok = persist_wait(flags(kPfO), nb, T, a.error, a.spin_limit); });
      if (!ok) return;
      persist_signal(flags(kPfGu) + bid, T);
      XPU_STAGE_MARK(kStampPfGu);
      // down + residual
      q3_gemv_residual_reg<1, NCI>(ly.down, a.h, a.x, H, I, g,
                                   [&] { ok = persist_wait(flags(kPfGu), nb, T, a.error, a.spin_limit); });
      if (!ok) return;
      persist_signal(flags(kPfDown) + bid, T);
      XPU_STAGE_MARK(kStampPfDown);
    }
    // final RMSNorm + lm_head with per-block argmax partials
    const uint32_t Tlog = tick0 + L + 1;
    {
      bool ok = true;
      q3_norm_gemv_logits_reg<2, NCH>(a.lm_head, a.x, a.final_norm, a.logits, V, H, a.eps, a.part_val, a.part_idx,
                                      a.part_bad, g, [&] { ok = persist_wait(flags(kPfDown), nb, Tlog - 1, a.error, a.spin_limit); });
      if (!ok) return;
    }
    persist_signal(flags(kPfLogits) + bid, Tlog);
    XPU_STAGE_MARK(kStampPfLogits);
    // every block: the argmax of the partials (NaN or infinity: 0xffffffff),
    // then the next step's input token
    if (!persist_wait(flags(kPfLogits), nb, Tlog, a.error, a.spin_limit)) return;
    float best = -__builtin_inff();
    uint32_t best_index = 0xffffffffu, bad = 0;
    for (uint32_t i = threadIdx.x; i < nb; i += blockDim.x) {
      bad |= a.part_bad[i];
      argmax_merge(best, best_index, a.part_val[i], a.part_idx[i]);
    }
    block_argmax(best, best_index, bad, redv, redi, redb);
    if (threadIdx.x == 0) {
      const uint32_t am = bad ? 0xffffffffu : (best_index == 0xffffffffu ? 0u : best_index);
      const uint32_t next_pos = p + 1;
      next_token = next_pos < n_prompt ? a.prompt[next_pos] : am;
      if (bid == 0) {
        a.state[2] = am;
        if (next_pos >= n_prompt && next_pos - n_prompt < a.gen_capacity) a.gen[next_pos - n_prompt] = am;
        if (next_pos == p_end) {
          a.state[0] = next_pos;
          a.state[1] = next_token;
        }
      }
    }
    __syncthreads();
    token = next_token;
    __syncthreads();
    XPU_STAGE_MARK(kStampPfArgmax);
  }
}

}  // namespace xpu

#define XPU_Q3_PERSIST(NCH, NCQ, NCI)                                                                       \
  extern "C" __global__ __launch_bounds__(256) void xpu_q3_persist_h##NCH##_q##NCQ##_i##NCI(                 \
      const xpu::PersistArgs *__restrict__ args, uint32_t p_begin, uint32_t p_end, uint32_t tick_base) { \
    xpu::persist_decode<NCH, NCQ, NCI>(*args, p_begin, p_end, tick_base);                                \
  }

// hidden / heads * 128 / intermediate of 256 / 512 / 512 (tiny) and
// 1024 / 2048 / 3072 (Qwen3-0.6B and the small test shape)
XPU_Q3_PERSIST(1, 1, 1)
XPU_Q3_PERSIST(2, 4, 6)
