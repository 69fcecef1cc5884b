// fa2_kernel_pp.h - fp16/bf16 forward kernel for grouped heads (Hq/Hkv >= 2):
// two wave groups in ping-pong over shared K/V tiles.
//
// A workgroup of 8 waves covers one q-block (128 rows) of TWO query heads of
// the same kv head: waves 0-3 (group 0) take the first head, waves 4-7
// (group 1) the second, 32 rows per wave.  Waves are placed on SIMD
// (wave % 4), so every SIMD holds one wave of each group.
//
// Per KV tile t a group runs two phases:
//   M(t): PV(t-1) and S(t)  - MFMA work (plus LDS fragment reads);
//   V(t): mask, max, exp, P, row sum, rescale  - VALU work.
// Group 1 runs one phase behind group 0 and every phase ends with a
// workgroup barrier, so in each phase one wave of a SIMD issues MFMAs while
// the other issues the softmax VALU work:
//
//   phase     0     1     2     3     4   ...  2T    2T+1
//   group 0   M(0)  V(0)  M(1)  V(1)  M(2)     M(T)  -
//   group 1   -     M(0)  V(0)  M(1)  V(1)     V(T-1) M(T)
//
// (M(T) is the last PV only.)  Both groups run the same straight-line code;
// group 1 takes one extra barrier before its first phase and group 0 one
// after its last, which is what offsets them.
//
// K and V tiles live in three LDS slots each (tile t in slot t % 3).  The
// waves of group 0 issue the direct-to-LDS loads of V(i+1) and K(i+2) at
// the start of their softmax phase V(i) (or of M(i), FA2_PP_DMA_IN_M) and
// wait for them at the end of V(i+1), just before the barrier that precedes
// their first use (M(i+2)); the last V tile is awaited before the final
// PV.  No slot is refilled before both groups have read it.
//
// Same arithmetic as fa2_fwd_lds_kernel (fa2_kernel_lds.h): transposed
// MFMA formulation, lazy rescale, exp2 with the folded scale, row sum of
// the rounded P; same results bit for bit.
#pragma once

#include "fa2_kernel_lds.h"

namespace fa2 {

constexpr int kPPWaves = 8;
constexpr int kPPThreads = kPPWaves * 64;
constexpr int kPPSlots = 3;

// Wave priority during the MFMA phase (0: unchanged).  Measured on MI355X
// (bf16 D=128): 2 beats 0 by 2-4% on c2/c3/c5.
#ifndef FA2_PP_PRIO
#define FA2_PP_PRIO 2
#endif
// 1: group 0 issues the tile loads at the start of its MFMA phase M(i)
// (the loads of V(i+1), K(i+2) then overlap M(i) and V(i)); 0: at the
// start of its softmax phase V(i).
#ifndef FA2_PP_DMA_IN_M
#define FA2_PP_DMA_IN_M 0
#endif
// LDS fragment reads run this many MFMAs ahead inside the MFMA phase.
#ifndef FA2_PP_AHEAD
#define FA2_PP_AHEAD 10
#endif

// Workgroup barrier without a memory fence: LDS reads of this wave are
// complete (lgkmcnt), outstanding direct-to-LDS loads are awaited
// separately (pp_wait_vm) by the wave that issued them.
// (The barrier itself is the convergent builtin, so the compiler never
// duplicates it into divergent paths; the empty asm statements keep LDS
// accesses on their side of it.)
__device__ __forceinline__ void pp_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int N>
__device__ __forceinline__ void pp_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int DT, int D, int MODE, bool BUF>
__global__ __launch_bounds__(kPPThreads, 1) void fa2_fwd_pp_kernel(KArgs a) {
  static_assert(DT != FA2_DTYPE_F32, "fp32 uses the register-staged kernel");
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int DC = D / 16;  // MFMA k-steps of S (16 head dims each)
  constexpr int DB = D / 32;  // 32-dim blocks of O^T
  constexpr int SB = kBN / 32;
  using G = SwzGeo<D>;
  using LD = DirectLoader<D, MODE, BUF, DT, kWaves>;  // group 0 loads
  constexpr int kI = LD::kInstr;
  constexpr int kTile = G::kTileBytes;

  __shared__ __attribute__((aligned(1024))) char lds[2 * kPPSlots * kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // waves w and w + 4 share SIMD w % 4
  const int wq = wave & 3;
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  const Work w = decode_work<MODE>(a, blockIdx.x, 2);
  if (!w.valid) return;
  const int group = a.hq / a.hkv;
  const bool hok = w.hg + grp < group;  // odd group: the second head may not exist
  const int64_t q_base = w.q_base + grp * a.q_sh;
  const int64_t o_base = w.o_base + grp * a.o_sh;
  const int q0 = w.qblk * kBM;
  const int split = blockIdx.y;
  const int S = a.num_splits;

  const int kv_end = kv_end_for_block(a.mask, q0, w.Lq, w.Lk, w.off);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const int t_begin = (ntiles * split) / S;
  const int t_end = (ntiles * (split + 1)) / S;
  const int T = t_end - t_begin;

  const int qrow = q0 + wq * kWaveRows + l32;
  u32x4 qf[DC];
  {
    const bool ok = hok && qrow < w.Lq;
    const int64_t base = q_base + static_cast<int64_t>(qrow) * a.q_ss + hi * 8;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      Raw8<DT> r;
      if (ok)
        load_raw8<DT>(r, a.q, base + c * 16);
      else
        zero_raw8<DT>(r);
      qf[c] = to16<DT>(r);
    }
  }

  // per-lane LDS offsets, as in fa2_fwd_lds_kernel
  const uint32_t koff0 = l32 * G::kRowBytes + ((hi ^ G::k(l32)) * 16);
  uint32_t voff0;
  {
    const int g = lane >> 4, i = lane & 15;
    const int r = 4 * (g >> 1) + (i >> 2);
    const int dim = 16 * (g & 1) + 4 * (i & 3);
    voff0 = r * G::kRowBytes + (((dim >> 3) ^ G::v(r)) * 16) + (dim & 7) * 2;
  }

  f32x16 o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = (f32x16){};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const int wq_first = q0 + wq * kWaveRows;
  const bool causal = a.mask != FA2_MASK_NONE;

  const LD ld(a, wq, lane);
  auto kslot = [&](int i) { return lds + (i % kPPSlots) * kTile; };
  auto vslot = [&](int i) { return lds + (kPPSlots + i % kPPSlots) * kTile; };

  f32x16 s[SB];
  u32x4 pf[kBN / 16];

  // M phase: PV of the previous tile, then S of this one.
  auto phase_m = [&](auto has_pv, auto has_s, int i) {
    constexpr bool kPV = decltype(has_pv)::value;
    constexpr bool kS = decltype(has_s)::value;
    // a scheduling region of its own: nothing moves in or out
    __builtin_amdgcn_sched_barrier(0);
#if FA2_PP_PRIO
    __builtin_amdgcn_s_setprio(FA2_PP_PRIO);
#endif
    // Consecutive MFMAs go to different accumulators (c-major for PV,
    // cc-major for S): an MFMA that depends on the one just issued waits for
    // it to finish, which doubles the time per MFMA.  Each accumulator still
    // sums in the same order.
    if constexpr (kPV) {
      const lds_char_t* vl = to_lds(vslot(i - 1));
#pragma unroll
      for (int c = 0; c < kBN / 16; ++c) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const uint32_t voff = voff0 ^ (64u * d);
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4i16_t*)(vl + (16 * c) * G::kRowBytes + voff));
          const v4i16 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4i16_t*)(vl + (16 * c + 8) * G::kRowBytes + voff));
          const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
          const u32x2 h2 = __builtin_bit_cast(u32x2, hi4);
          o[d] = mma32<BF>((u32x4){l2[0], l2[1], h2[0], h2[1]}, pf[c], o[d]);
        }
      }
    }
    if constexpr (kS) {
      const lds_char_t* kl = to_lds(kslot(i));
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) s[sb] = (f32x16){};
#pragma unroll
      for (int cc = 0; cc < DC; ++cc) {
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) {
          const u32x4 kf =
              *(const lds_u32x4_t*)(kl + sb * 32 * G::kRowBytes + (koff0 ^ (32u * cc)));
          s[sb] = mma32<BF>(kf, qf[cc], s[sb]);
        }
      }
    }
    // Order: the reads of the first kAhead MFMAs, then per MFMA k the MFMA
    // and the reads of MFMA k + kAhead (2 transposed V reads for a PV MFMA,
    // 1 K read for an S MFMA), so no MFMA waits on a just-issued read.
    {
      constexpr int kNPV = kPV ? DB * (kBN / 16) : 0;
      constexpr int kN = kNPV + (kS ? SB * DC : 0);
      constexpr int kAhead = FA2_PP_AHEAD < kN ? FA2_PP_AHEAD : kN;
      constexpr int kPre2 = kAhead < kNPV ? kAhead : kNPV;  // PV MFMAs among the first kAhead
      constexpr int kB1 = kNPV > kAhead ? kNPV - kAhead : 0;  // MFMAs followed by 2 reads
      if constexpr (kPre2 > 0) __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPre2, 0);
      if constexpr (kAhead > kPre2) __builtin_amdgcn_sched_group_barrier(0x100, kAhead - kPre2, 0);
#pragma unroll
      for (int k = 0; k < kB1; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
#pragma unroll
      for (int k = kB1; k < kN - kAhead; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kAhead, 0);
    }
#if FA2_PP_PRIO
    __builtin_amdgcn_s_setprio(0);
#endif
    __builtin_amdgcn_sched_barrier(0);
  };

  // V phase: online softmax of tile i (scores in s), P^T into pf.
  auto phase_v = [&](int i) {
    const int k0 = (t_begin + i) * kBN;
    if ((k0 + kBN > w.Lk) || (causal && (k0 + kBN - 1 > wq_first + w.off))) {
      int lim = w.Lk - 1 - k0 - hi * 4;
      if (causal) lim = min(lim, qrow + w.off - k0 - hi * 4);
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
          const int c = sb * 32 + (i2 >> 2) * 8 + (i2 & 3);
          if (c > lim) s[sb][i2] = -INFINITY;
        }
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < SB; ++sb)
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) mx = fmaxf(mx, s[sb][i2]);
    mx = max_xor32_valu(mx);
    const float mt = mx * a.scale_log2;
    const bool need = mt > m_run + kRescaleThreshold;
    const float alpha = fast_exp2(need ? (m_run - mt) : 0.0f);
    const float m_new = need ? mt : m_run;
    m_run = m_new;
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
      float p[16];
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2)
        p[i2] = fast_exp2(__builtin_fmaf(s[sb][i2], a.scale_log2, -m_use));
#pragma unroll
      for (int half = 0; half < 2; ++half)
        pf[sb * 2 + half] = (u32x4){pack2<BF>(p[half * 8 + 0], p[half * 8 + 1]),
                                    pack2<BF>(p[half * 8 + 2], p[half * 8 + 3]),
                                    pack2<BF>(p[half * 8 + 4], p[half * 8 + 5]),
                                    pack2<BF>(p[half * 8 + 6], p[half * 8 + 7])};
    }
    float rs = 0.f;
#pragma unroll
    for (int c = 0; c < kBN / 16; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) rs = dot2_ones<BF>(pf[c][j], rs);
    l_run = l_run * alpha + rs;
    if (__any(need)) {
#pragma unroll
      for (int d = 0; d < DB; ++d) o[d] *= alpha;
    }
  };

  // group 0: loads issued at the start of V(i); returns this wave's count
  auto issue_iter = [&](int i) -> int {
    int n = 0;
    if (i + 1 < T) {
      ld.template issue<true>(a, w, (t_begin + i + 1) * kBN, vslot(i + 1));
      n += kI;
    }
    if (i + 2 < T) {
      ld.template issue<false>(a, w, (t_begin + i + 2) * kBN, kslot(i + 2));
      n += kI;
    }
    return n;
  };
  // wait until at most n of this wave's loads are outstanding
  auto wait_vm = [&](int n) {
    if (n >= 2 * kI)
      pp_wait_vm<2 * kI>();
    else if (n >= kI)
      pp_wait_vm<kI>();
    else
      pp_wait_vm<0>();
  };
  using Y = std::integral_constant<bool, true>;
  using N = std::integral_constant<bool, false>;

  if (T > 0) {
    if (grp == 0) {
      ld.template issue<false>(a, w, t_begin * kBN, kslot(0));
      if (T > 1) ld.template issue<false>(a, w, (t_begin + 1) * kBN, kslot(1));
      ld.template issue<true>(a, w, t_begin * kBN, vslot(0));
      wait_vm(T > 1 ? 2 * kI : kI);  // K(0) has landed
    }
    pp_barrier();
    if (grp != 0) pp_barrier();  // group 1 runs one phase behind
    int n = 0;
#if FA2_PP_DMA_IN_M
    if (grp == 0) n = issue_iter(0);
#endif
    phase_m(N{}, Y{}, 0);
    pp_barrier();
    for (int i = 0; i + 1 < T; ++i) {
#if !FA2_PP_DMA_IN_M
      if (grp == 0) n = issue_iter(i);
#endif
      phase_v(i);
      // K(i+1) and V(i) (read from M(i+1) on) have landed; the loads of
      // the current issue may still be in flight
      if (grp == 0) wait_vm(n);
      pp_barrier();
#if FA2_PP_DMA_IN_M
      if (grp == 0) n = issue_iter(i + 1);
#endif
      phase_m(Y{}, Y{}, i + 1);
      pp_barrier();
    }
    phase_v(T - 1);
    if (grp == 0) pp_wait_vm<0>();  // V(T-1), read by the last PV
    pp_barrier();
    phase_m(Y{}, N{}, T);
    if (grp == 0) pp_barrier();  // pairs with group 1's last barrier
    // every wave is past its last LDS read: the whole LDS is free
    if (S == 1) pp_barrier();
  }

  if (!hok) return;
  const float l_tot = sum_xor32(l_run);
  if (S == 1) {
    static_assert(kPPWaves * OStage<D>::kBytes <= sizeof(lds), "O staging exceeds LDS");
    const float inv = 1.f / l_tot;  // 0/0 -> NaN for a row with no key, as the reference
    store_o_staged<DT, D>(o, inv, lds + wave * OStage<D>::kBytes, a.o, o_base, a.o_ss, wq_first,
                          w.Lq, lane);
  } else {
    // partials go to the slot the one-head-per-unit layout gives this head
    // (decode_work with heads = 1), which the combine kernel reads
    const int unit = ((w.pair / kXcds) * group + w.hg + grp) * kXcds + w.pair % kXcds;
    const int64_t slot = static_cast<int64_t>(split) * a.part_slots + unit;
    const int r = wq * kWaveRows + l32;
    if (hi == 0) {
      float* ml = a.part_ml + (slot * kBM + r) * 2;
      ml[0] = m_run;
      ml[1] = l_tot;
    }
    float* po = a.part_o + (slot * kBM + r) * D + hi * 4;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(po + d * 32 + g * 8) =
            (f32x4){o[d][g * 4 + 0], o[d][g * 4 + 1], o[d][g * 4 + 2], o[d][g * 4 + 3]};
  }
}

}  // namespace fa2
