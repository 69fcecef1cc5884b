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
// the start of their softmax phase V(i) and wait for them at the end of
// V(i+1), just before the barrier that precedes
// their first use (M(i+2)); the last V tile is awaited before the final
// PV.  No slot is refilled before both groups have read it.
//
// Same arithmetic as fa2_fwd_lds_kernel (fa2_kernel_lds.h): transposed
// MFMA formulation, lazy rescale, exp2 with the folded scale, row sum of
// the rounded P; same results bit for bit.
#pragma once

#include "fa2_kernel_lds.h"

namespace fa2 {

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr int kPPWaves = 8;
constexpr int kPPThreads = kPPWaves * 64;
constexpr int kPPSlots = 3;

// Wave priority during the MFMA phase (0: unchanged).  Measured on MI355X
// (bf16 D=128): 2 beats 0 by 2-4% on c2/c3/c5.
#ifndef FA2_PP_PRIO
#define FA2_PP_PRIO 2
#endif
// LDS fragment reads run this many MFMAs ahead inside the MFMA phase.
// Measured on MI355X (bf16 D=128, alternating runs on one box): 4 beats 10
// by 0.5-1.3 % on c3/c4/c5 (c2 within noise), 2-5 within 0.5 % of 4; fewer
// fragments in flight also free 24 VGPRs (221 -> 197).
#ifndef FA2_PP_AHEAD
#define FA2_PP_AHEAD 4
#endif

// Issue order of the exponent block of a softmax phase (per lane: 32 FMAs
// with the folded scale and max, 32 v_exp_f32, then the packing of P and
// its row sum): one FMA, one exponential, alternately, then the rest.
// Measured on MI355X (bf16 D=128, alternating runs on one box, against the
// compiler's own order, which issues the exponentials in bursts of 8-14):
// c5 +1.9-2.2 %, c3 +0.7-1.7 %, c4 +0.7 %, c2 within its spread; all-FMAs-
// then-all-exponentials and two halves of each measured no gain.  The
// compiler moves this block past the branches that follow the softmax
// phase (the vmcnt waits), so the groups are placed in the block that ends
// with the phase's barrier, right before pp_barrier().
__device__ __forceinline__ void pp_softmax_order() {
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // VALU (not transcendental)
    __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);  // transcendental
  }
  __builtin_amdgcn_sched_group_barrier(0x002, 32, 0);
}


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

// One unit of work: a q-block of two query heads of one kv head (and one
// split of its KV range).
struct PPUnit {
  Work w;
  int T, t_begin, q0;
  int64_t q_base, o_base;  // this group's head
  bool hok;                // this group's head exists (odd head groups)
  // balanced walk: the unit's start in its stream and its weight (KV tiles,
  // at least 1), and whether this workgroup runs only a piece of it
  int us, W;
  bool part;
};

// Balanced walk (paged, one q-block per sequence, more units than
// workgroups).  The units of XCD x (L = x mod kXcds) form Hq/Hkv/2 streams,
// one per head pair g, over the kv-head pairs of the XCD in order, unit
// (j, g) weighing max(T_j, 1) where T_j is the KV tile count of pair j's
// q-block.  The XCD's n_x workgroups are split evenly over the G streams:
// workgroup kx = blockIdx.x / kXcds takes stream g = kx % G and segment
// k = kx / G of it, tiles [k C, (k + 1) C) with C = ceil(total / ns), ns =
// n_x / G segments per stream.  So every workgroup runs at most C tiles, whatever
// the spread of the sequence lengths, and the workgroups of segment k of
// the streams run the same pair's tiles at about the same time, sharing its
// K/V in the XCD's L2.  A unit cut by segment boundaries runs as pieces;
// the last of them to finish (merge_take_last, or the one whose count
// completes the unit's, merge_count) merges the others' partials (fragment
// order, store_partial_frag) with its own registers, in piece order, and
// writes the output.  The cut points follow from the lengths alone and the
// merge order is fixed, so results do not depend on timing.
//
// pp_bal_locate (wave 0): the first unit (pair index j), the segment's
// start and end, the first unit's stream start and C, into sh[0..4].
template <int MODE>
__device__ void pp_bal_locate(const KArgs& a, int x, int upp, int ns, int k, int* sh) {
  const int lane = threadIdx.x & 63;
  const int np = a.npairs > x ? (a.npairs - x + kXcds - 1) / kXcds : 0;  // pairs of the XCD
  const int per = (np + 63) / 64;
  const int j0 = min(np, lane * per), j1 = min(np, j0 + per);
  auto weight = [&](int j) -> int {
    const Work w = decode_work<MODE>(a, x + kXcds * (j * upp), 2);
    if (!w.valid) return 1;
    const int kv_end = kv_end_for_block(a.mask, w.qblk * kBM, w.Lq, w.Lk, w.off);
    const int t = (kv_end + kBN - 1) / kBN;
    return t > 1 ? t : 1;
  };
  int sum = 0;
  for (int j = j0; j < j1; ++j) sum += weight(j);
  int incl = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d);
    if (lane >= d) incl += y;
  }
  const int total = __shfl(incl, 63);
  const int C = total > ns ? (total + ns - 1) / ns : 1;
  const int target = k * C;
  const int excl = incl - sum;
  if (excl <= target && target < incl) {  // one lane, or none past the end
    int us = excl, j = j0;
    for (;; ++j) {
      const int W = weight(j);
      if (target < us + W) break;
      us += W;
    }
    sh[0] = j;
    sh[1] = target;
    sh[2] = target + min(C, total - target);
    sh[3] = us;
    sh[4] = C;
  } else if (lane == 0 && target >= total) {
    sh[0] = 0;
    sh[1] = 0;
    sh[2] = 0;
    sh[3] = 0;
    sh[4] = C;
  }
}

// CLAIM: the unit walk by claims (KArgs::claim, ragged/paged only), a
// separate instantiation so that the static walk keeps its registers.
// INLINE: a ragged launch without a plan kernel (KArgs::inline_plan): the
// item list from build_inline_plan, and the splits merged here; a separate
// instantiation for the same reason.
// BAL: the balanced walk (pp_bal_locate), paged launches without a plan
// kernel, one split; likewise separate.
template <int DT, int D, int MODE, bool BUF, bool CLAIM = false, bool INLINE = false,
          bool BAL = false>
__global__ __launch_bounds__(kPPThreads, 1) void fa2_fwd_pp_kernel(KArgs a) {
  static_assert(DT != FA2_DTYPE_F32, "fp32 uses the register-staged kernel");
  static_assert(!INLINE || (MODE == FA2_LAYOUT_RAGGED && !CLAIM), "inline plans: ragged, static walk");
  static_assert(!BAL || (MODE == FA2_LAYOUT_PAGED && !CLAIM && !INLINE), "balanced walk: paged");
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int DC = D / 16;  // MFMA k-steps of S (16 head dims each)
  constexpr int DB = D / 32;  // 32-dim blocks of O^T
  constexpr int SB = kBN / 32;
  using G = SwzGeo<D>;
  using LD = DirectLoader<D, MODE, BUF, DT, kWaves>;  // group 0 loads
  constexpr int kI = LD::kInstr;
  constexpr int kTile = G::kTileBytes;
  constexpr int kSlotBytes = 2 * kPPSlots * kTile;
  constexpr int kStageDims = 64;  // output staged in passes of 64 dims
  constexpr int kStores = kOStoreOps<D, kStageDims>;

  // K/V slots, then one output staging region per wave (separate, so the
  // next unit's tiles can land while this unit's rows are being stored)
  __shared__ __attribute__((aligned(1024)))
  char lds[kSlotBytes + kPPWaves * OStage<kStageDims>::kBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // waves w and w + 4 share SIMD w % 4
  const int wq = wave & 3;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int group = a.hq / a.hkv;
  const int split = blockIdx.y;
  // a ragged launch without a plan kernel: the item list in LDS
  const InlinePlan* ip = nullptr;
  if constexpr (INLINE) {
    __shared__ InlinePlan iplan;
    build_inline_plan<MODE>(a, &iplan);
    ip = &iplan;
  }
  const int S = INLINE ? __builtin_amdgcn_readfirstlane(ip->splits) : launch_splits(a);
  if (split >= S) return;
  // Balanced walk: this workgroup's stream (XCD bal_x(), head pair
  // bal_g()) and segment (bal_k()); the segment's bounds and C stay in LDS
  // and are read at unit boundaries only, so that no scalar register is
  // added to the tile loop's.
  __shared__ int bal_sh[5];
  auto bal_x = [&]() { return static_cast<int>(blockIdx.x) % kXcds; };
  auto bal_upp = [&]() { return (group + 1) / 2; };
  auto bal_g = [&]() { return (static_cast<int>(blockIdx.x) / kXcds) % bal_upp(); };
  auto bal_k = [&]() { return (static_cast<int>(blockIdx.x) / kXcds) / bal_upp(); };
  auto bal_rd = [&](int i) { return __builtin_amdgcn_readfirstlane(bal_sh[i]); };
  if constexpr (BAL) {
    const int ns = ((static_cast<int>(gridDim.x) - bal_x() + kXcds - 1) / kXcds) / bal_upp();
    if (bal_k() >= ns) return;
    if (wave == 0) pp_bal_locate<MODE>(a, bal_x(), bal_upp(), ns, bal_k(), bal_sh);
    __syncthreads();
  }
  // part slot of head h of piece s of unit v (balanced walk): segment
  // v.us / C + s of the stream, its workgroup's first (kind 0: from the
  // segment's start) or last (kind 1: from inside to past its end) piece
  auto bal_slot = [&](const PPUnit& v, int s, int h, int C) -> int64_t {
    const int kf = v.us / C;
    const int kind = (s == 0 && v.us != kf * C) ? 1 : 0;
    const int wg = ((kf + s) * bal_upp() + bal_g()) * kXcds + bal_x();
    return static_cast<int64_t>((wg * 2 + kind) * 2 + h);
  };
  const bool causal = a.mask != FA2_MASK_NONE;
  char* const stage = lds + kSlotBytes + wave * OStage<kStageDims>::kBytes;

  // per-lane LDS offsets, as in fa2_fwd_lds_kernel
  const uint32_t koff0 = l32 * G::kRowBytes + ((hi ^ G::k(l32)) * 16);
  uint32_t voff0;
  {
    const int g = lane >> 4, i = lane & 15;
    const int r = 4 * (g >> 1) + (i >> 2);
    const int dim = 16 * (g & 1) + 4 * (i & 3);
    voff0 = r * G::kRowBytes + (((dim >> 3) ^ G::v(r)) * 16) + (dim & 7) * 2;
  }
  const LD ld(a, wq, lane);

  // Persistent: gridDim.x workgroups walk the units (heaviest first) in
  // rounds; odd rounds run backwards over blocks of kXcds workgroups, which
  // pairs heavy with light units and keeps each unit on the XCD that the
  // unit layout of decode_work intends.
  const int P = gridDim.x;
  auto unit_index = [&](int r) -> int {
    const int wg = blockIdx.x;
    int pos = wg;
    if (r & 1) pos = (P % kXcds) ? (P - 1 - wg) : ((P / kXcds - 1 - wg / kXcds) * kXcds + wg % kXcds);
    return r * P + pos;
  };
  auto make_unit = [&](int L, PPUnit& u) -> bool {
    u.w = decode_work<MODE, true>(a, L, 2, ip);
    if (!u.w.valid) return false;
    int kv_end;
    if (a.qpair) {  // MHA: q-blocks 2k (group 0) and 2k + 1 (group 1) of one head
      const int qb = 2 * u.w.qblk;
      u.q0 = (qb + grp) * kBM;
      u.hok = u.q0 < u.w.Lq;
      u.q_base = u.w.q_base;
      u.o_base = u.w.o_base;
      const int last = (qb + 1) * kBM < u.w.Lq ? qb + 1 : qb;  // same tiles for both groups
      kv_end = kv_end_for_block(a.mask, last * kBM, u.w.Lq, u.w.Lk, u.w.off);
    } else {
      u.hok = u.w.hg + grp < group;
      u.q_base = u.w.q_base + grp * a.q_sh;
      u.o_base = u.w.o_base + grp * a.o_sh;
      u.q0 = u.w.qblk * kBM;
      kv_end = kv_end_for_block(a.mask, u.q0, u.w.Lq, u.w.Lk, u.w.off);
    }
    const int ntiles = (kv_end + kBN - 1) / kBN;
    u.t_begin = (ntiles * split) / S;
    u.T = (ntiles * (split + 1)) / S - u.t_begin;
    return true;
  };
  // Claimed units (a.claim): workgroup g walks units L = c * kXcds + g mod
  // kXcds of its group, c = g / kXcds first, then the indices its group's
  // counter hands out; r is then c.  Units of a group are valid up to some
  // index and invalid after it (the work list's order), so the first invalid
  // one ends the walk.
  static_assert(!CLAIM || MODE != FA2_LAYOUT_DENSE, "claims need the plan kernel's counters");
  constexpr bool dyn = CLAIM;
  const int xg = blockIdx.x % kXcds;
  const int n_x = (P - xg + kXcds - 1) / kXcds;  // workgroups of the group
  // next valid unit at round >= r (uniform); false when none is left
  PPUnit cur;
  auto next_unit = [&](int& r, PPUnit& u) -> bool {
    if constexpr (BAL) {  // r: pair index in the stream, from the first unit's on
      // the unit's stream start: the first unit's, or the current unit's end
      const int us = r == bal_rd(0) ? bal_rd(3) : cur.us + cur.W;
      const int s0 = bal_rd(1), s1 = bal_rd(2);
      if (us >= s1) return false;
      if (!make_unit(bal_x() + kXcds * (r * bal_upp() + bal_g()), u)) return false;
      const int W = u.T > 1 ? u.T : 1;
      const int b = max(us, s0), e = min(us + W, s1);
      u.us = us;
      u.W = W;
      u.part = !(b == us && e == us + W);
      u.t_begin = b - us;
      u.T = u.T > 0 ? e - b : 0;
      return true;
    }
    if (dyn) {
      const int L = r * kXcds + xg;
      return L >= 0 && L < a.units && make_unit(L, u);
    }
    for (;; ++r) {
      const int L = unit_index(r);
      if (L >= a.units) return false;
      if (make_unit(L, u)) return true;
    }
  };

  u32x4 qf[DC];
  auto load_q = [&](const PPUnit& u) {
    const int qrow = u.q0 + wq * kWaveRows + l32;
    const bool ok = u.hok && qrow < u.w.Lq;
    const int64_t base = u.q_base + static_cast<int64_t>(qrow) * a.q_ss + hi * 8;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      Raw8<DT> r;
      if (ok)
        load_raw8<DT>(r, a.q, base + c * 16);
      else
        zero_raw8<DT>(r);
      qf[c] = to16<DT>(r);
    }
  };

  f32x16 o[DB];
  float m_run, l_run;
  f32x16 s[SB];
  u32x4 pf[kBN / 16];

  // wait until at most n of this wave's vector memory operations are
  // outstanding; n is one of the counts this kernel produces
  auto wait_vm = [&](int n) {
    if (n >= 2 * kI + kStores)
      pp_wait_vm<2 * kI + kStores>();
    else if (n >= kI + kStores)
      pp_wait_vm<kI + kStores>();
    else if (n >= kStores && kStores > 2 * kI)
      pp_wait_vm<kStores>();
    else if (n >= 2 * kI)
      pp_wait_vm<2 * kI>();
    else if (n >= kI)
      pp_wait_vm<kI>();
    else if (n >= DC)
      pp_wait_vm<DC>();
    else
      pp_wait_vm<0>();
  };
  using Y = std::integral_constant<bool, true>;
  using N = std::integral_constant<bool, false>;

  // Claims: wave 0 adds 1 to its group's counter (one lane, returning the
  // old value) a few tiles before its unit ends; the atomic is issued before
  // that phase's tile loads, so the phase's wait for them (vmcnt counts
  // complete in issue order) also covers it.  The claimed index goes to the
  // other waves through LDS across the phase barrier, in one of two words
  // by claim parity: a word is written again only after every wave has
  // passed the barrier that publishes the claim in between, after its read.
  __shared__ int claim_next[2];
  int nclaim = 0;
  uint32_t claimed = 0;
  auto claim_issue = [&]() {
    if (lane == 0)
      asm volatile("global_atomic_add %0, %1, %2, off sc0"
                   : "=v"(claimed)
                   : "v"(a.claim + xg), "v"(1u)
                   : "memory");
  };
  // after a wait that covers the atomic (vmcnt); before a pp_barrier()
  auto claim_publish = [&]() {
    asm volatile("" : "+v"(claimed));  // no use of the value before the wait
    const int c = __builtin_amdgcn_readfirstlane(claimed);
    if (lane == 0) claim_next[nclaim & 1] = n_x + c;
  };
  // after that barrier (all waves)
  auto claim_read = [&]() -> int {
    const int c = *static_cast<volatile int*>(&claim_next[nclaim & 1]);
    ++nclaim;
    return __builtin_amdgcn_readfirstlane(c);
  };
  constexpr int kClaimLead = 2;  // tiles between the claim and the unit's last tile

  int r = dyn ? static_cast<int>(blockIdx.x) / kXcds : (BAL ? bal_rd(0) : 0);
  if (!next_unit(r, cur)) return;
  int gb = 0;          // tile i of the current unit is tile gb + i of this workgroup's stream
  bool pre = false;    // the current unit's Q and first tiles were issued by the previous one
  for (;;) {
    const int T = cur.T;
    const PPUnit& u = cur;
    const Work& w = u.w;
    // The next unit is looked up at this one's tail, so that only one unit
    // is live during the tile loop (scalar registers).  Its Q and first
    // tiles are prefetched during this unit's last phases when it has
    // tiles and there is one split (the store count below is fixed then).
    PPUnit nxt;
    int rn = r + 1;
    bool has_next = false, pre_next = false;

    auto kslot = [&](int i) { return lds + ((gb + i) % kPPSlots) * kTile; };
    auto vslot = [&](int i) { return lds + (kPPSlots + (gb + i) % kPPSlots) * kTile; };
    const int qrow = u.q0 + wq * kWaveRows + l32;
    const int wq_first = u.q0 + wq * kWaveRows;

#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = (f32x16){};
    m_run = -INFINITY;
    l_run = 0.f;
    // group 1 loads its Q after the first barrier (below)
    if (!pre && grp == 0) load_q(u);

    // M phase: PV of the previous tile, then S of this one.
    auto phase_m = [&](auto has_pv, auto has_s, int i) {
      constexpr bool kPV = decltype(has_pv)::value;
      constexpr bool kS = decltype(has_s)::value;
      // slot bases resolved before the scheduling region (scalar work that
      // would otherwise sit between the reads the region is ordering)
      const uint32_t vbase = kPV ? lds_addr_of(vslot(i - 1)) : 0u;
      const uint32_t kbase = kS ? lds_addr_of(kslot(i)) : 0u;
      // a scheduling region of its own: nothing moves in or out
      __builtin_amdgcn_sched_barrier(0);
#if FA2_PP_PRIO
      __builtin_amdgcn_s_setprio(FA2_PP_PRIO);
#endif
      // Fragment k: the PV fragments first (c-major: V^T from two transposed
      // reads; consecutive MFMAs go to different accumulators), then the S
      // fragments (cc-major: one K row chunk).  Each accumulator still sums
      // in the same order.  The reads are written kAhead fragments ahead of
      // their MFMA, so that order holds even where the scheduler keeps the
      // source order.
      constexpr int kNPV = kPV ? DB * (kBN / 16) : 0;
      constexpr int kN = kNPV + (kS ? SB * DC : 0);
      constexpr int kAhead = FA2_PP_AHEAD < kN ? FA2_PP_AHEAD : kN;
      const lds_char_t* vl = lds_ptr(vbase);
      const lds_char_t* kl = lds_ptr(kbase);
      auto frag = [&](auto kc) -> u32x4 {
        constexpr int k = decltype(kc)::value;
        if constexpr (k < kNPV) {
          constexpr int c = k / DB, d = k % DB;
          const uint32_t voff = voff0 ^ (64u * d);
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4i16_t*)(vl + (16 * c) * G::kRowBytes + voff));
          const v4i16 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4i16_t*)(vl + (16 * c + 8) * G::kRowBytes + voff));
          const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
          const u32x2 h2 = __builtin_bit_cast(u32x2, hi4);
          return (u32x4){l2[0], l2[1], h2[0], h2[1]};
        } else {
          constexpr int kk = k - kNPV, cc = kk / SB, sb = kk % SB;
          return *(const lds_u32x4_t*)(kl + sb * 32 * G::kRowBytes + (koff0 ^ (32u * cc)));
        }
      };
      auto mma_k = [&](auto kc, const u32x4& f) {
        constexpr int k = decltype(kc)::value;
        if constexpr (k < kNPV) {
          constexpr int c = k / DB, d = k % DB;
          o[d] = mma32<BF>(f, pf[c], o[d]);
        } else {
          constexpr int kk = k - kNPV, cc = kk / SB, sb = kk % SB;
          s[sb] = mma32<BF>(f, qf[cc], s[sb]);
        }
      };
      if constexpr (kS) {
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) s[sb] = (f32x16){};
      }
      u32x4 fr[kN];
      static_for<kAhead>([&](auto kc) { fr[decltype(kc)::value] = frag(kc); });
      static_for<kN>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        mma_k(kc, fr[k]);
        if constexpr (k + kAhead < kN)
          fr[k + kAhead] = frag(std::integral_constant<int, k + kAhead>{});
      });
      // the same order as scheduling groups (reads of the first kAhead
      // fragments, then per MFMA k: the MFMA, the reads of fragment k + kAhead)
      {
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
      const int k0 = (u.t_begin + i) * kBN;
      if ((k0 + kBN > w.Lk) || (causal && (k0 + kBN - 1 > wq_first + w.off))) {
        int lim = w.Lk - 1 - k0 - hi * 4;
        if (causal) lim = min(lim, qrow + w.off - k0 - hi * 4);
        // key offset c is hidden iff lim - c < 0: the sign, spread over the
        // word, selects -inf (bit select, no compare masks in scalar registers)
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
          for (int i2 = 0; i2 < 16; ++i2) {
            const int c = sb * 32 + (i2 >> 2) * 8 + (i2 & 3);
            const uint32_t hide = static_cast<uint32_t>((lim - c) >> 31);
            // (bit_cast through a scalar: this compiler reads element 0 when
            // bit_cast is applied to a subscripted vector element)
            const float x = s[sb][i2];
            s[sb][i2] = __builtin_bit_cast(
                float, (hide & 0xFF800000u) | (~hide & __builtin_bit_cast(uint32_t, x)));
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
        ld.template issue<true>(a, w, (u.t_begin + i + 1) * kBN, vslot(i + 1));
        n += kI;
      }
      if (i + 2 < T) {
        ld.template issue<false>(a, w, (u.t_begin + i + 2) * kBN, kslot(i + 2));
        n += kI;
      }
      return n;
    };
    // group 0: the first tiles of unit v (K(0), K(1) if any, V(0)), whose
    // tile 0 is tile g0 of the stream
    auto issue_first = [&](const PPUnit& v, int g0) {
      char* k0s = lds + (g0 % kPPSlots) * kTile;
      char* k1s = lds + ((g0 + 1) % kPPSlots) * kTile;
      char* v0s = lds + (kPPSlots + g0 % kPPSlots) * kTile;
      ld.template issue<false>(a, v.w, v.t_begin * kBN, k0s);
      if (v.T > 1) ld.template issue<false>(a, v.w, (v.t_begin + 1) * kBN, k1s);
      ld.template issue<true>(a, v.w, v.t_begin * kBN, v0s);
    };

    // tile of the claim (T >= 2); a one-tile unit claims before its first barrier
    const int i_claim = T - 1 - kClaimLead > 0 ? T - 1 - kClaimLead : 0;
    if (T > 0) {
      if (grp == 0) {
        const bool claim_now = dyn && T == 1 && wave == 0;
        if (claim_now) claim_issue();
        if (!pre) {
          // K(1) and V(0) go out once K(0) and Q have landed: at a launch
          // every workgroup fetches these at once, and the first MFMA phase
          // needs only K(0) and Q (c5 +1.5 %, c2 and c3 unchanged)
          ld.template issue<false>(a, w, u.t_begin * kBN, kslot(0));
          pp_wait_vm<0>();
          if (T > 1) ld.template issue<false>(a, w, (u.t_begin + 1) * kBN, kslot(1));
          ld.template issue<true>(a, w, u.t_begin * kBN, vslot(0));
        } else {
          // K(0) and Q have landed: what was issued after K(0) may be in
          // flight (K(1), V(0), and the previous unit's output stores)
          wait_vm((T > 1 ? 2 * kI : kI) + kStores);
        }
        if (claim_now) {
          pp_wait_vm<0>();
          claim_publish();
        }
      }
      pp_barrier();
      if (grp != 0) {
        // Group 1 runs one phase behind.  Its Q loads go out now, under
        // group 0's first MFMA phase, instead of competing for HBM with
        // the loads that phase waits for (at a launch every workgroup
        // fetches its first Q and tiles at once: ~4 us before any MFMA).
        if (!pre) load_q(u);
        pp_barrier();
      }
      phase_m(N{}, Y{}, 0);
      pp_barrier();
      for (int i = 0; i + 1 < T; ++i) {
        int n = 0;
        const bool claim_now = dyn && i == i_claim && wave == 0;
        if (claim_now) claim_issue();
        if (grp == 0) n = issue_iter(i);
        phase_v(i);
        // K(i+1) and V(i) (read from M(i+1) on) have landed; the loads of
        // the current issue may still be in flight (n >= kI: the claim,
        // issued before them, has returned)
        if (grp == 0) wait_vm(n);
        if (claim_now) claim_publish();
        pp_softmax_order();
        pp_barrier();
        phase_m(Y{}, Y{}, i + 1);
        pp_barrier();
      }
      if (dyn) rn = claim_read();
      has_next = next_unit(rn, nxt);
      // (not when this unit's rows go out as partials: the waits after the
      // prefetch count the staged output stores)
      // (a piece of the balanced walk that writes partials waits for all of
      // them, and one that merges waits for its loads, before its stores)
      pre_next = has_next && nxt.T > 0 && S == 1 && !a.part_out;
      // Q of the next unit: this group's last S is done
      if (pre_next) load_q(nxt);
      phase_v(T - 1);
      // V(T-1), read by the last PV, has landed (the next Q may be in
      // flight).  A wave none of whose rows of the next unit exists skips
      // its Q loads as a whole (one branch per load pair, all on the same
      // wave-uniform condition), so it issued DC of them or none.
      if (grp == 0) {
        const bool q_issued = pre_next && nxt.hok && nxt.q0 + wq * kWaveRows < nxt.w.Lq;
        if (q_issued)
          pp_wait_vm<DC>();
        else
          pp_wait_vm<0>();
      }
      pp_softmax_order();
      pp_barrier();
      // the first tiles of the next unit go to slots no longer read
      if (pre_next && grp == 0) issue_first(nxt, gb + T);
      phase_m(Y{}, N{}, T);
      if (grp == 0) pp_barrier();  // pairs with group 1's last barrier
    } else {
      if (dyn) {
        // both groups have passed the same number of barriers here
        if (wave == 0) {
          claim_issue();
          pp_wait_vm<0>();
          claim_publish();
        }
        pp_barrier();
        rn = claim_read();
      }
      has_next = next_unit(rn, nxt);
    }

    // this wave's rows of the output, from v / l (staged through LDS)
    auto store_out = [&](const f32x16 (&v)[DB], float l) {
      const float inv = 1.f / l;  // 0/0 -> NaN for a row with no key, as the reference
      const int nrows = max(0, min(w.Lq - wq_first, kWaveRows));
      const __amdgpu_buffer_rsrc_t out = make_rsrc_uniform(
          static_cast<uint16_t*>(a.o) + u.o_base + static_cast<int64_t>(wq_first) * a.o_ss,
          static_cast<uint32_t>(nrows) * static_cast<uint32_t>(a.o_ss * 2));
      store_o_staged_buf<DT, D, kStageDims>(v, inv, stage, out, a.o_ss, lane);
    };
    if (BAL && u.part) {
      // Balanced walk, a piece of a cut unit (both groups, uniform): unless
      // every other piece has counted already, this piece's partials go out
      // and it counts; the last piece merges all of them, in piece order,
      // with its own from registers, and writes the output.
      __shared__ int bal_flag[2];
      const float l_tot = sum_xor32(l_run);
      const int C = bal_rd(4);
      const int kf = u.us / C;
      const int np = (u.us + u.W - 1) / C - kf + 1;
      const int mine = bal_k() - kf;
      const int unit0 = ((w.pair / kXcds) * group + w.hg) * kXcds + w.pair % kXcds;
      if (threadIdx.x == 0)
        *static_cast<volatile int*>(&bal_flag[0]) = merge_take_last(a, unit0, np) ? 1 : 0;
      __syncthreads();
      bool last = *static_cast<volatile int*>(&bal_flag[0]) != 0;
      if (!last) {
        if (u.hok) store_partial_frag<D>(a, bal_slot(u, mine, grp, C), wq, lane, m_run, l_tot, o);
        merge_publish();
        __syncthreads();
        last = merge_count(a, unit0, np, &bal_flag[1]);
      }
      if (last && u.hok) {
        // the pieces' partials are read after the count that made this piece
        // the last, which followed every other piece's stores.  Per element
        // the sum runs over the pieces in order; the dims go in two halves
        // (registers: this piece's O, half an accumulator, half a piece).
        auto piece_ml = [&](int s, float& ms, float& ls) {
          ms = m_run;
          ls = l_tot;
          if (s != mine) {
            const u32x2 ml = load_partial_frag_ml(a, bal_slot(u, s, grp, C), wq, l32);
            const uint32_t mw = ml[0], lw = ml[1];
            ms = __builtin_bit_cast(float, mw);
            ls = __builtin_bit_cast(float, lw);
          }
        };
        float g = -INFINITY;
        for (int s = 0; s < np; ++s) {
          float ms, ls;
          piece_ml(s, ms, ls);
          g = fmaxf(g, ms);
        }
        const float g_use = g == -INFINITY ? 0.f : g;
        float lsum = 0.f;
        for (int s = 0; s < np; ++s) {
          float ms, ls;
          piece_ml(s, ms, ls);
          lsum += fast_exp2(ms - g_use) * ls;
        }
        constexpr int kH = DB / 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          f32x16 acc[kH];
#pragma unroll
          for (int dd = 0; dd < kH; ++dd) acc[dd] = (f32x16){};
          for (int s = 0; s < np; ++s) {
            float ms, ls;
            piece_ml(s, ms, ls);
            const float wgt = fast_exp2(ms - g_use);
            const int64_t slot = bal_slot(u, s, grp, C);
#pragma unroll
            for (int dd = 0; dd < kH; ++dd) {
              const f32x16 x =
                  s == mine ? o[h * kH + dd] : load_partial_frag_o<D>(a, slot, wq, lane, h * kH + dd);
              acc[dd] += wgt * x;
            }
          }
#pragma unroll
          for (int dd = 0; dd < kH; ++dd) o[h * kH + dd] = acc[dd];
        }
        store_out(o, lsum);
      }
    } else if (u.hok) {
      const float l_tot = sum_xor32(l_run);
      if (S == 1 && !a.part_out) {
        store_out(o, l_tot);
      } else {
        // partials go to the slot the one-head-per-unit layout gives this
        // head (decode_work with heads = 1), which the combine kernel reads
        const int unit =
            ((w.pair / kXcds) * group + w.hg + grp) * kXcds + w.pair % kXcds;
        const int64_t slot = static_cast<int64_t>(split) * a.part_slots + unit;
        const int rr = wq * kWaveRows + l32;
        if (INLINE && a.merge_ctr)
          store_partial_rows<true, D>(a, slot, rr, hi, m_run, l_tot, o);
        else
          store_partial_rows<false, D>(a, slot, rr, hi, m_run, l_tot, o);
      }
    }
    // Splits merged in this kernel: the split that completes the unit's
    // count (kept in the first head's part slot) merges both heads.  Both
    // groups pass the same two barriers, so their pairing is unchanged.
    if (INLINE && S > 1 && a.merge_ctr) {
      __shared__ int merge_flag;
      merge_publish();
      __syncthreads();
      const int unit0 = ((w.pair / kXcds) * group + w.hg) * kXcds + w.pair % kXcds;
      if (merge_count(a, unit0, S, &merge_flag)) {
        const int q0 = w.qblk * kBM;
        const int rows = min(kBM, w.Lq - q0);
        merge_rows<DT, D, kPPThreads, kBM>(a, unit0, S, rows, w.o_base, q0);
        if (w.hg + 1 < group)
          merge_rows<DT, D, kPPThreads, kBM>(a, unit0 + kXcds, S, rows, w.o_base + a.o_sh,
                                                q0);
      }
    }

    if (!has_next) break;
    gb += T;
    pre = pre_next;
    cur = nxt;
    r = rn;
  }
}

}  // namespace fa2
