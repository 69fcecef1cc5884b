// fa2_kernel_decode.h - fp16/bf16 kernel of decode_attention and
// speculative_decode_attention (packed-head mode, KArgs::pack_m > 0).
//
// These calls read every K/V row once per kv head and do little arithmetic
// per byte (4 * rows FLOP per K/V element, rows = Hq/Hkv * M <= 64 per
// workgroup), so they are bound by HBM bandwidth: what matters is that
// every CU keeps enough bytes in flight and that the arithmetic never delays
// the next load.  The kernel therefore splits each workgroup into producer
// and consumer waves around a ring of kStages LDS slots:
//   * workgroup = 8 waves, one workgroup per CU (the ring takes 128 KiB of
//     LDS); it covers 64 unit rows (two chunks of 32) of one (sequence,
//     kv head, split);
//   * waves 4-7 (producers) only issue the direct-to-LDS DMAs of each 64-key
//     tile (DirectLoader, the prefill kernel's swizzled layout, a quarter of
//     the tile each; at D = 64 a tile is two 64-key sub-tiles, 128 keys),
//     keeping kStages - 1 tiles (96 KiB) in flight; after its part of tile j
//     has landed
//     (s_waitcnt vmcnt) a producer adds 1 to ready[j % kStages];
//   * waves 0-3 (consumers) wait for ready[] to count all four parts, compute
//     keys [32 (w & 1), +32) of each 64-key sub-tile for row chunk w >> 1 on
//     v_mfma_f32_32x32x16 (S^T = K Q^T, O^T = V^T P^T, the prefill kernel's
//     fragment layouts), then add 1 to done[j % kStages]; a producer reuses a
//     slot once done[] counts every active consumer;
//   * each consumer keeps its own running max / sum / O^T over its half of
//     the keys; the two halves are merged through LDS at the end.
// The counters live in LDS and only grow; a wave polls them with s_sleep
// between reads, and every poll gives up after KArgs::spin_cap reads
// (kDecSpinCap unless a test lowers it), so a wave cannot wait forever even
// if a counter were wrong.  A workgroup in which any wait gave up writes NaN
// for all its rows (output or split partials, which the merge turns into
// NaN rows) and adds 1 to g_decode_giveups, which fa2_decode_wait_giveups()
// reads: a wrong result is never silent.
//
// With several splits the kernel merges them itself (KArgs::merge_ctr): each
// split writes its partials at device scope and counts itself in the unit's
// merge word; the split that completes the count combines all partials with
// the combine kernel's arithmetic (combine_row), so the output is the same
// bit for bit and no combine launch follows.
#pragma once

#include "fa2_kernel_lds.h"

namespace fa2 {

constexpr int kDecRows = 64;      // unit rows per workgroup (two chunks of 32)
constexpr int kDecWaves = 8;      // 4 consumers + 4 producers
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kDecSpinCap = 1 << 16;  // ~5 ms of polling; real waits are microseconds

// Workgroups of the decode kernel in which a bounded wait gave up (one
// counter per device, read and reset by the host).
__device__ unsigned int g_decode_giveups;

// A ring slot holds kSub 64-key sub-tiles of K, then the same of V, so that
// one slot is 32 KiB at both head dims (the per-slot handshake costs the
// same whatever the slot size).
template <int D>
struct DecGeo {
  using G = SwzGeo<D>;
  static constexpr int kSub = D == 128 ? 1 : 2;
  static constexpr int kKeys = kSub * kBN;              // keys per slot
  static constexpr int kStages = 4;
  static constexpr int kHalf = kSub * G::kTileBytes;    // K (or V) part of a slot
  static constexpr int kSlot = 2 * kHalf;
  static constexpr int kLdsBytes = kStages * kSlot;
  // DMA instructions one producer wave issues per slot (K and V)
  static constexpr int kInstrPerTile = kSub * 2 * (G::kNC / 4);
};

// s_waitcnt vmcnt(n * IPT) for a wave-uniform n in [0, NS - 1]; the count
// must be an immediate.
template <int IPT, int NS>
__device__ __forceinline__ void wait_tiles_after(int n) {
  static_assert((NS - 1) * IPT <= 63, "vmcnt field");
#define FA2_WAIT_CASE(k)                                                                      \
  case k:                                                                                     \
    if constexpr (k <= NS - 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(k * IPT) : "memory"); \
    break;
  switch (n) {
    FA2_WAIT_CASE(1)
    FA2_WAIT_CASE(2)
    FA2_WAIT_CASE(3)
    FA2_WAIT_CASE(4)
    FA2_WAIT_CASE(5)
    FA2_WAIT_CASE(6)
    FA2_WAIT_CASE(7)
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
#undef FA2_WAIT_CASE
}

typedef __attribute__((address_space(3))) int lds_int_t;

// Wait until the LDS counter reaches `target`, at most `cap` polls (see
// above); false if the wait gave up.
__device__ __forceinline__ bool lds_wait_geq(lds_int_t* c, int target, int cap) {
  bool ok = false;
  for (int n = 0; n < cap; ++n) {
    if (__builtin_amdgcn_readfirstlane(*(volatile lds_int_t*)c) >= target) {
      ok = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");  // later LDS reads stay after the poll
  return ok;
}

// Add 1 to an LDS counter once per wave, after this wave's earlier LDS
// accesses (a wave's LDS operations are performed in order).
__device__ __forceinline__ void lds_signal(lds_int_t* c, int lane) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane == 0) __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int DT, int D, int MODE, bool BUF>
__global__ __launch_bounds__(kDecThreads, 1) void fa2_decode_kernel(KArgs a) {
  static_assert(DT != FA2_DTYPE_F32, "fp32 decode runs the register-staged kernel");
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int DC = D / 16;  // MFMA k-steps of S (16 head dims each)
  constexpr int DB = D / 32;  // 32-dim blocks of O^T
  using G = SwzGeo<D>;
  using DG = DecGeo<D>;
  constexpr int NS = DG::kStages;
  constexpr int IPT = DG::kInstrPerTile;
  constexpr int L = NS - 1;  // tiles a producer keeps in flight

  __shared__ __attribute__((aligned(1024))) char lds[DG::kLdsBytes];
  __shared__ int counters[2 * NS + 2];  // ready[NS], done[NS], a wait gave up, merge flag

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int kh = wave & 1;         // consumer: key half of every tile
  const int rc = (wave >> 1) & 1;  // consumer: row chunk

  const Work w = decode_work<MODE>(a, blockIdx.x);
  if (!w.valid) return;
  const int q0 = w.qblk * kDecRows;
  const int split = blockIdx.y;
  const int S = a.num_splits;

  constexpr int SUB = DG::kSub;
  const int ntiles = (w.Lk + DG::kKeys - 1) / DG::kKeys;
  const int t_begin = (ntiles * split) / S;
  const int T = (ntiles * (split + 1)) / S - t_begin;

  const int qrow = q0 + rc * kWaveRows + l32;
  const bool active = wave < 4 && q0 + rc * kWaveRows < w.Lq;
  // consumers that compute (both key halves of every row chunk with rows)
  const int nact = 2 * ((q0 < w.Lq ? 1 : 0) + (q0 + kWaveRows < w.Lq ? 1 : 0));

  lds_int_t* ready = (lds_int_t*)((__attribute__((address_space(3))) int*)counters);
  lds_int_t* done = ready + NS;
  lds_int_t* gave_up = done + NS;
  if (tid < 2 * NS + 1) ready[tid] = 0;
  bool waits_ok = true;  // every bounded wait of this wave reached its target
  __syncthreads();

  f32x16 o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = (f32x16){};
  float m_run = -INFINITY;  // running max of this lane's row, log2 domain
  float l_run = 0.f;        // running sum over this lane's keys

  auto slot = [&](int i) { return lds + (i % NS) * DG::kSlot; };

  if (wave >= 4) {
    // ---- producers ---------------------------------------------------------
    using Ld = DirectLoader<D, MODE, BUF, DT, kWaves, /*NT=*/true>;  // K/V are read once
    const Ld ld(a, wave - 4, lane);
    // paged caches with whole pages per wave and tile: the block-table
    // entries of tile i + 1 are read while tile i is issued
    const bool pre = Ld::uniform_pages(a);
    int rk[SUB], rv[SUB];
#pragma unroll
    for (int u = 0; u < SUB; ++u) rk[u] = rv[u] = 0;
    if (pre && T > 0) {
#pragma unroll
      for (int u = 0; u < SUB; ++u) {
        rk[u] = ld.prefetch_page(a, w, t_begin * DG::kKeys + u * kBN, false);
        rv[u] = ld.prefetch_page(a, w, t_begin * DG::kKeys + u * kBN, true);
      }
    }
    for (int i = 0; i < T; ++i) {
      // slot i % NS held tile i - NS: wait until every active consumer is done
      if (i >= NS) waits_ok &= lds_wait_geq(done + i % NS, nact * (i / NS), a.spin_cap);
      char* sl = slot(i);
      const int k0 = (t_begin + i) * DG::kKeys;
      if (pre) {
        int ck[SUB], cv[SUB];
#pragma unroll
        for (int u = 0; u < SUB; ++u) {
          ck[u] = rk[u];
          cv[u] = rv[u];
        }
        if (i + 1 < T) {
#pragma unroll
          for (int u = 0; u < SUB; ++u) {
            rk[u] = ld.prefetch_page(a, w, k0 + DG::kKeys + u * kBN, false);
            rv[u] = ld.prefetch_page(a, w, k0 + DG::kKeys + u * kBN, true);
          }
        }
#pragma unroll
        for (int u = 0; u < SUB; ++u)
          ld.template issue_at<false>(a, w, k0 + u * kBN, sl + u * G::kTileBytes, ck[u]);
#pragma unroll
        for (int u = 0; u < SUB; ++u)
          ld.template issue_at<true>(a, w, k0 + u * kBN, sl + DG::kHalf + u * G::kTileBytes,
                                     cv[u]);
      } else {
#pragma unroll
        for (int u = 0; u < SUB; ++u)
          ld.template issue<false>(a, w, k0 + u * kBN, sl + u * G::kTileBytes);
#pragma unroll
        for (int u = 0; u < SUB; ++u)
          ld.template issue<true>(a, w, k0 + u * kBN, sl + DG::kHalf + u * G::kTileBytes);
      }
      if (i >= L) {  // tile i - L has landed once only the L newer tiles are in flight
        wait_tiles_after<IPT, NS>(L);
        lds_signal(ready + (i - L) % NS, lane);
      }
    }
    for (int j = T > L ? T - L : 0; j < T; ++j) {
      wait_tiles_after<IPT, NS>(T - 1 - j);
      lds_signal(ready + j % NS, lane);
    }
  } else if (active) {
    // ---- consumers ---------------------------------------------------------
    const int qdiag = diag_row(a, qrow);
    const bool causal = a.mask != FA2_MASK_NONE;
    // Q^T fragments (B operand of S^T = K Q^T) of this lane's row
    u32x4 qf[DC];
    {
      const bool ok = qrow < w.Lq;
      const int64_t base = w.q_base + static_cast<int64_t>(qrow) * a.q_ss + hi * 8;
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
    // LDS byte offsets (prefill kernel layouts): K row 32*kh + l32, chunk
    // 2*cc + hi; V via the transpose read (source lane i of 16-lane group g
    // reads row 16c + 8rr + 4*(g/2) + i/4, dims 32db + 16(g%2) + 4(i%4)).
    const uint32_t koff0 = (kh * 32 + l32) * G::kRowBytes + ((hi ^ G::k(l32)) * 16);
    uint32_t voff0;
    {
      const int g = lane >> 4, i = lane & 15;
      const int r = 4 * (g >> 1) + (i >> 2);
      const int dim = 16 * (g & 1) + 4 * (i & 3);
      voff0 = r * G::kRowBytes + (((dim >> 3) ^ G::v(r)) * 16) + (dim & 7) * 2;
    }

    for (int i = 0; i < T; ++i) {
      // all four producers' parts
      waits_ok &= lds_wait_geq(ready + i % NS, 4 * (i / NS + 1), a.spin_cap);
#pragma unroll
      for (int u = 0; u < SUB; ++u) {
      const lds_char_t* kl = to_lds(slot(i)) + u * G::kTileBytes;
      const lds_char_t* vl = to_lds(slot(i)) + DG::kHalf + u * G::kTileBytes;
      const int k0 = (t_begin + i) * DG::kKeys + u * kBN;

      f32x16 s = (f32x16){};
#pragma unroll
      for (int cc = 0; cc < DC; ++cc) {
        const u32x4 kf = *(const lds_u32x4_t*)(kl + (koff0 ^ (32u * cc)));
        s = mma32<BF>(kf, qf[cc], s);
      }
      // key = k0 + 32*kh + 8*(i2/4) + 4*hi + i2%4: visible iff within the
      // sequence and, if causal, not past this row's diagonal (the smallest
      // diagonal of a unit is w.off, draft position 0); wave-uniform test
      const int kw0 = k0 + kh * 32;
      if ((kw0 + 32 > w.Lk) || (causal && (kw0 + 31 > w.off))) {
        const int kb = kw0 + hi * 4;
        int lim = w.Lk - 1 - kb;
        if (causal) lim = min(lim, qdiag + w.off - kb);
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2)
          if ((i2 >> 2) * 8 + (i2 & 3) > lim) s[i2] = -INFINITY;
      }

      float mx = -INFINITY;
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) mx = fmaxf(mx, s[i2]);
      mx = max_xor32_valu(mx);
      const float mt = mx * a.scale_log2;
      const bool need = mt > m_run + kRescaleThreshold;
      const float alpha = fast_exp2(need ? (m_run - mt) : 0.0f);
      m_run = need ? mt : m_run;
      const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
      u32x4 pf[2];
      {
        float p[16];
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2)
          p[i2] = fast_exp2(__builtin_fmaf(s[i2], a.scale_log2, -m_use));
#pragma unroll
        for (int half = 0; half < 2; ++half)
          pf[half] = (u32x4){pack2<BF>(p[half * 8 + 0], p[half * 8 + 1]),
                             pack2<BF>(p[half * 8 + 2], p[half * 8 + 3]),
                             pack2<BF>(p[half * 8 + 4], p[half * 8 + 5]),
                             pack2<BF>(p[half * 8 + 6], p[half * 8 + 7])};
      }
      float rs = 0.f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) rs = dot2_ones<BF>(pf[c][j], rs);
      l_run = l_run * alpha + rs;
      if (__any(need)) {
#pragma unroll
        for (int d = 0; d < DB; ++d) o[d] *= alpha;
      }
      // O^T += V^T P^T over this wave's two 16-key chunks
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int row = kh * 32 + c * 16;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const uint32_t voff = voff0 ^ (64u * d);
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4i16_t*)(vl + row * G::kRowBytes + voff));
          const v4i16 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4i16_t*)(vl + (row + 8) * G::kRowBytes + voff));
          const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
          const u32x2 h2 = __builtin_bit_cast(u32x2, hi4);
          o[d] = mma32<BF>((u32x4){l2[0], l2[1], h2[0], h2[1]}, pf[c], o[d]);
        }
      }
      }  // sub-tiles
      lds_signal(done + i % NS, lane);  // this wave's reads of the slot are complete
    }
  }

  // ---- merge the two key halves of each row chunk through LDS ------------
  // layout (the ring is drained): per row chunk, m[2][32] and l[2][32],
  // then the kh = 1 consumer's O^T (32 rows x D fp32)
  constexpr int kMergeO = kWaveRows * D * 4;
  constexpr int kMergeChunk = 4 * kWaveRows * 4 + kMergeO;
  static_assert(2 * kMergeChunk <= DG::kLdsBytes, "merge area");
  static_assert(2 * OStage<D>::kBytes <= DG::kLdsBytes, "output staging");
  // (producers take part in these barriers and do no merge work)
  if (!waits_ok && lane == 0) *(volatile lds_int_t*)gave_up = 1;
  __syncthreads();  // every wave is done with the ring
  const bool poisoned = *(volatile lds_int_t*)gave_up != 0;
  if (poisoned && tid == 0) __hip_atomic_fetch_add(&g_decode_giveups, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
  typedef __attribute__((address_space(3))) float lds_float_t;
  char* mc = lds + rc * kMergeChunk;
  lds_float_t* mm = (lds_float_t*)to_lds(mc);  // m[2][32], l[2][32]
  lds_char_t* po = to_lds(mc + 4 * kWaveRows * 4);
  const bool cons = wave < 4;
  const float l_tot = sum_xor32(l_run);
  if (cons && hi == 0) mm[kh * 32 + l32] = m_run;
  __syncthreads();
  const float m_all = cons ? fmaxf(m_run, mm[(kh ^ 1) * 32 + l32]) : 0.f;
  const float f = (m_all == -INFINITY) ? 0.f : fast_exp2(m_run - m_all);
  const float l_mine = l_tot * f;
  if (cons && kh == 1) {
    if (hi == 0) mm[64 + l32] = l_mine;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(lds_u32x4_t*)(po + (l32 * D + d * 32 + g * 8 + hi * 4) * 4) =
            __builtin_bit_cast(u32x4, (f32x4){o[d][g * 4 + 0] * f, o[d][g * 4 + 1] * f,
                                              o[d][g * 4 + 2] * f, o[d][g * 4 + 3] * f});
  }
  __syncthreads();
  float l_sum = 0.f;
  if (cons && kh == 0) {
    l_sum = l_mine + mm[64 + l32];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 x = __builtin_bit_cast(
            f32x4, *(const lds_u32x4_t*)(po + (l32 * D + d * 32 + g * 8 + hi * 4) * 4));
#pragma unroll
        for (int j = 0; j < 4; ++j) o[d][g * 4 + j] = o[d][g * 4 + j] * f + x[j];
      }
  }
  __syncthreads();  // the merge area is reused for the output staging
  // a wait gave up: these rows may have read an unfinished tile
  auto poison = [&]() {
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[d][j] = __builtin_nanf("");
    l_sum = 1.f;
  };
  if (S == 1) {
    if (!cons || kh != 0) return;
    if (poisoned) poison();
    const float inv = 1.f / l_sum;  // 0/0 -> NaN for a row with no key, as the reference
    store_o_staged<DT, D>(o, inv, lds + rc * OStage<D>::kBytes, a.o, w.o_base, a.o_ss,
                          q0 + rc * kWaveRows, w.Lq, lane);
    return;
  }
  if (cons && kh == 0) {
    if (poisoned) poison();
    // split partials (m, l, unnormalised O) of the rows that exist
    const int64_t slot_id = static_cast<int64_t>(split) * a.part_slots + blockIdx.x;
    const int r = rc * kWaveRows + l32;
    // (read by the merge of this kernel at device scope, or by the combine)
    if (qrow < w.Lq && r < a.part_rows) {
      if (a.merge_ctr)
        store_partial_rows<true, D>(a, slot_id, r, hi, m_all, l_sum, o);
      else
        store_partial_rows<false, D>(a, slot_id, r, hi, m_all, l_sum, o);
    }
  }
  if (!a.merge_ctr) return;  // the combine kernel merges
  // the split that completes the unit's count merges its partials
  merge_publish();
  __syncthreads();
  if (!merge_count(a, blockIdx.x, S, counters + 2 * NS + 1)) return;
  merge_rows<DT, D, kDecThreads, kDecRows>(a, blockIdx.x, S, min(a.part_rows, w.Lq - q0),
                                           w.o_base, q0);
}

}  // namespace fa2
