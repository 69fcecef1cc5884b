// fa2_kernel_short.h - fp16/bf16 forward kernel for calls too small to fill
// the GPU (a few 128-row q-blocks, short KV ranges).
//
// The other kernels give one q-block's whole KV sweep to one workgroup, so a
// small call lasts as long as its longest sweep (c1: 16 workgroups, the
// longest walking 8 tiles one after another).  Here a workgroup of 4 waves
// takes one 32-row query block of one head, and its KV tiles are dealt to
// the waves round-robin: each wave loads its own tiles into its own LDS
// slots (direct-to-LDS, the swizzled layouts of fa2_kernel_lds.h), runs the
// same transposed MFMA steps and online softmax as the other kernels over
// them, and the 4 partial states (row max m, row sum l, unnormalised O) are
// merged through LDS at the end:
//   M = max_w m_w,  f_w = 2^(m_w - M)  (0 for a wave with no visible key),
//   out = sum_w f_w O_w / sum_w f_w l_w
// (the log-sum-exp merge of the split partials, attention.py:659-746, done
// inside the workgroup, so no partial buffer and no combine launch).  Q is
// loaded once per workgroup into LDS (K's swizzle) and read by all waves.
#pragma once

#include "fa2_kernel_pp.h"

namespace fa2 {

constexpr int kShWaves = 4;
constexpr int kShThreads = kShWaves * 64;
constexpr int kShRows = 32;              // query rows per workgroup
constexpr int kShSub = kBM / kShRows;    // workgroups per 128-row work item
constexpr int kShMaxTiles = 32;          // KV ranges (64-key tiles) the automatic choice
constexpr int kShMinTiles = 8;           // gives this kernel

template <int DT, int D, int MODE, bool BUF>
// (LDS: two workgroups per CU at D = 64, one at 128)
__global__ __launch_bounds__(kShThreads, D > 64 ? 1 : 2) void fa2_fwd_short_kernel(KArgs a) {
  static_assert(DT != FA2_DTYPE_F32, "fp32 uses the register-staged kernel");
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int DC = D / 16;  // MFMA k-steps of S (16 head dims each)
  constexpr int DB = D / 32;  // 32-dim blocks of O^T
  constexpr int SB = kBN / 32;
  using G = SwzGeo<D>;
  using LD = DirectLoader<D, MODE, BUF, DT, 1>;  // each wave loads whole tiles
  constexpr int kI = LD::kInstr;
  constexpr int kTile = G::kTileBytes;
  constexpr int kQInstr = kShRows * G::kRowBytes / 1024 / kShWaves;  // Q DMAs per wave
  constexpr int kOPitch = D + 4;  // merge rows (floats); the pad spreads banks
  static_assert(kQInstr >= 1 && kQInstr * kShWaves * 1024 == kShRows * G::kRowBytes, "Q split");
  static_assert(kShRows * kOPitch * 4 <= 2 * kTile, "a wave's merge rows fit its tile slots");

  // per wave: K slot, V slot (reused by the merge); then Q, then row stats
  __shared__ __attribute__((aligned(1024))) char lds[kShWaves * 2 * kTile + kShRows * G::kRowBytes];
  __shared__ float mrow[kShWaves][kShRows];
  __shared__ float lrow[kShWaves][kShRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const bool causal = a.mask != FA2_MASK_NONE;

  // grid.x = (work items x q heads, in decode_work's layout) x kShSub: the
  // kShSub 32-row blocks of one unit are `units` ids apart, so they run on
  // the XCD that decode_work's layout gives the unit
  const int units = gridDim.x / kShSub;
  const int sub = blockIdx.x / units;
  const int L = blockIdx.x - sub * units;
  const Work w = decode_work<MODE>(a, L, 1);
  if (!w.valid) return;
  const int q0 = w.qblk * kBM + sub * kShRows;
  if (q0 >= w.Lq) return;
  int kv_end = w.Lk;
  if (causal) kv_end = max(0, min(w.Lk, min(q0 + kShRows, w.Lq) + w.off));
  const int T = (kv_end + kBN - 1) / kBN;

  char* const kslot = lds + wave * 2 * kTile;
  char* const vslot = kslot + kTile;
  char* const qlds = lds + kShWaves * 2 * kTile;
  const LD ld(a, 0, lane);

  // Q rows q0.. into LDS with K's layout (row r, 16-byte chunk c at slot
  // c ^ k(r)): this wave's kQInstr instructions; rows past Lq read zeros
  {
    const int nrows = max(0, min(w.Lq - q0, kShRows));
    const uint32_t rsb = static_cast<uint32_t>(a.q_ss * 2);
    const u32x4 qr = rsrc_words(static_cast<const uint16_t*>(a.q) + w.q_base +
                                    static_cast<int64_t>(q0) * a.q_ss,
                                static_cast<uint32_t>(nrows) * rsb);
#pragma unroll
    for (int j = 0; j < kQInstr; ++j) {
      const int idx = (wave * kQInstr + j) * 64 + lane;  // 16-byte slot of the Q block
      const int r = idx / G::kNC, slot = idx % G::kNC;
      dma_buffer_x4(qr, lds_addr_of(qlds) + (wave * kQInstr + j) * 1024,
                    r * rsb + ((slot ^ G::k(r)) * 16));
    }
  }
  // this wave's first tile
  if (wave < T) {
    ld.template issue<false>(a, w, wave * kBN, kslot);
    ld.template issue<true>(a, w, wave * kBN, vslot);
    pp_wait_vm<2 * kI>();  // Q landed (K, V may be in flight)
  } else {
    pp_wait_vm<0>();
  }
  pp_barrier();  // every wave's part of Q has landed

  // per-lane LDS offsets, as in fa2_fwd_lds_kernel
  const uint32_t koff0 = l32 * G::kRowBytes + ((hi ^ G::k(l32)) * 16);
  uint32_t voff0;
  {
    const int g = lane >> 4, i = lane & 15;
    const int r = 4 * (g >> 1) + (i >> 2);
    const int dim = 16 * (g & 1) + 4 * (i & 3);
    voff0 = r * G::kRowBytes + (((dim >> 3) ^ G::v(r)) * 16) + (dim & 7) * 2;
  }
  u32x4 qf[DC];
  {
    const lds_char_t* ql = lds_ptr(lds_addr_of(qlds));
#pragma unroll
    for (int c = 0; c < DC; ++c) qf[c] = *(const lds_u32x4_t*)(ql + (koff0 ^ (32u * c)));
  }

  f32x16 o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = (f32x16){};
  float m_run = -INFINITY, l_run = 0.f;
  const int qrow = q0 + l32;
  const lds_char_t* kl = lds_ptr(lds_addr_of(kslot));
  const lds_char_t* vl = lds_ptr(lds_addr_of(vslot));

  for (int t = wave; t < T; t += kShWaves) {
    const int k0 = t * kBN;
    const bool more = t + kShWaves < T;
    pp_wait_vm<kI>();  // K(t) has landed (V(t) may be in flight)
    // S^T = K Q^T
    f32x16 s[SB];
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) s[sb] = (f32x16){};
#pragma unroll
    for (int cc = 0; cc < DC; ++cc)
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        const u32x4 f = *(const lds_u32x4_t*)(kl + sb * 32 * G::kRowBytes + (koff0 ^ (32u * cc)));
        s[sb] = mma32<BF>(f, qf[cc], s[sb]);
      }
    // the K slot is free once this wave's reads of it are done
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (more) ld.template issue<false>(a, w, k0 + kShWaves * kBN, kslot);

    // online softmax of this tile (as fa2_fwd_pp_kernel's softmax phase)
    if ((k0 + kBN > w.Lk) || (causal && (k0 + kBN - 1 > q0 + w.off))) {
      int lim = w.Lk - 1 - k0 - hi * 4;
      if (causal) lim = min(lim, qrow + w.off - k0 - hi * 4);
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
          const int c = sb * 32 + (i2 >> 2) * 8 + (i2 & 3);
          const uint32_t hide = static_cast<uint32_t>((lim - c) >> 31);
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
    u32x4 pf[kBN / 16];
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

    // V(t) has landed (K(t + 4), issued after it, may be in flight)
    if (more)
      pp_wait_vm<kI>();
    else
      pp_wait_vm<0>();
    // O^T += V^T P^T
#pragma unroll
    for (int c = 0; c < kBN / 16; ++c)
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
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (more) ld.template issue<true>(a, w, k0 + kShWaves * kBN, vslot);
  }

  // Merge the 4 waves' states.  Each wave's row max is whole after the
  // lane^32 exchange; its row sum is split over the lane halves.
  if (hi == 0) mrow[wave][l32] = m_run;
  pp_barrier();
  float mall = -INFINITY;
#pragma unroll
  for (int v = 0; v < kShWaves; ++v) mall = fmaxf(mall, mrow[v][l32]);
  // 2^(m_w - M); 0 for a wave that saw no key of this row (m_w = -inf)
  const float f = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - mall);
  const float lw = sum_xor32(l_run) * f;
  if (hi == 0) lrow[wave][l32] = lw;
  {
    // this wave's O rows into its own (no longer read) tile slots
    __attribute__((address_space(3))) float* ob =
        (__attribute__((address_space(3))) float*)lds_ptr(lds_addr_of(kslot));
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(__attribute__((address_space(3))) f32x4*)(ob + l32 * kOPitch + d * 32 + g * 8 + hi * 4) =
            (f32x4){o[d][g * 4 + 0] * f, o[d][g * 4 + 1] * f, o[d][g * 4 + 2] * f,
                    o[d][g * 4 + 3] * f};
  }
  pp_barrier();
  // 8 threads per row, D / 8 dims each: sum the 4 waves, normalise, store
  {
    constexpr int kPer = D / 8;
    const int r = tid >> 3, part = tid & 7;
    float acc[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) acc[e] = 0.f;
    float lsum = 0.f;
#pragma unroll
    for (int v = 0; v < kShWaves; ++v) {
      const __attribute__((address_space(3))) float* ob =
          (const __attribute__((address_space(3))) float*)lds_ptr(lds_addr_of(lds + v * 2 * kTile));
#pragma unroll
      for (int e = 0; e < kPer; e += 4) {
        const f32x4 x =
            *(const __attribute__((address_space(3))) f32x4*)(ob + r * kOPitch + part * kPer + e);
        acc[e] += x[0];
        acc[e + 1] += x[1];
        acc[e + 2] += x[2];
        acc[e + 3] += x[3];
      }
      lsum += lrow[v][r];
    }
    const float inv = 1.f / lsum;  // 0/0 -> NaN for a row with no key, as the reference
    if (q0 + r < w.Lq) {
      uint16_t* dst = static_cast<uint16_t*>(a.o) + w.o_base +
                      static_cast<int64_t>(q0 + r) * a.o_ss + part * kPer;
#pragma unroll
      for (int e = 0; e < kPer; e += 8)
        *reinterpret_cast<u32x4*>(dst + e) =
            (u32x4){pack2<BF>(acc[e] * inv, acc[e + 1] * inv),
                    pack2<BF>(acc[e + 2] * inv, acc[e + 3] * inv),
                    pack2<BF>(acc[e + 4] * inv, acc[e + 5] * inv),
                    pack2<BF>(acc[e + 6] * inv, acc[e + 7] * inv)};
    }
  }
}

}  // namespace fa2
