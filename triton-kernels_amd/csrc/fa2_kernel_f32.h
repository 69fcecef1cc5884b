// fa2_kernel_f32.h - forward kernel with fp32 arithmetic: fp32 operands and
// fp32 softmax weights on v_mfma_f32_32x32x2_f32.
//
// Serves the entry points whose reference computes fp32 tensors in fp32:
//   flash_attention_v1 (kernels/attention.py:177, 196-197, 225-240: q, k, v
//     cast to fp32, P = exp(qk - max) in fp32, acc += P V);
//   decode_attention (kernels/decode.py:84, 92-160) and
//   speculative_decode_attention (kernels/speculative_decode.py:91-175):
//     q, k, v in fp32, weights in fp32 (packed-head mode, KArgs::pack_m).
// flash_attention_v2 rounds fp32 operands to fp16 (attention.py:547-633): it
// runs the 16-bit kernels on fp16 copies, or the register-staged kernel of
// fa2_device.h.
//
// Layout (one workgroup = 4 waves, 128 query rows, 32 per wave; KV tiles of
// 64 keys, one K and one V tile in LDS):
//   * K and V rows go HBM -> LDS with direct-to-LDS buffer loads
//     (DirectLoader with fp32 rows), chunks XOR-swizzled (SwzGeo32);
//   * S^T = K Q^T: the 2-wide k-steps of the MFMA take head dims
//     (8g + j, 8g + 4 + j) for lane halves 0/1, so one 16-byte LDS read of a
//     K row feeds four MFMAs, and Q stays in registers as float4 chunks;
//   * O^T = V^T P^T: k-step v of a 32-key block takes keys
//     8(v/4) + v%4 and + 4, exactly the keys of accumulator register v of
//     the S^T block, so P goes from the softmax into the MFMA unchanged; the
//     V^T operand is one fp32 per lane, read from V's row-major tile (no
//     transpose anywhere);
//   * K(t+1) streams in while the softmax and PV of tile t run, V(t+1)
//     while the S of tile t+1 runs (two barriers per tile).
#pragma once

#include "fa2_kernel_lds.h"

namespace fa2 {

__device__ __forceinline__ f32x16 mma32_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) f32x4 lds_f32x4_t;
typedef __attribute__((address_space(3))) float lds_float_t;

template <int DT, int D, int MODE, bool BUF>
__global__ __launch_bounds__(kThreads, D > 128 ? 1 : 2) void fa2_fwd_f32_kernel(KArgs a) {
  static_assert(DT == FA2_DTYPE_F32, "fp32 tensors only");
  constexpr int DG = D / 8;   // 8-dim groups of Q^T: 4 MFMA k-steps each
  constexpr int DB = D / 32;  // 32-dim blocks of O^T
  constexpr int SB = kBN / 32;
  using G = SwzGeo32<D>;
  using LD = DirectLoader<D, MODE, BUF, DT>;

  __shared__ __attribute__((aligned(1024))) char lds[2 * G::kTileBytes];
  char* const kbuf = lds;
  char* const vbuf = lds + G::kTileBytes;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  const Work w = decode_work<MODE>(a, blockIdx.x);
  if (!w.valid) return;
  const int q0 = w.qblk * kBM;
  const int split = blockIdx.y;
  const int S = launch_splits(a);
  if (split >= S) return;
  const int kv_end = kv_end_for_unit(a, q0, w.Lq, w.Lk, w.off);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const int t_begin = (ntiles * split) / S;
  const int T = (ntiles * (split + 1)) / S - t_begin;

  // Q^T: lane (l32, hi) holds dims 8g + 4hi + j of row qrow (zeros past dv)
  const int qrow = q0 + wave * kWaveRows + l32;
  f32x4 qf[DG];
  {
    const bool ok = qrow < w.Lq;
    const float* qp =
        static_cast<const float*>(a.q) + w.q_base + static_cast<int64_t>(qrow) * a.q_ss + hi * 4;
#pragma unroll
    for (int g = 0; g < DG; ++g)
      qf[g] = (ok && 8 * g + 4 * hi < a.dv) ? *reinterpret_cast<const f32x4*>(qp + 8 * g)
                                            : (f32x4){0.f, 0.f, 0.f, 0.f};
  }

  f32x16 o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = (f32x16){};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const int wq_first = q0 + wave * kWaveRows;
  const int wq_diag = a.pack_m > 0 ? 0 : wq_first;
  const int qdiag = diag_row(a, qrow);
  const bool causal = a.mask != FA2_MASK_NONE;
  // a wave whose rows all lie past the unit's end only loads and syncs
  const bool active = wq_first < w.Lq;

  const LD ld(a, tid);
  const lds_char_t* kl = to_lds(kbuf);
  const lds_char_t* vl = to_lds(vbuf);
  // K: row sb*32 + l32, chunk (2g + hi) ^ k(row); the swizzle of rows
  // l32 and l32 + 32 agree (it depends on row & 15)
  const uint32_t krow = l32 * G::kRowBytes;
  const int ksw = G::k(l32);

  if (T > 0) {
    ld.template issue<false>(a, w, t_begin * kBN, kbuf);
    ld.template issue<true>(a, w, t_begin * kBN, vbuf);
    lds_fill_barrier();
    for (int i = 0; i < T; ++i) {
      const int k0 = (t_begin + i) * kBN;
      f32x16 s[SB];
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) s[sb] = (f32x16){};
      if (active) {
#pragma unroll
        for (int g = 0; g < DG; ++g) {
          f32x4 kc[SB];
#pragma unroll
          for (int sb = 0; sb < SB; ++sb)
            kc[sb] = *(const lds_f32x4_t*)(kl + sb * 32 * G::kRowBytes + krow +
                                           (((2 * g + hi) ^ ksw) * 16));
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int sb = 0; sb < SB; ++sb) s[sb] = mma32_f32(kc[sb][j], qf[g][j], s[sb]);
        }
      }
      // every wave is done with K(i); V(i) has landed
      lds_fill_barrier();
      if (i + 1 < T) ld.template issue<false>(a, w, k0 + kBN, kbuf);
      if (active) {
        if ((k0 + kBN > w.Lk) || (causal && (k0 + kBN - 1 > wq_diag + w.off))) {
          // key = k0 + 32sb + 8(i2/4) + 4hi + i2%4: visible iff its offset
          // from k0 + 4hi is <= lim
          int lim = w.Lk - 1 - k0 - hi * 4;
          if (causal) lim = min(lim, qdiag + w.off - k0 - hi * 4);
#pragma unroll
          for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int i2 = 0; i2 < 16; ++i2) {
              const int c = sb * 32 + (i2 >> 2) * 8 + (i2 & 3);
              if (c > lim) s[sb][i2] = -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
          for (int i2 = 0; i2 < 16; ++i2) mx = fmaxf(mx, s[sb][i2]);
        mx = max_xor32(mx);
        const float mt = mx * a.scale_log2;
        const bool need = mt > m_run + kRescaleThreshold;
        const float alpha = fast_exp2(need ? (m_run - mt) : 0.0f);
        m_run = need ? mt : m_run;
        const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
        float rs = 0.f;
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
          for (int i2 = 0; i2 < 16; ++i2) {
            s[sb][i2] = fast_exp2(__builtin_fmaf(s[sb][i2], a.scale_log2, -m_use));
            rs += s[sb][i2];
          }
        l_run = l_run * alpha + rs;
        if (__any(need)) {
#pragma unroll
          for (int d = 0; d < DB; ++d) o[d] *= alpha;
        }
        // O^T += V^T P^T: k-step (sb, v) takes key 32sb + 8(v/4) + 4hi + v%4
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = sb * 32 + (v >> 2) * 8 + hi * 4 + (v & 3);
            const lds_char_t* vrow = vl + key * G::kRowBytes + (l32 & 3) * 4;
            const int vsw = G::v(key);
#pragma unroll
            for (int d = 0; d < DB; ++d) {
              const int chunk = ((d * 32 + l32) >> 2) ^ vsw;
              const float vf = *(const lds_float_t*)(vrow + chunk * 16);
              o[d] = mma32_f32(vf, s[sb][v], o[d]);
            }
          }
      }
      // every wave is done with V(i); K(i+1) has landed
      lds_fill_barrier();
      if (i + 1 < T) ld.template issue<true>(a, w, k0 + kBN, vbuf);
    }
  }

  const float l_tot = sum_xor32(l_run);
  if (S == 1) {
    if (qrow < w.Lq) {
      const float inv = 1.f / l_tot;  // 0/0 -> NaN for a row with no key, as the reference
      float* op = static_cast<float*>(a.o) + w.o_base + static_cast<int64_t>(qrow) * a.o_ss +
                  hi * 4;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (d * 32 + g * 8 + hi * 4 >= a.dv) continue;  // padding dims (head_dim 16, 32)
          *reinterpret_cast<f32x4*>(op + d * 32 + g * 8) =
              (f32x4){o[d][g * 4 + 0] * inv, o[d][g * 4 + 1] * inv, o[d][g * 4 + 2] * inv,
                      o[d][g * 4 + 3] * inv};
        }
    }
  } else {
    // split partials: slot (split, workgroup), row r of the q-block
    const int64_t slot = static_cast<int64_t>(split) * a.part_slots + blockIdx.x;
    const int r = wave * kWaveRows + l32;
    if (qrow < w.Lq && r < a.part_rows) {
      if (hi == 0) {
        float* ml = a.part_ml + (slot * a.part_rows + r) * 2;
        ml[0] = m_run;
        ml[1] = l_tot;
      }
      float* po = a.part_o + (slot * a.part_rows + r) * D + hi * 4;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(po + d * 32 + g * 8) =
              (f32x4){o[d][g * 4 + 0], o[d][g * 4 + 1], o[d][g * 4 + 2], o[d][g * 4 + 3]};
    }
  }
}

}  // namespace fa2
