// fa2_kernel_decode_f32.h - fp32 decode_attention / speculative_decode_attention
// for units of few rows (Hq/Hkv * M <= kDecF32MaxRows): dot products on the
// VALU, no MFMA.
//
// The references compute fp32 decode in fp32 (decode.py:84, 92-160;
// speculative_decode.py:91-175).  A unit's rows are the query heads of one
// kv head times the drafts (packed-head mode, KArgs::pack_m), here at most 8
// (d1: 1, d2: 4, s1: 8), far fewer than a 32-row MFMA block.  The work per
// key is R * D FMAs for S and as many for P.V against 8 * D bytes of K and V,
// so these calls are HBM-bound with a VALU kernel as well, and every lane
// carries useful rows:
//   * workgroup = 4 waves; a lane holds CH head dims (CH * R <= 64 floats of
//     q, as many of O) of one key slot: the NC = D / CH lanes of a slot split
//     one K/V row, so a wave instruction reads KPW whole rows (KPW = 64 / NC);
//   * per step each slot takes the next key of its stream: partial dots over
//     CH dims, a butterfly over the slot's NC lanes, then an exact online
//     softmax per row (running max, rescale, P) and O += P V on the lane's
//     dims.  The loads of the next step are in flight during this one;
//   * at the end the slots of a wave merge by a butterfly over the slot
//     lanes and the 4 waves through LDS, in a fixed order (deterministic),
//     into (m, l, O) per row: the output, or split partials that the last
//     split merges (KArgs::merge_ctr, as the 16-bit decode kernel does).
#pragma once

#include "fa2_kernel_lds.h"

namespace fa2 {

constexpr int kDecF32MaxRows = 8;
constexpr int kDecF32Waves = 4;
constexpr int kDecF32Threads = 64 * kDecF32Waves;

template <int D, int R>
struct DecF32Geo {
  static constexpr int CH = (64 / R) < 16 ? 64 / R : 16;  // head dims per lane
  static constexpr int NC = D / CH;                       // lanes per key slot
  static constexpr int KPW = 64 / NC;                     // key slots per wave
  static constexpr int NV = CH / 4;                       // float4 per lane and row
  static_assert(NC >= 1 && NC <= 64 && KPW * NC == 64, "geometry");
};

// R: the unit's row capacity (4 or 8); rows past the unit's own are zero
template <int D, int MODE, int R>
__global__ __launch_bounds__(kDecF32Threads, 2) void fa2_decode_f32_kernel(KArgs a) {
  using G = DecF32Geo<D, R>;
  constexpr int CH = G::CH, NC = G::NC, KPW = G::KPW, NV = G::NV;
  constexpr int KPS = KPW * kDecF32Waves;  // keys per workgroup step

  __shared__ float mrg_o[kDecF32Waves][R][D];   // per wave: merged O of its slots
  __shared__ float mrg_ml[kDecF32Waves][R][2];  // and (m, l)
  __shared__ int merge_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slot = lane / NC;  // key slot of the wave
  const int c = lane % NC;     // dim chunk: dims [c * CH, c * CH + CH)

  const Work w = decode_work<MODE>(a, blockIdx.x);
  if (!w.valid) return;
  const int split = blockIdx.y;
  const int S = launch_splits(a);
  if (split >= S) return;
  const int rows = min(w.Lq - w.qblk * a.block_rows, R);
  const int row0 = w.qblk * a.block_rows;
  // keys of this split, in kBN-key tiles as the other kernels split them
  const int ntiles = (w.Lk + kBN - 1) / kBN;
  const int k_begin = ((ntiles * split) / S) * kBN;
  const int k_end = min(((ntiles * (split + 1)) / S) * kBN, w.Lk);
  const bool causal = a.mask != FA2_MASK_NONE;

  // q chunk of every row, and each row's last visible key (bottom-right per
  // draft position under the causal mask)
  f32x4 q[R][NV];
  int last[R];
  const float* qp = static_cast<const float*>(a.q) + w.q_base + c * CH;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool ok = r < rows;
#pragma unroll
    for (int v = 0; v < NV; ++v)
      q[r][v] = ok ? *reinterpret_cast<const f32x4*>(qp + static_cast<int64_t>(row0 + r) * a.q_ss +
                                                     4 * v)
                   : (f32x4){0.f, 0.f, 0.f, 0.f};
    last[r] = causal ? min(w.Lk - 1, w.off + diag_row(a, row0 + r)) : w.Lk - 1;
  }

  // element offset of key n's row (from the layout's K/V base), a clamped key
  // when n is past the range (its scores are masked)
  const float* kbase = static_cast<const float*>(a.k) + w.k_base + c * CH;
  const float* vbase = static_cast<const float*>(a.v) + w.v_base + c * CH;
  auto row_of = [&](int n, int64_t ss) -> int64_t {
    n = min(n, max(k_end - 1, 0));
    if constexpr (MODE == FA2_LAYOUT_PAGED) {
      int pidx, poff;
      if (a.page_shift >= 0) {
        pidx = n >> a.page_shift;
        poff = n & (a.page_size - 1);
      } else {
        pidx = n / a.page_size;
        poff = n - pidx * a.page_size;
      }
      const int page = a.k_table[w.b * a.k_table_stride + pidx];
      return (static_cast<int64_t>(page) * a.page_size + poff) * ss;
    } else {
      return static_cast<int64_t>(n) * ss;
    }
  };
  auto row_of_v = [&](int n) -> int64_t {
    if constexpr (MODE == FA2_LAYOUT_PAGED) {
      n = min(n, max(k_end - 1, 0));
      int pidx, poff;
      if (a.page_shift >= 0) {
        pidx = n >> a.page_shift;
        poff = n & (a.page_size - 1);
      } else {
        pidx = n / a.page_size;
        poff = n - pidx * a.page_size;
      }
      const int page = a.v_table[w.b * a.v_table_stride + pidx];
      return (static_cast<int64_t>(page) * a.page_size + poff) * a.v_ss;
    } else {
      return row_of(n, a.v_ss);
    }
  };

  float m[R], l[R];
  f32x4 o[R][NV];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) o[r][v] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }

  f32x4 kx[NV], vx[NV];
  auto load = [&](int k0, f32x4 (&kd)[NV], f32x4 (&vd)[NV]) {
    const int n = k0 + wave * KPW + slot;
    const float* kp = kbase + row_of(n, a.k_ss);
    const float* vp = vbase + row_of_v(n);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      kd[v] = *reinterpret_cast<const f32x4*>(kp + 4 * v);
      vd[v] = *reinterpret_cast<const f32x4*>(vp + 4 * v);
    }
  };
  if (k_begin < k_end) load(k_begin, kx, vx);
  for (int k0 = k_begin; k0 < k_end; k0 += KPS) {
    f32x4 kn[NV], vn[NV];
    if (k0 + KPS < k_end) load(k0 + KPS, kn, vn);
    const int n = k0 + wave * KPW + slot;
    float s[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_fmaf(q[r][v][j], kx[v][j], acc);
      s[r] = acc;
    }
    // the full dot products: a butterfly over the slot's NC lanes
#pragma unroll
    for (int off = 1; off < NC; off <<= 1)
#pragma unroll
      for (int r = 0; r < R; ++r) s[r] += __shfl_xor(s[r], off);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float x = (n < k_end && n <= last[r]) ? s[r] * a.scale_log2 : -INFINITY;
      const float mn = fmaxf(m[r], x);
      const float mu = (mn == -INFINITY) ? 0.f : mn;
      const float alpha = fast_exp2(m[r] - mu);
      const float p = fast_exp2(x - mu);
      l[r] = l[r] * alpha + p;
#pragma unroll
      for (int v = 0; v < NV; ++v) o[r][v] = o[r][v] * alpha + p * vx[v];
      m[r] = mn;
    }
    if (k0 + KPS < k_end) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        kx[v] = kn[v];
        vx[v] = vn[v];
      }
    }
  }

  // merge two (m, l, O) states: this lane's and another's
  auto merge = [&](int r, float m2, float l2, const f32x4 (&o2)[NV]) {
    const float mn = fmaxf(m[r], m2);
    const float mu = (mn == -INFINITY) ? 0.f : mn;
    const float a1 = fast_exp2(m[r] - mu), a2 = fast_exp2(m2 - mu);
    l[r] = l[r] * a1 + l2 * a2;
#pragma unroll
    for (int v = 0; v < NV; ++v) o[r][v] = o[r][v] * a1 + o2[v] * a2;
    m[r] = mn;
  };
  // the wave's slots, by a butterfly over the slot bits of the lane
#pragma unroll
  for (int off = NC; off < 64; off <<= 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f32x4 o2[NV];
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int j = 0; j < 4; ++j) o2[v][j] = __shfl_xor(o[r][v][j], off);
      const float m2 = __shfl_xor(m[r], off), l2 = __shfl_xor(l[r], off);
      merge(r, m2, l2, o2);
    }
  }
  // the waves, through LDS, in wave order
  if (slot == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int v = 0; v < NV; ++v)
        *reinterpret_cast<f32x4*>(&mrg_o[wave][r][c * CH + 4 * v]) = o[r][v];
      if (c == 0) {
        mrg_ml[wave][r][0] = m[r];
        mrg_ml[wave][r][1] = l[r];
      }
    }
  }
  __syncthreads();
  const bool writer = wave == 0 && slot == 0;
  if (writer) {
#pragma unroll
    for (int ww = 1; ww < kDecF32Waves; ++ww)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        f32x4 o2[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v)
          o2[v] = *reinterpret_cast<const f32x4*>(&mrg_o[ww][r][c * CH + 4 * v]);
        merge(r, mrg_ml[ww][r][0], mrg_ml[ww][r][1], o2);
      }
  }

  if (S == 1) {
    if (!writer) return;
    float* op = static_cast<float*>(a.o) + w.o_base + c * CH;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= rows) continue;
      const float inv = 1.f / l[r];  // 0/0 -> NaN for a row with no key, as the reference
#pragma unroll
      for (int v = 0; v < NV; ++v)
        *reinterpret_cast<f32x4*>(op + static_cast<int64_t>(row0 + r) * a.o_ss + 4 * v) =
            o[r][v] * inv;
    }
    return;
  }
  // split partials (m, l, unnormalised O) of the unit's rows
  if (writer) {
    const int64_t slot_id = static_cast<int64_t>(split) * a.part_slots + blockIdx.x;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= rows || r >= a.part_rows) continue;
      float* ml = a.part_ml + (slot_id * a.part_rows + r) * 2;
      float* po = a.part_o + (slot_id * a.part_rows + r) * D + c * CH;
      if (a.merge_ctr) {
        if (c == 0) {
          st_dev2(ml, m[r], l[r]);
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) st_dev4(po + 4 * v, o[r][v]);
      } else {
        if (c == 0) {
          ml[0] = m[r];
          ml[1] = l[r];
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) *reinterpret_cast<f32x4*>(po + 4 * v) = o[r][v];
      }
    }
  }
  if (!a.merge_ctr) return;  // the combine kernel merges
  // the split that completes the unit's count merges its partials
  merge_publish();
  __syncthreads();
  if (!merge_count(a, blockIdx.x, S, &merge_flag)) return;
  merge_rows<FA2_DTYPE_F32, D, kDecF32Threads, R>(a, blockIdx.x, S, min(a.part_rows, rows),
                                                  w.o_base, row0);
}

}  // namespace fa2
