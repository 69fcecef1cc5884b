// fa2_device.h - gfx950 device code of the flash_attention_v2 forward pass.
//
// Algorithm (restated from harsh-vsingh/triton-kernels kernels/attention.py):
//   S = (Q K^T) * scale, masked (:596-598), online softmax with running max
//   and running sum (:600-611), acc = acc * alpha + P V (:635-636), split-KV
//   partials combined by a log-sum-exp merge (:659-746).
//
// CDNA4 mapping (independent of the reference's Triton tiling):
//   * workgroup = 4 wave64s, 128 query rows (32 per wave), KV tiles of 64 keys;
//   * the transposed problem is computed, S^T = K Q^T and O^T = V^T P^T, on
//     v_mfma_f32_32x32x16_{bf16,f16}: each lane then owns ONE query row
//     (lane & 31) and the row statistics need one cross-lane exchange
//     (lane ^ 32) instead of a 32-lane reduction;
//   * Q^T fragments stay in VGPRs for the whole KV sweep;
//   * K tiles are staged row-major in LDS, V tiles transposed ([dim][key],
//     keys permuted inside each 16-key chunk) so that the P^T fragment produced
//     by the S^T MFMA is consumed by the PV MFMA straight from registers;
//   * K/V tiles are double-buffered in LDS, the next tile's global loads are
//     in flight while the current tile is on the MFMA pipes;
//   * exp is v_exp_f32 (2^x) with scale*log2(e) folded into one FMA;
//   * causal: tiles past the diagonal are never loaded, masks are evaluated
//     only on diagonal / sequence-end tiles, and a wave skips a tile that is
//     fully masked for its 32 rows;
//   * dense causal launches the heaviest q-blocks first; ragged and paged
//     launches read a heaviest-first work list built on the device by
//     fa2_plan_kernel (no host synchronisation, unlike attention.py:847).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa2.h"

namespace fa2 {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 128;       // query rows per workgroup
constexpr int kWaveRows = 32;  // query rows per wave
constexpr int kBN = 64;        // keys per KV tile
constexpr int kCostBuckets = 4096;
constexpr int kPlanThreads = 1024;

// ---------------------------------------------------------------------------
// Kernel arguments (one POD passed by value).
// ---------------------------------------------------------------------------
struct KArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* q_indptr;
  const int32_t* kv_indptr;
  const int32_t* k_table;
  const int32_t* v_table;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t k_table_stride, v_table_stride;
  int32_t batch, hq, hkv, q_len, kv_len, page_size;
  int32_t nqb;          // dense: q-blocks per sequence; paged: same
  int32_t work_ub;      // ragged/paged: capacity of the work list
  int32_t mask;         // enum fa2_mask
  int32_t num_splits;   // >= 1
  float scale_log2;     // softmax_scale * log2(e)
  const int2* work;     // ragged/paged work list (b, q-block), heaviest first
  const int32_t* work_count;
  float* part_ml;       // split partials: (m, l) per row
  float* part_o;        // split partials: unnormalised O per row
};

// ---------------------------------------------------------------------------
// Element types.
// ---------------------------------------------------------------------------
template <int DT>
struct Elt;
template <>
struct Elt<FA2_DTYPE_F16> {
  static constexpr bool kBF = false;
  static constexpr int kBytes = 2;
};
template <>
struct Elt<FA2_DTYPE_BF16> {
  static constexpr bool kBF = true;
  static constexpr int kBytes = 2;
};
template <>
struct Elt<FA2_DTYPE_F32> {
  static constexpr bool kBF = false;  // fp32 operands are rounded to fp16
  static constexpr int kBytes = 4;
};

// 8 consecutive elements of one row as loaded from HBM (raw, unconverted).
template <int DT>
struct Raw8 {
  u32x4 w[Elt<DT>::kBytes / 2];
};

template <bool BF>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (BF) {
    bf16x2 v = __builtin_convertvector((f32x2){a, b}, bf16x2);
    return __builtin_bit_cast(uint32_t, v);
  } else {
    f16x2 v = __builtin_convertvector((f32x2){a, b}, f16x2);
    return __builtin_bit_cast(uint32_t, v);
  }
}

// Raw8 -> 8 packed 16-bit compute elements.
template <int DT>
__device__ __forceinline__ u32x4 to16(const Raw8<DT>& r) {
  if constexpr (DT == FA2_DTYPE_F32) {
    f32x4 a = __builtin_bit_cast(f32x4, r.w[0]);
    f32x4 b = __builtin_bit_cast(f32x4, r.w[1]);
    return (u32x4){pack2<false>(a[0], a[1]), pack2<false>(a[2], a[3]),
                   pack2<false>(b[0], b[1]), pack2<false>(b[2], b[3])};
  } else {
    return r.w[0];
  }
}

template <int DT>
__device__ __forceinline__ void load_raw8(Raw8<DT>& r, const void* base, int64_t off) {
  if constexpr (DT == FA2_DTYPE_F32) {
    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(base) + off);
    r.w[0] = p[0];
    r.w[1] = p[1];
  } else {
    r.w[0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + off);
  }
}

template <int DT>
__device__ __forceinline__ void zero_raw8(Raw8<DT>& r) {
#pragma unroll
  for (int i = 0; i < Elt<DT>::kBytes / 2; ++i) r.w[i] = (u32x4){0u, 0u, 0u, 0u};
}

template <bool BF>
__device__ __forceinline__ f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (BF) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32, 64); }

// ---------------------------------------------------------------------------
// Work decoding: workgroup id -> (sequence, head, q-block) and addressing.
// ---------------------------------------------------------------------------
struct Work {
  bool valid;
  int b, h, kvh, qblk;
  int Lq, Lk;
  int64_t q_base, o_base;  // element offset of row 0 of this (sequence, head)
  int64_t q_rs, o_rs;      // row strides
  int64_t k_base, v_base;  // dense/ragged: row 0 of this (sequence, kv head);
                           // paged: kv-head offset only
  int64_t k_rs, v_rs;
  int off;                 // causal diagonal offset: key j visible iff j <= i + off
};

template <int MODE>
__device__ __forceinline__ Work decode_work(const KArgs& a, int L) {
  Work w;
  w.valid = true;
  w.h = L % a.hq;
  const int item = L / a.hq;
  const int group = a.hq / a.hkv;
  w.kvh = w.h / group;  // == h * Hkv / Hq (attention.py:463)
  if constexpr (MODE == FA2_LAYOUT_DENSE) {
    const int rank = item / a.batch;
    w.b = item % a.batch;
    // heaviest q-blocks first under a causal mask
    w.qblk = (a.mask != FA2_MASK_NONE) ? (a.nqb - 1 - rank) : rank;
    w.Lq = a.q_len;
    w.Lk = a.kv_len;
    w.q_base = w.b * a.q_sb + w.h * a.q_sh;
    w.o_base = w.b * a.o_sb + w.h * a.o_sh;
    w.k_base = w.b * a.k_sb + w.kvh * a.k_sh;
    w.v_base = w.b * a.v_sb + w.kvh * a.v_sh;
  } else {
    if (item >= *a.work_count) {
      w.valid = false;
      return w;
    }
    const int2 it = a.work[item];
    w.b = it.x;
    w.qblk = it.y;
    if constexpr (MODE == FA2_LAYOUT_RAGGED) {
      const int qs = a.q_indptr[w.b];
      const int ks = a.kv_indptr[w.b];
      w.Lq = a.q_indptr[w.b + 1] - qs;
      w.Lk = a.kv_indptr[w.b + 1] - ks;
      w.q_base = qs * a.q_ss + w.h * a.q_sh;
      w.o_base = qs * a.o_ss + w.h * a.o_sh;
      w.k_base = ks * a.k_ss + w.kvh * a.k_sh;
      w.v_base = ks * a.v_ss + w.kvh * a.v_sh;
    } else {  // paged: dense q/o, lengths in kv_indptr
      w.Lq = a.q_len;
      w.Lk = a.kv_indptr[w.b];
      w.q_base = w.b * a.q_sb + w.h * a.q_sh;
      w.o_base = w.b * a.o_sb + w.h * a.o_sh;
      w.k_base = w.kvh * a.k_sh;
      w.v_base = w.kvh * a.v_sh;
    }
  }
  if (w.Lk < 0) w.Lk = 0;
  if (w.Lq < 0) w.Lq = 0;
  w.q_rs = a.q_ss;
  w.o_rs = a.o_ss;
  w.k_rs = a.k_ss;
  w.v_rs = a.v_ss;
  w.off = (a.mask == FA2_MASK_CAUSAL_BOTTOM_RIGHT) ? (w.Lk - w.Lq) : 0;
  return w;
}

// Number of keys a q-block [q0, q0+BM) can see (exclusive end), >= 0.
__device__ __forceinline__ int kv_end_for_block(int mask, int q0, int Lq, int Lk, int off) {
  if (mask == FA2_MASK_NONE) return Lk;
  int qe = min(q0 + kBM, Lq);
  int e = min(Lk, qe + off);
  return e > 0 ? e : 0;
}

// ---------------------------------------------------------------------------
// LDS layout. K: [2][BN][D + 8] row-major.  V: [2][D][BN + 8] transposed
// with each 16-key chunk stored in the order keys 0-3, 8-11, 4-7, 12-15.
// Row paddings of 16 bytes keep ds_read_b128 accesses conflict-free.
// ---------------------------------------------------------------------------
template <int D>
struct Lds {
  static constexpr int kKStride = D + 8;
  static constexpr int kVStride = kBN + 8;
  static constexpr int kKTile = kBN * kKStride;
  static constexpr int kVTile = D * kVStride;
  static constexpr int kElems = 2 * kKTile + 2 * kVTile;
  static constexpr int kBytes = kElems * 2;
};

// position of key kk (0..63) inside a transposed V row
__device__ __forceinline__ int vpos(int kk) {
  const int g = (kk >> 2) & 3;
  return (kk & ~15) | (((g & 1) << 3) | ((g >> 1) << 2)) | (kk & 3);
}

// Global -> register staging of one K/V tile, then register -> LDS.
template <int DT, int D, int MODE>
struct TileLoader {
  static constexpr int kTPR = D / 8;                  // threads per K row
  static constexpr int kRowsPerPass = kThreads / kTPR;
  static constexpr int kKPasses = kBN / kRowsPerPass;
  static constexpr int kKPT = kBN * D / (8 * kThreads);  // V keys per thread
  static_assert(kKPasses >= 1 && kKPT >= 1 && kKPT <= 4, "tile shape");

  Raw8<DT> kr[kKPasses];
  Raw8<DT> vr[kKPT];

  __device__ __forceinline__ static int64_t paged_row(const int32_t* table, int64_t tstride,
                                                      int b, int n, int page) {
    const int pg = table[b * tstride + n / page];
    return static_cast<int64_t>(pg) * page + (n % page);
  }

  __device__ __forceinline__ void issue(const KArgs& a, const Work& w, int k0, int tid) {
    // K: row-major rows, 8 elements per thread per pass.
    const int kcol = (tid % kTPR) * 8;
#pragma unroll
    for (int p = 0; p < kKPasses; ++p) {
      const int n = k0 + tid / kTPR + p * kRowsPerPass;
      if (n < w.Lk) {
        int64_t off;
        if constexpr (MODE == FA2_LAYOUT_PAGED)
          off = w.k_base + paged_row(a.k_table, a.k_table_stride, w.b, n, a.page_size) * w.k_rs;
        else
          off = w.k_base + static_cast<int64_t>(n) * w.k_rs;
        load_raw8<DT>(kr[p], a.k, off + kcol);
      } else {
        zero_raw8<DT>(kr[p]);
      }
    }
    // V: kKPT consecutive keys x 8 dims per thread.
    const int vcol = (tid % kTPR) * 8;
    const int vkey = (tid / kTPR) * kKPT;
#pragma unroll
    for (int j = 0; j < kKPT; ++j) {
      const int n = k0 + vkey + j;
      if (n < w.Lk) {
        int64_t off;
        if constexpr (MODE == FA2_LAYOUT_PAGED)
          off = w.v_base + paged_row(a.v_table, a.v_table_stride, w.b, n, a.page_size) * w.v_rs;
        else
          off = w.v_base + static_cast<int64_t>(n) * w.v_rs;
        load_raw8<DT>(vr[j], a.v, off + vcol);
      } else {
        zero_raw8<DT>(vr[j]);
      }
    }
  }

  __device__ __forceinline__ void commit(uint16_t* ks, uint16_t* vt, int tid) const {
    using L = Lds<D>;
    const int kcol = (tid % kTPR) * 8;
#pragma unroll
    for (int p = 0; p < kKPasses; ++p) {
      const int row = tid / kTPR + p * kRowsPerPass;
      *reinterpret_cast<u32x4*>(ks + row * L::kKStride + kcol) = to16<DT>(kr[p]);
    }
    const int vcol = (tid % kTPR) * 8;
    const int vkey = (tid / kTPR) * kKPT;
    u32x4 x[kKPT];
#pragma unroll
    for (int j = 0; j < kKPT; ++j) x[j] = to16<DT>(vr[j]);
    const int pos = vpos(vkey);  // kKPT <= 4 consecutive keys stay adjacent
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int word = d >> 1;
      const bool hi = d & 1;
      uint16_t* dst = vt + (vcol + d) * L::kVStride + pos;
      if constexpr (kKPT == 4) {
        uint32_t e0 = hi ? (x[0][word] >> 16) : (x[0][word] & 0xffffu);
        uint32_t e1 = hi ? (x[1][word] >> 16) : (x[1][word] & 0xffffu);
        uint32_t e2 = hi ? (x[2][word] >> 16) : (x[2][word] & 0xffffu);
        uint32_t e3 = hi ? (x[3][word] >> 16) : (x[3][word] & 0xffffu);
        *reinterpret_cast<u32x2*>(dst) = (u32x2){e0 | (e1 << 16), e2 | (e3 << 16)};
      } else if constexpr (kKPT == 2) {
        uint32_t e0 = hi ? (x[0][word] >> 16) : (x[0][word] & 0xffffu);
        uint32_t e1 = hi ? (x[1][word] >> 16) : (x[1][word] & 0xffffu);
        *reinterpret_cast<uint32_t*>(dst) = e0 | (e1 << 16);
      } else {
        uint32_t e0 = hi ? (x[0][word] >> 16) : (x[0][word] & 0xffffu);
        *dst = static_cast<uint16_t>(e0);
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Forward kernel.
// ---------------------------------------------------------------------------
template <int DT, int D, int MODE>
__global__ __launch_bounds__(kThreads, 2) void fa2_fwd_kernel(KArgs a) {
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int DC = D / 16;  // 16-wide head-dim chunks of Q^T (MFMA k-steps)
  constexpr int DB = D / 32;  // 32-row head-dim blocks of O^T
  constexpr int SB = kBN / 32;
  using L = Lds<D>;

  __shared__ __attribute__((aligned(16))) uint16_t lds[L::kElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  const Work w = decode_work<MODE>(a, blockIdx.x);
  if (!w.valid) return;
  const int q0 = w.qblk * kBM;
  const int split = blockIdx.y;
  const int S = a.num_splits;

  // KV tile range of this split.
  const int kv_end = kv_end_for_block(a.mask, q0, w.Lq, w.Lk, w.off);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const int t_begin = (ntiles * split) / S;
  const int t_end = (ntiles * (split + 1)) / S;

  // Q^T fragments: lane holds query row q0 + 32*wave + l32, dims c*16+8*hi..+7.
  const int qrow = q0 + wave * kWaveRows + l32;
  u32x4 qf[DC];
  {
    const bool ok = qrow < w.Lq;
    const int64_t base = w.q_base + static_cast<int64_t>(qrow) * w.q_rs + hi * 8;
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

  f32x16 o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = (f32x16){};
  float m_run = -INFINITY;  // running max, log2 domain (already scaled)
  float l_run = 0.f;        // running sum of this lane's keys

  uint16_t* ks_base = lds;
  uint16_t* vt_base = lds + 2 * L::kKTile;

  // first (wave-row) query index and the last one of this wave
  const int wq_first = q0 + wave * kWaveRows;
  const int wq_last = wq_first + kWaveRows - 1;
  const bool causal = a.mask != FA2_MASK_NONE;

  TileLoader<DT, D, MODE> ld;
  if (t_begin < t_end) {
    ld.issue(a, w, t_begin * kBN, tid);
    ld.commit(ks_base, vt_base, tid);
  }
  __syncthreads();

  for (int t = t_begin; t < t_end; ++t) {
    const int buf = (t - t_begin) & 1;
    const int k0 = t * kBN;
    const bool more = (t + 1) < t_end;
    if (more) ld.issue(a, w, k0 + kBN, tid);

    const uint16_t* ks = ks_base + buf * L::kKTile;
    const uint16_t* vt = vt_base + buf * L::kVTile;

    // wave-uniform: does this tile hold any visible key for this wave's rows?
    const bool wave_live = !causal || (k0 <= wq_last + w.off);
    if (wave_live) {
      // S^T = K Q^T for 64 keys x 32 queries.
      f32x16 s[SB];
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        s[sb] = (f32x16){};
        const uint16_t* krow = ks + (sb * 32 + l32) * L::kKStride + hi * 8;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          const u32x4 kf = *reinterpret_cast<const u32x4*>(krow + c * 16);
          s[sb] = mma32<BF>(kf, qf[c], s[sb]);
        }
      }
      // Mask only where needed: sequence end or the causal diagonal.
      const bool need_mask = (k0 + kBN > w.Lk) || (causal && (k0 + kBN - 1 > wq_first + w.off));
      if (need_mask) {
        const int qi = qrow;
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = k0 + sb * 32 + (i >> 2) * 8 + hi * 4 + (i & 3);
            const bool ok = (key < w.Lk) && (!causal || key <= qi + w.off);
            if (!ok) s[sb][i] = -INFINITY;
          }
        }
      }
      // Online softmax (row = this lane's query).
      float mx = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < SB; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sb][i]);
      mx = fmaxf(mx, xor32(mx));
      const float m_new = fmaxf(m_run, mx * a.scale_log2);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      m_run = m_new;
      float rs = 0.f;
      u32x4 pf[kBN / 16];
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          p[i] = fast_exp2(__builtin_fmaf(s[sb][i], a.scale_log2, -m_use));
          rs += p[i];
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          pf[sb * 2 + half] = (u32x4){pack2<BF>(p[half * 8 + 0], p[half * 8 + 1]),
                                      pack2<BF>(p[half * 8 + 2], p[half * 8 + 3]),
                                      pack2<BF>(p[half * 8 + 4], p[half * 8 + 5]),
                                      pack2<BF>(p[half * 8 + 6], p[half * 8 + 7])};
        }
      }
      l_run = l_run * alpha + rs;
#pragma unroll
      for (int d = 0; d < DB; ++d) o[d] *= alpha;
      // O^T += V^T P^T
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const uint16_t* vrow = vt + (d * 32 + l32) * L::kVStride + hi * 8;
#pragma unroll
        for (int c = 0; c < kBN / 16; ++c) {
          const u32x4 vf = *reinterpret_cast<const u32x4*>(vrow + c * 16);
          o[d] = mma32<BF>(vf, pf[c], o[d]);
        }
      }
    }

    if (more) ld.commit(ks_base + (buf ^ 1) * L::kKTile, vt_base + (buf ^ 1) * L::kVTile, tid);
    __syncthreads();
  }

  const float l_tot = l_run + xor32(l_run);
  if (S == 1) {
    if (qrow < w.Lq) {
      const float inv = 1.f / l_tot;  // 0/0 -> NaN for a row with no key, as the reference
      const int64_t base = w.o_base + static_cast<int64_t>(qrow) * w.o_rs + hi * 4;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t off = base + d * 32 + g * 8;
          const float x0 = o[d][g * 4 + 0] * inv, x1 = o[d][g * 4 + 1] * inv;
          const float x2 = o[d][g * 4 + 2] * inv, x3 = o[d][g * 4 + 3] * inv;
          if constexpr (DT == FA2_DTYPE_F32) {
            *reinterpret_cast<f32x4*>(static_cast<float*>(a.o) + off) = (f32x4){x0, x1, x2, x3};
          } else {
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.o) + off) =
                (u32x2){pack2<BF>(x0, x1), pack2<BF>(x2, x3)};
          }
        }
      }
    }
  } else {
    // Split partials: slot (split, workgroup), row r of the q-block.
    const int64_t slot = static_cast<int64_t>(split) * gridDim.x + blockIdx.x;
    const int r = wave * kWaveRows + l32;
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

// ---------------------------------------------------------------------------
// Split-KV combine: O = sum_s 2^(m_s-g) O_s / sum_s 2^(m_s-g) l_s, g = max m_s
// (attention.py:710-724 restated in the log2 domain).
// ---------------------------------------------------------------------------
template <int DT, int D, int MODE>
__global__ __launch_bounds__(kThreads) void fa2_combine_kernel(KArgs a) {
  const Work w = decode_work<MODE>(a, blockIdx.x);
  if (!w.valid) return;
  const int q0 = w.qblk * kBM;
  constexpr int kTPR = D / 4;  // threads per row, 4 floats each
  constexpr int kRowsPerPass = kThreads / kTPR;
  const int S = a.num_splits;
  const int G = gridDim.x;
  const int col = (threadIdx.x % kTPR) * 4;
  for (int r = threadIdx.x / kTPR; r < kBM; r += kRowsPerPass) {
    const int qrow = q0 + r;
    if (qrow >= w.Lq) break;
    float g = -INFINITY;
    for (int s = 0; s < S; ++s) {
      const int64_t slot = static_cast<int64_t>(s) * G + blockIdx.x;
      g = fmaxf(g, a.part_ml[(slot * kBM + r) * 2]);
    }
    const float g_use = (g == -INFINITY) ? 0.f : g;
    float lsum = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < S; ++s) {
      const int64_t slot = static_cast<int64_t>(s) * G + blockIdx.x;
      const float m = a.part_ml[(slot * kBM + r) * 2];
      const float l = a.part_ml[(slot * kBM + r) * 2 + 1];
      const float wgt = fast_exp2(m - g_use);
      lsum += wgt * l;
      const f32x4 x = *reinterpret_cast<const f32x4*>(a.part_o + (slot * kBM + r) * D + col);
      acc += wgt * x;
    }
    const float inv = 1.f / lsum;
    const int64_t off = w.o_base + static_cast<int64_t>(qrow) * w.o_rs + col;
    if constexpr (DT == FA2_DTYPE_F32) {
      *reinterpret_cast<f32x4*>(static_cast<float*>(a.o) + off) = acc * inv;
    } else {
      constexpr bool BF = Elt<DT>::kBF;
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.o) + off) =
          (u32x2){pack2<BF>(acc[0] * inv, acc[1] * inv), pack2<BF>(acc[2] * inv, acc[3] * inv)};
    }
  }
}

// ---------------------------------------------------------------------------
// Plan kernel (ragged / paged): builds the (sequence, q-block) work list in
// descending order of KV tiles to process (longest-processing-time first),
// by a counting sort over tile counts.  One workgroup; no host sync.
// ---------------------------------------------------------------------------
template <int MODE>
__device__ __forceinline__ void seq_lens(const KArgs& a, int b, int& Lq, int& Lk) {
  if constexpr (MODE == FA2_LAYOUT_RAGGED) {
    Lq = a.q_indptr[b + 1] - a.q_indptr[b];
    Lk = a.kv_indptr[b + 1] - a.kv_indptr[b];
  } else {
    Lq = a.q_len;
    Lk = a.kv_indptr[b];
  }
  if (Lq < 0) Lq = 0;
  if (Lk < 0) Lk = 0;
}

__device__ __forceinline__ int block_cost(int mask, int j, int Lq, int Lk) {
  const int off = (mask == FA2_MASK_CAUSAL_BOTTOM_RIGHT) ? (Lk - Lq) : 0;
  const int e = kv_end_for_block(mask, j * kBM, Lq, Lk, off);
  const int tiles = (e + kBN - 1) / kBN;
  return tiles < kCostBuckets - 1 ? tiles : kCostBuckets - 1;
}

template <int MODE>
__global__ __launch_bounds__(kPlanThreads) void fa2_plan_kernel(KArgs a, int2* work,
                                                                int32_t* work_count) {
  __shared__ int hist[kCostBuckets];
  __shared__ int scan[kPlanThreads];
  const int tid = threadIdx.x;
  for (int i = tid; i < kCostBuckets; i += kPlanThreads) hist[i] = 0;
  __syncthreads();
  for (int b = tid; b < a.batch; b += kPlanThreads) {
    int Lq, Lk;
    seq_lens<MODE>(a, b, Lq, Lk);
    const int nq = (Lq + kBM - 1) / kBM;
    for (int j = 0; j < nq; ++j) atomicAdd(&hist[block_cost(a.mask, j, Lq, Lk)], 1);
  }
  __syncthreads();
  // Exclusive scan in descending cost order: bucket c starts after all
  // buckets c' > c.  Thread t owns buckets [(P-1-t)*4, +4) from the top.
  constexpr int kPer = kCostBuckets / kPlanThreads;
  int local[kPer];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    local[i] = hist[kCostBuckets - 1 - (tid * kPer + i)];
    sum += local[i];
  }
  scan[tid] = sum;
  __syncthreads();
  for (int step = 1; step < kPlanThreads; step <<= 1) {
    const int v = (tid >= step) ? scan[tid - step] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  int run = scan[tid] - sum;
  const int total = scan[kPlanThreads - 1];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    hist[kCostBuckets - 1 - (tid * kPer + i)] = run;  // becomes the cursor
    run += local[i];
  }
  __syncthreads();
  for (int b = tid; b < a.batch; b += kPlanThreads) {
    int Lq, Lk;
    seq_lens<MODE>(a, b, Lq, Lk);
    const int nq = (Lq + kBM - 1) / kBM;
    for (int j = 0; j < nq; ++j) {
      const int pos = atomicAdd(&hist[block_cost(a.mask, j, Lq, Lk)], 1);
      if (pos < a.work_ub) work[pos] = make_int2(b, j);
    }
  }
  if (tid == 0) *work_count = total < a.work_ub ? total : a.work_ub;
}

}  // namespace fa2
