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
//   * software pipeline: K runs one tile ahead of V, so the S MFMAs of tile
//     t+1 are issued in the same basic block as the softmax VALU work of tile
//     t; the global loads of K(t+2) and V(t+1) are in flight meanwhile and
//     land in the other half of the double-buffered LDS;
//   * K/V rows are read with buffer loads whose hardware range check returns
//     zeros past the sequence end (no per-row branches); the descriptor is
//     rebased per tile on the scalar unit;
//   * exp is v_exp_f32 (2^x) with scale*log2(e) folded into one FMA; the
//     O rescale is skipped unless a row max grew by more than 2^8 (the
//     stale max is shared by O and the row sum, so the result is exact);
//   * causal: tiles past the diagonal are never loaded, masks are evaluated
//     only on diagonal / sequence-end tiles;
//   * dense causal launches the heaviest q-blocks first; ragged and paged
//     launches read a work list built on the device by fa2_plan_kernel (no
//     host synchronisation, unlike attention.py:847): heaviest first, or
//     sequence-major when the two-head kernel claims its units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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
constexpr int kPlanFastBatch = 256;  // decode plans up to this batch rank items directly
constexpr float kRescaleThreshold = 8.0f;  // log2 units: P <= 2^8 between rescales
// LDS operand reads are issued this many MFMAs ahead of their MFMA
#ifndef FA2_READ_AHEAD
#define FA2_READ_AHEAD 4
#endif
constexpr int kReadAhead = FA2_READ_AHEAD;
// buffer descriptor word 3 for gfx9-family raw (stride 0) buffers, 32-bit data format
constexpr int kBufferFlags = 0x00020000;

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
  int32_t page_shift;   // log2(page_size) if a power of two, else -1
  int32_t nqb;          // dense/paged: q-blocks per sequence
  int32_t work_ub;      // ragged/paged: capacity of the work list
  int32_t npairs;       // work_ub * hkv: (item, kv head) pairs the grid covers
  int32_t mask;         // enum fa2_mask
  int32_t num_splits;   // >= 1
  int32_t part_slots;   // split partials: slots per split (one per (item, head) unit)
  int32_t units;        // two-head kernel: units its persistent grid walks
  float scale_log2;     // softmax_scale * log2(e)
  uint32_t pool_bytes_k;  // paged + buffer path: bytes of the k cache from the kv-head 0 row 0
  uint32_t pool_bytes_v;
  const int2* work;     // ragged/paged work list (b, q-block) from the plan kernel; null: no plan
  const int32_t* work_count;
  float* part_ml;       // split partials: (m, l) per row
  float* part_o;        // split partials: unnormalised O per row
  int32_t part_rows;    // split partials: rows per slot (kBM; the row count in packed mode)
  // Packed-head (decode) mode when > 0: q/o are [B, Hq, pack_m, D] for every
  // K/V layout, and the Hq/Hkv query heads of one kv head form the rows of a
  // single unit, row r = (head in group) * pack_m + draft position; q_len is
  // then the unit's row count Hq/Hkv * pack_m.  Causal is bottom-right per
  // draft position: row r sees key j iff j <= Lk - pack_m + r % pack_m.
  int32_t pack_m;
  int32_t block_rows;   // unit rows per q-block of the launched kernel (kBM; decode kernel 64)
  // Head dims the tensors hold (<= the kernel's D).  The register-staged
  // kernel serves head_dim 16 and 32 with its D = 64 tiles: dims >= dv are
  // read as zeros (they add nothing to Q.K^T and give zero output columns)
  // and are never stored.
  int32_t dv;
  int32_t spin_cap;  // polls after which a decode-kernel ring wait gives up
  // Two-head kernel on MHA (Hq == Hkv, one split): a unit is a pair
  // of q-blocks (2k, 2k + 1) of one head, one per wave group, both over the
  // KV tiles of block 2k + 1 (the extra tiles are fully masked for block 2k
  // under a causal mask and add exact zeros); nqb then counts pairs.
  int32_t qpair;
  // Two-head kernel with a plan and one split: kXcds unit counters, zeroed
  // by the plan kernel.  Workgroup g takes unit g first and then claims the
  // next units of its group (g mod kXcds) from counter g mod kXcds; the plan
  // lists each sequence's q-blocks together (sequence-major).  null: the
  // static round walk over a heaviest-first list.
  int32_t* claim;
  // Ragged/paged launches with automatic splits: the split count the plan
  // kernel derives from the longest KV sweep (<= num_splits, the host's
  // bound from the total KV rows), which the forward and combine kernels
  // use instead of num_splits.  null: num_splits.
  int32_t* split_count;
  // fp32 tensors on the 16-bit kernels (q/k/v are fp16 copies): the forward
  // kernel writes split partials even with one split, and the combine
  // kernel writes the fp32 output from them.
  int32_t part_out;
  // Split merge inside the forward kernel (no combine launch): one 64-bit
  // word per unit (part slot), (tag << kMergeCountBits) | count of the
  // splits that have written their partials.  A word whose tag differs
  // from merge_tag counts as zero, so the words need no clearing between
  // calls; the split that completes the count merges the unit's partials
  // and leaves (tag, 0), so a replay of the same launch (same tag) starts
  // from zero as well.  null: partials go to the combine kernel.
  uint64_t* merge_ctr;
  uint64_t merge_tag;  // nonzero, < 2^kMergeTagBits - 1, distinct per call
  // Ragged launch without a plan kernel, all of whose workgroups are
  // resident at once: each workgroup derives the item list (InlinePlan) and,
  // with automatic splits (auto_splits), the split count from the sequence
  // lengths itself.
  int32_t inline_plan;
  int32_t auto_splits;
};

constexpr int kMergeCountBits = 24;
constexpr int kMergeTagBits = 64 - kMergeCountBits;

// Fewest KV tiles a split keeps (the automatic split heuristic).
constexpr int kMinSplitTiles = 16;

// The launch's split count: blockIdx.y >= it has no work.
__device__ __forceinline__ int launch_splits(const KArgs& a) {
  return a.split_count ? __builtin_amdgcn_readfirstlane(*a.split_count) : a.num_splits;
}

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
__device__ __forceinline__ void buf_raw8(Raw8<DT>& r, __amdgpu_buffer_rsrc_t rs, uint32_t voff) {
  r.w[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, 0));
  if constexpr (DT == FA2_DTYPE_F32)
    r.w[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16, 0, 0));
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

// acc + x.lo + x.hi for a packed pair of 16-bit values (v_dot2 with (1, 1))
template <bool BF>
__device__ __forceinline__ float dot2_ones(uint32_t x, float acc) {
  if constexpr (BF) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x),
                                           (bf16x2){(__bf16)1.0f, (__bf16)1.0f}, acc, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x),
                                  (f16x2){(_Float16)1.0f, (_Float16)1.0f}, acc, false);
  }
}

// Reductions over the lane pair (l, l ^ 32) through ds_bpermute.
__device__ __forceinline__ float max_xor32(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }
__device__ __forceinline__ float sum_xor32(float x) { return x + __shfl_xor(x, 32, 64); }

// The same maximum on the VALU (v_permlane32_swap, gfx950), for code that runs
// while other waves saturate the LDS pipeline, which ds_bpermute also uses.
// swap(a, b) exchanges the upper half of a with the lower half of b, so with
// a = b = x the two results hold x[l & 31] and x[32 + (l & 31)] in every lane.
// Both results pass through integer variables and an empty asm: this
// compiler reads element 0 when bit_cast is applied to a subscripted vector
// element (bit_cast<float>(result[1]) becomes result[0]), which silently
// turns the reduction into the identity.
__device__ __forceinline__ float max_xor32_valu(float x) {
  const unsigned xb = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(xb, xb, false, false);
  unsigned lo = r[0], up = r[1];
  asm volatile("" : "+v"(lo), "+v"(up));
  return fmaxf(__builtin_bit_cast(float, lo), __builtin_bit_cast(float, up));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kBufferFlags);
}

// The same descriptor from wave-uniform values that the compiler may hold in
// VGPRs: every word goes through v_readfirstlane, so each buffer instruction
// takes it from SGPRs directly.  (A descriptor the compiler believes
// divergent is wrapped in a waterfall loop per instruction, which also
// serialises every store behind its own LDS read.)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_uniform(const void* base,
                                                                    uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b)));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t n = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(bytes)));
  void* p = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)n, kBufferFlags);
}

// ---------------------------------------------------------------------------
// Work decoding: workgroup id -> (sequence, head, q-block) and addressing.
// ---------------------------------------------------------------------------
struct Work {
  bool valid;
  int b, h, kvh, qblk;
  int pair;                // (item, kv head) pair index
  int hg;                  // h - kvh * (Hq / Hkv): head index within the kv group
  int Lq, Lk;
  int64_t q_base, o_base;  // element offset of row 0 of this (sequence, head)
  int64_t k_base, v_base;  // dense/ragged: row 0 of this (sequence, kv head);
                           // paged: kv-head offset only
  int off;                 // causal diagonal offset: key j visible iff j <= i + off
};

// Item list of a ragged launch without a plan kernel (KArgs::inline_plan),
// built in LDS by every workgroup (build_inline_plan): item i is q-block (or
// q-block pair) i - cum[b] of the sequence b with cum[b] <= i < cum[b + 1],
// sequence by sequence; every workgroup of such a launch is resident at once,
// so the order of the items does not matter.
constexpr int kInlinePlanMaxBatch = 256;
// Balanced walk of the two-head kernel: kv-head pairs per lane of the wave
// that locates a workgroup's segment (at most 64 * kBalMaxPer per XCD).
constexpr int kBalMaxPer = 16;
struct InlinePlan {
  int cum[kInlinePlanMaxBatch + 1];
  int qi[kInlinePlanMaxBatch + 1];  // copies of q_indptr and kv_indptr
  int ki[kInlinePlanMaxBatch + 1];
  int max_cost;  // KV tiles of the heaviest item
  int splits;    // the launch's split count
};

// Workgroup ids are dispatched round-robin over the 8 XCDs (each with its own
// L2).  Ids are laid out as ((blk * G + g) * 8 + p): the 8 (item, kv head)
// pairs of block `blk` go to 8 different XCDs, and the G query heads that
// share one kv head land on the same XCD at ids 8 apart, so their K/V tiles
// are fetched into one L2.  Items (and so LPT order) ascend with blk.
constexpr int kXcds = 8;

// A unit may cover `heads` consecutive query heads of one kv group (the
// ping-pong kernel takes two); w.h is then the first of them.
// ip: the inline plan's table (null: none); UNI: its reads pass through
// readfirstlane (they are wave-uniform), so that a kernel that derives loop
// bounds from the result keeps them in scalar registers.
template <int MODE, bool UNI = false>
__device__ __forceinline__ Work decode_work(const KArgs& a, int L, int heads = 1,
                                            const InlinePlan* ip = nullptr) {
  Work w;
  w.valid = true;
  const int group = a.hq / a.hkv;
  const int units = a.pack_m > 0 ? 1 : (group + heads - 1) / heads;
  const int p = L % kXcds;
  const int rest = L / kXcds;
  const int g = rest % units;
  const int pair = (rest / units) * kXcds + p;
  if (pair >= a.npairs) {
    w.valid = false;
    return w;
  }
  w.pair = pair;
  const int item = pair / a.hkv;
  w.kvh = pair % a.hkv;
  w.hg = g * heads;
  w.h = w.kvh * group + w.hg;  // kv head = h * Hkv / Hq (attention.py:463)
  if constexpr (MODE == FA2_LAYOUT_DENSE) {
    const int rank = item / a.batch;
    w.b = item % a.batch;
    // heaviest q-blocks first under a causal mask
    w.qblk = (a.mask != FA2_MASK_NONE && a.pack_m == 0) ? (a.nqb - 1 - rank) : rank;
    w.Lq = a.q_len;
    w.Lk = a.kv_len;
    w.q_base = w.b * a.q_sb + w.h * a.q_sh;
    w.o_base = w.b * a.o_sb + w.h * a.o_sh;
    w.k_base = w.b * a.k_sb + w.kvh * a.k_sh;
    w.v_base = w.b * a.v_sb + w.kvh * a.v_sh;
  } else {
    int2 it;
    if (a.work) {
      if (item >= *a.work_count) {
        w.valid = false;
        return w;
      }
      it = a.work[item];
    } else if (MODE == FA2_LAYOUT_RAGGED && ip) {
      auto rd = [](const int& x) { return UNI ? __builtin_amdgcn_readfirstlane(x) : x; };
      if (item >= rd(ip->cum[a.batch])) {
        w.valid = false;
        return w;
      }
      int lo = 0, hi = a.batch;  // the last b with cum[b] <= item
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (rd(ip->cum[mid]) <= item) lo = mid;
        else hi = mid;
      }
      it = make_int2(lo, item - rd(ip->cum[lo]));
    } else {
      // no plan (uniform q-block count, every workgroup resident at once, so
      // the order does not matter): items in (q-block, sequence) order
      if (item >= a.batch * a.nqb) {
        w.valid = false;
        return w;
      }
      it = make_int2(item % a.batch, item / a.batch);
    }
    w.b = it.x;
    w.qblk = it.y;
    if constexpr (MODE == FA2_LAYOUT_RAGGED) {
      // (the offsets from the inline plan's copies in LDS when there is one)
      auto rd = [](const int& x) { return UNI ? __builtin_amdgcn_readfirstlane(x) : x; };
      const int ks = ip ? rd(ip->ki[w.b]) : a.kv_indptr[w.b];
      w.Lk = (ip ? rd(ip->ki[w.b + 1]) : a.kv_indptr[w.b + 1]) - ks;
      if (a.pack_m > 0) {  // decode: dense q/o over a ragged K/V
        w.Lq = a.q_len;
        w.q_base = w.b * a.q_sb + w.h * a.q_sh;
        w.o_base = w.b * a.o_sb + w.h * a.o_sh;
      } else {
        const int qs = ip ? rd(ip->qi[w.b]) : a.q_indptr[w.b];
        w.Lq = (ip ? rd(ip->qi[w.b + 1]) : a.q_indptr[w.b + 1]) - qs;
        w.q_base = qs * a.q_ss + w.h * a.q_sh;
        w.o_base = qs * a.o_ss + w.h * a.o_sh;
      }
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
  w.off = (a.mask == FA2_MASK_CAUSAL_BOTTOM_RIGHT) ? (w.Lk - (a.pack_m > 0 ? a.pack_m : w.Lq))
                                                   : 0;
  return w;
}

// Query position of unit row `row` on the causal diagonal: the row itself,
// or its draft position in packed-head mode.
__device__ __forceinline__ int diag_row(const KArgs& a, int row) {
  return a.pack_m > 0 ? row % a.pack_m : row;
}

// Number of keys a q-block [q0, q0+BM) can see (exclusive end), >= 0.
__device__ __forceinline__ int kv_end_for_block(int mask, int q0, int Lq, int Lk, int off) {
  if (mask == FA2_MASK_NONE) return Lk;
  int qe = min(q0 + kBM, Lq);
  int e = min(Lk, qe + off);
  return e > 0 ? e : 0;
}

// The same for a unit; in packed-head mode the last draft position of every
// block sees the whole sequence.
__device__ __forceinline__ int kv_end_for_unit(const KArgs& a, int q0, int Lq, int Lk, int off) {
  return a.pack_m > 0 ? Lk : kv_end_for_block(a.mask, q0, Lq, Lk, off);
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

// Global -> register staging of K and V tiles, then register -> LDS.
// Dense/ragged (BUF): buffer loads through one descriptor per tile, based at
// the tile's first row (64-bit) and covering its rows inside the sequence,
// whose range check zero-fills rows past the end.  Paged, BUF: the byte
// offsets of every row of the page pool fit in 31 bits (buffer loads from
// the pool base); !BUF: 64-bit global loads of rows clamped to the last
// valid row (finite data, masked by the softmax).
template <int DT, int D, int MODE, bool BUF>
struct TileLoader {
  static constexpr int kEB = Elt<DT>::kBytes;
  static constexpr int kTPR = D / 8;  // threads per K row
  static constexpr int kRowsPerPass = kThreads / kTPR;
  static constexpr int kKPasses = kBN / kRowsPerPass;
  static constexpr int kKPT = kBN * D / (8 * kThreads);  // V keys per thread
  static_assert(kKPasses >= 1 && (kKPT == 1 || kKPT == 2 || kKPT == 4 || kKPT == 8),
                "tile shape");
  // a 16-byte chunk outside the valid head dims: buffer offset past any range
  static constexpr uint32_t kOut = 0xFFFFFF00u;

  Raw8<DT> kr[kKPasses];
  Raw8<DT> vr[kKPT];
  int krow0, vkey0, col;  // this thread's first K row, first V key, column (elements)
  bool cok;               // col < dv: the column holds data (else zeros)

  __device__ __forceinline__ TileLoader(int tid, int dv) {
    krow0 = tid / kTPR;
    col = (tid % kTPR) * 8;
    vkey0 = (tid / kTPR) * kKPT;
    cok = col < dv;
  }

  __device__ __forceinline__ static int paged_row(const int32_t* table, int64_t tstride, int b,
                                                  int n, int page) {
    const int pg = table[b * tstride + n / page];
    return pg * page + (n % page);
  }

  __device__ __forceinline__ void issue_k(const KArgs& a, const Work& w, int k0) {
    if constexpr (BUF) {
      if constexpr (MODE == FA2_LAYOUT_PAGED) {
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc_uniform(static_cast<const char*>(a.k) + w.k_base * kEB, a.pool_bytes_k);
#pragma unroll
        for (int p = 0; p < kKPasses; ++p) {
          const int n = k0 + krow0 + p * kRowsPerPass;
          const int nc = min(n, w.Lk - 1);
          const uint32_t row = paged_row(a.k_table, a.k_table_stride, w.b, nc, a.page_size);
          const uint32_t off = row * static_cast<uint32_t>(a.k_ss * kEB) + col * kEB;
          buf_raw8<DT>(kr[p], rs, (n < w.Lk && cok) ? off : kOut);
        }
      } else {
        const uint32_t rsb = static_cast<uint32_t>(a.k_ss * kEB);
        // the descriptor covers this tile's rows inside the sequence only
        const uint32_t lim = static_cast<uint32_t>(min(max(w.Lk - k0, 0), kBN)) * rsb;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc_uniform(
            static_cast<const char*>(a.k) + (w.k_base + static_cast<int64_t>(k0) * a.k_ss) * kEB,
            lim);
#pragma unroll
        for (int p = 0; p < kKPasses; ++p)
          buf_raw8<DT>(kr[p], rs, cok ? (krow0 + p * kRowsPerPass) * rsb + col * kEB : kOut);
      }
    } else {
#pragma unroll
      for (int p = 0; p < kKPasses; ++p) {
        const int n = min(k0 + krow0 + p * kRowsPerPass, w.Lk - 1);
        int64_t off;
        if constexpr (MODE == FA2_LAYOUT_PAGED)
          off = w.k_base +
                static_cast<int64_t>(paged_row(a.k_table, a.k_table_stride, w.b, n, a.page_size)) *
                    a.k_ss;
        else
          off = w.k_base + static_cast<int64_t>(n) * a.k_ss;
        if (cok)
          load_raw8<DT>(kr[p], a.k, off + col);
        else
          zero_raw8<DT>(kr[p]);
      }
    }
  }

  __device__ __forceinline__ void issue_v(const KArgs& a, const Work& w, int k0) {
    if constexpr (BUF) {
      if constexpr (MODE == FA2_LAYOUT_PAGED) {
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc_uniform(static_cast<const char*>(a.v) + w.v_base * kEB, a.pool_bytes_v);
#pragma unroll
        for (int j = 0; j < kKPT; ++j) {
          const int n = k0 + vkey0 + j;
          const int nc = min(n, w.Lk - 1);
          const uint32_t row = paged_row(a.v_table, a.v_table_stride, w.b, nc, a.page_size);
          const uint32_t off = row * static_cast<uint32_t>(a.v_ss * kEB) + col * kEB;
          buf_raw8<DT>(vr[j], rs, (n < w.Lk && cok) ? off : kOut);
        }
      } else {
        const uint32_t rsb = static_cast<uint32_t>(a.v_ss * kEB);
        // the descriptor covers this tile's rows inside the sequence only
        const uint32_t lim = static_cast<uint32_t>(min(max(w.Lk - k0, 0), kBN)) * rsb;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc_uniform(
            static_cast<const char*>(a.v) + (w.v_base + static_cast<int64_t>(k0) * a.v_ss) * kEB,
            lim);
#pragma unroll
        for (int j = 0; j < kKPT; ++j)
          buf_raw8<DT>(vr[j], rs, cok ? (vkey0 + j) * rsb + col * kEB : kOut);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kKPT; ++j) {
        const int n = min(k0 + vkey0 + j, w.Lk - 1);
        int64_t off;
        if constexpr (MODE == FA2_LAYOUT_PAGED)
          off = w.v_base +
                static_cast<int64_t>(paged_row(a.v_table, a.v_table_stride, w.b, n, a.page_size)) *
                    a.v_ss;
        else
          off = w.v_base + static_cast<int64_t>(n) * a.v_ss;
        if (cok)
          load_raw8<DT>(vr[j], a.v, off + col);
        else
          zero_raw8<DT>(vr[j]);
      }
    }
  }

  __device__ __forceinline__ void commit_k(uint16_t* ks) const {
    using L = Lds<D>;
#pragma unroll
    for (int p = 0; p < kKPasses; ++p) {
      const int row = krow0 + p * kRowsPerPass;
      *reinterpret_cast<u32x4*>(ks + row * L::kKStride + col) = to16<DT>(kr[p]);
    }
  }

  __device__ __forceinline__ void commit_v(uint16_t* vt) const {
    using L = Lds<D>;
    u32x4 x[kKPT];
#pragma unroll
    for (int j = 0; j < kKPT; ++j) x[j] = to16<DT>(vr[j]);
    // groups of up to 4 consecutive keys stay adjacent in a transposed row
    constexpr int kG = kKPT < 4 ? kKPT : 4;
#pragma unroll
    for (int g0 = 0; g0 < kKPT; g0 += kG) {
      const int pos = vpos(vkey0 + g0);
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const int word = d >> 1;
        // v_perm_b32 byte selectors: low halves (d even) or high halves (d odd)
        const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;
        uint16_t* dst = vt + (col + d) * L::kVStride + pos;
        if constexpr (kG == 4) {
          const uint32_t a01 = __builtin_amdgcn_perm(x[g0 + 1][word], x[g0][word], sel);
          const uint32_t a23 = __builtin_amdgcn_perm(x[g0 + 3][word], x[g0 + 2][word], sel);
          *reinterpret_cast<u32x2*>(dst) = (u32x2){a01, a23};
        } else if constexpr (kG == 2) {
          *reinterpret_cast<uint32_t*>(dst) = __builtin_amdgcn_perm(x[1][word], x[0][word], sel);
        } else {
          *dst = static_cast<uint16_t>((d & 1) ? (x[0][word] >> 16) : (x[0][word] & 0xffffu));
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Forward kernel.
// ---------------------------------------------------------------------------
// S of the next tile is software-pipelined against the softmax of the current
// one where the registers allow it (two waves per SIMD = 256 VGPRs).
template <int D>
struct Pipe {
#ifdef FA2_PIPE_D128
  static constexpr bool value = true;
#else
  static constexpr bool value = D <= 64;
#endif
};

// D = 256 holds one wave per SIMD (O^T alone is 128 VGPRs per lane).
template <int DT, int D, int MODE, bool BUF, bool PIPE = Pipe<D>::value>
__global__ __launch_bounds__(kThreads, D > 128 ? 1 : 2) void fa2_fwd_kernel(KArgs a) {
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
  const int S = launch_splits(a);
  if (split >= S) return;

  // KV tile range of this split.
  const int kv_end = kv_end_for_unit(a, q0, w.Lq, w.Lk, w.off);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const int t_begin = (ntiles * split) / S;
  const int t_end = (ntiles * (split + 1)) / S;
  const int T = t_end - t_begin;

  // Q^T fragments: lane holds query row q0 + 32*wave + l32, dims c*16+8*hi..+7.
  const int qrow = q0 + wave * kWaveRows + l32;
  u32x4 qf[DC];
  {
    const bool ok = qrow < w.Lq;
    const int64_t base = w.q_base + static_cast<int64_t>(qrow) * a.q_ss + hi * 8;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      Raw8<DT> r;
      if (ok && c * 16 + hi * 8 < a.dv)
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
  // first row of the wave; its rows' smallest diagonal position and this lane's
  const int wq_first = q0 + wave * kWaveRows;
  const int wq_diag = a.pack_m > 0 ? 0 : wq_first;
  const int qdiag = diag_row(a, qrow);
  const bool causal = a.mask != FA2_MASK_NONE;

  TileLoader<DT, D, MODE, BUF> ld(tid, a.dv);

  // S^T block for the tile held in K buffer `kb`.
  auto compute_s = [&](f32x16 (&s)[SB], int kb) {
    const uint16_t* ks = ks_base + kb * L::kKTile;
    // accumulators interleaved (c-major): back-to-back dependent MFMAs stall
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) s[sb] = (f32x16){};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        const uint16_t* krow = ks + (sb * 32 + l32) * L::kKStride + hi * 8;
        const u32x4 kf = *reinterpret_cast<const u32x4*>(krow + c * 16);
        s[sb] = mma32<BF>(kf, qf[c], s[sb]);
      }
    }
  };

  // One pipeline step: softmax + PV of tile i (scores in s_cur), S of tile
  // i+1 into s_nxt, loads of K(i+2) and V(i+1).  `last` (a compile-time
  // flag) marks the final tile, which has no successor.
  auto step = [&](auto last, int i, f32x16 (&s_cur)[SB], f32x16 (&s_nxt)[SB]) {
    constexpr bool kLast = decltype(last)::value;
    const int t = t_begin + i;
    const int k0 = t * kBN;
    constexpr bool has_next = !kLast;
    // PIPE: K runs two tiles ahead (S of tile t+1 is computed in this step);
    // otherwise K and V both run one tile ahead and S(t) is computed here.
    const bool has_k2 = PIPE ? (!kLast && (i + 2 < T)) : has_next;
    if (has_k2) ld.issue_k(a, w, k0 + (PIPE ? 2 : 1) * kBN);
    if constexpr (has_next) ld.issue_v(a, w, k0 + kBN);
    if constexpr (!PIPE) compute_s(s_cur, i & 1);

    // masks only at the sequence end or on the causal diagonal (wave-uniform)
    if ((k0 + kBN > w.Lk) || (causal && (k0 + kBN - 1 > wq_diag + w.off))) {
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
          const int key = k0 + sb * 32 + (i2 >> 2) * 8 + hi * 4 + (i2 & 3);
          const bool ok = (key < w.Lk) && (!causal || key <= qdiag + w.off);
          if (!ok) s_cur[sb][i2] = -INFINITY;
        }
      }
    }

    if constexpr (has_next && PIPE) compute_s(s_nxt, (i + 1) & 1);

    // online softmax of tile i (row = this lane's query)
    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < SB; ++sb)
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) mx = fmaxf(mx, s_cur[sb][i2]);
    mx = max_xor32(mx);
    const float mt = mx * a.scale_log2;
    const bool need = mt > m_run + kRescaleThreshold;
    const float alpha = need ? fast_exp2(m_run - mt) : 1.0f;
    const float m_new = need ? mt : m_run;
    m_run = m_new;
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    float rs = 0.f;
    u32x4 pf[kBN / 16];
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
      float p[16];
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) {
        p[i2] = fast_exp2(__builtin_fmaf(s_cur[sb][i2], a.scale_log2, -m_use));
        rs += p[i2];
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
    if (__any(need)) {
#pragma unroll
      for (int d = 0; d < DB; ++d) o[d] *= alpha;
    }
    // O^T += V^T P^T
    const uint16_t* vt = vt_base + (i & 1) * L::kVTile;
#pragma unroll
    for (int c = 0; c < kBN / 16; ++c) {
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const uint16_t* vrow = vt + (d * 32 + l32) * L::kVStride + hi * 8;
        const u32x4 vf = *reinterpret_cast<const u32x4*>(vrow + c * 16);
        o[d] = mma32<BF>(vf, pf[c], o[d]);
      }
    }
    if (has_k2) ld.commit_k(ks_base + ((PIPE ? i : i + 1) & 1) * L::kKTile);
    if constexpr (has_next) {
      ld.commit_v(vt_base + ((i + 1) & 1) * L::kVTile);
      __syncthreads();
    }
  };
  using NotLast = std::integral_constant<bool, false>;
  using Last = std::integral_constant<bool, true>;

  f32x16 sA[SB], sB[SB];
  if (T > 0) {
    ld.issue_k(a, w, t_begin * kBN);
    ld.issue_v(a, w, t_begin * kBN);
    ld.commit_k(ks_base);
    ld.commit_v(vt_base);
    if (PIPE && T > 1) {
      ld.issue_k(a, w, (t_begin + 1) * kBN);
      ld.commit_k(ks_base + L::kKTile);
    }
    __syncthreads();
    if constexpr (PIPE) {
      compute_s(sA, 0);
      // step 0 rewrites K buffer 0 with K(t0+2): all waves must be done
      // reading K(t0) first
      __syncthreads();
    }
    int i = 0;
    if constexpr (D > 128) {
      // one step per iteration: a second inlined step does not fit the registers
      for (; i + 1 < T; ++i) step(NotLast{}, i, sA, sB);
      step(Last{}, i, sA, sB);
    } else {
      for (; i + 2 < T; i += 2) {
        step(NotLast{}, i, sA, sB);
        step(NotLast{}, i + 1, sB, sA);
      }
      if (i + 1 < T) {
        step(NotLast{}, i, sA, sB);
        step(Last{}, i + 1, sB, sA);
      } else {
        step(Last{}, i, sA, sB);
      }
    }
  }

  const float l_tot = sum_xor32(l_run);
  if (S == 1 && !a.part_out) {
    if (qrow < w.Lq) {
      const float inv = 1.f / l_tot;  // 0/0 -> NaN for a row with no key, as the reference
      const int64_t base = w.o_base + static_cast<int64_t>(qrow) * a.o_ss + hi * 4;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (d * 32 + g * 8 + hi * 4 >= a.dv) continue;  // padding dims (head_dim 16, 32)
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
    // Split partials: slot (split, workgroup), row r of the q-block; only
    // rows the combine reads (r < part_rows, q0 + r < Lq) are written.
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

// ---------------------------------------------------------------------------
// Split-KV combine: O = sum_s 2^(m_s-g) O_s / sum_s 2^(m_s-g) l_s, g = max m_s
// (attention.py:710-724 restated in the log2 domain).  Grid (units, row
// chunks): each thread owns 4 columns of one row and walks the splits four
// at a time, so the loads of different splits are in flight together (a
// loop with one split per step is latency-bound at large split counts).
// ---------------------------------------------------------------------------
template <int D>
constexpr int kCombineRows = kThreads / (D / 4);  // rows per workgroup

// Cache policy of the partials of a merge inside a forward kernel: `sc1`
// (device scope), coherent across the XCDs' L2 caches without the cache-wide
// writeback and invalidate of a release/acquire fence.
constexpr int kCpolSc1 = 16;

// Device-scope stores of partials from per-lane addresses (relaxed
// agent-scope atomic stores: `global_store_dword ... sc1`).
__device__ __forceinline__ void st_dev2(float* p, float x, float y) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(p + 1, y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev4(float* p, f32x4 x) {
  const float x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
  st_dev2(p, x0, x1);
  st_dev2(p + 2, x2, x3);
}

// Row r, columns col..col+3 of the unit in part slot `unit` (of S splits),
// written to the output element offset `off`.
template <int DT, int D>
__device__ __forceinline__ void combine_row(const KArgs& a, int unit, int r, int col, int S,
                                            int64_t off) {
  const int64_t G = a.part_slots;
  const int64_t R = a.part_rows;
  const float* ml = a.part_ml + (static_cast<int64_t>(unit) * R + r) * 2;
  const float* po = a.part_o + (static_cast<int64_t>(unit) * R + r) * D + col;
  const int64_t ml_step = G * R * 2, o_step = G * R * D;  // one split further
  float g = -INFINITY;
  int s = 0;
  for (; s + 4 <= S; s += 4) {
    const float m0 = ml[(s + 0) * ml_step], m1 = ml[(s + 1) * ml_step];
    const float m2 = ml[(s + 2) * ml_step], m3 = ml[(s + 3) * ml_step];
    g = fmaxf(g, fmaxf(fmaxf(m0, m1), fmaxf(m2, m3)));
  }
  for (; s < S; ++s) g = fmaxf(g, ml[s * ml_step]);
  const float g_use = (g == -INFINITY) ? 0.f : g;
  float lsum = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  s = 0;
  for (; s + 4 <= S; s += 4) {
    float m[4], l[4];
    f32x4 x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m[j] = ml[(s + j) * ml_step];
      l[j] = ml[(s + j) * ml_step + 1];
      x[j] = *reinterpret_cast<const f32x4*>(po + (s + j) * o_step);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // splits in order, as the one-at-a-time loop
      const float wgt = fast_exp2(m[j] - g_use);
      lsum += wgt * l[j];
      acc += wgt * x[j];
    }
  }
  for (; s < S; ++s) {
    const float wgt = fast_exp2(ml[s * ml_step] - g_use);
    lsum += wgt * ml[s * ml_step + 1];
    acc += wgt * *reinterpret_cast<const f32x4*>(po + s * o_step);
  }
  const float inv = 1.f / lsum;  // 0/0 -> NaN for a row with no key, as the reference
  if constexpr (DT == FA2_DTYPE_F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(a.o) + off) = acc * inv;
  } else {
    constexpr bool BF = Elt<DT>::kBF;
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.o) + off) =
        (u32x2){pack2<BF>(acc[0] * inv, acc[1] * inv), pack2<BF>(acc[2] * inv, acc[3] * inv)};
  }
}

template <int DT, int D, int MODE>
__global__ __launch_bounds__(kThreads) void fa2_combine_kernel(KArgs a) {
  const int S = launch_splits(a);
  if (S <= 1 && !a.part_out) return;  // the forward kernel wrote the output
  const Work w = decode_work<MODE>(a, blockIdx.x);
  if (!w.valid) return;
  constexpr int kTPR = D / 4;  // threads per row, 4 floats each
  const int r = blockIdx.y * kCombineRows<D> + threadIdx.x / kTPR;
  const int col = (threadIdx.x % kTPR) * 4;
  const int qrow = w.qblk * a.block_rows + r;
  if (r >= a.part_rows || qrow >= w.Lq || col >= a.dv) return;
  combine_row<DT, D>(a, blockIdx.x, r, col, S,
                     w.o_base + static_cast<int64_t>(qrow) * a.o_ss + col);
}

// Split merge inside the forward kernel (KArgs::merge_ctr).  The threads that
// write this unit's partials do so with store_partial_rows<true>; then every thread of
// the workgroup calls merge_publish (its stores have been performed at
// device scope) and, after a workgroup barrier, merge_count; `flag` is one
// LDS word of scratch.  merge_count returns true in every thread of the
// workgroup whose split completed the unit's count: it then merges
// (merge_rows, reading the partials at device scope).
__device__ __forceinline__ void merge_publish() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__device__ __forceinline__ bool merge_count(const KArgs& a, int unit, int S, int* flag) {
  if (threadIdx.x == 0) {
    uint64_t* c = a.merge_ctr + unit;
    const uint64_t tag = a.merge_tag;
    uint64_t old = __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint64_t cnt;
    for (;;) {
      cnt = (old >> kMergeCountBits) == tag ? (old & ((uint64_t(1) << kMergeCountBits) - 1)) : 0;
      const uint64_t nw = (tag << kMergeCountBits) | (cnt + 1);
      if (__hip_atomic_compare_exchange_strong(c, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        break;
    }
    const bool last = static_cast<int>(cnt) + 1 == S;
    // the next launch with this tag (a graph replay) starts from zero; no
    // split of this launch adds to the word after the last one
    if (last)
      __hip_atomic_store(c, tag << kMergeCountBits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *static_cast<volatile int*>(flag) = last ? 1 : 0;
  }
  __syncthreads();
  // (the partials are read after this, at device scope: the count that made
  // this split the last was taken after every split's stores were performed)
  return *static_cast<volatile int*>(flag) != 0;
}

// Split partials of one row (this lane's half: hi), the O^T accumulator
// layout of the 16-bit kernels (row l32, dims 32d + 8g + 4hi + j at
// o[d][4g + j]), into part slot `slot` (split * part_slots + unit); DEV:
// written at device scope (`sc1` buffer stores) for a merge in the kernel.
template <bool DEV, int D>
__device__ __forceinline__ void store_partial_rows(const KArgs& a, int64_t slot, int r, int hi,
                                                   float m, float l, const f32x16 (&o)[D / 32]) {
  if constexpr (DEV) {
    const uint32_t R = static_cast<uint32_t>(a.part_rows);
    const __amdgpu_buffer_rsrc_t rm = make_rsrc_uniform(a.part_ml + slot * R * 2, R * 8);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc_uniform(a.part_o + slot * R * D, R * D * 4);
    if (hi == 0)
      __builtin_amdgcn_raw_buffer_store_b64(
          (u32x2){__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, l)}, rm,
          static_cast<uint32_t>(r) * 8, 0, kCpolSc1);
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, (f32x4){o[d][g * 4 + 0], o[d][g * 4 + 1], o[d][g * 4 + 2],
                                              o[d][g * 4 + 3]}),
            ro, static_cast<uint32_t>(r * D + d * 32 + g * 8 + hi * 4) * 4, 0, kCpolSc1);
  } else {
    if (hi == 0) {
      float* ml = a.part_ml + (slot * a.part_rows + r) * 2;
      ml[0] = m;
      ml[1] = l;
    }
    float* po = a.part_o + (slot * a.part_rows + r) * D + hi * 4;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(po + d * 32 + g * 8) =
            (f32x4){o[d][g * 4 + 0], o[d][g * 4 + 1], o[d][g * 4 + 2], o[d][g * 4 + 3]};
  }
}

// Partials in fragment order (the two-head kernel's balanced walk): wave wq's
// (m, l) of row wq * 32 + l32 at that row, and its O^T accumulator o[d]
// (dims 32d + 8g + 4hi + j at o[d][4g + j]) at chunk ((wq * D / 32 + d) * 4 +
// g) * 64 + lane of 16 bytes, so that one store or load of the wave covers
// 1 KB in a row.  Written and read at device scope (sc1) by the workgroups
// of one unit's pieces; only they read this layout.
template <int D>
__device__ __forceinline__ void store_partial_frag(const KArgs& a, int64_t slot, int wq,
                                                   int lane, float m, float l,
                                                   const f32x16 (&o)[D / 32]) {
  const uint32_t R = static_cast<uint32_t>(a.part_rows);
  const __amdgpu_buffer_rsrc_t rm = make_rsrc_uniform(a.part_ml + slot * R * 2, R * 8);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc_uniform(a.part_o + slot * R * D, R * D * 4);
  if (lane < 32)
    __builtin_amdgcn_raw_buffer_store_b64(
        (u32x2){__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, l)}, rm,
        static_cast<uint32_t>(wq * 32 + lane) * 8, 0, kCpolSc1);
#pragma unroll
  for (int d = 0; d < D / 32; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(u32x4, (f32x4){o[d][g * 4 + 0], o[d][g * 4 + 1], o[d][g * 4 + 2],
                                            o[d][g * 4 + 3]}),
          ro, static_cast<uint32_t>(((wq * (D / 32) + d) * 4 + g) * 64 + lane) * 16, 0,
          kCpolSc1);
}

// (m, l) of this lane's row from a fragment-order slot
__device__ __forceinline__ u32x2 load_partial_frag_ml(const KArgs& a, int64_t slot, int wq,
                                                      int l32) {
  const uint32_t R = static_cast<uint32_t>(a.part_rows);
  const __amdgpu_buffer_rsrc_t rm = make_rsrc_uniform(a.part_ml + slot * R * 2, R * 8);
  return __builtin_amdgcn_raw_buffer_load_b64(rm, static_cast<uint32_t>(wq * 32 + l32) * 8, 0,
                                              kCpolSc1);
}

// O^T block d of this lane from a fragment-order slot
template <int D>
__device__ __forceinline__ f32x16 load_partial_frag_o(const KArgs& a, int64_t slot, int wq,
                                                      int lane, int d) {
  const uint32_t R = static_cast<uint32_t>(a.part_rows);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc_uniform(a.part_o + slot * R * D, R * D * 4);
  f32x16 x;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 c = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                   ro, static_cast<uint32_t>(((wq * (D / 32) + d) * 4 + g) * 64 + lane) * 16, 0,
                   kCpolSc1));
    x[g * 4 + 0] = c[0];
    x[g * 4 + 1] = c[1];
    x[g * 4 + 2] = c[2];
    x[g * 4 + 3] = c[3];
  }
  return x;
}

// A unit's merge word (merge_count's) when every other piece has counted:
// the caller is the last piece and takes the word back to (tag, 0) without
// having written its partials.  Thread 0; true if taken.
__device__ __forceinline__ bool merge_take_last(const KArgs& a, int unit, int S) {
  uint64_t* c = a.merge_ctr + unit;
  const uint64_t tag = a.merge_tag;
  uint64_t old = __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t cnt =
      (old >> kMergeCountBits) == tag ? (old & ((uint64_t(1) << kMergeCountBits) - 1)) : 0;
  if (static_cast<int>(cnt) + 1 != S) return false;
  return __hip_atomic_compare_exchange_strong(c, &old, tag << kMergeCountBits, __ATOMIC_RELAXED,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The merge itself: rows [0, rows) (rows <= MAXR) of the partials of
// pieces 0..S-1, piece s in part slot slot_of(s), the output of row r at
// o_base + (row0 + r) * o_ss; NT threads of the workgroup, each taking 4
// columns of MAXR / (NT / (D / 4)) rows.  The partials are read at device
// scope, a chunk of a thread's rows at once: with at most SM pieces, every
// piece's (m, l) and O in one pass; otherwise the running maxima of four
// pieces at a time, then (m, l) and O piece by piece.  Per row and column
// the arithmetic is combine_row's, in the same order.
// (The rows a thread holds at once are bounded for registers.)
template <int DT, int D, int NT, int MAXR, int SM, typename SlotOf>
__device__ __forceinline__ void merge_rows_sm(const KArgs& a, SlotOf slot_of, int S, int rows,
                                              int64_t o_base, int row0) {
  constexpr int kTPR = D / 4;
  constexpr int kRPP = NT / kTPR;                   // rows per pass of the workgroup
  constexpr int kRows = (MAXR + kRPP - 1) / kRPP;   // rows per thread
  constexpr int kCap = (SM > 0 ? 16 / SM : 4) / (D > 128 ? 2 : 1);
  constexpr int kIt = kRows < kCap ? kRows : kCap;  // rows per thread per chunk
  const int col = (threadIdx.x % kTPR) * 4;
  const uint32_t R = static_cast<uint32_t>(a.part_rows);
  auto rsrc_ml = [&](int s) {
    return make_rsrc_uniform(a.part_ml + slot_of(s) * static_cast<int64_t>(R) * 2, R * 8);
  };
  auto rsrc_o = [&](int s) {
    return make_rsrc_uniform(a.part_o + slot_of(s) * static_cast<int64_t>(R) * D, R * D * 4);
  };
  auto ld_ml = [&](__amdgpu_buffer_rsrc_t rs, int r) {
    return __builtin_amdgcn_raw_buffer_load_b64(rs, static_cast<uint32_t>(r) * 8, 0, kCpolSc1);
  };
  auto ld_o = [&](__amdgpu_buffer_rsrc_t rs, int r) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<uint32_t>(r * D + col) * 4, 0,
                                                 kCpolSc1);
  };
  // (bit_cast through scalars: this compiler reads element 0 when bit_cast
  // is applied to a subscripted vector element)
  auto fl = [](uint32_t w) { return __builtin_bit_cast(float, w); };
  for (int c0 = threadIdx.x / kTPR; c0 < rows; c0 += kIt * kRPP) {  // chunks of kIt rows
    float g[kIt], lsum[kIt];
    f32x4 acc[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      g[it] = -INFINITY;
      lsum[it] = 0.f;
      acc[it] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (SM > 0) {
      u32x2 ml[SM][kIt];
      u32x4 x[SM][kIt];
#pragma unroll
      for (int s = 0; s < SM; ++s) {
        if (s < S) {
          const __amdgpu_buffer_rsrc_t rm = rsrc_ml(s);
          const __amdgpu_buffer_rsrc_t ro = rsrc_o(s);
#pragma unroll
          for (int it = 0; it < kIt; ++it) {
            if (c0 + it * kRPP < rows) {
              ml[s][it] = ld_ml(rm, c0 + it * kRPP);
              x[s][it] = ld_o(ro, c0 + it * kRPP);
            }
          }
        }
      }
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        if (c0 + it * kRPP >= rows) continue;
#pragma unroll
        for (int s = 0; s < SM; ++s) {
          const uint32_t mw = ml[s][it][0];
          if (s < S) g[it] = fmaxf(g[it], fl(mw));
        }
        const float g_use = g[it] == -INFINITY ? 0.f : g[it];
#pragma unroll
        for (int s = 0; s < SM; ++s) {
          if (s < S) {
            const uint32_t mw = ml[s][it][0], lw = ml[s][it][1];
            const float wgt = fast_exp2(fl(mw) - g_use);
            lsum[it] += wgt * fl(lw);
            acc[it] += wgt * __builtin_bit_cast(f32x4, x[s][it]);
          }
        }
      }
    } else {
      int s = 0;
      for (; s + 4 <= S; s += 4) {
        float m[4][kIt];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const __amdgpu_buffer_rsrc_t rs = rsrc_ml(s + j);
#pragma unroll
          for (int it = 0; it < kIt; ++it) {
            const uint32_t mw = c0 + it * kRPP < rows ? ld_ml(rs, c0 + it * kRPP)[0] : 0u;
            m[j][it] = c0 + it * kRPP < rows ? fl(mw) : -INFINITY;
          }
        }
#pragma unroll
        for (int it = 0; it < kIt; ++it)
          g[it] = fmaxf(g[it], fmaxf(fmaxf(m[0][it], m[1][it]), fmaxf(m[2][it], m[3][it])));
      }
      for (; s < S; ++s) {
        const __amdgpu_buffer_rsrc_t rs = rsrc_ml(s);
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
          if (c0 + it * kRPP < rows) {
            const uint32_t mw = ld_ml(rs, c0 + it * kRPP)[0];
            g[it] = fmaxf(g[it], fl(mw));
          }
        }
      }
#pragma unroll
      for (int it = 0; it < kIt; ++it)
        if (g[it] == -INFINITY) g[it] = 0.f;  // (g_use)
      for (s = 0; s < S; ++s) {
        const __amdgpu_buffer_rsrc_t rm = rsrc_ml(s);
        const __amdgpu_buffer_rsrc_t ro = rsrc_o(s);
        u32x2 ml[kIt];
        u32x4 x[kIt];
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
          if (c0 + it * kRPP < rows) {
            ml[it] = ld_ml(rm, c0 + it * kRPP);
            x[it] = ld_o(ro, c0 + it * kRPP);
          }
        }
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
          if (c0 + it * kRPP < rows) {
            const uint32_t mw = ml[it][0], lw = ml[it][1];
            const float wgt = fast_exp2(fl(mw) - g[it]);
            lsum[it] += wgt * fl(lw);
            acc[it] += wgt * __builtin_bit_cast(f32x4, x[it]);
          }
        }
      }
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int r = c0 + it * kRPP;
      if (r >= rows || col >= a.dv) continue;
      const float inv = 1.f / lsum[it];  // 0/0 -> NaN for a row with no key, as the reference
      const int64_t off = o_base + static_cast<int64_t>(row0 + r) * a.o_ss + col;
      if constexpr (DT == FA2_DTYPE_F32) {
        *reinterpret_cast<f32x4*>(static_cast<float*>(a.o) + off) = acc[it] * inv;
      } else {
        constexpr bool BF = Elt<DT>::kBF;
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.o) + off) =
            (u32x2){pack2<BF>(acc[it][0] * inv, acc[it][1] * inv),
                    pack2<BF>(acc[it][2] * inv, acc[it][3] * inv)};
      }
    }
  }
}

// pieces in arbitrary part slots (slot_of(s), s < S)
template <int DT, int D, int NT, int MAXR, typename SlotOf>
__device__ __forceinline__ void merge_rows_at(const KArgs& a, SlotOf slot_of, int S, int rows,
                                              int64_t o_base, int row0) {
  if (S <= 2)
    merge_rows_sm<DT, D, NT, MAXR, 2>(a, slot_of, S, rows, o_base, row0);
  else if (S <= 4)
    merge_rows_sm<DT, D, NT, MAXR, 4>(a, slot_of, S, rows, o_base, row0);
  else
    merge_rows_sm<DT, D, NT, MAXR, 0>(a, slot_of, S, rows, o_base, row0);
}

// the splits of one unit: split s in slot s * part_slots + unit
template <int DT, int D, int NT, int MAXR>
__device__ __forceinline__ void merge_rows(const KArgs& a, int unit, int S, int rows,
                                           int64_t o_base, int row0) {
  const int64_t G = a.part_slots;
  merge_rows_at<DT, D, NT, MAXR>(
      a, [=](int s) { return static_cast<int64_t>(s) * G + unit; }, S, rows, o_base, row0);
}

// ---------------------------------------------------------------------------
// Plan kernel (ragged / paged): builds the (sequence, q-block) work list in
// descending order of KV tiles to process (longest-processing-time first),
// by a counting sort over tile counts (small decode batches: by ranking each
// sequence directly).  One workgroup; no host sync.
// ---------------------------------------------------------------------------
template <int MODE>
__device__ __forceinline__ void seq_lens(const KArgs& a, int b, int& Lq, int& Lk) {
  if constexpr (MODE == FA2_LAYOUT_RAGGED) {
    Lq = a.pack_m > 0 ? a.q_len : a.q_indptr[b + 1] - a.q_indptr[b];
    Lk = a.kv_indptr[b + 1] - a.kv_indptr[b];
  } else {
    Lq = a.q_len;
    Lk = a.kv_indptr[b];
  }
  if (Lq < 0) Lq = 0;
  if (Lk < 0) Lk = 0;
}

__device__ __forceinline__ int block_cost(int mask, int j, int Lq, int Lk, bool packed) {
  const int off = (mask == FA2_MASK_CAUSAL_BOTTOM_RIGHT) ? (Lk - Lq) : 0;
  const int e = packed ? Lk : kv_end_for_block(mask, j * kBM, Lq, Lk, off);
  const int tiles = (e + kBN - 1) / kBN;
  return tiles < kCostBuckets - 1 ? tiles : kCostBuckets - 1;
}

// Work items of a sequence with nq q-blocks: the q-blocks, or with
// KArgs::qpair the pairs (2j, 2j + 1), which cost what block 2j + 1 (or a
// lone last block 2j) costs.
__device__ __forceinline__ int plan_items(const KArgs& a, int nq) {
  return a.qpair ? (nq + 1) / 2 : nq;
}
__device__ __forceinline__ int plan_cost_block(const KArgs& a, int j, int nq) {
  return a.qpair ? min(2 * j + 1, nq - 1) : j;
}

// The item list and split count of a launch without a plan kernel
// (KArgs::inline_plan, batch <= kInlinePlanMaxBatch), called by all threads
// of the workgroup: the first wave writes the sequence offsets, the items of
// each sequence as the plan kernel counts them, their prefix sums and the
// plan kernel's split count (the host's heuristic with the longest KV sweep
// in place of its bound), then one barrier.
template <int MODE>
__device__ __forceinline__ void build_inline_plan(const KArgs& a, InlinePlan* ip) {
  static_assert(MODE == FA2_LAYOUT_RAGGED, "ragged launches only");
  // the first wave alone (kPer sequences per lane), one barrier for all
  constexpr int kPer = (kInlinePlanMaxBatch + 63) / 64;
  const int tid = threadIdx.x;
  if (tid < 64) {
    int qs[kPer + 1], ks[kPer + 1];
#pragma unroll
    for (int j = 0; j <= kPer; ++j) {
      const int t = min(tid * kPer + j, a.batch);
      qs[j] = a.q_indptr[t];
      ks[j] = a.kv_indptr[t];
    }
    int ni[kPer], sum = 0, cost = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int b = tid * kPer + j;
      const int Lq = max(qs[j + 1] - qs[j], 0);  // as seq_lens
      const int Lk = max(ks[j + 1] - ks[j], 0);
      const int nq = (Lq + a.block_rows - 1) / a.block_rows;
      ni[j] = b < a.batch ? plan_items(a, nq) : 0;
      if (ni[j] > 0)
        cost = max(cost, block_cost(a.mask, plan_cost_block(a, ni[j] - 1, nq), Lq, Lk,
                                    a.pack_m > 0));
      sum += ni[j];
      if (b <= a.batch) {
        ip->qi[b] = qs[j];
        ip->ki[b] = ks[j];
      }
    }
    int incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d);
      if (tid >= d) incl += y;
      cost = max(cost, __shfl_xor(cost, d));
    }
    int run = incl - sum;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int b = tid * kPer + j;
      run += ni[j];
      if (b < a.batch) ip->cum[b + 1] = run;
    }
    if (tid == 0) {
      ip->cum[0] = 0;
      ip->max_cost = cost;
      const int s = cost / kMinSplitTiles;
      ip->splits = !a.auto_splits ? a.num_splits : (s < 1 ? 1 : (s < a.num_splits ? s : a.num_splits));
    }
    if (tid == 63 && a.batch == 64 * kPer) {  // the end offsets of a full table
      ip->qi[a.batch] = qs[kPer];
      ip->ki[a.batch] = ks[kPer];
    }
  }
  __syncthreads();
}

// fp32 -> fp16 copies of q, k and v, rounded as the 16-bit kernels round
// fp32 operands (to16): flash_attention_v2 converts its fp32 inputs to fp16
// before every product (attention.py:547, 569, 621).  Segment i copies a
// [n0][n1][n2][D] view (element strides s0, s1, s2; dims contiguous) into a
// contiguous buffer; D / 8 threads per row, 8 elements each, one launch for
// all three.
struct ConvSeg {
  const float* src;
  int64_t s0, s1, s2;
  int32_t n1, n2;
  int64_t rows;
  uint16_t* dst;
};
struct ConvArgs {
  ConvSeg seg[3];
};
constexpr int kConvThreads = 256;
template <int D>
__global__ __launch_bounds__(kConvThreads) void fa2_to_f16_kernel(ConvArgs c) {
  constexpr int kTPR = D / 8;
  int64_t row = (static_cast<int64_t>(blockIdx.x) * kConvThreads + threadIdx.x) / kTPR;
  const int col = static_cast<int>(threadIdx.x % kTPR) * 8;  // kConvThreads % kTPR == 0
  int i = 0;
  while (i < 3 && row >= c.seg[i].rows) row -= c.seg[i++].rows;
  if (i == 3) return;
  const ConvSeg& g = c.seg[i];
  const int64_t i2 = row % g.n2, r1 = row / g.n2;
  const int64_t i1 = r1 % g.n1, i0 = r1 / g.n1;
  const float* p = g.src + i0 * g.s0 + i1 * g.s1 + i2 * g.s2 + col;
  Raw8<FA2_DTYPE_F32> r;
  r.w[0] = *reinterpret_cast<const u32x4*>(p);
  r.w[1] = *reinterpret_cast<const u32x4*>(p + 4);
  *reinterpret_cast<u32x4*>(g.dst + row * D + col) = to16<FA2_DTYPE_F32>(r);
}

template <int MODE>
__global__ __launch_bounds__(kPlanThreads) void fa2_plan_kernel(KArgs a, int2* work,
                                                                int32_t* work_count) {
  __shared__ int hist[kCostBuckets];
  __shared__ int seq_cost[kPlanThreads];  // the decode fast path's per-sequence costs
  const int tid = threadIdx.x;
  if (a.pack_m > 0 && a.q_len <= a.block_rows && a.batch <= kPlanFastBatch) {
    // Decode with one q-block per sequence and a small batch: item b's
    // position is its rank by cost (ties by sequence index), one pass.
    int c = 0;
    if (tid < a.batch) {
      int Lq, Lk;
      seq_lens<MODE>(a, tid, Lq, Lk);
      c = block_cost(a.mask, 0, Lq, Lk, true);
      seq_cost[tid] = c;
    }
    __syncthreads();
    if (tid < a.batch) {
      int rank = 0;
      for (int u = 0; u < a.batch; ++u) {
        const int cu = seq_cost[u];
        rank += (cu > c || (cu == c && u < tid)) ? 1 : 0;
      }
      if (rank < a.work_ub) work[rank] = make_int2(tid, 0);
    }
    if (tid == 0) *work_count = a.batch < a.work_ub ? a.batch : a.work_ub;
    return;
  }
  // Sequence-major list (claimed units): every sequence's items form one
  // run, heaviest first, and the runs are ordered by their heaviest item,
  // so the workgroups that claim consecutive units of a group share one
  // sequence's K/V in their L2.  An item's cost never decreases with its
  // q-block under any mask, so item j of n sits at n - 1 - j in its run.
  const bool seq_major = a.claim != nullptr;
  if (seq_major && tid < kXcds) a.claim[tid] = 0;
  __shared__ int max_cost;  // KV tiles of the heaviest item
  if (tid == 0) max_cost = 0;
  for (int i = tid; i < kCostBuckets; i += kPlanThreads) hist[i] = 0;
  __syncthreads();
  int lq0 = 0, lk0 = 0;  // this thread's first sequence, kept for the second pass
  for (int b = tid; b < a.batch; b += kPlanThreads) {
    int Lq, Lk;
    seq_lens<MODE>(a, b, Lq, Lk);
    if (b == tid) {
      lq0 = Lq;
      lk0 = Lk;
    }
    const int nq = (Lq + a.block_rows - 1) / a.block_rows;
    const int ni = plan_items(a, nq);
    if (ni > 0 && a.split_count)
      atomicMax(&max_cost,
                block_cost(a.mask, plan_cost_block(a, ni - 1, nq), Lq, Lk, a.pack_m > 0));
    if (seq_major) {
      if (ni > 0)
        atomicAdd(&hist[block_cost(a.mask, plan_cost_block(a, ni - 1, nq), Lq, Lk, false)], ni);
      continue;
    }
    for (int j = 0; j < ni; ++j)
      atomicAdd(&hist[block_cost(a.mask, plan_cost_block(a, j, nq), Lq, Lk, a.pack_m > 0)], 1);
  }
  __syncthreads();
  // the host's heuristic with the longest sweep in place of its bound
  if (tid == 0 && a.split_count) {
    const int s = max_cost / kMinSplitTiles;
    *a.split_count = s < 1 ? 1 : (s < a.num_splits ? s : a.num_splits);
  }
  // Exclusive scan in descending cost order: bucket c starts after all
  // buckets c' > c.  Thread t owns buckets [(P-1-t)*4, +4) from the top.
  // A scan inside each wave (lane shuffles), then over the wave totals:
  // two barriers.
  constexpr int kPer = kCostBuckets / kPlanThreads;
  constexpr int kPlanWaves = kPlanThreads / 64;
  __shared__ int wave_total[kPlanWaves];
  int local[kPer];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    local[i] = hist[kCostBuckets - 1 - (tid * kPer + i)];
    sum += local[i];
  }
  const int lane = tid & 63, wv = tid >> 6;
  int incl = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d);
    if (lane >= d) incl += y;
  }
  if (lane == 63) wave_total[wv] = incl;
  __syncthreads();
  if (wv == 0) {
    int t = lane < kPlanWaves ? wave_total[lane] : 0;
#pragma unroll
    for (int d = 1; d < kPlanWaves; d <<= 1) {
      const int y = __shfl_up(t, d);
      if (lane >= d) t += y;
    }
    if (lane < kPlanWaves) wave_total[lane] = t;  // inclusive
  }
  __syncthreads();
  int run = incl - sum + (wv > 0 ? wave_total[wv - 1] : 0);
  const int total = wave_total[kPlanWaves - 1];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    hist[kCostBuckets - 1 - (tid * kPer + i)] = run;  // becomes the cursor
    run += local[i];
  }
  __syncthreads();
  for (int b = tid; b < a.batch; b += kPlanThreads) {
    int Lq = lq0, Lk = lk0;
    if (b != tid) seq_lens<MODE>(a, b, Lq, Lk);
    const int nq = (Lq + a.block_rows - 1) / a.block_rows;
    const int ni = plan_items(a, nq);
    if (seq_major) {
      if (ni > 0) {
        const int pos0 = atomicAdd(
            &hist[block_cost(a.mask, plan_cost_block(a, ni - 1, nq), Lq, Lk, false)], ni);
        for (int j = 0; j < ni; ++j) {
          const int pos = pos0 + ni - 1 - j;
          if (pos < a.work_ub) work[pos] = make_int2(b, j);
        }
      }
      continue;
    }
    for (int j = 0; j < ni; ++j) {
      const int pos =
          atomicAdd(&hist[block_cost(a.mask, plan_cost_block(a, j, nq), Lq, Lk, a.pack_m > 0)], 1);
      if (pos < a.work_ub) work[pos] = make_int2(b, j);
    }
  }
  if (tid == 0) *work_count = total < a.work_ub ? total : a.work_ub;
}

}  // namespace fa2
