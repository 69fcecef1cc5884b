// fa2_kernel_lds.h - fp16/bf16 forward kernel with direct HBM->LDS tiles.
//
// Same math and work decomposition as the register-staged kernel in
// fa2_device.h (which remains the fp32 path), with the tile traffic moved
// off the VALU:
//   * K and V tiles are written to LDS by `buffer_load_dwordx4 ... lds`
//     (gfx950 direct-to-LDS, 16 bytes per lane): no staging registers, no
//     ds_write; out-of-range rows read as zeros through the buffer range
//     check (dense/ragged) or a range-violating offset (paged);
//   * rows are stored unpadded with an XOR swizzle of their 16-byte chunks,
//     chosen so that both the ds_read_b128 of K (one row per lane) and the
//     ds_read_b64_tr_b16 of V hit distinct banks;
//   * V stays row-major: ds_read_b64_tr_b16 transposes 4 keys x 16 dims per
//     16-lane group, so two of them give the V^T MFMA operand (one head dim
//     and 8 keys per lane) in the key order of the P^T fragment;
//   * the S MFMAs of tile t+1 share a basic block with the softmax of tile t.
#pragma once

#include "fa2_device.h"

namespace fa2 {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) char lds_char_t;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4_t;

// Row geometry and swizzles (16-byte chunk units) for a head dim D.
template <int D>
struct SwzGeo {
  static constexpr int kNC = D / 8;          // chunks per row
  static constexpr int kRowBytes = D * 2;
  static constexpr int kTileBytes = kBN * kRowBytes;
  // K rows are read one row per lane (16 lanes per bank cycle): 16 rows
  // must land on 16 distinct chunk slots of a 256-byte bank window.
  __device__ __forceinline__ static int k(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
  // V rows are read 4 rows x 4 chunks per 32 lanes by the transpose read.
  __device__ __forceinline__ static int v(int r) {
    return D == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2);
  }
};

// The same for fp32 rows (the fp32-arithmetic kernel, fa2_kernel_f32.h), D >= 64.
template <int D>
struct SwzGeo32 {
  static constexpr int kNC = D / 4;  // chunks per row
  static constexpr int kRowBytes = D * 4;
  static constexpr int kTileBytes = kBN * kRowBytes;
  static_assert(kNC >= 16, "fp32 rows of at least 64 dims");
  // K is read one row per lane (16 lanes per pass): 16 rows at one chunk
  // column go to 16 distinct 16-byte bank groups.
  __device__ __forceinline__ static int k(int r) { return r & 15; }
  // V is read one dim per lane, keys r (lanes 0-31) and r + 4 (lanes 32-63):
  // the two rows' 128-byte runs land on opposite halves of the 64 banks.
  __device__ __forceinline__ static int v(int r) { return ((r >> 2) & 1) << 3; }
};

__device__ __forceinline__ lds_char_t* to_lds(void* p) {
  return (lds_char_t*)((__attribute__((address_space(3))) uint16_t*)(uint16_t*)p);
}

// Direct-to-LDS loads are issued through inline asm: the compiler then does
// not see an asynchronous LDS write and cannot serialise every later LDS read
// behind it (it cannot tell the double-buffer halves apart).  Completion is
// awaited explicitly by lds_fill_barrier() before the buffer is read; the
// waits the compiler emits for its own loads only get more conservative
// (vector-memory loads retire in order).  No "memory" clobber: the target
// buffer is not read before the next barrier (volatile asm is not moved
// across it), the source K/V is never written, and without the clobber the
// block-table reads stay eligible for the scalar unit.
//
// M0 (the LDS destination of these loads) is an operand of the statement, so
// the compiler writes it and knows it is read; its hazard recognizer does not
// look inside inline asm, so the wait states gfx950 needs before the load are
// written out (the counts hipcc emits around the equivalent builtins):
//   * a VALU write of an SGPR (v_readfirstlane / v_readlane, which produce
//     the descriptor words and restore spilled SGPRs) followed by a vector
//     memory instruction that reads that SGPR: 5 wait states (s_nop 4);
//   * an SALU write of M0 followed by a load to LDS: 1 (s_nop 0).
//
// NT selects the non-temporal cache policy (`nt`), for data that the launch
// reads once (decode's K/V: +2 % on d1, d2 and s1).  Prefill keeps the default:
// its K/V tiles are read again by the other units of a kv head from L2
// (`nt` there measured c3 -4.6 %, c2 -1.6 %).
template <bool NT = false>
__device__ __forceinline__ void dma_buffer_x4(u32x4 rsrc, uint32_t lds_addr, uint32_t voff) {
  if constexpr (NT)
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
                 :
                 : "v"(voff), "s"(rsrc),
                   "{m0}"(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_addr))));
  else
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rsrc),
                   "{m0}"(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_addr))));
}

template <bool NT = false>
__device__ __forceinline__ void dma_global_x4(const void* gptr, uint32_t lds_addr) {
  if constexpr (NT)
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(gptr), "{m0}"(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_addr))));
  else
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gptr), "{m0}"(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_addr))));
}

// One 32-bit read of read-only global memory at a wave-uniform address through
// the scalar unit (the block table is written before the kernel starts; the
// scalar cache is invalidated at launch).
__device__ __forceinline__ int scalar_load_i32(const int32_t* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a)));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32)));
  const uint64_t sa = (static_cast<uint64_t>(hi) << 32) | lo;
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(sa));
  return v;
}

// Buffer descriptor as four SGPR words (base, stride 0, num_records, flags).
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t w0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b)));
  const uint32_t w1 = static_cast<uint32_t>(
      __builtin_amdgcn_readfirstlane(static_cast<int>((b >> 32) & 0xFFFFu)));
  const uint32_t w2 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(bytes)));
  return (u32x4){w0, w1, w2, static_cast<uint32_t>(kBufferFlags)};
}

__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(to_lds(const_cast<void*>(p))));
}

// LDS pointer at byte address `addr` (an integer conversion: the LDS null
// pointer is 0xFFFFFFFF, so offsets must not be added to a converted null).
__device__ __forceinline__ lds_char_t* lds_ptr(uint32_t addr) {
  return (lds_char_t*)(static_cast<uintptr_t>(addr));
}

// Tile loads shared by NW waves (each issues kInstr 1 KiB instructions);
// NT: non-temporal loads (see dma_buffer_x4).
template <int D, int MODE, bool BUF, int DT, int NW = kWaves, bool NT = false>
struct DirectLoader {
  using G = std::conditional_t<DT == FA2_DTYPE_F32, SwzGeo32<D>, SwzGeo<D>>;
  static constexpr int kEB = Elt<DT>::kBytes;
  static constexpr int kInstr = G::kNC / NW;  // 1 KiB wave instructions per tensor per tile
  static_assert(kInstr * NW == G::kNC, "tile must split evenly over the loading waves");
  static_assert(kInstr >= 1, "head dim");
  // fp32 tiles of 64 dims also serve head_dim 16 and 32 (KArgs::dv): the
  // chunks past dv are zero-filled, never read from memory
  static constexpr bool kDV = DT == FA2_DTYPE_F32 && D == 64;

  // dense/ragged: byte offset (row * stride + swizzled chunk) of this lane's
  // slot for instruction j, relative to the tile's first row (paged: to the
  // first row of the instruction).  fp32 tiles (kLazy) compute them when
  // issuing instead of holding 2 * kInstr registers through the kernel.
  static constexpr bool kLazy = DT == FA2_DTYPE_F32;
  uint32_t kvo[kLazy ? 1 : kInstr], vvo[kLazy ? 1 : kInstr];
  uint32_t krs, vrs;  // row strides in bytes
  int wave, lane;
  // bit j: the source chunk this lane loads with instruction j holds data
  // (head dims below dv); only tracked when kDV
  uint32_t kmask, vmask;
  __device__ __forceinline__ bool kok(int j) const { return !kDV || ((kmask >> j) & 1u); }
  __device__ __forceinline__ bool vok(int j) const { return !kDV || ((vmask >> j) & 1u); }
  template <bool IS_V>
  __device__ __forceinline__ bool cok(int j) const { return IS_V ? vok(j) : kok(j); }

  // byte offset of this lane's slot for instruction j: dense/ragged from
  // the tile's first row; paged from the first row of the instruction's
  // kRPI-row group (its page row is added by the caller)
  template <bool IS_V>
  __device__ __forceinline__ uint32_t offset(int j) const {
    const int r = row_of(j);
    const int rr = (MODE == FA2_LAYOUT_PAGED) ? lane_row() : r;
    return rr * (IS_V ? vrs : krs) + ((slot_of() ^ (IS_V ? G::v(r) : G::k(r))) * 16);
  }
  template <bool IS_V>
  __device__ __forceinline__ uint32_t src_off(int j) const {
    if constexpr (kLazy) return offset<IS_V>(j);
    else return IS_V ? vvo[j] : kvo[j];
  }

  // tile row and 16-byte slot of this lane for wave instruction j
  __device__ __forceinline__ int row_of(int j) const {
    return ((wave * kInstr + j) * 64 + lane) / G::kNC;
  }
  __device__ __forceinline__ int slot_of() const { return lane % G::kNC; }

  // tile rows covered by one wave instruction, and this lane's row among them
  static constexpr int kRPI = 64 / G::kNC;
  // consecutive tile rows covered by one wave's kInstr instructions
  static constexpr int kSpan = kInstr * kRPI;
  __device__ __forceinline__ int lane_row() const { return lane / G::kNC; }

  __device__ __forceinline__ DirectLoader(const KArgs& a, int tid)
      : DirectLoader(a, __builtin_amdgcn_readfirstlane(tid >> 6), tid & 63) {}

  // wv: index of this wave among the NW loading waves
  __device__ __forceinline__ DirectLoader(const KArgs& a, int wv, int ln) {
    wave = wv;
    lane = ln;
    kmask = vmask = 0u;
    krs = static_cast<uint32_t>(a.k_ss * kEB);
    vrs = static_cast<uint32_t>(a.v_ss * kEB);
#pragma unroll
    for (int j = 0; j < kInstr; ++j) {
      const int r = row_of(j);
      if constexpr (!kLazy) {
        kvo[j] = offset<false>(j);
        vvo[j] = offset<true>(j);
      }
      if constexpr (kDV) {
        constexpr int kPerChunk = 16 / kEB;  // elements per 16-byte chunk
        kmask |= static_cast<uint32_t>((slot_of() ^ G::k(r)) * kPerChunk < a.dv) << j;
        vmask |= static_cast<uint32_t>((slot_of() ^ G::v(r)) * kPerChunk < a.dv) << j;
      }
    }
  }

  // Physical row of logical row n0 (uniform across the wave) and whether the
  // kRPI rows n0.. share its page (page_size a multiple of kRPI): then one
  // scalar table read serves the whole instruction.
  __device__ __forceinline__ static int paged_row_uniform(const KArgs& a, const int32_t* table,
                                                          int64_t tstride, int b, int n) {
    int pidx, poff;
    if (a.page_shift >= 0) {
      pidx = n >> a.page_shift;
      poff = n & (a.page_size - 1);
    } else {
      pidx = n / a.page_size;
      poff = n - pidx * a.page_size;
    }
    // The index is wave-uniform: read the entry with a scalar load (SMEM,
    // counted by lgkmcnt, so it never waits behind the K/V DMAs in vmcnt).
    const int idx = __builtin_amdgcn_readfirstlane(static_cast<int>(b * tstride + pidx));
    return scalar_load_i32(table + idx) * a.page_size + poff;
  }

  // Callers that read the table ahead of its use (decode producers): true
  // when one table entry serves each wave's kSpan rows of a tile.
  __device__ __forceinline__ static bool uniform_pages(const KArgs& a) {
    return MODE == FA2_LAYOUT_PAGED && a.page_size % kSpan == 0;
  }

  // Descriptor of `rows` cache rows starting at physical row `prow` of the
  // pool at `pool` (64-bit base on the scalar unit, so the pool may exceed
  // the 32-bit offset range).  A row outside the pool (when its size is
  // known: kv_len > 0) gets an empty range: the loads return zeros instead
  // of reading outside the allocation.
  __device__ __forceinline__ static u32x4 page_rsrc(const KArgs& a, const char* pool, int prow,
                                                    int rows, uint32_t rsb) {
    const bool inside = prow >= 0 && (a.kv_len <= 0 || prow <= a.kv_len - rows);
    const char* base = pool + (inside ? static_cast<int64_t>(prow) * rsb : 0);
    return rsrc_words(base, inside ? static_cast<uint32_t>(rows) * rsb : 0u);
  }

  // Block-table entry of this wave's first row of the tile at k0, through a
  // constant-address-space load: a scalar load whose wait the compiler
  // places at the first use, so it can be issued a tile ahead (the entry is
  // returned raw; issue_at turns it into a row).
  __device__ __forceinline__ int prefetch_page(const KArgs& a, const Work& w, int k0,
                                               bool is_v) const {
    typedef __attribute__((address_space(4))) const int32_t const_i32_t;
    const int n = min(k0 + wave * kSpan, w.Lk - 1);
    const int pidx = a.page_shift >= 0 ? (n >> a.page_shift) : n / a.page_size;
    const int32_t* tbl = is_v ? a.v_table : a.k_table;
    const int64_t ts = is_v ? a.v_table_stride : a.k_table_stride;
    const int idx = __builtin_amdgcn_readfirstlane(static_cast<int>(w.b * ts + pidx));
    return ((const_i32_t*)tbl)[idx];
  }

  // issue<IS_V> for uniform_pages() with the table entry from prefetch_page.
  template <bool IS_V>
  __device__ __forceinline__ void issue_at(const KArgs& a, const Work& w, int k0, void* dst,
                                           int page) const {
    const void* src = IS_V ? a.v : a.k;
    const int64_t base = IS_V ? w.v_base : w.k_base;
    const uint32_t ldst = lds_addr_of(dst) + wave * kInstr * 1024;
    const uint32_t rsb = static_cast<uint32_t>((IS_V ? a.v_ss : a.k_ss) * kEB);
    const int n0 = k0 + wave * kSpan;
    const int nc = min(n0, w.Lk - 1);
    const int poff = a.page_shift >= 0 ? (nc & (a.page_size - 1)) : nc % a.page_size;
    const int prow = __builtin_amdgcn_readfirstlane(page * a.page_size + poff);
    const u32x4 rsrc =
        page_rsrc(a, static_cast<const char*>(src) + base * kEB, prow, kSpan, rsb);
#pragma unroll
    for (int j = 0; j < kInstr; ++j) {
      const uint32_t off = j * kRPI * rsb + src_off<IS_V>(j);
      dma_buffer_x4<NT>(rsrc, ldst + j * 1024,
                        (n0 + j * kRPI + lane_row() < w.Lk && cok<IS_V>(j)) ? off : 0xFFFFFF00u);
    }
  }

  __device__ __forceinline__ static int paged_row(const int32_t* table, int64_t tstride, int b,
                                                  int n, int page) {
    const int pg = table[b * tstride + n / page];
    return pg * page + (n % page);
  }

  // Issue the loads of one tile of K (IS_V=false) or V into `dst`.
  // Dense/ragged: one descriptor per tile, based at the tile's first row and
  // covering only its rows inside the sequence (rows past the end read as
  // zeros).  Paged with page_size a multiple of the rows one wave (kSpan) or
  // one instruction (kRPI) covers: one scalar table read and one descriptor
  // per wave or per instruction, based at that physical row.  Every
  // descriptor has a 64-bit base and a small range, so the size of the
  // tensor or pool is not limited by the 32-bit buffer offsets.  Other page
  // sizes look up every lane's row: through 32-bit offsets from the pool
  // base when the pool fits them (BUF), else through 64-bit addresses.
  template <bool IS_V>
  __device__ __forceinline__ void issue(const KArgs& a, const Work& w, int k0, void* dst) const {
    const void* src = IS_V ? a.v : a.k;
    const int64_t rs = IS_V ? a.v_ss : a.k_ss;
    const int64_t base = IS_V ? w.v_base : w.k_base;
    const uint32_t ldst = lds_addr_of(dst) + wave * kInstr * 1024;
    const uint32_t rsb = static_cast<uint32_t>(rs * kEB);
    if constexpr (MODE == FA2_LAYOUT_PAGED) {
      const char* pool = static_cast<const char*>(src) + base * kEB;
      const int32_t* tbl = IS_V ? a.v_table : a.k_table;
      const int64_t ts = IS_V ? a.v_table_stride : a.k_table_stride;
      if (a.page_size % kSpan == 0) {
        // the wave's kSpan rows (starting at a multiple of kSpan) lie in
        // one page: one table read for all its instructions
        const int n0 = k0 + wave * kSpan;  // uniform
        const int prow = paged_row_uniform(a, tbl, ts, w.b, min(n0, w.Lk - 1));
        const u32x4 rsrc = page_rsrc(a, pool, prow, kSpan, rsb);
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
          const uint32_t off = j * kRPI * rsb + src_off<IS_V>(j);
          dma_buffer_x4<NT>(rsrc, ldst + j * 1024,
                            (n0 + j * kRPI + lane_row() < w.Lk && cok<IS_V>(j)) ? off : 0xFFFFFF00u);
        }
      } else if (a.page_size % kRPI == 0) {
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
          const int n0 = k0 + (wave * kInstr + j) * kRPI;  // uniform
          const int prow = paged_row_uniform(a, tbl, ts, w.b, min(n0, w.Lk - 1));
          const u32x4 rsrc = page_rsrc(a, pool, prow, kRPI, rsb);
          const uint32_t off = src_off<IS_V>(j);
          dma_buffer_x4<NT>(rsrc, ldst + j * 1024,
                            (n0 + lane_row() < w.Lk && cok<IS_V>(j)) ? off : 0xFFFFFF00u);
        }
      } else if constexpr (BUF) {
        const u32x4 rsrc = rsrc_words(pool, IS_V ? a.pool_bytes_v : a.pool_bytes_k);
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
          const int r = row_of(j);
          const int n = k0 + r;
          const int nc = min(n, w.Lk - 1);
          const uint32_t prow = static_cast<uint32_t>(paged_row(tbl, ts, w.b, nc, a.page_size));
          const uint32_t col = (slot_of() ^ (IS_V ? G::v(r) : G::k(r))) * 16;
          dma_buffer_x4<NT>(rsrc, ldst + j * 1024,
                            (n < w.Lk && cok<IS_V>(j)) ? prow * rsb + col : 0xFFFFFF00u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
          const int r = row_of(j);
          const int n = min(k0 + r, w.Lk - 1);  // clamped: finite data, masked later
          const int64_t prow = paged_row(tbl, ts, w.b, n, a.page_size);
          // (a chunk past dv reads the row's first chunk instead: finite data
          // that meets zero q dims, or V columns that are never stored)
          const uint32_t col =
              cok<IS_V>(j) ? (slot_of() ^ (IS_V ? G::v(r) : G::k(r))) * 16 : 0u;
          dma_global_x4<NT>(pool + prow * rs * kEB + col, ldst + j * 1024);
        }
      }
    } else {
      // rows past the sequence read as zeros (a tile wholly past it: none)
      const uint32_t lim = static_cast<uint32_t>(min(max(w.Lk - k0, 0), kBN)) * rsb;
      const u32x4 rsrc = rsrc_words(
          static_cast<const char*>(src) + (base + static_cast<int64_t>(k0) * rs) * kEB, lim);
#pragma unroll
      for (int j = 0; j < kInstr; ++j)
        dma_buffer_x4<NT>(rsrc, ldst + j * 1024,
                          cok<IS_V>(j) ? src_off<IS_V>(j) : 0xFFFFFF00u);
    }
  }
};

typedef __attribute__((address_space(3))) u32x2 lds_u32x2_t;

// Output rows go out through LDS: in the O^T accumulator a lane holds 4
// dims of one row per register group, so direct stores write 8-byte pieces
// of 32 different rows per instruction.  Each wave instead writes its 32 x D
// tile (normalised, rounded) into its own LDS region and reads it back as
// whole rows: every global store then covers 16-byte chunks of complete rows.
template <int D>
struct OStage {
  static constexpr int kStride = D * 2 + 16;  // row pitch; the pad spreads banks
  static constexpr int kBytes = kWaveRows * kStride;
};

// o: this wave's O^T accumulators (row l32, dims 32d + 8g + 4hi + j at
// o[d][4g + j]); inv: 1 / row sum of this lane's row; stage: the wave's
// region of OStage<D>::kBytes; rows row0.. of the output at `base`, only
// rows < Lq are stored.
template <int DT, int D>
__device__ __forceinline__ void store_o_staged(const f32x16 (&o)[D / 32], float inv, char* stage,
                                               void* out, int64_t base, int64_t o_ss, int row0,
                                               int Lq, int lane) {
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int kS = OStage<D>::kStride;
  constexpr int kChunks = D / 8;              // 16-byte chunks per row
  constexpr int kRowsPerRead = 64 / kChunks;  // rows covered by one wave read
  const int l32 = lane & 31, hi = lane >> 5;
  lds_char_t* st = to_lds(stage);
#pragma unroll
  for (int d = 0; d < D / 32; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *(lds_u32x2_t*)(st + l32 * kS + (d * 32 + g * 8 + hi * 4) * 2) =
          (u32x2){pack2<BF>(o[d][g * 4 + 0] * inv, o[d][g * 4 + 1] * inv),
                  pack2<BF>(o[d][g * 4 + 2] * inv, o[d][g * 4 + 3] * inv)};
  const int ch = lane % kChunks;
#pragma unroll
  for (int it = 0; it < kWaveRows / kRowsPerRead; ++it) {
    const int r = it * kRowsPerRead + lane / kChunks;
    const u32x4 v = *(const lds_u32x4_t*)(st + r * kS + ch * 16);
    if (row0 + r < Lq)
      __builtin_nontemporal_store(
          v, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + base +
                                      static_cast<int64_t>(row0 + r) * o_ss + ch * 8));
  }
}

// Cache policy of the output stores: non-temporal (`nt`).  Nothing in the
// launch reads the output back, and streaming it out of L2 leaves fewer dirty
// lines for the write-back at the end of the kernel.  Measured in alternating
// runs on one box: c2 (74 us launches) +1 to +8 % per step, c3, c4 and c5
// (0.4 to 1 ms launches) unchanged.
constexpr int kStoreNT = 2;

// The same through buffer stores in passes of DP dims (stage: OStage<DP>
// bytes).  The descriptor `out` starts at row row0 of the tile and covers
// only the rows < Lq, which the hardware range check enforces: every store
// instruction is issued whatever the row count (a fixed vmcnt contribution
// of kOStoreOps<D, DP> per lane).
template <int D, int DP>
constexpr int kOStoreOps = (D / DP) * (kWaveRows * DP / 512);

template <int DT, int D, int DP>
__device__ __forceinline__ void store_o_staged_buf(const f32x16 (&o)[D / 32], float inv,
                                                   char* stage, __amdgpu_buffer_rsrc_t out,
                                                   int64_t o_ss, int lane) {
  static_assert(D % DP == 0 && DP % 32 == 0, "pass width");
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int kS = OStage<DP>::kStride;
  constexpr int kChunks = DP / 8;             // 16-byte chunks per staged row
  constexpr int kRowsPerRead = 64 / kChunks;  // rows covered by one wave read
  const int l32 = lane & 31, hi = lane >> 5;
  const uint32_t rs = static_cast<uint32_t>(o_ss * 2);
  lds_char_t* st = to_lds(stage);
  const int ch = lane % kChunks;
#pragma unroll
  for (int p = 0; p < D / DP; ++p) {
#pragma unroll
    for (int dd = 0; dd < DP / 32; ++dd) {
      const int d = p * (DP / 32) + dd;
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(lds_u32x2_t*)(st + l32 * kS + (dd * 32 + g * 8 + hi * 4) * 2) =
            (u32x2){pack2<BF>(o[d][g * 4 + 0] * inv, o[d][g * 4 + 1] * inv),
                    pack2<BF>(o[d][g * 4 + 2] * inv, o[d][g * 4 + 3] * inv)};
    }
    // all reads of the pass first, then the stores back to back
    constexpr int kIt = kWaveRows / kRowsPerRead;
    u32x4 v[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int r = it * kRowsPerRead + lane / kChunks;
      v[it] = *(const lds_u32x4_t*)(st + r * kS + ch * 16);
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int r = it * kRowsPerRead + lane / kChunks;
      __builtin_amdgcn_raw_buffer_store_b128(v[it], out, r * rs + (p * DP + ch * 8) * 2, 0,
                                             kStoreNT);
    }
  }
}

// Wait for this wave's outstanding direct-to-LDS loads (vmcnt), then barrier.
__device__ __forceinline__ void lds_fill_barrier() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

#ifndef FA2_LDS_OCCUPANCY
#define FA2_LDS_OCCUPANCY 2
#endif
// PIPE: K runs two tiles ahead and the S MFMAs of tile t+1 are interleaved
// (sched_group_barrier, FA2_SGB VALU instructions per MFMA) with the softmax
// of tile t in one basic block; otherwise K runs one tile ahead and S(t)
// starts step t.  Measured on MI355X, bf16 D=128 (same run): c2 625 -> 675,
// c5 960 -> 1010 TFLOP/s for plain -> pipelined+interleaved.
#ifndef FA2_LDS_PIPE
#define FA2_LDS_PIPE 1
#endif
#define FA2_LDS_PIPE_DEFAULT(D) (FA2_LDS_PIPE != 0 && (D) <= 128)
#ifndef FA2_SGB
#define FA2_SGB 7
#endif
template <int DT, int D, int MODE, bool BUF, bool PIPE = FA2_LDS_PIPE_DEFAULT(D)>
__global__ __launch_bounds__(kThreads, D > 128 ? 1 : FA2_LDS_OCCUPANCY) void fa2_fwd_lds_kernel(KArgs a) {
  static_assert(DT != FA2_DTYPE_F32, "fp32 uses the register-staged kernel");
  constexpr bool BF = Elt<DT>::kBF;
  constexpr int DC = D / 16;  // MFMA k-steps of S (16 head dims each)
  constexpr int DB = D / 32;  // 32-dim blocks of O^T
  constexpr int SB = kBN / 32;
  using G = SwzGeo<D>;

  __shared__ __attribute__((aligned(1024))) char lds[4 * G::kTileBytes];
  // K buffers 0, 1 then V buffers 0, 1 (addresses computed, not read from an
  // array of LDS pointers, which a loop-carried index cannot select)
  auto kbuf = [&](int j) { return lds + (j & 1) * G::kTileBytes; };
  auto vbuf = [&](int j) { return lds + (2 + (j & 1)) * G::kTileBytes; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  // a ragged launch without a plan kernel: the item list in LDS
  const InlinePlan* ip = nullptr;
  if constexpr (MODE == FA2_LAYOUT_RAGGED) {
    __shared__ InlinePlan iplan;
    if (a.inline_plan) {
      build_inline_plan<MODE>(a, &iplan);
      ip = &iplan;
    }
  }
  const Work w = decode_work<MODE>(a, blockIdx.x, 1, ip);
  if (!w.valid) return;
  const int q0 = w.qblk * kBM;
  const int split = blockIdx.y;
  const int S = ip ? ip->splits : launch_splits(a);
  if (split >= S) return;

  const int kv_end = kv_end_for_unit(a, q0, w.Lq, w.Lk, w.off);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const int t_begin = (ntiles * split) / S;
  const int t_end = (ntiles * (split + 1)) / S;
  const int T = t_end - t_begin;

  // Q^T fragments (B operand of S^T = K Q^T): query row q0+32*wave+l32.
  const int qrow = q0 + wave * kWaveRows + l32;
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

  // Per-lane LDS byte offsets.  K (A operand of S^T): row sb*32 + l32, chunk
  // 2*cc + hi.  Both row blocks share the swizzle (32 = 0 mod 16 rows).
  // The swizzle only flips chunk bits, i.e. address bits below the row
  // offset, so offset(cc) = offset(0) ^ (32 * cc) for K and
  // offset(db) = offset(0) ^ (64 * db) for V (one register each).
  const uint32_t koff0 = l32 * G::kRowBytes + ((hi ^ G::k(l32)) * 16);
  // V (A operand of O^T via the transpose read): source lane i of 16-lane
  // group g reads row 16c + 8rr + 4*(g/2) + i/4, dims 32db + 16(g%2) + 4(i%4).
  uint32_t voff0;
  {
    const int g = lane >> 4, i = lane & 15;
    const int r = 4 * (g >> 1) + (i >> 2);  // + 16c + 8rr (multiples of 8: same swizzle)
    const int dim = 16 * (g & 1) + 4 * (i & 3);
    voff0 = r * G::kRowBytes + (((dim >> 3) ^ G::v(r)) * 16) + (dim & 7) * 2;
  }

  f32x16 o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = (f32x16){};
  float m_run = -INFINITY;
  float l_run = 0.f;
  // first row of the wave; its rows' smallest diagonal position and this lane's
  const int wq_first = q0 + wave * kWaveRows;
  const int wq_diag = a.pack_m > 0 ? 0 : wq_first;
  const int qdiag = diag_row(a, qrow);
  const bool causal = a.mask != FA2_MASK_NONE;
  // A wave whose 32 rows all lie past the unit's end (small packed-head
  // units, the last q-block of a sequence) only loads tiles and keeps the
  // barriers; it computes nothing.
  const bool active = q0 + wave * kWaveRows < w.Lq;

  const DirectLoader<D, MODE, BUF, DT> ld(a, tid);

  // (no s_setprio here: it would end the scheduling region and undo the
  // interleaving of these MFMAs with the softmax)
  auto compute_s = [&](f32x16 (&s)[SB], const char* kb) {
    const lds_char_t* kl = to_lds(const_cast<char*>(kb));
    // accumulators interleaved (cc-major): back-to-back dependent MFMAs stall
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
  };

  auto step = [&](auto last, int i, f32x16 (&s_cur)[SB], f32x16 (&s_nxt)[SB]) {
    constexpr bool kLast = decltype(last)::value;
    const int t = t_begin + i;
    const int k0 = t * kBN;
    if constexpr (!kLast) {
      if (PIPE ? (i + 2 < T) : true)
        ld.template issue<false>(a, w, k0 + (PIPE ? 2 : 1) * kBN, kbuf((PIPE ? i : i + 1) & 1));
      ld.template issue<true>(a, w, k0 + kBN, vbuf((i + 1) & 1));
    }
    if (active) {
    // scores of tile i must exist before they are masked
    if constexpr (!PIPE) compute_s(s_cur, kbuf(i & 1));
    if ((k0 + kBN > w.Lk) || (causal && (k0 + kBN - 1 > wq_diag + w.off))) {
      // key = k0 + 4*hi + c with c a compile-time offset per accumulator:
      // visible iff c <= lim (sequence end and, if causal, the diagonal)
      int lim = w.Lk - 1 - k0 - hi * 4;
      if (causal) lim = min(lim, qdiag + w.off - k0 - hi * 4);
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
          const int c = sb * 32 + (i2 >> 2) * 8 + (i2 & 3);
          if (c > lim) s_cur[sb][i2] = -INFINITY;
        }
      }
    }
    if constexpr (!kLast && PIPE) compute_s(s_nxt, kbuf((i + 1) & 1));

    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < SB; ++sb)
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) mx = fmaxf(mx, s_cur[sb][i2]);
    mx = max_xor32(mx);
    const float mt = mx * a.scale_log2;
    const bool need = mt > m_run + kRescaleThreshold;
    // branch-free (exp2(0) = 1) so the whole softmax stays one basic block
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
        p[i2] = fast_exp2(__builtin_fmaf(s_cur[sb][i2], a.scale_log2, -m_use));
#pragma unroll
      for (int half = 0; half < 2; ++half)
        pf[sb * 2 + half] = (u32x4){pack2<BF>(p[half * 8 + 0], p[half * 8 + 1]),
                                    pack2<BF>(p[half * 8 + 2], p[half * 8 + 3]),
                                    pack2<BF>(p[half * 8 + 4], p[half * 8 + 5]),
                                    pack2<BF>(p[half * 8 + 6], p[half * 8 + 7])};
    }
    // row sum of the rounded P, i.e. of exactly the weights the PV MFMA
    // applies: one v_dot2 (x . (1,1) + acc, fp32 accumulate) per packed pair
    float rs = 0.f;
#pragma unroll
    for (int c = 0; c < kBN / 16; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) rs = dot2_ones<BF>(pf[c][j], rs);
    l_run = l_run * alpha + rs;
#if FA2_SGB > 0
    // Interleave the S(t+1) MFMAs with the softmax VALU work of tile t inside
    // this basic block, with the K fragment reads running kReadAhead MFMAs
    // ahead so that no MFMA waits on a just-issued LDS read:
    //   R x kReadAhead, then per MFMA: 1 MFMA, N VALU, 1 R (for MFMA k + ahead)
    if constexpr (PIPE && !kLast) {
      constexpr int kN = SB * DC;
      constexpr int kAhead = kReadAhead < kN ? kReadAhead : kN;
      __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
      for (int k = 0; k < kN; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, FA2_SGB, 0);
        if (k + kAhead < kN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
#endif
    // The rescale branch is rarely taken; tying its condition to the row sum
    // (never -1) keeps the compiler from hoisting it above the exps, which
    // would split the MFMA/softmax block in two.
    if (__any(need) && rs != -1.0f) {
#pragma unroll
      for (int d = 0; d < DB; ++d) o[d] *= alpha;
    }
    // O^T += V^T P^T; V^T fragments from two transposed reads per MFMA
    const lds_char_t* vl = to_lds(vbuf(i & 1));
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
#if FA2_SGB > 0
    {
      // V reads run kReadAhead MFMAs ahead of the PV MFMAs (2 reads each)
      constexpr int kN = DB * (kBN / 16);
      constexpr int kAhead = kReadAhead < kN ? kReadAhead : kN;
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * kAhead, 1);
#pragma unroll
      for (int k = 0; k < kN; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        if (k + kAhead < kN) __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      }
    }
#endif
    }  // active
    if constexpr (!kLast) lds_fill_barrier();
  };
  using NotLast = std::integral_constant<bool, false>;
  using Last = std::integral_constant<bool, true>;

  f32x16 sA[SB], sB[SB];
  if (T > 0) {
    ld.template issue<false>(a, w, t_begin * kBN, kbuf(0));
    ld.template issue<true>(a, w, t_begin * kBN, vbuf(0));
    if (PIPE && T > 1) ld.template issue<false>(a, w, (t_begin + 1) * kBN, kbuf(1));
    lds_fill_barrier();
    if constexpr (PIPE) {
      if (active) compute_s(sA, kbuf(0));
      // step 0 refills kbuf(0) with K(t0+2): every wave must have finished
      // reading K(t0) first (the barrier also waits for the LDS reads)
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
    static_assert(kWaves * OStage<D>::kBytes <= sizeof(lds), "O staging exceeds LDS");
    __syncthreads();  // the last tile's buffers may still be read by other waves
    const float inv = 1.f / l_tot;  // 0/0 -> NaN for a row with no key, as the reference
    store_o_staged<DT, D>(o, inv, lds + wave * OStage<D>::kBytes, a.o, w.o_base, a.o_ss,
                          wq_first, w.Lq, lane);
  } else {
    // only rows the merge reads (r < part_rows, q0 + r < Lq) are written
    const int64_t slot = static_cast<int64_t>(split) * a.part_slots + blockIdx.x;
    const int r = wave * kWaveRows + l32;
    if (qrow < w.Lq && r < a.part_rows) {
      if (MODE == FA2_LAYOUT_RAGGED && a.merge_ctr)
        store_partial_rows<true, D>(a, slot, r, hi, m_run, l_tot, o);
      else
        store_partial_rows<false, D>(a, slot, r, hi, m_run, l_tot, o);
    }
    // (only ragged launches merge here: KArgs::inline_plan)
    if (MODE == FA2_LAYOUT_RAGGED && a.merge_ctr) {  // the split that completes the count merges
      __shared__ int merge_flag;
      merge_publish();
      __syncthreads();
      if (merge_count(a, blockIdx.x, S, &merge_flag))
        merge_rows<DT, D, kThreads, kBM>(a, blockIdx.x, S, min(a.part_rows, w.Lq - q0), w.o_base,
                                    q0);
    }
  }
}

}  // namespace fa2
