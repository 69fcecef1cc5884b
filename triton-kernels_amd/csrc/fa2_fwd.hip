// fa2_fwd.hip - C ABI and launch logic of the gfx950 flash_attention_v2
// forward pass (declared in include/fa2.h).
//
// Replaces the host half of harsh-vsingh/triton-kernels
// kernels/attention.py:836-925: split heuristic (:836-841), workspace
// (:852-864) and the partial + merge launches (:882-925).  Differences:
//   * when the grid already fills the GPU no split is made and the forward
//     kernel writes O directly (the reference always writes fp32 partials and
//     launches a merge, even for split_k == 1);
//   * ragged/paged schedules come from a device-side plan kernel, so there is
//     no `.item()` host synchronisation (attention.py:847);
//   * no allocation: the caller passes the workspace.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <random>

#include "fa2_device.h"
#include "fa2_kernel_lds.h"
#include "fa2_kernel_pp.h"
#include "fa2_kernel_short.h"
#include "fa2_kernel_decode.h"
#include "fa2_kernel_decode_f32.h"
#include "fa2_kernel_f32.h"
#include "fa2_kv_append.h"

// 1: fp16/bf16 with an even number of query heads per kv head run the
// two-head ping-pong kernel; 0: always the one-head kernel.
#ifndef FA2_PP
#define FA2_PP 1
#endif
// 1: the two-head kernel runs one workgroup per CU over all units
#ifndef FA2_PP_PERSISTENT
#define FA2_PP_PERSISTENT 1
#endif
// 1: calls too small to fill the GPU run the short-problem kernel (see make_plan)
#ifndef FA2_SHORT
#define FA2_SHORT 1
#endif
// 1: fp32 tensors of flash_attention_v2 (fp16 rounding) run the 16-bit
// kernels on fp16 copies (see make_plan); 0: the register-staged kernel
#ifndef FA2_F32_CONV
#define FA2_F32_CONV 1
#endif
// 1: ragged/paged two-head launches claim units from per-XCD counters
// (KArgs::claim); 0: the static round walk
// 1: paged calls with one q-block per sequence and more two-head units than
// CUs take the balanced walk (see make_plan); 0: rounds of whole units
#ifndef FA2_PP_BAL
#define FA2_PP_BAL 1
#endif
#ifndef FA2_PP_CLAIM
#define FA2_PP_CLAIM 1
#endif
// 1: the decode kernel merges its own splits (KArgs::merge_ctr); 0: a
// combine launch after it
#ifndef FA2_DECODE_FOLD
#define FA2_DECODE_FOLD 1
#endif
// 1: fp32 decode units of at most kDecF32MaxRows rows run the VALU decode
// kernel (see make_plan_packed); 0: the fp32-MFMA kernel
#ifndef FA2_DECODE_F32_VALU
#define FA2_DECODE_F32_VALU 1
#endif
// 1: ragged launches that fit the GPU at once run without the plan kernel
// and merge their own splits (see make_plan); 0: plan and combine launches
#ifndef FA2_INLINE_PLAN
#define FA2_INLINE_PLAN 1
#endif

namespace fa2 {
namespace {

// fp32 decode (the fp32-MFMA kernel in packed-head mode): automatic splits
// aim at this many workgroups per CU, keeping this many KV tiles per split
constexpr int64_t kF32DecodeWgsPerCu = 8;
constexpr int64_t kF32DecodeMinTiles = 32;
// the VALU fp32 decode kernel (two workgroups per CU): workgroups per CU and
// KV tiles per split its automatic splits aim at.  Measured on MI355X (us per
// call at 1 / 2 / 4 / 8 / 16 forced splits): d1 263 / 153 / 130 / 135 / 151,
// s1 464 / 250 / 163 / 171 / 195, d2 634 / 480 / 492 / 526 / 607; these
// constants pick 4, 4 and 2.
constexpr int64_t kDecF32WgsPerCu = 4;
constexpr int64_t kDecF32MinTiles = 32;

// byte offset of the kXcds claim counters after the work list's item count
// (within the 256 bytes reserved there; a cache line of their own)
constexpr size_t kClaimOffset = 128;

constexpr int kMaxDevices = 64;
std::once_flag g_cu_once[kMaxDevices];
int g_cu_count[kMaxDevices];

int cu_count_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(g_cu_once[dev], [dev] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cu_count[dev] = n;
  });
  return g_cu_count[dev];
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int elt_bytes(int dtype) { return dtype == FA2_DTYPE_F32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool stride_ok(int64_t s, int eb) { return ((s * eb) & 15) == 0; }

// Head dims the reference kernels take (a power of two that tl.dot accepts).
bool head_dim_ok(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }

// The MFMA/LDS kernels are built for 64 and 128; the register-staged kernel
// also for 256, and serves 16 and 32 with its D = 64 tiles (KArgs::dv).
bool fast_dim(int64_t d) { return d == 64 || d == 128; }
int64_t tile_dim(int64_t d) { return d < 64 ? 64 : d; }

// Number of work units (q-block x head) the forward launch covers, and the
// capacity of the ragged/paged work list.
struct Plan {
  int64_t work_ub;  // (sequence, q-block) slots
  int64_t npairs;   // work_ub * Hkv
  int64_t grid_x;   // npairs rounded up to kXcds, times Hq / Hkv
  bool pp;          // two-head ping-pong kernel
  bool shortk;      // short-problem kernel: 32-row blocks, KV split over the waves
  bool qpair;       // ... on MHA, two q-blocks of one head per unit (KArgs::qpair)
  int64_t grid_pp;  // its grid: npairs rounded up to kXcds, times Hq / Hkv / 2
  int splits;
  int part_rows;    // split partials: rows per slot
  int64_t dim;      // head dims of the launched kernel's tiles (>= head_dim)
  int64_t rows;     // query rows of one unit's sequence (packed: Hq/Hkv * M)
  int block_rows;   // rows per q-block of the launched kernel
  bool dec;         // packed fp16/bf16: the decode kernel
  bool f32;         // fp32 arithmetic: the fp32-MFMA kernel
  bool decf32;      // packed fp32 with few rows per unit: the VALU decode kernel
  bool conv;        // fp32 tensors with the reference's fp16 rounding: fp16 copies in the
                    // workspace, the 16-bit kernels, partials and an fp32 combine
  bool plan;        // ragged/paged: the plan kernel orders the work list
  bool dev_splits;  // ... and lowers the automatic split count (KArgs::split_count)
  bool buf;         // paged: every row of the pool has a 31-bit byte offset
  bool fold;        // splits merged by the forward kernel (KArgs::merge_ctr), no combine
  bool inline_plan; // ragged without the plan kernel (KArgs::inline_plan)
  bool bal;         // paged: the two-head kernel's balanced walk (pp_bal_locate)
  int64_t bal_slots;  // ... its part slots (4 per workgroup)
  int64_t max_wgs;  // cap on the persistent grid (0: none)
  uint32_t pool_bytes_k, pool_bytes_v;
  size_t off_work, off_count, off_ml, off_o, off_ctr, off_cq, off_ck, off_cv, total;
};

// K/V tiles are read through buffer descriptors.  Dense and ragged tiles, and
// paged tiles whose page size is a multiple of the rows one DMA instruction
// covers, get a descriptor per tile or page with a 64-bit base: any tensor
// size.  The remaining paged loads (other page sizes, and the register-staged
// kernel) address rows by 32-bit offsets from the pool base, which needs the
// pool's size (kv_len rows) to fit 31 bits; otherwise they use 64-bit global
// loads (the BUF = false kernels).  Rows must not overlap (stride >= D).
bool buffer_path_ok(const fa2_params* p, uint32_t* kbytes, uint32_t* vbytes) {
  const int64_t eb = elt_bytes(p->dtype);
  const int64_t lim = (int64_t(1) << 31) - 1024;
  if (p->layout != FA2_LAYOUT_PAGED) return true;
  if (p->kv_len <= 0) return false;
  if (p->k_ss < p->head_dim || p->v_ss < p->head_dim) return false;
  const int64_t kb = p->kv_len * p->k_ss * eb;
  const int64_t vb = p->kv_len * p->v_ss * eb;
  if (kb > lim || vb > lim) return false;
  *kbytes = static_cast<uint32_t>(kb);
  *vbytes = static_cast<uint32_t>(vb);
  return true;
}

int validate(const fa2_params* p) {
  if (!p) return FA2_ERR_NULL_POINTER;
  if (p->layout < FA2_LAYOUT_DENSE || p->layout > FA2_LAYOUT_PAGED) return FA2_ERR_BAD_LAYOUT;
  if (p->dtype < FA2_DTYPE_F16 || p->dtype > FA2_DTYPE_F32) return FA2_ERR_BAD_DTYPE;
  if (p->mask < FA2_MASK_NONE || p->mask > FA2_MASK_CAUSAL_BOTTOM_RIGHT) return FA2_ERR_BAD_MASK;
  if (!head_dim_ok(p->head_dim)) return FA2_ERR_HEAD_DIM;
  if (p->batch < 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->q_len < 0 || p->kv_len < 0)
    return FA2_ERR_BAD_SHAPE;
  if (p->q_heads % p->kv_heads != 0) return FA2_ERR_BAD_SHAPE;
  if (p->num_splits < 0 || p->num_splits > FA2_MAX_SPLITS) return FA2_ERR_SPLITS;
  if (p->layout == FA2_LAYOUT_RAGGED && (!p->q_indptr || !p->kv_indptr)) return FA2_ERR_RAGGED_ARGS;
  if (p->layout == FA2_LAYOUT_PAGED &&
      (!p->kv_indptr || !p->k_block_table || !p->v_block_table || p->page_size <= 0 ||
       p->k_table_stride < 0 || p->v_table_stride < 0))
    return FA2_ERR_PAGED_ARGS;
  const int eb = elt_bytes(p->dtype);
  const int64_t strides[] = {p->q_sb, p->q_sh, p->q_ss, p->k_sb, p->k_sh, p->k_ss,
                             p->v_sb, p->v_sh, p->v_ss, p->o_sb, p->o_sh, p->o_ss};
  for (int64_t s : strides)
    if (!stride_ok(s, eb)) return FA2_ERR_ALIGNMENT;
  // 32-bit counters inside the kernels
  const int64_t lim = INT32_MAX / 2;
  if (p->batch > lim || p->q_heads > 65536 || p->q_len > lim || p->kv_len > lim ||
      p->page_size > lim)
    return FA2_ERR_TOO_LARGE;
  // a tile's (or page's, or q-block's) rows are addressed by 32-bit offsets
  // from its first row: row strides up to 32 MiB
  const int64_t row_lim = int64_t(1) << 25;
  if (p->q_ss * eb > row_lim || p->k_ss * eb > row_lim || p->v_ss * eb > row_lim ||
      p->o_ss * eb > row_lim)
    return FA2_ERR_TOO_LARGE;
  if (p->max_workgroups < 0 || p->kv_len_max < 0) return FA2_ERR_BAD_SHAPE;
  if (p->arith < FA2_ARITH_REFERENCE || p->arith > FA2_ARITH_FP32) return FA2_ERR_BAD_DTYPE;
  if (p->decode_spin_cap < 0) return FA2_ERR_BAD_SHAPE;
  if (p->kernel < FA2_KERNEL_AUTO || p->kernel > FA2_KERNEL_SHORT) return FA2_ERR_BAD_SHAPE;
  return FA2_OK;
}

// Decode / speculative decode: the fa2_fwd checks minus the ragged q_indptr,
// plus the mask set and the packed q/o row layout (include/fa2.h).
int validate_decode(const fa2_params* p) {
  if (!p) return FA2_ERR_NULL_POINTER;
  if (p->mask == FA2_MASK_CAUSAL_TOP_LEFT) return FA2_ERR_BAD_MASK;
  if (p->layout == FA2_LAYOUT_RAGGED) {
    if (!p->kv_indptr) return FA2_ERR_RAGGED_ARGS;
    fa2_params c = *p;
    c.q_indptr = p->kv_indptr;  // unused in decode; satisfies the shared check
    int s = validate(&c);
    if (s != FA2_OK) return s;
  } else {
    int s = validate(p);
    if (s != FA2_OK) return s;
  }
  // unit row r = (head in group) * M + m lives at r * q_ss from the group's
  // first head (M = 1: the row stride is the head stride)
  if (p->q_heads / p->kv_heads > 1 &&
      (p->q_sh != p->q_len * p->q_ss || p->o_sh != p->q_len * p->o_ss))
    return FA2_ERR_Q_LAYOUT;
  return FA2_OK;
}

bool empty_problem(const fa2_params* p) {
  return p->batch == 0 || p->q_len == 0;
}

int finish_plan(const fa2_params* p, Plan* pl);

// Longest KV range any sequence can have, for the split heuristic (lengths
// themselves live on the device): N (dense), Tkv (ragged), the pool's rows
// (paged: a heuristic bound, pages may repeat), each capped by the caller's
// kv_len_max (paged: block-table width * page_size).
int64_t kv_upper_bound(const fa2_params* p) {
  int64_t ub = p->kv_len > 0 ? p->kv_len : INT32_MAX;
  if (p->kv_len_max > 0 && p->kv_len_max < ub) ub = p->kv_len_max;
  // top-left causal: row i sees keys j <= i, so no sweep is longer than the
  // query rows (dense/paged: the rows per sequence; ragged: all of them)
  if (p->mask == FA2_MASK_CAUSAL_TOP_LEFT && p->q_len > 0 && p->q_len < ub) ub = p->q_len;
  return ub;
}

int make_plan(const fa2_params* p, Plan* pl, bool query_device, bool allow_conv = true,
              bool allow_bal = true) {
  const int64_t nqb = cdiv(p->q_len, kBM);
  // fp32 tensors of flash_attention_v2, whose reference rounds every operand
  // to fp16 (attention.py:547, 569, 621) and keeps fp32 partials that a
  // second kernel merges into the output (:636-746): dense and ragged calls
  // at head_dim 64/128 convert q, k and v to fp16 copies in the workspace
  // and run the 16-bit kernels, which write fp32 partials even unsplit;
  // the combine kernel writes the fp32 output.  Paged pools are not copied.
  pl->conv = FA2_F32_CONV && allow_conv && p->dtype == FA2_DTYPE_F32 &&
             p->arith != FA2_ARITH_FP32 && p->layout != FA2_LAYOUT_PAGED &&
             fast_dim(p->head_dim);
  const bool half = p->dtype != FA2_DTYPE_F32 || pl->conv;  // the 16-bit kernels
  if (p->layout == FA2_LAYOUT_DENSE)
    pl->work_ub = nqb * p->batch;
  else if (p->layout == FA2_LAYOUT_RAGGED)
    pl->work_ub = nqb + p->batch;  // sum_b ceil(Lq_b/BM) <= ceil(Tq/BM) + B
  else
    pl->work_ub = nqb * p->batch;
  // (item, kv head) pairs rounded up to whole blocks of kXcds pairs, each
  // pair expanded to its Hq/Hkv query heads (decode_work)
  pl->npairs = pl->work_ub * p->kv_heads;
  const int64_t group = p->q_heads / p->kv_heads;
  pl->grid_x = cdiv(pl->npairs, kXcds) * kXcds * group;
  if (pl->grid_x > INT32_MAX || pl->npairs > INT32_MAX) return FA2_ERR_TOO_LARGE;
  pl->dim = tile_dim(p->head_dim);
  pl->pp = FA2_PP && half && group % 2 == 0 && fast_dim(p->head_dim);
  pl->grid_pp = cdiv(pl->npairs, kXcds) * kXcds * cdiv(group, 2);

  // A call whose regular grid fills at most half of the CUs and whose KV
  // range is short runs the short-problem kernel (fa2_kernel_short.h): four
  // workgroups per 128-row q-block, each splitting its KV tiles over its 4
  // waves and merging them in LDS, so the launch lasts about a quarter of
  // the longest KV sweep instead of all of it, with no combine launch.
  // Only with automatic splits and no grid cap (the persistent kernel's
  // tests cap the grid).
  pl->shortk = false;
  if (p->kernel == FA2_KERNEL_SHORT && p->num_splits <= 1 && p->max_workgroups == 0 &&
      p->dtype != FA2_DTYPE_F32 && fast_dim(p->head_dim)) {
    pl->shortk = true;
  } else if (FA2_SHORT && p->kernel == FA2_KERNEL_AUTO && p->num_splits == 0 &&
             p->max_workgroups == 0 && p->dtype != FA2_DTYPE_F32 && fast_dim(p->head_dim)) {
    // It pays only when its whole grid is resident at once (LDS: two
    // workgroups per CU at head_dim 64, one at 128) and the regular
    // kernel's KV sweeps are long enough for the split to matter.  Measured
    // on MI355X (HIP-graph replays, GPU time): c1 (B1 H8 L512 D64 causal,
    // 128 short workgroups) 15.5 -> 6.5 us; the reference benchmark's
    // B16 x 8-head points need 512 short workgroups at D128 and run
    // 9-12 us regular against 11-12 short.
    const int64_t cus = query_device ? cu_count_current_device() : 256;
    const int64_t resident = cus * (p->head_dim <= 64 ? 2 : 1);
    const int64_t tiles = cdiv(kv_upper_bound(p), kBN);
    if (pl->grid_x * kShSub <= resident && tiles >= kShMinTiles && tiles <= kShMaxTiles)
      pl->shortk = true;
  }
  int splits = pl->shortk ? 1 : p->num_splits;
  if (splits == 0) {
    // Split the KV sweep only when the grid cannot fill the GPU (two
    // resident workgroups per CU) and every split keeps >= 16 KV tiles
    // (1024 keys).  Measured on MI355X (bf16 D128): a split costs its fp32
    // partials' round trip and the combine launch, so short KV runs best
    // unsplit (B1 Hq32/8 L512 causal: 17.8 us unsplit, 21.9 at 2 splits;
    // MHA L1024: 29.6 vs 39.1), while long KV with few units wants the
    // splits (B1 Hq8 Lq128 Lk16384: 343 us unsplit, 34 at 16 splits).
    const int64_t cus = query_device ? cu_count_current_device() : 256;
    const int64_t slots = 2 * cus;
    const int64_t tiles = cdiv(kv_upper_bound(p), kBN);
    splits = 1;
    const int64_t units = pl->npairs * (p->q_heads / p->kv_heads);  // real workgroups
    if (units > 0 && units < slots) {
      int64_t s = cdiv(slots, units);
      const int64_t by_tiles = tiles / kMinSplitTiles;
      if (s > by_tiles) s = by_tiles;
      if (s > FA2_MAX_SPLITS) s = FA2_MAX_SPLITS;
      if (s < 1) s = 1;
      splits = static_cast<int>(s);
    }
  }
  pl->splits = splits;
  // The two-head kernel runs one workgroup of two heads per CU.  When that
  // grid does not cover every CU, the one-head kernel's twice as many
  // workgroups (two per CU) finish sooner.  Measured on MI355X (the
  // reference benchmark's B16 Hq8/Hkv2 D128 bf16 points, µs per call): at
  // q128, 64 two-head workgroups per split, the one-head kernel is faster
  // on 23 of 24 points (dense 3-12 %, paged 3-14 %, ragged 10-24 %; ragged
  // full kv2048 5 % slower); at q512, 256 two-head workgroups, the two-head
  // kernel is 6-61 % faster on dense and paged points.  Ragged calls whose
  // sequences average >= 2048 visible keys keep the two-head kernel (full
  // q128 kv2048: 50.2 us against 52.8).  (Ragged items are estimated by
  // their lower bound; grids capped by max_workgroups keep the two-head
  // kernel.)
  if (pl->pp && p->max_workgroups == 0) {
    const int64_t cus = query_device ? cu_count_current_device() : 256;
    const bool ragged = p->layout == FA2_LAYOUT_RAGGED;
    const int64_t items = ragged ? std::max<int64_t>(nqb, p->batch) : pl->work_ub;
    const int64_t wgs = cdiv(items * p->kv_heads, kXcds) * kXcds * cdiv(group, 2) * splits;
    int64_t keys = 0;  // ragged: average visible keys per sequence
    if (ragged && p->batch > 0) {
      keys = p->kv_len / p->batch;
      if (p->mask == FA2_MASK_CAUSAL_TOP_LEFT) keys = std::min<int64_t>(keys, p->q_len / p->batch);
    }
    if (wgs < cus && keys < 2048) pl->pp = false;
  }
  // MHA, one split: the two-head kernel pairs q-blocks of one head (B2 H32
  // L2048 D128 bf16: causal 660 -> 713 TFLOP/s, non-causal 803 -> 882).
  // Ragged and paged only when sequences average >= 4 q-blocks: a sequence
  // with one q-block leaves the second wave group without rows.
  const bool many_qblocks = p->layout == FA2_LAYOUT_DENSE ||
                            (p->layout == FA2_LAYOUT_PAGED && nqb >= 4) ||
                            (p->layout == FA2_LAYOUT_RAGGED && p->batch > 0 &&
                             p->q_len >= 4 * kBM * p->batch);
  // (the partial slots of a two-head unit assume two heads, not two q-blocks)
  pl->qpair = FA2_PP && p->dtype != FA2_DTYPE_F32 && group == 1 && fast_dim(p->head_dim) &&
              splits == 1 && many_qblocks && !pl->shortk;
  if (pl->shortk) pl->pp = false;
  if (pl->qpair) {
    pl->pp = true;
    // ragged keeps its bound (sum over sequences of their pairs <= nqb + batch)
    if (p->layout != FA2_LAYOUT_RAGGED) pl->work_ub = cdiv(nqb, 2) * p->batch;
    pl->npairs = pl->work_ub * p->kv_heads;
    pl->grid_x = cdiv(pl->npairs, kXcds) * kXcds * group;
    pl->grid_pp = cdiv(pl->npairs, kXcds) * kXcds;
  }
  pl->rows = p->q_len;
  pl->block_rows = kBM;
  pl->dec = false;
  pl->f32 = p->dtype == FA2_DTYPE_F32 && p->arith == FA2_ARITH_FP32;
  pl->decf32 = false;
  pl->plan = p->layout != FA2_LAYOUT_DENSE;
  // The split count above rests on the longest KV sweep any sequence can
  // have; for ragged K/V that is the total of all sequences (the lengths
  // stay on the device).  The plan kernel knows the longest sweep and lowers
  // the count: a launch then runs the splits it needs out of a grid sized
  // for the bound (the others exit at once), and with one the combine
  // kernel exits at once.  Measured on MI355X (B16 Hq8/Hkv2 q128 kv128
  // ragged, bf16 D128): 2 splits of 1 tile each, forward 14.1 us + combine
  // 6.0 us.
  pl->dev_splits = pl->plan && p->num_splits == 0 && splits > 1;
  // A paged launch whose workgroups all fit on the GPU at once needs no
  // list: every sequence has the same q-block count, so decode_work maps
  // workgroups to items directly, and with every workgroup resident their
  // order does not matter.  Measured on MI355X (B16 Hq8/Hkv2 q128 kv128
  // paged, bf16 D128): the plan launch was 4.0 us of a 15.1 us call.
  if (p->layout == FA2_LAYOUT_PAGED && !pl->dev_splits) {
    const int64_t cus = query_device ? cu_count_current_device() : 256;
    const int64_t per_split =
        pl->shortk ? pl->grid_x * kShSub : (pl->pp ? pl->grid_pp : pl->grid_x);
    if (per_split * splits <= cus) pl->plan = false;
  }
  pl->part_rows = kBM;  // the two-head kernel's partial slots assume kBM
  pl->fold = false;
  // A ragged launch whose workgroups are all resident at once needs no list
  // either: every workgroup of the two-head or the one-head kernel derives
  // the items (and the split count the plan kernel would derive) from the
  // sequence lengths itself, and the order of the items does not matter.
  // With several splits the forward kernel then merges them itself, so
  // neither the plan nor the combine kernel is launched.
  pl->inline_plan = false;
  const bool lds_dim = p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256;
  if (FA2_INLINE_PLAN && p->layout == FA2_LAYOUT_RAGGED && half && !pl->conv && !pl->f32 &&
      !pl->shortk && lds_dim && p->batch <= kInlinePlanMaxBatch && p->max_workgroups == 0) {
    const int64_t cus = query_device ? cu_count_current_device() : 256;
    const int64_t resident = pl->pp ? 1 : (p->head_dim > 128 ? 1 : FA2_LDS_OCCUPANCY);
    const int64_t per_split = pl->pp ? pl->grid_pp : pl->grid_x;
    if (per_split * splits <= cus * resident) {
      pl->inline_plan = true;
      pl->plan = false;
      pl->dev_splits = false;
      pl->fold = splits > 1;
    }
  }
  // Paged calls with one q-block per sequence and more two-head units than
  // CUs: the balanced walk instead of rounds of whole units, so that no
  // workgroup runs more than its share of the KV tiles (fa2_kernel_pp.h).
  // Whole units leave the longest workgroup at the sum of its two units,
  // which unequal lengths push well past the mean: c4 (32 sequences of
  // 512-8192 keys, 128 new rows each, Hq32/Hkv8 D128), 164 tiles against a
  // mean of 138.  No plan kernel: the units are in (sequence, kv head)
  // order.  Each workgroup's stream is one head pair of one XCD, so the
  // workgroups per XCD are a multiple of the head pairs.
  pl->bal = false;
  pl->bal_slots = 0;
  if (FA2_PP_BAL && allow_bal && p->layout == FA2_LAYOUT_PAGED && pl->pp && !pl->qpair &&
      !pl->shortk && splits == 1 && p->num_splits == 0 && p->max_workgroups == 0 && nqb == 1) {
    const int64_t cus = query_device ? cu_count_current_device() : 256;
    const int64_t upp = cdiv(group, 2);
    const int64_t tiles = cdiv(kv_upper_bound(p), kBN) + 1;
    if (pl->grid_pp > cus && cus % kXcds == 0 && (cus / kXcds) % upp == 0 &&
        pl->npairs <= kXcds * 64 * kBalMaxPer && tiles * cdiv(pl->npairs, kXcds) < (1 << 30)) {
      pl->bal = true;
      pl->plan = false;
      pl->bal_slots = 4 * cus;
    }
  }
  return finish_plan(p, pl);
}

// Buffer path and workspace layout, common to both plans.
int finish_plan(const fa2_params* p, Plan* pl) {
  const int splits = pl->splits;
  pl->pool_bytes_k = pl->pool_bytes_v = 0;
  pl->buf = buffer_path_ok(p, &pl->pool_bytes_k, &pl->pool_bytes_v);
  pl->max_wgs = p->max_workgroups;
  if (pl->bal && !pl->buf) {  // (built for the buffer path only)
    pl->bal = false;
    pl->bal_slots = 0;
    pl->plan = true;
  }

  size_t off = 0;
  pl->off_work = off;
  if (p->layout != FA2_LAYOUT_DENSE) off += static_cast<size_t>(pl->work_ub) * sizeof(int2);
  off = (off + 255) & ~size_t(255);
  pl->off_count = off;  // the item count, the split count, the claim counters at kClaimOffset
  if (p->layout != FA2_LAYOUT_DENSE) off += 256;
  const bool parts = splits > 1 || pl->conv;
  if (!parts) pl->fold = false;
  pl->off_ctr = off;  // one merge word per one-head unit
  if (pl->fold || pl->bal) off += static_cast<size_t>(pl->grid_x) * sizeof(uint64_t);
  off = (off + 255) & ~size_t(255);
  const size_t slots =
      pl->bal ? static_cast<size_t>(pl->bal_slots) : parts ? static_cast<size_t>(splits) * pl->grid_x : 0;
  pl->off_ml = off;
  off += slots * pl->part_rows * 2 * sizeof(float);
  off = (off + 255) & ~size_t(255);
  pl->off_o = off;
  off += slots * pl->part_rows * pl->dim * sizeof(float);
  // fp16 copies: q [B][Hq][Lq][D] or [Tq][Hq][D], k and v likewise
  const int64_t qrows = p->layout == FA2_LAYOUT_DENSE ? p->batch * p->q_len : p->q_len;
  const int64_t kvrows = p->layout == FA2_LAYOUT_DENSE ? p->batch * p->kv_len : p->kv_len;
  auto copy = [&](size_t& at, int64_t rows, int64_t heads) {
    off = (off + 255) & ~size_t(255);
    at = off;
    if (pl->conv) off += static_cast<size_t>(rows) * heads * p->head_dim * 2;
  };
  copy(pl->off_cq, qrows, p->q_heads);
  copy(pl->off_ck, kvrows, p->kv_heads);
  copy(pl->off_cv, kvrows, p->kv_heads);
  pl->total = off;
  return FA2_OK;
}

// Decode / speculative decode: the Hq/Hkv query heads of a kv head and the M
// query tokens of a sequence form the rows of one unit (packed-head mode), so
// a unit streams each K/V row once.  These calls are HBM-bound: the KV sweep
// is split until the grid holds several workgroups per slot, for balance
// over unequal sequence lengths.
int make_plan_packed(const fa2_params* p, Plan* pl, bool query_device) {
  const int64_t group = p->q_heads / p->kv_heads;
  pl->rows = group * p->q_len;
  if (pl->rows > INT32_MAX / 2) return FA2_ERR_TOO_LARGE;
  // fp16/bf16 at head_dim 64/128: the decode kernel (64-row blocks, one
  // workgroup per CU); otherwise the register-staged kernel (128-row blocks)
  pl->dim = tile_dim(p->head_dim);
  pl->dec = p->dtype != FA2_DTYPE_F32 && fast_dim(p->head_dim);
  pl->f32 = p->dtype == FA2_DTYPE_F32;  // decode's reference computes fp32 in fp32
  pl->conv = false;
  // fp32 units of at most kDecF32MaxRows rows: the VALU decode kernel, whose
  // units hold 4 or 8 rows
  pl->decf32 = FA2_DECODE_F32_VALU && pl->f32 &&
               (p->head_dim == 64 || p->head_dim == 128) && pl->rows <= kDecF32MaxRows;
  pl->block_rows = pl->dec ? kDecRows : (pl->decf32 ? (pl->rows <= 4 ? 4 : 8) : kBM);
  const int64_t nqb = cdiv(pl->rows, pl->block_rows);
  pl->work_ub = nqb * p->batch;
  pl->npairs = pl->work_ub * p->kv_heads;
  pl->grid_x = cdiv(pl->npairs, kXcds) * kXcds;
  if (pl->grid_x > INT32_MAX || pl->npairs > INT32_MAX) return FA2_ERR_TOO_LARGE;
  pl->pp = false;
  pl->shortk = false;
  pl->qpair = false;
  pl->grid_pp = 0;
  int splits = p->num_splits;
  if (splits == 0) {
    const int64_t cus = query_device ? cu_count_current_device() : 256;
    // The decode kernel holds a CU alone: one workgroup per CU, >= 8 tiles
    // per split to keep its LDS ring in steady state (measured on MI355X:
    // 128 units of 128 tiles run best at 2 splits, 512 units at 1).  The
    // fp32 kernel (two workgroups per CU, no deep K/V pipeline) is
    // latency-bound: it wants several rounds of workgroups, each sweeping
    // >= 32 tiles (measured on MI355X, fp32 decode, us per call at 1 / 2 /
    // 4 / 8 workgroups per CU and >= 8 tiles: d1 (128 units of 128 tiles)
    // 338 / 180 / 187 / 204 at 2 / 4 / 8 / 16 splits; d2 (512 units, up to
    // 128 tiles) 1730 / 1731 / 1148 / 1105 at 1 / 1 / 2 / 4 splits).
    const int64_t target =
        pl->dec ? cus : (pl->decf32 ? cus * kDecF32WgsPerCu : cus * kF32DecodeWgsPerCu);
    const int64_t min_tiles = pl->dec ? 8 : (pl->decf32 ? kDecF32MinTiles : kF32DecodeMinTiles);
    const int64_t tiles = cdiv(kv_upper_bound(p), kBN);
    splits = 1;
    if (pl->npairs > 0 && pl->npairs < target) {
      int64_t sp = cdiv(target, pl->npairs);
      const int64_t by_tiles = tiles / min_tiles;
      if (sp > by_tiles) sp = by_tiles;
      if (sp > FA2_MAX_SPLITS) sp = FA2_MAX_SPLITS;
      if (sp < 1) sp = 1;
      splits = static_cast<int>(sp);
    }
  }
  pl->splits = splits;
  pl->part_rows = static_cast<int>(pl->rows < pl->block_rows ? pl->rows : pl->block_rows);
  // Every sequence has the same q-block count here, so decode_work can map
  // workgroups to items without a list; the heaviest-first order only pays
  // when the grid runs in more than one round (the decode kernel: one
  // workgroup per CU; the fp32 kernel: two).  (d1: the 4.8 us plan launch
  // was 7 % of the step.)
  pl->plan = p->layout != FA2_LAYOUT_DENSE;
  pl->dev_splits = false;
  const int64_t resident = pl->dec ? 1 : (pl->dim > 128 ? 1 : 2);  // workgroups per CU
  if (pl->plan && (pl->dec || pl->f32) && query_device &&
      pl->grid_x * splits <= cu_count_current_device() * resident)
    pl->plan = false;
  // The decode kernel merges its own splits: the last split of a unit to
  // finish combines the unit's partials, so no combine launch follows.
  pl->fold = FA2_DECODE_FOLD && (pl->dec || pl->decf32) && splits > 1;
  pl->inline_plan = false;
  pl->bal = false;
  pl->bal_slots = 0;
  return finish_plan(p, pl);
}

// Launch kernel K<..., BUF> with BUF = pl.buf; only paged layouts ever run
// the BUF = false kernels (dense and ragged tiles are always rebased).
#define FA2_LAUNCH_BUF(KERNEL, GRID, BLOCK)                                       \
  do {                                                                           \
    if constexpr (MODE == FA2_LAYOUT_PAGED) {                                    \
      if (!pl.buf) {                                                             \
        hipLaunchKernelGGL((KERNEL<DT, D, MODE, false>), GRID, BLOCK, 0, st, a); \
        break;                                                                   \
      }                                                                          \
    }                                                                            \
    hipLaunchKernelGGL((KERNEL<DT, D, MODE, true>), GRID, BLOCK, 0, st, a);      \
  } while (0)

// Persistent grid of the two-head kernel: at most one workgroup per CU
// walks the units.
int64_t pp_workgroups(const Plan& pl) {
  int64_t wgs = pl.grid_pp;
  if (pl.splits == 1 && FA2_PP_PERSISTENT) {
    const int64_t cus = cu_count_current_device();
    if (wgs > cus) wgs = cus;
  }
  if (pl.max_wgs > 0 && wgs > pl.max_wgs) wgs = pl.max_wgs;
  return wgs;
}

template <int DT, int D, int MODE>
int launch_typed(KArgs a, const Plan& pl, hipStream_t st) {
  const bool pp_launch = DT != FA2_DTYPE_F32 && (D == 64 || D == 128) && a.dv == D &&
                         pl.pp && !pl.shortk && !pl.dec && !pl.f32;
  const int64_t pp_wgs = pp_launch ? pp_workgroups(pl) : 0;
  // Ragged/paged two-head launches with one split whose sequences span
  // more than one q-block on average claim their units from per-XCD
  // counters over a sequence-major list (KArgs::claim), so that the
  // workgroups of an XCD run the q-blocks of one or two sequences at a time
  // and share their K/V in its L2.  Measured on MI355X (c3, ragged causal,
  // 16 sequences of 128-4096 tokens): HBM traffic 1903 -> 821 MB per
  // launch (2.36x -> 1.02x the algorithmic bytes), 961/968 -> 971/971 TFLOP/s.
  // With one q-block per sequence (c4) both lists have the same order and
  // the static walk measured 1 % faster.
  const bool multi_block = MODE == FA2_LAYOUT_RAGGED ? a.q_len > kBM * a.batch : a.nqb > 1;
  if (FA2_PP_CLAIM && MODE != FA2_LAYOUT_DENSE && pl.plan && pp_launch && pl.splits == 1 &&
      pp_wgs >= kXcds && multi_block && (MODE != FA2_LAYOUT_PAGED || pl.buf))
    a.claim = const_cast<int32_t*>(a.work_count) + kClaimOffset / sizeof(int32_t);
  if constexpr (MODE != FA2_LAYOUT_DENSE) {
    if (pl.plan)
      hipLaunchKernelGGL((fa2_plan_kernel<MODE>), dim3(1), dim3(kPlanThreads), 0, st, a,
                         const_cast<int2*>(a.work), const_cast<int32_t*>(a.work_count));
  }
  const dim3 grid(pl.grid_x, pl.splits);
  if constexpr (DT == FA2_DTYPE_F32 && (D == 64 || D == 128)) {
    if (pl.decf32) {
      if (pl.block_rows == 4)
        hipLaunchKernelGGL((fa2_decode_f32_kernel<D, MODE, 4>), grid, dim3(kDecF32Threads), 0, st,
                           a);
      else
        hipLaunchKernelGGL((fa2_decode_f32_kernel<D, MODE, 8>), grid, dim3(kDecF32Threads), 0, st,
                           a);
      if (pl.splits > 1 && !pl.fold)
        hipLaunchKernelGGL((fa2_combine_kernel<DT, D, MODE>),
                           dim3(pl.grid_x, cdiv(pl.part_rows, kCombineRows<D>)), dim3(kThreads),
                           0, st, a);
      return hipGetLastError() == hipSuccess ? FA2_OK : FA2_ERR_HIP;
    }
  }
  if constexpr (DT == FA2_DTYPE_F32) {
    if (pl.f32) {
      FA2_LAUNCH_BUF(fa2_fwd_f32_kernel, grid, dim3(kThreads));
      if (pl.splits > 1)
        hipLaunchKernelGGL((fa2_combine_kernel<DT, D, MODE>),
                           dim3(pl.grid_x, cdiv(pl.part_rows, kCombineRows<D>)), dim3(kThreads),
                           0, st, a);
      return hipGetLastError() == hipSuccess ? FA2_OK : FA2_ERR_HIP;
    }
  }
  if constexpr (DT != FA2_DTYPE_F32 && (D == 64 || D == 128)) {
    if (pl.dec) {
      FA2_LAUNCH_BUF(fa2_decode_kernel, grid, dim3(kDecThreads));
      if (pl.splits > 1 && !pl.fold)
        hipLaunchKernelGGL((fa2_combine_kernel<DT, D, MODE>),
                           dim3(pl.grid_x, cdiv(pl.part_rows, kCombineRows<D>)), dim3(kThreads),
                           0, st, a);
      return hipGetLastError() == hipSuccess ? FA2_OK : FA2_ERR_HIP;
    }
  }
  bool generic = true;  // the register-staged kernel (fp32, head dims 16 and 32)
  if constexpr (DT != FA2_DTYPE_F32 && (D == 64 || D == 128 || D == 256)) {
    if (a.dv == D) {
      generic = false;
      // (the two-head kernel's three K/V slots do not fit LDS at D = 256)
      bool launched = false;
      if constexpr (D <= 128) {
        if (pl.shortk) {
          FA2_LAUNCH_BUF(fa2_fwd_short_kernel, dim3(static_cast<uint32_t>(pl.grid_x * kShSub)),
                         dim3(kShThreads));
          launched = true;
        } else if (pl.pp) {
          const dim3 gpp(static_cast<uint32_t>(pp_wgs), pl.splits);
          if constexpr (MODE != FA2_LAYOUT_DENSE) {
            if (a.claim)
              hipLaunchKernelGGL((fa2_fwd_pp_kernel<DT, D, MODE, true, true>), gpp,
                                 dim3(kPPThreads), 0, st, a);
            else if (MODE == FA2_LAYOUT_RAGGED && a.inline_plan)
              hipLaunchKernelGGL((fa2_fwd_pp_kernel<DT, D, FA2_LAYOUT_RAGGED, true, false, true>),
                                 gpp, dim3(kPPThreads), 0, st, a);
            else if (MODE == FA2_LAYOUT_PAGED && pl.bal)
              hipLaunchKernelGGL(
                  (fa2_fwd_pp_kernel<DT, D, FA2_LAYOUT_PAGED, true, false, false, true>), gpp,
                  dim3(kPPThreads), 0, st, a);
            else
              FA2_LAUNCH_BUF(fa2_fwd_pp_kernel, gpp, dim3(kPPThreads));
          } else {
            FA2_LAUNCH_BUF(fa2_fwd_pp_kernel, gpp, dim3(kPPThreads));
          }
          launched = true;
        }
      }
      if (!launched) FA2_LAUNCH_BUF(fa2_fwd_lds_kernel, grid, dim3(kThreads));
    }
  }
  if (generic) FA2_LAUNCH_BUF(fa2_fwd_kernel, grid, dim3(kThreads));
  const dim3 cgrid(pl.grid_x, cdiv(pl.part_rows, kCombineRows<D>));
  if (a.part_out) {  // fp32 output of fp16 copies (Plan::conv)
    hipLaunchKernelGGL((fa2_combine_kernel<FA2_DTYPE_F32, D, MODE>), cgrid, dim3(kThreads), 0, st,
                       a);
  } else if (pl.splits > 1 && !pl.fold) {
    hipLaunchKernelGGL((fa2_combine_kernel<DT, D, MODE>), cgrid, dim3(kThreads), 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? FA2_OK : FA2_ERR_HIP;
}

template <int DT, int D>
int launch_mode(int mode, const KArgs& a, const Plan& pl, hipStream_t st) {
  switch (mode) {
    case FA2_LAYOUT_DENSE: return launch_typed<DT, D, FA2_LAYOUT_DENSE>(a, pl, st);
    case FA2_LAYOUT_RAGGED: return launch_typed<DT, D, FA2_LAYOUT_RAGGED>(a, pl, st);
    default: return launch_typed<DT, D, FA2_LAYOUT_PAGED>(a, pl, st);
  }
}

// d: the plan's tile head dim (64 also serves head_dim 16 and 32)
template <int DT>
int launch_dim(int64_t d, int mode, const KArgs& a, const Plan& pl, hipStream_t st) {
  if (d == 64) return launch_mode<DT, 64>(mode, a, pl, st);
  if (d == 128) return launch_mode<DT, 128>(mode, a, pl, st);
  return launch_mode<DT, 256>(mode, a, pl, st);
}

}  // namespace
}  // namespace fa2

using namespace fa2;

extern "C" int fa2_abi_version(void) { return 7; }

extern "C" size_t fa2_params_size(void) { return sizeof(fa2_params); }

extern "C" const char* fa2_strerror(int s) {
  switch (s) {
    case FA2_OK: return "success";
    case FA2_ERR_NULL_POINTER: return "a required pointer is NULL";
    case FA2_ERR_BAD_LAYOUT: return "layout must be dense (0), ragged (1) or paged (2)";
    case FA2_ERR_BAD_DTYPE:
      return "dtype must be f16 (0), bf16 (1) or f32 (2), arith reference (0) or fp32 (1)";
    case FA2_ERR_BAD_MASK: return "mask must be none (0), top-left causal (1) or bottom-right causal (2)";
    case FA2_ERR_BAD_SHAPE: return "invalid shape (negative size or q_heads % kv_heads != 0)";
    case FA2_ERR_HEAD_DIM: return "unsupported head_dim (supported: 16, 32, 64, 128, 256)";
    case FA2_ERR_ALIGNMENT: return "tensor rows must start on 16-byte boundaries";
    case FA2_ERR_PAGED_ARGS: return "paged layout needs kv_indptr (lengths), both block tables and page_size > 0";
    case FA2_ERR_RAGGED_ARGS: return "ragged layout needs q_indptr and kv_indptr";
    case FA2_ERR_WORKSPACE: return "workspace is missing or smaller than fa2_fwd_workspace_size";
    case FA2_ERR_SPLITS: return "num_splits must be in [0, FA2_MAX_SPLITS]";
    case FA2_ERR_HIP: return "a HIP launch or runtime call failed";
    case FA2_ERR_TOO_LARGE: return "a size exceeds the kernels' 32-bit index range";
    case FA2_ERR_Q_LAYOUT:
      return "decode: q/o head stride must equal q_len * row stride (contiguous heads)";
    case FA2_ERR_SCRATCH:
      return "fa2_fwd_noalloc: the call needs more than the static scratch "
             "(FA2_NOALLOC_SCRATCH_BYTES = 32 MiB per device)";
    default: return "unknown fa2 status";
  }
}

namespace fa2 {
namespace {

int workspace_size(const fa2_params* p, size_t* bytes, bool packed) {
  if (!bytes) return FA2_ERR_NULL_POINTER;
  int s = packed ? validate_decode(p) : validate(p);
  if (s != FA2_OK) return s;
  if (empty_problem(p)) {
    *bytes = 0;
    return FA2_OK;
  }
  Plan pl{};
  s = packed ? make_plan_packed(p, &pl, p->num_splits == 0)
             : make_plan(p, &pl, p->num_splits == 0);
  if (s != FA2_OK) return s;
  *bytes = pl.total;
  return FA2_OK;
}

// allow_conv = false: fp32 tensors keep the register-staged kernel (no
// fp16 copies in the workspace; fa2_fwd_noalloc when they do not fit)
// Tag of one call's merge words (KArgs::merge_tag): a process-wide counter
// from a random start, skipping the values a cleared or all-ones word holds.
uint64_t next_merge_tag() {
  constexpr uint64_t kMask = (uint64_t(1) << kMergeTagBits) - 1;
  static std::atomic<uint64_t> next{[] {
    std::random_device rd;
    return (static_cast<uint64_t>(rd()) << 32) ^ rd();
  }()};
  for (;;) {
    const uint64_t t = next.fetch_add(1, std::memory_order_relaxed) & kMask;
    if (t != 0 && t != kMask) return t;
  }
}

int run(const fa2_params* p, void* stream, bool packed, bool allow_conv = true,
        bool allow_bal = true) {
  int s = packed ? validate_decode(p) : validate(p);
  if (s != FA2_OK) return s;
  if (empty_problem(p)) return FA2_OK;
  if (!p->q || !p->k || !p->v || !p->o) return FA2_ERR_NULL_POINTER;
  if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o))
    return FA2_ERR_ALIGNMENT;
  Plan pl{};
  s = packed ? make_plan_packed(p, &pl, p->num_splits == 0)
             : make_plan(p, &pl, p->num_splits == 0, allow_conv, allow_bal);
  if (s != FA2_OK) return s;
  if (pl.total > 0 && (!p->workspace || p->workspace_bytes < pl.total)) return FA2_ERR_WORKSPACE;

  KArgs a{};
  a.q = p->q;
  a.k = p->k;
  a.v = p->v;
  a.o = p->o;
  a.q_indptr = p->q_indptr;
  a.kv_indptr = p->kv_indptr;
  a.k_table = p->k_block_table;
  a.v_table = p->v_block_table;
  a.q_sb = p->q_sb; a.q_sh = p->q_sh; a.q_ss = p->q_ss;
  a.k_sb = p->k_sb; a.k_sh = p->k_sh; a.k_ss = p->k_ss;
  a.v_sb = p->v_sb; a.v_sh = p->v_sh; a.v_ss = p->v_ss;
  a.o_sb = p->o_sb; a.o_sh = p->o_sh; a.o_ss = p->o_ss;
  a.k_table_stride = p->k_table_stride;
  a.v_table_stride = p->v_table_stride;
  a.batch = static_cast<int32_t>(p->batch);
  a.hq = static_cast<int32_t>(p->q_heads);
  a.hkv = static_cast<int32_t>(p->kv_heads);
  a.q_len = static_cast<int32_t>(pl.rows);  // packed: rows of a unit
  a.kv_len = static_cast<int32_t>(p->kv_len);
  a.page_size = static_cast<int32_t>(p->page_size > 0 ? p->page_size : 1);
  a.page_shift = -1;
  for (int s = 0; s < 31; ++s)
    if ((int64_t(1) << s) == a.page_size) a.page_shift = s;
  a.nqb = static_cast<int32_t>(cdiv(pl.rows, pl.block_rows));
  a.qpair = pl.qpair ? 1 : 0;
  if (pl.qpair) a.nqb = static_cast<int32_t>(cdiv(a.nqb, 2));  // q-block pairs
  a.block_rows = pl.block_rows;
  a.work_ub = static_cast<int32_t>(pl.work_ub);
  a.npairs = static_cast<int32_t>(pl.npairs);
  a.mask = p->mask;
  a.num_splits = pl.splits;
  a.part_slots = static_cast<int32_t>(pl.grid_x);
  a.units = static_cast<int32_t>(pl.grid_pp);
  a.scale_log2 = p->softmax_scale * 1.4426950408889634f;
  a.pool_bytes_k = pl.pool_bytes_k;
  a.pool_bytes_v = pl.pool_bytes_v;
  char* ws = static_cast<char*>(p->workspace);
  a.work = pl.plan ? reinterpret_cast<const int2*>(ws + pl.off_work) : nullptr;
  a.work_count = pl.plan ? reinterpret_cast<const int32_t*>(ws + pl.off_count) : nullptr;
  a.split_count = pl.dev_splits ? reinterpret_cast<int32_t*>(ws + pl.off_count) + 1 : nullptr;
  const bool parts = pl.splits > 1 || pl.conv || pl.bal;
  a.part_ml = parts ? reinterpret_cast<float*>(ws + pl.off_ml) : nullptr;
  a.part_o = parts ? reinterpret_cast<float*>(ws + pl.off_o) : nullptr;
  a.part_rows = pl.part_rows;
  const bool merges = pl.fold || pl.bal;
  a.merge_ctr = merges ? reinterpret_cast<uint64_t*>(ws + pl.off_ctr) : nullptr;
  a.merge_tag = merges ? next_merge_tag() : 0;
  a.inline_plan = pl.inline_plan ? 1 : 0;
  a.auto_splits = p->num_splits == 0 ? 1 : 0;
  a.pack_m = packed ? static_cast<int32_t>(p->q_len) : 0;
  a.dv = static_cast<int32_t>(p->head_dim);
  a.spin_cap = p->decode_spin_cap > 0 ? p->decode_spin_cap : kDecSpinCap;

  hipStream_t st = static_cast<hipStream_t>(stream);
  if (pl.conv) {
    // q, k, v -> contiguous fp16 copies ([B][H][L][D] dense, [T][H][D]
    // ragged), then the 16-bit kernels with an fp32 combine
    const bool dense = p->layout == FA2_LAYOUT_DENSE;
    const int64_t D = p->head_dim;
    uint16_t* cq = reinterpret_cast<uint16_t*>(ws + pl.off_cq);
    uint16_t* ck = reinterpret_cast<uint16_t*>(ws + pl.off_ck);
    uint16_t* cv = reinterpret_cast<uint16_t*>(ws + pl.off_cv);
    auto seg = [&](const void* src, int64_t sb, int64_t sh, int64_t ss, int64_t len,
                   int64_t heads, uint16_t* dst) {
      ConvSeg g;
      g.src = static_cast<const float*>(src);
      if (dense) {  // [B][H][L]
        g.s0 = sb; g.s1 = sh; g.s2 = ss;
        g.n1 = static_cast<int32_t>(heads);
        g.n2 = static_cast<int32_t>(len);
        g.rows = p->batch * heads * len;
      } else {  // [T][H]
        g.s0 = 0; g.s1 = ss; g.s2 = sh;
        g.n1 = static_cast<int32_t>(len);
        g.n2 = static_cast<int32_t>(heads);
        g.rows = len * heads;
      }
      g.dst = dst;
      return g;
    };
    ConvArgs c;
    c.seg[0] = seg(p->q, p->q_sb, p->q_sh, p->q_ss, p->q_len, p->q_heads, cq);
    c.seg[1] = seg(p->k, p->k_sb, p->k_sh, p->k_ss, p->kv_len, p->kv_heads, ck);
    c.seg[2] = seg(p->v, p->v_sb, p->v_sh, p->v_ss, p->kv_len, p->kv_heads, cv);
    const int64_t rows = c.seg[0].rows + c.seg[1].rows + c.seg[2].rows;
    const int64_t blocks = cdiv(rows * (D / 8), kConvThreads);
    if (blocks > INT32_MAX) return FA2_ERR_TOO_LARGE;
    if (blocks > 0) {
      if (D == 64)
        hipLaunchKernelGGL((fa2_to_f16_kernel<64>), dim3(static_cast<uint32_t>(blocks)),
                           dim3(kConvThreads), 0, st, c);
      else
        hipLaunchKernelGGL((fa2_to_f16_kernel<128>), dim3(static_cast<uint32_t>(blocks)),
                           dim3(kConvThreads), 0, st, c);
    }
    auto strides = [&](int64_t len, int64_t heads, int64_t& sb, int64_t& sh, int64_t& ss) {
      if (dense) {
        sb = heads * len * D; sh = len * D; ss = D;
      } else {
        sb = 0; sh = D; ss = heads * D;
      }
    };
    a.q = cq;
    a.k = ck;
    a.v = cv;
    strides(p->q_len, p->q_heads, a.q_sb, a.q_sh, a.q_ss);
    strides(p->kv_len, p->kv_heads, a.k_sb, a.k_sh, a.k_ss);
    strides(p->kv_len, p->kv_heads, a.v_sb, a.v_sh, a.v_ss);
    a.part_out = 1;
    return launch_dim<FA2_DTYPE_F16>(pl.dim, p->layout, a, pl, st);
  }
  switch (p->dtype) {
    case FA2_DTYPE_F16: return launch_dim<FA2_DTYPE_F16>(pl.dim, p->layout, a, pl, st);
    case FA2_DTYPE_BF16: return launch_dim<FA2_DTYPE_BF16>(pl.dim, p->layout, a, pl, st);
    default: return launch_dim<FA2_DTYPE_F32>(pl.dim, p->layout, a, pl, st);
  }
}

}  // namespace
}  // namespace fa2

extern "C" int fa2_fwd_workspace_size(const fa2_params* p, size_t* bytes) {
  return workspace_size(p, bytes, false);
}

extern "C" int fa2_fwd(const fa2_params* p, void* stream) { return run(p, stream, false); }

// ---- fa2_fwd_noalloc: the workspace in a static device array ---------------
//
// Each device holds its own copy of `scratch` from the module's load until
// the process ends.  In host code the array's name is only a stand-in for the
// symbol: its device address comes from hipGetSymbolAddress, once per device
// with that device current, and only that address reaches the kernels.
// Nothing in it has to start at zero: the plan kernel writes the work list,
// its count, the split count and zeroes the claim counters, and every split
// partial the combine reads is written by the forward kernel of the same
// call.
static __device__ __align__(256) unsigned char scratch[FA2_NOALLOC_SCRATCH_BYTES];

namespace fa2 {
namespace {

std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// This device's copy of `scratch`, or null if the lookup failed.  Only a
// successful lookup is kept: a failed one is tried again on the next call.
void* scratch_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  if (void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire)) return ptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (!ptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  return ptr;
}

}  // namespace
}  // namespace fa2

extern "C" int fa2_fwd_noalloc(const fa2_params* p, void* stream) {
  int s = validate(p);
  if (s != FA2_OK) return s;
  if (empty_problem(p)) return FA2_OK;
  constexpr size_t cap = FA2_NOALLOC_SCRATCH_BYTES;
  fa2_params c = *p;
  Plan pl{};
  // The plan with fp16 copies of fp32 tensors (the faster kernel, and the
  // one fa2_fwd runs) comes first, with fewer automatic splits until its
  // workspace fits; fp32 tensors fall back to the register-staged kernel
  // only when even one split with copies does not fit.
  bool bal = true;  // the balanced walk, while its part slots fit
  auto fit = [&](bool allow_conv) -> int {
    c = *p;
    bal = true;
    int r = make_plan(&c, &pl, c.num_splits == 0, allow_conv);
    if (r != FA2_OK) return r;
    if (pl.bal && pl.total > cap) {  // whole units need no part slots
      bal = false;
      r = make_plan(&c, &pl, c.num_splits == 0, allow_conv, false);
      if (r != FA2_OK) return r;
    }
    if (p->num_splits == 0)
      for (int sp = pl.splits - 1; sp >= 1 && pl.total > cap; --sp) {
        c.num_splits = sp;
        r = make_plan(&c, &pl, false, allow_conv);
        if (r != FA2_OK) return r;
      }
    return FA2_OK;
  };
  bool conv = true;
  s = fit(true);
  if (s != FA2_OK) return s;
  if (pl.total > cap && pl.conv) {
    conv = false;
    s = fit(false);
    if (s != FA2_OK) return s;
  }
  if (pl.total > cap) return FA2_ERR_SCRATCH;
  void* ws = scratch_current_device();
  if (!ws) return FA2_ERR_HIP;
  c.workspace = ws;
  c.workspace_bytes = cap;
  return run(&c, stream, false, conv, bal);
}

extern "C" int fa2_decode_workspace_size(const fa2_params* p, size_t* bytes) {
  return workspace_size(p, bytes, true);
}

extern "C" int fa2_decode_fwd(const fa2_params* p, void* stream) { return run(p, stream, true); }

extern "C" int fa2_decode_wait_giveups(uint32_t* count, int reset) {
  if (!count) return FA2_ERR_NULL_POINTER;
  unsigned int v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(fa2::g_decode_giveups), sizeof(v), 0,
                          hipMemcpyDeviceToHost) != hipSuccess)
    return FA2_ERR_HIP;
  *count = v;
  if (reset) {
    const unsigned int z = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(fa2::g_decode_giveups), &z, sizeof(z), 0,
                          hipMemcpyHostToDevice) != hipSuccess)
      return FA2_ERR_HIP;
  }
  return FA2_OK;
}

extern "C" size_t fa2_kv_append_params_size(void) { return sizeof(fa2_kv_append_params); }

extern "C" int fa2_kv_append(const fa2_kv_append_params* p, void* stream) {
  if (!p) return FA2_ERR_NULL_POINTER;
  if (p->dtype < FA2_DTYPE_F16 || p->dtype > FA2_DTYPE_F32) return FA2_ERR_BAD_DTYPE;
  if (p->batch < 0 || p->kv_heads <= 0 || p->head_dim <= 0 || p->num_rows < 0 ||
      p->page_size <= 0 || p->num_pages < 0 || p->table_width < 0 || p->k_table_stride < 0 ||
      p->v_table_stride < 0)
    return FA2_ERR_BAD_SHAPE;
  if (p->batch == 0 || p->num_rows == 0) return FA2_OK;
  // V is optional (all three V pointers null: only K is written)
  const bool has_v = p->v_new || p->v_cache || p->v_block_table;
  if (!p->k_new || !p->k_cache || !p->new_indptr || !p->k_block_table ||
      (has_v && (!p->v_new || !p->v_cache || !p->v_block_table)))
    return FA2_ERR_NULL_POINTER;
  const int64_t eb = elt_bytes(p->dtype);
  const int64_t row_bytes = p->head_dim * eb;
  if (row_bytes % 16) return FA2_ERR_ALIGNMENT;
  const int64_t strides[] = {p->new_ts, p->new_hs, p->cache_ts, p->cache_hs};
  for (int64_t st : strides)
    if (!stride_ok(st, static_cast<int>(eb))) return FA2_ERR_ALIGNMENT;
  if (!aligned16(p->k_new) || !aligned16(p->k_cache) ||
      (has_v && (!aligned16(p->v_new) || !aligned16(p->v_cache))))
    return FA2_ERR_ALIGNMENT;
  const int64_t lim = INT32_MAX / 2;
  if (p->batch > lim || p->num_rows > lim || p->page_size > lim || p->table_width > lim ||
      p->kv_heads * (row_bytes / 16) > lim)
    return FA2_ERR_TOO_LARGE;
  AppendArgs a{};
  a.k_new = static_cast<const char*>(p->k_new);
  a.v_new = static_cast<const char*>(p->v_new);
  a.k_cache = static_cast<char*>(p->k_cache);
  a.v_cache = static_cast<char*>(p->v_cache);
  a.indptr = p->new_indptr;
  a.start = p->start_pos;
  a.k_table = p->k_block_table;
  a.v_table = p->v_block_table;
  a.new_ts = p->new_ts * eb;
  a.new_hs = p->new_hs * eb;
  a.cache_ts = p->cache_ts * eb;
  a.cache_hs = p->cache_hs * eb;
  a.k_table_stride = p->k_table_stride;
  a.v_table_stride = p->v_table_stride;
  a.num_pages = p->num_pages;
  a.batch = static_cast<int32_t>(p->batch);
  a.heads = static_cast<int32_t>(p->kv_heads);
  a.head_chunks = static_cast<int32_t>(row_bytes / 16);
  a.row_chunks = static_cast<int32_t>(p->kv_heads * (row_bytes / 16));
  a.num_rows = static_cast<int32_t>(p->num_rows);
  a.page_size = static_cast<int32_t>(p->page_size);
  a.table_width = static_cast<int32_t>(p->table_width);
  const int64_t grid = (p->num_rows + kAppendRows - 1) / kAppendRows;
  hipLaunchKernelGGL(fa2_kv_append_kernel, dim3(static_cast<uint32_t>(grid)),
                     dim3(kAppendThreads), 0, static_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? FA2_OK : FA2_ERR_HIP;
}

