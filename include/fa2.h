/*
 * fa2.h - C ABI of the MI355X (gfx950) flash_attention_v2 forward pass.
 *
 * This is the drop-in boundary behind the Python entry point
 * `flash_attention_v2(q, k, v, *, is_causal, q_indptr, kv_indptr,
 * k_block_table, v_block_table, kv_page_size)`.
 *
 * Reference interface replaced (harsh-vsingh/triton-kernels):
 *   kernels/attention.py:749-927  host wrapper `flash_attention_v2`
 *   kernels/attention.py:430-656  `_flash_attentionv2_partial_kernel`
 *   kernels/attention.py:659-746  `_flash_attentionv2_merge_kernel`
 * The reference binds its kernels through Triton's launcher; the Python
 * wrapper of this library binds these entry points through ctypes.
 *
 * All pointers are device pointers except `params` itself.  Sizes and
 * strides are in ELEMENTS of the tensor they describe; the last (head_dim)
 * dimension of q, k, v and o must be contiguous.  No entry point allocates
 * device memory: scratch space comes from the caller through
 * `workspace` (size from fa2_fwd_workspace_size).  No entry point performs a
 * host<->device synchronisation; fa2_fwd only enqueues work on `stream`.
 */
#ifndef FA2_H_
#define FA2_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layout of q/k/v/o, the reference's `TYPE` constexpr
 * (kernels/attention.py:465-514; mode select at :766-767). */
enum fa2_layout {
  FA2_LAYOUT_DENSE = 0,  /* q,o [B,Hq,M,D]; k,v [B,Hkv,N,D]                    */
  FA2_LAYOUT_RAGGED = 1, /* q,o [Tq,Hq,D]; k,v [Tkv,Hkv,D]; q_indptr/kv_indptr
                            are exclusive prefix sums, int32 [B+1]             */
  FA2_LAYOUT_PAGED = 2   /* q,o [B,Hq,M,D]; k,v caches [pages*page_size,Hkv,D];
                            kv_indptr holds per-sequence KV LENGTHS int32 [B];
                            k/v_block_table int32 [B, >=ceil(len/page_size)] */
};

/* Element type of q, k, v and o (all four share it, attention.py:762). */
enum fa2_dtype {
  FA2_DTYPE_F16 = 0,  /* fp16 MFMA, fp32 accumulation                          */
  FA2_DTYPE_BF16 = 1, /* bf16 MFMA, fp32 accumulation                          */
  FA2_DTYPE_F32 = 2   /* fp32 tensors; arithmetic per fa2_arith                */
};

/* Arithmetic for fp32 tensors (fp16/bf16 tensors ignore it).
 * FA2_ARITH_REFERENCE: what the reference entry point does - fa2_fwd as
 *   flash_attention_v2 (operands and softmax weights rounded to fp16,
 *   attention.py:547,572,594,607,614,633); fa2_decode_fwd as decode_attention
 *   and speculative_decode_attention (fp32 throughout, decode.py:84,143-160,
 *   speculative_decode.py:91,150-175).
 * FA2_ARITH_FP32: fa2_fwd in fp32 throughout, as flash_attention_v1
 *   (attention.py:177,196-197,225-240). */
enum fa2_arith {
  FA2_ARITH_REFERENCE = 0,
  FA2_ARITH_FP32 = 1
};

/* Causal mask.  TOP_LEFT is the reference's `is_causal=True`
 * (attention.py:566-569: key j visible to query i iff j <= i, per-sequence
 * local indices), identical to SDPA `is_causal=True`.  BOTTOM_RIGHT (key j
 * visible iff j <= i + Lk - Lq) has no counterpart in the reference; it is
 * the chunked-prefill alignment and is reachable only through this ABI or
 * the wrapper's keyword `causal_alignment="bottom_right"`. */
enum fa2_mask {
  FA2_MASK_NONE = 0,
  FA2_MASK_CAUSAL_TOP_LEFT = 1,
  FA2_MASK_CAUSAL_BOTTOM_RIGHT = 2
};

/* Return codes. */
enum fa2_status {
  FA2_OK = 0,
  FA2_ERR_NULL_POINTER = 1,
  FA2_ERR_BAD_LAYOUT = 2,
  FA2_ERR_BAD_DTYPE = 3,
  FA2_ERR_BAD_MASK = 4,
  FA2_ERR_BAD_SHAPE = 5,       /* negative sizes, Hq % Hkv != 0, ...          */
  FA2_ERR_HEAD_DIM = 6,        /* head_dim not in the supported set            */
  FA2_ERR_ALIGNMENT = 7,       /* a row start is not 16-byte aligned           */
  FA2_ERR_PAGED_ARGS = 8,      /* missing table / page size / lengths          */
  FA2_ERR_RAGGED_ARGS = 9,     /* missing indptr                                */
  FA2_ERR_WORKSPACE = 10,      /* workspace missing or smaller than required   */
  FA2_ERR_SPLITS = 11,         /* num_splits out of range                       */
  FA2_ERR_HIP = 12,            /* a HIP runtime call or a launch failed         */
  FA2_ERR_TOO_LARGE = 13,      /* a size exceeds the kernels' 32-bit counters  */
  FA2_ERR_Q_LAYOUT = 14,       /* decode: the rows of the query heads sharing a
                                  kv head are not one strided run
                                  (q_sh != q_len * q_ss, likewise o; with M = 1
                                  pass q_ss = q_sh)                             */
  FA2_ERR_SCRATCH = 15         /* fa2_fwd_noalloc: the call needs more scratch
                                  than FA2_NOALLOC_SCRATCH_BYTES               */
};

/* Supported head dims (the reference accepts any power of two via
 * tl.arange; these are the instantiated tile shapes). */
#define FA2_MAX_SPLITS 64

typedef struct fa2_params {
  int32_t layout;     /* enum fa2_layout */
  int32_t dtype;      /* enum fa2_dtype  */
  int32_t mask;       /* enum fa2_mask   */
  int32_t num_splits; /* split-KV factor: 0 = automatic, 1..FA2_MAX_SPLITS */

  int64_t batch;      /* B (ragged: q_indptr.numel()-1)                       */
  int64_t q_heads;    /* Hq                                                    */
  int64_t kv_heads;   /* Hkv, Hq % Hkv == 0; q head h reads kv head h*Hkv/Hq  */
  int64_t head_dim;   /* D: 16, 32, 64, 128 or 256                             */
  int64_t q_len;      /* dense/paged: M (rows per sequence); ragged: Tq       */
  int64_t kv_len;     /* dense: N; ragged: Tkv; paged: rows of the k/v caches
                         (pages*page_size), or 0 if unknown - per-sequence
                         lengths always come from kv_indptr                    */

  /* Element strides.  Dense/paged q and o use (batch, head, row); ragged q/o
   * and every token-major k/v use (token, head) and ignore *_sb. */
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;

  const void* q;
  const void* k;
  const void* v;
  void* o;

  const int32_t* q_indptr;      /* ragged only                               */
  const int32_t* kv_indptr;     /* ragged: prefix sums; paged: lengths       */
  const int32_t* k_block_table; /* paged only                                */
  const int32_t* v_block_table; /* paged only                                */
  int64_t k_table_stride;       /* row stride of k_block_table (elements)    */
  int64_t v_table_stride;       /* row stride of v_block_table (elements)    */
  int64_t page_size;            /* tokens per page (paged only)              */

  float softmax_scale;          /* reference: head_dim ** -0.5 (:897)        */
  /* Upper limit on the workgroups of the persistent forward kernel (fp16 /
   * bf16 prefill with an even number of query heads per kv head, or MHA):
   * 0 = one workgroup per compute unit.  A smaller value leaves compute
   * units to concurrent work; each workgroup then walks more units.  No
   * counterpart in the reference (its grid is fixed by :873-880). */
  int32_t max_workgroups;

  /* Device scratch, >= fa2_fwd_workspace_size (fa2_decode_workspace_size),
   * with any prior content: it never needs clearing.  (A call that merges its
   * splits inside the forward kernel counts them in words tagged per call and
   * leaves them at zero for a replay of itself.)  One workspace per call in
   * flight. */
  void* workspace;
  size_t workspace_bytes;

  /* An upper bound of every sequence's KV length, or 0 if unknown (paged:
   * the wrapper passes block-table width * page_size, the reference's N,
   * attention.py:834).  Used only to size the split-KV factor; lengths
   * always come from kv_indptr. */
  int64_t kv_len_max;

  int32_t arith;      /* enum fa2_arith (fp32 tensors only)                    */

  /* fa2_decode_fwd, fp16/bf16: polls after which a wait of the decode
   * kernel's producer/consumer ring gives up (0 = the library's bound, about
   * 5 ms).  A wait that gives up poisons its rows with NaN and counts in
   * fa2_decode_wait_giveups().  Only tests set it, to exercise that path from
   * the host.  No counterpart in the reference, whose decode kernels do not
   * synchronise waves. */
  int32_t decode_spin_cap;

  /* fa2_fwd, fp16/bf16, head_dim 64 or 128: which forward kernel serves the
   * call (enum fa2_kernel).  FA2_KERNEL_AUTO lets the library choose: calls
   * whose regular grid fills at most half of the compute units and whose KV
   * range is at most 32 tiles of 64 keys run the short-problem kernel (the KV
   * tiles of each 32-row query block split over the waves of one workgroup,
   * merged in LDS); FA2_KERNEL_REGULAR never uses it; FA2_KERNEL_SHORT uses it
   * whenever dtype and head dim allow (num_splits 0 or 1, no max_workgroups).
   * Results agree within rounding, not bit for bit.  No counterpart in the
   * reference; tests use it to reach each kernel on small shapes. */
  int32_t kernel;
} fa2_params;

enum fa2_kernel {
  FA2_KERNEL_AUTO = 0,
  FA2_KERNEL_REGULAR = 1,
  FA2_KERNEL_SHORT = 2
};

/* Bytes of device workspace fa2_fwd needs for `p` (0 is possible).
 * Replaces the reference's per-call torch.empty of running_sum/max/acc
 * (attention.py:852-864).  fp32 tensors with FA2_ARITH_REFERENCE at
 * head_dim 64/128 (dense, ragged) also hold fp16 copies of q, k and v there,
 * as the reference rounds every fp32 operand to fp16.  Paged calls with one
 * q-block per sequence and more two-head units than compute units hold the
 * partials of units their balanced walk cuts into pieces (4 * CUs * 128 *
 * (2 + head_dim) * 4 bytes).  Host-only: touches
 * no device state except a one-time, cached query of the current device's
 * compute-unit count. */
int fa2_fwd_workspace_size(const fa2_params* p, size_t* bytes);

/* Validate `p` and enqueue the forward pass on `stream` (a hipStream_t;
 * NULL = the legacy default stream).  Replaces attention.py:836-925
 * (split heuristic, workspace, partial + merge launches).  Returns FA2_OK
 * or an error code; validation errors are reported before any launch. */
int fa2_fwd(const fa2_params* p, void* stream);

/* fa2_fwd for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  `p->workspace` is ignored: the ragged/paged
 * work list and the split-KV partials live in a static device array of
 * FA2_NOALLOC_SCRATCH_BYTES that the library holds on every device it runs on
 * until the process ends.  Paged calls that fa2_fwd runs with the balanced
 * walk run whole units here (the walk's partial slots do not fit the array);
 * automatic splits (num_splits = 0) are reduced until
 * the call fits that array, and fp32 tensors whose fp16 copies do not fit
 * run the register-staged kernel instead; a call that still does not fit, or
 * a forced num_splits that does not, returns FA2_ERR_SCRATCH before any launch.  The
 * entry point calls no allocating routine.  Every call on one device shares
 * that device's array: calls that overlap in time on one device (e.g. on two
 * streams) race and give wrong results; serialise them.  Otherwise the same
 * contract and results as fa2_fwd (bit-identical when the split factor and
 * the kernel are the same). */
#define FA2_NOALLOC_SCRATCH_BYTES (32u << 20)
int fa2_fwd_noalloc(const fa2_params* p, void* stream);

/* Static, human-readable text for a status code. */
const char* fa2_strerror(int status);

/* ---- decode and speculative decode ---------------------------------------
 *
 * The same parameter block serves `decode_attention` and
 * `speculative_decode_attention`, with these meanings:
 *   q, o      [B, Hq, M, D] for EVERY layout (M = q_len >= 1 query tokens per
 *             sequence: 1 for decode, the draft length for speculative decode;
 *             `decode_attention`'s [B, Hq, D] is M = 1);
 *   k, v      per `layout` exactly as above (dense [B,Hkv,N,D]; ragged
 *             [Tkv,Hkv,D] with kv_indptr = prefix sums [B+1]; paged caches
 *             with kv_indptr = lengths [B] and block tables); q_indptr unused;
 *   mask      FA2_MASK_NONE, or FA2_MASK_CAUSAL_BOTTOM_RIGHT for the
 *             speculative causal mask: query token m of a sequence of Lk keys
 *             sees key j iff j <= Lk - M + m (the last M keys are the drafts);
 *             FA2_MASK_CAUSAL_TOP_LEFT is rejected;
 *   layout of q/o: the Hq/Hkv heads of one kv head must be one run of rows,
 *             q_sh == q_len * q_ss (true for contiguous tensors; for M = 1 the
 *             row stride is the head stride, q_ss = q_sh); likewise o.
 * Internally the Hq/Hkv query heads that share a kv head are computed as the
 * rows of one unit, so each K/V row is read from HBM once per kv head.  The
 * computation is that of fa2_fwd (same dtypes and rounding, fp32 softmax
 * statistics).  A sequence with no visible key gives NaN rows (the
 * reference's 0/0, kernels/decode.py:318-327).
 *
 * Reference interfaces replaced:
 *   kernels/decode.py:203-331             `decode_attention` host wrapper
 *   kernels/decode.py:22-170, 173-200     split kernel + merge kernel
 *   kernels/speculative_decode.py:228-365 `speculative_decode_attention`
 *   kernels/speculative_decode.py:22-225  split kernel + merge kernel      */

/* Bytes of device workspace fa2_decode_fwd needs for `p`. */
int fa2_decode_workspace_size(const fa2_params* p, size_t* bytes);

/* Validate `p` and enqueue decode / speculative-decode attention on `stream`
 * (a hipStream_t).  Returns FA2_OK or an error code; validation errors are
 * reported before any launch.  No allocation, no host synchronisation. */
int fa2_decode_fwd(const fa2_params* p, void* stream);

/* Number of bounded waits in the fp16/bf16 decode kernel that gave up on the
 * current device since the library was loaded (or since the last reset),
 * into *count; reset != 0 sets it back to 0.  A wait gives up only if a
 * ring counter never reaches its target (never, in a correct run) or under a
 * tiny decode_spin_cap; the rows of such a workgroup are then NaN.
 * Synchronous (a device-to-host copy).  No counterpart in the reference: a
 * diagnostic for callers that want to assert no wait ever gave up. */
int fa2_decode_wait_giveups(uint32_t* count, int reset);

/* ---- paged KV-cache writer -------------------------------------------------
 *
 * Writes new K/V rows into the paged caches the attention entry points read.
 * The reference has no kernel for this step: its paged layout is built on
 * the host by tests/test_attention.py:101-134 (`allocate_paged_cache`, pages
 * in sequence order, table padding 0), tests/test_decode.py:93-130 and
 * benchmarks/attention.py:351-431 (`build_paged_cache`, padding -1).  The
 * format is theirs: a cache is [num_pages * page_size, kv_heads, head_dim],
 * and logical row n of sequence b lives at row
 * table[b][n / page_size] * page_size + n % page_size.
 *
 * Sequence b's new rows k_new[new_indptr[b] + j] (j < new_indptr[b+1] -
 * new_indptr[b]) go to logical positions start_pos[b] + j (start_pos NULL:
 * 0, i.e. building a cache; the current lengths: appending decode tokens).
 * Rows whose logical page is >= table_width, or whose table entry is outside
 * [0, num_pages), are skipped (never written).  v_new, v_cache and
 * v_block_table may all be NULL: then only K is written.  Strides are in ELEMENTS;
 * head_dim must be contiguous and rows 16-byte aligned; k_new/v_new share
 * strides, as do the two caches.  No allocation, no host synchronisation. */
typedef struct fa2_kv_append_params {
  int32_t dtype;            /* enum fa2_dtype of caches and new rows          */
  int32_t reserved0;
  int64_t batch;            /* B                                               */
  int64_t kv_heads;         /* H                                               */
  int64_t head_dim;         /* D                                               */
  int64_t num_rows;         /* rows of k_new / v_new (= new_indptr[B])         */
  int64_t page_size;        /* P (tokens per page)                             */
  int64_t num_pages;        /* pages of each cache (cache rows / P)            */
  int64_t table_width;      /* columns of the block tables                     */
  int64_t k_table_stride;   /* row strides of the block tables (elements)      */
  int64_t v_table_stride;
  int64_t new_ts, new_hs;   /* element strides (row, head) of k_new / v_new    */
  int64_t cache_ts, cache_hs; /* element strides (row, head) of the caches     */
  const void* k_new;
  const void* v_new;
  void* k_cache;
  void* v_cache;
  const int32_t* new_indptr;    /* [B+1] prefix sums over the new rows         */
  const int32_t* start_pos;     /* [B] first logical position, or NULL (0)     */
  const int32_t* k_block_table; /* [B, table_width]                            */
  const int32_t* v_block_table;
} fa2_kv_append_params;

/* Validate `p` and enqueue the writes on `stream`.  Returns FA2_OK or an
 * error code (before any launch). */
int fa2_kv_append(const fa2_kv_append_params* p, void* stream);

/* sizeof(fa2_kv_append_params) as compiled into the library (binding check). */
size_t fa2_kv_append_params_size(void);

/* Version of this ABI (bumped on any change to fa2_params or the entry points).  No counterpart
 * in the reference: lets a binding refuse a library it was not written for. */
int fa2_abi_version(void);

/* sizeof(fa2_params) as compiled into the library.  No counterpart in the
 * reference: lets an FFI binding (ctypes here) check its struct mirror. */
size_t fa2_params_size(void);

#ifdef __cplusplus
}
#endif

#endif /* FA2_H_ */
