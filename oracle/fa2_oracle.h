/*
 * fa2_oracle.h - CPU restatement of the reference flash_attention_v2
 * (harsh-vsingh/triton-kernels kernels/attention.py:430-927), decode_attention
 * (kernels/decode.py:22-331) and speculative_decode_attention
 * (kernels/speculative_decode.py:22-365).
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * CPU-baseline leg of bench.py as the checker; never by the product path.
 *
 * Inputs are fp32 host arrays holding values already representable in the
 * tensor dtype under test (an exact upcast of fp16/bf16 data).  Strides and
 * layouts follow include/fa2.h.
 */
#ifndef FA2_ORACLE_H_
#define FA2_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { FA2O_LAYOUT_DENSE = 0, FA2O_LAYOUT_RAGGED = 1, FA2O_LAYOUT_PAGED = 2 };
enum { FA2O_MASK_NONE = 0, FA2O_MASK_CAUSAL_TOP_LEFT = 1, FA2O_MASK_CAUSAL_BOTTOM_RIGHT = 2 };
enum { FA2O_ROUND_NONE = 0, FA2O_ROUND_F16 = 1, FA2O_ROUND_BF16 = 2 };
/* Planted mistakes, used only by tests that show each pinning check fails
 * on a plausible bug: */
enum {
  FA2O_MUT_NONE = 0,
  FA2O_MUT_NO_RESCALE = 1,   /* acc not multiplied by alpha               */
  FA2O_MUT_CAUSAL_OFF1 = 2,  /* causal mask j < i instead of j <= i       */
  FA2O_MUT_HEAD_MAP = 3,     /* kv head h % Hkv instead of h * Hkv / Hq   */
  FA2O_MUT_K_AS_V = 4,       /* P multiplies K instead of V               */
  FA2O_MUT_NO_SCALE = 5,     /* softmax scale dropped                     */
  FA2O_MUT_PAGE_OFFSET = 6   /* paged row = page * P (offset n % P lost)  */
};

typedef struct fa2o_args {
  int32_t layout, mask;
  int32_t operand_round; /* rounding applied to q, k, v before use        */
  int32_t p_round;       /* rounding applied to P before P V and sum(P)   */
  int32_t block_m;       /* reference: 64 (attention.py:843)              */
  int32_t block_n;       /* reference: autotuned 32/64/128 (:367-419)     */
  int32_t split_k;       /* reference: attention.py:836-841               */
  int32_t mutation;      /* 0; >0 plants a known mistake (tests of the checks) */
  int64_t batch, q_heads, kv_heads, head_dim, q_len, kv_len;
  int64_t q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, o_sb, o_sh, o_ss;
  const float* q;
  const float* k;
  const float* v;
  float* o;
  const int32_t* q_indptr;
  const int32_t* kv_indptr;
  const int32_t* k_table;
  const int32_t* v_table;
  int64_t k_table_stride, v_table_stride, page_size;
  float scale;
  int32_t reserved2;
} fa2o_args;

int fa2o_fwd(const fa2o_args* a);
/* decode_attention (spec = 0, kernels/decode.py) and
 * speculative_decode_attention (spec = 1, kernels/speculative_decode.py):
 * q/o [B, Hq, M = q_len, D] for every K/V layout; mask NONE or, speculative
 * causal, BOTTOM_RIGHT (draft m sees key n iff n <= Lk - M + m). */
int fa2o_decode(const fa2o_args* a, int spec);
float fa2o_round_f16(float x);
float fa2o_round_bf16(float x);

#ifdef __cplusplus
}
#endif

#endif
