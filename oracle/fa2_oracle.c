/*
 * fa2_oracle.c - CPU restatement of harsh-vsingh/triton-kernels
 * `flash_attention_v2` (kernels/attention.py:430-927).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests,
 * `__graft_entry__.smoke()` and bench.py's CPU-baseline leg compare the HIP
 * kernels against.  Nothing in the product path loads it.
 *
 * What is restated, and from where:
 *   - layouts and the meaning of q_indptr / kv_indptr / block tables
 *     (attention.py:465-514, 766-834): dense [B,H,S,D]; ragged token-major
 *     [T,H,D] with exclusive prefix sums; paged KV [pages*P,Hkv,D] whose
 *     per-sequence LENGTHS are in kv_indptr and whose table row b holds the
 *     physical page of logical page n//P (attention.py:575-594, 617-633);
 *   - head map kv_head = h * Hkv / Hq (attention.py:463);
 *   - the q-block loop bound for causal masks (attention.py:553-557) and the
 *     top-left causal mask q_idx >= k_idx plus k_idx < Lk (:563-569);
 *   - the split-K partial recurrence over key blocks pid2, pid2+S, ...
 *     (attention.py:559-636): scores in fp32 scaled by head_dim**-0.5,
 *     running max m, alpha = exp(m_old - m_new), P = exp(S - m_new) rounded
 *     to the operand type, l = l*alpha + sum(P), acc = acc*alpha + P V;
 *   - the log-sum-exp merge across splits (attention.py:697-724),
 *     including its 0/0 = NaN for a row that sees no key.
 * Extensions used only by this build's tests: a bottom-right causal
 * alignment (key j visible iff j <= i + Lk - Lq) and a selectable rounding
 * of the operands and of P (none / fp16 as the reference / bf16), so that
 * the same code states both the reference's numerics and those of the bf16
 * MFMA kernel.
 *
 * Rows are independent, so the restatement walks one query row at a time
 * through exactly the key blocks its q-block (BLOCK_M = 64, :843) visits.
 * Built with OpenMP (oracle/Makefile), the (sequence, q head) units run on
 * several threads; each row's arithmetic is the same sequential code, so
 * the results do not depend on the thread count.
 */
#include "fa2_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- rounding (round-to-nearest-even) ---------------------------------- */

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> bf16 -> fp32 */
float fa2o_round_bf16(float x) {
  uint32_t u = f2u(x);
  if ((u & 0x7f800000u) == 0x7f800000u) { /* inf / nan */
    if (u & 0x007fffffu) return u2f(u | 0x00400000u);
    return x;
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return u2f(u & 0xffff0000u);
}

/* fp32 -> fp16 -> fp32 (IEEE binary16, subnormals kept, overflow to inf) */
float fa2o_round_f16(float x) {
  if (isnan(x)) return x;
  float ax = fabsf(x);
  if (ax >= 65520.0f) return copysignf(INFINITY, x); /* rounds past max finite 65504 */
  if (ax < 6.103515625e-05f) {                       /* subnormal range: quantum 2^-24 */
    const float q = 5.9604644775390625e-08f;
    float t = ax / q;                                /* exact: power-of-two divisor */
    float r = nearbyintf(t);                         /* default mode: ties to even */
    return copysignf(r * q, x);
  }
  /* normal range: keep 11 significant bits */
  int e;
  frexpf(ax, &e);                                    /* ax = m * 2^e, m in [0.5,1) */
  float q = ldexpf(1.0f, e - 11);
  float r = nearbyintf(ax / q) * q;
  return copysignf(r, x);
}

static float rnd(float x, int mode) {
  if (mode == FA2O_ROUND_F16) return fa2o_round_f16(x);
  if (mode == FA2O_ROUND_BF16) return fa2o_round_bf16(x);
  return x;
}

/* ---- addressing --------------------------------------------------------- */

typedef struct {
  int64_t Lq, Lk;
  int64_t q_base, o_base, k_base, v_base; /* element offsets (paged k/v: head only) */
} seq_t;

static void seq_info(const fa2o_args* a, int64_t b, int64_t h, int64_t kvh, seq_t* s) {
  if (a->layout == FA2O_LAYOUT_DENSE) {
    s->Lq = a->q_len;
    s->Lk = a->kv_len;
    s->q_base = b * a->q_sb + h * a->q_sh;
    s->o_base = b * a->o_sb + h * a->o_sh;
    s->k_base = b * a->k_sb + kvh * a->k_sh;
    s->v_base = b * a->v_sb + kvh * a->v_sh;
  } else if (a->layout == FA2O_LAYOUT_RAGGED) {
    int64_t qs = a->q_indptr[b], ks = a->kv_indptr[b];
    s->Lq = a->q_indptr[b + 1] - qs;
    s->Lk = a->kv_indptr[b + 1] - ks;
    s->q_base = qs * a->q_ss + h * a->q_sh;
    s->o_base = qs * a->o_ss + h * a->o_sh;
    s->k_base = ks * a->k_ss + kvh * a->k_sh;
    s->v_base = ks * a->v_ss + kvh * a->v_sh;
  } else {
    s->Lq = a->q_len;
    s->Lk = a->kv_indptr[b];
    s->q_base = b * a->q_sb + h * a->q_sh;
    s->o_base = b * a->o_sb + h * a->o_sh;
    s->k_base = kvh * a->k_sh;
    s->v_base = kvh * a->v_sh;
  }
  if (s->Lq < 0) s->Lq = 0;
  if (s->Lk < 0) s->Lk = 0;
}

/* element offset of key n's row (without the column) */
static int64_t key_row(const fa2o_args* a, const seq_t* s, int64_t b, int64_t n, int is_v) {
  if (a->layout == FA2O_LAYOUT_PAGED) {
    const int32_t* tbl = is_v ? a->v_table : a->k_table;
    int64_t ts = is_v ? a->v_table_stride : a->k_table_stride;
    int64_t page = tbl[b * ts + n / a->page_size];
    int64_t row = page * a->page_size + (a->mutation == FA2O_MUT_PAGE_OFFSET ? 0 : n % a->page_size);
    return (is_v ? s->v_base : s->k_base) + row * (is_v ? a->v_ss : a->k_ss);
  }
  return (is_v ? s->v_base : s->k_base) + n * (is_v ? a->v_ss : a->k_ss);
}

/* ---- forward ------------------------------------------------------------- */

int fa2o_fwd(const fa2o_args* a) {
  if (!a || !a->q || !a->k || !a->v || !a->o) return 1;
  if (a->q_heads <= 0 || a->kv_heads <= 0 || a->q_heads % a->kv_heads) return 2;
  if (a->block_m <= 0 || a->block_n <= 0 || a->split_k <= 0) return 3;
  const int64_t D = a->head_dim, BM = a->block_m, BN = a->block_n, S = a->split_k;
  const int opr = a->operand_round, prd = a->p_round;

  /* (sequence, q head) units are independent and write disjoint rows:
   * spread over threads when built with OpenMP; each row's arithmetic is
   * the same sequential code either way */
  const int64_t units = a->batch * a->q_heads;
  int err = 0;
#ifdef _OPENMP
#pragma omp parallel
#endif
  {
  float* qv = (float*)malloc(sizeof(float) * D);
  float* sc = (float*)malloc(sizeof(float) * BN);
  float* acc = (float*)malloc(sizeof(float) * S * D);
  float* mm = (float*)malloc(sizeof(float) * S);
  float* ll = (float*)malloc(sizeof(float) * S);
  const int ok = qv && sc && acc && mm && ll;
  if (!ok) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
    err = 4;
  }

#ifdef _OPENMP
#pragma omp for schedule(dynamic)
#endif
  for (int64_t u = 0; u < units; ++u) {
    {
      if (!ok) continue;
      const int64_t b = u / a->q_heads, h = u % a->q_heads;
      const int64_t kvh = (a->mutation == FA2O_MUT_HEAD_MAP) ? h % a->kv_heads
                                                              : h * a->kv_heads / a->q_heads;
      seq_t s;
      seq_info(a, b, h, kvh, &s);
      const int64_t off = (a->mask == FA2O_MASK_CAUSAL_BOTTOM_RIGHT) ? s.Lk - s.Lq : 0;
      for (int64_t i = 0; i < s.Lq; ++i) {
        /* the q-block's key-block bound (attention.py:553-557) */
        const int64_t blk_m = (i / BM) * BM;
        int64_t nblocks;
        if (a->mask == FA2O_MASK_CAUSAL_TOP_LEFT) {
          /* reference: cdiv(min(blk_m + BLOCK_M, Lq), BLOCK_N), not clamped to Lk */
          const int64_t last_q = blk_m + BM < s.Lq ? blk_m + BM : s.Lq;
          nblocks = (last_q + BN - 1) / BN;
        } else if (a->mask == FA2O_MASK_CAUSAL_BOTTOM_RIGHT) {
          const int64_t last_q = blk_m + BM < s.Lq ? blk_m + BM : s.Lq;
          int64_t end = last_q + off;
          if (end > s.Lk) end = s.Lk;
          nblocks = end > 0 ? (end + BN - 1) / BN : 0;
        } else {
          nblocks = (s.Lk + BN - 1) / BN;
        }
        for (int64_t d = 0; d < D; ++d) qv[d] = rnd(a->q[s.q_base + i * a->q_ss + d], opr);
        for (int64_t sp = 0; sp < S; ++sp) {
          float m = -INFINITY, l = 0.f;
          float* ac = acc + sp * D;
          for (int64_t d = 0; d < D; ++d) ac[d] = 0.f;
          for (int64_t kb = sp; kb < nblocks; kb += S) {
            float bmax = -INFINITY;
            for (int64_t j = 0; j < BN; ++j) {
              const int64_t n = kb * BN + j;
              int ok = n < s.Lk;
              if (ok && a->mask != FA2O_MASK_NONE)
                ok = (a->mutation == FA2O_MUT_CAUSAL_OFF1) ? n < i + off : n <= i + off;
              if (!ok) {
                sc[j] = -INFINITY;
                continue;
              }
              const float* kr = a->k + key_row(a, &s, b, n, 0);
              float dot = 0.f;
              for (int64_t d = 0; d < D; ++d) dot += qv[d] * rnd(kr[d], opr);
              sc[j] = (a->mutation == FA2O_MUT_NO_SCALE) ? dot : dot * a->scale;
              if (sc[j] > bmax) bmax = sc[j];
            }
            const float mnew = m > bmax ? m : bmax;
            const float alpha = expf(m - mnew); /* -inf - -inf = NaN, as the reference */
            float psum = 0.f;
            if (a->mutation != FA2O_MUT_NO_RESCALE)
              for (int64_t d = 0; d < D; ++d) ac[d] *= alpha;
            for (int64_t j = 0; j < BN; ++j) {
              const float p = rnd(expf(sc[j] - mnew), prd);
              psum += p;
              const int64_t n = kb * BN + j;
              if (n < s.Lk) {
                const float* vr = (a->mutation == FA2O_MUT_K_AS_V) ? a->k + key_row(a, &s, b, n, 0)
                                                                   : a->v + key_row(a, &s, b, n, 1);
                for (int64_t d = 0; d < D; ++d) ac[d] += p * rnd(vr[d], opr);
              } else {
                /* rows past the length load as 0.0 (attention.py:613-633) */
                for (int64_t d = 0; d < D; ++d) ac[d] += p * 0.0f;
              }
            }
            l = l * alpha + psum;
            m = mnew;
          }
          mm[sp] = m;
          ll[sp] = l;
        }
        /* merge (attention.py:710-724) */
        float g = -INFINITY;
        for (int64_t sp = 0; sp < S; ++sp) g = mm[sp] > g ? mm[sp] : g;
        float tot = 0.f;
        float* orow = a->o + s.o_base + i * a->o_ss;
        for (int64_t d = 0; d < D; ++d) orow[d] = 0.f;
        for (int64_t sp = 0; sp < S; ++sp) {
          const float w = expf(mm[sp] - g);
          tot += ll[sp] * w;
          for (int64_t d = 0; d < D; ++d) orow[d] += acc[sp * D + d] * w;
        }
        for (int64_t d = 0; d < D; ++d) orow[d] = orow[d] / tot;
      }
    }
  }
  free(qv); free(sc); free(acc); free(mm); free(ll);
  }
  return err;
}

/* ---- decode_attention / speculative_decode_attention --------------------
 *
 * Restates kernels/decode.py (spec = 0) and kernels/speculative_decode.py
 * (spec = 1).  q and o are [B, Hq, M, D] for every K/V layout (decode: M = 1,
 * the reference's [B, Hq, D]); K/V follow a->layout as above, with
 * kv_indptr = prefix sums (ragged, decode.py:57-66) or lengths (paged,
 * decode.py:68-75); the dense layout gives every sequence kv_len keys
 * (decode.py:55).  Per (sequence, q head, query m):
 *   - key blocks of BLOCK_N, block i handled by split i % S (the loop
 *     `while pid0 < total: ... pid0 += SPLIT_K`, decode.py:88-162,
 *     speculative_decode.py:95-178);
 *   - scores in fp32, scaled, -inf past the sequence end (decode.py:146-149)
 *     and, speculative + causal, for drafts after m: key n is hidden iff
 *     n >= Lk - M and n - (Lk - M) > m (speculative_decode.py:89, 155-160);
 *   - decode: m' = max(m, max_j s_j), alpha = exp(m - m'), P = exp(s - m'),
 *     acc = acc*alpha + sum P v, l = l*alpha + sum P (decode.py:151-160);
 *   - speculative: the same with a guarded max - while no key has been
 *     visible the stabiliser is 0 and alpha, P are 0
 *     (speculative_decode.py:165-177);
 *   - merge: g = max_s m_s, O = sum_s e^(m_s - g) acc_s / sum_s e^(m_s - g) l_s
 *     (decode.py:188-200, speculative_decode.py:211-226); a sequence with no
 *     visible key gives 0/0 = NaN.
 * The reference computes these in fp32 from upcast inputs (decode.py:96-144);
 * its speculative kernel forms Q K^T and P V with tl.dot on fp32 operands,
 * which NVIDIA hardware may run in TF32: the restatement keeps those
 * products in fp32 (operand_round / p_round "none"), a difference far below
 * the reference tolerance.  operand_round / p_round select the rounding of
 * this build's MFMA kernels for the strict error-floor comparison. */
int fa2o_decode(const fa2o_args* a, int spec) {
  if (!a || !a->q || !a->k || !a->v || !a->o) return 1;
  if (a->q_heads <= 0 || a->kv_heads <= 0 || a->q_heads % a->kv_heads) return 2;
  if (a->block_n <= 0 || a->split_k <= 0 || a->q_len <= 0) return 3;
  const int64_t D = a->head_dim, BN = a->block_n, S = a->split_k, M = a->q_len;
  const int opr = a->operand_round, prd = a->p_round;
  const int causal = a->mask != FA2O_MASK_NONE;

  /* (sequence, q head) units are independent and write disjoint rows:
   * spread over threads when built with OpenMP; each row's arithmetic is
   * the same sequential code either way */
  const int64_t units = a->batch * a->q_heads;
  int err = 0;
#ifdef _OPENMP
#pragma omp parallel
#endif
  {
  float* qv = (float*)malloc(sizeof(float) * D);
  float* sc = (float*)malloc(sizeof(float) * BN);
  float* acc = (float*)malloc(sizeof(float) * S * D);
  float* mm = (float*)malloc(sizeof(float) * S);
  float* ll = (float*)malloc(sizeof(float) * S);
  const int ok = qv && sc && acc && mm && ll;
  if (!ok) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
    err = 4;
  }
#ifdef _OPENMP
#pragma omp for schedule(dynamic)
#endif
  for (int64_t u = 0; u < units; ++u) {
    {
      if (!ok) continue;
      const int64_t b = u / a->q_heads, h = u % a->q_heads;
      const int64_t kvh = (a->mutation == FA2O_MUT_HEAD_MAP) ? h % a->kv_heads
                                                              : h * a->kv_heads / a->q_heads;
      seq_t s;
      s.Lq = M;
      s.q_base = b * a->q_sb + h * a->q_sh;
      s.o_base = b * a->o_sb + h * a->o_sh;
      if (a->layout == FA2O_LAYOUT_DENSE) {
        s.Lk = a->kv_len;
        s.k_base = b * a->k_sb + kvh * a->k_sh;
        s.v_base = b * a->v_sb + kvh * a->v_sh;
      } else if (a->layout == FA2O_LAYOUT_RAGGED) {
        const int64_t ks = a->kv_indptr[b];
        s.Lk = a->kv_indptr[b + 1] - ks;
        s.k_base = ks * a->k_ss + kvh * a->k_sh;
        s.v_base = ks * a->v_ss + kvh * a->v_sh;
      } else {
        s.Lk = a->kv_indptr[b];
        s.k_base = kvh * a->k_sh;
        s.v_base = kvh * a->v_sh;
      }
      if (s.Lk < 0) s.Lk = 0;
      const int64_t draft_start = s.Lk - M;
      const int64_t total = (s.Lk + BN - 1) / BN;
      for (int64_t i = 0; i < M; ++i) {
        for (int64_t d = 0; d < D; ++d) qv[d] = rnd(a->q[s.q_base + i * a->q_ss + d], opr);
        for (int64_t sp = 0; sp < S; ++sp) {
          float m = -INFINITY, l = 0.f;
          float* ac = acc + sp * D;
          for (int64_t d = 0; d < D; ++d) ac[d] = 0.f;
          for (int64_t kb = sp; kb < total; kb += S) {
            float bmax = -INFINITY;
            for (int64_t j = 0; j < BN; ++j) {
              const int64_t n = kb * BN + j;
              int ok = n < s.Lk;
              if (ok && causal && n >= draft_start)
                ok = (a->mutation == FA2O_MUT_CAUSAL_OFF1) ? n - draft_start < i
                                                           : n - draft_start <= i;
              if (!ok) {
                sc[j] = -INFINITY;
                continue;
              }
              const float* kr = a->k + key_row(a, &s, b, n, 0);
              float dot = 0.f;
              for (int64_t d = 0; d < D; ++d) dot += qv[d] * rnd(kr[d], opr);
              sc[j] = (a->mutation == FA2O_MUT_NO_SCALE) ? dot : dot * a->scale;
              if (sc[j] > bmax) bmax = sc[j];
            }
            float mnew = m > bmax ? m : bmax;
            float alpha;
            int none = 0;
            if (spec) {
              none = mnew == -INFINITY;
              if (none) mnew = 0.f;
              alpha = none ? 0.f : expf(m - mnew);
            } else {
              alpha = expf(m - mnew);
            }
            float psum = 0.f;
            if (a->mutation != FA2O_MUT_NO_RESCALE)
              for (int64_t d = 0; d < D; ++d) ac[d] *= alpha;
            for (int64_t j = 0; j < BN; ++j) {
              const int64_t n = kb * BN + j;
              const float p = none ? 0.f : rnd(expf(sc[j] - mnew), prd);
              psum += p;
              if (n < s.Lk && p != 0.f) {
                const float* vr = (a->mutation == FA2O_MUT_K_AS_V) ? a->k + key_row(a, &s, b, n, 0)
                                                                   : a->v + key_row(a, &s, b, n, 1);
                for (int64_t d = 0; d < D; ++d) ac[d] += p * rnd(vr[d], opr);
              }
            }
            l = l * alpha + psum;
            m = mnew;
          }
          mm[sp] = m;
          ll[sp] = l;
        }
        float g = -INFINITY;
        for (int64_t sp = 0; sp < S; ++sp) g = mm[sp] > g ? mm[sp] : g;
        float tot = 0.f;
        float* orow = a->o + s.o_base + i * a->o_ss;
        for (int64_t d = 0; d < D; ++d) orow[d] = 0.f;
        for (int64_t sp = 0; sp < S; ++sp) {
          const float w = expf(mm[sp] - g);
          tot += ll[sp] * w;
          for (int64_t d = 0; d < D; ++d) orow[d] += acc[sp * D + d] * w;
        }
        for (int64_t d = 0; d < D; ++d) orow[d] = orow[d] / tot;
      }
    }
  }
  free(qv); free(sc); free(acc); free(mm); free(ll);
  }
  return err;
}

