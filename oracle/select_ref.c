/*
 * Slot-literal CPU restatement of the reference's top-k selection kernel.
 *
 * TEST INFRASTRUCTURE ONLY: linked by tests/ and bench.py's CPU-baseline leg,
 * never by the product library.
 *
 * Restates, step by step, `lighthouse_selection_chunked_topk_kernel` and its
 * wrapper from src/lighthouse_selection_cuda.py (reference repository):
 *   - bitonic_sort_descending            :41-110
 *   - per-(b, h, tile) block body        :114-331
 *       level loop / c_l / K_end          :162-187
 *       qk and kq streaming sorts         :189-258
 *       kq-reject emission after warm-up  :260-272
 *       final [TQ | TK] emission          :274-289
 *       level-1 leaf emission             :293-322
 *       parents for the next level        :324-327
 *   - slot sizing, -1 fill, int32 key sort + gather  :383-400, :425-427
 *
 * Unlike the structural formulation in lh_oracle.py, this one writes every
 * entry into the reference's output slot (`out_off` bookkeeping included) and
 * then sorts the int32 keys, exactly as the reference does.  The two
 * formulations are compared by the tests.
 *
 * Keys: float_to_ordered_uint of c_l*i (unselected) or c_l*(i+1) - 2^(1-l)
 * (selected), :11-25.  2^(1-l) is computed exactly with ldexpf, and the level
 * offsets with exact integer sums of the level lengths (equal to the
 * reference's closed form whenever S is a multiple of p^(L-1)).
 *
 * mode 0 ("strict"): the reference's own slot layout; the geometry must be
 *   inside the domain where the reference neither asserts nor overruns.
 * mode 1 ("generalized"): each tile writes into a private slot range large
 *   enough for its emissions; holes are dropped after the key sort.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TOPK 128
#define HALF 64
#define SENT (-1e6f)

static void sort128(float *s, int *x, int tie_lower) {
  for (int k = 2; k <= TOPK; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = 0; i < TOPK; ++i) {
        int ixj = i ^ j;
        if (ixj <= i) continue;
        int desc = (i & k) == 0;
        float a = s[i], b = s[ixj];
        int swap;
        if (!tie_lower) {
          swap = desc ? (a < b) : (a > b);
        } else {
          long long ai = x[i] < 0 ? (1LL << 40) : x[i];
          long long bi = x[ixj] < 0 ? (1LL << 40) : x[ixj];
          int b_better = (b > a) || (b == a && bi < ai);
          int a_better = (a > b) || (a == b && ai < bi);
          swap = desc ? b_better : a_better;
        }
        if (swap) {
          s[i] = b; s[ixj] = a;
          int t = x[i]; x[i] = x[ixj]; x[ixj] = t;
        }
      }
    }
  }
}

static int32_t ordered_key(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t o = (f >= 0.0f) ? (u ^ 0x80000000u) : (~u);
  return (int32_t)o;
}

/* One block of the reference kernel.  keys/vals point at this tile's first
 * slot; `cap` bounds the slots this tile may write (mode 1).  Returns the
 * number of slots advanced (final out_off), or -1 on a write past `cap`. */
static int run_tile(const float *sq, const float *sk, int32_t *keys, int32_t *vals, int cap,
                    int L, int p, int N, int tile, int NCC, int tie_lower) {
  int parent[TOPK];
  float tq_s[HALF], tk_s[HALF], ss[TOPK];
  int tq_x[HALF], tk_x[HALF], sx[TOPK];
  int shift = 0;
  while ((1 << shift) < p) ++shift;
  for (int i = 0; i < TOPK; ++i) parent[i] = -1;
  int out_off = 0;
  int tile_start = tile * NCC, tile_end = tile_start + NCC;

  for (int level = L; level >= 1; --level) {
    int c_l = 1;
    for (int i = 0; i < level - 1; ++i) c_l *= p;
    int K_end = N / c_l - 1;
    int level_offset = 0;
    for (int l = 1, c = 1; l < level; ++l, c *= p) level_offset += N / c;
    int num_K, use_parents;
    if (level == L) { num_K = tile_end - tile_start; use_parents = 0; }
    else { num_K = p * TOPK; use_parents = 1; }
    int K_end_abs = (K_end >= 0) ? (K_end + level_offset) : -1;

    if (level > 1) {
      for (int i = 0; i < HALF; ++i) { tq_s[i] = SENT; tq_x[i] = -1; tk_s[i] = SENT; tk_x[i] = -1; }
      int nb = (num_K + HALF - 1) / HALF;
      for (int batch = 0; batch < nb; ++batch) {
        int kv_start = batch * HALF;
        for (int t = 0; t < HALF; ++t) { ss[t] = tq_s[t]; sx[t] = tq_x[t]; }
        for (int bi = 0; bi < HALF; ++bi) {
          int abs_col = kv_start + bi, K_idx = -1;
          if (abs_col < num_K) {
            if (use_parents) {
              int pidx = abs_col >> shift, coff = abs_col & (p - 1);
              int pval = (pidx < TOPK) ? parent[pidx] : -1;
              if (pval >= 0) { K_idx = pval * p + coff; if (K_idx > K_end || K_idx < 0) K_idx = -1; }
            } else {
              K_idx = tile_start + abs_col;
            }
          }
          int K_abs = (K_idx >= 0) ? K_idx + level_offset : -1;
          int valid = K_abs >= 0 && K_abs <= K_end_abs && K_end >= 0;
          ss[HALF + bi] = valid ? sq[K_abs] : SENT;
          sx[HALF + bi] = K_idx;
        }
        sort128(ss, sx, tie_lower);
        int rej[HALF];
        for (int t = 0; t < HALF; ++t) { tq_s[t] = ss[t]; tq_x[t] = sx[t]; rej[t] = sx[HALF + t]; }
        for (int t = 0; t < HALF; ++t) { ss[t] = tk_s[t]; sx[t] = tk_x[t]; }
        for (int t = 0; t < HALF; ++t) {
          int r = rej[t];
          int ra = (r >= 0) ? r + level_offset : -1;
          int v = ra >= 0 && ra <= K_end_abs && K_end >= 0;
          ss[HALF + t] = v ? sk[ra] : SENT;
          sx[HALF + t] = r;
        }
        sort128(ss, sx, tie_lower);
        for (int t = 0; t < HALF; ++t) { tk_s[t] = ss[t]; tk_x[t] = sx[t]; }
        if (batch >= TOPK / HALF) {
          for (int t = 0; t < HALF; ++t) {
            int d = sx[HALF + t];
            int da = (d >= 0) ? d + level_offset : -1;
            if (da >= 0 && da <= K_end_abs && K_end >= 0) {
              int slot = out_off + t;
              if (slot >= cap) return -1;
              keys[slot] = ordered_key((float)(c_l * d));
              vals[slot] = da;
            }
          }
          out_off += HALF;
        }
        if (batch == nb - 1) {
          for (int t = 0; t < TOPK; ++t) {
            int ti = t < HALF ? tq_x[t] : tk_x[t - HALF];
            if (ti >= 0) {
              int slot = out_off + t;
              if (slot >= cap) return -1;
              float f = (float)(c_l * (ti + 1)) - ldexpf(1.0f, 1 - level);
              keys[slot] = ordered_key(f);
              vals[slot] = ti + level_offset;
            }
          }
          out_off += TOPK;
        }
      }
    } else {
      int nb = (num_K + TOPK - 1) / TOPK;
      for (int batch = 0; batch < nb; ++batch) {
        int kv_start = batch * TOPK;
        for (int t = 0; t < TOPK; ++t) {
          int abs_col = kv_start + t, K_idx = -1;
          if (abs_col < num_K) {
            int pidx = abs_col >> shift, coff = abs_col & (p - 1);
            int pval = (pidx < TOPK) ? parent[pidx] : -1;
            if (pval >= 0) { K_idx = pval * p + coff; if (K_idx > K_end || K_idx < 0) K_idx = -1; }
          }
          int K_abs = (K_idx >= 0) ? K_idx + level_offset : -1;
          if (K_abs >= 0 && K_abs <= K_end_abs && K_end >= 0) {
            int slot = out_off + t;
            if (slot >= cap) return -1;
            keys[slot] = ordered_key((float)(c_l * K_idx));
            vals[slot] = K_abs;
          }
        }
        int cnt = num_K - kv_start < TOPK ? num_K - kv_start : TOPK;
        out_off += cnt;
      }
    }
    for (int t = 0; t < HALF; ++t) { parent[t] = tq_x[t]; parent[HALF + t] = tk_x[t]; }
  }
  return out_off;
}

typedef struct { int32_t key; int32_t val; int32_t ord; } kv_t;

static int cmp_kv(const void *a, const void *b) {
  const kv_t *x = (const kv_t *)a, *y = (const kv_t *)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  return x->ord < y->ord ? -1 : (x->ord > y->ord); /* stable */
}

/* scores: [BH, S_tot] fp32 rows (contiguous); out: [BH, out_len] int32.
 * Returns 0 on success, negative on error:
 *   -1 bad arguments, -2 out of the strict domain (mode 0), -3 slot overrun,
 *   -4 out_len does not match, -5 allocation failure. */
int lh_ref_select(const float *scores_qk, const float *scores_kq, int BH, int S_tot,
                  int S, int L, int p, int topk, int tie_lower, int mode,
                  int32_t *out, int out_len) {
  if (L < 1 || p < 2 || (p & (p - 1)) || topk % TOPK || topk < TOPK || topk / 2 < p) return -1;
  int T = topk / TOPK;
  int cL = 1;
  for (int i = 0; i < L - 1; ++i) cL *= p;
  int coarsest = S / cL;
  int NCC = coarsest / T;
  int ref_slots = NCC + (L - 1) * p * TOPK; /* compute_output_indices_selection(S//T, L, p, 128) */
  int ref_total = coarsest + (L - 1) * p * topk;
  if (mode == 0) {
    if (NCC < TOPK || NCC % HALF || coarsest % T || S % cL) return -2;
    if (out_len != ref_total) return -4;
  }
  int cap = (mode == 0) ? ref_slots : (((NCC + HALF - 1) / HALF) * HALF + HALF + (L - 1) * p * TOPK);
  int total_slots = (mode == 0) ? ref_total : cap * T;
  kv_t *buf = (kv_t *)malloc(sizeof(kv_t) * (size_t)total_slots);
  int32_t *keys = (int32_t *)malloc(sizeof(int32_t) * (size_t)total_slots);
  int32_t *vals = (int32_t *)malloc(sizeof(int32_t) * (size_t)total_slots);
  if (!buf || !keys || !vals) { free(buf); free(keys); free(vals); return -5; }
  int rc = 0;
  for (int bh = 0; bh < BH && rc == 0; ++bh) {
    const float *sq = scores_qk + (size_t)bh * S_tot;
    const float *sk = scores_kq + (size_t)bh * S_tot;
    for (int i = 0; i < total_slots; ++i) { keys[i] = -1; vals[i] = -1; }
    for (int tile = 0; tile < T; ++tile) {
      int base = tile * cap;
      int r = run_tile(sq, sk, keys + base, vals + base, cap, L, p, S, tile, NCC, tie_lower);
      if (r < 0 || (mode == 0 && r != ref_slots)) { rc = -3; break; }
    }
    if (rc) break;
    for (int i = 0; i < total_slots; ++i) { buf[i].key = keys[i]; buf[i].val = vals[i]; buf[i].ord = i; }
    qsort(buf, (size_t)total_slots, sizeof(kv_t), cmp_kv);
    int n = 0;
    for (int i = 0; i < total_slots; ++i) {
      if (mode == 1 && buf[i].key == -1) continue;
      if (n < out_len) out[(size_t)bh * out_len + n] = buf[i].val;
      ++n;
    }
    if (n != out_len) { rc = -4; break; }
  }
  free(buf); free(keys); free(vals);
  return rc;
}
