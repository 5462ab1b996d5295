/*
 * sa_oracle.c -- CPU oracle of the bit-exact parts of the sparse-attention hot path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (and __graft_entry__.smoke) through
 * oracle/native.py to check the HIP kernels; never linked into libsa_hip.so.
 *
 * Built with -ffp-contract=off: every fp32 operation below is one IEEE operation in the
 * written order, which is the contract the GPU kernels follow.
 *
 * Functions and the reference code they restate:
 *   oracle_block_pool      block means of q/k (the block-score estimator's pooling,
 *                          utils/mask_related.py:40-81, made deterministic: mean of every
 *                          token of the block instead of 8 random samples)
 *   oracle_block_topk      block scores, per-row top-k (utils/block_sparse_attn_kernel.py:31-39,
 *                          SparseGen_Plus.py:28-50), text rows/columns forced dense
 *                          (SparseGen_Plus.py:81-82), union with a local window, compaction
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bf16_to_f32(uint16_t x) {
  uint32_t u = (uint32_t)x << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* pooled[bh][blk][d] = (x[t0][d] + x[t0+1][d] + ... ) / n, fp32, tokens ascending. */
void oracle_block_pool(const uint16_t* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                       int block, float* pooled) {
  const int nb = (L + block - 1) / block;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h)
      for (int blk = 0; blk < nb; ++blk) {
        const int t0 = blk * block;
        const int n = (L - t0) < block ? (L - t0) : block;
        float* out = pooled + (((int64_t)b * H + h) * nb + blk) * D;
        for (int d = 0; d < D; ++d) {
          float s = 0.0f;
          for (int t = 0; t < n; ++t) s = s + bf16_to_f32(x[b * sb + h * sh + (int64_t)(t0 + t) * sl + d]);
          out[d] = s / (float)n;
        }
      }
}

static uint32_t order_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct {
  uint32_t ord;
  int32_t idx;
} oracle_key;

/* score descending (total order on bit patterns), then index ascending */
static int cmp_key(const void* pa, const void* pb) {
  const oracle_key* a = (const oracle_key*)pa;
  const oracle_key* b = (const oracle_key*)pb;
  if (a->ord != b->ord) return a->ord > b->ord ? -1 : 1;
  return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

float oracle_block_score(const float* qrow, const float* krow, int D) {
  float acc = 0.0f;
  for (int d = 0; d < D; ++d) acc = fmaf(qrow[d], krow[d], acc);
  return acc;
}

/*
 * For each of BH*nqb rows: scores against nkb pooled key blocks (or scores_in), keep the
 * first `topk` in (score desc, index asc) order, OR text rows/columns (< n_text) and the
 * local bitmap [nqb][nkb] (nullable), write ascending kv lists and the dense 0/1 mask.
 */
void oracle_block_topk(const float* qp, const float* kp, const float* scores_in, int BH, int nqb, int nkb,
                       int D, int topk, int n_text, const uint8_t* local, int32_t* kv_idx, int max_cnt,
                       int32_t* kv_cnt, uint8_t* mask_out, float* scores_out) {
  oracle_key* keys = (oracle_key*)malloc(sizeof(oracle_key) * (size_t)nkb);
  uint8_t* keep = (uint8_t*)malloc((size_t)nkb);
  for (int bh = 0; bh < BH; ++bh)
    for (int r = 0; r < nqb; ++r) {
      const int64_t row = (int64_t)bh * nqb + r;
      for (int c = 0; c < nkb; ++c) {
        float s;
        if (scores_in)
          s = scores_in[row * nkb + c];
        else
          s = oracle_block_score(qp + row * D, kp + ((int64_t)bh * nkb + c) * D, D);
        if (scores_out) scores_out[row * nkb + c] = s;
        keys[c].ord = order_bits(s);
        keys[c].idx = c;
      }
      qsort(keys, (size_t)nkb, sizeof(oracle_key), cmp_key);
      memset(keep, 0, (size_t)nkb);
      for (int i = 0; i < topk && i < nkb; ++i) keep[keys[i].idx] = 1;
      int cnt = 0;
      for (int c = 0; c < nkb; ++c) {
        int on = keep[c] || c < n_text || r < n_text || (local && local[(int64_t)r * nkb + c]);
        if (mask_out) mask_out[row * nkb + c] = (uint8_t)on;
        if (on) {
          if (cnt < max_cnt) kv_idx[row * max_cnt + cnt] = c;
          ++cnt;
        }
      }
      kv_cnt[row] = cnt < max_cnt ? cnt : max_cnt;
    }
  free(keys);
  free(keep);
}

/*
 * Local 3-D window on block centre tokens (the combined mask's static part), restating the
 * union of local windows used by the reference's sparse patterns (SildingTileAttention.py
 * :18-87 tile window, SmartAttention.py:56-67 frame band, LocalGlobalAttention.py:114-179):
 * block b is represented by token min(b*block + block/2, L-1); both blocks must be video;
 * |dt|, |dh|, |dw| of their (t, h, w) within the radii.
 */
void oracle_local_window(int L, int block, int text_len, int T, int Hp, int Wp, int dt, int dh, int dw,
                         uint8_t* bitmap) {
  (void)T;
  const int nb = (L + block - 1) / block;
  for (int qb = 0; qb < nb; ++qb) {
    int cq = qb * block + block / 2;
    if (cq > L - 1) cq = L - 1;
    for (int kb = 0; kb < nb; ++kb) {
      int ck = kb * block + block / 2;
      if (ck > L - 1) ck = L - 1;
      int on = 0;
      if (cq >= text_len && ck >= text_len) {
        const int vq = cq - text_len, vk = ck - text_len;
        const int tq = vq / (Hp * Wp), hq = (vq / Wp) % Hp, wq = vq % Wp;
        const int tk = vk / (Hp * Wp), hk = (vk / Wp) % Hp, wk = vk % Wp;
        on = abs(tq - tk) <= dt && abs(hq - hk) <= dh && abs(wq - wk) <= dw;
      }
      bitmap[(int64_t)qb * nb + kb] = (uint8_t)on;
    }
  }
}
