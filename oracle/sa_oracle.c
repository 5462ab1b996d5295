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
 *   oracle_energy_list     energy-threshold and adaptive top-k selection of
 *                          transfer_attn_to_mask (SparseGen_Plus.py:12-84) over fp32 scores
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
 * transfer_attn_to_mask (SparseGen_Plus.py:12-84) per row: sort (score desc, index asc),
 * cum[j] = sequential fp32 sum of the first j+1 sorted scores, total = cum[n-1];
 *   mode 0 "energy" (:52-78): k = first j with cum[j] >= thr*total (n if cum[n-1] < thr*total),
 *          clamped to [min_keep, max_keep]; keep the first k sorted columns;
 *   mode 1 "topk" (:28-50): k0 = init_k, e = cum[k0-1]; if e < 0.6*total and k0 < n:
 *          k = min(3*k0, n); if e < 0.9*total and k0 < n: k = min(k/3*2, n);
 *   mode 2 "inclusive" (mask_related.py:224-232, 366-376): j = first position with
 *          cum[j] >= thr*total (n-1 if none: the last position is forced on), keep the first
 *          j+1 sorted columns, then clamped to [min_keep, max_keep];
 *   mode 3 "cumulative <=" (mask_related.py:378-391): keep every sorted position j with
 *          cum[j] <= thr*total, and the last sorted position;
 * then text rows/columns (< n_text) forced on (:81-82); ascending kv lists and 0/1 mask.
 */
void oracle_energy_list(const float* scores, int BH, int nqb, int nkb, int mode, float thr, int min_keep,
                        int max_keep, int init_k, int n_text, int32_t* kv_idx, int max_cnt, int32_t* kv_cnt,
                        uint8_t* mask_out) {
  oracle_key* keys = (oracle_key*)malloc(sizeof(oracle_key) * (size_t)nkb);
  float* cum = (float*)malloc(sizeof(float) * (size_t)nkb);
  uint8_t* keep = (uint8_t*)malloc((size_t)nkb);
  const int n = nkb;
  for (int64_t row = 0; row < (int64_t)BH * nqb; ++row) {
    const float* s = scores + row * n;
    for (int c = 0; c < n; ++c) {
      keys[c].ord = order_bits(s[c]);
      keys[c].idx = c;
    }
    qsort(keys, (size_t)n, sizeof(oracle_key), cmp_key);
    float acc = 0.0f;
    for (int j = 0; j < n; ++j) {
      acc += s[keys[j].idx];
      cum[j] = acc;
    }
    const float total = cum[n - 1];
    int k;
    if (mode == 0) {
      const float target = thr * total;
      int first = n;
      for (int j = 0; j < n; ++j)
        if (cum[j] >= target) {
          first = j;
          break;
        }
      k = total < target ? n : first;
      if (k < min_keep) k = min_keep;
      if (k > max_keep) k = max_keep;
    } else if (mode == 2) {
      const float target = thr * total;
      int first = n - 1;
      for (int j = 0; j < n; ++j)
        if (cum[j] >= target) {
          first = j;
          break;
        }
      k = first + 1;
      if (k < min_keep) k = min_keep;
      if (k > max_keep) k = max_keep;
    } else if (mode == 3) {
      const float target = thr * total;
      k = 0;
      while (k < n && cum[k] <= target) ++k;
    } else {
      const int k0 = init_k;
      const float e = cum[k0 - 1];
      k = k0;
      if (!(e >= 0.6f * total) && k0 < n) k = (3 * k < n) ? 3 * k : n;
      if (!(e >= 0.9f * total) && k0 < n) k = (k / 3 * 2 < n) ? k / 3 * 2 : n;
    }
    memset(keep, 0, (size_t)n);
    for (int j = 0; j < k && j < n; ++j) keep[keys[j].idx] = 1;
    if (mode == 3) keep[keys[n - 1].idx] = 1;
    const int r = (int)(row % nqb);
    int cnt = 0;
    for (int c = 0; c < n; ++c) {
      const int on = keep[c] || r < n_text || c < n_text;
      if (mask_out) mask_out[row * n + c] = (uint8_t)on;
      if (on) {
        if (cnt < max_cnt) kv_idx[row * max_cnt + cnt] = c;
        ++cnt;
      }
    }
    kv_cnt[row] = cnt < max_cnt ? cnt : max_cnt;
  }
  free(keys);
  free(cum);
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

/* ---------------------------------------------------------------------------------------
 * Token merging (utils/merge_unmerge.py:34-156, MergeAttention.py:21-49).
 */

/*
 * Partition (merge_unmerge.py:62-92): build the {-1 = dst, 0 = src} buffer over frames
 * 1..T-1 cell by cell (one dst per (st, sy, sx) cell at offset choice[cell], 0 = top-left),
 * then a stable argsort puts dst before src; the first frame is prepended to dst.
 */
void oracle_tome_partition(int T, int Hp, int Wp, int sx, int sy, int st, const int32_t* choice, int32_t* a_idx,
                           int32_t* b_idx, int* n_src, int* n_dst) {
  const int frame = Hp * Wp, t1 = T - 1;
  const int hsy = Hp / sy, wsx = Wp / sx, tst = t1 / st;
  const int n = t1 * frame;
  int* buf = (int*)calloc((size_t)(n > 0 ? n : 1), sizeof(int));
  int cellno = 0;
  for (int a = 0; a < tst; ++a)
    for (int b = 0; b < hsy; ++b)
      for (int c = 0; c < wsx; ++c, ++cellno) {
        const int o = choice ? choice[cellno] : 0;
        const int ot = o / (sy * sx), oy = (o / sx) % sy, ox = o % sx;
        buf[((a * st + ot) * Hp + (b * sy + oy)) * Wp + (c * sx + ox)] = -1;
      }
  int nb = 0, na = 0;
  for (int i = 0; i < frame; ++i) b_idx[nb++] = i;
  for (int v = -1; v <= 0; ++v)          /* stable argsort of a {-1, 0} array */
    for (int i = 0; i < n; ++i)
      if (buf[i] == v) {
        if (v < 0) b_idx[nb++] = frame + i;
        else a_idx[na++] = frame + i;
      }
  *n_src = na;
  *n_dst = nb;
  free(buf);
}

/* Metric: mode 0 head-sum of k per batch ([B][N][64]); mode 1 per head (k,|k|,v,|v|). */
void oracle_tome_metric(const uint16_t* k, const uint16_t* v, int64_t sb, int64_t sh, int64_t sl, int B, int H,
                        int L, int text_len, int mode, float* out) {
  const int N = L - text_len, D = 64;
  if (mode == 0) {
    for (int b = 0; b < B; ++b)
      for (int n = 0; n < N; ++n) {
        float m[64];
        for (int d = 0; d < D; ++d) m[d] = 0.0f;
        for (int h = 0; h < H; ++h)
          for (int d = 0; d < D; ++d) m[d] = m[d] + bf16_to_f32(k[b * sb + h * sh + (int64_t)(text_len + n) * sl + d]);
        float ss = 0.0f;
        for (int d = 0; d < D; ++d) ss = fmaf(m[d], m[d], ss);
        const float nrm = sqrtf(ss);
        for (int d = 0; d < D; ++d) out[((int64_t)b * N + n) * D + d] = m[d] / nrm;
      }
  } else {
    const int C = 2 * D + 2;
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int n = 0; n < N; ++n) {
          float ch[130];
          const int64_t base = b * sb + h * sh + (int64_t)(text_len + n) * sl;
          for (int d = 0; d < D; ++d) ch[d] = bf16_to_f32(k[base + d]);
          for (int d = 0; d < D; ++d) ch[D + 1 + d] = bf16_to_f32(v[base + d]);
          float kq = 0.0f, vq = 0.0f;
          for (int d = 0; d < D; ++d) kq = fmaf(ch[d], ch[d], kq);
          for (int d = 0; d < D; ++d) vq = fmaf(ch[D + 1 + d], ch[D + 1 + d], vq);
          ch[D] = sqrtf(kq);
          ch[2 * D + 1] = sqrtf(vq);
          float ss = 0.0f;
          for (int c = 0; c < C; ++c) ss = fmaf(ch[c], ch[c], ss);
          const float nrm = sqrtf(ss);
          float* o = out + (((int64_t)b * H + h) * N + n) * C;
          for (int c = 0; c < C; ++c) o[c] = ch[c] / nrm;
        }
  }
}

static float oracle_round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  memcpy(&x, &u, 4);
  return x;
}

/* Best dst of each src (merge_unmerge.py:102, :108): fmaf-chain scores, scan over dst in
 * order, first maximum wins. a_idx may be any subset of the srcs. */
void oracle_tome_argmax(const float* metric, int G, int N, int C, const int32_t* a_idx, int n_a,
                        const int32_t* b_idx, int n_dst, int32_t* node_idx, float* node_max) {
  for (int g = 0; g < G; ++g) {
    const float* mg = metric + (int64_t)g * N * C;
    for (int s = 0; s < n_a; ++s) {
      float best = -INFINITY;
      int bi = 0;
      for (int d = 0; d < n_dst; ++d) {
        float acc = 0.0f;
        for (int c = 0; c < C; ++c) acc = fmaf(mg[(int64_t)a_idx[s] * C + c], mg[(int64_t)b_idx[d] * C + c], acc);
        if (acc > best) {
          best = acc;
          bi = d;
        }
      }
      node_max[(int64_t)g * n_a + s] = best;
      node_idx[(int64_t)g * n_a + s] = bi;
    }
  }
}

/* Maps from node_max/node_idx (merge_unmerge.py:109-116, MergeAttention.py:163-167): edge
 * order = stable sort of node_max descending, dst_idx, dst counts, the unmerge map and the
 * bf16 log-size key bias. */
void oracle_tome_maps(const float* node_max, const int32_t* node_idx, int G, int N, const int32_t* a_idx,
                      const int32_t* b_idx, int n_src, int n_dst, int r, int text_len, int32_t* edge,
                      int32_t* dst_idx, int32_t* dst_cnt, int32_t* row_of_token, float* key_bias) {
  const int L = text_len + N, Lm = L - r, U = n_src - r;
  oracle_key* keys = (oracle_key*)malloc(sizeof(oracle_key) * (size_t)(n_src > 0 ? n_src : 1));
  for (int g = 0; g < G; ++g) {
    for (int s = 0; s < n_src; ++s) {
      keys[s].ord = order_bits(node_max[(int64_t)g * n_src + s]);
      keys[s].idx = s;
    }
    qsort(keys, (size_t)n_src, sizeof(oracle_key), cmp_key);
    int32_t* cnt = dst_cnt + (int64_t)g * n_dst;
    int32_t* rot = row_of_token + (int64_t)g * L;
    for (int d = 0; d < n_dst; ++d) cnt[d] = 0;
    for (int t = 0; t < text_len; ++t) rot[t] = t;
    for (int e = 0; e < n_src; ++e) {
      const int s = keys[e].idx;
      edge[(int64_t)g * n_src + e] = s;
      if (e < r) {
        const int d = node_idx[(int64_t)g * n_src + s];
        dst_idx[(int64_t)g * r + e] = d;
        cnt[d] += 1;
        rot[text_len + a_idx[s]] = text_len + U + d;
      } else {
        rot[text_len + a_idx[s]] = text_len + (e - r);
      }
    }
    for (int d = 0; d < n_dst; ++d) rot[text_len + b_idx[d]] = text_len + U + d;
    for (int j = 0; j < Lm; ++j) {
      const int d = j - text_len - U;
      key_bias[(int64_t)g * Lm + j] = d >= 0 ? oracle_round_bf16(logf(oracle_round_bf16((float)(1 + cnt[d])))) : 0.0f;
    }
  }
  free(keys);
}

/* Matching and maps for each group (merge_unmerge.py:99-116): argmax then maps. */
void oracle_tome_match(const float* metric, int G, int N, int C, const int32_t* a_idx, const int32_t* b_idx,
                       int n_src, int n_dst, int r, int text_len, int32_t* node_idx, float* node_max, int32_t* edge,
                       int32_t* dst_idx, int32_t* dst_cnt, int32_t* row_of_token, float* key_bias) {
  oracle_tome_argmax(metric, G, N, C, a_idx, n_src, b_idx, n_dst, node_idx, node_max);
  oracle_tome_maps(node_max, node_idx, G, N, a_idx, b_idx, n_src, n_dst, r, text_len, edge, dst_idx, dst_cnt,
                   row_of_token, key_bias);
}

/* merge of one [B,H,L,64] bf16 tensor (merge_unmerge.py:119-128): fp32 sum of the dst then
 * its srcs in edge order, divided by the count, rounded to bf16. out [B,H,Lm,64]. */
void oracle_tome_merge(const uint16_t* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int heads_per_group,
                       int N, int text_len, const int32_t* a_idx, const int32_t* b_idx, int n_src, int n_dst, int r,
                       const int32_t* edge, const int32_t* dst_idx, uint16_t* out) {
  const int L = text_len + N, Lm = L - r, U = n_src - r, D = 64;
  const int G = B * H / heads_per_group;
  /* members of each dst in edge order: stable counting sort of the edges by dst */
  int32_t* ptr = (int32_t*)calloc((size_t)G * (n_dst + 1), sizeof(int32_t));
  int32_t* mem = (int32_t*)malloc(sizeof(int32_t) * (size_t)G * (r > 0 ? r : 1));
  for (int g = 0; g < G; ++g) {
    int32_t* pg = ptr + (int64_t)g * (n_dst + 1);
    for (int e = 0; e < r; ++e) pg[dst_idx[(int64_t)g * r + e] + 1] += 1;
    for (int d = 0; d < n_dst; ++d) pg[d + 1] += pg[d];
    int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_dst > 0 ? n_dst : 1));
    memcpy(cur, pg, sizeof(int32_t) * (size_t)n_dst);
    for (int e = 0; e < r; ++e) mem[(int64_t)g * r + cur[dst_idx[(int64_t)g * r + e]]++] = e;
    free(cur);
  }
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int g = (b * H + h) / heads_per_group;
      const uint16_t* xb = x + b * sb + h * sh;
      uint16_t* ob = out + ((int64_t)b * H + h) * Lm * D;
      for (int j = 0; j < Lm; ++j) {
        if (j < text_len + U) {
          const int tok = j < text_len ? j : text_len + a_idx[edge[(int64_t)g * n_src + r + (j - text_len)]];
          memcpy(ob + (int64_t)j * D, xb + (int64_t)tok * sl, D * sizeof(uint16_t));
          continue;
        }
        const int d = j - text_len - U;
        float s[64];
        int n = 1;
        for (int c = 0; c < D; ++c) s[c] = bf16_to_f32(xb[(int64_t)(text_len + b_idx[d]) * sl + c]);
        for (int p = ptr[(int64_t)g * (n_dst + 1) + d]; p < ptr[(int64_t)g * (n_dst + 1) + d + 1]; ++p) {
          const int tok = text_len + a_idx[edge[(int64_t)g * n_src + mem[(int64_t)g * r + p]]];
          for (int c = 0; c < D; ++c) s[c] = s[c] + bf16_to_f32(xb[(int64_t)tok * sl + c]);
          ++n;
        }
        for (int c = 0; c < D; ++c) {
          float val = n > 1 ? oracle_round_bf16(s[c] / (float)n) : s[c];
          uint32_t u;
          memcpy(&u, &val, 4);
          ob[(int64_t)j * D + c] = (uint16_t)(u >> 16);
        }
      }
    }
  free(ptr);
  free(mem);
}
