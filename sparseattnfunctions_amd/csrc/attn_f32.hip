// Block-sparse attention forward for fp32 q, k, v: the reference kernel takes any float type
// (utils/block_sparse_attn_kernel.py:52-209: tl.dot of the loaded tiles, P cast to v's dtype,
// :107, i.e. kept in fp32 here). Same list contract as sa_block_sparse_fwd (attn_fwd.hip);
// head dim 64 or 128, no key bias. A pooling mode serves attn_with_pooling in fp32
// (utils/attn_pooling_kernel.py:230-287, which computes in fp32): each row's largest scaled
// logit per 32- or 64-key column and its log2-sum-exp2 are stored for the pooled-map reduce,
// with grouped key heads and a causal diagonal tile.
//
// One wave computes one 64-row query block with v_mfma_f32_16x16x4_f32 (head dim 128: two
// 64-wide halves of d in the S contraction, eight 16-row d blocks of O^T). Operand layouts of
// that instruction: A (16 x 4) lane l holds A[l % 16][l / 16], B (4 x 16) lane l holds
// B[l / 16][l % 16], D (16 x 16) lane l holds D[4 (l / 16) + i][l % 16], i < 4. Both
// contractions use an order of their index that keeps each lane's operands contiguous:
//   S^T = K Q^T over d: k-slot g = l / 16 and step s take d = 16 g + s, so lane l reads 16
//     consecutive floats of one K row and of one Q row;
//   O^T = V^T P^T over the 64 keys of a tile: 16-key group kb16, k-slot g and step i take key
//     16 kb16 + 4 g + i, which is where the S^T output already holds P (D row 4 g + i), so P
//     is the B operand in place; the A operand is V[key][d] for d = 16 dblk + l % 16.
// A sum over d (or over keys) in any order is the same sum; only the fp32 rounding order
// differs from a sequential loop. The running row maximum is kept per 64-key tile (exact
// rescale, no threshold), P = exp2(S * scale * log2(e) - m) in fp32, row sums in fp32.
// Keys past Lk and list entries outside [0, nkb) get P = 0; their K/V loads are clamped to
// the last key row, so every load is inside the tensors.
#include "sa_common.h"

#include <cmath>

namespace {

constexpr int kBlk = 64;     // rows per query block == keys per key block
constexpr int kWavesF32 = 4;  // independent waves per workgroup
constexpr float kLog2eF32 = 1.4426950408889634f;

struct F32Args {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t q_sb, q_sh, q_sl;
  int64_t k_sb, k_sh, k_sl;
  int64_t v_sb, v_sh, v_sl;
  int64_t o_sb, o_sh, o_sl;
  int H, Lq, Lk, nqb, nkb;
  int n_items;
  const int32_t* order;  // dispatch slot -> item, -1 = idle; may be null
  int n_slots;
  const int32_t* kv_idx;
  const int32_t* kv_cnt;
  int max_cnt;
  int list_bh_stride;  // list row = bh * list_bh_stride + qb (0: lists shared by heads)
  float scale_log2;    // sm_scale * log2(e)
  int kv_rep;          // query heads per key/value head
  int causal;          // the tile of key block qb masks keys past the query (Lq == Lk)
  // Pooling (kPool 32 or 64): the row's maximum scaled logit (log2 domain) per kPool-key
  // column to pool_r[((bh * nqb + row / 64) * pool_ncol + column) * 64 + row % 64] and its
  // log2-sum-exp2 to pool_lse[bh * pool_lpad + row].
  float* pool_r;
  int pool_ncol;
  float* pool_lse;
  int pool_lpad;
};

__device__ inline sa_f32x4 mfma16x4(float a, float b, sa_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// max / sum over the four lanes r, r + 16, r + 32, r + 48 (the k-slots of one MFMA column).
__device__ inline float slot_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ inline float slot_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

template <int kD, int kPool>
__global__ __launch_bounds__(64 * kWavesF32, kD == 64 ? 2 : 1) void bsa_fwd_f32_kernel(F32Args a) {
  static_assert(kD == 64 || kD == 128, "head dim 64 or 128");
  static_assert(kPool == 0 || kPool == 32 || kPool == 64, "pooling columns of 32 or 64 keys");
  constexpr int kHalf = kD / 64;   // 64-wide halves of d
  constexpr int kDB = kD / 16;     // 16-row d blocks of O^T
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = blockIdx.x * kWavesF32 + wave;
  if (slot >= a.n_slots) return;
  const int item = __builtin_amdgcn_readfirstlane(a.order ? a.order[slot] : slot);
  if (item < 0 || item >= a.n_items) return;
  const int bh = item / a.nqb;
  const int qb = item - bh * a.nqb;
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int hk = a.kv_rep > 1 ? h / a.kv_rep : h;
  const int r = lane & 15;  // MFMA row of A, column of B and D
  const int g = lane >> 4;  // MFMA k-slot

  const int64_t list_row = (int64_t)bh * a.list_bh_stride + qb;
  int cnt = a.kv_cnt[list_row];
  cnt = cnt < 0 ? 0 : (cnt > a.max_cnt ? a.max_cnt : cnt);
  const __attribute__((address_space(4))) int32_t* list =
      (const __attribute__((address_space(4))) int32_t*)(a.kv_idx + list_row * a.max_cnt);

  const float* qbase = a.q + b * a.q_sb + h * a.q_sh;
  const float* khead = a.k + b * a.k_sb + hk * a.k_sh;
  const float* vhead = a.v + b * a.v_sb + hk * a.v_sh;
  float* obase = a.o + b * a.o_sb + h * a.o_sh;

  // Q^T B operands: qop[j][hf][s] = Q[qb * 64 + 16 j + r][64 hf + 16 g + s] (rows clamped into
  // Lq; the clamped rows are never stored).
  float qop[4][kHalf][16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = min(qb * kBlk + 16 * j + r, a.Lq - 1);
#pragma unroll
    for (int hf = 0; hf < kHalf; ++hf) {
      const float4* p = reinterpret_cast<const float4*>(qbase + (int64_t)row * a.q_sl + 64 * hf + 16 * g);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 w = p[c];
        qop[j][hf][4 * c] = w.x;
        qop[j][hf][4 * c + 1] = w.y;
        qop[j][hf][4 * c + 2] = w.z;
        qop[j][hf][4 * c + 3] = w.w;
      }
    }
  }

  sa_f32x4 acc[kDB][4];  // [dblk][j]: O^T[16 dblk + 4 g + i][16 j + r]
  float m[4], l[4];      // per query column j: running max (log2 domain) and this lane's row-sum part
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int dblk = 0; dblk < kDB; ++dblk) acc[dblk][j] = sa_f32x4{0.f, 0.f, 0.f, 0.f};
  }

  for (int it = 0; it < cnt; ++it) {
    const int kb = list[it];
    const bool ok = (unsigned)kb < (unsigned)a.nkb;
    const int key0 = ok ? kb * kBlk : 0;
    const int nvalid = ok ? min(kBlk, a.Lk - key0) : 0;
    const bool diag = kPool != 0 && a.causal && kb == qb;  // causal lists exist for pooling only

    // ---- S^T[16 kb16 + 4 g + i][16 j + r] in S[kb16][j][i].
    sa_f32x4 S[4][4];
#pragma unroll
    for (int kb16 = 0; kb16 < 4; ++kb16) {
      const int key = min(key0 + 16 * kb16 + r, a.Lk - 1);
      float kop[kHalf][16];
#pragma unroll
      for (int hf = 0; hf < kHalf; ++hf) {
        const float4* p = reinterpret_cast<const float4*>(khead + (int64_t)key * a.k_sl + 64 * hf + 16 * g);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float4 w = p[c];
          kop[hf][4 * c] = w.x;
          kop[hf][4 * c + 1] = w.y;
          kop[hf][4 * c + 2] = w.z;
          kop[hf][4 * c + 3] = w.w;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sa_f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int hf = 0; hf < kHalf; ++hf)
#pragma unroll
          for (int s = 0; s < 16; ++s) t = mfma16x4(kop[hf][s], qop[j][hf][s], t);
        S[kb16][j] = t;
      }
    }

    // ---- Masks (keys past Lk; keys past the query on the causal diagonal tile), pooled
    // column maxima, running maximum per query, then P = exp2(S * sc - m) in place and the
    // row sums.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb16 = 0; kb16 < 4; ++kb16)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kk = 16 * kb16 + 4 * g + i;
          if (kk >= nvalid || (kPool != 0 && diag && kk > 16 * j + r)) S[kb16][j][i] = -INFINITY;
          mx = fmaxf(mx, S[kb16][j][i]);
        }
      if constexpr (kPool != 0) {
        if (ok) {
          constexpr int kCols = kBlk / kPool;  // columns per tile
#pragma unroll
          for (int cc = 0; cc < kCols; ++cc) {
            float x = -INFINITY;
#pragma unroll
            for (int kb16 = cc * (4 / kCols); kb16 < (cc + 1) * (4 / kCols); ++kb16)
#pragma unroll
              for (int i = 0; i < 4; ++i) x = fmaxf(x, S[kb16][j][i]);
            x = slot_max(x) * a.scale_log2;  // scale > 0
            if (g == 0)
              a.pool_r[(((int64_t)bh * a.nqb + qb) * a.pool_ncol + kb * kCols + cc) * kBlk + 16 * j + r] = x;
          }
        }
      }
      const float cand = slot_max(mx) * a.scale_log2;  // scale > 0
      const float m_new = fmaxf(m[j], cand);
      if (m_new != -INFINITY) {  // otherwise nothing is accumulated yet and every P is 0
        const float alpha = exp2f(m[j] - m_new);  // 0 when m = -inf
        m[j] = m_new;
        l[j] *= alpha;
#pragma unroll
        for (int dblk = 0; dblk < kDB; ++dblk) acc[dblk][j] *= alpha;
      }
      const float mu = m[j] == -INFINITY ? 0.f : m[j];
#pragma unroll
      for (int kb16 = 0; kb16 < 4; ++kb16)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = exp2f(fmaf(S[kb16][j][i], a.scale_log2, -mu));  // -inf -> 0
          S[kb16][j][i] = p;
          l[j] += p;
        }
    }

    // ---- O^T += V^T P^T: key 16 kb16 + 4 g + i, A = V[key][16 dblk + r], B = P in place.
#pragma unroll
    for (int kb16 = 0; kb16 < 4; ++kb16)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = min(key0 + 16 * kb16 + 4 * g + i, a.Lk - 1);
        const float* vrow = vhead + (int64_t)key * a.v_sl + r;
        float vop[kDB];
#pragma unroll
        for (int dblk = 0; dblk < kDB; ++dblk) vop[dblk] = vrow[16 * dblk];
#pragma unroll
        for (int dblk = 0; dblk < kDB; ++dblk)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[dblk][j] = mfma16x4(vop[dblk], S[kb16][j][i], acc[dblk][j]);
      }
  }

  // ---- Epilogue: out = acc / l; an empty list writes 0. Pooling: the row's log2-sum-exp2.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float l_tot = slot_sum(l[j]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int row = qb * kBlk + 16 * j + r;
    if constexpr (kPool != 0) {
      if (g == 0) a.pool_lse[(int64_t)bh * a.pool_lpad + row] = (m[j] == -INFINITY ? 0.f : m[j]) + log2f(l_tot);
    }
    if (row < a.Lq) {
      float* orow = obase + (int64_t)row * a.o_sl;
#pragma unroll
      for (int dblk = 0; dblk < kDB; ++dblk) {
        const sa_f32x4 A = acc[dblk][j];
        *reinterpret_cast<float4*>(orow + 16 * dblk + 4 * g) = make_float4(A[0] * inv, A[1] * inv, A[2] * inv, A[3] * inv);
      }
    }
  }
}

}  // namespace

namespace {

int launch_f32(const float* q, const int64_t q_strides[3], const float* k, const int64_t k_strides[3],
               const float* v, const int64_t v_strides[3], float* out, const int64_t out_strides[3], int B, int H,
               int Lq, int Lk, int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt, bool lists_shared,
               float sm_scale, const int32_t* work_order, int64_t n_slots, int kv_rep, bool causal, int pool_cols,
               float* pool_r, float* pool_lse, void* stream, const char* fn) {
  SA_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides && kv_idx && kv_cnt,
             "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && Lq > 0 && Lk > 0, "%s: bad shape B=%d H=%d Lq=%d Lk=%d", fn, B, H, Lq, Lk);
  if (D != 64 && D != 128) return sa::fail(SA_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", fn, D);
  SA_REQUIRE(max_cnt > 0, "%s: max_cnt must be > 0", fn);
  SA_REQUIRE(std::isfinite(sm_scale) && sm_scale > 0.f, "%s: sm_scale must be finite and > 0", fn);
  SA_REQUIRE(kv_rep >= 1 && H % kv_rep == 0, "%s: kv_rep=%d must divide H=%d", fn, kv_rep, H);
  SA_REQUIRE(!causal || (Lq == Lk && pool_cols), "%s: causal needs Lq == Lk and pooling", fn);
  const void* ptrs[4] = {q, k, v, out};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return sa::fail(SA_ERR_UNSUPPORTED, "%s: tensor base not 16-byte aligned", fn);
  const int64_t* strides[4] = {q_strides, k_strides, v_strides, out_strides};
  for (const int64_t* st : strides)
    for (int i = 0; i < 3; ++i)
      if (st[i] % 4 != 0) return sa::fail(SA_ERR_UNSUPPORTED, "%s: strides must be multiples of 4 elements", fn);
  const int nqb = sa::cdiv(Lq, kBlk);
  const int64_t n_items = (int64_t)B * H * nqb;
  SA_REQUIRE(n_items < (1LL << 30), "%s: too many query blocks", fn);
  if (work_order) {
    SA_REQUIRE(n_slots > 0 && n_slots % kWavesF32 == 0, "%s: n_slots must be a positive multiple of 4", fn);
  } else {
    n_slots = (n_items + kWavesF32 - 1) / kWavesF32 * kWavesF32;
  }
  SA_REQUIRE(n_slots / kWavesF32 < (1LL << 31), "%s: grid too large", fn);
  F32Args a;
  a.q = q; a.k = k; a.v = v; a.o = out;
  a.q_sb = q_strides[0]; a.q_sh = q_strides[1]; a.q_sl = q_strides[2];
  a.k_sb = k_strides[0]; a.k_sh = k_strides[1]; a.k_sl = k_strides[2];
  a.v_sb = v_strides[0]; a.v_sh = v_strides[1]; a.v_sl = v_strides[2];
  a.o_sb = out_strides[0]; a.o_sh = out_strides[1]; a.o_sl = out_strides[2];
  a.H = H; a.Lq = Lq; a.Lk = Lk; a.nqb = nqb; a.nkb = sa::cdiv(Lk, kBlk);
  a.n_items = (int)n_items;
  a.order = work_order;
  a.n_slots = (int)n_slots;
  a.kv_idx = kv_idx; a.kv_cnt = kv_cnt; a.max_cnt = max_cnt;
  a.list_bh_stride = lists_shared ? 0 : nqb;
  a.scale_log2 = sm_scale * kLog2eF32;
  a.kv_rep = kv_rep;
  a.causal = causal ? 1 : 0;
  a.pool_r = pool_r;
  a.pool_ncol = pool_cols ? a.nkb * (kBlk / pool_cols) : 0;
  a.pool_lse = pool_lse;
  a.pool_lpad = nqb * kBlk;
  SA_REQUIRE(pool_cols == 0 || (pool_r && pool_lse), "%s: pooling needs its buffers", fn);
  const dim3 grid((unsigned)(n_slots / kWavesF32)), blk(64 * kWavesF32);
  hipStream_t s = sa::as_stream(stream);
  if (D == 64) {
    if (pool_cols == 32) hipLaunchKernelGGL((bsa_fwd_f32_kernel<64, 32>), grid, blk, 0, s, a);
    else if (pool_cols == 64) hipLaunchKernelGGL((bsa_fwd_f32_kernel<64, 64>), grid, blk, 0, s, a);
    else hipLaunchKernelGGL((bsa_fwd_f32_kernel<64, 0>), grid, blk, 0, s, a);
  } else {
    if (pool_cols == 32) hipLaunchKernelGGL((bsa_fwd_f32_kernel<128, 32>), grid, blk, 0, s, a);
    else if (pool_cols == 64) hipLaunchKernelGGL((bsa_fwd_f32_kernel<128, 64>), grid, blk, 0, s, a);
    else hipLaunchKernelGGL((bsa_fwd_f32_kernel<128, 0>), grid, blk, 0, s, a);
  }
  return sa::check_launch(fn);
}

}  // namespace

namespace sa {
// fp32 attention in pooling mode for the pooled-map entry point (attn_fwd.hip).
int attn_f32_pooling(const float* q, const int64_t q_strides[3], const float* k, const int64_t k_strides[3],
                     const float* v, const int64_t v_strides[3], float* out, const int64_t out_strides[3], int B,
                     int H, int L, int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt, int kv_rep,
                     bool causal, float sm_scale, int pool_cols, float* pool_r, float* pool_lse, void* stream,
                     const char* fn) {
  return launch_f32(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, L, L, D, kv_idx, kv_cnt,
                    max_cnt, true, sm_scale, nullptr, 0, kv_rep, causal, pool_cols, pool_r, pool_lse, stream, fn);
}
}  // namespace sa

extern "C" int sa_block_sparse_fwd_f32(const float* q, const int64_t q_strides[3], const float* k,
                                       const int64_t k_strides[3], const float* v, const int64_t v_strides[3],
                                       float* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk, int D,
                                       const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                       const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                       const int32_t* work_order, int64_t n_slots, void* stream) {
  const char* fn = "sa_block_sparse_fwd_f32";
  (void)bias_strides;
  if (key_bias) return sa::fail(SA_ERR_UNSUPPORTED, "%s: key_bias (bf16 and fp16 only)", fn);
  return launch_f32(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, false, sm_scale, work_order, n_slots, 1, false, 0, nullptr, nullptr, stream, fn);
}
