// Head routing of the 1.5-5B pattern attention (unified_judge, partern_attention.py:463-521)
// for gfx950.
//
//   probs_kernel       one wave per (head, 32 sampled query rows): S^T = K Q^T with
//                      v_mfma_f32_32x32x16_bf16 over all sampled keys (optional additive bias
//                      on the first keys), row max and sum in a first pass, then the
//                      probabilities of a key range written row-major (through LDS, 128-byte
//                      rows) in a second pass;
//   share_kernel       judge_sparsity (:468-476): per query row, the probability mass of its
//                      K largest entries (K-th largest found by a bit search on the fp32
//                      bit patterns, its last bits over the compacted bucket), one workgroup
//                      per row;
//   gram_kernel        judge_similarity (:477-514): for key frame f2, the Gram matrix
//                      G[f1][f3] = sum_{s1,s2} P[f1 s1][f2 s2] * P[f3 s1][f2 s2] of the
//                      frame-pair patterns (their inner products and norms), as partial sums
//                      over chunks of s1;
//   finish_kernel      per head: mean share > 0.9 (sparse), mean cosine similarity of the
//                      patterns sharing a key frame > 0.9 (twice), and the routing decision.
#include <cmath>

#include "sa_common.h"

namespace {

constexpr int kD = 64;
constexpr float kLog2e = 1.4426950408889634f;

typedef unsigned jd_u32x4 __attribute__((ext_vector_type(4)));
typedef float jd_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short jd_u16x2 __attribute__((ext_vector_type(2)));

__device__ inline sa_f32x16 score_tile_k(const jd_u32x4 (&kop)[4], const sa_bf16x8 (&qf)[4]) {
  sa_f32x16 t = {};
#pragma unroll
  for (int s = 0; s < 4; ++s)
    t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(sa_bf16x8, kop[s]), qf[s], t, 0, 0, 0);
  return t;
}

__device__ inline void load_k(const uint16_t* kp, jd_u32x4 (&kop)[4]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) kop[s] = *reinterpret_cast<const jd_u32x4*>(kp + 16 * s);
}

__device__ inline sa_f32x16 score_tile(const uint16_t* kp, const sa_bf16x8 (&qf)[4]) {
  jd_u32x4 kop[4];
  load_k(kp, kop);
  return score_tile_k(kop, qf);
}

// ---------------------------------------------------------------------------------------
struct ProbArgs {
  const uint16_t* qs;  // [BH][rows_pad][64]
  const uint16_t* ks;  // [BH][keys_pad][64]
  int rows, rows_pad, keys, keys_pad;
  float scale_log2;
  int n_bias;
  float bias_log2;     // added to keys < n_bias (log2 domain)
  int c_lo, c_hi;      // key range written
  float* P;            // P[bh*p_bh + r*p_row + (key - c_lo)]
  int64_t p_bh, p_row;
  int ng;              // rows_pad / 32
  int vec_ok;          // 16-byte stores possible (P, strides and c_lo multiples of 4 floats)
  int64_t total;       // BH * ng
};

__global__ __launch_bounds__(256) void probs_kernel(ProbArgs a) {
  __shared__ float tile[4][32][36];  // [wave][query row][key], rows 16-byte aligned
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave;
  if (wid >= a.total) return;  // no workgroup barriers below
  const int64_t bh = wid / a.ng;
  const int g = (int)(wid - bh * a.ng);
  const int col = lane & 31, hh = lane >> 5;
  sa_bf16x8 qf[4];
  {
    const uint16_t* qp = a.qs + (bh * a.rows_pad + 32 * g + col) * kD + 8 * hh;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = __builtin_bit_cast(sa_bf16x8, *reinterpret_cast<const jd_u32x4*>(qp + 16 * s));
  }
  const uint16_t* kbase = a.ks + (bh * a.keys_pad + col) * kD + 8 * hh;
  // Logits (log2 domain) of key tile kt; -inf past the keys. Whole tiles inside the key
  // range and on one side of the bias boundary need no per-element tests.
  auto logits = [&](const sa_f32x16& t, int kt, float (&x)[16]) {
    if (32 * kt + 32 <= a.keys && (32 * kt + 32 <= a.n_bias || 32 * kt >= a.n_bias)) {
      const float tb = 32 * kt < a.n_bias ? a.bias_log2 : 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = fmaf(t[i], a.scale_log2, tb);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = 32 * kt + 8 * (i >> 2) + 4 * hh + (i & 3);
        x[i] = key >= a.keys ? -INFINITY : fmaf(t[i], a.scale_log2, key < a.n_bias ? a.bias_log2 : 0.f);
      }
    }
  };
  float m = -INFINITY, l = 0.f;
  for (int kt = 0; kt < a.keys_pad / 32; ++kt) {
    const sa_f32x16 t = score_tile(kbase + (int64_t)kt * 32 * kD, qf);
    float x[16], tmax = -INFINITY;
    logits(t, kt, x);
#pragma unroll
    for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, x[i]);
    const float mn = fmaxf(m, tmax);
    if (mn != -INFINITY) {
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) sum += __builtin_amdgcn_exp2f(x[i] - mn);
      l = l * __builtin_amdgcn_exp2f(m - mn) + sum;
      m = mn;
    }
  }
  {
    const auto mo = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    const auto lo = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    const float m0 = __uint_as_float(mo[0]), m1 = __uint_as_float(mo[1]);
    const float M = fmaxf(m0, m1);
    l = __uint_as_float(lo[0]) * __builtin_amdgcn_exp2f(m0 - M) + __uint_as_float(lo[1]) * __builtin_amdgcn_exp2f(m1 - M);
    m = M;
  }
  const float inv = 1.f / l;
  const int row0 = 32 * g;
  const int c4 = lane & 7;  // lane writes keys 4*c4 .. 4*c4+3 of rows lane/8 + 8j
  for (int kt = a.c_lo / 32; kt * 32 < a.c_hi; ++kt) {
    const sa_f32x16 t = score_tile(kbase + (int64_t)kt * 32 * kD, qf);
    float x[16];
    logits(t, kt, x);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      tile[wave][col][8 * (i >> 2) + 4 * hh + (i & 3)] = __builtin_amdgcn_exp2f(x[i] - m) * inv;
    __builtin_amdgcn_wave_barrier();
    // 8 lanes per row: each store instruction writes 128 contiguous bytes of 8 rows.
    const int key0 = 32 * kt + 4 * c4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 8 * j + (lane >> 3);
      if (row0 + r >= a.rows) continue;
      float* dst = a.P + bh * a.p_bh + (int64_t)(row0 + r) * a.p_row;
      const float4 v = *reinterpret_cast<const float4*>(&tile[wave][r][4 * c4]);
      const int o = key0 - a.c_lo;  // column of key0 in P
      if (a.vec_ok && key0 >= a.c_lo && key0 + 4 <= a.c_hi) {
        // streamed: P is far larger than the caches, K stays resident
        __builtin_nontemporal_store(jd_f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<jd_f32x4*>(dst + o));
      } else {
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (key0 + u >= a.c_lo && key0 + u < a.c_hi) dst[o + u] = e[u];
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------------------
// share_kernel: one workgroup per (bh, row) over n probabilities (n <= 16384).
struct ShareArgs {
  const float* P;
  int64_t p_bh, p_row;
  int rows, n, K;
  int vec_ok;  // P, p_bh and p_row multiples of 16 bytes
  float* share;  // [BH][rows]
  int64_t total;
};

__device__ inline uint32_t wave_sum_u(uint32_t x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}
__device__ inline float wave_sum_f(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Thread t holds entries t, t + 256, ... (at most 64 of them) in registers. The K-th largest
// bit pattern (p >= 0: bit patterns order as the values) is the largest thr with
// #{v >= thr} >= K, found bit by bit from the top. The first kShareHi bits are searched over
// every entry. The entries that share those bits (the bucket) are then compacted into LDS in
// thread order, and one wave finishes the search over them; entries above the bucket always
// count. A bucket larger than kShareCap entries continues the search over every entry.
constexpr int kShareHi = 12;
constexpr int kShareCap = 2048;

__device__ inline uint32_t wave_incl_scan_u(uint32_t x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

__global__ __launch_bounds__(256) void share_kernel(ShareArgs a) {
  constexpr int kPer = 64;
  __shared__ uint32_t part_u[2][4];
  __shared__ float part_f[4];
  __shared__ uint32_t buck[kShareCap];
  __shared__ uint32_t wtot[2][4];
  __shared__ uint32_t thr_out;
  const int64_t w = blockIdx.x;
  if (w >= a.total) return;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t bh = w / a.rows;
  const int r = (int)(w - bh * a.rows);
  const float* src = a.P + bh * a.p_bh + (int64_t)r * a.p_row;
  uint32_t v[kPer];  // 0 past n; the order of the entries does not matter below
  if (a.vec_ok) {    // 16-byte loads: entries 4t + 1024q .. +3
#pragma unroll
    for (int q = 0; q < kPer / 4; ++q) {
      const int i = 4 * t + 1024 * q;
      if (i + 4 <= a.n) {
        const uint4 u = *reinterpret_cast<const uint4*>(src + i);
        v[4 * q] = u.x;
        v[4 * q + 1] = u.y;
        v[4 * q + 2] = u.z;
        v[4 * q + 3] = u.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * q + e] = i + e < a.n ? __float_as_uint(src[i + e]) : 0u;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = t + 256 * j;
      v[j] = i < a.n ? __float_as_uint(src[i]) : 0u;
    }
  }
  // Counting step over every entry (double-buffered partials, one barrier per step).
  auto step = [&](uint32_t thr, int bit) {
    const uint32_t cand = thr | (1u << bit);
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) c += v[j] >= cand;
    c = wave_sum_u(c);
    if (lane == 0) part_u[bit & 1][wave] = c;
    __syncthreads();
    const uint32_t tot = part_u[bit & 1][0] + part_u[bit & 1][1] + part_u[bit & 1][2] + part_u[bit & 1][3];
    return tot >= (uint32_t)a.K ? cand : thr;
  };
  // The first kShareHi steps compare top bits only (their candidates' low 16 bits are zero),
  // two entries per register: the top halves of non-negative fp32 patterns are below 0x8000
  // and the candidates' at most 0x8000, so x < c is the sign bit of the 16-bit difference
  // x - c (packed subtract, shift and add; no compare results in VCC).
  jd_u16x2 hp[kPer / 2];
#pragma unroll
  for (int i = 0; i < kPer / 2; ++i)
    hp[i] = jd_u16x2{(unsigned short)(v[2 * i] >> 16), (unsigned short)(v[2 * i + 1] >> 16)};
  auto step_hi = [&](uint32_t thr, int bit) {
    const uint32_t cand = thr | (1u << bit);
    const unsigned short c16 = (unsigned short)(cand >> 16);
    const jd_u16x2 cc = {c16, c16};
    jd_u16x2 lt = {0, 0};
#pragma unroll
    for (int i = 0; i < kPer / 2; ++i) lt += (jd_u16x2)(hp[i] - cc) >> (unsigned short)15;
    uint32_t c = (uint32_t)kPer - ((uint32_t)lt.x + (uint32_t)lt.y);
    c = wave_sum_u(c);
    if (lane == 0) part_u[bit & 1][wave] = c;
    __syncthreads();
    const uint32_t tot = part_u[bit & 1][0] + part_u[bit & 1][1] + part_u[bit & 1][2] + part_u[bit & 1][3];
    return tot >= (uint32_t)a.K ? cand : thr;
  };
  static_assert(32 - kShareHi >= 16, "the packed steps need candidates with zero low 16 bits");
  uint32_t thr = 0;
  for (int bit = 31; bit >= 32 - kShareHi; --bit) thr = step_hi(thr, bit);
  // Bucket: entries whose top kShareHi bits equal thr's; above: entries with larger top bits.
  const uint32_t hi = thr >> (32 - kShareHi);
  uint32_t nb = 0, above = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const uint32_t tb = v[j] >> (32 - kShareHi);
    nb += tb == hi;
    above += tb > hi;
  }
  const uint32_t nb_incl = wave_incl_scan_u(nb, lane);
  const uint32_t above_w = wave_sum_u(above);
  if (lane == 63) wtot[0][wave] = nb_incl;
  if (lane == 0) wtot[1][wave] = above_w;
  __syncthreads();
  uint32_t nb_off = nb_incl - nb;
  for (int q = 0; q < wave; ++q) nb_off += wtot[0][q];
  const uint32_t nb_tot = wtot[0][0] + wtot[0][1] + wtot[0][2] + wtot[0][3];
  const uint32_t above_tot = wtot[1][0] + wtot[1][1] + wtot[1][2] + wtot[1][3];
  if (nb_tot <= (uint32_t)kShareCap) {
    uint32_t o = nb_off;
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if ((v[j] >> (32 - kShareHi)) == hi) buck[o++] = v[j];
    __syncthreads();
    if (wave == 0) {
      // want-th largest in the bucket, want = K - above_tot >= 1 (the top bits are maximal)
      const uint32_t want = (uint32_t)a.K - above_tot;
      uint32_t x[kShareCap / 64];
#pragma unroll
      for (int i = 0; i < kShareCap / 64; ++i) {
        const uint32_t idx = (uint32_t)(lane + 64 * i);
        x[i] = idx < nb_tot ? buck[idx] : 0u;  // 0 is below every candidate (it has bits set)
      }
      uint32_t th = thr;
      for (int bit = 31 - kShareHi; bit >= 0; --bit) {
        const uint32_t cand = th | (1u << bit);
        uint32_t c = 0;
#pragma unroll
        for (int i = 0; i < kShareCap / 64; ++i) c += x[i] >= cand;
        if (wave_sum_u(c) >= want) th = cand;
      }
      if (lane == 0) thr_out = th;
    }
    __syncthreads();
    thr = thr_out;
  } else {
    for (int bit = 31 - kShareHi; bit >= 0; --bit) thr = step(thr, bit);
  }
  // Mass above thr, plus thr for the ties needed to make K.
  float sum = 0.f;
  uint32_t gt = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (v[j] > thr) {
      sum += __uint_as_float(v[j]);
      ++gt;
    }
  }
  sum = wave_sum_f(sum);
  gt = wave_sum_u(gt);
  __syncthreads();
  if (lane == 0) {
    part_f[wave] = sum;
    part_u[0][wave] = gt;
  }
  __syncthreads();
  if (t == 0) {
    const float s4 = ((part_f[0] + part_f[1]) + part_f[2]) + part_f[3];
    const uint32_t g4 = part_u[0][0] + part_u[0][1] + part_u[0][2] + part_u[0][3];
    a.share[bh * a.rows + r] = s4 + (float)((int)a.K - (int)g4) * __uint_as_float(thr);
  }
}

// ---------------------------------------------------------------------------------------
// gram_kernel: one workgroup per (bh, key frame f2, chunk of kGramChunk sample positions s1).
// Thread t takes columns s2 = t, t + 256, ... of frame f2 and accumulates, over its s1 chunk,
// the products of the F values P[f1*ns + s1][f2*ns + s2] (f1 = 0..F-1) of each column.
// Partial sums go to G_part[bh][f2][chunk][pair]; the finish kernel adds the chunks in order.
constexpr int kGramChunk = 8;

struct GramArgs {
  const float* P;
  int64_t p_bh, p_row;
  int ns, n_chunks;
  float* G;  // [BH][F][n_chunks][F*(F+1)/2]
  int64_t total;
};

template <int F>
__global__ __launch_bounds__(256) void gram_kernel(GramArgs a) {
  constexpr int NP = F * (F + 1) / 2;
  __shared__ float part[4][NP];
  const int64_t w = blockIdx.x;
  if (w >= a.total) return;
  const int t = threadIdx.x, wave = t >> 6;
  const int64_t bhf = w / a.n_chunks;
  const int chunk = (int)(w - bhf * a.n_chunks);
  const int64_t bh = bhf / F;
  const int f2 = (int)(bhf - bh * F);
  const int s1_lo = chunk * kGramChunk, s1_hi = min(a.ns, s1_lo + kGramChunk);
  float acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) acc[p] = 0.f;
  const float* base = a.P + bh * a.p_bh + (int64_t)f2 * a.ns;
  for (int s2 = t; s2 < a.ns; s2 += 256) {
    for (int s1 = s1_lo; s1 < s1_hi; ++s1) {
      float x[F];
#pragma unroll
      for (int f1 = 0; f1 < F; ++f1) x[f1] = base[(int64_t)(f1 * a.ns + s1) * a.p_row + s2];
      int p = 0;
#pragma unroll
      for (int f1 = 0; f1 < F; ++f1)
#pragma unroll
        for (int f3 = f1; f3 < F; ++f3) {
          acc[p] = fmaf(x[f1], x[f3], acc[p]);
          ++p;
        }
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float r = wave_sum_f(acc[p]);
    if ((t & 63) == 0) part[wave][p] = r;
  }
  __syncthreads();
  float* out = a.G + (bhf * a.n_chunks + chunk) * NP;
  for (int p = t; p < NP; p += 256) out[p] = ((part[0][p] + part[1][p]) + part[2][p]) + part[3][p];
}

// ---------------------------------------------------------------------------------------
// simgram_kernel: judge_similarity with the probabilities kept on chip. One wave per (bh,
// chunk of kGramChunk = 8 sample positions s1). Its three 32-column query groups hold the
// F frames' rows f1*ns + s1 of the 8 positions, 12 columns per position: flat column
// 32 g + col = 12 j + f1 for position j of the chunk (columns with f1 >= F and positions
// past ns are zero queries whose results are never used).
//   pass 1: row max and sum over every key, bias on the T text keys (as probs_kernel);
//   pass 2, per key frame f2: the probabilities of the frame's ns keys, 32 at a time, go
//           through LDS ([key][flat column]); lane (key k, half sl) then adds, for each of
//           its positions 4 sl .. 4 sl + 3, the products P[f1][k] P[f3][k] of the
//           position's F rows into F(F+1)/2 per-lane sums. After the frame the 64 lanes' sums are added through LDS, in lane
//           order, into G[bh][f2][chunk][pair].
struct SimGramArgs {
  const uint16_t* qs;  // [BH][rows_pad][64], row f*ns + s
  const uint16_t* ks;  // [BH][keys_pad][64], T text keys then F*ns sampled keys
  int ns, T, keys, keys_pad, rows_pad;
  float scale_log2, bias_log2;
  float* G;  // [BH][F][n_chunks][NP]
  int n_chunks;
  int64_t total;  // BH * n_chunks
};

constexpr int kSgWidth = 12;                            // columns per position (F <= 12)
constexpr int kSgGroups = kGramChunk * kSgWidth / 32;  // query groups per wave
static_assert(kGramChunk * kSgWidth == 32 * kSgGroups, "positions fill whole query groups");
// LDS row stride (floats) of the P tile [key][flat column]: stride / 4 odd, so a b128 read
// by 16 lanes of consecutive keys covers 16 distinct 4-bank chunks (64 banks).
constexpr int kSgStride = 32 * kSgGroups + 4;

template <int F>
__global__ __launch_bounds__(256, 2) void simgram_kernel(SimGramArgs a) {
  static_assert(F >= 1 && F <= 12, "frames");
  constexpr int NP = F * (F + 1) / 2;
  constexpr int kRed = 64 * NP;
  constexpr int kTile = 32 * kSgStride;
  constexpr int kLds = kRed > kTile ? kRed : kTile;
  constexpr int kRead = (F + 3) / 4;  // 16-byte reads per row of F values
  __shared__ __attribute__((aligned(16))) float lds[4][kLds];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave;
  if (wid >= a.total) return;  // no workgroup barriers below
  const int64_t bh = wid / a.n_chunks;
  const int chunk = (int)(wid - bh * a.n_chunks);
  const int col = lane & 31, hh = lane >> 5;
  float* L = lds[wave];

  sa_bf16x8 qf[kSgGroups][4];
#pragma unroll
  for (int g = 0; g < kSgGroups; ++g) {
    const int flat = 32 * g + col;
    const int s1 = chunk * kGramChunk + flat / kSgWidth, f1 = flat % kSgWidth;
    const bool ok = f1 < F && s1 < a.ns;
    const uint16_t* qp = a.qs + (bh * a.rows_pad + (ok ? f1 * a.ns + s1 : 0)) * kD + 8 * hh;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const jd_u32x4 w = ok ? *reinterpret_cast<const jd_u32x4*>(qp + 16 * s) : jd_u32x4{0u, 0u, 0u, 0u};
      qf[g][s] = __builtin_bit_cast(sa_bf16x8, w);
    }
  }

  // ---- pass 1: row statistics over every key
  float m[kSgGroups], l[kSgGroups];
#pragma unroll
  for (int g = 0; g < kSgGroups; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
  }
  const uint16_t* kbase = a.ks + (bh * a.keys_pad + col) * kD + 8 * hh;
  for (int kt = 0; kt < a.keys_pad / 32; ++kt) {
    jd_u32x4 kop[4];
    load_k(kbase + (int64_t)kt * 32 * kD, kop);
    const bool uniform = 32 * kt + 32 <= a.keys && (32 * kt + 32 <= a.T || 32 * kt >= a.T);
    const float tb = 32 * kt < a.T ? a.bias_log2 : 0.f;
#pragma unroll
    for (int g = 0; g < kSgGroups; ++g) {
      const sa_f32x16 t = score_tile_k(kop, qf[g]);
      float x[16], tmax = -INFINITY;
      if (uniform) {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = fmaf(t[i], a.scale_log2, tb);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = 32 * kt + 8 * (i >> 2) + 4 * hh + (i & 3);
          x[i] = key >= a.keys ? -INFINITY : fmaf(t[i], a.scale_log2, key < a.T ? a.bias_log2 : 0.f);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, x[i]);
      const float mn = fmaxf(m[g], tmax);
      if (mn != -INFINITY) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) sum += __builtin_amdgcn_exp2f(x[i] - mn);
        l[g] = l[g] * __builtin_amdgcn_exp2f(m[g] - mn) + sum;
        m[g] = mn;
      }
    }
  }
  float inv[kSgGroups];
#pragma unroll
  for (int g = 0; g < kSgGroups; ++g) {
    const auto mo = __builtin_amdgcn_permlane32_swap(__float_as_uint(m[g]), __float_as_uint(m[g]), false, false);
    const auto lo = __builtin_amdgcn_permlane32_swap(__float_as_uint(l[g]), __float_as_uint(l[g]), false, false);
    const float m0 = __uint_as_float(mo[0]), m1 = __uint_as_float(mo[1]);
    const float M = fmaxf(m0, m1);
    const float lt = __uint_as_float(lo[0]) * __builtin_amdgcn_exp2f(m0 - M) +
                     __uint_as_float(lo[1]) * __builtin_amdgcn_exp2f(m1 - M);
    m[g] = M;
    inv[g] = 1.f / lt;
  }

  // ---- pass 2: per key frame, probabilities through LDS and the pair products. Columns of
  // positions past ns (zero queries, whose uniform rows are not samples) write zeros.
  bool pos_ok[kSgGroups];
#pragma unroll
  for (int g = 0; g < kSgGroups; ++g) {
    const int flat = 32 * g + col;
    pos_ok[g] = chunk * kGramChunk + flat / kSgWidth < a.ns && flat % kSgWidth < F;
  }
  const int my_key = lane & 31, sl = lane >> 5;
  const int n_kt = (a.ns + 31) / 32;
  float acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) acc[p] = 0.f;
  for (int f2 = 0; f2 < F; ++f2) {
    const int frame0 = a.T + f2 * a.ns;
    for (int t = 0; t < n_kt; ++t) {
      jd_u32x4 kop[4];
      load_k(a.ks + (bh * a.keys_pad + min(frame0 + 32 * t + col, a.keys_pad - 1)) * kD + 8 * hh, kop);
#pragma unroll
      for (int g = 0; g < kSgGroups; ++g) {
        const sa_f32x16 tt = score_tile_k(kop, qf[g]);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kr = 8 * (i >> 2) + 4 * hh + (i & 3);
          const float pv = (pos_ok[g] && 32 * t + kr < a.ns)
                               ? __builtin_amdgcn_exp2f(fmaf(tt[i], a.scale_log2, -m[g])) * inv[g] : 0.f;
          L[kr * kSgStride + 32 * g + col] = pv;
        }
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < kGramChunk / 2; ++j) {
        float x[4 * kRead];
        const float* rp = L + my_key * kSgStride + kSgWidth * (kGramChunk / 2 * sl + j);
#pragma unroll
        for (int u = 0; u < kRead; ++u) {
          const float4 v4 = *reinterpret_cast<const float4*>(rp + 4 * u);
          x[4 * u] = v4.x;
          x[4 * u + 1] = v4.y;
          x[4 * u + 2] = v4.z;
          x[4 * u + 3] = v4.w;
        }
        int p = 0;
#pragma unroll
        for (int f1 = 0; f1 < F; ++f1)
#pragma unroll
          for (int f3 = f1; f3 < F; ++f3) {
            acc[p] = fmaf(x[f1], x[f3], acc[p]);
            ++p;
          }
      }
      __builtin_amdgcn_wave_barrier();
    }
    // lanes' sums -> LDS [lane][pair] -> lane p adds pair p over the 64 lanes in order
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      L[lane * NP + p] = acc[p];
      acc[p] = 0.f;
    }
    __builtin_amdgcn_wave_barrier();
    float* out = a.G + ((bh * F + f2) * a.n_chunks + chunk) * NP;
    for (int p = lane; p < NP; p += 64) {
      float sum = 0.f;
      for (int q = 0; q < 64; ++q) sum += L[q * NP + p];
      out[p] = sum;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------------------
struct FinishArgs {
  const float* share;  // [BH][rows] or null
  const float* G1;     // [BH][F][n_chunks][NP] partials or null
  const float* G2;
  int BH, rows, F, n_chunks;
  float sparse_thr, sim_thr;
  float* share_mean;  // [BH]
  float* col1;        // [BH]
  float* col2;        // [BH]
  int32_t* use;       // [BH]
};

// Block sum over the 256 threads in a fixed order (per-wave shuffles, then the four waves).
__device__ float block_sum(float x, float* red /* LDS [4] */) {
  x = wave_sum_f(x);
  const int t = threadIdx.x;
  __syncthreads();
  if ((t & 63) == 0) red[t >> 6] = x;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

// Mean cosine similarity of the patterns sharing a key frame, from one head's Gram partials:
// col = mean over f2 of mean over (f1, f3) of G[f2][f1][f3] / sqrt(G[f2][f1][f1] G[f2][f3][f3]).
__device__ float col_sim(const float* Gp, int F, int n_chunks, float* gs /* LDS [F * NP] */, float* red) {
  const int t = threadIdx.x;
  const int NP = F * (F + 1) / 2;
  __syncthreads();
  for (int e = t; e < F * NP; e += 256) {
    const int f2 = e / NP, p = e - f2 * NP;
    float s = 0.f;
    for (int c = 0; c < n_chunks; ++c) s += Gp[((int64_t)f2 * n_chunks + c) * NP + p];
    gs[e] = s;
  }
  __syncthreads();
  auto at = [&](const float* g, int i, int j) {
    if (i > j) {
      const int tmp = i;
      i = j;
      j = tmp;
    }
    return g[i * F - i * (i - 1) / 2 + (j - i)];
  };
  float part = 0.f;
  for (int u = t; u < F * F * F; u += 256) {
    const int f2 = u / (F * F), f1 = (u / F) % F, f3 = u % F;
    const float* g = gs + f2 * NP;
    part += at(g, f1, f3) / sqrtf(at(g, f1, f1) * at(g, f3, f3));
  }
  return block_sum(part, red) / (float)(F * F * F);
}

// One 256-thread workgroup per head.
__global__ __launch_bounds__(256) void finish_kernel(FinishArgs a) {
  __shared__ float gs[12 * 78];
  __shared__ float red[4];
  const int bh = blockIdx.x;
  if (bh >= a.BH) return;
  const int t = threadIdx.x;
  float s = 0.f;
  if (a.share) {
    for (int r = t; r < a.rows; r += 256) s += a.share[(int64_t)bh * a.rows + r];
    s = block_sum(s, red) / (float)a.rows;
  }
  const int NP = a.F * (a.F + 1) / 2;
  const int64_t gstride = (int64_t)a.F * a.n_chunks * NP;
  const float c1 = a.G1 ? col_sim(a.G1 + bh * gstride, a.F, a.n_chunks, gs, red) : 0.f;
  const float c2 = a.G2 ? col_sim(a.G2 + bh * gstride, a.F, a.n_chunks, gs, red) : 0.f;
  if (t == 0) {
    a.share_mean[bh] = s;
    a.col1[bh] = c1;
    a.col2[bh] = c2;
    a.use[bh] = (!(s > a.sparse_thr) && c1 > a.sim_thr && c2 > a.sim_thr) ? 1 : 0;
  }
}

}  // namespace

extern "C" int sa_sampled_probs(const uint16_t* q_rows, const uint16_t* k_rows, int BH, int rows, int rows_pad,
                                int keys, int keys_pad, float sm_scale, int n_bias, float bias, int c_lo, int c_hi,
                                float* P, int64_t p_bh_stride, int64_t p_row_stride, void* stream) {
  const char* fn = "sa_sampled_probs";
  SA_REQUIRE(q_rows && k_rows && P, "%s: null pointer", fn);
  SA_REQUIRE(reinterpret_cast<uintptr_t>(q_rows) % 16 == 0 && reinterpret_cast<uintptr_t>(k_rows) % 16 == 0,
             "%s: q_rows/k_rows must be 16-byte aligned", fn);
  SA_REQUIRE(BH > 0 && rows > 0 && keys > 0, "%s: bad shape", fn);
  SA_REQUIRE(rows_pad % 32 == 0 && rows_pad >= rows && keys_pad % 32 == 0 && keys_pad >= keys,
             "%s: rows_pad/keys_pad must be multiples of 32 covering rows/keys", fn);
  SA_REQUIRE(0 <= c_lo && c_lo < c_hi && c_hi <= keys, "%s: bad key range [%d, %d)", fn, c_lo, c_hi);
  SA_REQUIRE(std::isfinite(sm_scale) && sm_scale > 0.f, "%s: bad sm_scale", fn);
  SA_REQUIRE(p_row_stride >= c_hi - c_lo, "%s: p_row_stride too small", fn);
  ProbArgs a;
  a.qs = q_rows; a.ks = k_rows; a.rows = rows; a.rows_pad = rows_pad; a.keys = keys; a.keys_pad = keys_pad;
  a.scale_log2 = sm_scale * kLog2e; a.n_bias = n_bias; a.bias_log2 = bias * kLog2e;
  a.c_lo = c_lo; a.c_hi = c_hi; a.P = P; a.p_bh = p_bh_stride; a.p_row = p_row_stride;
  a.ng = rows_pad / 32; a.total = (int64_t)BH * a.ng;
  a.vec_ok = (reinterpret_cast<uintptr_t>(P) % 16 == 0 && p_row_stride % 4 == 0 && p_bh_stride % 4 == 0 &&
              c_lo % 4 == 0) ? 1 : 0;
  hipLaunchKernelGGL(probs_kernel, dim3((unsigned)((a.total + 3) / 4)), dim3(256), 0, sa::as_stream(stream), a);
  return sa::check_launch(fn);
}

extern "C" int sa_topk_share(const float* P, int64_t p_bh_stride, int64_t p_row_stride, int BH, int rows, int n,
                             int K, float* share, void* stream) {
  const char* fn = "sa_topk_share";
  SA_REQUIRE(P && share, "%s: null pointer", fn);
  SA_REQUIRE(BH > 0 && rows > 0 && n > 0 && K >= 1 && K <= n, "%s: bad shape (1 <= K <= n)", fn);
  if (n > 16384) return sa::fail(SA_ERR_UNSUPPORTED, "%s: n=%d > 16384", fn, n);
  ShareArgs a;
  a.P = P; a.p_bh = p_bh_stride; a.p_row = p_row_stride; a.rows = rows; a.n = n; a.K = K; a.share = share;
  a.vec_ok = (reinterpret_cast<uintptr_t>(P) % 16 == 0 && p_bh_stride % 4 == 0 && p_row_stride % 4 == 0) ? 1 : 0;
  a.total = (int64_t)BH * rows;
  hipLaunchKernelGGL(share_kernel, dim3((unsigned)a.total), dim3(256), 0, sa::as_stream(stream), a);
  return sa::check_launch(fn);
}

extern "C" int sa_pattern_gram(const float* P, int64_t p_bh_stride, int64_t p_row_stride, int BH, int F, int ns,
                               float* G, void* stream) {
  const char* fn = "sa_pattern_gram";
  SA_REQUIRE(P && G, "%s: null pointer", fn);
  SA_REQUIRE(BH > 0 && ns > 0 && ns <= 512, "%s: bad shape (ns <= 512)", fn);
  SA_REQUIRE(F >= 1 && F <= 12, "%s: frames %d outside [1, 12]", fn, F);
  GramArgs a;
  a.P = P; a.p_bh = p_bh_stride; a.p_row = p_row_stride; a.ns = ns; a.G = G;
  a.n_chunks = (ns + kGramChunk - 1) / kGramChunk;
  a.total = (int64_t)BH * F * a.n_chunks;
  const dim3 g((unsigned)a.total), blk(256);
  hipStream_t s = sa::as_stream(stream);
  switch (F) {
#define SA_GRAM_CASE(n)\
  case n:              \
    hipLaunchKernelGGL(gram_kernel<n>, g, blk, 0, s, a);\
    break;
    SA_GRAM_CASE(1) SA_GRAM_CASE(2) SA_GRAM_CASE(3) SA_GRAM_CASE(4) SA_GRAM_CASE(5) SA_GRAM_CASE(6)
    SA_GRAM_CASE(7) SA_GRAM_CASE(8) SA_GRAM_CASE(9) SA_GRAM_CASE(10) SA_GRAM_CASE(11) SA_GRAM_CASE(12)
#undef SA_GRAM_CASE
  }
  return sa::check_launch(fn);
}

extern "C" int sa_pattern_judge_finish(const float* share, const float* G1, const float* G2, int BH, int rows, int F,
                                       int ns, float sparse_thr, float sim_thr, float* share_mean, float* col1, float* col2,
                                       int32_t* use, void* stream) {
  const char* fn = "sa_pattern_judge_finish";
  SA_REQUIRE(share_mean && col1 && col2 && use, "%s: null output", fn);
  SA_REQUIRE(BH > 0 && rows > 0 && F >= 1 && F <= 12 && ns > 0, "%s: bad shape", fn);
  FinishArgs a;
  a.share = share; a.G1 = G1; a.G2 = G2; a.BH = BH; a.rows = rows; a.F = F;
  a.n_chunks = (ns + kGramChunk - 1) / kGramChunk;
  a.sparse_thr = sparse_thr; a.sim_thr = sim_thr; a.share_mean = share_mean; a.col1 = col1; a.col2 = col2; a.use = use;
  hipLaunchKernelGGL(finish_kernel, dim3((unsigned)BH), dim3(256), 0, sa::as_stream(stream), a);
  return sa::check_launch(fn);
}

extern "C" int sa_pattern_sim_gram(const uint16_t* q_rows, const uint16_t* k_rows, int BH, int F, int ns, int T,
                                   int rows_pad, int keys_pad, float sm_scale, float bias, float* G, void* stream) {
  const char* fn = "sa_pattern_sim_gram";
  SA_REQUIRE(q_rows && k_rows && G, "%s: null pointer", fn);
  SA_REQUIRE(reinterpret_cast<uintptr_t>(q_rows) % 16 == 0 && reinterpret_cast<uintptr_t>(k_rows) % 16 == 0,
             "%s: q_rows/k_rows must be 16-byte aligned", fn);
  SA_REQUIRE(BH > 0 && F >= 1 && F <= 12 && ns > 0 && T >= 0, "%s: bad shape (1 <= F <= 12)", fn);
  SA_REQUIRE(rows_pad % 32 == 0 && rows_pad >= F * ns && keys_pad % 32 == 0 && keys_pad >= T + F * ns,
             "%s: rows_pad/keys_pad must be multiples of 32 covering F*ns / T+F*ns", fn);
  SA_REQUIRE(std::isfinite(sm_scale) && sm_scale > 0.f && std::isfinite(bias), "%s: bad sm_scale/bias", fn);
  SimGramArgs a;
  a.qs = q_rows; a.ks = k_rows; a.ns = ns; a.T = T; a.keys = T + F * ns; a.keys_pad = keys_pad; a.rows_pad = rows_pad;
  a.scale_log2 = sm_scale * kLog2e; a.bias_log2 = bias * kLog2e; a.G = G;
  a.n_chunks = (ns + kGramChunk - 1) / kGramChunk;
  a.total = (int64_t)BH * a.n_chunks;
  const dim3 grid((unsigned)((a.total + 3) / 4)), blk(256);
  hipStream_t s = sa::as_stream(stream);
  switch (F) {
#define SA_SG_CASE(n) \
  case n: hipLaunchKernelGGL(simgram_kernel<n>, grid, blk, 0, s, a); break;
    SA_SG_CASE(1) SA_SG_CASE(2) SA_SG_CASE(3) SA_SG_CASE(4) SA_SG_CASE(5) SA_SG_CASE(6)
    SA_SG_CASE(7) SA_SG_CASE(8) SA_SG_CASE(9) SA_SG_CASE(10) SA_SG_CASE(11) SA_SG_CASE(12)
#undef SA_SG_CASE
  }
  return sa::check_launch(fn);
}
