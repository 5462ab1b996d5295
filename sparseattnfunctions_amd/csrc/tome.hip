// Token merging (ToMe bipartite soft matching) for video tokens on gfx950.
//
// Replaces bipartite_soft_matching_video and its merge / unmerge closures
// (special_attentions/utils/merge_unmerge.py:34-156) as used by MergeAttention
// (MergeAttention.py:21-49):
//   partition  first frame all dst; later frames one dst per (st, sy, sx) cell, the rest src
//              (:62-92), dst|src order = stable argsort of the {-1, 0} buffer (:82);
//   metric     cosine-normalised matching metric (:100);
//   match      scores = a @ b^T, node_max/node_idx = max over dst (:102, :108), fused so the
//              [n_src, n_dst] score matrix is never materialised;
//   edges      edge order = argsort(node_max, descending) (:109), src_idx = first r,
//              unm_idx = the rest, dst_idx = node_idx[src_idx] (:110-112), sizes (:113-116);
//   merge      [text | unm | dst] with dst = mean(dst, merged srcs) (scatter_reduce mean,
//              include_self, :119-135);
//   unmerge    every token reads its merged row (:137-154).
//
// Determinism contract (built with -ffp-contract=off, matched by oracle/sa_oracle.c):
//   metric: head sums in head order / dot products as fmaf chains in channel order, norm
//   = sqrtf(fmaf chain of squares), value / norm (IEEE); scores: fmaf chain over channels;
//   argmax ties -> lowest dst position; edge order: node_max descending (total order on fp32
//   bits) then src position ascending (a stable sort; torch's argsort order is unspecified);
//   merged dst value: fp32 sum of the dst token then its srcs in edge order, divided by the
//   count, rounded to bf16. Integer counters use atomics (order-independent).
#include <math.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "sa_common.h"

namespace {

constexpr int kD = 64;           // head dim handled here
constexpr int kMaxC = 2 * kD + 2;  // channels of the per-head (k, |k|, v, |v|) metric
constexpr int kMTile = 128;      // src rows per match workgroup, dst columns per dst tile
constexpr int kMChunk = 16;      // channels staged in LDS per step
constexpr int kMLd = kMTile + 4;  // channel-major LDS row (16-byte aligned; 4-bank offset per row)
constexpr int kMMaxSplits = 16;  // dst splits of the match grid
constexpr int kRankTile = 256;   // keys per sorted rank tile

__device__ inline float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ inline uint32_t order_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Round-to-nearest-even fp32 -> bf16 -> fp32 (finite inputs).
__device__ inline float round_bf16(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(r & 0xffff0000u);
}

__device__ inline void add_row(float* acc, const uint16_t* row) {
#pragma unroll
  for (int c8 = 0; c8 < kD / 8; ++c8) {
    const uint4 w = *reinterpret_cast<const uint4*>(row + 8 * c8);
    acc[8 * c8 + 0] += bf16lo(w.x); acc[8 * c8 + 1] += bf16hi(w.x);
    acc[8 * c8 + 2] += bf16lo(w.y); acc[8 * c8 + 3] += bf16hi(w.y);
    acc[8 * c8 + 4] += bf16lo(w.z); acc[8 * c8 + 5] += bf16hi(w.z);
    acc[8 * c8 + 6] += bf16lo(w.w); acc[8 * c8 + 7] += bf16hi(w.w);
  }
}

// ---------------------------------------------------------------------------------------
// Metric. Mode 0: per batch, sum over heads of k (the head mean up to the factor 1/H, which
// the normalisation removes) -> [B][N][64] (metric_sum_kernel). Mode 1: per head, (k, |k|, v,
// |v|) as in MergeAttention.py:26-31 -> [B*H][N][130], one thread per output row.
struct MetricArgs {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
  int B, H, N, text_len, mode;
  float* out;
};

__global__ __launch_bounds__(256) void metric_kernel(MetricArgs a) {  // mode 1
  const int64_t rows = (int64_t)a.B * a.H * a.N;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows) return;
  {
    const int64_t bh = i / a.N;
    const int n = (int)(i - bh * a.N);
    const int64_t b = bh / a.H, h = bh - b * a.H;
    float kk[kD], vv[kD];
#pragma unroll
    for (int d = 0; d < kD; ++d) kk[d] = vv[d] = 0.f;
    add_row(kk, a.k + b * a.k_sb + h * a.k_sh + (int64_t)(a.text_len + n) * a.k_sl);
    add_row(vv, a.v + b * a.v_sb + h * a.v_sh + (int64_t)(a.text_len + n) * a.v_sl);
    float kq = 0.f, vq = 0.f;
#pragma unroll
    for (int d = 0; d < kD; ++d) kq = fmaf(kk[d], kk[d], kq);
#pragma unroll
    for (int d = 0; d < kD; ++d) vq = fmaf(vv[d], vv[d], vq);
    const float kn = sqrtf(kq), vn = sqrtf(vq);
    float ss = 0.f;
#pragma unroll
    for (int d = 0; d < kD; ++d) ss = fmaf(kk[d], kk[d], ss);
    ss = fmaf(kn, kn, ss);
#pragma unroll
    for (int d = 0; d < kD; ++d) ss = fmaf(vv[d], vv[d], ss);
    ss = fmaf(vn, vn, ss);
    const float nrm = sqrtf(ss);
    float* o = a.out + i * kMaxC;
#pragma unroll
    for (int d = 0; d < kD; ++d) o[d] = kk[d] / nrm;
    o[kD] = kn / nrm;
#pragma unroll
    for (int d = 0; d < kD; ++d) o[kD + 1 + d] = vv[d] / nrm;
    o[2 * kD + 1] = vn / nrm;
  }
}

// Mode 0 with 8 lanes per output row: lane (row, s = lane & 7) sums dims 8s..8s+7 of the
// row over the heads in head order (the loads of 16 heads are issued before their adds),
// then the row's 64 sums pass through LDS so that every lane forms the norm with the same
// fmaf chain over d = 0..63 ascending as the one-thread form; each lane writes its 8 dims.
// One thread per row left 35 100 threads for the C4 metric (about two waves per CU), each
// walking its 30 head rows in turn: 36.9 us against 27.6 us.
constexpr int kMetricHeadsInFlight = 16;

__global__ __launch_bounds__(256) void metric_sum_kernel(MetricArgs a) {
  __shared__ __attribute__((aligned(16))) float rows_lds[32][kD + 4];
  const int64_t rows = (int64_t)a.B * a.N;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
  const int sl = threadIdx.x & 7;
  const int lr = threadIdx.x >> 3;  // row of the workgroup
  const bool ok = i < rows;
  const int64_t ic = ok ? i : rows - 1;
  const int64_t b = ic / a.N;
  const int n = (int)(ic - b * a.N);
  const uint16_t* p = a.k + b * a.k_sb + (int64_t)(a.text_len + n) * a.k_sl + 8 * sl;
  float m[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int h0 = 0; h0 < a.H; h0 += kMetricHeadsInFlight) {
    uint4 w[kMetricHeadsInFlight];
#pragma unroll
    for (int u = 0; u < kMetricHeadsInFlight; ++u)
      w[u] = *reinterpret_cast<const uint4*>(p + (int64_t)min(h0 + u, a.H - 1) * a.k_sh);
#pragma unroll
    for (int u = 0; u < kMetricHeadsInFlight; ++u) {
      if (h0 + u < a.H) {
        m[0] += bf16lo(w[u].x); m[1] += bf16hi(w[u].x); m[2] += bf16lo(w[u].y); m[3] += bf16hi(w[u].y);
        m[4] += bf16lo(w[u].z); m[5] += bf16hi(w[u].z); m[6] += bf16lo(w[u].w); m[7] += bf16hi(w[u].w);
      }
    }
  }
  float* r = rows_lds[lr];
  *reinterpret_cast<float4*>(r + 8 * sl) = make_float4(m[0], m[1], m[2], m[3]);
  *reinterpret_cast<float4*>(r + 8 * sl + 4) = make_float4(m[4], m[5], m[6], m[7]);
  __syncthreads();
  float ss = 0.f;
#pragma unroll
  for (int d = 0; d < kD; d += 4) {
    const float4 x = *reinterpret_cast<const float4*>(r + d);
    ss = fmaf(x.x, x.x, ss);
    ss = fmaf(x.y, x.y, ss);
    ss = fmaf(x.z, x.z, ss);
    ss = fmaf(x.w, x.w, ss);
  }
  if (!ok) return;
  const float nrm = sqrtf(ss);
  float* o = a.out + i * kD + 8 * sl;
  *reinterpret_cast<float4*>(o) = make_float4(m[0] / nrm, m[1] / nrm, m[2] / nrm, m[3] / nrm);
  *reinterpret_cast<float4*>(o + 4) = make_float4(m[4] / nrm, m[5] / nrm, m[6] / nrm, m[7] / nrm);
}

// Row normalisation of a caller-supplied metric [rows][C]: x / sqrtf(fmaf chain of x^2).
__global__ __launch_bounds__(256) void normalize_kernel(const float* in, int64_t rows, int C, float* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows) return;
  const float* x = in + i * C;
  float ss = 0.f;
  for (int c = 0; c < C; ++c) ss = fmaf(x[c], x[c], ss);
  const float nrm = sqrtf(ss);
  for (int c = 0; c < C; ++c) out[i * C + c] = x[c] / nrm;
}

// ---------------------------------------------------------------------------------------
// Match: for each src, the dst of largest score (fmaf chain over channels) in this
// workgroup's dst range; ties -> lowest dst position. Workgroup = 128 src x dst range in
// 128-column dst tiles; thread (ty, tx) owns src rows 8ty..8ty+7 and dst columns
// 8tx..8tx+7 of each tile (64 accumulators: two 16-byte LDS reads per operand and channel
// feed 64 FMAs). Channels are staged 16 at a time, channel-major (As[c][row], Bs[c][col]),
// and every score still runs its fmaf chain over c = 0..C-1 in order.
struct MatchArgs {
  const float* metric;  // [G][N][C]
  int G, N, C;
  const int32_t* a_idx;
  const int32_t* b_idx;
  int n_src, n_dst;
  int splits, dst_per_split;  // dst_per_split: a multiple of kMTile
  float* part_max;  // [G][splits][n_src]
  int32_t* part_idx;
};

__device__ inline bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__global__ __launch_bounds__(256) void match_kernel(MatchArgs a) {
  __shared__ __attribute__((aligned(16))) float As[kMChunk * kMLd];
  __shared__ __attribute__((aligned(16))) float Bs[kMChunk * kMLd];
  const int C = a.C;
  const int g = blockIdx.y, split = blockIdx.z;
  const int s0 = blockIdx.x * kMTile;
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const float* mg = a.metric + (int64_t)g * a.N * C;
  float best[8];
  int bidx[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    best[i] = -INFINITY;
    bidx[i] = 0;
  }
  const int d_lo = split * a.dst_per_split;
  const int d_hi = min(a.n_dst, d_lo + a.dst_per_split);
  for (int d0 = d_lo; d0 < d_hi; d0 += kMTile) {
    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;
    for (int c0 = 0; c0 < C; c0 += kMChunk) {
      const int nc = min(kMChunk, C - c0);
      __syncthreads();
      // Element e: row e / 16, channel c0 + e % 16 (16 consecutive channels of one row per
      // 16 threads; the transposed stores hit 64 distinct banks per wave).
      for (int e = tid; e < kMTile * kMChunk; e += 256) {
        const int r = e >> 4, cc = e & 15;
        const int s = s0 + r, d = d0 + r;
        As[cc * kMLd + r] = (s < a.n_src && cc < nc) ? mg[(int64_t)a.a_idx[s] * C + c0 + cc] : 0.f;
        Bs[cc * kMLd + r] = (d < d_hi && cc < nc) ? mg[(int64_t)a.b_idx[d] * C + c0 + cc] : 0.f;
      }
      __syncthreads();
      for (int cc = 0; cc < nc; ++cc) {
        const float4 a0 = *reinterpret_cast<const float4*>(As + cc * kMLd + 8 * ty);
        const float4 a1 = *reinterpret_cast<const float4*>(As + cc * kMLd + 8 * ty + 4);
        const float4 b0 = *reinterpret_cast<const float4*>(Bs + cc * kMLd + 8 * tx);
        const float4 b1 = *reinterpret_cast<const float4*>(Bs + cc * kMLd + 8 * tx + 4);
        const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = d0 + 8 * tx + j;
      if (d < d_hi) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (better(acc[i][j], d, best[i], bidx[i])) {
            best[i] = acc[i][j];
            bidx[i] = d;
          }
        }
      }
    }
  }
  // Reduce over the 16 tx lanes sharing ty (a 16-lane DPP row group of the wave).
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ov = __shfl_xor(best[i], off, 16);
      const int oi = __shfl_xor(bidx[i], off, 16);
      if (better(ov, oi, best[i], bidx[i])) {
        best[i] = ov;
        bidx[i] = oi;
      }
    }
  }
  if (tx == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = s0 + 8 * ty + i;
      if (s < a.n_src) {
        const int64_t o = ((int64_t)g * a.splits + split) * a.n_src + s;
        a.part_max[o] = best[i];
        a.part_idx[o] = bidx[i];
      }
    }
  }
}

// Match on the matrix core for C = 64 (the head-averaged k metric). v_mfma_f32_16x16x4_f32
// adds its four products to the accumulator as an fmaf chain over k = 0..3 in order
// (checked on the hardware against fmaf chains for normal and subnormal operands), so the
// 16 chained steps j (channels 4j .. 4j + 3) give every score the same fmaf chain over
// c = 0..63 as match_kernel, and the maxima are bit-identical. D[m][n] = score(dst m, src n):
// lane l holds A[m = l % 16][k = l / 16] (a staged dst row), B[k = l / 16][n = l % 16] (its
// src rows, kept in registers for the whole range) and D rows 4 (l / 16) .. + 3 of column
// l % 16. Workgroup: 4 waves x 64 src rows (4 blocks of 16), the split's dst range in
// 64-row tiles staged in LDS (double-buffered, loaded into registers one tile ahead).
constexpr int kMfC = 64;           // channels
constexpr int kMfSrcW = 64;        // src rows per wave
constexpr int kMfSrc = 4 * kMfSrcW;
constexpr int kMfDst = 64;         // dst rows per staged tile
constexpr int kMfLd = kMfC + 4;    // floats per staged dst row: A reads hit 64 distinct banks

__global__ __launch_bounds__(256, 2) void match_mfma_kernel(MatchArgs a) {
  __shared__ __attribute__((aligned(16))) float dl[2][kMfDst * kMfLd];
  const int g = blockIdx.y, split = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m16 = lane & 15, kg = lane >> 4;
  const float* mg = a.metric + (int64_t)g * a.N * kMfC;
  const int sw0 = blockIdx.x * kMfSrc + wave * kMfSrcW;
  // B operands: src block sb, step j = channel 4j + kg of src row sw0 + 16 sb + m16.
  float bop[4][kMfC / 4];
#pragma unroll
  for (int sb = 0; sb < 4; ++sb) {
    const int sr = sw0 + 16 * sb + m16;
    const float* row = sr < a.n_src ? mg + (int64_t)a.a_idx[sr] * kMfC : nullptr;
#pragma unroll
    for (int j = 0; j < kMfC / 4; ++j) bop[sb][j] = row ? row[4 * j + kg] : 0.f;
  }
  float best[4];
  int bidx[4];
#pragma unroll
  for (int sb = 0; sb < 4; ++sb) {
    best[sb] = -INFINITY;
    bidx[sb] = 0;
  }
  const int d_lo = split * a.dst_per_split;
  const int d_hi = min(a.n_dst, d_lo + a.dst_per_split);
  // Staging: thread tid holds float4 q = tid + 256 i of a tile, row q / 16, channels
  // 4 (q % 16) .. + 3 (rows past the range are zero and never compete).
  float4 pre[4];
  auto load_tile = [&](int d0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + 256 * i, d = d0 + (q >> 4);
      pre[i] = d < d_hi ? *reinterpret_cast<const float4*>(mg + (int64_t)a.b_idx[d] * kMfC + 4 * (q & 15))
                        : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + 256 * i;
      *reinterpret_cast<float4*>(&dl[buf][(q >> 4) * kMfLd + 4 * (q & 15)]) = pre[i];
    }
  };
  int buf = 0;
  if (d_lo < d_hi) {
    load_tile(d_lo);
    store_tile(0);
  }
  __syncthreads();
  for (int d0 = d_lo; d0 < d_hi; d0 += kMfDst) {  // workgroup-uniform trip count
    const bool more = d0 + kMfDst < d_hi;
    if (more) load_tile(d0 + kMfDst);
    // A lane meets its dst rows in ascending order (tiles ascending, d = d0 + 16 db + 4 kg + i
    // within a tile), so a tie never replaces the lower index: `better` reduces to v > best.
    // Rows past d_hi exist only in the range's last tile. Dst block db's maxima are taken
    // while block db + 1's MFMAs run (they do not depend on each other).
    const bool full = d0 + kMfDst <= d_hi;
    const float* t = dl[buf] + m16 * kMfLd + kg;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      sa_f32x4 acc[4];  // [src block]
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) acc[sb] = sa_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < kMfC / 4; ++j) {
        const float aop = t[16 * db * kMfLd + 4 * j];
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) acc[sb] = __builtin_amdgcn_mfma_f32_16x16x4f32(aop, bop[sb][j], acc[sb], 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = d0 + 16 * db + 4 * kg + i;
        if (full || d < d_hi) {
#pragma unroll
          for (int sb = 0; sb < 4; ++sb) {
            const bool gt = acc[sb][i] > best[sb];
            best[sb] = gt ? acc[sb][i] : best[sb];
            bidx[sb] = gt ? d : bidx[sb];
          }
        }
      }
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  // Lanes m16 + 16 kg hold the same src columns over different dst rows.
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      const float ov = __shfl_xor(best[sb], off);
      const int oi = __shfl_xor(bidx[sb], off);
      if (better(ov, oi, best[sb], bidx[sb])) {
        best[sb] = ov;
        bidx[sb] = oi;
      }
    }
  }
  if (kg == 0) {
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      const int sr = sw0 + 16 * sb + m16;
      if (sr < a.n_src) {
        const int64_t o = ((int64_t)g * a.splits + split) * a.n_src + sr;
        a.part_max[o] = best[sb];
        a.part_idx[o] = bidx[sb];
      }
    }
  }
}

// Dst splits of the match grid: whole 128-column tiles, at most kMMaxSplits splits.
int match_tiles_per_split(int n_dst) {
  const int n_dt = (n_dst + kMTile - 1) / kMTile;
  return (n_dt + kMMaxSplits - 1) / kMMaxSplits;
}
int match_splits(int n_dst) {
  const int n_dt = (n_dst + kMTile - 1) / kMTile;
  const int per = match_tiles_per_split(n_dst);
  return std::max(1, (n_dt + per - 1) / per);
}

// ---------------------------------------------------------------------------------------
// Map construction kernels (one thread per element).
struct MapArgs {
  sa_tome_maps m;
  const float* part_max;
  const int32_t* part_idx;
  int splits;
};

// Combine dst splits in ascending order (ties keep the lower split = lower dst) and zero
// the dst counters of the later passes.
__global__ void combine_kernel(MapArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const sa_tome_maps& m = a.m;
  if (i < (int64_t)m.G * m.n_src) {
    const int64_t g = i / m.n_src, s = i - g * m.n_src;
    float bv = -INFINITY;
    int bi = 0;
    for (int k = 0; k < a.splits; ++k) {
      const int64_t o = (g * a.splits + k) * m.n_src + s;
      if (better(a.part_max[o], a.part_idx[o], bv, bi)) {
        bv = a.part_max[o];
        bi = a.part_idx[o];
      }
    }
    m.node_max[i] = bv;
    m.node_idx[i] = bi;
  }
  if (i < (int64_t)m.G * m.n_dst) {
    m.dst_cnt[i] = 0;
    m.dst_cursor[i] = 0;
  }
}

// rank[s] = #{s' : node_max[s'] ranks before node_max[s]} (descending value, then position).
// Composite keys (order_bits << 32 | ~position) are distinct and larger exactly when earlier
// in that order; keys of positions past n_src are 0, below every real key. The keys of each
// group are cut into tiles of kRankTile, each sorted descending by one wave
// (rank_sort_kernel); a key's rank is then the sum over the tiles of the number of larger
// keys, a binary search in each sorted tile (rank_kernel).
constexpr int kRankE = kRankTile / 64;   // keys per lane of a tile sort
constexpr int kRankChunkTiles = 32;       // sorted tiles staged in LDS at once (64 KB)

__device__ inline uint64_t rank_key(const float* nm, int j, int n) {
  return j < n ? ((uint64_t)order_bits(nm[j]) << 32) | (uint32_t)~j : 0ull;
}

__global__ __launch_bounds__(64) void rank_sort_kernel(sa_tome_maps m, uint64_t* sorted) {
  const int lane = threadIdx.x, t = blockIdx.x, g = blockIdx.y;
  const float* nm = m.node_max + (int64_t)g * m.n_src;
  uint64_t key[kRankE];
#pragma unroll
  for (int e = 0; e < kRankE; ++e) key[e] = rank_key(nm, t * kRankTile + 64 * e + lane, m.n_src);
  sa_wave_bitonic_desc<kRankE>(key, lane);
  uint64_t* out = sorted + ((int64_t)g * gridDim.x + t) * kRankTile;
#pragma unroll
  for (int e = 0; e < kRankE; ++e) out[64 * e + lane] = key[e];
}

// The keys above `mine` form a prefix of a descending tile; its length by binary search.
__device__ inline int rank_prefix(const uint64_t* tile, uint64_t mine) {
  int p = 0;
#pragma unroll
  for (int step = kRankTile / 2; step > 0; step >>= 1)
    if (tile[p + step - 1] > mine) p += step;
  return p == kRankTile - 1 && tile[kRankTile - 1] > mine ? kRankTile : p;
}

__global__ __launch_bounds__(256) void rank_kernel(sa_tome_maps m, const uint64_t* sorted, int n_tiles) {
  __shared__ __attribute__((aligned(16))) uint64_t keys[kRankChunkTiles * kRankTile];
  const int g = blockIdx.y;
  const int s = blockIdx.x * 256 + threadIdx.x;
  const uint64_t mine = rank_key(m.node_max + (int64_t)g * m.n_src, s, m.n_src);
  const uint64_t* src = sorted + (int64_t)g * n_tiles * kRankTile;
  int count = 0;
  for (int t0 = 0; t0 < n_tiles; t0 += kRankChunkTiles) {
    const int nt = min(kRankChunkTiles, n_tiles - t0);
    __syncthreads();
    // Tiles past n_tiles are staged as 0 keys (they count nothing), so the searches below
    // need no guard: one independent search per staged tile, their LDS reads overlapping.
    {
      // kPer 16-byte loads (two keys each) per thread, all in flight before the stores.
      constexpr int kPer = kRankChunkTiles * kRankTile / 2 / 256;  // key pairs per thread
      const uint4* src4 = reinterpret_cast<const uint4*>(src + (int64_t)t0 * kRankTile);
      uint4 w[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int e2 = threadIdx.x + 256 * u;  // key pair e2 = keys 2 e2, 2 e2 + 1
        w[u] = 2 * e2 < nt * kRankTile ? src4[e2] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) reinterpret_cast<uint4*>(keys)[threadIdx.x + 256 * u] = w[u];
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kRankChunkTiles; ++t) count += rank_prefix(keys + t * kRankTile, mine);
  }
  if (s < m.n_src) {
    m.rank[(int64_t)g * m.n_src + s] = count;
    m.edge[(int64_t)g * m.n_src + count] = s;  // the edge order: edge[rank[s]] = s
  }
}


// dst_idx, dst counts, the unmerge map for every token and the source row of every
// merged row (merged_src).
__global__ void assign_kernel(sa_tome_maps m) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)m.G * m.L) return;
  const int64_t g = i / m.L;
  const int t = (int)(i - g * m.L);
  const int T = m.text_len, U = m.n_src - m.r;
  int32_t* rot = m.row_of_token + g * m.L;
  int32_t* msrc = m.merged_src + g * m.Lm;
  if (t < T) {
    rot[t] = t;
    msrc[t] = t;
  } else if (t < T + m.n_src) {  // edge position e = t - T
    const int e = t - T;
    const int s = m.edge[g * m.n_src + e];
    const int tok = T + m.a_idx[s];
    if (e < m.r) {
      const int d = m.node_idx[g * m.n_src + s];
      m.dst_idx[g * m.r + e] = d;
      atomicAdd(&m.dst_cnt[g * m.n_dst + d], 1);
      rot[tok] = T + U + d;
    } else {
      rot[tok] = T + (e - m.r);
      msrc[T + (e - m.r)] = tok;
    }
  } else if (t < T + m.n_src + m.n_dst) {
    const int d = t - T - m.n_src;
    rot[T + m.b_idx[d]] = T + U + d;
    msrc[T + U + d] = T + m.b_idx[d];
  }
}

// Per group: exclusive scan of dst counts -> dst_ptr; key bias of every merged row.
__global__ __launch_bounds__(1024) void scan_kernel(sa_tome_maps m) {
  __shared__ int32_t part[1024];
  const int g = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = m.n_dst;
  const int per = (n + 1023) / 1024;
  const int lo = min(n, tid * per), hi = min(n, lo + per);
  const int32_t* cnt = m.dst_cnt + (int64_t)g * n;
  int sum = 0;
  for (int d = lo; d < hi; ++d) sum += cnt[d];
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {  // inclusive Hillis-Steele scan
    const int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = tid > 0 ? part[tid - 1] : 0;
  int32_t* ptr = m.dst_ptr + (int64_t)g * (n + 1);
  for (int d = lo; d < hi; ++d) {
    ptr[d] = run;
    run += cnt[d];
  }
  if (tid == 1023) ptr[n] = part[1023];
  // Proportional-attention bias log(size) rounded to bf16 (MergeAttention.py:163-167).
  const int T = m.text_len, U = m.n_src - m.r;
  float* kb = m.key_bias + (int64_t)g * m.Lm;
  for (int j = tid; j < m.Lm; j += 1024) {
    const int d = j - T - U;
    kb[j] = d >= 0 ? round_bf16(logf(round_bf16((float)(1 + cnt[d])))) : 0.f;
  }
}

__global__ void fill_kernel(sa_tome_maps m) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)m.G * m.r) return;
  const int64_t g = i / m.r;
  const int e = (int)(i - g * m.r);
  const int d = m.dst_idx[i];
  const int p = atomicAdd(&m.dst_cursor[g * m.n_dst + d], 1);
  m.members[g * m.r + m.dst_ptr[g * (m.n_dst + 1) + d] + p] = e;
}

// Members of each dst in ascending edge order, then the token row of each member
// (member_rows): the merge reads one index per member. One wave per dst: the members are
// distinct edge positions, so each one's place is the number of smaller members, counted
// against the whole segment in 64-member chunks (broadcast with readlane); a segment of more
// than kSortMaxMembers (the ranks of kSortChunks chunks, kept in registers) is insertion-sorted
// by lane 0.
constexpr int kSortChunks = 16;
constexpr int kSortMaxMembers = 64 * kSortChunks;

__global__ __launch_bounds__(256) void sort_kernel(sa_tome_maps m) {
  const int lane = threadIdx.x & 63;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6;  // (group, dst) of this wave
  if (i >= (int64_t)m.G * m.n_dst) return;
  const int64_t g = i / m.n_dst;
  const int d = (int)(i - g * m.n_dst);
  const int32_t* ptr = m.dst_ptr + g * (m.n_dst + 1);
  int32_t* mem = m.members + g * m.r;
  const int lo = __builtin_amdgcn_readfirstlane(ptr[d]), hi = __builtin_amdgcn_readfirstlane(ptr[d + 1]);
  const int n = hi - lo;
  if (n <= 0) return;
  const int32_t* edge = m.edge + g * m.n_src;
  int32_t* rows = m.member_rows + g * m.r;
  if (n > kSortMaxMembers) {
    if (lane == 0) {
      for (int x = lo + 1; x < hi; ++x) {
        const int v = mem[x];
        int y = x - 1;
        while (y >= lo && mem[y] > v) {
          mem[y + 1] = mem[y];
          --y;
        }
        mem[y + 1] = v;
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    for (int x = lo + lane; x < hi; x += 64) rows[x] = m.text_len + m.a_idx[edge[mem[x]]];
    return;
  }
  const int nc = (n + 63) >> 6;  // chunks of the segment (wave-uniform)
  int val[kSortChunks], rank[kSortChunks];
#pragma unroll
  for (int c = 0; c < kSortChunks; ++c) {
    val[c] = c < nc && 64 * c + lane < n ? mem[lo + 64 * c + lane] : INT_MAX;
    rank[c] = 0;
  }
#pragma unroll
  for (int cj = 0; cj < kSortChunks; ++cj) {
    if (cj < nc) {
      const int nj = min(64, n - 64 * cj);
      for (int j = 0; j < nj; ++j) {
        const int u = __builtin_amdgcn_readlane(val[cj], j);
#pragma unroll
        for (int c = 0; c < kSortChunks; ++c)
          if (c < nc) rank[c] += u < val[c];
      }
    }
  }
  // Every member was read into val before any store below (the stores depend on the ranks,
  // which depend on every lane's value).
#pragma unroll
  for (int c = 0; c < kSortChunks; ++c) {
    if (c < nc && 64 * c + lane < n) {
      mem[lo + rank[c]] = val[c];
      rows[lo + rank[c]] = m.text_len + m.a_idx[edge[val[c]]];
    }
  }
}

// ---------------------------------------------------------------------------------------
// Merge: out[b, h, j] = mean of the tokens of merged row j, for up to three tensors that
// share the maps (q, k, v). 8 lanes per row (16 B each). Row j reads merged_src[j]; a dst
// row with merged srcs then reads its member rows from the flat member_rows list, four
// members' loads in flight at a time, and adds them in edge order after the dst token.
constexpr int kMergeMax = 3;

struct MergeArgs {
  sa_tome_maps m;
  const uint16_t* x[kMergeMax];
  int64_t x_sb[kMergeMax], x_sh[kMergeMax], x_sl[kMergeMax];
  uint16_t* out[kMergeMax];
  int64_t o_sb[kMergeMax], o_sh[kMergeMax], o_sl[kMergeMax];
  int B, H, heads_per_group;
};

__device__ inline void add_u4(float* s, uint4 w) {
  s[0] += bf16lo(w.x); s[1] += bf16hi(w.x); s[2] += bf16lo(w.y); s[3] += bf16hi(w.y);
  s[4] += bf16lo(w.z); s[5] += bf16hi(w.z); s[6] += bf16lo(w.w); s[7] += bf16hi(w.w);
}

// Two or three tensors: one merged row per 8 lanes; a dst row's members are loaded only
// once its member range is known, kU at a time (clamped to the last member).
template <int kN>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
  constexpr int kU = 4;  // member loads in flight
  const sa_tome_maps& m = a.m;
  const int c8 = threadIdx.x & 7;
  const int64_t n_rows = (int64_t)a.B * a.H * m.Lm;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
  if (row >= n_rows) return;
  const int64_t bh = row / m.Lm;
  const int j = (int)(row - bh * m.Lm);
  const int64_t g = bh / a.heads_per_group;
  const int d0 = m.text_len + m.n_src - m.r;  // first dst row
  const int src = m.merged_src[g * m.Lm + j];
  int lo = 0, hi = 0;
  if (j >= d0) {
    const int32_t* ptr = m.dst_ptr + g * (m.n_dst + 1) + (j - d0);
    lo = ptr[0];
    hi = ptr[1];
  }
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const uint16_t* xb[kN];
  uint4 w0[kN];
#pragma unroll
  for (int t = 0; t < kN; ++t) {
    xb[t] = a.x[t] + b * a.x_sb[t] + h * a.x_sh[t] + 8 * c8;
    w0[t] = *reinterpret_cast<const uint4*>(xb[t] + (int64_t)src * a.x_sl[t]);
  }
  uint4 res[kN];
  if (lo == hi) {
#pragma unroll
    for (int t = 0; t < kN; ++t) res[t] = w0[t];
  } else {
    float s[kN][8];
#pragma unroll
    for (int t = 0; t < kN; ++t) {
      const uint4 w = w0[t];
      s[t][0] = bf16lo(w.x); s[t][1] = bf16hi(w.x); s[t][2] = bf16lo(w.y); s[t][3] = bf16hi(w.y);
      s[t][4] = bf16lo(w.z); s[t][5] = bf16hi(w.z); s[t][6] = bf16lo(w.w); s[t][7] = bf16hi(w.w);
    }
    const int32_t* mr = m.member_rows + g * m.r;
    for (int p = lo; p < hi; p += kU) {
      int rr[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) rr[u] = mr[min(p + u, hi - 1)];  // clamped: always a member
      uint4 w[kU][kN];
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int t = 0; t < kN; ++t) w[u][t] = *reinterpret_cast<const uint4*>(xb[t] + (int64_t)rr[u] * a.x_sl[t]);
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (p + u < hi) {
#pragma unroll
          for (int t = 0; t < kN; ++t) add_u4(s[t], w[u][t]);
        }
    }
    const float n = (float)(1 + hi - lo);
#pragma unroll
    for (int t = 0; t < kN; ++t) {
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo16 = __float_as_uint(round_bf16(s[t][2 * q] / n)) >> 16;
        const uint32_t hi16 = __float_as_uint(round_bf16(s[t][2 * q + 1] / n)) & 0xffff0000u;
        o[q] = lo16 | hi16;
      }
      res[t] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
#pragma unroll
  for (int t = 0; t < kN; ++t)
    *reinterpret_cast<uint4*>(a.out[t] + b * a.o_sb[t] + h * a.o_sh[t] + (int64_t)j * a.o_sl[t] + 8 * c8) = res[t];
}

// One tensor (the reference closure's merge of a single tensor): one merged row per 8 lanes,
// with the loads in three dependent levels: (1) merged_src[j] and, for a dst row, its member
// range from dst_ptr; (2) the row's own token and its first kU member indices; (3) those
// members' rows, loaded only by the lanes of rows that have them. Members past the first kU
// follow in batches of kU. C4, inputs larger than the last-level cache: 53.8 us, against
// 58.6 us with merge_kernel's member loads (which wait for the member range inside the
// row's branch). With three tensors this form is 2 % slower than merge_kernel.
template <int kN>
__global__ __launch_bounds__(256) void merge_early_kernel(MergeArgs a) {
  constexpr int kU = 4;  // member loads in flight
  const sa_tome_maps& m = a.m;
  const int c8 = threadIdx.x & 7;
  const int64_t n_rows = (int64_t)a.B * a.H * m.Lm;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
  if (row >= n_rows) return;
  const int64_t bh = row / m.Lm;
  const int j = (int)(row - bh * m.Lm);
  const int64_t g = bh / a.heads_per_group;
  const int d0 = m.text_len + m.n_src - m.r;  // first dst row
  const int src = m.merged_src[g * m.Lm + j];
  int lo = 0, hi = 0;
  if (j >= d0) {
    const int32_t* ptr = m.dst_ptr + g * (m.n_dst + 1) + (j - d0);
    lo = ptr[0];
    hi = ptr[1];
  }
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const uint16_t* xb[kN];
  uint4 w0[kN];
#pragma unroll
  for (int t = 0; t < kN; ++t) {
    xb[t] = a.x[t] + b * a.x_sb[t] + h * a.x_sh[t] + 8 * c8;
    w0[t] = *reinterpret_cast<const uint4*>(xb[t] + (int64_t)src * a.x_sl[t]);
  }
  const int32_t* mr = m.member_rows + g * m.r;
  int rr[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) rr[u] = lo + u < hi ? mr[lo + u] : -1;
  uint4 w[kU][kN];
#pragma unroll
  for (int u = 0; u < kU; ++u)
#pragma unroll
    for (int t = 0; t < kN; ++t)
      w[u][t] = rr[u] >= 0 ? *reinterpret_cast<const uint4*>(xb[t] + (int64_t)rr[u] * a.x_sl[t])
                           : make_uint4(0, 0, 0, 0);
  uint4 res[kN];
  if (lo == hi) {
#pragma unroll
    for (int t = 0; t < kN; ++t) res[t] = w0[t];
  } else {
    float s[kN][8];
#pragma unroll
    for (int t = 0; t < kN; ++t) {
      const uint4 x = w0[t];
      s[t][0] = bf16lo(x.x); s[t][1] = bf16hi(x.x); s[t][2] = bf16lo(x.y); s[t][3] = bf16hi(x.y);
      s[t][4] = bf16lo(x.z); s[t][5] = bf16hi(x.z); s[t][6] = bf16lo(x.w); s[t][7] = bf16hi(x.w);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (lo + u < hi) {
#pragma unroll
        for (int t = 0; t < kN; ++t) add_u4(s[t], w[u][t]);
      }
    for (int p = lo + kU; p < hi; p += kU) {  // members in edge order, kU at a time
      int rq[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) rq[u] = mr[min(p + u, hi - 1)];  // clamped: always a member
      uint4 wq[kU][kN];
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int t = 0; t < kN; ++t) wq[u][t] = *reinterpret_cast<const uint4*>(xb[t] + (int64_t)rq[u] * a.x_sl[t]);
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (p + u < hi) {
#pragma unroll
          for (int t = 0; t < kN; ++t) add_u4(s[t], wq[u][t]);
        }
    }
    const float n = (float)(1 + hi - lo);
#pragma unroll
    for (int t = 0; t < kN; ++t) {
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo16 = __float_as_uint(round_bf16(s[t][2 * q] / n)) >> 16;
        const uint32_t hi16 = __float_as_uint(round_bf16(s[t][2 * q + 1] / n)) & 0xffff0000u;
        o[q] = lo16 | hi16;
      }
      res[t] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
#pragma unroll
  for (int t = 0; t < kN; ++t)
    *reinterpret_cast<uint4*>(a.out[t] + b * a.o_sb[t] + h * a.o_sh[t] + (int64_t)j * a.o_sl[t] + 8 * c8) = res[t];
}

// Unmerge: out[b, h, t] = xm[b, h, row_of_token[t]].
__global__ __launch_bounds__(256) void unmerge_kernel(MergeArgs a) {
  const sa_tome_maps& m = a.m;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
  const int c8 = threadIdx.x & 7;
  if (row >= (int64_t)a.B * a.H * m.L) return;
  const int64_t bh = row / m.L;
  const int t = (int)(row - bh * m.L);
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t g = bh / a.heads_per_group;
  const int src_row = m.row_of_token[g * m.L + t];
  const uint4 w =
      *reinterpret_cast<const uint4*>(a.x[0] + b * a.x_sb[0] + h * a.x_sh[0] + (int64_t)src_row * a.x_sl[0] + 8 * c8);
  *reinterpret_cast<uint4*>(a.out[0] + b * a.o_sb[0] + h * a.o_sh[0] + (int64_t)t * a.o_sl[0] + 8 * c8) = w;
}

int check_maps(const sa_tome_maps* m, const char* fn) {
  SA_REQUIRE(m, "%s: null maps", fn);
  SA_REQUIRE(m->G > 0 && m->N > 0 && m->text_len >= 0 && m->n_src >= 0 && m->n_dst > 0 &&
                 m->n_src + m->n_dst == m->N && m->r >= 0 && m->r <= m->n_src && m->L == m->text_len + m->N &&
                 m->Lm == m->L - m->r,
             "%s: inconsistent map sizes", fn);
  SA_REQUIRE(m->a_idx && m->b_idx && m->node_idx && m->node_max && m->rank && m->edge && m->dst_cnt &&
                 m->dst_cursor && m->dst_ptr && m->row_of_token && m->key_bias && m->merged_src &&
                 (m->r == 0 || (m->dst_idx && m->members && m->member_rows)),
             "%s: null map buffer", fn);
  return SA_OK;
}

inline unsigned grid256(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

extern "C" int sa_tome_partition(int T, int Hp, int Wp, int sx, int sy, int st, const int32_t* cell_choice,
                                 int32_t* a_idx, int32_t* b_idx, int* n_src, int* n_dst) {
  SA_REQUIRE(n_src && n_dst, "sa_tome_partition: null count pointers");
  SA_REQUIRE(T >= 1 && Hp > 0 && Wp > 0 && sx > 0 && sy > 0 && st > 0, "sa_tome_partition: bad geometry");
  const int frame = Hp * Wp;
  const int t1 = T - 1;  // frames after the first
  const int hs = Hp / sy, ws = Wp / sx, ts = t1 / st;
  const int cell = st * sy * sx;
  // buffer over frames 1..T-1: 1 = dst, 0 = src (merge_unmerge.py:71-79).
  std::vector<uint8_t> is_dst((size_t)t1 * frame, 0);
  for (int ct = 0; ct < ts; ++ct)
    for (int ch = 0; ch < hs; ++ch)
      for (int cw = 0; cw < ws; ++cw) {
        const int idx = cell_choice ? cell_choice[((int64_t)ct * hs + ch) * ws + cw] : 0;
        SA_REQUIRE(idx >= 0 && idx < cell, "sa_tome_partition: cell_choice %d outside [0, %d)", idx, cell);
        const int dt = idx / (sy * sx), dy = (idx / sx) % sy, dx = idx % sx;
        is_dst[((size_t)(ct * st + dt) * Hp + (ch * sy + dy)) * Wp + (cw * sx + dx)] = 1;
      }
  int nd = frame, ns = 0;
  for (size_t i = 0; i < is_dst.size(); ++i) (is_dst[i] ? nd : ns) += 1;
  *n_src = ns;
  *n_dst = nd;
  if (!a_idx && !b_idx) return sa::ok();
  SA_REQUIRE(a_idx && b_idx, "sa_tome_partition: need both a_idx and b_idx");
  int pb = 0, pa = 0;
  for (int t = 0; t < frame; ++t) b_idx[pb++] = t;  // first frame: all dst (:83, :91)
  for (size_t i = 0; i < is_dst.size(); ++i)          // stable dst|src split (:82)
    if (is_dst[i]) b_idx[pb++] = frame + (int)i;
  for (size_t i = 0; i < is_dst.size(); ++i)
    if (!is_dst[i]) a_idx[pa++] = frame + (int)i;
  return sa::ok();
}

extern "C" int sa_tome_metric(const uint16_t* k, const int64_t k_strides[3], const uint16_t* v,
                              const int64_t v_strides[3], int B, int H, int L, int D, int text_len, int mode,
                              float* metric, void* stream) {
  SA_REQUIRE(k && k_strides && metric, "sa_tome_metric: null pointer");
  SA_REQUIRE(mode == 0 || mode == 1, "sa_tome_metric: mode must be 0 (head-sum k) or 1 (per-head k,|k|,v,|v|)");
  SA_REQUIRE(mode == 0 || (v && v_strides), "sa_tome_metric: mode 1 needs v");
  SA_REQUIRE(B > 0 && H > 0 && L > text_len && text_len >= 0, "sa_tome_metric: bad shape");
  if (D != kD) return sa::fail(SA_ERR_UNSUPPORTED, "sa_tome_metric: head_dim %d (only 64)", D);
  const uint16_t* ps[2] = {k, v};
  const int64_t* ss[2] = {k_strides, v_strides};
  for (int t = 0; t < (mode == 1 ? 2 : 1); ++t) {
    if (reinterpret_cast<uintptr_t>(ps[t]) % 16) return sa::fail(SA_ERR_UNSUPPORTED, "sa_tome_metric: base not 16-byte aligned");
    for (int i = 0; i < 3; ++i)
      if (ss[t][i] % 8) return sa::fail(SA_ERR_UNSUPPORTED, "sa_tome_metric: strides must be multiples of 8");
  }
  MetricArgs a;
  a.k = k; a.v = v;
  a.k_sb = k_strides[0]; a.k_sh = k_strides[1]; a.k_sl = k_strides[2];
  a.v_sb = v ? v_strides[0] : 0; a.v_sh = v ? v_strides[1] : 0; a.v_sl = v ? v_strides[2] : 0;
  a.B = B; a.H = H; a.N = L - text_len; a.text_len = text_len; a.mode = mode; a.out = metric;
  const int64_t rows = mode == 0 ? (int64_t)B * a.N : (int64_t)B * H * a.N;
  if (mode == 0)
    hipLaunchKernelGGL(metric_sum_kernel, dim3(grid256(rows * 8)), dim3(256), 0, sa::as_stream(stream), a);
  else
    hipLaunchKernelGGL(metric_kernel, dim3(grid256(rows)), dim3(256), 0, sa::as_stream(stream), a);
  return sa::check_launch("sa_tome_metric");
}

extern "C" int sa_tome_normalize(const float* metric, int64_t rows, int C, float* out, void* stream) {
  SA_REQUIRE(metric && out && rows > 0 && C > 0, "sa_tome_normalize: bad arguments");
  hipLaunchKernelGGL(normalize_kernel, dim3(grid256(rows)), dim3(256), 0, sa::as_stream(stream), metric, rows, C, out);
  return sa::check_launch("sa_tome_normalize");
}

namespace {
// Matching and map construction with the split partials (G * splits * max(n_src, 1) floats
// of maxima, then as many int32 positions) at `partials`: every entry the combine step reads
// is written by match_kernel first, so the buffer needs no clearing.
int tome_match_impl(const float* metric, int C, const sa_tome_maps& m, void* partials, hipStream_t s,
                    const char* fn) {
  int rc;
  const int splits = match_splits(m.n_dst);
  float* part_max = reinterpret_cast<float*>(partials);
  int32_t* part_idx = reinterpret_cast<int32_t*>(part_max + (int64_t)m.G * splits * std::max(m.n_src, 1));
  if (m.n_src > 0) {
    MatchArgs a;
    a.metric = metric; a.G = m.G; a.N = m.N; a.C = C; a.a_idx = m.a_idx; a.b_idx = m.b_idx;
    a.n_src = m.n_src; a.n_dst = m.n_dst; a.splits = splits;
    a.dst_per_split = match_tiles_per_split(m.n_dst) * kMTile;
    a.part_max = part_max; a.part_idx = part_idx;
    // match_mfma_kernel stages dst rows with 16-byte loads; a metric base that is not 16-byte
    // aligned takes match_kernel (scalar metric loads, the same fixed-order sums and maps).
    if (C == kMfC && reinterpret_cast<uintptr_t>(metric) % 16 == 0)
      hipLaunchKernelGGL(match_mfma_kernel, dim3((m.n_src + kMfSrc - 1) / kMfSrc, m.G, splits), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(match_kernel, dim3((m.n_src + kMTile - 1) / kMTile, m.G, splits), dim3(256), 0, s, a);
    if ((rc = sa::check_launch(fn))) return rc;
  }
  MapArgs ma;
  ma.m = m; ma.part_max = part_max; ma.part_idx = part_idx; ma.splits = splits;
  const int64_t n0 = (int64_t)m.G * std::max(m.n_src, m.n_dst);
  hipLaunchKernelGGL(combine_kernel, dim3(grid256(n0)), dim3(256), 0, s, ma);
  if (m.n_src > 0) {
    // The sorted tiles reuse the workspace: the split partials are dead after combine_kernel.
    const int n_tiles = (m.n_src + kRankTile - 1) / kRankTile;
    uint64_t* sorted = reinterpret_cast<uint64_t*>(partials);
    hipLaunchKernelGGL(rank_sort_kernel, dim3(n_tiles, m.G), dim3(64), 0, s, m, sorted);
    hipLaunchKernelGGL(rank_kernel, dim3((m.n_src + 255) / 256, m.G), dim3(256), 0, s, m, sorted, n_tiles);
  }
  hipLaunchKernelGGL(assign_kernel, dim3(grid256((int64_t)m.G * m.L)), dim3(256), 0, s, m);
  hipLaunchKernelGGL(scan_kernel, dim3(m.G), dim3(1024), 0, s, m);
  if (m.r > 0) {
    hipLaunchKernelGGL(fill_kernel, dim3(grid256((int64_t)m.G * m.r)), dim3(256), 0, s, m);
    hipLaunchKernelGGL(sort_kernel, dim3(grid256((int64_t)m.G * m.n_dst * 64)), dim3(256), 0, s, m);  // a wave per dst
  }
  return sa::check_launch(fn);
}

// The workspace holds the split partials of the match (8 bytes per group, split and src),
// then the rank's sorted key tiles (8 bytes per group and padded src).
int64_t match_partial_bytes(int G, int n_src, int n_dst) {
  const int64_t partials = (int64_t)G * match_splits(n_dst) * std::max(n_src, 1) * 8;
  const int64_t tiles = (int64_t)G * ((n_src + kRankTile - 1) / kRankTile) * kRankTile * 8;
  return std::max(partials, tiles);
}

// ---- allocation-free matching ---------------------------------------------------------
// The split partials of sa_tome_match_noalloc live in this file-scope device array (one copy
// per GPU, held for the life of the process). Host code never passes `scratch` itself to a
// kernel: the name is a host-side stand-in; its device address on the current GPU comes from
// hipGetSymbolAddress on that GPU's first call and is kept per device.
constexpr int64_t kNoAllocScratchBytes = 16ll << 20;
static __device__ __attribute__((aligned(256))) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices];

int scratch_address(void** out, const char* fn) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return sa::fail(SA_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return sa::fail(SA_ERR_UNSUPPORTED, "%s: device %d >= %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return sa::fail(SA_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return SA_OK;
}
}  // namespace

extern "C" int sa_tome_match_workspace(int G, int n_src, int n_dst, int64_t* bytes) {
  SA_REQUIRE(bytes && G > 0 && n_src >= 0 && n_dst > 0, "sa_tome_match_workspace: bad arguments");
  *bytes = match_partial_bytes(G, n_src, n_dst);
  return sa::ok();
}

extern "C" int sa_tome_match(const float* metric, int C, sa_tome_maps* maps, void* workspace, int64_t ws_bytes,
                             void* stream) {
  int rc = check_maps(maps, "sa_tome_match");
  if (rc) return rc;
  SA_REQUIRE(metric && workspace, "sa_tome_match: null metric/workspace");
  SA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "sa_tome_match: workspace not 16-byte aligned");
  SA_REQUIRE(C > 0 && C <= kMaxC, "sa_tome_match: C=%d outside [1, %d]", C, kMaxC);
  const sa_tome_maps& m = *maps;
  const int64_t need = match_partial_bytes(m.G, m.n_src, m.n_dst);
  SA_REQUIRE(ws_bytes >= need, "sa_tome_match: workspace %lld < %lld bytes", (long long)ws_bytes, (long long)need);
  return tome_match_impl(metric, C, m, workspace, sa::as_stream(stream), "sa_tome_match");
}

extern "C" int sa_tome_match_noalloc(const float* metric, int C, sa_tome_maps* maps, void* stream) {
  const char* fn = "sa_tome_match_noalloc";
  int rc = check_maps(maps, fn);
  if (rc) return rc;
  SA_REQUIRE(metric, "%s: null metric", fn);
  SA_REQUIRE(C > 0 && C <= kMaxC, "%s: C=%d outside [1, %d]", fn, C, kMaxC);
  const sa_tome_maps& m = *maps;
  const int64_t need = match_partial_bytes(m.G, m.n_src, m.n_dst);
  SA_REQUIRE(need <= kNoAllocScratchBytes,
             "%s: G=%d, n_src=%d, n_dst=%d need %lld bytes of partials, above the %lld-byte device scratch "
             "(use sa_tome_match with a workspace)",
             fn, m.G, m.n_src, m.n_dst, (long long)need, (long long)kNoAllocScratchBytes);
  void* partials = nullptr;
  if ((rc = scratch_address(&partials, fn))) return rc;
  return tome_match_impl(metric, C, m, partials, sa::as_stream(stream), fn);
}

namespace {
int launch_merge(bool unmerge, int n, const uint16_t* const* x, const int64_t* xs, int B, int H, int D,
                 int heads_per_group, const sa_tome_maps* maps, uint16_t* const* out, const int64_t* os,
                 void* stream, const char* fn) {
  int rc = check_maps(maps, fn);
  if (rc) return rc;
  SA_REQUIRE(n >= 1 && n <= (unmerge ? 1 : kMergeMax), "%s: %d tensors (1..%d)", fn, n, unmerge ? 1 : kMergeMax);
  SA_REQUIRE(x && xs && out && os, "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && heads_per_group > 0 && H % heads_per_group == 0, "%s: bad B/H/heads_per_group", fn);
  SA_REQUIRE((int64_t)B * H / heads_per_group == maps->G, "%s: B*H/heads_per_group != maps->G", fn);
  if (D != kD) return sa::fail(SA_ERR_UNSUPPORTED, "%s: head_dim %d (only 64)", fn, D);
  MergeArgs a;
  a.m = *maps;
  for (int t = 0; t < n; ++t) {
    SA_REQUIRE(x[t] && out[t], "%s: null tensor %d", fn, t);
    if (reinterpret_cast<uintptr_t>(x[t]) % 16 || reinterpret_cast<uintptr_t>(out[t]) % 16)
      return sa::fail(SA_ERR_UNSUPPORTED, "%s: base not 16-byte aligned", fn);
    for (int i = 0; i < 3; ++i)
      if (xs[3 * t + i] % 8 || os[3 * t + i] % 8)
        return sa::fail(SA_ERR_UNSUPPORTED, "%s: strides must be multiples of 8", fn);
    a.x[t] = x[t]; a.x_sb[t] = xs[3 * t]; a.x_sh[t] = xs[3 * t + 1]; a.x_sl[t] = xs[3 * t + 2];
    a.out[t] = out[t]; a.o_sb[t] = os[3 * t]; a.o_sh[t] = os[3 * t + 1]; a.o_sl[t] = os[3 * t + 2];
  }
  a.B = B; a.H = H; a.heads_per_group = heads_per_group;
  const int64_t rows = (int64_t)B * H * (unmerge ? maps->L : maps->Lm);
  SA_REQUIRE(rows * 8 / 256 < (1LL << 31), "%s: grid too large", fn);
  hipStream_t s = sa::as_stream(stream);
  const dim3 grid(grid256(rows * 8)), blk(256);
  // 8 lanes per merged row, 32 rows per workgroup
  if (unmerge) hipLaunchKernelGGL(unmerge_kernel, grid, blk, 0, s, a);
  else if (n == 1) hipLaunchKernelGGL(merge_early_kernel<1>, grid, blk, 0, s, a);
  else if (n == 2) hipLaunchKernelGGL(merge_kernel<2>, grid, blk, 0, s, a);
  else hipLaunchKernelGGL(merge_kernel<3>, grid, blk, 0, s, a);
  return sa::check_launch(fn);
}
}  // namespace

extern "C" int sa_tome_merge(const uint16_t* x, const int64_t x_strides[3], int B, int H, int D, int heads_per_group,
                             const sa_tome_maps* maps, uint16_t* out, const int64_t out_strides[3], void* stream) {
  SA_REQUIRE(x_strides && out_strides, "sa_tome_merge: null strides");
  return launch_merge(false, 1, &x, x_strides, B, H, D, heads_per_group, maps, &out, out_strides, stream,
                      "sa_tome_merge");
}

extern "C" int sa_tome_merge_multi(int n, const uint16_t* const* x, const int64_t* x_strides, int B, int H, int D,
                                   int heads_per_group, const sa_tome_maps* maps, uint16_t* const* out,
                                   const int64_t* out_strides, void* stream) {
  return launch_merge(false, n, x, x_strides, B, H, D, heads_per_group, maps, out, out_strides, stream,
                      "sa_tome_merge_multi");
}

extern "C" int sa_tome_unmerge(const uint16_t* xm, const int64_t xm_strides[3], int B, int H, int D,
                               int heads_per_group, const sa_tome_maps* maps, uint16_t* out,
                               const int64_t out_strides[3], void* stream) {
  SA_REQUIRE(xm_strides && out_strides, "sa_tome_unmerge: null strides");
  return launch_merge(true, 1, &xm, xm_strides, B, H, D, heads_per_group, maps, &out, out_strides, stream,
                      "sa_tome_unmerge");
}

// ---------------------------------------------------------------------------------------
// Token permutation gathers: out[b, h, j] = x[b, h, idx[j]] (the sliding-tile layout of
// SildingTileAttention.py:111-143 and the 1.5-5B rearranger of combined_attn.py:17-41).
namespace {
__global__ __launch_bounds__(256) void gather_tokens_kernel(const uint16_t* x, int64_t x_sb, int64_t x_sh,
                                                            int64_t x_sl, int L_in, const int32_t* idx, int L_out,
                                                            int H, int64_t rows, uint16_t* out, int64_t o_sb,
                                                            int64_t o_sh, int64_t o_sl, int nchunk) {
  // Eight lanes per row, each moving 16-byte chunks c8, c8 + 8, ... of the row's nchunk.
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
  if (row >= rows) return;
  const int c8 = threadIdx.x & 7;
  const int64_t bh = row / L_out;
  const int j = (int)(row - bh * L_out);
  const int64_t b = bh / H, h = bh - b * H;
  const int src = idx[j];
  const bool valid = (unsigned)src < (unsigned)L_in;  // outside [0, L_in): a zero row (padding)
  const uint16_t* xr = x + b * x_sb + h * x_sh + (int64_t)(valid ? src : 0) * x_sl;
  uint16_t* orow = out + b * o_sb + h * o_sh + (int64_t)j * o_sl;
  for (int c = c8; c < nchunk; c += 8) {
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (valid) w = *reinterpret_cast<const uint4*>(xr + 8 * c);
    *reinterpret_cast<uint4*>(orow + 8 * c) = w;
  }
}
}  // namespace

extern "C" int sa_gather_tokens(const uint16_t* x, const int64_t x_strides[3], int B, int H, int L_in, int D,
                                const int32_t* idx, int L_out, uint16_t* out, const int64_t out_strides[3],
                                void* stream) {
  SA_REQUIRE(x && x_strides && idx && out && out_strides, "sa_gather_tokens: null pointer");
  SA_REQUIRE(B > 0 && H > 0 && L_in > 0 && L_out > 0, "sa_gather_tokens: bad shape");
  if (D <= 0 || D % 8) return sa::fail(SA_ERR_UNSUPPORTED, "sa_gather_tokens: head_dim %d (a multiple of 8)", D);
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return sa::fail(SA_ERR_UNSUPPORTED, "sa_gather_tokens: base not 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    if (x_strides[i] % 8 || out_strides[i] % 8) return sa::fail(SA_ERR_UNSUPPORTED, "sa_gather_tokens: strides must be multiples of 8");
  const int64_t rows = (int64_t)B * H * L_out;
  hipLaunchKernelGGL(gather_tokens_kernel, dim3(grid256(rows * 8)), dim3(256), 0, sa::as_stream(stream), x,
                     x_strides[0], x_strides[1], x_strides[2], L_in, idx, L_out, H, rows, out, out_strides[0],
                     out_strides[1], out_strides[2], D / 8);
  return sa::check_launch("sa_gather_tokens");
}
