// Block-mask construction for gfx950: mean-pooled Q/K block scores, per-row top-k, union
// with text rows/columns and an optional static local window, compaction to kv lists.
//
// Replaces the reference's mask builders that feed the block-sparse kernel:
//   get_sparse_attn_mask_from_topk (utils/block_sparse_attn_kernel.py:31-39): torch.topk
//     over block scores + scatter into a dense bool mask;
//   transfer_attn_to_mask (SparseGen_Plus.py:12-84): sort/scatter per row, then text rows and
//     columns forced dense (:81-82);
//   calc_attn_block_sum_efficient (utils/mask_related.py:40-81): block scores, here from
//     deterministic block means instead of 8 random samples per block.
//
// Bit-exactness contract (this translation unit is built with -ffp-contract=off):
//   pooled[d] = (sum_{t in block, ascending} x[t][d]) / n_t      fp32 adds, IEEE division
//   score     = fmaf chain over d = 0..D-1 ascending, starting from 0
//   order     = score descending, then key-block index ascending (total order on fp32 bit
//               patterns: -0 < +0, NaNs at the ends by sign)
// The CPU oracle (oracle/sa_oracle.c) computes the same sequence of IEEE operations.
#include "sa_common.h"

namespace {

constexpr int kPoolD = 64;        // head dim handled by the pooling kernel
constexpr int kRowsPerWG = 24;    // score rows per top-k workgroup
constexpr int kTopkR = 3;         // score rows per top-k wave (8 waves per workgroup)
constexpr int kColChunk = 64;     // key blocks staged in LDS per step
constexpr int kKpStride = 68;     // LDS stride (floats) of a staged pooled-K row (float4, conflict-free)
static_assert(kColChunk == 64, "topk_kernel maps chunk e to the wave's key column 64e + lane");

// ---------------------------------------------------------------------------------------
// Pooling (blockIdx.y selects the tensor, q or k). Block size 64: pool64_kernel. Other block
// sizes: pool_kernel, wave = 8 blocks; lane = (block lane>>3, dims 8*(lane&7)..+7); each
// lane sums its block's tokens sequentially with 16-byte loads.
struct PoolArgs {
  const uint16_t* x[2];
  int64_t sb[2], sh[2], sl[2];
  float* out[2];
  int H, L, block, nb;
  int64_t total_blocks;  // B*H*nb
  // With k16 (block 64, sa_block_pool_k16): the k pass also writes the fp16-score workspace of
  // the attention, k16 = fp16(k) [B*H][L][64] and k16_norm2[block] = the block's largest
  // squared row norm (fp32 bits), as sa_block_sparse_fwd_k16_prepare computes them.
  uint16_t* k16;
  uint32_t* k16_norm2;
};

typedef _Float16 sa_f16x2 __attribute__((ext_vector_type(2)));

__device__ inline float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__global__ __launch_bounds__(256) void pool_kernel(PoolArgs a) {
  const int t = blockIdx.y;
  const int64_t gblk = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
  if (gblk >= a.total_blocks) return;
  const int dg = threadIdx.x & 7;
  const int64_t bh = gblk / a.nb;
  const int blk = (int)(gblk - bh * a.nb);
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int t0 = blk * a.block;
  const int n = min(a.block, a.L - t0);
  const uint16_t* p = a.x[t] + b * a.sb[t] + h * a.sh[t] + (int64_t)t0 * a.sl[t] + 8 * dg;
  const int64_t sl = a.sl[t];
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int i = 0;
  for (; i + 16 <= n; i += 16) {
    uint4 w[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) w[u] = *reinterpret_cast<const uint4*>(p + (int64_t)(i + u) * sl);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      s[0] += bf16lo(w[u].x); s[1] += bf16hi(w[u].x);
      s[2] += bf16lo(w[u].y); s[3] += bf16hi(w[u].y);
      s[4] += bf16lo(w[u].z); s[5] += bf16hi(w[u].z);
      s[6] += bf16lo(w[u].w); s[7] += bf16hi(w[u].w);
    }
  }
  for (; i < n; ++i) {
    const uint4 w = *reinterpret_cast<const uint4*>(p + (int64_t)i * sl);
    s[0] += bf16lo(w.x); s[1] += bf16hi(w.x);
    s[2] += bf16lo(w.y); s[3] += bf16hi(w.y);
    s[4] += bf16lo(w.z); s[5] += bf16hi(w.z);
    s[6] += bf16lo(w.w); s[7] += bf16hi(w.w);
  }
  const float fn = (float)n;
  float4* o = reinterpret_cast<float4*>(a.out[t] + gblk * kPoolD + 8 * dg);
  o[0] = make_float4(s[0] / fn, s[1] / fn, s[2] / fn, s[3] / fn);
  o[1] = make_float4(s[4] / fn, s[5] / fn, s[6] / fn, s[7] / fn);
}

// Block size 64: one wave per block. Its 8 row loads are coalesced (8 lanes per 128-byte
// row, 8 rows per instruction: 1 KB of a contiguous head per instruction, where pool_kernel's
// instructions touch 8 blocks 8 KB apart), staged in the wave's 8 KB of LDS, and read back
// so that lane l sums dim l over the block's rows in ascending order -- the same additions
// in the same order as pool_kernel. C2 (273 MB): 40.8 against 45.0 us.
constexpr int kPoolRowB = 128;  // LDS bytes per staged row
__global__ __launch_bounds__(256) void pool64_kernel(PoolArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[4 * 64 * kPoolRowB];
  const int t = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t g = (int64_t)blockIdx.x * 4 + wave;
  unsigned char* wl = lds + wave * 64 * kPoolRowB;
  int n = 0;  // rows of block g (0: past the last block)
  const uint16_t* p = a.x[t];
  if (g < a.total_blocks) {
    const int64_t bh = g / a.nb;
    const int blk = (int)(g - bh * a.nb);
    const int64_t b = bh / a.H, h = bh - b * a.H;
    n = min(64, a.L - blk * 64);
    p += b * a.sb[t] + h * a.sh[t] + (int64_t)blk * 64 * a.sl[t] + 8 * (lane & 7);
  }
  uint4 w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 8 * j + (lane >> 3);
    w[j] = row < n ? *reinterpret_cast<const uint4*>(p + (int64_t)row * a.sl[t]) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 8 * j + (lane >> 3);
    *reinterpret_cast<uint4*>(wl + row * kPoolRowB + 16 * (lane & 7)) = w[j];
  }
  if (t == 1 && a.k16 && n > 0) {
    // fp16 copy of the block's key rows (round to nearest even) and its largest squared row
    // norm: per row an fmaf chain over the lane's 8 dims, then the row's 8 lanes in a fixed
    // order (the arithmetic of k16_kernel in attn_fwd.hip, so both give the same bits).
    const int64_t bh = g / a.nb;
    const int blk = (int)(g - bh * a.nb);
    uint16_t* dst = a.k16 + (bh * a.L + (int64_t)blk * 64) * kPoolD + 8 * (lane & 7);
    uint32_t mx = 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = 8 * j + (lane >> 3);
      const uint32_t e[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
      uint32_t o[4];
      float nr = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x0 = bf16lo(e[i]), x1 = bf16hi(e[i]);
        nr = fmaf(x1, x1, fmaf(x0, x0, nr));
        const sa_f16x2 h2 = {(_Float16)x0, (_Float16)x1};
        o[i] = __builtin_bit_cast(uint32_t, h2);
      }
      nr += __shfl_xor(nr, 1);
      nr += __shfl_xor(nr, 2);
      nr += __shfl_xor(nr, 4);
      if (row < n) {
        mx = max(mx, __float_as_uint(nr));
        *reinterpret_cast<uint4*>(dst + (int64_t)row * kPoolD) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
    if (lane == 0) a.k16_norm2[g] = mx;
  }
  __syncthreads();
  if (n == 0) return;
  // Lanes 2m and 2m + 1 read the two halves of one dword: 32 distinct banks per read.
  const uint16_t* src = reinterpret_cast<const uint16_t*>(wl) + lane;
  float s = 0.f;
  if (n == 64) {
#pragma unroll
    for (int r = 0; r < 64; ++r) s += __uint_as_float((uint32_t)src[r * (kPoolRowB / 2)] << 16);
  } else {
    for (int r = 0; r < n; ++r) s += __uint_as_float((uint32_t)src[r * (kPoolRowB / 2)] << 16);
  }
  a.out[t][g * kPoolD + lane] = s / (float)n;
}

// ---------------------------------------------------------------------------------------
// Top-k: workgroup = kRowsPerWG score rows of one (b, h); wave w selects rows kR w .. kR w + kR - 1.
struct TopkArgs {
  const float* qp;         // [BH][nqb][D] (null when scores_in is given)
  const float* kp;         // [BH][nkb][D]
  const float* scores_in;  // [BH][nqb][nkb] or null
  int nqb, nkb, D, topk, n_text;
  const uint8_t* local;  // [nqb][nkb] or null
  int32_t* kv_idx;
  int max_cnt;
  int32_t* kv_cnt;
  uint8_t* mask_out;   // [BH][nqb][nkb] or null
  float* scores_out;   // [BH][nqb][nkb] or null
  int row_groups;      // ceil(nqb / kRowsPerWG)
};

__device__ inline uint32_t order_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Selection per row (one wave): the k-th largest 32-bit ordered score T is found by a
// 32-step bitwise search (each step counts keys >= candidate with ballots), then one pass
// in ascending column order keeps every key > T and the lowest-index keys == T until k are
// kept -- exactly the first k columns in (score descending, column ascending) order -- and
// writes the union with text rows/columns and the local window as the ascending kv list.
template <int NCH, int kR>
__global__ __launch_bounds__(64 * kRowsPerWG / kR) void topk_kernel(TopkArgs a) {
  constexpr int kThreads = 64 * kRowsPerWG / kR;  // kR score rows per wave
  __shared__ __attribute__((aligned(16))) float k_lds[kColChunk * kKpStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: rows are wave-uniform
  const int bh = blockIdx.x / a.row_groups;
  const int r0 = (blockIdx.x - bh * a.row_groups) * kRowsPerWG;
  const int64_t row_base = (int64_t)bh * a.nqb;
  const int nch = (a.nkb + 63) >> 6;
  const int k = a.topk < a.nkb ? a.topk : a.nkb;

  // Lane `lane` of wave w holds column 64e + lane of rows kR w + u as ordered keys (0 =
  // unused). The score loop below produces exactly this mapping, so the scores go from
  // the FMA accumulators into the keys without an LDS round trip; the workgroup's LDS is
  // only the staged q rows and one 64-column chunk of pooled K.
  uint32_t key[kR][NCH];
  bool live[kR];
#pragma unroll
  for (int u = 0; u < kR; ++u) live[u] = r0 + wave * kR + u < a.nqb;  // wave-uniform

  if (a.scores_in) {
#pragma unroll
    for (int u = 0; u < kR; ++u) {
      const int64_t row = row_base + r0 + wave * kR + u;
#pragma unroll
      for (int e = 0; e < NCH; ++e) {
        const int c = 64 * e + lane;
        const bool valid = live[u] && e < nch && c < a.nkb;
        float sc = 0.f;
        if (valid) sc = a.scores_in[row * a.nkb + c];
        key[u][e] = valid ? order_bits(sc) : 0u;
        if (a.scores_out && valid) a.scores_out[row * a.nkb + c] = sc;
      }
    }
  } else {
    // 64-column chunks of pooled K staged in LDS as float4; the wave's kR q rows come through
    // scalar loads (wave-uniform rows; rows past nqb read row nqb - 1 and are discarded).
    // score = fmaf chain over d ascending (the same order as the oracle), kR rows per thread.
    const float* kpb = a.kp + (int64_t)bh * a.nkb * kPoolD;
    const int rg = wave * kR;
    const __attribute__((address_space(4))) float* qrow[kR];
#pragma unroll
    for (int u = 0; u < kR; ++u)
      qrow[u] = (const __attribute__((address_space(4))) float*)(a.qp + (row_base + min(r0 + rg + u, a.nqb - 1)) * kPoolD);
    // Chunk e + 1 of pooled K is loaded into registers while chunk e is scored, so only
    // the first chunk's load latency is exposed. Thread t holds float4 t + kThreads j (j < kPer)
    // of a chunk: column (t + kThreads j) / 16, dims 4 ((t + kThreads j) % 16) .. + 3.
    constexpr int kPer = kColChunk * (kPoolD / 4) / kThreads;  // float4 per thread and chunk
    static_assert(kPer * kThreads == kColChunk * (kPoolD / 4), "a chunk is whole float4 per thread");
    float4 pre[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {  // chunk 0
      const int i = tid + kThreads * j;
      pre[j] = i < min(kColChunk, a.nkb) * (kPoolD / 4)
                   ? *reinterpret_cast<const float4*>(kpb + (int64_t)(i >> 4) * kPoolD + 4 * (i & 15))
                   : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int e = 0; e < NCH; ++e) {
#pragma unroll
      for (int u = 0; u < kR; ++u) key[u][e] = 0u;
      if (e < nch) {  // workgroup-uniform, so the barriers below are too
        const int c0 = e * kColChunk;
        __syncthreads();
        const int nc = min(kColChunk, a.nkb - c0);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int i = tid + kThreads * j;
          if (i < nc * (kPoolD / 4)) *reinterpret_cast<float4*>(&k_lds[(i >> 4) * kKpStride + 4 * (i & 15)]) = pre[j];
        }
        __syncthreads();
        if (e + 1 < nch) {  // chunk e + 1 into registers while chunk e is scored
          const int c1 = c0 + kColChunk;
          const int nc1 = min(kColChunk, a.nkb - c1);
#pragma unroll
          for (int j = 0; j < kPer; ++j) {
            const int i = tid + kThreads * j;
            if (i < nc1 * (kPoolD / 4))
              pre[j] = *reinterpret_cast<const float4*>(kpb + (int64_t)(c1 + (i >> 4)) * kPoolD + 4 * (i & 15));
          }
        }
        if (lane < nc) {
          float acc[kR];
#pragma unroll
          for (int u = 0; u < kR; ++u) acc[u] = 0.f;
#pragma unroll 4
          for (int d = 0; d < kPoolD; d += 4) {
            const float4 kv = *reinterpret_cast<const float4*>(&k_lds[lane * kKpStride + d]);
#pragma unroll
            for (int u = 0; u < kR; ++u) {
              const float4 qv = make_float4(qrow[u][d], qrow[u][d + 1], qrow[u][d + 2], qrow[u][d + 3]);
              acc[u] = fmaf(qv.x, kv.x, acc[u]);
              acc[u] = fmaf(qv.y, kv.y, acc[u]);
              acc[u] = fmaf(qv.z, kv.z, acc[u]);
              acc[u] = fmaf(qv.w, kv.w, acc[u]);
            }
          }
#pragma unroll
          for (int u = 0; u < kR; ++u) {
            if (!live[u]) continue;
            key[u][e] = order_bits(acc[u]);
            if (a.scores_out) a.scores_out[(row_base + r0 + rg + u) * a.nkb + c0 + lane] = acc[u];
          }
        }
      }
    }
  }

  // The wave's kR rows are selected together: their 32-step searches are independent chains
  // of ballot -> popcount -> compare, interleaved to hide each other's latency.
  // The search keeps thr = the largest prefix with count(key >= thr) >= k. Once a candidate
  // has exactly k keys at or above it, every later accepted candidate has exactly k as well,
  // and the k-th largest key is the smallest of those k: count(key >= m + 1) < k for that
  // minimum m. So the wave stops when each of its rows has seen an exact count, and every
  // row then takes thr = min{key >= thr} (for a row that ran all 32 steps thr is already a
  // key, and the minimum returns it). On C2 rows this ends the search after ~20 of 32 steps.
  uint32_t thr[kR];  // the k-th largest key (0 when k == 0: nothing selected)
#pragma unroll
  for (int u = 0; u < kR; ++u) thr[u] = 0u;
  if (k > 0) {
    // Bit u set: row u has seen an exact count (rows past nqb never search). Scalar.
    int exact = 0;
#pragma unroll
    for (int u = 0; u < kR; ++u) exact |= live[u] ? 0 : 1 << u;
    for (int bit = 31; bit >= 0 && exact != (1 << kR) - 1; --bit) {
#pragma unroll
      for (int u = 0; u < kR; ++u) {
        const uint32_t cand = thr[u] | (1u << bit);
        int count = 0;
#pragma unroll
        for (int e = 0; e < NCH; ++e) count += __popcll(__ballot(key[u][e] >= cand));
        if (count >= k) thr[u] = cand;
        exact |= count == k ? 1 << u : 0;
      }
    }
#pragma unroll
    for (int u = 0; u < kR; ++u) {
      uint32_t m = 0xffffffffu;
#pragma unroll
      for (int e = 0; e < NCH; ++e) m = key[u][e] >= thr[u] ? min(m, key[u][e]) : m;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) m = min(m, (uint32_t)__shfl_xor((int)m, off));
      thr[u] = m;
    }
  }
#pragma unroll
  for (int u = 0; u < kR; ++u) {
    if (!live[u]) break;  // wave-uniform; later rows are past nqb as well
    const int r = r0 + wave * kR + u;
    const int64_t row = row_base + r;
    int need = 0;  // keys equal to thr to keep, lowest columns first
    if (k > 0) {
      int gt = 0;
#pragma unroll
      for (int e = 0; e < NCH; ++e) gt += __popcll(__ballot(key[u][e] > thr[u]));
      need = k - gt;
    }
    const bool text_row = r < a.n_text;
    const uint8_t* loc = a.local ? a.local + (int64_t)r * a.nkb : nullptr;
    int32_t* out = a.kv_idx + row * a.max_cnt;
    int total = 0;
    int ties = 0;
#pragma unroll
    for (int e = 0; e < NCH; ++e) {
      const int c = 64 * e + lane;
      const bool valid = e < nch && c < a.nkb;
      const bool tie = valid && k > 0 && key[u][e] == thr[u];
      const uint64_t tb = __ballot(tie);
      const int tie_rank = ties + __builtin_amdgcn_mbcnt_hi((uint32_t)(tb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)tb, 0));
      ties += __popcll(tb);
      bool on = false;
      if (valid) {
        const bool sel = k > 0 && (key[u][e] > thr[u] || (tie && tie_rank < need));
        on = sel || text_row || c < a.n_text;
        if (loc) on = on || loc[c] != 0;
        if (a.mask_out) a.mask_out[row * a.nkb + c] = on ? 1 : 0;
      }
      const uint64_t bal = __ballot(on);
      const int pre = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
      if (on && total + pre < a.max_cnt) out[total + pre] = c;
      total += __popcll(bal);
    }
    if (lane == 0) a.kv_cnt[row] = total < a.max_cnt ? total : a.max_cnt;
  }
}

}  // namespace

namespace {
int block_pool(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k, const int64_t k_strides[3], int B,
               int H, int L, int D, int block, float* q_pooled, float* k_pooled, uint16_t* k16, uint32_t* k16_norm2,
               void* stream);
}  // namespace

extern "C" int sa_block_pool(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                             const int64_t k_strides[3], int B, int H, int L, int D, int block,
                             float* q_pooled, float* k_pooled, void* stream) {
  return block_pool(q, q_strides, k, k_strides, B, H, L, D, block, q_pooled, k_pooled, nullptr, nullptr, stream);
}

extern "C" int sa_block_pool_k16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                 const int64_t k_strides[3], int B, int H, int L, int D, float* q_pooled,
                                 float* k_pooled, void* workspace, int64_t workspace_bytes, void* stream) {
  SA_REQUIRE(k && k_strides && k_pooled, "sa_block_pool_k16: null k");
  SA_REQUIRE(B > 0 && H > 0 && L > 0, "sa_block_pool_k16: bad shape B=%d H=%d L=%d", B, H, L);
  SA_REQUIRE(workspace && reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
             "sa_block_pool_k16: workspace null or not 256-byte aligned");
  SA_REQUIRE(workspace_bytes >= sa::k16_ws_bytes(B, H, L), "sa_block_pool_k16: workspace of %lld bytes < %lld",
             (long long)workspace_bytes, (long long)sa::k16_ws_bytes(B, H, L));
  uint16_t* k16 = static_cast<uint16_t*>(workspace);
  uint32_t* norm2 = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + sa::k16_bytes(B, H, L));
  return block_pool(q, q_strides, k, k_strides, B, H, L, D, 64, q_pooled, k_pooled, k16, norm2, stream);
}

namespace {
int block_pool(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k, const int64_t k_strides[3], int B,
               int H, int L, int D, int block, float* q_pooled, float* k_pooled, uint16_t* k16, uint32_t* k16_norm2,
               void* stream) {
  SA_REQUIRE(q && q_strides && q_pooled, "sa_block_pool: null pointer");
  SA_REQUIRE(!k || (k_strides && k_pooled), "sa_block_pool: k given without k_strides/k_pooled");
  SA_REQUIRE(B > 0 && H > 0 && L > 0 && block > 0, "sa_block_pool: bad shape B=%d H=%d L=%d block=%d", B, H, L, block);
  if (D != kPoolD) return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_pool: head_dim %d (only 64)", D);
  const uint16_t* xs[2] = {q, k};
  const int64_t* ss[2] = {q_strides, k_strides};
  for (int t = 0; t < 2; ++t) {
    if (!xs[t]) continue;
    if (reinterpret_cast<uintptr_t>(xs[t]) % 16)
      return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_pool: tensor base not 16-byte aligned");
    for (int i = 0; i < 3; ++i)
      if (ss[t][i] % 8) return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_pool: strides must be multiples of 8");
  }
  PoolArgs a;
  a.k16 = k16;
  a.k16_norm2 = k16_norm2;
  a.H = H; a.L = L; a.block = block; a.nb = sa::cdiv(L, block);
  a.total_blocks = (int64_t)B * H * a.nb;
  const int nt = k ? 2 : 1;
  for (int t = 0; t < 2; ++t) {
    const int s = t < nt ? t : 0;
    a.x[t] = xs[s]; a.sb[t] = ss[s][0]; a.sh[t] = ss[s][1]; a.sl[t] = ss[s][2];
    a.out[t] = s == 0 ? q_pooled : k_pooled;
  }
  if (block == 64) {
    const int64_t grid = (a.total_blocks + 3) / 4;  // one block per wave, 4 waves per workgroup
    SA_REQUIRE(grid < (1LL << 31), "sa_block_pool: grid too large");
    hipLaunchKernelGGL(pool64_kernel, dim3((unsigned)grid, nt), dim3(256), 0, sa::as_stream(stream), a);
    return sa::check_launch("sa_block_pool");
  }
  const int64_t grid = (a.total_blocks * 8 + 255) / 256;
  SA_REQUIRE(grid < (1LL << 31), "sa_block_pool: grid too large");
  hipLaunchKernelGGL(pool_kernel, dim3((unsigned)grid, nt), dim3(256), 0, sa::as_stream(stream), a);
  return sa::check_launch("sa_block_pool");
}
}  // namespace

extern "C" int sa_block_topk_kv_list(const float* q_pooled, const float* k_pooled, const float* scores_in,
                                     int BH, int nqb, int nkb, int D, int topk, int n_text_blocks,
                                     const uint8_t* local_bitmap, int32_t* kv_idx, int max_cnt,
                                     int32_t* kv_cnt, uint8_t* mask_out, float* scores_out, void* stream) {
  SA_REQUIRE(kv_idx && kv_cnt, "sa_block_topk_kv_list: null kv list");
  SA_REQUIRE(scores_in || (q_pooled && k_pooled), "sa_block_topk_kv_list: need scores_in or q/k pooled");
  SA_REQUIRE(BH > 0 && nqb > 0 && nkb > 0, "sa_block_topk_kv_list: bad shape BH=%d nqb=%d nkb=%d", BH, nqb, nkb);
  SA_REQUIRE(topk >= 0 && n_text_blocks >= 0, "sa_block_topk_kv_list: negative topk/n_text_blocks");
  SA_REQUIRE(max_cnt >= nkb, "sa_block_topk_kv_list: max_cnt=%d < nkb=%d", max_cnt, nkb);
  if (!scores_in && D != kPoolD) return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_topk_kv_list: D=%d (only 64)", D);
  if (nkb > 1024) return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_topk_kv_list: nkb=%d > 1024", nkb);
  TopkArgs a;
  a.qp = q_pooled; a.kp = k_pooled; a.scores_in = scores_in;
  a.nqb = nqb; a.nkb = nkb; a.D = D; a.topk = topk; a.n_text = n_text_blocks;
  a.local = local_bitmap; a.kv_idx = kv_idx; a.max_cnt = max_cnt; a.kv_cnt = kv_cnt;
  a.mask_out = mask_out; a.scores_out = scores_out;
  a.row_groups = sa::cdiv(nqb, kRowsPerWG);
  const int64_t grid = (int64_t)BH * a.row_groups;
  SA_REQUIRE(grid < (1LL << 31), "sa_block_topk_kv_list: grid too large");
  hipStream_t s = sa::as_stream(stream);
  if (nkb <= 256) {
    hipLaunchKernelGGL((topk_kernel<4, kTopkR>), dim3((unsigned)grid), dim3(64 * kRowsPerWG / kTopkR), 0, s, a);
  } else if (nkb <= 320) {
    hipLaunchKernelGGL((topk_kernel<5, kTopkR>), dim3((unsigned)grid), dim3(64 * kRowsPerWG / kTopkR), 0, s, a);
  } else if (nkb <= 512) {
    hipLaunchKernelGGL((topk_kernel<8, kTopkR>), dim3((unsigned)grid), dim3(64 * kRowsPerWG / kTopkR), 0, s, a);
  } else {
    hipLaunchKernelGGL((topk_kernel<16, kTopkR>), dim3((unsigned)grid), dim3(64 * kRowsPerWG / kTopkR), 0, s, a);
  }
  return sa::check_launch("sa_block_topk_kv_list");
}
