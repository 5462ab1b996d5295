// The adaptive block-mask source of SparseGen_Plus for gfx950: sampled block scores and the
// energy-threshold (or adaptive top-k) selection per score row.
//
// Replaces, in the reference:
//   random_sample_tokens + pad_to_multiple (utils/mask_related.py:2-37): per 64-token block,
//     the tokens at the `num_keep` largest of 64 uniform draws (torch.topk, sorted), the tail
//     block padded by repeating the last token;
//   calc_attn_block_sum_efficient (utils/mask_related.py:40-81): softmax(sq sk^T / 8) over
//     the sampled tokens, summed over num_keep x num_keep cells (conv2d with a ones kernel);
//   transfer_attn_to_mask (SparseGen_Plus.py:12-84): per row, sort descending, cumulative
//     energy, keep the prefix before the threshold crossing clamped to [min, max] ("energy"),
//     or the adaptive top-k rule ("topk"); text rows and columns forced dense (:81-82).
//
// Three kernels:
//   sample_gather_kernel   one wave per (tensor, b*h, block): ranks the 64 draws, writes the
//                          token ids and copies the sampled rows to a compact bf16 buffer.
//   sampled_pool_kernel    one wave per (b*h, 32 sampled query rows), four waves of one head per
//                          workgroup sharing each LDS-staged key tile: S^T = K Q^T with
//                          v_mfma_f32_32x32x16_bf16 over all sampled keys, twice (row max and
//                          sum, then probabilities), summing each num_keep x num_keep cell.
//   energy_list_kernel     one wave per score row: rank, sorted prefix sums, the kept count,
//                          and the ascending kv list with text rows and columns.
//
// Numerics: the sampled scores are fp32 (the reference rounds the scores, the softmax and the
// pooled sums to bf16). The selection is bit-exact given the scores: ranks use the total order
// (score descending, column ascending) and the prefix sums are sequential fp32 additions in
// rank order; this translation unit is built with -ffp-contract=off.
#include "sa_common.h"

namespace {

constexpr int kD = 64;
constexpr float kLog2eOver8 = 0.18033688011112042f;  // log2(e) / 8: the reference's fixed "/ 8"

typedef unsigned est_u32x4 __attribute__((ext_vector_type(4)));

__device__ inline float from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
__device__ inline uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------------------
struct SampleArgs {
  const float* rand[2];  // [B*H][nb][64] uniform draws
  const uint16_t* x[2];  // [B,H,L,64] bf16, strided
  int64_t sb[2], sh[2], sl[2];
  int32_t* tok[2];       // [B*H][nb*S] token ids (nullable)
  uint16_t* out[2];      // [B*H][ns_pad][64] sampled rows
  int H, L, nb, S, ns_pad;
  int64_t per_tensor;    // B*H*nb waves per tensor
  int64_t total;         // waves in the grid
};

__global__ __launch_bounds__(256) void sample_gather_kernel(SampleArgs a) {
  __shared__ uint32_t key_lds[4][64];
  __shared__ int32_t tok_lds[4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave;
  if (wid >= a.total) return;  // no workgroup barriers below
  const int t = wid >= a.per_tensor ? 1 : 0;
  const int64_t rest = wid - t * a.per_tensor;
  const int64_t bh = rest / a.nb;
  const int blk = (int)(rest - bh * a.nb);
  const uint32_t key = order_key(a.rand[t][rest * 64 + lane]);
  key_lds[wave][lane] = key;
  __builtin_amdgcn_wave_barrier();
  // Rank in (draw descending, position ascending): torch.topk(sorted=True) order.
  int rank = 0;
  for (int j = 0; j < 64; ++j) {
    const uint32_t kj = key_lds[wave][j];
    rank += (kj > key) || (kj == key && j < lane);
  }
  const int S = a.S;
  const int ns = a.nb * S;
  if (rank < S) {
    const int token = min(blk * 64 + lane, a.L - 1);  // the padded tail repeats token L-1
    tok_lds[wave][rank] = token;
    if (a.tok[t]) a.tok[t][bh * ns + (int64_t)blk * S + rank] = token;
  }
  __builtin_amdgcn_wave_barrier();
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const uint16_t* src = a.x[t] + b * a.sb[t] + h * a.sh[t];
  uint16_t* dst = a.out[t] + (bh * a.ns_pad + (int64_t)blk * S) * kD;
  for (int e = lane; e < S * 8; e += 64) {
    const int row = e >> 3, chunk = e & 7;
    const int token = tok_lds[wave][row];
    *reinterpret_cast<uint4*>(dst + row * kD + 8 * chunk) =
        *reinterpret_cast<const uint4*>(src + (int64_t)token * a.sl[t] + 8 * chunk);
  }
}

// ---------------------------------------------------------------------------------------
struct PoolSArgs {
  const uint16_t* sq;  // [BH][ns_pad][64]
  const uint16_t* sk;  // [BH][ns_pad][64]
  float* pooled;       // [BH][nb][nb]
  int nb, ns, ns_pad, ng;
  int wg_per_bh;       // ceil(ng / 4): workgroups per head
};

// Sampled-key tiles in LDS: 32 keys x 8 chunks of 16 bytes, chunk c of key r at slot
// r * 8 + (c ^ ((r >> 1) & 7)). Any 16 consecutive lanes of an operand read (keys 2k, 2k+1
// for 8 k, one chunk) or of a tile store then touch 16 distinct 16-byte bank groups.
__device__ inline int kslot(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }

__device__ inline sa_f32x16 tile_scores(const est_u32x4* kt, int col, int hh, const sa_bf16x8 (&qf)[4]) {
  est_u32x4 kop[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) kop[s] = kt[kslot(col, 2 * s + hh)];
  sa_f32x16 t = {};
#pragma unroll
  for (int s = 0; s < 4; ++s)
    t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(sa_bf16x8, kop[s]), qf[s], t, 0, 0, 0);
  return t;
}

// Workgroup: the 4 query groups 4w .. 4w + 3 of head bh, one per wave; wave v takes sampled
// query rows 32g .. 32g+31 (lane column = query 32g + lane%32), g = 4w + v. C element i of a
// 32-key tile is key 32kt + 8(i/4) + 4(lane/32) + i%4. The four waves read the same keys:
// each 32-key tile is loaded once per workgroup (one coalesced 16-byte load per thread, the
// next tile's in flight while this one is scored) into one of two LDS buffers; one barrier
// per tile orders the store before the reads, and the reads of a buffer before its
// rewrite two tiles later. Waves past ng take part in the loads and barriers only.
template <int S>
__global__ __launch_bounds__(256) void sampled_pool_kernel(PoolSArgs a) {
  __shared__ est_u32x4 kt_lds[2][32 * 8];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t bh = blockIdx.x / a.wg_per_bh;
  const int g = (int)(blockIdx.x - bh * a.wg_per_bh) * 4 + wave;
  const bool active = g < a.ng;  // wave-uniform
  const int col = lane & 31, hh = lane >> 5;
  sa_bf16x8 qf[4];
  {
    const uint16_t* qp = a.sq + (bh * a.ns_pad + 32 * min(g, a.ng - 1) + col) * kD + 8 * hh;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = __builtin_bit_cast(sa_bf16x8, *reinterpret_cast<const est_u32x4*>(qp + 16 * s));
  }
  const int nkt = a.ns_pad / 32;
  // This thread's share of every tile: key r = tid / 8, chunk c = tid % 8.
  const int ld_r = threadIdx.x >> 3, ld_c = threadIdx.x & 7;
  const est_u32x4* ksrc = reinterpret_cast<const est_u32x4*>(a.sk + (bh * a.ns_pad + ld_r) * kD) + ld_c;
  const int ld_slot = kslot(ld_r, ld_c);
  constexpr int kTileU4 = 32 * kD / 8;  // 16-byte units per tile

  // Pass 1: row max and row sum of exp2 (online, per lane over its keys).
  float m = -INFINITY, l = 0.f;
  est_u32x4 pre = ksrc[0];
  for (int kt = 0; kt < nkt; ++kt) {
    kt_lds[kt & 1][ld_slot] = pre;
    __syncthreads();
    if (kt + 1 < nkt) pre = ksrc[(int64_t)(kt + 1) * kTileU4];
    if (!active) continue;
    const sa_f32x16 t = tile_scores(kt_lds[kt & 1], col, hh, qf);
    float x[16];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = 32 * kt + 8 * (i >> 2) + 4 * hh + (i & 3);
      x[i] = key < a.ns ? t[i] * kLog2eOver8 : -INFINITY;
      tmax = fmaxf(tmax, x[i]);
    }
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

  // Pass 2: probabilities, summed per (query block, key block) cell. Its tiles continue pass
  // 1's buffer alternation (step nkt + kt), so every store still goes to the buffer read two
  // steps earlier, which the barrier of the step in between has released.
  constexpr int kBlocks = 32 / S;  // key blocks per 32-key tile
  const int qblk = (32 * g + col) / S;
  const bool writer = active && hh == 0 && (col % S) == 0 && qblk < a.nb;
  float* prow = a.pooled + (bh * a.nb + (writer ? qblk : 0)) * a.nb;
  pre = ksrc[0];
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = (nkt + kt) & 1;
    kt_lds[buf][ld_slot] = pre;
    __syncthreads();
    if (kt + 1 < nkt) pre = ksrc[(int64_t)(kt + 1) * kTileU4];
    if (!active) continue;
    const sa_f32x16 t = tile_scores(kt_lds[buf], col, hh, qf);
    float bs[kBlocks];
#pragma unroll
    for (int j = 0; j < kBlocks; ++j) bs[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = 32 * kt + 8 * (i >> 2) + 4 * hh + (i & 3);
      const float p = key < a.ns ? __builtin_amdgcn_exp2f(t[i] * kLog2eOver8 - m) * inv : 0.f;
      bs[(8 * (i >> 2)) / S] += p;
    }
    // Sum over the S query lanes of the block and the two lane halves (keys 4hh + ...).
#pragma unroll
    for (int j = 0; j < kBlocks; ++j) {
#pragma unroll
      for (int msk = 1; msk < S; msk <<= 1) bs[j] += __shfl_xor(bs[j], msk);
      bs[j] += __shfl_xor(bs[j], 32);
    }
    if (writer) {
#pragma unroll
      for (int j = 0; j < kBlocks; ++j) {
        const int J = kt * kBlocks + j;
        if (J < a.nb) prow[J] = bs[j];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
struct EnergyArgs {
  const float* scores;  // [rows][nkb]
  int64_t rows;
  int nqb, nkb, mode;
  float threshold;
  int min_keep, max_keep, init_k, n_text;
  int32_t* kv_idx;
  int max_cnt;
  int32_t* kv_cnt;
  uint8_t* mask_out;  // [rows][nkb] or null
};

template <int NCH>
__global__ __launch_bounds__(256) void energy_list_kernel(EnergyArgs a) {
  constexpr int NPAD = 64 * NCH;
  // Sort width: the row padded to a power of two; E keys per lane.
  constexpr int NSORT = NCH <= 4 ? 256 : NCH <= 8 ? 512 : 1024;
  constexpr int E = NSORT / 64;
  static_assert(NPAD <= NSORT, "sort width");
  // Rows of more than 320 blocks are sorted (O(n log^2 n)); shorter rows rank every entry
  // against every other (O(n^2), faster there: 0.105 against 0.115 ms at 278 blocks).
  constexpr bool kSort = NCH >= 8;
  __shared__ __attribute__((aligned(16))) uint64_t key_lds[4][kSort ? 2 : NPAD];
  __shared__ float cum_lds[4][NPAD];
  __shared__ uint8_t keep_lds[4][NPAD];  // 1: the column is among the first k of the order
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= a.rows) return;  // no workgroup barriers below
  const int n = a.nkb;
  const float* src = a.scores + row * n;
  // Composite keys (order_key << 32 | ~column): larger = earlier in (score descending,
  // column ascending), and all distinct; entries past n hold 0, below every valid key.
  uint64_t key[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = 64 * e + lane;
    key[e] = (e < NCH && c < n) ? ((uint64_t)order_key(src[c]) << 32) | (uint32_t)~c : 0ull;
    if (e < NCH) keep_lds[wave][c] = 0;
  }
  int rank[NCH];  // rank path: position of this lane's entry e in the order
  if constexpr (kSort) {
    // Bitonic network, descending (sa_wave_bitonic_desc): sorted position p then holds the
    // p-th key, and the key gives back its value and column.
    sa_wave_bitonic_desc<E>(key, lane);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int p = 64 * e + lane;
      if (p < n) cum_lds[wave][p] = from_order_key((uint32_t)(key[e] >> 32));
    }
  } else {
    // Rank = the number of larger keys; the value goes to its sorted slot.
#pragma unroll
    for (int e = 0; e < NCH; ++e) {
      key_lds[wave][64 * e + lane] = key[e];
      rank[e] = 0;
    }
    __builtin_amdgcn_wave_barrier();
    for (int j0 = 0; j0 < n; j0 += 2) {  // two keys per 16-byte broadcast read
      const uint4 k2 = *reinterpret_cast<const uint4*>(&key_lds[wave][j0]);
      const uint64_t kq[2] = {((uint64_t)k2.y << 32) | k2.x, ((uint64_t)k2.w << 32) | k2.z};
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < NCH; ++e) rank[e] += kq[t] > key[e];
    }
#pragma unroll
    for (int e = 0; e < NCH; ++e)
      if (64 * e + lane < n) cum_lds[wave][rank[e]] = from_order_key((uint32_t)(key[e] >> 32));
  }
  __builtin_amdgcn_wave_barrier();
  // Sequential prefix sums in rank order (the fixed order the oracle repeats).
  if (lane == 0) {
    float acc = 0.f;
    for (int j = 0; j < n; ++j) {
      acc += cum_lds[wave][j];
      cum_lds[wave][j] = acc;
    }
  }
  __builtin_amdgcn_wave_barrier();
  const float total = cum_lds[wave][n - 1];
  int k;
  if (a.mode == 0) {
    // "energy": the prefix before the first position whose cumulative energy reaches
    // threshold * total (all n if the total itself stays below it), then [min, max].
    const float target = a.threshold * total;
    int first = n;
#pragma unroll
    for (int e = NCH - 1; e >= 0; --e) {
      const int c = 64 * e + lane;
      const uint64_t hit = __ballot(c < n && cum_lds[wave][c] >= target);
      if (hit) first = 64 * e + __builtin_ctzll(hit);
    }
    k = total < target ? n : first;
    k = min(max(k, a.min_keep), a.max_keep);
  } else if (a.mode == 2 || a.mode == 3) {
    // "inclusive" (2): through the first position whose cumulative energy reaches
    // threshold * total (the last position when none does), then [min, max].
    // "cumulative <=" (3): the positions whose cumulative energy stays <= threshold * total
    // (a prefix: the sums do not decrease), plus the last position (added below).
    const float target = a.threshold * total;
    int first = n;
#pragma unroll
    for (int e = NCH - 1; e >= 0; --e) {
      const int c = 64 * e + lane;
      const float cv = c < n ? cum_lds[wave][c] : 0.f;
      const bool hit_c = c < n && (a.mode == 2 ? cv >= target : !(cv <= target));
      const uint64_t hit = __ballot(hit_c);
      if (hit) first = 64 * e + __builtin_ctzll(hit);
    }
    if (a.mode == 2) {
      k = (first < n ? first : n - 1) + 1;
      k = min(max(k, a.min_keep), a.max_keep);
    } else {
      k = first;
    }
  } else {
    // "topk": start from init_k; below 60 % of the energy triple it, then (below 90 %)
    // take two thirds of the result, both capped at n.
    const int k0 = a.init_k;
    const float cur = cum_lds[wave][k0 - 1];
    const bool met60 = cur >= 0.6f * total;
    const bool met90 = cur >= 0.9f * total;
    k = k0;
    if (!met60 && k0 < n) k = min(k * 3, n);
    if (!met90 && k0 < n) k = min(k / 3 * 2, n);
  }
  // The first k of the order, by column.
  if constexpr (kSort) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int p = 64 * e + lane;
      if (p < n && (p < k || (a.mode == 3 && p == n - 1))) keep_lds[wave][~(uint32_t)key[e]] = 1;
    }
  } else {
#pragma unroll
    for (int e = 0; e < NCH; ++e)
      if (64 * e + lane < n && (rank[e] < k || (a.mode == 3 && rank[e] == n - 1))) keep_lds[wave][64 * e + lane] = 1;
  }
  __builtin_amdgcn_wave_barrier();
  const int r = (int)(row % a.nqb);
  const bool text_row = r < a.n_text;
  int32_t* out = a.kv_idx + row * a.max_cnt;
  int total_on = 0;
#pragma unroll
  for (int e = 0; e < NCH; ++e) {
    const int c = 64 * e + lane;
    const bool valid = c < n;
    const bool on = valid && (keep_lds[wave][c] != 0 || text_row || c < a.n_text);
    if (a.mask_out && valid) a.mask_out[row * n + c] = on ? 1 : 0;
    const uint64_t bal = __ballot(on);
    const int pre = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
    if (on && total_on + pre < a.max_cnt) out[total_on + pre] = c;
    total_on += __popcll(bal);
  }
  if (lane == 0) a.kv_cnt[row] = total_on < a.max_cnt ? total_on : a.max_cnt;
}

}  // namespace

extern "C" int sa_sample_block_tokens(const float* rand_q, const uint16_t* q, const int64_t q_strides[3],
                                      const float* rand_k, const uint16_t* k, const int64_t k_strides[3],
                                      int B, int H, int L, int D, int num_keep, int32_t* tok_q, int32_t* tok_k,
                                      uint16_t* q_sampled, uint16_t* k_sampled, int ns_pad, void* stream) {
  SA_REQUIRE(rand_q && q && q_strides && q_sampled, "sa_sample_block_tokens: null pointer");
  SA_REQUIRE(!k || (rand_k && k_strides && k_sampled), "sa_sample_block_tokens: k given without rand_k/k_strides/k_sampled");
  SA_REQUIRE(B > 0 && H > 0 && L > 0, "sa_sample_block_tokens: bad shape B=%d H=%d L=%d", B, H, L);
  SA_REQUIRE(num_keep >= 1 && num_keep <= 64, "sa_sample_block_tokens: num_keep=%d outside [1, 64]", num_keep);
  if (D != kD) return sa::fail(SA_ERR_UNSUPPORTED, "sa_sample_block_tokens: head_dim %d (only 64)", D);
  const int nb = sa::cdiv(L, 64);
  SA_REQUIRE(ns_pad >= nb * num_keep, "sa_sample_block_tokens: ns_pad=%d < nb*num_keep=%d", ns_pad, nb * num_keep);
  const uint16_t* xs[2] = {q, k};
  const int64_t* ss[2] = {q_strides, k_strides};
  for (int t = 0; t < 2; ++t) {
    if (!xs[t]) continue;
    if (reinterpret_cast<uintptr_t>(xs[t]) % 16)
      return sa::fail(SA_ERR_UNSUPPORTED, "sa_sample_block_tokens: tensor base not 16-byte aligned");
    for (int i = 0; i < 3; ++i)
      if (ss[t][i] % 8) return sa::fail(SA_ERR_UNSUPPORTED, "sa_sample_block_tokens: strides must be multiples of 8");
  }
  SampleArgs a;
  const int nt = k ? 2 : 1;
  for (int t = 0; t < 2; ++t) {
    const int s = t < nt ? t : 0;
    a.rand[t] = s ? rand_k : rand_q;
    a.x[t] = xs[s];
    a.sb[t] = ss[s][0]; a.sh[t] = ss[s][1]; a.sl[t] = ss[s][2];
    a.tok[t] = s ? tok_k : tok_q;
    a.out[t] = s ? k_sampled : q_sampled;
  }
  a.H = H; a.L = L; a.nb = nb; a.S = num_keep; a.ns_pad = ns_pad;
  a.per_tensor = (int64_t)B * H * nb;
  a.total = a.per_tensor * nt;
  const int64_t grid = (a.total + 3) / 4;
  SA_REQUIRE(grid < (1LL << 31), "sa_sample_block_tokens: grid too large");
  hipLaunchKernelGGL(sample_gather_kernel, dim3((unsigned)grid), dim3(256), 0, sa::as_stream(stream), a);
  return sa::check_launch("sa_sample_block_tokens");
}

extern "C" int sa_sampled_block_scores(const uint16_t* q_sampled, const uint16_t* k_sampled, int BH, int nb,
                                       int num_keep, int ns_pad, float* pooled, void* stream) {
  SA_REQUIRE(q_sampled && k_sampled && pooled, "sa_sampled_block_scores: null pointer");
  SA_REQUIRE(BH > 0 && nb > 0, "sa_sampled_block_scores: bad shape BH=%d nb=%d", BH, nb);
  if (num_keep != 8 && num_keep != 16)
    return sa::fail(SA_ERR_UNSUPPORTED, "sa_sampled_block_scores: num_keep=%d (8 or 16)", num_keep);
  SA_REQUIRE(ns_pad % 32 == 0 && ns_pad >= nb * num_keep && ns_pad < nb * num_keep + 32,
             "sa_sampled_block_scores: ns_pad=%d must be nb*num_keep rounded up to 32", ns_pad);
  PoolSArgs a;
  a.sq = q_sampled; a.sk = k_sampled; a.pooled = pooled;
  a.nb = nb; a.ns = nb * num_keep; a.ns_pad = ns_pad; a.ng = ns_pad / 32;
  a.wg_per_bh = (a.ng + 3) / 4;
  const int64_t grid = (int64_t)BH * a.wg_per_bh;
  SA_REQUIRE(grid < (1LL << 31), "sa_sampled_block_scores: grid too large");
  hipStream_t s = sa::as_stream(stream);
  if (num_keep == 8) {
    hipLaunchKernelGGL(sampled_pool_kernel<8>, dim3((unsigned)grid), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(sampled_pool_kernel<16>, dim3((unsigned)grid), dim3(256), 0, s, a);
  }
  return sa::check_launch("sa_sampled_block_scores");
}

extern "C" int sa_energy_kv_list(const float* scores, int BH, int nqb, int nkb, int mode, float threshold,
                                 int min_keep, int max_keep, int init_k, int n_text_blocks, int32_t* kv_idx,
                                 int max_cnt, int32_t* kv_cnt, uint8_t* mask_out, void* stream) {
  SA_REQUIRE(scores && kv_idx && kv_cnt, "sa_energy_kv_list: null pointer");
  SA_REQUIRE(BH > 0 && nqb > 0 && nkb > 0, "sa_energy_kv_list: bad shape BH=%d nqb=%d nkb=%d", BH, nqb, nkb);
  SA_REQUIRE(mode >= 0 && mode <= 3, "sa_energy_kv_list: mode %d (0 energy, 1 topk, 2 inclusive, 3 cumulative <=)",
             mode);
  SA_REQUIRE(n_text_blocks >= 0, "sa_energy_kv_list: negative n_text_blocks");
  SA_REQUIRE(max_cnt >= nkb, "sa_energy_kv_list: max_cnt=%d < nkb=%d", max_cnt, nkb);
  if (mode == 1) SA_REQUIRE(init_k >= 1 && init_k <= nkb, "sa_energy_kv_list: init_k=%d outside [1, %d]", init_k, nkb);
  if (nkb > 1024) return sa::fail(SA_ERR_UNSUPPORTED, "sa_energy_kv_list: nkb=%d > 1024", nkb);
  EnergyArgs a;
  a.scores = scores; a.rows = (int64_t)BH * nqb; a.nqb = nqb; a.nkb = nkb; a.mode = mode;
  a.threshold = threshold; a.min_keep = min_keep; a.max_keep = max_keep; a.init_k = init_k;
  a.n_text = n_text_blocks; a.kv_idx = kv_idx; a.max_cnt = max_cnt; a.kv_cnt = kv_cnt; a.mask_out = mask_out;
  const int64_t grid = (a.rows + 3) / 4;
  SA_REQUIRE(grid < (1LL << 31), "sa_energy_kv_list: grid too large");
  hipStream_t s = sa::as_stream(stream);
  if (nkb <= 256) {
    hipLaunchKernelGGL(energy_list_kernel<4>, dim3((unsigned)grid), dim3(256), 0, s, a);
  } else if (nkb <= 320) {
    hipLaunchKernelGGL(energy_list_kernel<5>, dim3((unsigned)grid), dim3(256), 0, s, a);
  } else if (nkb <= 512) {
    hipLaunchKernelGGL(energy_list_kernel<8>, dim3((unsigned)grid), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(energy_list_kernel<16>, dim3((unsigned)grid), dim3(256), 0, s, a);
  }
  return sa::check_launch("sa_energy_kv_list");
}
