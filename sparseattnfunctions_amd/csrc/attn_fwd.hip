// Block-sparse attention forward for gfx950 (CDNA4), bf16 in / bf16 out, fp32 softmax.
//
// Replaces the Triton `_fwd_kernel` / `_fwd_kernel_inner` of
// special_attentions/utils/block_sparse_attn_kernel.py:52-209 and its host wrapper
// `_forward` (:211-265). Same arithmetic contract: S = q k^T * sm_scale, keys past Lk in
// the last block masked to -inf (:87-89), online softmax in fp32, P rounded to bf16 before
// P.V (:107), out = acc / l (:201-203). Differences by design: the key blocks to visit come
// from a compacted per-row list (kv_idx/kv_cnt) instead of a scan of the dense mask; the
// softmax runs in the exp2 domain with log2(e) folded into the scale; an empty row writes 0.
//
// Work decomposition. One wave64 owns one (b, h, 64-row query block) work item; a
// workgroup holds 4 independent waves (no workgroup barriers). Per 64-key tile a wave
// computes S^T = K Q^T and O^T = V^T P^T with v_mfma_f32_32x32x16_bf16 (2 query groups of
// 32 rows x 2 key chunks x 4 d-steps, then 2 d-chunks x 2 query groups x 4 key-steps:
// 32 MFMAs = 1 MFLOP). Each lane holds one query column of S^T, so row statistics need
// one cross-half exchange. K is loaded from global memory straight into MFMA A-operand
// registers; V is loaded coalesced and written transposed into a wave-private LDS tile,
// read back as V^T A-operands. The loads of tile i+1 are issued while tile i is computed.
//
// Softmax economy (VALU is the co-bottleneck at d = 64): the running max is only raised
// when a tile exceeds it by more than kRescaleLog2 (then p <= 2^kRescaleLog2), so the
// accumulator rescale is rare; row sums accumulate the bf16-rounded P pairs with
// v_dot2c_f32_bf16; maxima use v_max3_f32.
//
// Scheduling: a host-built work order maps dispatch slots to items so that each XCD
// (workgroups round-robin over 8 XCDs) processes a contiguous range of heads, longest
// (text) rows first.
#include <math.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "sa_common.h"

namespace {

constexpr int kBlock = 64;       // query rows per block == keys per key block
constexpr int kHeadDim = 64;     // head dimension handled by this kernel
constexpr int kWaves = 4;        // independent waves per workgroup
constexpr int kVtStride = 68;    // LDS row stride (bf16) of the V^T tile: 32 rows hit 64 banks once
constexpr int kVtElems = kHeadDim * kVtStride;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;
#ifndef SA_ATTN_MIN_WAVES
#define SA_ATTN_MIN_WAVES 2
#endif

struct FwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t q_sb, q_sh, q_sl;
  int64_t k_sb, k_sh, k_sl;
  int64_t v_sb, v_sh, v_sl;
  int64_t o_sb, o_sh, o_sl;
  int H, Lq, Lk, nqb, nkb;
  int n_items;             // B*H*nqb
  const int32_t* order;    // dispatch slot -> item (bh*nqb + qb), -1 = idle; may be null
  int n_slots;
  const int32_t* kv_idx;
  const int32_t* kv_cnt;
  int max_cnt;
  const float* bias;
  int64_t bias_sb, bias_sh;
  float scale_log2;  // sm_scale * log2(e)
  int list_bh_stride;          // list row = bh * list_bh_stride + qb (0: lists shared by heads)
  const int32_t* kv_slot;      // [rows][max_cnt] tile-mask slot of each entry, -1 = full tile
  const uint64_t* tile_masks;  // [slots][64] bit k of row r: query r may attend key k
};

__device__ inline sa_bf16x8 as_bf16x8(uint4 x) { return __builtin_bit_cast(sa_bf16x8, x); }

__device__ inline sa_f32x16 mfma32(sa_bf16x8 a, sa_bf16x8 b, sa_f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline uint32_t word(const uint4& x, int j) {
  return j == 0 ? x.x : (j == 1 ? x.y : (j == 2 ? x.z : x.w));
}

// Byte select: {lo16(a), lo16(b)} (kHi = false) or {hi16(a), hi16(b)} (kHi = true).
template <bool kHi>
__device__ inline uint32_t pack_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, kHi ? 0x07060302u : 0x05040100u);
}

typedef __bf16 sa_bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 pair (round to nearest even, v_cvt_pk_bf16_f32).
__device__ inline uint32_t cvt_pk_bf16(float a, float b) {
  sa_bf16x2 r = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, r);
}

__device__ inline float dot2_bf16_ones(uint32_t pair, float acc) {
  const sa_bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(sa_bf16x2, pair), ones, acc, false);
}

// All loads below are unconditional with row indices clamped into [0, L): a per-lane
// condition would become an exec-masked branch, and the compiler then cannot count the
// loads in flight and waits for all of them (s_waitcnt vmcnt(0)) before any use. Rows
// clamped past Lk belong to keys whose scores are masked to -inf (their V rows meet p = 0;
// clamped data is finite), and clamped Q rows past Lq are never stored.

// K tile as MFMA A operands: kr[c][s] = K[key0 + 32c + col][16s + 8hh .. +7].
__device__ inline void load_k(const FwdArgs& a, const uint16_t* kbase, int key0, int col, int hh,
                              uint4 (&kr)[2][4]) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int key = min(key0 + 32 * c + col, a.Lk - 1);
    const uint16_t* p = kbase + (int64_t)key * a.k_sl + 8 * hh;
#pragma unroll
    for (int s = 0; s < 4; ++s) kr[c][s] = *reinterpret_cast<const uint4*>(p + 16 * s);
  }
}

// V tile rows for the transposed LDS write: vr[p][e] = V[key0 + 4kq + e][8(dg + 4p) .. +7].
__device__ inline void load_v(const FwdArgs& a, const uint16_t* vbase, int key0, int lane,
                              uint4 (&vr)[2][4]) {
  const int kq = lane & 15, dg = lane >> 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int key = min(key0 + 4 * kq + e, a.Lk - 1);
    const uint16_t* p = vbase + (int64_t)key * a.v_sl + 8 * dg;
#pragma unroll
    for (int p2 = 0; p2 < 2; ++p2) vr[p2][e] = *reinterpret_cast<const uint4*>(p + 32 * p2);
  }
}

__device__ inline void store_vt(uint16_t* vt, int lane, const uint4 (&vr)[2][4]) {
  const int kq = lane & 15, dg = lane >> 4;
#pragma unroll
  for (int p2 = 0; p2 < 2; ++p2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w0 = word(vr[p2][0], j), w1 = word(vr[p2][1], j);
      const uint32_t w2 = word(vr[p2][2], j), w3 = word(vr[p2][3], j);
      const int d = 8 * (dg + 4 * p2) + 2 * j;
      *reinterpret_cast<uint2*>(vt + d * kVtStride + 4 * kq) =
          make_uint2(pack_halves<false>(w0, w1), pack_halves<false>(w2, w3));
      *reinterpret_cast<uint2*>(vt + (d + 1) * kVtStride + 4 * kq) =
          make_uint2(pack_halves<true>(w0, w1), pack_halves<true>(w2, w3));
    }
  }
}

// V^T A operand for d-chunk dc, key step (c, u): V^T[32dc + col][32c + 16u + 4hh + {0..3, 8..11}].
__device__ inline sa_bf16x8 read_vt(const uint16_t* vt, int dc, int c, int u, int col, int hh) {
  const uint16_t* r = vt + (32 * dc + col) * kVtStride + 32 * c + 16 * u + 4 * hh;
  const uint2 lo = *reinterpret_cast<const uint2*>(r);
  const uint2 hi = *reinterpret_cast<const uint2*>(r + 8);
  return as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// Softmax of one query group's 16 S^T values of a 32-key half (element i -> key
// 8(i/4) + 4hh + (i%4) of the half) into 8 packed bf16 P pairs; updates the running max m
// (log2 domain, scaled) and the lane-partial row sum l. Returns true (wave-uniform) when
// the running max was raised; then *alpha is the factor for the accumulator.
template <bool kBias>
__device__ inline bool softmax16(sa_f32x16& s, const float (&bl)[16], float scale_log2, float& m, float& l,
                                 uint32_t (&pk)[8], float& alpha) {
  if (kBias) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = fmaf(s[i], scale_log2, bl[i]);
  }
  float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
  for (int i = 3; i < 15; i += 2) mx = fmaxf(fmaxf(mx, s[i]), s[i + 1]);
  mx = fmaxf(mx, s[15]);
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float cand = kBias ? mx : mx * scale_log2;  // scale_log2 > 0
  // Raise the running max only when this half-tile exceeds it by more than the threshold
  // (always on the first one, where m = -inf).
  const bool raise = __ballot(cand > m + kRescaleLog2) != 0;
  if (raise) {
    const float m_new = fmaxf(m, cand);
    alpha = fast_exp2(m - m_new);  // 0 when m = -inf
    l *= alpha;
    m = m_new;
  }
  const float m_use = (m == -INFINITY) ? 0.f : m;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    float p0, p1;
    if (kBias) {
      p0 = fast_exp2(s[i] - m_use);
      p1 = fast_exp2(s[i + 1] - m_use);
    } else {
      p0 = fast_exp2(fmaf(s[i], scale_log2, -m_use));
      p1 = fast_exp2(fmaf(s[i + 1], scale_log2, -m_use));
    }
    pk[i >> 1] = cvt_pk_bf16(p0, p1);
    l = dot2_bf16_ones(pk[i >> 1], l);
  }
  return raise;
}

// P^T B operand for key step u of a half: elements 8u..8u+7.
__device__ inline sa_bf16x8 p_operand(const uint32_t (&pk)[8], int u) {
  return as_bf16x8(make_uint4(pk[4 * u], pk[4 * u + 1], pk[4 * u + 2], pk[4 * u + 3]));
}

template <bool kBias, bool kMask>
__global__ __launch_bounds__(256, SA_ATTN_MIN_WAVES) void bsa_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kWaves][kVtElems];
  // Key bias of the current tile (log2 domain), staged with V: one load per lane.
  __shared__ __attribute__((aligned(16))) float bias_lds[kBias ? kWaves : 1][kBlock];

  const int lane = threadIdx.x & 63;
  // Wave-uniform values are made provably uniform (readfirstlane) so that the list and
  // order reads below are scalar loads: a vector load would need s_waitcnt vmcnt(0),
  // which would also wait for the K/V prefetches in flight.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31;  // query column within a 32-row group (MFMA n index)
  const int hh = lane >> 5;   // lane half (MFMA k group)
  const int slot = blockIdx.x * kWaves + wave;
  if (slot >= a.n_slots) return;
  const int item = __builtin_amdgcn_readfirstlane(a.order ? a.order[slot] : slot);
  if (item < 0 || item >= a.n_items) return;  // idle slot (no workgroup barriers below)
  const int bh = item / a.nqb;
  const int qb = item - bh * a.nqb;
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  uint16_t* vt = vt_lds[wave];

  const int64_t list_row = (int64_t)bh * a.list_bh_stride + qb;
  int cnt = a.kv_cnt[list_row];
  cnt = cnt < 0 ? 0 : (cnt > a.max_cnt ? a.max_cnt : cnt);
  const int32_t* list = a.kv_idx + list_row * a.max_cnt;
  const int32_t* slots = kMask ? a.kv_slot + list_row * a.max_cnt : nullptr;

  const uint16_t* qbase = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kbase = a.k + b * a.k_sb + h * a.k_sh;
  const uint16_t* vbase = a.v + b * a.v_sb + h * a.v_sh;
  uint16_t* obase = a.o + b * a.o_sb + h * a.o_sh;
  const float* bbase = kBias ? a.bias + b * a.bias_sb + h * a.bias_sh : nullptr;

  // Q^T B operands: qf[g][s] = q[qb*64 + 32g + col][16s + 8hh .. +7].
  sa_bf16x8 qf[2][4];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int row = min(qb * kBlock + 32 * g + col, a.Lq - 1);
    const uint16_t* p = qbase + (int64_t)row * a.q_sl + 8 * hh;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[g][s] = as_bf16x8(*reinterpret_cast<const uint4*>(p + 16 * s));
  }

  sa_f32x16 acc[2][2];  // [dc][g]
#pragma unroll
  for (int dc = 0; dc < 2; ++dc)
#pragma unroll
    for (int g = 0; g < 2; ++g) acc[dc][g] = sa_f32x16{};
  float m[2] = {-INFINITY, -INFINITY};
  float l[2] = {0.f, 0.f};

  // Skip list entries outside the key-block grid.
  auto next_valid = [&](int it) {
    while (it < cnt && (unsigned)list[it] >= (unsigned)a.nkb) ++it;
    return it;
  };

  int it = next_valid(0);
  uint4 kr[2][4];
  uint4 vr[2][4];
  float bv = 0.f;  // bias of key `lane` of the prefetched tile (kBias only)
  float* bl_lds = bias_lds[kBias ? wave : 0];
  auto load_bias = [&](int key0) {
    if (kBias) bv = bbase[min(key0 + lane, a.Lk - 1)] * kLog2e;
  };
  // Tile masks (kMask only): rows 32g + col of the current / prefetched tile's mask.
  uint64_t mw_cur[2] = {~0ull, ~0ull}, mw_next[2] = {~0ull, ~0ull};
  int slot_cur = -1, slot_next = -1;
  auto load_mask = [&](int it_) {
    if (kMask) {
      slot_next = it_ < cnt ? slots[it_] : -1;
      const uint64_t* mrow = a.tile_masks + (int64_t)max(slot_next, 0) * kBlock;
      mw_next[0] = mrow[col];
      mw_next[1] = mrow[32 + col];
    }
  };
  int kb_cur = it < cnt ? list[it] : 0;
  if (it < cnt) {
    load_k(a, kbase, kb_cur * kBlock, col, hh, kr);
    load_v(a, vbase, kb_cur * kBlock, lane, vr);
    load_bias(kb_cur * kBlock);
    load_mask(it);
    store_vt(vt, lane, vr);
    if (kBias) bl_lds[lane] = bv;
    slot_cur = slot_next;
    mw_cur[0] = mw_next[0];
    mw_cur[1] = mw_next[1];
  }
  int it_next = next_valid(it + 1);
  // Prefetches are issued every iteration (past the end of the list they re-load the
  // current block) so the loop body has the same loads in flight on every path.
  int kb_next = it_next < cnt ? list[it_next] : kb_cur;
  if (it < cnt) {
    load_v(a, vbase, kb_next * kBlock, lane, vr);
    load_bias(kb_next * kBlock);
    load_mask(it_next);
  }

  while (it < cnt) {
    const int key0 = kb_cur * kBlock;
    const int nvalid = min(kBlock, a.Lk - key0);
    // Two 32-key halves per tile keep one half's S (32 VGPRs) and P (16) live at a time.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      sa_f32x16 s[2];  // [g]: S^T of keys 32c.., query group g
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        sa_f32x16 t = {};
#pragma unroll
        for (int st = 0; st < 4; ++st) t = mfma32(as_bf16x8(kr[c][st]), qf[g][st], t);
        s[g] = t;
      }
      if (c == 1) load_k(a, kbase, kb_next * kBlock, col, hh, kr);

      if (nvalid < kBlock) {  // keys past Lk in the last (partial) block
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = 32 * c + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (key >= nvalid) {
            s[0][i] = -INFINITY;
            s[1][i] = -INFINITY;
          }
        }
      }
      if (kMask && slot_cur >= 0) {  // token-level mask of a tile cut by a mask boundary
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const uint32_t half = (uint32_t)(mw_cur[g] >> (32 * c));
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = 8 * (i >> 2) + 4 * hh + (i & 3);
            if (!((half >> key) & 1u)) s[g][i] = -INFINITY;
          }
        }
      }
      float bl[16];
      if (kBias) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int key = key0 + 32 * c + 8 * q4 + 4 * hh;
          const float4 b4 = *reinterpret_cast<const float4*>(bl_lds + (key - key0));
          bl[4 * q4 + 0] = b4.x;
          bl[4 * q4 + 1] = b4.y;
          bl[4 * q4 + 2] = b4.z;
          bl[4 * q4 + 3] = b4.w;
        }
      }

      uint32_t pk[2][8];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        float alpha = 1.f;
        if (softmax16<kBias>(s[g], bl, a.scale_log2, m[g], l[g], pk[g], alpha)) {
#pragma unroll
          for (int dc = 0; dc < 2; ++dc) acc[dc][g] *= alpha;
        }
      }
      // O^T += V^T P^T over this half's two 16-key steps.
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int dc = 0; dc < 2; ++dc) {
          const sa_bf16x8 va = read_vt(vt, dc, c, u, col, hh);
#pragma unroll
          for (int g = 0; g < 2; ++g) acc[dc][g] = mfma32(va, p_operand(pk[g], u), acc[dc][g]);
        }
      }
    }

    // ---- V^T of the next tile into the (now free) LDS tile; prefetch the one after.
    // LDS accesses of one wave execute in order and the compiler keeps the program order
    // of these aliasing accesses, so no fence is needed (a fence would also wait for the
    // global prefetches).
    it = it_next;
    kb_cur = kb_next;
    store_vt(vt, lane, vr);
    if (kBias) bl_lds[lane] = bv;
    slot_cur = slot_next;
    mw_cur[0] = mw_next[0];
    mw_cur[1] = mw_next[1];
    it_next = next_valid(it + 1);
    kb_next = it_next < cnt ? list[it_next] : kb_cur;
    load_v(a, vbase, kb_next * kBlock, lane, vr);
    load_bias(kb_next * kBlock);
    load_mask(it_next);
  }

  // ---- Epilogue: out = acc / l (each lane half holds a partial l of its keys).
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float l_tot = l[g] + __shfl_xor(l[g], 32);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int row = qb * kBlock + 32 * g + col;
    if (row < a.Lq) {
      uint16_t* orow = obase + (int64_t)row * a.o_sl;
#pragma unroll
      for (int dc = 0; dc < 2; ++dc) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const sa_f32x16& A = acc[dc][g];
          // element 4q4 + j is d = 32dc + 8q4 + 4hh + j
          *reinterpret_cast<uint2*>(orow + 32 * dc + 8 * q4 + 4 * hh) =
              make_uint2(cvt_pk_bf16(A[4 * q4] * inv, A[4 * q4 + 1] * inv),
                         cvt_pk_bf16(A[4 * q4 + 2] * inv, A[4 * q4 + 3] * inv));
        }
      }
    }
  }
}

}  // namespace

extern "C" int sa_attn_work_order(int B, int H, int nqb, int n_text_blocks, int n_xcd, int32_t* order,
                                  int64_t* n_slots) {
  SA_REQUIRE(n_slots, "sa_attn_work_order: null n_slots");
  SA_REQUIRE(B > 0 && H > 0 && nqb > 0 && n_text_blocks >= 0 && n_xcd > 0,
             "sa_attn_work_order: bad arguments B=%d H=%d nqb=%d n_text=%d n_xcd=%d", B, H, nqb, n_text_blocks, n_xcd);
  const int64_t n_items = (int64_t)B * H * nqb;
  SA_REQUIRE(n_items < (1LL << 30), "sa_attn_work_order: too many items");
  // Contiguous bh-major chunks of (nearly) equal size, one per XCD.
  std::vector<int64_t> lo(n_xcd + 1);
  for (int x = 0; x <= n_xcd; ++x) lo[x] = n_items * x / n_xcd;
  int64_t max_chunk = 0;
  for (int x = 0; x < n_xcd; ++x) max_chunk = std::max<int64_t>(max_chunk, lo[x + 1] - lo[x]);
  const int64_t wg_per_xcd = (max_chunk + kWaves - 1) / kWaves;
  const int64_t total = wg_per_xcd * n_xcd * kWaves;
  *n_slots = total;
  if (!order) return sa::ok();
  for (int64_t i = 0; i < total; ++i) order[i] = -1;
  std::vector<int32_t> chunk;
  for (int x = 0; x < n_xcd; ++x) {
    chunk.clear();
    // Text rows (longest lists) first, then the rest; bh-major within each class.
    for (int pass = 0; pass < 2; ++pass)
      for (int64_t it = lo[x]; it < lo[x + 1]; ++it) {
        const bool text = (it % nqb) < n_text_blocks;
        if (text == (pass == 0)) chunk.push_back((int32_t)it);
      }
    // Workgroup w of this XCD is dispatch index w*n_xcd + x (round-robin dispatch).
    for (size_t p = 0; p < chunk.size(); ++p) {
      const int64_t w = (int64_t)p / kWaves;
      order[(w * n_xcd + x) * kWaves + (int64_t)p % kWaves] = chunk[p];
    }
  }
  return sa::ok();
}

namespace {

int launch_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k, const int64_t k_strides[3],
               const uint16_t* v, const int64_t v_strides[3], uint16_t* out, const int64_t out_strides[3], int B,
               int H, int Lq, int Lk, int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
               bool lists_shared, const int32_t* kv_slot, const uint64_t* tile_masks, const float* key_bias,
               const int64_t bias_strides[2], float sm_scale, const int32_t* work_order, int64_t n_slots,
               void* stream, const char* fn) {
  SA_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides && kv_idx && kv_cnt,
             "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && Lq > 0 && Lk > 0, "%s: bad shape B=%d H=%d Lq=%d Lk=%d", fn, B, H, Lq, Lk);
  if (D != kHeadDim) return sa::fail(SA_ERR_UNSUPPORTED, "%s: head_dim %d (only 64)", fn, D);
  SA_REQUIRE(std::isfinite(sm_scale) && sm_scale > 0.f, "%s: sm_scale must be finite and > 0", fn);
  const int nqb = sa::cdiv(Lq, kBlock);
  const int nkb = sa::cdiv(Lk, kBlock);
  SA_REQUIRE(max_cnt > 0, "%s: max_cnt must be > 0", fn);
  SA_REQUIRE(!key_bias || bias_strides, "%s: key_bias without bias_strides", fn);
  const int64_t n_items = (int64_t)B * H * nqb;
  SA_REQUIRE(n_items < (1LL << 30), "%s: too many query blocks", fn);
  if (work_order) {
    SA_REQUIRE(n_slots > 0 && n_slots % kWaves == 0, "%s: n_slots must be a positive multiple of 4", fn);
  } else {
    n_slots = (n_items + kWaves - 1) / kWaves * kWaves;
  }
  // 16-byte vector accesses: base pointers 16-byte aligned, row strides multiples of 8 elements.
  const void* ptrs[4] = {q, k, v, out};
  for (const void* p : ptrs) {
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return sa::fail(SA_ERR_UNSUPPORTED, "%s: tensor base not 16-byte aligned", fn);
  }
  const int64_t* strides[4] = {q_strides, k_strides, v_strides, out_strides};
  for (const int64_t* s : strides) {
    for (int i = 0; i < 3; ++i) {
      if (s[i] % 8 != 0) return sa::fail(SA_ERR_UNSUPPORTED, "%s: strides must be multiples of 8 elements", fn);
    }
  }
  const int64_t grid = n_slots / kWaves;
  SA_REQUIRE(grid < (1LL << 31), "%s: grid too large", fn);

  FwdArgs a;
  a.q = q; a.k = k; a.v = v; a.o = out;
  a.q_sb = q_strides[0]; a.q_sh = q_strides[1]; a.q_sl = q_strides[2];
  a.k_sb = k_strides[0]; a.k_sh = k_strides[1]; a.k_sl = k_strides[2];
  a.v_sb = v_strides[0]; a.v_sh = v_strides[1]; a.v_sl = v_strides[2];
  a.o_sb = out_strides[0]; a.o_sh = out_strides[1]; a.o_sl = out_strides[2];
  a.H = H; a.Lq = Lq; a.Lk = Lk; a.nqb = nqb; a.nkb = nkb;
  a.n_items = (int)n_items;
  a.order = work_order;
  a.n_slots = (int)n_slots;
  a.kv_idx = kv_idx; a.kv_cnt = kv_cnt; a.max_cnt = max_cnt;
  a.bias = key_bias;
  a.bias_sb = key_bias ? bias_strides[0] : 0;
  a.bias_sh = key_bias ? bias_strides[1] : 0;
  a.scale_log2 = sm_scale * kLog2e;
  a.list_bh_stride = lists_shared ? 0 : nqb;
  a.kv_slot = kv_slot;
  a.tile_masks = tile_masks;

  hipStream_t s = sa::as_stream(stream);
  const dim3 g((unsigned)grid), blk(64 * kWaves);
  if (kv_slot) {
    if (key_bias) return sa::fail(SA_ERR_UNSUPPORTED, "%s: tile masks with key_bias", fn);
    hipLaunchKernelGGL((bsa_fwd_kernel<false, true>), g, blk, 0, s, a);
  } else if (key_bias) {
    hipLaunchKernelGGL((bsa_fwd_kernel<true, false>), g, blk, 0, s, a);
  } else {
    hipLaunchKernelGGL((bsa_fwd_kernel<false, false>), g, blk, 0, s, a);
  }
  return sa::check_launch(fn);
}

}  // namespace

extern "C" int sa_block_sparse_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                   const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                   uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                   int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                   const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                   const int32_t* work_order, int64_t n_slots, void* stream) {
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, false, nullptr, nullptr, key_bias, bias_strides, sm_scale, work_order, n_slots, stream,
                    "sa_block_sparse_fwd");
}

extern "C" int sa_block_sparse_fwd_tilemask(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                            const int64_t k_strides[3], const uint16_t* v,
                                            const int64_t v_strides[3], uint16_t* out, const int64_t out_strides[3],
                                            int B, int H, int Lq, int Lk, int D, const int32_t* kv_idx,
                                            const int32_t* kv_cnt, const int32_t* kv_slot, int max_cnt,
                                            int lists_shared, const uint64_t* tile_masks, float sm_scale,
                                            const int32_t* work_order, int64_t n_slots, void* stream) {
  SA_REQUIRE(kv_slot && tile_masks, "sa_block_sparse_fwd_tilemask: null kv_slot/tile_masks");
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, lists_shared != 0, kv_slot, tile_masks, nullptr, nullptr, sm_scale, work_order, n_slots,
                    stream, "sa_block_sparse_fwd_tilemask");
}
