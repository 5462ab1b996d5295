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
// Work decomposition: one workgroup of two wave64s per (b, h, 64-row query block). Each
// wave owns 32 query rows and computes S^T = K Q^T and O^T = V^T P^T with
// v_mfma_f32_32x32x16_bf16, so every lane holds one query column of S^T and the row max
// needs a single cross-half exchange. K (row-major) and V (transposed) tiles of 64 keys are
// staged through double-buffered LDS; the global loads of tile i+1 are in flight while
// tile i is computed.
#include <math.h>

#include <cmath>

#include "sa_common.h"

namespace {

constexpr int kBlock = 64;     // query rows per block == keys per key block
constexpr int kHeadDim = 64;   // head dimension handled by this kernel
constexpr int kThreads = 128;  // two wave64s
constexpr int kRowPad = 72;    // LDS row stride in bf16 elements (K rows, V^T rows)
constexpr int kTileElems = kBlock * kRowPad;
constexpr float kLog2e = 1.4426950408889634f;

struct FwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t q_sb, q_sh, q_sl;
  int64_t k_sb, k_sh, k_sl;
  int64_t v_sb, v_sh, v_sl;
  int64_t o_sb, o_sh, o_sl;
  int H, Lq, Lk, nqb, nkb, BH;
  const int32_t* kv_idx;
  const int32_t* kv_cnt;
  int max_cnt;
  const float* bias;
  int64_t bias_sb, bias_sh;
  float scale_log2;  // sm_scale * log2(e)
};

__device__ inline sa_bf16x8 as_bf16x8(sa_u16x8 x) { return __builtin_bit_cast(sa_bf16x8, x); }

__device__ inline sa_f32x16 mfma32(sa_bf16x8 a, sa_bf16x8 b, sa_f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Per-thread staging registers of one K/V tile between the global load and the LDS store.
struct TileRegs {
  uint4 k[4];
  uint4 v[4];
  float bias;
};

// Global -> registers for key block kb (zero-filled past Lk or for an invalid kb).
template <bool kBias>
__device__ inline void load_tile(const FwdArgs& a, const uint16_t* kbase, const uint16_t* vbase,
                                 const float* bbase, int kb, int tid, TileRegs& r) {
  const bool kb_ok = (unsigned)kb < (unsigned)a.nkb;
  const int key0 = kb * kBlock;
  // K: 512 16-byte chunks, thread t takes keys (t>>3)+16i, dims 8*(t&7)..+7.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = (tid >> 3) + 16 * i;
    const int kg = key0 + key;
    if (kb_ok && kg < a.Lk) {
      r.k[i] = *reinterpret_cast<const uint4*>(kbase + (int64_t)kg * a.k_sl + 8 * (tid & 7));
    } else {
      r.k[i] = make_uint4(0, 0, 0, 0);
    }
  }
  // V: thread t takes keys 4*(t&15)..+3, dims 8*(t>>4)..+7, to be written transposed.
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int kg = key0 + 4 * (tid & 15) + e;
    if (kb_ok && kg < a.Lk) {
      r.v[e] = *reinterpret_cast<const uint4*>(vbase + (int64_t)kg * a.v_sl + 8 * (tid >> 4));
    } else {
      r.v[e] = make_uint4(0, 0, 0, 0);
    }
  }
  if (kBias) {
    r.bias = 0.f;
    if (tid < kBlock) {
      const int kg = key0 + tid;
      r.bias = (kb_ok && kg < a.Lk) ? bbase[kg] * kLog2e : 0.f;
    }
  }
}

__device__ inline uint32_t word(const uint4& x, int j) {
  return j == 0 ? x.x : (j == 1 ? x.y : (j == 2 ? x.z : x.w));
}

// Byte select: {lo16(a), lo16(b)} for kHi = false, {hi16(a), hi16(b)} for kHi = true.
template <bool kHi>
__device__ inline uint32_t pack_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, kHi ? 0x07060302u : 0x05040100u);
}

template <bool kBias>
__device__ inline void store_tile(uint16_t* k_lds, uint16_t* vt_lds, float* b_lds, int tid,
                                  const TileRegs& r) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = (tid >> 3) + 16 * i;
    *reinterpret_cast<uint4*>(k_lds + key * kRowPad + 8 * (tid & 7)) = r.k[i];
  }
  // V^T: row d8+x gets keys key4..key4+3 (one 8-byte store per d).
  const int key4 = 4 * (tid & 15);
  const int d8 = 8 * (tid >> 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w0 = word(r.v[0], j), w1 = word(r.v[1], j);
    const uint32_t w2 = word(r.v[2], j), w3 = word(r.v[3], j);
    *reinterpret_cast<uint2*>(vt_lds + (d8 + 2 * j) * kRowPad + key4) =
        make_uint2(pack_halves<false>(w0, w1), pack_halves<false>(w2, w3));
    *reinterpret_cast<uint2*>(vt_lds + (d8 + 2 * j + 1) * kRowPad + key4) =
        make_uint2(pack_halves<true>(w0, w1), pack_halves<true>(w2, w3));
  }
  if (kBias) {
    if (tid < kBlock) b_lds[tid] = r.bias;
  }
}

template <bool kBias>
__global__ __launch_bounds__(kThreads) void bsa_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][kTileElems];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][kTileElems];
  __shared__ float b_lds[2][kBlock];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // query row within the wave (MFMA n index)
  const int hh = lane >> 5;   // lane half (MFMA k group)

  // Query blocks are visited block-row major, so the text rows (longest lists, block
  // rows 0..3 for CogVideoX) are dispatched first.
  const int wg = blockIdx.x;
  const int qb = wg / a.BH;
  const int bh = wg - qb * a.BH;
  const int b = bh / a.H;
  const int h = bh - b * a.H;

  const int64_t list_row = (int64_t)bh * a.nqb + qb;
  int cnt = a.kv_cnt[list_row];
  cnt = cnt < 0 ? 0 : (cnt > a.max_cnt ? a.max_cnt : cnt);
  const int32_t* list = a.kv_idx + list_row * a.max_cnt;

  const uint16_t* qbase = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kbase = a.k + b * a.k_sb + h * a.k_sh;
  const uint16_t* vbase = a.v + b * a.v_sb + h * a.v_sh;
  uint16_t* obase = a.o + b * a.o_sb + h * a.o_sh;
  const float* bbase = kBias ? a.bias + b * a.bias_sb + h * a.bias_sh : nullptr;

  // Q^T fragments (MFMA B operand): lane holds q[row][16s + 8hh .. +7] for s = 0..3.
  const int qrow = qb * kBlock + wave * 32 + col;
  sa_bf16x8 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    sa_u16x8 t = {0, 0, 0, 0, 0, 0, 0, 0};
    if (qrow < a.Lq) t = *reinterpret_cast<const sa_u16x8*>(qbase + (int64_t)qrow * a.q_sl + 16 * s + 8 * hh);
    qf[s] = as_bf16x8(t);
  }

  sa_f32x16 acc0 = {}, acc1 = {};
  float m_i = -INFINITY;
  float l_i = 0.f;

  TileRegs regs;
  int kb_cur = 0;
  if (cnt > 0) {
    kb_cur = list[0];
    load_tile<kBias>(a, kbase, vbase, bbase, kb_cur, tid, regs);
    store_tile<kBias>(k_lds[0], vt_lds[0], b_lds[0], tid, regs);
  }
  __syncthreads();

  for (int it = 0; it < cnt; ++it) {
    const int buf = it & 1;
    int kb_next = 0;
    if (it + 1 < cnt) {
      kb_next = list[it + 1];
      load_tile<kBias>(a, kbase, vbase, bbase, kb_next, tid, regs);
    }

    // ---- S^T = K Q^T for keys [0,32) and [32,64) of the tile.
    const uint16_t* kl = k_lds[buf];
    sa_f32x16 s0 = {}, s1 = {};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const sa_bf16x8 a0 = as_bf16x8(*reinterpret_cast<const sa_u16x8*>(kl + col * kRowPad + 16 * st + 8 * hh));
      const sa_bf16x8 a1 = as_bf16x8(*reinterpret_cast<const sa_u16x8*>(kl + (32 + col) * kRowPad + 16 * st + 8 * hh));
      s0 = mfma32(a0, qf[st], s0);
      s1 = mfma32(a1, qf[st], s1);
    }
    // Element i of s_c is key 32c + 8(i/4) + 4hh + (i%4) of the tile, query `col`.

    const bool kb_ok = (unsigned)kb_cur < (unsigned)a.nkb;
    const int nvalid = kb_ok ? min(kBlock, a.Lk - kb_cur * kBlock) : 0;
    if (nvalid < kBlock) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = 8 * (i >> 2) + 4 * hh + (i & 3);
        if (key >= nvalid) s0[i] = -INFINITY;
        if (key + 32 >= nvalid) s1[i] = -INFINITY;
      }
    }

    float m_new;
    if (kBias) {
      const float* bl = b_lds[buf];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = 8 * (i >> 2) + 4 * hh + (i & 3);
        s0[i] = fmaf(s0[i], a.scale_log2, bl[key]);
        s1[i] = fmaf(s1[i], a.scale_log2, bl[key + 32]);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fmaxf(s0[i], s1[i]));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      m_new = fmaxf(m_i, mx);
    } else {
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fmaxf(s0[i], s1[i]));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      m_new = fmaxf(m_i, mx * a.scale_log2);
    }
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_i - m_use);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (kBias) {
        s0[i] = fast_exp2(s0[i] - m_use);
        s1[i] = fast_exp2(s1[i] - m_use);
      } else {
        s0[i] = fast_exp2(fmaf(s0[i], a.scale_log2, -m_use));
        s1[i] = fast_exp2(fmaf(s1[i], a.scale_log2, -m_use));
      }
      psum += s0[i] + s1[i];
    }
    l_i = l_i * alpha + psum;
    m_i = m_new;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc0[i] *= alpha;
      acc1[i] *= alpha;
    }

    // P^T as MFMA B operands: step (c, u) holds keys 32c + 16u + [0, 16).
    sa_bf16x8 pb[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pb[0][u][j] = (__bf16)s0[8 * u + j];
        pb[1][u][j] = (__bf16)s1[8 * u + j];
      }
    }

    // ---- O^T += V^T P^T. A operand: V^T[d][keys 32c+16u+4hh+{0..3}, +8+{0..3}].
    const uint16_t* vl = vt_lds[buf];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int kofs = 32 * c + 16 * u + 4 * hh;
        const uint16_t* r0 = vl + col * kRowPad + kofs;
        const uint16_t* r1 = vl + (32 + col) * kRowPad + kofs;
        const sa_u16x4 lo0 = *reinterpret_cast<const sa_u16x4*>(r0);
        const sa_u16x4 hi0 = *reinterpret_cast<const sa_u16x4*>(r0 + 8);
        const sa_u16x4 lo1 = *reinterpret_cast<const sa_u16x4*>(r1);
        const sa_u16x4 hi1 = *reinterpret_cast<const sa_u16x4*>(r1 + 8);
        const sa_u16x8 v0 = {lo0[0], lo0[1], lo0[2], lo0[3], hi0[0], hi0[1], hi0[2], hi0[3]};
        const sa_u16x8 v1 = {lo1[0], lo1[1], lo1[2], lo1[3], hi1[0], hi1[1], hi1[2], hi1[3]};
        acc0 = mfma32(as_bf16x8(v0), pb[c][u], acc0);
        acc1 = mfma32(as_bf16x8(v1), pb[c][u], acc1);
      }
    }

    if (it + 1 < cnt) store_tile<kBias>(k_lds[buf ^ 1], vt_lds[buf ^ 1], b_lds[buf ^ 1], tid, regs);
    __syncthreads();
    kb_cur = kb_next;
  }

  // ---- Epilogue: out = acc / l; each lane half holds a partial l over its keys.
  const float l_tot = l_i + __shfl_xor(l_i, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qrow < a.Lq) {
    uint16_t* orow = obase + (int64_t)qrow * a.o_sl;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      sa_bf16x4 w0, w1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w0[j] = (__bf16)(acc0[4 * g + j] * inv);
        w1[j] = (__bf16)(acc1[4 * g + j] * inv);
      }
      // acc_dc element 4g+j is d = 32dc + 8g + 4hh + j.
      *reinterpret_cast<sa_bf16x4*>(orow + 8 * g + 4 * hh) = w0;
      *reinterpret_cast<sa_bf16x4*>(orow + 32 + 8 * g + 4 * hh) = w1;
    }
  }
}

// One wave per list row: ballot-compact the set entries of mask row (b, h, m).
__global__ __launch_bounds__(256) void mask_to_list_kernel(const uint8_t* __restrict__ mask, int64_t s0,
                                                          int64_t s1, int64_t s2, int64_t s3, int H,
                                                          int nqb, int nkb, int64_t rows,
                                                          int32_t* __restrict__ kv_idx, int max_cnt,
                                                          int32_t* __restrict__ kv_cnt) {
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t bh = row / nqb;
  const int m = (int)(row - bh * nqb);
  const int64_t b = bh / H;
  const int64_t h = bh - b * H;
  const uint8_t* base = mask + b * s0 + h * s1 + (int64_t)m * s2;
  int32_t* out = kv_idx + row * max_cnt;
  int total = 0;
  for (int n0 = 0; n0 < nkb; n0 += 64) {
    const int n = n0 + lane;
    const bool on = n < nkb && base[(int64_t)n * s3] != 0;
    const uint64_t bal = __ballot(on);
    const int pre = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
    if (on) out[total + pre] = n;
    total += __popcll(bal);
  }
  if (lane == 0) kv_cnt[row] = total;
}

}  // namespace

extern "C" int sa_mask_to_kv_list(const uint8_t* mask, const int64_t mask_strides[4], int B, int H,
                                  int nqb, int nkb, int32_t* kv_idx, int max_cnt, int32_t* kv_cnt,
                                  void* stream) {
  SA_REQUIRE(mask && mask_strides && kv_idx && kv_cnt, "sa_mask_to_kv_list: null pointer");
  SA_REQUIRE(B > 0 && H > 0 && nqb > 0 && nkb > 0, "sa_mask_to_kv_list: bad shape B=%d H=%d nqb=%d nkb=%d", B, H, nqb, nkb);
  SA_REQUIRE(max_cnt >= nkb, "sa_mask_to_kv_list: max_cnt=%d < nkb=%d", max_cnt, nkb);
  const int64_t rows = (int64_t)B * H * nqb;
  const int64_t blocks = (rows + 3) / 4;
  SA_REQUIRE(blocks < (1LL << 31), "sa_mask_to_kv_list: too many rows");
  hipLaunchKernelGGL(mask_to_list_kernel, dim3((unsigned)blocks), dim3(256), 0, sa::as_stream(stream), mask,
                     mask_strides[0], mask_strides[1], mask_strides[2], mask_strides[3], H, nqb, nkb, rows,
                     kv_idx, max_cnt, kv_cnt);
  return sa::check_launch("sa_mask_to_kv_list");
}

extern "C" int sa_block_sparse_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                   const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                   uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                   int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                   const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                   void* stream) {
  SA_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides && kv_idx && kv_cnt,
             "sa_block_sparse_fwd: null pointer");
  SA_REQUIRE(B > 0 && H > 0 && Lq > 0 && Lk > 0, "sa_block_sparse_fwd: bad shape B=%d H=%d Lq=%d Lk=%d", B, H, Lq, Lk);
  if (D != kHeadDim) return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_sparse_fwd: head_dim %d (only 64)", D);
  SA_REQUIRE(std::isfinite(sm_scale) && sm_scale > 0.f, "sa_block_sparse_fwd: sm_scale must be finite and > 0");
  const int nqb = sa::cdiv(Lq, kBlock);
  const int nkb = sa::cdiv(Lk, kBlock);
  SA_REQUIRE(max_cnt > 0, "sa_block_sparse_fwd: max_cnt must be > 0");
  SA_REQUIRE(!key_bias || bias_strides, "sa_block_sparse_fwd: key_bias without bias_strides");
  // 16-byte vector accesses: base pointers 16-byte aligned, row strides multiples of 8 elements.
  const void* ptrs[4] = {q, k, v, out};
  for (const void* p : ptrs) {
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_sparse_fwd: tensor base not 16-byte aligned");
  }
  const int64_t* strides[4] = {q_strides, k_strides, v_strides, out_strides};
  for (const int64_t* s : strides) {
    for (int i = 0; i < 3; ++i) {
      if (s[i] % 8 != 0)
        return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_sparse_fwd: strides must be multiples of 8 elements");
    }
  }
  const int64_t grid = (int64_t)B * H * nqb;
  SA_REQUIRE(grid < (1LL << 31), "sa_block_sparse_fwd: grid too large");

  FwdArgs a;
  a.q = q; a.k = k; a.v = v; a.o = out;
  a.q_sb = q_strides[0]; a.q_sh = q_strides[1]; a.q_sl = q_strides[2];
  a.k_sb = k_strides[0]; a.k_sh = k_strides[1]; a.k_sl = k_strides[2];
  a.v_sb = v_strides[0]; a.v_sh = v_strides[1]; a.v_sl = v_strides[2];
  a.o_sb = out_strides[0]; a.o_sh = out_strides[1]; a.o_sl = out_strides[2];
  a.H = H; a.Lq = Lq; a.Lk = Lk; a.nqb = nqb; a.nkb = nkb; a.BH = B * H;
  a.kv_idx = kv_idx; a.kv_cnt = kv_cnt; a.max_cnt = max_cnt;
  a.bias = key_bias;
  a.bias_sb = key_bias ? bias_strides[0] : 0;
  a.bias_sh = key_bias ? bias_strides[1] : 0;
  a.scale_log2 = sm_scale * kLog2e;

  hipStream_t s = sa::as_stream(stream);
  if (key_bias) {
    hipLaunchKernelGGL(bsa_fwd_kernel<true>, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL(bsa_fwd_kernel<false>, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
  }
  return sa::check_launch("sa_block_sparse_fwd");
}
