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
// workgroup holds 4 independent waves (no workgroup barriers) and two workgroups share a
// CU (2 waves per SIMD). Per 64-key tile a wave computes S^T = K Q^T and O^T = V^T P^T
// with v_mfma_f32_32x32x16_bf16 (16 + 16 MFMAs = 1 MFLOP); each lane holds one query
// column of S^T, so row statistics need one cross-half exchange. Plain lists at head dim 128
// run bsa_fwd_pair_kernel instead: two waves of 32 query rows share each block's tiles, so
// that two waves fit a SIMD.
//
// Data movement. An MFMA operand load straight from global memory puts a different row in
// every lane, so each 1 KB load costs the address unit ~64 cache-line lookups; that, not
// bandwidth, bounded the previous design. Here each K and V tile (64 rows x 128 B) is copied
// by 8 coalesced buffer_load ... lds instructions each (8 lanes per 128-byte row) into a
// wave-private LDS buffer with a 16-byte-chunk XOR swizzle, then read as operands: K with
// ds_read_b128, V^T with the transposing ds_read_b64_tr_b16 (V stays [key][d] in memory).
// The swizzle makes both read patterns bank-conflict free. One K and one V buffer per wave:
// the next tile's K is requested as soon as this tile's K operands are in registers, the
// next V as soon as the V operands are, so each copy has a full tile of compute to land.
// Rows past Lk read as zero (the buffer descriptor's size ends at the last row).
//
// Softmax economy: the running max is only raised when a tile exceeds it by more than
// kRescaleLog2 (then p <= 2^kRescaleLog2), so the accumulator rescale is rare; row sums
// accumulate the bf16-rounded P pairs with v_dot2c_f32_bf16; maxima use v_max3_f32. A
// first pass skips the max entirely (bf16: P = exp2(S * scale); fp16, whose P has 5 exponent
// bits: P = exp2(S * scale - m0) with m0 the row's maximum in the item's first tile), exact
// while the row sums stay in range, which is checked; items whose sums leave range are
// redone with the running max.
//
// Scheduling: a host-built work order maps dispatch slots to items so that each XCD
// (workgroups round-robin over 8 XCDs) processes a contiguous range of heads, longest
// (text) rows first.
#include <math.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <type_traits>
#include <vector>

#include "sa_common.h"

namespace {

constexpr int kBlock = 64;       // query rows per block == keys per key block
constexpr int kHeadDim = 64;     // head dimension handled by this kernel
constexpr int kWaves = 4;        // independent waves per workgroup
// Floats per key-range partial: acc [64 rows][kD], row sums [64], row maxima [64].
template <int kD>
constexpr int kSplitFloats = kBlock * kD + 2 * kBlock;
constexpr int kTileBytes = kBlock * kHeadDim * 2;  // one K or V tile: 64 rows x 128 B
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;
// fp16 scores: largest |S * scale_log2| bound (Cauchy-Schwarz of the row norms) for which an
// item uses them, and the squared-norm limit below 65504^2 (the largest fp16 value).
constexpr float kK16Bound = 32.0f;
constexpr float kK16NormMax = 4.0e9f;

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef short sa_i16x4v __attribute__((ext_vector_type(4)));
typedef unsigned sa_u32x4v __attribute__((ext_vector_type(4)));

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
  // Key-range split (n_parts > 1; plain lists only): slot (bh * n_parts + p) * nqb + qb
  // computes list positions [cnt * p / n_parts, cnt * (p + 1) / n_parts) of item bh * nqb + qb
  // and stores its unnormalised partial to ws[item * n_parts + p] (kSplitFloats each: acc
  // [64 rows][kD], then the row sums and the row maxima, log2 domain); split_merge_kernel
  // forms the output. `order` is not read.
  int n_parts;
  float* ws;
  const int32_t* kv_idx;
  const int32_t* kv_cnt;
  int max_cnt;
  const float* bias;
  int64_t bias_sb, bias_sh;
  float sm_scale;
  float scale_log2;  // sm_scale * log2(e)
  int list_bh_stride;          // list row = bh * list_bh_stride + qb (0: lists shared by heads)
  const int32_t* kv_slot;      // [rows][max_cnt] tile-mask slot of each entry, -1 = full tile
  const uint64_t* tile_masks;  // [slots][64] bit k of row r: query r may attend key k
  const int32_t* q_rows;       // [Lq] q row of query i (outside [0, q_src_rows): zeros); null = i
  const int32_t* o_rows;       // [Lq] out row of query i (outside [0, o_dst_rows): dropped); null = i
  int q_src_rows, o_dst_rows;
  int kv_rep;                  // query heads per key/value head (key head of query head h: h / kv_rep)
  // Pooling mode (kPool > 0): per query row, the maximum scaled logit (log2 domain) of every
  // kPool-key column is stored to pool_r[((bh * nqb + row / 64) * pool_ncol + column) * 64 +
  // row % 64] (one query block's maxima are contiguous), and the row's log2-sum-exp2 to
  // pool_lse[bh * pool_lpad + row]; pool_ncol = nkb * 64 / kPool, pool_lpad = nqb * 64.
  float* pool_r;
  int pool_ncol;
  int pool_lpad;
  float* pool_lse;  // null: not stored
  // Fused pooled map (pool_po non-null; pooled block size = kPool): after its item the wave
  // forms the Po rows of its own query rows, Po[i][c] = max over the rows r of query block i
  // of exp2(R[c][r] - lse[r]), each Po row then divided by its sum. Po rows and columns are
  // kPool-token blocks; Po is [B][H][pool_nd][pool_nd] with a unit last stride.
  float* pool_po;
  int64_t po_sb, po_sh, po_si;
  int pool_nd;      // cdiv(Lq, kPool)
  int pool_causal;  // columns past the query's diagonal 64-key tile were never computed: 0
  // fp16 scores (kK16): k16 = fp16 copy of k, contiguous [B*H][Lk][64]; k16_norm2[bh * nkb +
  // kb] = the largest squared row norm of key block kb of head bh (fp32 bits). An item whose
  // bound passes computes S = K16 (fp16(q * scale_log2))^T, already in the exp2 domain.
  const uint16_t* k16;
  const uint32_t* k16_norm2;
};

__device__ inline sa_bf16x8 as_bf16x8(uint4 x) { return __builtin_bit_cast(sa_bf16x8, x); }
__device__ inline sa_bf16x8 as_bf16x8(sa_u32x4v x) { return __builtin_bit_cast(sa_bf16x8, x); }

__device__ inline sa_f32x16 mfma32(sa_bf16x8 a, sa_bf16x8 b, sa_f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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

typedef _Float16 sa_f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 sa_f16x8 __attribute__((ext_vector_type(8)));

// Operand element type of a launch: the MFMA, the rounding of P (and of the output) to the
// element type (round to nearest even), and the row-sum dot of a packed pair with ones.
template <typename T>
struct Elem;
template <>
struct Elem<__bf16> {
  typedef sa_bf16x8 v8;
  __device__ static inline v8 as8(sa_u32x4v x) { return as_bf16x8(x); }
  __device__ static inline sa_f32x16 mfma(v8 a, v8 b, sa_f32x16 c) { return mfma32(a, b, c); }
  __device__ static inline uint32_t pack(float a, float b) { return cvt_pk_bf16(a, b); }
  __device__ static inline float dot2_ones(uint32_t pair, float acc) { return dot2_bf16_ones(pair, acc); }
};
template <>
struct Elem<_Float16> {
  typedef sa_f16x8 v8;
  __device__ static inline v8 as8(sa_u32x4v x) { return __builtin_bit_cast(sa_f16x8, x); }
  __device__ static inline sa_f32x16 mfma(v8 a, v8 b, sa_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack(float a, float b) {  // v_cvt_pk_f16_f32
    const sa_f16x2 r = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ static inline float dot2_ones(uint32_t pair, float acc) {
    const sa_f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(sa_f16x2, pair), ones, acc, false);
  }
};

// max / sum of x over lanes l and l ^ 32 (v_permlane32_swap: no LDS traffic).
__device__ inline float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 16-byte chunk swizzle of LDS tile row r (depends on r mod 16). Chunk c of row r is stored
// at chunk c ^ swz(r). With 64 or 32 LDS banks it makes conflict-free (a) the K operand
// reads, 16 lanes reading 16 consecutive rows at one chunk, and (b) the transposed V reads,
// 32 lanes reading 4 consecutive rows x 4 chunks.
__device__ inline int swz(int r) {
  const int j = (r >> 1) & 7;
  return (((j & 1) << 2) | (j >> 1)) ^ ((r & 1) << 1);
}

__device__ inline sa_u32x4v lds_read_b128(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) sa_u32x4v*>(p);
}
// ds_read_b64_tr_b16: within each 16-lane group, lane i points at 4 consecutive bf16 (row
// i/4, columns 4(i%4)..+3 of a 4 x 16 block); lane j receives column j of that block.
__device__ inline uint2 lds_read_tr16(const lds_u8* p) {
  const sa_i16x4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) sa_i16x4v*)(p));
  return __builtin_bit_cast(uint2, v);
}
typedef unsigned sa_u32x2v __attribute__((ext_vector_type(2)));
// The same read issued as inline assembly: the compiler's wait analysis cannot tell these
// reads from the copies still landing in the other LDS buffers and would otherwise wait for
// all of them; the caller waits for the reads explicitly (lgkm_wait_pair).
template <int kOff>
__device__ inline sa_u32x2v lds_read_tr16_asm(uint32_t addr) {
  sa_u32x2v r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(kOff));
  return r;
}

// Copy one 64-row tile into LDS: instruction i, lane l -> row 8i + l/8 (tile-relative),
// 16-byte slot l of the i-th KB of `dst`. goff[p] = lane offset for rows with (row/8) odd
// (p = 1) or even (p = 0); it holds the swizzle. Offsets at or past `bytes` read as zero.
__device__ inline void dma_tile(const void* base, uint32_t bytes, uint32_t tile_off, uint32_t row_bytes,
                                const uint32_t (&goff)[2], lds_u8* dst) {
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                                                        (int)bytes, 0x00020000);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_u8*)(dst + 1024 * i), 16,
                                             tile_off + 8 * i * row_bytes + goff[i & 1], 0, 0, 0);
}

// dma_tile for a tile of contiguous 128-byte rows (head dim 64, row stride 64 elements): the
// same copies, with the descriptors based at the tile's rows 0 and 32, so that the lane
// offsets stay loop invariant and the instruction offset (added to both the global and the
// LDS address) steps the 8-row groups; no per-tile vector address arithmetic. Each
// descriptor's size ends at the same byte as dma_tile's (0 when row 32 lies past it): a lane
// reads offset goff + 1024 j of the descriptor at off iff off + goff + 1024 j < bytes, so rows
// past Lk read as zero as before.
__device__ inline void dma_tile_c128(const uint16_t* base, uint32_t bytes, uint32_t tile_off,
                                     const uint32_t (&goff)[2], lds_u8* dst) {
#pragma unroll
  for (int hq = 0; hq < 2; ++hq) {
    // Wave-uniform by construction; readfirstlane lets the compiler build the descriptor
    // in scalar registers.
    const uint32_t off = __builtin_amdgcn_readfirstlane(tile_off + 4096u * hq);
    const uint32_t end = __builtin_amdgcn_readfirstlane(bytes);
    const int size = __builtin_amdgcn_readfirstlane(end - min(off, end));
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(reinterpret_cast<const uint8_t*>(base) + off), (short)0, size, 0x00020000);
    lds_u8* d = dst + 4096 * hq;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, d, 16, goff[0], 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, d, 16, goff[1], 0, 1024, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, d, 16, goff[0], 0, 2048, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, d, 16, goff[1], 0, 3072, 0);
  }
}

// Waits until at most n LDS reads are outstanding (n in 0..14, even), tying the wait to
// the two registers it makes valid so that nothing reads them earlier.
__device__ __forceinline__ void lgkm_wait_pair(int n, sa_u32x2v& a, sa_u32x2v& b) {
  switch (n) {
    case 14: asm volatile("s_waitcnt lgkmcnt(14)" : "+v"(a), "+v"(b)); break;
    case 12: asm volatile("s_waitcnt lgkmcnt(12)" : "+v"(a), "+v"(b)); break;
    case 10: asm volatile("s_waitcnt lgkmcnt(10)" : "+v"(a), "+v"(b)); break;
    case 8: asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(a), "+v"(b)); break;
    case 6: asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(a), "+v"(b)); break;
    case 4: asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(a), "+v"(b)); break;
    case 2: asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(a), "+v"(b)); break;
    default: asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b) : : "memory"); break;
  }
}

// s_waitcnt encodings (gfx9): vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int kWaitLgkm0 = 0xC07F;

// T: bf16 or fp16 operands (and output). kD: head dim 64 or 128. A 128-dim row is staged as
// two 128-byte half rows in two half tiles with the 64-dim layout, so every read pattern of
// the 64-dim kernel applies per half; at 128 dims a wave holds ~350 registers, so one
// workgroup (one wave per SIMD) runs per CU. (Plain head-dim-128 lists without key-range
// parts run bsa_fwd_pair_kernel; this kernel serves their bias, tile-mask, pooling and split
// launches.)
// kDV: value columns that enter P.V and the output, kD or 32 (head dim 64: v tiles are
// copied as usual and only their first 32 columns are read; out has 32 columns).
template <bool kBias, bool kMask, int kPool, typename T = __bf16, int kD = 64, int kDV = kD, bool kK16 = false>
__global__ __launch_bounds__(256, kD == 64 ? 2 : 1) void bsa_fwd_kernel(FwdArgs a) {
  static_assert(!kK16 || (!kMask && kPool == 0 && std::is_same<T, __bf16>::value && kD == 64 && kDV == 64),
                "fp16 scores: plain or key-bias bf16 lists at head dim 64");
  // With fp16 scores the key bias arrives multiplied by log2(e) (the entry point's scaled copy).
  constexpr bool kBiasLog2 = kK16;
  static_assert(kPool == 0 || ((kPool == 32 || kPool == 64) && !kBias), "pooling: 32- or 64-key columns, no bias");
  static_assert(kD == 64 || kD == 128, "head dim 64 or 128");
  static_assert(kDV == kD || (kDV == 32 && kD == 64 && kPool == 0 && !kMask), "32 value columns: head dim 64");
  typedef Elem<T> E;
  constexpr int kDS = kD / 16;     // 16-wide d steps of S = K Q^T
  constexpr int kDC = kDV / 32;    // 32-row d chunks of O^T
  constexpr int kHalves = kD / 64;  // 128-byte half rows per token
  constexpr int kVC = kDC / kHalves;  // d chunks of O^T per 128-byte half row of v
  // Separate LDS objects for K, V and bias so that the compiler's own wait analysis can
  // tell a copy into one from a read of another.
  __shared__ __attribute__((aligned(1024))) uint8_t k_lds[kWaves * kTileBytes * kHalves];
  __shared__ __attribute__((aligned(1024))) uint8_t v_lds[kWaves * kTileBytes * kHalves];
  // Bias rows: three 64-key slots per wave (list positions of even and odd index, and a slot
  // for the copies issued past the end of the list, which nothing reads).
  __shared__ __attribute__((aligned(16))) float b_lds[kBias ? kWaves * 3 * kBlock : 4];
  // Tile-mask rows of the tile in flight (64 words per wave), copied like K and V.
  __shared__ __attribute__((aligned(16))) uint64_t m_lds[kMask ? kWaves * kBlock : 2];
  // Vector-memory operations per tile, in issue order: group K = [mask rows (2 copies into
  // LDS, cut tiles only)] [K (8 per half)], group V = [bias of the next tile (1)] [V (8 per
  // half)]. The waits below count them.
  constexpr int kGroupK = 8 * kHalves + (kMask ? 2 : 0);
  constexpr int kGroupV = 8 * kHalves + (kBias ? 1 : 0);

  const int lane = threadIdx.x & 63;
  // Wave-uniform values are made provably uniform (readfirstlane) so that the list, slot
  // and order reads are scalar loads, which leave the vector-memory counter alone.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31;  // query column within a 32-row group (MFMA n index)
  const int hh = lane >> 5;   // lane half (MFMA k group)
  const int slot = blockIdx.x * kWaves + wave;
  if (slot >= a.n_slots) return;
  // Key-range parts exist for plain lists only; the other variants compile without them.
  constexpr bool kSplit = !kBias && !kMask && kPool == 0 && kDV == kD && !kK16;
  const bool split = kSplit && a.n_parts > 1;
  int item, part = 0;
  if (split) {
    const int per_bh = a.n_parts * a.nqb;
    const int bh_s = slot / per_bh;
    const int rem = slot - bh_s * per_bh;
    part = rem / a.nqb;
    item = bh_s * a.nqb + (rem - part * a.nqb);
  } else {
    item = __builtin_amdgcn_readfirstlane(a.order ? a.order[slot] : slot);
  }
  if (item < 0 || item >= a.n_items) return;  // idle slot (no workgroup barriers below)
  const int bh = item / a.nqb;
  const int qb = item - bh * a.nqb;
  const int b = bh / a.H;
  const int h = bh - b * a.H;

  const int64_t list_row = (int64_t)bh * a.list_bh_stride + qb;
  int cnt = a.kv_cnt[list_row];
  cnt = cnt < 0 ? 0 : (cnt > a.max_cnt ? a.max_cnt : cnt);
  int beg = 0;  // list positions [beg, cnt) of this wave
  if (split) {
    beg = cnt * part / a.n_parts;
    cnt = cnt * (part + 1) / a.n_parts;
  }
  __builtin_assume(beg >= 0);
  // Constant address space: the compiler may use scalar loads (nothing here writes them).
  const __attribute__((address_space(4))) int32_t* list =
      (const __attribute__((address_space(4))) int32_t*)(a.kv_idx + list_row * a.max_cnt);
  const __attribute__((address_space(4))) int32_t* slots =
      kMask ? (const __attribute__((address_space(4))) int32_t*)(a.kv_slot + list_row * a.max_cnt) : nullptr;

  const uint16_t* qbase = a.q + b * a.q_sb + h * a.q_sh;
  const int hk = a.kv_rep > 1 ? h / a.kv_rep : h;
  const uint16_t* khead = a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vhead = a.v + b * a.v_sb + hk * a.v_sh;
  uint16_t* obase = a.o + b * a.o_sb + h * a.o_sh;
  const float* bhead = kBias ? a.bias + b * a.bias_sb + h * a.bias_sh : nullptr;
  uint32_t krow = (uint32_t)(a.k_sl * 2);
  const uint32_t vrow = (uint32_t)(a.v_sl * 2);
  uint32_t kbytes = (uint32_t)(a.Lk - 1) * krow + 2 * kHeadDim;
  const uint32_t vbytes = (uint32_t)(a.Lk - 1) * vrow + 2 * kHeadDim;
  bool c128 = krow == 128 && vrow == 128;  // contiguous d = 64 rows: dma_tile_c128
  lds_u8* kl = (lds_u8*)k_lds + wave * kTileBytes * kHalves;
  lds_u8* vl = (lds_u8*)v_lds + wave * kTileBytes * kHalves;
  float* bl_lds = b_lds + (kBias ? wave * 3 * kBlock : 0);

  // Lane constants: copy offsets, K operand read offsets, V^T transposed read offsets.
  uint32_t kgo[2], vgo[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int r = 8 * p + (lane >> 3);
    const int chunk = (lane & 7) ^ swz(r);
    kgo[p] = (lane >> 3) * krow + 16 * chunk;
    vgo[p] = (lane >> 3) * vrow + 16 * chunk;
  }
  // K A-operand of (key chunk c, d-step s): K[32c + col][16s + 8hh .. +7] = row 32c + col,
  // chunk 2s + hh (+ 4096 c).
  int kro[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) kro[s] = 128 * col + 16 * ((2 * s + hh) ^ swz(col));
  // V^T A-operand of (d-chunk dc, key step 32c + 16u): two transposed reads t = 0, 1 of rows
  // 32c + 16u + 8t + 4hq + 0..3 at d = 32dc + 16dg + 4(i%4) (lane = 16(2hq + dg) + i); lane
  // 16(2hq + dg) + j receives d = 32dc + 16dg + j, keys 16u + 8t + 4hq + 0..3, the key slots
  // of the P^T B operand (S^T rows 8(e/4) + 4hh + e%4).
  int vro[2][2];
  {
    const int i = lane & 15, g4 = lane >> 4;
    const int hq = g4 >> 1, dg = g4 & 1;
#pragma unroll
    for (int dc = 0; dc < 2; ++dc)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = 8 * t + 4 * hq + (i >> 2);
        const int chunk = 4 * dc + 2 * dg + ((i & 3) >> 1);
        vro[dc][t] = 128 * r + 16 * (chunk ^ swz(r)) + 8 * (i & 1);
      }
  }

  // Q^T B operands: qf[g][s] = q[qb*64 + 32g + col][16s + 8hh .. +7] (rows clamped into Lq;
  // clamped rows are never stored). With a row map, query i reads q row q_rows[i] (zeros
  // when that is outside the tensor: padding rows of a remapped layout).
  typename E::v8 qf[2][kDS];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    int row = min(qb * kBlock + 32 * g + col, a.Lq - 1);
    bool zero = false;
    if (a.q_rows) {
      row = a.q_rows[row];
      zero = (unsigned)row >= (unsigned)a.q_src_rows;
      row = zero ? 0 : row;
    }
    const uint16_t* p = qbase + (int64_t)row * a.q_sl + 8 * hh;
#pragma unroll
    for (int s = 0; s < kDS; ++s) {
      const uint4 w = *reinterpret_cast<const uint4*>(p + 16 * s);
      qf[g][s] = __builtin_bit_cast(typename E::v8, zero ? make_uint4(0u, 0u, 0u, 0u) : w);
    }
  }

  sa_f32x16 acc[kDC][2];  // [dc][g]
  float m[2];
  float l[2];

  // An entry outside [0, nkb) copies block 0 and is masked out entirely.
  auto entry = [&](int it) -> int { return it < cnt ? list[it] : -1; };
  auto block_ok = [&](int kb) { return (unsigned)kb < (unsigned)a.nkb; };
  int mslot = -1;  // mask slot of the tile in flight (-1: not cut)
  // Group K of tile `kb` (list position it): mask rows, K copy.
  auto issue_k = [&](int kb, int it) {
    const uint32_t kb0 = block_ok(kb) ? (uint32_t)kb * kBlock : 0u;
    if (kMask) {
      mslot = it < cnt ? slots[it] : -1;
      if (mslot >= 0) {  // the 512 bytes of a cut tile's rows, two 4-byte copies per lane
        const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint64_t*>(a.tile_masks + (int64_t)mslot * kBlock), (short)0, kBlock * 8, 0x00020000);
        lds_u8* md = (lds_u8*)(m_lds + (kMask ? wave * kBlock : 0));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, md, 4, lane * 4, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, md, 4, lane * 4, 0, 256, 0);
      }
    }
    if (kD == 64 && c128) {
      dma_tile_c128(khead, kbytes, kb0 * krow, kgo, kl);
    } else {
#pragma unroll
      for (int hf = 0; hf < kHalves; ++hf)
        dma_tile(khead + 64 * hf, kbytes, kb0 * krow, krow, kgo, kl + hf * kTileBytes);
    }
  };
  // Bias copy of list position `it` (keys past Lk read as zero) into slot it % 2, or into
  // the unread slot 2 past the end of the list.
  auto issue_bias = [&](int it) {
    const int kb = entry(it);
    const uint32_t kb0 = block_ok(kb) ? (uint32_t)kb * kBlock : 0u;
    const int bslot = it < cnt ? (it & 1) : 2;
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(bhead), (short)0,
                                                                        a.Lk * 4, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_u8*)(bl_lds + bslot * kBlock), 4, (kb0 + lane) * 4, 0, 0, 0);
  };
  // Group V of tile `kb` (list position it): the bias copy of position it + 1 (two tiles
  // ahead of its use, so it has landed when the tile's K copy is waited for), V copy.
  auto issue_v = [&](int kb, int it) {
    const uint32_t kb0 = block_ok(kb) ? (uint32_t)kb * kBlock : 0u;
    if (kBias) issue_bias(it + 1);
    if (kD == 64 && c128) {
      dma_tile_c128(vhead, vbytes, kb0 * vrow, vgo, vl);
    } else {
#pragma unroll
      for (int hf = 0; hf < kHalves; ++hf)
        dma_tile(vhead + 64 * hf, vbytes, kb0 * vrow, vrow, vgo, vl + hf * kTileBytes);
    }
  };

  // fp16 scores: the item takes them when max |q_i * scale_log2| * max |k_j| (largest row
  // norms of its query rows and of the head's keys) is at most kK16Bound, which bounds every
  // |S * scale_log2| of the item by Cauchy-Schwarz, and both squared norms are below
  // kK16NormMax, so no element reaches the fp16 range limit. k16 then equals k from 2^-17 up
  // (smaller elements move by at most 2^-25) and fp16(q * scale_log2) has a relative error of
  // at most 2^-11 per element (absolute 2^-25 below fp16's normal range): each logit moves by
  // about 2^-11 * kK16Bound at most in the exp2 domain. Otherwise (or with a NaN) the item runs
  // on the bf16 operands. The item's first K tile (from k16) and V tile are requested before the
  // bound is known; an item that fails it waits for them and starts again from k.
  bool use16 = false;
  bool issued16 = false;  // the first copies of the fp16 pass are in flight
  if constexpr (kK16) {
    // The head's largest squared key norm: its block norms, 64 per load, maximum over the wave
    // (loaded before the copies below, which the loop's wait counts then find alone in flight).
    const uint32_t* bn = a.k16_norm2 + (int64_t)bh * a.nkb;
    uint32_t kmax = 0u;
    for (int j0 = 0; j0 < a.nkb; j0 += 256) {
      uint32_t v4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v4[u] = bn[min(j0 + 64 * u + lane, a.nkb - 1)];  // clamped: the maximum is unchanged
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) kmax = max(kmax, v4[u]);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
    const uint16_t* const k_bf = khead;
    const uint32_t krow_bf = krow, kbytes_bf = kbytes, kgo_bf[2] = {kgo[0], kgo[1]};
    const bool c128_bf = c128;
    khead = a.k16 + (int64_t)bh * a.Lk * kHeadDim;
    krow = 2 * kHeadDim;
    kbytes = (uint32_t)a.Lk * krow;
    c128 = vrow == 128;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int r = 8 * p + (lane >> 3);
      kgo[p] = (lane >> 3) * krow + 16 * ((lane & 7) ^ swz(r));
    }
    if (cnt > beg) {  // the first copies of run(), in its order
      const int kb0 = entry(beg);
      if (kBias) issue_bias(beg);
      issue_k(kb0, beg);
      issue_v(kb0, beg);
      issued16 = true;
    }
    const float qs = a.scale_log2;
    float n2[2] = {0.f, 0.f};
    uint32_t h16[2][kDS][4];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int s = 0; s < kDS; ++s) {
        const sa_u32x4v w = __builtin_bit_cast(sa_u32x4v, qf[g][s]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x0 = __uint_as_float(w[i] << 16) * qs, x1 = __uint_as_float(w[i] & 0xffff0000u) * qs;
          n2[g] = fmaf(x1, x1, fmaf(x0, x0, n2[g]));
          h16[g][s][i] = Elem<_Float16>::pack(x0, x1);
        }
      }
    float qn2 = fmaxf(xhalf_sum(n2[0]), xhalf_sum(n2[1]));  // rows 32g + col of the lane's column
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) qn2 = fmaxf(qn2, __shfl_xor(qn2, o));
    qn2 = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(qn2)));  // equal in every lane
    const float kn2 = __uint_as_float(__builtin_amdgcn_readfirstlane(kmax));
    use16 = qn2 < kK16NormMax && kn2 < kK16NormMax && qn2 * kn2 <= kK16Bound * kK16Bound;
    if (use16) {
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int s = 0; s < kDS; ++s)
          qf[g][s] = __builtin_bit_cast(typename E::v8, sa_u32x4v{h16[g][s][0], h16[g][s][1], h16[g][s][2], h16[g][s][3]});
    } else {
      // The requested copies land before the bf16 pass requests its own into the same buffers.
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      issued16 = false;
      khead = k_bf;
      krow = krow_bf;
      kbytes = kbytes_bf;
      c128 = c128_bf;
      kgo[0] = kgo_bf[0];
      kgo[1] = kgo_bf[1];
    }
  }

  // One pass over the item's key blocks. Fast pass (kSafe = false): P = exp2(S) with no
  // max subtraction. Softmax is invariant to a common factor, and bf16 P keeps fp32's
  // exponent range, so this equals the max-subtracted result as long as the scores stay in
  // range; the caller checks the row sums afterwards and redoes the item with the safe pass
  // (running max, lazy rescale) otherwise.
  auto run = [&](auto safe_tag, auto k16_tag, bool first_issued) __attribute__((always_inline)) {
    constexpr bool kSafe = decltype(safe_tag)::value;
    constexpr bool kQ16 = decltype(k16_tag)::value;  // fp16 K and pre-scaled q: S in the exp2 domain
    // fp16 P keeps 5 exponent bits, so its fast pass subtracts a fixed per-row offset.
    constexpr bool kOffset = !kSafe && !std::is_same<T, __bf16>::value;
#pragma unroll
    for (int dc = 0; dc < kDC; ++dc)
#pragma unroll
      for (int g = 0; g < 2; ++g) acc[dc][g] = sa_f32x16{};
    m[0] = m[1] = -INFINITY;
    l[0] = l[1] = 0.f;
    int it = beg;
    int kb = entry(beg);
    if (cnt > beg && !first_issued) {  // (the fp16 fast pass requested its first tile above)
      if (kBias) issue_bias(beg);
      issue_k(kb, beg);
      issue_v(kb, beg);
    }
    if constexpr (kMask) {
      // The group K size varies with the tiles (mask rows of cut tiles only), and the
      // compiler's wait analysis then carries the Q operand loads into the loop, where it
      // would wait for every copy in flight before the first MFMA of each tile. Wait for them
      // here (everything older than the prologue's copies) and redefine the Q registers
      // after the wait, so that the loop sees no load behind them.
      if (cnt > beg) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kGroupK - 2 + kGroupV));
      else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int s = 0; s < kDS; ++s) asm volatile("" : "+v"(qf[g][s]));
    }
    while (it < cnt) {
      // Past the end of the list the copies re-load the current block, so every iteration
      // has the same operations in flight.
      const int it_next = it + 1 < cnt ? it + 1 : it;
      const int kb_next = entry(it_next);
      const int nvalid = block_ok(kb) ? min(kBlock, a.Lk - kb * kBlock) : 0;
      const int mslot_cur = mslot;

      // ---- K operands of this tile, then request the next tile's group K.
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kGroupV));
      // This tile's mask rows (group K, landed by the wait above), read before the next
      // tile's group K reuses the buffer.
      uint64_t mw_cur[2] = {~0ull, ~0ull};
      if (kMask && mslot_cur >= 0) {
        const uint64_t* mr = m_lds + (kMask ? wave * kBlock : 0);
        mw_cur[0] = mr[col];
        mw_cur[1] = mr[32 + col];
      }
      sa_u32x4v kop[2][kDS];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s = 0; s < kDS; ++s) kop[c][s] = lds_read_b128(kl + (s >> 2) * kTileBytes + kro[s & 3] + 4096 * c);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      issue_k(kb_next, it_next);

      // ---- S^T = K Q^T: S[g][c] element e is key 32c + 8(e/4) + 4hh + e%4, query 32g + col.
      // fp16 scores with a key bias: the MFMA chains start from the tile's biases (log2 units),
      // so S = K (q * scale_log2)^T + bias * log2(e) takes no VALU at all.
      sa_f32x16 bias0[2] = {};
      if constexpr (kQ16 && kBias) {
        // This tile's bias copy was issued before the previous tile's V copy, so the wait for
        // this tile's K copy at the top covered it.
        const float* bt = bl_lds + (it & 1) * kBlock;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const float4 b4 = *reinterpret_cast<const float4*>(bt + 32 * c + 8 * q4 + 4 * hh);
            bias0[c][4 * q4] = b4.x;
            bias0[c][4 * q4 + 1] = b4.y;
            bias0[c][4 * q4 + 2] = b4.z;
            bias0[c][4 * q4 + 3] = b4.w;
          }
      }
      sa_f32x16 S[2][2];

#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          sa_f32x16 t = bias0[c];
#pragma unroll
          for (int s = 0; s < kDS; ++s) {
            if constexpr (kQ16)
              t = Elem<_Float16>::mfma(Elem<_Float16>::as8(kop[c][s]), __builtin_bit_cast(sa_f16x8, qf[g][s]), t);
            else
              t = E::mfma(E::as8(kop[c][s]), qf[g][s], t);
          }
          S[g][c] = t;
        }
      
      if (kBias && !kQ16) {  // S = (s * sm_scale + bias) * log2(e), the exp2 domain
        // This tile's bias copy was issued before the previous tile's V copy, so the wait for
        // this tile's K copy at the top covered it.
        const float* bt = bl_lds + (it & 1) * kBlock;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const float4 b4 = *reinterpret_cast<const float4*>(bt + 32 * c + 8 * q4 + 4 * hh);
            const float bq[4] = {kBiasLog2 ? b4.x : b4.x * kLog2e, kBiasLog2 ? b4.y : b4.y * kLog2e,
                                 kBiasLog2 ? b4.z : b4.z * kLog2e, kBiasLog2 ? b4.w : b4.w * kLog2e};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              S[0][c][4 * q4 + j] = fmaf(S[0][c][4 * q4 + j], a.scale_log2, bq[j]);
              S[1][c][4 * q4 + j] = fmaf(S[1][c][4 * q4 + j], a.scale_log2, bq[j]);
            }
          }
      }
      if (nvalid < kBlock) {  // keys past Lk, or an entry outside the grid
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            if (32 * c + 8 * (e >> 2) + 4 * hh + (e & 3) >= nvalid) {
              S[0][c][e] = -INFINITY;
              S[1][c][e] = -INFINITY;
            }
          }
      }
      if (kMask && mslot_cur >= 0) {  // token-level mask of a tile cut by a mask boundary
        // Element e of S[g][c] is key 32c + 8(e/4) + 4hh + e%4: its bit, sign-extended to
        // 0 or all ones (v_bfe_i32), selects between the score and -inf (v_bfi_b32).
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int bits = (int)((uint32_t)(mw_cur[g] >> (32 * c)) >> (4 * hh));
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const uint32_t keep = (uint32_t)__builtin_amdgcn_sbfe(bits, 8 * (e >> 2) + (e & 3), 1);
              S[g][c][e] = __uint_as_float((__float_as_uint(S[g][c][e]) & keep) | (0xFF800000u & ~keep));
            }
          }
      }

      // ---- P = exp2(S * sc - m) in bf16 and the row sums (m = 0 in the fast pass).
      const float sc = (kBias || kQ16) ? 1.f : a.scale_log2;  // S is already scaled (bias, fp16 scores)
      if constexpr (kPool != 0) {
        // Row maxima of the scaled logits per kPool-key column. Lane l stores row
        // qb * 64 + l (query group hh, column col): one 256-byte store per column.
        if (block_ok(kb)) {
          constexpr int kCols = kBlock / kPool;  // columns per tile: 2 (32-key) or 1 (64-key)
          float* rp = a.pool_r + (((int64_t)bh * a.nqb + qb) * a.pool_ncol + kb * kCols) * kBlock + lane;
#pragma unroll
          for (int cc = 0; cc < kCols; ++cc) {
            float mx[2];
#pragma unroll
            for (int g = 0; g < 2; ++g) {
              float x = -INFINITY;
#pragma unroll
              for (int c = (kCols == 2 ? cc : 0); c < (kCols == 2 ? cc + 1 : 2); ++c)
#pragma unroll
                for (int e = 0; e < 16; ++e) x = fmaxf(x, S[g][c][e]);
              mx[g] = xhalf_max(x) * sc;  // sc > 0: max(S) * sc = max(S * sc)
            }
            rp[cc * kBlock] = hh ? mx[1] : mx[0];
          }
        }
      }
      float mu[2] = {0.f, 0.f};
      // Row max of this tile's scaled scores (sc > 0: max(S) * sc = max(S * sc)).
      auto tile_row_max = [&](int g) {
        float mx = fmaxf(fmaxf(S[g][0][0], S[g][0][1]), S[g][0][2]);
#pragma unroll
        for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, S[g][0][e]), S[g][0][e + 1]);
        mx = fmaxf(fmaxf(mx, S[g][0][15]), S[g][1][0]);
#pragma unroll
        for (int e = 1; e < 15; e += 2) mx = fmaxf(fmaxf(mx, S[g][1][e]), S[g][1][e + 1]);
        mx = fmaxf(mx, S[g][1][15]);
        return xhalf_max(mx) * sc;
      };
      if (kOffset) {
        // fp16 fast pass: the first tile's row maxima are the exp2 offsets of the whole item.
        if (it == beg) {
#pragma unroll
          for (int g = 0; g < 2; ++g) m[g] = tile_row_max(g);
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) mu[g] = (m[g] == -INFINITY) ? 0.f : m[g];
      }
      if (kSafe) {
        // Row max; the running max is raised only when this tile exceeds it by more than
        // the threshold (always on the first tile, where m = -inf).
        float cand[2];
        bool raise = false;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          cand[g] = tile_row_max(g);
          raise |= cand[g] > m[g] + kRescaleLog2;
        }
        if (__ballot(raise) != 0) {
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            const float m_new = fmaxf(m[g], cand[g]);
            // 0 when m = -inf; a row with no key yet (m_new = -inf: every key so far masked, while
            // another row of the wave raised its maximum) has nothing to rescale.
            const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m[g] - m_new);
            m[g] = m_new;
            l[g] *= alpha;
#pragma unroll
            for (int dc = 0; dc < kDC; ++dc) acc[dc][g] *= alpha;
          }
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) mu[g] = (m[g] == -INFINITY) ? 0.f : m[g];
      }
      // In the order the S MFMA chains complete (c outer): the first softmax work needs only
      // the first half of the S MFMAs. Each row sum l[g] still adds its pairs c-major.
      uint32_t P[2][2][8];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            const float p0 = fast_exp2(kSafe || kOffset ? fmaf(S[g][c][e], sc, -mu[g]) : S[g][c][e] * sc);
            const float p1 = fast_exp2(kSafe || kOffset ? fmaf(S[g][c][e + 1], sc, -mu[g]) : S[g][c][e + 1] * sc);
            P[g][c][e >> 1] = E::pack(p0, p1);
            l[g] = E::dot2_ones(P[g][c][e >> 1], l[g]);
          }

      // ---- V^T operands of this tile, then request the next tile's V.
      // The next tile's group K holds its two mask-row copies only if that tile is cut.
      if (kMask && mslot < 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kGroupK - 2));
      else __builtin_amdgcn_s_waitcnt(waitcnt_vm(kGroupK));
      // The reads are issued in the order the P·V MFMAs consume them, and each MFMA pair
      // waits only for its own two reads (LDS reads return in order; the full wait first
      // leaves no scalar load outstanding, so the counts are exact). The next tile's V
      // copy overwrites this buffer, so it is requested after the last read has landed.
      // At 128 dims each half tile (d chunks 2hp, 2hp + 1) is read and consumed in turn.
#pragma unroll
      for (int hp = 0; hp < kHalves; ++hp) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        sa_u32x2v vr[2][2][2][2];  // [c][u][dc][t]
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int dc = 0; dc < kVC; ++dc)
#pragma unroll
              for (int t = 0; t < 2; ++t) {
                const uint32_t base = (uint32_t)(uintptr_t)(vl + hp * kTileBytes + vro[dc][t]);
                vr[c][u][dc][t] = (c == 0 ? (u == 0 ? lds_read_tr16_asm<0>(base) : lds_read_tr16_asm<2048>(base))
                                          : (u == 0 ? lds_read_tr16_asm<4096>(base) : lds_read_tr16_asm<6144>(base)));
              }

        // ---- O^T += V^T P^T over the tile's four 16-key steps.
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int dc = 0; dc < kVC; ++dc) {
              constexpr int kReads = 8 * kVC;
              const int done = 2 * ((c * 2 + u) * kVC + dc) + 2;  // reads this MFMA pair needs
              lgkm_wait_pair(kReads - done, vr[c][u][dc][0], vr[c][u][dc][1]);
              const sa_u32x4v vop = {vr[c][u][dc][0].x, vr[c][u][dc][0].y, vr[c][u][dc][1].x, vr[c][u][dc][1].y};
#pragma unroll
              for (int g = 0; g < 2; ++g)
                acc[kVC * hp + dc][g] = E::mfma(E::as8(vop),
                                              E::as8(sa_u32x4v{P[g][c][4 * u], P[g][c][4 * u + 1], P[g][c][4 * u + 2],
                                                               P[g][c][4 * u + 3]}),
                                              acc[kVC * hp + dc][g]);
            }
      }
      issue_v(kb_next, it + 1);

      it = it + 1;
      kb = kb_next;
    }
    // The copies requested after the last tile land in this wave's LDS: wait for them
    // before the LDS is read again or the wave ends.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  };

  auto run_item = [&](auto safe_tag, bool first_issued) __attribute__((always_inline)) {
    if constexpr (kK16) {
      if (use16) run(safe_tag, std::true_type{}, first_issued);
      else run(safe_tag, std::false_type{}, false);
    } else {
      run(safe_tag, std::false_type{}, false);
    }
  };
  run_item(std::false_type{}, issued16);
  // The fast pass is exact unless a row's sum left [2^-90, 2^90] (bf16: scores far from 0,
  // where exp2 would lose range; fp16: a later tile's P at or above 2^16 times the largest P of
  // the first tile, where fp16 P rounds to inf) or an accumulator overflowed; then redo the
  // item safely.
  if (cnt > beg) {
    bool bad = false;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const float l_tot = xhalf_sum(l[g]);
      bad |= !(l_tot >= 0x1p-90f && l_tot <= 0x1p90f);
      float amax = 0.f;
#pragma unroll
      for (int dc = 0; dc < kDC; ++dc)
#pragma unroll
        for (int e = 0; e < 16; e += 2) amax = fmaxf(fmaxf(amax, fabsf(acc[dc][g][e])), fabsf(acc[dc][g][e + 1]));
      bad |= !(amax <= 3.0e38f);
    }
    if (__ballot(bad) != 0) run_item(std::true_type{}, false);
  }

  // ---- Epilogue: out = acc / l (each lane half holds a partial l of its keys).
  float row_lse = 0.f;  // pooling: log2-sum-exp2 of row qb * 64 + lane
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float l_tot = xhalf_sum(l[g]);
    if (split) {  // partial of a key-range part: acc, row sum, row max (0 in the fast pass)
      float* w = a.ws + ((int64_t)item * a.n_parts + part) * kSplitFloats<kD>;
      const int r = 32 * g + col;
#pragma unroll
      for (int dc = 0; dc < kDC; ++dc)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const sa_f32x16& A = acc[dc][g];
          *reinterpret_cast<float4*>(w + r * kD + 32 * dc + 8 * q4 + 4 * hh) =
              make_float4(A[4 * q4], A[4 * q4 + 1], A[4 * q4 + 2], A[4 * q4 + 3]);
        }
      if (hh == 0) {
        w[kBlock * kD + r] = l_tot;
        w[kBlock * kD + kBlock + r] = m[g] == -INFINITY ? 0.f : m[g];
      }
      continue;
    }
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if constexpr (kPool != 0) {
      // log2-sum-exp2 of the row: P = exp2(S * sc - m) / l_tot (m = -inf: the fast pass, 0).
      if (g == hh) {
        row_lse = (m[g] == -INFINITY ? 0.f : m[g]) + log2f(l_tot);
        if (a.pool_lse) a.pool_lse[(int64_t)bh * a.pool_lpad + qb * kBlock + lane] = row_lse;
      }
    }
    int row = qb * kBlock + 32 * g + col;
    bool store = row < a.Lq;
    if (store && a.o_rows) {  // remapped layout: query i goes to out row o_rows[i]
      row = a.o_rows[row];
      store = (unsigned)row < (unsigned)a.o_dst_rows;
    }
    if (store) {
      uint16_t* orow = obase + (int64_t)row * a.o_sl;
#pragma unroll
      for (int dc = 0; dc < kDC; ++dc) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const sa_f32x16& A = acc[dc][g];
          // element 4q4 + j is d = 32dc + 8q4 + 4hh + j
          *reinterpret_cast<uint2*>(orow + 32 * dc + 8 * q4 + 4 * hh) =
              make_uint2(E::pack(A[4 * q4] * inv, A[4 * q4 + 1] * inv), E::pack(A[4 * q4 + 2] * inv, A[4 * q4 + 3] * inv));
        }
      }
    }
  }

  if constexpr (kPool != 0) {
    if (a.pool_po) {
      // Fused pooled map. Lane l reads back the maxima it stored for row qb * 64 + l
      // (R[c][l] at pool_r[... + c * 64 + l]: its own stores, so program order makes them
      // visible). Po row of the lane: query block qb (64-row blocks) or 2 qb + hh (32-row
      // blocks: each lane half is one Po row). Per chunk of 32 columns every lane forms
      // x[j] = exp2(R - lse) (0 for rows past Lq and columns never computed), and a
      // butterfly over the 32 lanes of each half takes the maxima: at the stage of offset
      // o the lane keeps the half of its o * 2 values selected by lane bit o and takes the
      // maximum with its partner's copy of that half, so lane l ends with column l & 31
      // (a last exchange across the halves for 64-row blocks). One store per chunk writes
      // the row's 32 columns; a second pass divides the row by its sum, reading back the
      // same lanes' own stores.
      constexpr int kCols = kBlock / kPool;  // columns per 64-key tile
      const bool row_ok = qb * kBlock + lane < a.Lq;
      const int ncol = a.pool_nd;
      const int cend = a.pool_causal ? min(ncol, (qb + 1) * kCols) : ncol;
      const float* rb = a.pool_r + ((int64_t)bh * a.nqb + qb) * a.pool_ncol * kBlock + lane;
      const int pr = qb * kCols + (kCols == 2 ? hh : 0);
      const bool writer = pr < a.pool_nd && (kCols == 2 || hh == 0);
      float* po = a.pool_po + b * a.po_sb + h * a.po_sh + (int64_t)min(pr, a.pool_nd - 1) * a.po_si;
      const int j_lane = lane & 31;
      float tot = 0.f;  // this lane's columns, then summed over the 32 lanes
      for (int c0 = 0; c0 < ncol; c0 += 32) {
        // Every load is issued (at a computed column, clamped) before any is used.
        float x[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) x[j] = rb[(int64_t)min(c0 + j, cend - 1) * kBlock];
#pragma unroll
        for (int j = 0; j < 32; ++j)
          x[j] = __builtin_amdgcn_exp2f(((c0 + j < cend && row_ok) ? x[j] : -INFINITY) - row_lse);
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) {
          const bool up = (lane & o) != 0;
#pragma unroll
          for (int i = 0; i < o; ++i) {
            const float send = up ? x[i] : x[i + o];
            const float keep = up ? x[i + o] : x[i];
            x[i] = fmaxf(keep, __shfl_xor(send, o));
          }
        }
        float vmax = x[0];  // column c0 + (lane & 31)
        if (kCols == 1) vmax = fmaxf(vmax, __shfl_xor(vmax, 32));
        tot += vmax;
        if (writer && c0 + j_lane < ncol) po[c0 + j_lane] = vmax;
      }
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) tot += __shfl_xor(tot, o);
      if (writer) {
        for (int c = j_lane; c < ncol; c += 32) po[c] = po[c] / tot;
      }
    }
  }
}


// Workgroup barrier with no memory fence: the waits before it are explicit (a fence would
// also wait for the copies in flight). The clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Head dim 128, plain lists: one query block per workgroup of two waves (a wave pair). Wave g
// holds query rows 32g .. 32g + 31 of the block: its Q^T operands, O^T accumulators and S^T
// take half the registers of a 64-row wave (216 VGPRs against ~350), so two waves run per
// SIMD where bsa_fwd_kernel fits one. The pair shares one K and one V tile in LDS, and wave g
// copies the 128-byte half rows of d half g of each (the half tiles of bsa_fwd_kernel). Four
// workgroup barriers per tile order the copies and the reads: K landed, K read (the K buffer
// may be refilled), V landed, V read. Same operations per sum in the same order as
// bsa_fwd_kernel: bit-identical outputs. (At head dim 64 the same scheme, three waves per
// SIMD, was slower than bsa_fwd_kernel's two 64-row waves.)
// Slots: the four slots of dispatch group w (the work order's unit, placed on XCD w % 8)
// go to the workgroups x = 32 (w / 8) + 8 i + w % 8, i = 0..3, which the dispatcher places
// on the same XCD.
template <typename T, bool kK16 = false>
__global__ __launch_bounds__(128, 2) void bsa_fwd_pair_kernel(FwdArgs a) {
  static_assert(!kK16 || std::is_same<T, __bf16>::value, "fp16 scores take bf16 inputs");
  typedef Elem<T> E;
  constexpr int kD = 128;
  constexpr int kDS = kD / 16;        // 16-wide d steps of S = K Q^T
  constexpr int kDC = kD / 32;        // 32-row d chunks of O^T
  constexpr int kHalves = kD / 64;    // 128-byte half tiles per K or V tile
  constexpr int kCopies = 8;          // copy instructions per wave and tile, each of K and V
  __shared__ __attribute__((aligned(1024))) uint8_t k_lds[kHalves * kTileBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t v_lds[kHalves * kTileBytes];
  __shared__ int redo_lds[2];
  __shared__ float qn_lds[2];  // fp16 scores: each wave's largest squared query-row norm

  const int lane = threadIdx.x & 63;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // query rows 32g .. 32g + 31
  const int col = lane & 31;
  const int hh = lane >> 5;
  const int x = blockIdx.x;
  const int slot = 4 * (8 * (x >> 5) + (x & 7)) + ((x >> 3) & 3);
  int item = -1;
  if (slot < a.n_slots) item = __builtin_amdgcn_readfirstlane(a.order ? a.order[slot] : slot);
  // Both waves take the same branch: no barrier is left unmatched.
  if (item < 0 || item >= a.n_items) return;
  const int bh = item / a.nqb;
  const int qb = item - bh * a.nqb;
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int64_t list_row = (int64_t)bh * a.list_bh_stride + qb;
  int cnt = a.kv_cnt[list_row];
  cnt = cnt < 0 ? 0 : (cnt > a.max_cnt ? a.max_cnt : cnt);
  const __attribute__((address_space(4))) int32_t* list =
      (const __attribute__((address_space(4))) int32_t*)(a.kv_idx + list_row * a.max_cnt);

  const uint16_t* qbase = a.q + b * a.q_sb + h * a.q_sh;
  const int hk = a.kv_rep > 1 ? h / a.kv_rep : h;
  const uint16_t* khead = a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vhead = a.v + b * a.v_sb + hk * a.v_sh;
  uint32_t krow = (uint32_t)(a.k_sl * 2);
  const uint32_t vrow = (uint32_t)(a.v_sl * 2);
  uint32_t kbytes = (uint32_t)(a.Lk - 1) * krow + 2 * kHeadDim;
  const uint32_t vbytes = (uint32_t)(a.Lk - 1) * vrow + 2 * kHeadDim;
  lds_u8* const kl = (lds_u8*)k_lds;
  lds_u8* const vl = (lds_u8*)v_lds;

  uint32_t kgo[2], vgo[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int r = 8 * p + (lane >> 3);
    const int chunk = (lane & 7) ^ swz(r);
    kgo[p] = (lane >> 3) * krow + 16 * chunk;
    vgo[p] = (lane >> 3) * vrow + 16 * chunk;
  }
  int kro[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) kro[s] = 128 * col + 16 * ((2 * s + hh) ^ swz(col));
  int vro[2][2];
  {
    const int i = lane & 15, g4 = lane >> 4;
    const int hq = g4 >> 1, dg = g4 & 1;
#pragma unroll
    for (int dc = 0; dc < 2; ++dc)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = 8 * t + 4 * hq + (i >> 2);
        const int chunk = 4 * dc + 2 * dg + ((i & 3) >> 1);
        vro[dc][t] = 128 * r + 16 * (chunk ^ swz(r)) + 8 * (i & 1);
      }
  }

  // Q^T B operands of query row qb * 64 + 32g + col (clamped into Lq; clamped rows are never
  // stored; with a row map, q row q_rows[i], zeros outside q).
  typename E::v8 qf[kDS];
  {
    int row = min(qb * kBlock + 32 * g + col, a.Lq - 1);
    bool zero = false;
    if (a.q_rows) {
      row = a.q_rows[row];
      zero = (unsigned)row >= (unsigned)a.q_src_rows;
      row = zero ? 0 : row;
    }
    const uint16_t* p = qbase + (int64_t)row * a.q_sl + 8 * hh;
#pragma unroll
    for (int s = 0; s < kDS; ++s) {
      const uint4 w = *reinterpret_cast<const uint4*>(p + 16 * s);
      qf[s] = __builtin_bit_cast(typename E::v8, zero ? make_uint4(0u, 0u, 0u, 0u) : w);
    }
  }
  // fp16 scores: the head's largest squared key norm (its block norms, clamped loads).
  uint32_t kmax = 0u;
  if constexpr (kK16) {
    const uint32_t* bn = a.k16_norm2 + (int64_t)bh * a.nkb;
    for (int j0 = 0; j0 < a.nkb; j0 += 256) {
      uint32_t v4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v4[u] = bn[min(j0 + 64 * u + lane, a.nkb - 1)];
#pragma unroll
      for (int u = 0; u < 4; ++u) kmax = max(kmax, v4[u]);
    }
  }
  // The Q operands have landed before the first copy is issued, so that no load issued
  // before the loop is pending inside it.
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));

  // fp16 scores, as in bsa_fwd_kernel: the pair takes them when max |q_i * scale_log2| *
  // max |k_j| <= kK16Bound over its 64 query rows (both waves' rows: they decide together,
  // since their barriers must match) and the head's keys, with both squared norms below
  // kK16NormMax; q is then rounded to fp16 after the scaling and the K tiles come from the
  // fp16 copy of k. Otherwise the pair runs on the bf16 operands.
  bool use16 = false;
  if constexpr (kK16) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
    const float qs = a.scale_log2;
    float n2 = 0.f;
    uint32_t h16[kDS][4];
#pragma unroll
    for (int s = 0; s < kDS; ++s) {
      const sa_u32x4v w = __builtin_bit_cast(sa_u32x4v, qf[s]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x0 = __uint_as_float(w[i] << 16) * qs, x1 = __uint_as_float(w[i] & 0xffff0000u) * qs;
        n2 = fmaf(x1, x1, fmaf(x0, x0, n2));
        h16[s][i] = Elem<_Float16>::pack(x0, x1);
      }
    }
    float qn2 = xhalf_sum(n2);  // row 32g + col
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) qn2 = fmaxf(qn2, __shfl_xor(qn2, o));
    if (lane == 0) qn_lds[g] = qn2;
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    wg_barrier();
    qn2 = fmaxf(qn_lds[0], qn_lds[1]);
    qn2 = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(qn2)));
    const float kn2 = __uint_as_float(__builtin_amdgcn_readfirstlane(kmax));
    use16 = qn2 < kK16NormMax && kn2 < kK16NormMax && qn2 * kn2 <= kK16Bound * kK16Bound;
    if (use16) {
#pragma unroll
      for (int s = 0; s < kDS; ++s)
        qf[s] = __builtin_bit_cast(typename E::v8, sa_u32x4v{h16[s][0], h16[s][1], h16[s][2], h16[s][3]});
      khead = a.k16 + (int64_t)bh * a.Lk * kD;
      krow = 2 * kD;
      kbytes = (uint32_t)(a.Lk - 1) * krow + 2 * kHeadDim;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int r = 8 * p + (lane >> 3);
        kgo[p] = (lane >> 3) * krow + 16 * ((lane & 7) ^ swz(r));
      }
    }
  }

  sa_f32x16 acc[kDC];
  float m = -INFINITY, l = 0.f;

  auto block_ok = [&](int kb) { return (unsigned)kb < (unsigned)a.nkb; };
  // This wave's share of the copy of tile kb: the half tile of d half g (all 64 rows).
  auto copy_share = [&](const uint16_t* head, uint32_t bytes, uint32_t row, const uint32_t (&go)[2], lds_u8* dst,
                        int kb) {
    const uint32_t off = (block_ok(kb) ? (uint32_t)kb * kBlock : 0u) * row;
    dma_tile(head + 64 * g, bytes, off, row, go, dst + g * kTileBytes);
  };
  auto issue_k = [&](int kb) { copy_share(khead, kbytes, krow, kgo, kl, kb); };
  auto issue_v = [&](int kb) { copy_share(vhead, vbytes, vrow, vgo, vl, kb); };

  // One pass over the list. Fast pass (kSafe = false): P = exp2(S) with no max (fp16: minus
  // the row's maximum over the first tile), checked by the caller; safe pass: running max
  // with lazy rescale.
  auto run = [&](auto safe_tag, auto k16_tag) __attribute__((always_inline)) {
    constexpr bool kSafe = decltype(safe_tag)::value;
    constexpr bool kQ16 = decltype(k16_tag)::value;  // fp16 K and pre-scaled q: S in the exp2 domain
    constexpr bool kOffset = !kSafe && !std::is_same<T, __bf16>::value;
#pragma unroll
    for (int dc = 0; dc < kDC; ++dc) acc[dc] = sa_f32x16{};
    m = -INFINITY;
    l = 0.f;
    int kb = cnt > 0 ? list[0] : -1;
    if (cnt > 0) {
      issue_k(kb);
      issue_v(kb);
    }
    for (int it = 0; it < cnt; ++it) {
      // Past the end of the list the copies re-load the current block, so every iteration
      // has the same copies in flight.
      const int kb_next = it + 1 < cnt ? list[it + 1] : kb;
      // ---- K landed (own share: the wait; the partner's: the barrier).
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies));
      wg_barrier();
      sa_u32x4v kop[2][kDS];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s = 0; s < kDS; ++s) kop[c][s] = lds_read_b128(kl + (s >> 2) * kTileBytes + kro[s & 3] + 4096 * c);
      sa_f32x16 S[2];  // S^T of keys 32c + ..., query row 32g + col
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        sa_f32x16 t = {};
#pragma unroll
        for (int s = 0; s < kDS; ++s) {
          if constexpr (kQ16)
            t = Elem<_Float16>::mfma(Elem<_Float16>::as8(kop[c][s]), __builtin_bit_cast(sa_f16x8, qf[s]), t);
          else
            t = E::mfma(E::as8(kop[c][s]), qf[s], t);
        }
        S[c] = t;
      }
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      // ---- Both waves hold their K operands: refill the K buffer.
      wg_barrier();
      issue_k(kb_next);
      const int nvalid = block_ok(kb) ? min(kBlock, a.Lk - kb * kBlock) : 0;
      if (nvalid < kBlock) {  // keys past Lk, or an entry outside the grid
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (32 * c + 8 * (e >> 2) + 4 * hh + (e & 3) >= nvalid) S[c][e] = -INFINITY;
      }
      const float sc = kQ16 ? 1.f : a.scale_log2;  // fp16 scores: S is already scaled
      float mu = 0.f;
      // Row max of this tile's scaled scores (sc > 0: max(S) * sc = max(S * sc)).
      auto tile_row_max = [&]() {
        float mx = fmaxf(fmaxf(S[0][0], S[0][1]), S[0][2]);
#pragma unroll
        for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, S[0][e]), S[0][e + 1]);
        mx = fmaxf(fmaxf(mx, S[0][15]), S[1][0]);
#pragma unroll
        for (int e = 1; e < 15; e += 2) mx = fmaxf(fmaxf(mx, S[1][e]), S[1][e + 1]);
        mx = fmaxf(mx, S[1][15]);
        return xhalf_max(mx) * sc;
      };
      if (kOffset) {  // fp16 fast pass: the first tile's row max is the item's exp2 offset
        if (it == 0) m = tile_row_max();
        mu = m == -INFINITY ? 0.f : m;
      }
      if (kSafe) {
        const float cand = tile_row_max();
        if (__ballot(cand > m + kRescaleLog2) != 0) {
          const float m_new = fmaxf(m, cand);
          // A row with no key yet (m_new = -inf) has nothing to rescale.
          const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m - m_new);
          m = m_new;
          l *= alpha;
#pragma unroll
          for (int dc = 0; dc < kDC; ++dc) acc[dc] *= alpha;
        }
        mu = m == -INFINITY ? 0.f : m;
      }
      uint32_t P[2][8];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float p0 = fast_exp2(kSafe || kOffset ? fmaf(S[c][e], sc, -mu) : S[c][e] * sc);
          const float p1 = fast_exp2(kSafe || kOffset ? fmaf(S[c][e + 1], sc, -mu) : S[c][e + 1] * sc);
          P[c][e >> 1] = E::pack(p0, p1);
          l = E::dot2_ones(P[c][e >> 1], l);
        }
      // ---- V landed (own share: the wait; the partner's: the barrier).
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies));
      wg_barrier();
#pragma unroll
      for (int hp = 0; hp < kHalves; ++hp) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        sa_u32x2v vr[2][2][2][2];  // [c][u][dc][t]
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int dc = 0; dc < 2; ++dc)
#pragma unroll
              for (int t = 0; t < 2; ++t) {
                const uint32_t base = (uint32_t)(uintptr_t)(vl + hp * kTileBytes + vro[dc][t]);
                vr[c][u][dc][t] = (c == 0 ? (u == 0 ? lds_read_tr16_asm<0>(base) : lds_read_tr16_asm<2048>(base))
                                          : (u == 0 ? lds_read_tr16_asm<4096>(base) : lds_read_tr16_asm<6144>(base)));
              }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int dc = 0; dc < 2; ++dc) {
              const int done = 2 * ((c * 2 + u) * 2 + dc) + 2;  // reads this MFMA needs
              lgkm_wait_pair(16 - done, vr[c][u][dc][0], vr[c][u][dc][1]);
              const sa_u32x4v vop = {vr[c][u][dc][0].x, vr[c][u][dc][0].y, vr[c][u][dc][1].x, vr[c][u][dc][1].y};
              acc[2 * hp + dc] = E::mfma(
                  E::as8(vop), E::as8(sa_u32x4v{P[c][4 * u], P[c][4 * u + 1], P[c][4 * u + 2], P[c][4 * u + 3]}),
                  acc[2 * hp + dc]);
            }
      }
      // ---- Both waves hold their V operands: refill the V buffer.
      wg_barrier();
      issue_v(kb_next);
      kb = kb_next;
    }
    // The copies requested after the last tile land in LDS: wait for them before the LDS
    // is written again or the wave ends.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  };
  auto run_item = [&](auto safe_tag) __attribute__((always_inline)) {
    if constexpr (kK16) {
      if (use16) run(safe_tag, std::true_type{});
      else run(safe_tag, std::false_type{});
    } else {
      run(safe_tag, std::false_type{});
    }
  };

  run_item(std::false_type{});
  // The fast pass is exact unless a row's sum left [2^-90, 2^90] (fp16: P rounded to inf)
  // or an accumulator overflowed; then the pair redoes its block with the safe pass. Both
  // waves decide together (their barriers must match).
  bool bad = false;
  if (cnt > 0) {
    const float l_tot = xhalf_sum(l);
    bad = !(l_tot >= 0x1p-90f && l_tot <= 0x1p90f);
    float amax = 0.f;
#pragma unroll
    for (int dc = 0; dc < kDC; ++dc)
#pragma unroll
      for (int e = 0; e < 16; e += 2) amax = fmaxf(fmaxf(amax, fabsf(acc[dc][e])), fabsf(acc[dc][e + 1]));
    bad |= !(amax <= 3.0e38f);
  }
  const int wave_bad = __ballot(bad) != 0;
  if (lane == 0) redo_lds[g] = wave_bad;
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  wg_barrier();
  const bool redo = (redo_lds[0] | redo_lds[1]) != 0;
  if (redo) run_item(std::true_type{});

  // ---- Epilogue: out = acc / l (each lane half holds a partial l of its keys).
  const float l_tot = xhalf_sum(l);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  int row = qb * kBlock + 32 * g + col;
  bool store = row < a.Lq;
  if (store && a.o_rows) {  // remapped layout: query i goes to out row o_rows[i]
    row = a.o_rows[row];
    store = (unsigned)row < (unsigned)a.o_dst_rows;
  }
  if (store) {
    uint16_t* orow = a.o + b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_sl;
#pragma unroll
    for (int dc = 0; dc < kDC; ++dc)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const sa_f32x16& A = acc[dc];
        // element 4q4 + j is d = 32dc + 8q4 + 4hh + j
        *reinterpret_cast<uint2*>(orow + 32 * dc + 8 * q4 + 4 * hh) =
            make_uint2(E::pack(A[4 * q4] * inv, A[4 * q4 + 1] * inv), E::pack(A[4 * q4 + 2] * inv, A[4 * q4 + 3] * inv));
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

// Fused pooled map of a pooling-mode launch (FwdArgs::pool_po): Po [B][H][nd][nd] fp32.
struct PoolOut {
  float* po;
  int64_t sb, sh, si;
  int nd;
  int causal;
};

// Output of key-range split items: one workgroup per item, thread t forms row t / 4, head
// dims (t % 4) * kD / 4 + 0 .. kD / 4 - 1, from the item's n_parts partials (in part order):
// out = sum_p acc_p * 2^(m_p - M) / sum_p l_p * 2^(m_p - M), M = max_p m_p.
template <typename T, int kD>
__global__ __launch_bounds__(256) void split_merge_kernel(FwdArgs a) {
  typedef Elem<T> E;
  constexpr int kSeg = kD / 4;
  const int item = blockIdx.x;
  if (item >= a.n_items) return;
  const int bh = item / a.nqb;
  const int qb = item - bh * a.nqb;
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int r = threadIdx.x >> 2;
  const int d0 = (threadIdx.x & 3) * kSeg;
  const float* w0 = a.ws + (int64_t)item * a.n_parts * kSplitFloats<kD>;
  float mx = -INFINITY;
  for (int p = 0; p < a.n_parts; ++p) mx = fmaxf(mx, w0[(int64_t)p * kSplitFloats<kD> + kBlock * kD + kBlock + r]);
  float lsum = 0.f;
  float o[kSeg];
#pragma unroll
  for (int j = 0; j < kSeg; ++j) o[j] = 0.f;
  for (int p = 0; p < a.n_parts; ++p) {
    const float* w = w0 + (int64_t)p * kSplitFloats<kD>;
    const float f = exp2f(w[kBlock * kD + kBlock + r] - mx);
    lsum = fmaf(w[kBlock * kD + r], f, lsum);
#pragma unroll
    for (int j = 0; j < kSeg; j += 4) {
      const float4 x = *reinterpret_cast<const float4*>(w + r * kD + d0 + j);
      o[j] = fmaf(x.x, f, o[j]);
      o[j + 1] = fmaf(x.y, f, o[j + 1]);
      o[j + 2] = fmaf(x.z, f, o[j + 2]);
      o[j + 3] = fmaf(x.w, f, o[j + 3]);
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  int row = qb * kBlock + r;
  if (row >= a.Lq) return;
  if (a.o_rows) {
    row = a.o_rows[row];
    if ((unsigned)row >= (unsigned)a.o_dst_rows) return;
  }
  uint16_t* orow = a.o + b * a.o_sb + h * a.o_sh + (int64_t)row * a.o_sl + d0;
#pragma unroll
  for (int j = 0; j < kSeg; j += 8)
    *reinterpret_cast<uint4*>(orow + j) =
        make_uint4(E::pack(o[j] * inv, o[j + 1] * inv), E::pack(o[j + 2] * inv, o[j + 3] * inv),
                   E::pack(o[j + 4] * inv, o[j + 5] * inv), E::pack(o[j + 6] * inv, o[j + 7] * inv));
}

// Key-range split of a launch with few items: parts per item so that the parts fill the
// wave slots of n_cus CUs once (resident waves per CU: 8 at head dim 64, 4 at 128), with at
// least kSplitPartTiles list positions per part at the list width; 1 = no split (also below
// kSplitMinTiles, or when the items already fill half the slots). A pure function of its
// arguments: the caller passes the result to the split entry points, so a launch's bits
// depend on nothing but its arguments.
constexpr int kSplitMinTiles = 64;
constexpr int kSplitPartTiles = 32;
constexpr int kSplitMaxParts = 16;

int split_parts(int64_t n_items, int max_cnt, int D, int n_cus) {
  if (max_cnt < kSplitMinTiles) return 1;
  const int64_t slots = (int64_t)n_cus * (D == 64 ? 2 : 1) * kWaves;
  if (n_items * 2 > slots) return 1;
  const int64_t p = std::min<int64_t>({slots / n_items, max_cnt / kSplitPartTiles, kSplitMaxParts});
  return p > 1 ? (int)p : 1;
}

size_t split_workspace_bytes(int64_t n_items, int D, int parts) {
  return (size_t)n_items * parts * (D == 64 ? kSplitFloats<64> : kSplitFloats<128>) * sizeof(float);
}

// One kernel variant per (tile masks, key bias, pooling columns): the caller has rejected
// the combinations of tile masks or pooling with a key bias.
template <typename T, int kD>
void launch_variant(const FwdArgs& a, dim3 g, dim3 blk, hipStream_t s, bool mask, bool bias, int pool_cols,
                    bool v32 = false) {
  if constexpr (kD == 64 && std::is_same<T, __bf16>::value) {
    if (a.k16) {  // fp16 scores (the caller has rejected every mode but the key bias)
      if (bias) hipLaunchKernelGGL((bsa_fwd_kernel<true, false, 0, T, kD, kD, true>), g, blk, 0, s, a);
      else hipLaunchKernelGGL((bsa_fwd_kernel<false, false, 0, T, kD, kD, true>), g, blk, 0, s, a);
      return;
    }
    if (v32) {  // 32 value columns (the caller has rejected tile masks and pooling)
      if (bias) hipLaunchKernelGGL((bsa_fwd_kernel<true, false, 0, T, kD, 32>), g, blk, 0, s, a);
      else hipLaunchKernelGGL((bsa_fwd_kernel<false, false, 0, T, kD, 32>), g, blk, 0, s, a);
      return;
    }
  }
  if constexpr (kD == 128) {
    if (!mask && !bias && pool_cols == 0 && a.n_parts == 1) {  // plain lists: wave pairs
      // Workgroup x runs slot 4 (8 (x / 32) + x % 8) + (x / 8) % 4: the four slots of each
      // dispatch group on that group's XCD.
      const int64_t groups = a.n_slots / kWaves;
      const dim3 pg((unsigned)((groups + 7) / 8 * 32));
      if constexpr (std::is_same<T, __bf16>::value) {
        if (a.k16) {  // fp16 scores
          hipLaunchKernelGGL((bsa_fwd_pair_kernel<T, true>), pg, dim3(128), 0, s, a);
          return;
        }
      }
      hipLaunchKernelGGL((bsa_fwd_pair_kernel<T>), pg, dim3(128), 0, s, a);
      return;
    }
  }
  if (mask) {
    if (pool_cols == 32) hipLaunchKernelGGL((bsa_fwd_kernel<false, true, 32, T, kD>), g, blk, 0, s, a);
    else if (pool_cols == 64) hipLaunchKernelGGL((bsa_fwd_kernel<false, true, 64, T, kD>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((bsa_fwd_kernel<false, true, 0, T, kD>), g, blk, 0, s, a);
  } else if (bias) {
    hipLaunchKernelGGL((bsa_fwd_kernel<true, false, 0, T, kD>), g, blk, 0, s, a);
  } else {
    if (pool_cols == 32) hipLaunchKernelGGL((bsa_fwd_kernel<false, false, 32, T, kD>), g, blk, 0, s, a);
    else if (pool_cols == 64) hipLaunchKernelGGL((bsa_fwd_kernel<false, false, 64, T, kD>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((bsa_fwd_kernel<false, false, 0, T, kD>), g, blk, 0, s, a);
  }
}

int launch_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k, const int64_t k_strides[3],
               const uint16_t* v, const int64_t v_strides[3], uint16_t* out, const int64_t out_strides[3], int B,
               int H, int Lq, int Lk, int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
               bool lists_shared, const int32_t* kv_slot, const uint64_t* tile_masks, const float* key_bias,
               const int64_t bias_strides[2], float sm_scale, const int32_t* work_order, int64_t n_slots,
               const int32_t* q_rows, int q_src_rows, const int32_t* o_rows, int o_dst_rows, void* stream,
               const char* fn, int kv_rep = 1, int pool_cols = 0, float* pool_r = nullptr,
               float* pool_lse = nullptr, const PoolOut* pool_out = nullptr, bool fp16 = false,
               bool v32 = false, int parts = 1, void* split_ws = nullptr, int64_t split_ws_bytes = 0,
               const uint16_t* k16 = nullptr, const uint32_t* k16_norm2 = nullptr) {
  SA_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides && kv_idx && kv_cnt,
             "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && Lq > 0 && Lk > 0, "%s: bad shape B=%d H=%d Lq=%d Lk=%d", fn, B, H, Lq, Lk);
  if (D != 64 && D != 128) return sa::fail(SA_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", fn, D);
  SA_REQUIRE(std::isfinite(sm_scale) && sm_scale > 0.f, "%s: sm_scale must be finite and > 0", fn);
  const int nqb = sa::cdiv(Lq, kBlock);
  const int nkb = sa::cdiv(Lk, kBlock);
  SA_REQUIRE(max_cnt > 0, "%s: max_cnt must be > 0", fn);
  SA_REQUIRE(!key_bias || bias_strides, "%s: key_bias without bias_strides", fn);
  SA_REQUIRE(!q_rows || q_src_rows > 0, "%s: q_rows given with q_src_rows=%d", fn, q_src_rows);
  SA_REQUIRE(!o_rows || o_dst_rows > 0, "%s: o_rows given with o_dst_rows=%d", fn, o_dst_rows);
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
  // K/V tiles are copied through 32-bit buffer offsets relative to each head's first row.
  for (const int64_t* st : {k_strides, v_strides}) {
    if ((int64_t)(Lk - 1) * st[2] * 2 + 2 * D > INT_MAX)
      return sa::fail(SA_ERR_UNSUPPORTED, "%s: key rows of one head span more than 2 GiB", fn);
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
  a.n_parts = 1;
  a.ws = nullptr;
  a.k16 = k16;
  a.k16_norm2 = k16_norm2;
  if (k16 && (!k16_norm2 || (D != 64 && !(D == 128 && !key_bias)) || fp16 || v32 || kv_slot || pool_cols ||
              parts != 1 || q_rows || o_rows || kv_rep != 1))
    return sa::fail(SA_ERR_UNSUPPORTED,
                    "%s: fp16 scores need plain or key-bias bf16 lists at head dim 64, or plain ones at 128", fn);
  a.kv_idx = kv_idx; a.kv_cnt = kv_cnt; a.max_cnt = max_cnt;
  a.bias = key_bias;
  a.bias_sb = key_bias ? bias_strides[0] : 0;
  a.bias_sh = key_bias ? bias_strides[1] : 0;
  a.sm_scale = sm_scale;
  a.scale_log2 = sm_scale * kLog2e;
  a.list_bh_stride = lists_shared ? 0 : nqb;
  a.kv_slot = kv_slot;
  a.tile_masks = tile_masks;
  a.q_rows = q_rows;
  a.o_rows = o_rows;
  a.q_src_rows = q_rows ? q_src_rows : Lq;
  a.o_dst_rows = o_rows ? o_dst_rows : Lq;
  a.kv_rep = kv_rep;
  a.pool_r = pool_r;
  a.pool_ncol = pool_cols ? nkb * (kBlock / pool_cols) : 0;
  a.pool_lpad = nqb * kBlock;
  a.pool_lse = pool_lse;
  a.pool_po = pool_out ? pool_out->po : nullptr;
  a.po_sb = pool_out ? pool_out->sb : 0;
  a.po_sh = pool_out ? pool_out->sh : 0;
  a.po_si = pool_out ? pool_out->si : 0;
  a.pool_nd = pool_out ? pool_out->nd : 0;
  a.pool_causal = pool_out ? pool_out->causal : 0;
  SA_REQUIRE(pool_cols == 0 || (pool_r && (pool_lse || pool_out) && !q_rows && !o_rows),
             "%s: pooling needs its buffers and no row maps", fn);
  SA_REQUIRE(!pool_out || (pool_out->po && pool_cols && Lq == Lk && pool_out->nd == sa::cdiv(Lq, pool_cols)),
             "%s: fused pooled map needs pooling columns of the map's block size", fn);

  if (kv_slot && key_bias) return sa::fail(SA_ERR_UNSUPPORTED, "%s: tile masks with key_bias", fn);
  if (v32 && (D != 64 || fp16 || kv_slot || pool_cols))
    return sa::fail(SA_ERR_UNSUPPORTED, "%s: 32 value columns need bf16, head dim 64, no tile masks or pooling", fn);
  if (pool_cols && key_bias) return sa::fail(SA_ERR_UNSUPPORTED, "%s: pooling with key_bias", fn);
  hipStream_t s = sa::as_stream(stream);
  const bool mask = kv_slot != nullptr, bias = key_bias != nullptr;
  // Few items with long plain lists leave most wave slots idle: with parts > 1 each item's
  // list is split into key ranges, one wave each, whose partials go to the caller's
  // workspace, and split_merge_kernel forms the outputs from them.
  int64_t grid_x = grid;
  if (parts > 1) {
    if (mask || bias || pool_cols || v32)
      return sa::fail(SA_ERR_UNSUPPORTED, "%s: key-range parts with tile masks, key_bias, pooling or 32 value columns",
                      fn);
    SA_REQUIRE(parts <= kSplitMaxParts, "%s: parts=%d > %d", fn, parts, kSplitMaxParts);
    const size_t need = split_workspace_bytes(n_items, D, parts);
    SA_REQUIRE(split_ws, "%s: null workspace with parts=%d", fn, parts);
    SA_REQUIRE(reinterpret_cast<uintptr_t>(split_ws) % 16 == 0, "%s: workspace not 16-byte aligned", fn);
    SA_REQUIRE(split_ws_bytes >= 0 && (size_t)split_ws_bytes >= need, "%s: workspace of %lld bytes < %zu", fn,
               (long long)split_ws_bytes, need);
    SA_REQUIRE(n_items * parts < (1LL << 30), "%s: too many key-range parts", fn);
    a.n_parts = parts;
    a.ws = static_cast<float*>(split_ws);
    a.n_slots = (int)((n_items * parts + kWaves - 1) / kWaves * kWaves);
    grid_x = a.n_slots / kWaves;
  }
  const dim3 g((unsigned)grid_x), blk(64 * kWaves);
  if (fp16) {
    if (D == 64) launch_variant<_Float16, 64>(a, g, blk, s, mask, bias, pool_cols);
    else launch_variant<_Float16, 128>(a, g, blk, s, mask, bias, pool_cols);
  } else {
    if (D == 64) launch_variant<__bf16, 64>(a, g, blk, s, mask, bias, pool_cols, v32);
    else launch_variant<__bf16, 128>(a, g, blk, s, mask, bias, pool_cols);
  }
  if (a.n_parts > 1) {
    const dim3 gm((unsigned)n_items), bm(256);
    if (fp16) {
      if (D == 64) hipLaunchKernelGGL((split_merge_kernel<_Float16, 64>), gm, bm, 0, s, a);
      else hipLaunchKernelGGL((split_merge_kernel<_Float16, 128>), gm, bm, 0, s, a);
    } else {
      if (D == 64) hipLaunchKernelGGL((split_merge_kernel<__bf16, 64>), gm, bm, 0, s, a);
      else hipLaunchKernelGGL((split_merge_kernel<__bf16, 128>), gm, bm, 0, s, a);
    }
  }
  return sa::check_launch(fn);
}

}  // namespace

extern "C" int sa_attn_split_parts(int64_t n_items, int max_cnt, int D, int n_cus, int* parts) {
  SA_REQUIRE(parts, "sa_attn_split_parts: null parts");
  SA_REQUIRE(n_items > 0 && max_cnt > 0 && (D == 64 || D == 128) && n_cus > 0,
             "sa_attn_split_parts: bad arguments n_items=%lld max_cnt=%d D=%d n_cus=%d", (long long)n_items, max_cnt,
             D, n_cus);
  *parts = split_parts(n_items, max_cnt, D, n_cus);
  return sa::ok();
}

extern "C" int sa_attn_split_workspace(int64_t n_items, int D, int parts, int64_t* bytes) {
  SA_REQUIRE(bytes, "sa_attn_split_workspace: null bytes");
  SA_REQUIRE(n_items > 0 && n_items < (1LL << 30) && (D == 64 || D == 128) && parts >= 1 && parts <= kSplitMaxParts,
             "sa_attn_split_workspace: bad arguments n_items=%lld D=%d parts=%d", (long long)n_items, D, parts);
  *bytes = parts > 1 ? (int64_t)split_workspace_bytes(n_items, D, parts) : 0;
  return sa::ok();
}

namespace {

int fwd_split(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k, const int64_t k_strides[3],
              const uint16_t* v, const int64_t v_strides[3], uint16_t* out, const int64_t out_strides[3], int B, int H,
              int Lq, int Lk, int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt, float sm_scale,
              const int32_t* q_rows, int q_src_rows, const int32_t* o_rows, int o_dst_rows, int parts,
              void* workspace, int64_t workspace_bytes, void* stream, bool fp16, const char* fn) {
  SA_REQUIRE(parts >= 1, "%s: parts=%d must be >= 1", fn, parts);
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, false, nullptr, nullptr, nullptr, nullptr, sm_scale, nullptr, 0, q_rows, q_src_rows,
                    o_rows, o_dst_rows, stream, fn, 1, 0, nullptr, nullptr, nullptr, fp16, false, parts, workspace,
                    workspace_bytes);
}

}  // namespace

extern "C" int sa_block_sparse_fwd_split(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                         const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                         uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                         int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                         float sm_scale, const int32_t* q_rows, int q_src_rows, const int32_t* o_rows,
                                         int o_dst_rows, int parts, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
  return fwd_split(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                   max_cnt, sm_scale, q_rows, q_src_rows, o_rows, o_dst_rows, parts, workspace, workspace_bytes,
                   stream, false, "sa_block_sparse_fwd_split");
}

extern "C" int sa_block_sparse_fwd_split_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                             const int64_t k_strides[3], const uint16_t* v,
                                             const int64_t v_strides[3], uint16_t* out, const int64_t out_strides[3],
                                             int B, int H, int Lq, int Lk, int D, const int32_t* kv_idx,
                                             const int32_t* kv_cnt, int max_cnt, float sm_scale,
                                             const int32_t* q_rows, int q_src_rows, const int32_t* o_rows,
                                             int o_dst_rows, int parts, void* workspace, int64_t workspace_bytes,
                                             void* stream) {
  return fwd_split(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                   max_cnt, sm_scale, q_rows, q_src_rows, o_rows, o_dst_rows, parts, workspace, workspace_bytes,
                   stream, true, "sa_block_sparse_fwd_split_f16");
}

extern "C" int sa_block_sparse_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                   const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                   uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                   int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                   const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                   const int32_t* work_order, int64_t n_slots, void* stream) {
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, false, nullptr, nullptr, key_bias, bias_strides, sm_scale, work_order, n_slots, nullptr,
                    0, nullptr, 0, stream, "sa_block_sparse_fwd");
}

namespace {

// fp16 copy of k for the fp16-score mode: k16[bh][j] = fp16(k[b][h][j]) (round to nearest
// even: exact for 2^-17 <= |k| < 65504, fp16's subnormal grid below), and blk_norm2[bh * nkb +
// kb] = the largest squared row norm of key block kb (fp32 fmaf chain over the 64 dims, as float
// bits, compared as unsigned: the norms are non-negative, and NaN bits compare above every
// finite or infinite norm, so a NaN row fails the attention kernel's bound). One wave per
// 64-row key block, 8 lanes per row (16 bytes each). sa_block_pool_k16 writes the same from
// the pooling pass.
struct K16Args {
  const uint16_t* k;
  int64_t k_sb, k_sh, k_sl;
  int H, Lk, nkb;
  int64_t n_blocks;  // B * H * nkb
  uint16_t* k16;
  uint32_t* blk_norm2;  // [n_blocks]
};

template <int kD>
__global__ __launch_bounds__(256) void k16_kernel(K16Args a) {
  constexpr int kLpr = kD / 8;        // lanes per row, 16 bytes each
  constexpr int kRpp = 64 / kLpr;     // rows per load of the wave
  constexpr int kPass = kBlock / kRpp;
  const int lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (blk >= a.n_blocks) return;
  const int64_t bh = blk / a.nkb;
  const int kb = (int)(blk - bh * a.nkb);
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int c8 = lane % kLpr;
  const uint16_t* src = a.k + b * a.k_sb + h * a.k_sh + 8 * c8;
  uint16_t* dst = a.k16 + bh * (int64_t)a.Lk * kD + 8 * c8;
  uint4 w[kPass];
#pragma unroll
  for (int i = 0; i < kPass; ++i) {  // rows past Lk load the last row, which is neither stored nor counted
    const int r = min(kb * kBlock + kRpp * i + lane / kLpr, a.Lk - 1);
    w[i] = *reinterpret_cast<const uint4*>(src + (int64_t)r * a.k_sl);
  }
  uint32_t mx = 0u;  // float bits of the largest squared norm seen
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int r = kb * kBlock + kRpp * i + lane / kLpr;
    const uint32_t e[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
    uint32_t o[4];
    float n = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x0 = __uint_as_float(e[j] << 16), x1 = __uint_as_float(e[j] & 0xffff0000u);
      n = fmaf(x1, x1, fmaf(x0, x0, n));
      o[j] = Elem<_Float16>::pack(x0, x1);
    }
    // the row's kLpr lanes, in a fixed order
#pragma unroll
    for (int off = 1; off < kLpr; off <<= 1) n += __shfl_xor(n, off);
    if (r < a.Lk) {
      mx = max(mx, __float_as_uint(n));
      *reinterpret_cast<uint4*>(dst + (int64_t)r * kD) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
#pragma unroll
  for (int off = kLpr; off < 64; off <<= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  if (lane == 0) a.blk_norm2[blk] = mx;
}

using sa::k16_bytes;
using sa::k16_ws_bytes;

// bias2[(b * H + h) * Lk + j] = bias[b * sb + h * sh + j] * log2(e): the key bias in the exp2
// domain for the fp16-score kernel (the bf16-score kernel forms the same product per tile).
__global__ __launch_bounds__(256) void bias_log2_kernel(const float* bias, int64_t sb, int64_t sh, int H, int Lk,
                                                        int64_t n, float* bias2) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t bh = i / Lk, j = i - bh * Lk;
  const int64_t b = bh / H, h = bh - b * H;
  bias2[i] = bias[b * sb + h * sh + j] * kLog2e;
}

}  // namespace

extern "C" int sa_block_sparse_fwd_k16_workspace(int B, int H, int Lk, int D, int with_bias, int64_t* bytes) {
  SA_REQUIRE(bytes, "sa_block_sparse_fwd_k16_workspace: null bytes");
  SA_REQUIRE(B > 0 && H > 0 && Lk > 0, "sa_block_sparse_fwd_k16_workspace: bad shape B=%d H=%d Lk=%d", B, H, Lk);
  if (D != kHeadDim && !(D == 128 && !with_bias))
    return sa::fail(SA_ERR_UNSUPPORTED, "sa_block_sparse_fwd_k16_workspace: head_dim %d (64; 128 without a key bias)", D);
  *bytes = with_bias ? sa::k16_ws_bytes_bias(B, H, Lk) : k16_ws_bytes(B, H, Lk, D);
  return sa::ok();
}

namespace {

int k16_prepare(const uint16_t* k, const int64_t k_strides[3], int B, int H, int Lk, int D, void* workspace,
                int64_t workspace_bytes, void* stream, const char* fn) {
  SA_REQUIRE(k && k_strides, "%s: null k", fn);
  SA_REQUIRE(B > 0 && H > 0 && Lk > 0, "%s: bad shape B=%d H=%d Lk=%d", fn, B, H, Lk);
  if (D != kHeadDim && D != 128) return sa::fail(SA_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", fn, D);
  const int64_t need = k16_ws_bytes(B, H, Lk, D);
  SA_REQUIRE(workspace && reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "%s: workspace null or not 256-byte aligned",
             fn);
  SA_REQUIRE(workspace_bytes >= need, "%s: workspace of %lld bytes < %lld", fn, (long long)workspace_bytes,
             (long long)need);
  if (reinterpret_cast<uintptr_t>(k) % 16 != 0 || k_strides[0] % 8 || k_strides[1] % 8 || k_strides[2] % 8)
    return sa::fail(SA_ERR_UNSUPPORTED, "%s: k base not 16-byte aligned or strides not multiples of 8", fn);
  K16Args ka;
  ka.k = k; ka.k_sb = k_strides[0]; ka.k_sh = k_strides[1]; ka.k_sl = k_strides[2];
  ka.H = H; ka.Lk = Lk; ka.nkb = sa::cdiv(Lk, kBlock);
  ka.n_blocks = (int64_t)B * H * ka.nkb;
  ka.k16 = static_cast<uint16_t*>(workspace);
  ka.blk_norm2 = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + k16_bytes(B, H, Lk, D));
  SA_REQUIRE(ka.n_blocks / kWaves < (1LL << 31), "%s: grid too large", fn);
  hipStream_t s = sa::as_stream(stream);
  const dim3 grid((unsigned)((ka.n_blocks + kWaves - 1) / kWaves));
  if (D == 128) hipLaunchKernelGGL(k16_kernel<128>, grid, dim3(64 * kWaves), 0, s, ka);
  else hipLaunchKernelGGL(k16_kernel<64>, grid, dim3(64 * kWaves), 0, s, ka);
  return sa::check_launch(fn);
}

}  // namespace

extern "C" int sa_block_sparse_fwd_k16_prepare(const uint16_t* k, const int64_t k_strides[3], int B, int H, int Lk,
                                               int D, void* workspace, int64_t workspace_bytes, void* stream) {
  return k16_prepare(k, k_strides, B, H, Lk, D, workspace, workspace_bytes, stream, "sa_block_sparse_fwd_k16_prepare");
}

extern "C" int sa_block_sparse_fwd_k16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                       const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                       uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                       int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                       const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                       const int32_t* work_order, int64_t n_slots, int prepared, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  const char* fn = "sa_block_sparse_fwd_k16";
  SA_REQUIRE(!key_bias || bias_strides, "%s: key_bias without bias_strides", fn);
  if (key_bias) {
    SA_REQUIRE(B > 0 && H > 0 && Lk > 0, "%s: bad shape B=%d H=%d Lk=%d", fn, B, H, Lk);
    if (D != kHeadDim) return sa::fail(SA_ERR_UNSUPPORTED, "%s: a key bias needs head_dim 64, got %d", fn, D);
    SA_REQUIRE(workspace_bytes >= sa::k16_ws_bytes_bias(B, H, Lk), "%s: workspace of %lld bytes < %lld with key_bias",
               fn, (long long)workspace_bytes, (long long)sa::k16_ws_bytes_bias(B, H, Lk));
  }
  int rc = prepared ? SA_OK : k16_prepare(k, k_strides, B, H, Lk, D, workspace, workspace_bytes, stream, fn);
  if (rc) return rc;
  if (prepared) {  // the same checks of the workspace, without the launches
    SA_REQUIRE(B > 0 && H > 0 && Lk > 0, "%s: bad shape B=%d H=%d Lk=%d", fn, B, H, Lk);
    if (D != kHeadDim && D != 128) return sa::fail(SA_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", fn, D);
    SA_REQUIRE(workspace && reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
               "%s: workspace null or not 256-byte aligned", fn);
    SA_REQUIRE(workspace_bytes >= k16_ws_bytes(B, H, Lk, D), "%s: workspace of %lld bytes < %lld", fn,
               (long long)workspace_bytes, (long long)k16_ws_bytes(B, H, Lk, D));
  }
  const uint16_t* k16 = static_cast<const uint16_t*>(workspace);
  const uint32_t* norm2 =
      reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(workspace) + k16_bytes(B, H, Lk, D));
  const float* bias2 = nullptr;
  int64_t bias2_strides[2] = {(int64_t)H * Lk, Lk};
  if (key_bias) {  // the bias in log2 units, behind the k16 part of the workspace
    float* b2 = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + sa::k16_bias_offset(B, H, Lk));
    const int64_t n = (int64_t)B * H * Lk;
    hipLaunchKernelGGL(bias_log2_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, sa::as_stream(stream),
                       key_bias, bias_strides[0], bias_strides[1], H, Lk, n, b2);
    if ((rc = sa::check_launch(fn))) return rc;
    bias2 = b2;
  }
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, false, nullptr, nullptr, bias2, bias2_strides, sm_scale, work_order, n_slots, nullptr, 0,
                    nullptr, 0, stream, fn, 1, 0, nullptr, nullptr, nullptr, false, false, 1, nullptr, 0, k16, norm2);
}

extern "C" int sa_block_sparse_fwd_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                       const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                       uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                       int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                       const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                       const int32_t* work_order, int64_t n_slots, void* stream) {
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, false, nullptr, nullptr, key_bias, bias_strides, sm_scale, work_order, n_slots, nullptr,
                    0, nullptr, 0, stream, "sa_block_sparse_fwd_f16", 1, 0, nullptr, nullptr, nullptr, true);
}

extern "C" int sa_block_sparse_fwd_v32(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                       const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                       uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                       const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                       const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                       const int32_t* work_order, int64_t n_slots, void* stream) {
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, 64, kv_idx, kv_cnt,
                    max_cnt, false, nullptr, nullptr, key_bias, bias_strides, sm_scale, work_order, n_slots, nullptr,
                    0, nullptr, 0, stream, "sa_block_sparse_fwd_v32", 1, 0, nullptr, nullptr, nullptr, false, true);
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
                    nullptr, 0, nullptr, 0, stream, "sa_block_sparse_fwd_tilemask");
}

extern "C" int sa_block_sparse_fwd_mapped(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                          const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                          uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                                          int D, const int32_t* kv_idx, const int32_t* kv_cnt, const int32_t* kv_slot,
                                          int max_cnt, int lists_shared, const uint64_t* tile_masks,
                                          const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                          const int32_t* q_rows, int q_src_rows, const int32_t* o_rows,
                                          int o_dst_rows, const int32_t* work_order, int64_t n_slots, void* stream) {
  SA_REQUIRE(!kv_slot == !tile_masks, "sa_block_sparse_fwd_mapped: kv_slot and tile_masks go together");
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, lists_shared != 0, kv_slot, tile_masks, key_bias, bias_strides, sm_scale, work_order,
                    n_slots, q_rows, q_src_rows, o_rows, o_dst_rows, stream, "sa_block_sparse_fwd_mapped");
}

extern "C" int sa_block_sparse_fwd_mapped_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                              const int64_t k_strides[3], const uint16_t* v,
                                              const int64_t v_strides[3], uint16_t* out,
                                              const int64_t out_strides[3], int B, int H, int Lq, int Lk, int D,
                                              const int32_t* kv_idx, const int32_t* kv_cnt, const int32_t* kv_slot,
                                              int max_cnt, int lists_shared, const uint64_t* tile_masks,
                                              const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                              const int32_t* q_rows, int q_src_rows, const int32_t* o_rows,
                                              int o_dst_rows, const int32_t* work_order, int64_t n_slots,
                                              void* stream) {
  SA_REQUIRE(!kv_slot == !tile_masks, "sa_block_sparse_fwd_mapped_f16: kv_slot and tile_masks go together");
  return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, Lq, Lk, D, kv_idx, kv_cnt,
                    max_cnt, lists_shared != 0, kv_slot, tile_masks, key_bias, bias_strides, sm_scale, work_order,
                    n_slots, q_rows, q_src_rows, o_rows, o_dst_rows, stream, "sa_block_sparse_fwd_mapped_f16", 1, 0,
                    nullptr, nullptr, nullptr, true);
}

// ---------------------------------------------------------------------------------------
// Pooled attention map (attn_with_pooling, utils/attn_pooling_kernel.py:18-289): the
// attention kernel in pooling mode stores each row's maximum scaled logit per 32- or 64-key
// column. For 32- and 64-token blocks the same kernel then forms Po from them (FwdArgs::
// pool_po); for 128-token blocks it also stores the rows' log2-sum-exp2, and
// pool_reduce_kernel turns them into
//   Po[i][j] = max over rows r of query block i, keys of key block j of exp2(R[c][r] - lse[r])
// (the largest softmax probability of the block), each row of Po divided by its sum.
namespace {

constexpr int kPoolMaxNd = 8192;  // key blocks per row (dynamic LDS of the reduce: 32 KB)

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct PoolLayout {
  int nqb, nkb, G, ncol_alloc, lpad;
  size_t idx, cnt, slot, mask, r, lse, total;  // byte offsets into the workspace
};

PoolLayout pool_layout(int B, int H, int L, int block_size) {
  PoolLayout p;
  p.nqb = p.nkb = sa::cdiv(L, kBlock);
  p.G = block_size == 32 ? 32 : 64;
  p.ncol_alloc = p.nkb * (kBlock / p.G);
  p.lpad = p.nqb * kBlock;
  size_t o = 0;
  p.idx = o;  o += align256((size_t)p.nqb * p.nkb * 4);
  p.cnt = o;  o += align256((size_t)p.nqb * 4);
  p.slot = o; o += align256((size_t)p.nqb * p.nkb * 4);
  p.mask = o; o += align256(kBlock * 8);
  p.r = o;    o += align256((size_t)B * H * p.ncol_alloc * p.lpad * 4);
  p.lse = o;  o += align256((size_t)B * H * p.lpad * 4);
  p.total = o;
  return p;
}

// Dense (all key blocks) or causal (blocks <= the query block, the diagonal tile masked
// to keys <= query) kv lists, shared by every head; mask slot 0 = lower triangle.
struct PoolListArgs {
  int32_t* idx;
  int32_t* cnt;
  int32_t* slot;
  uint64_t* mask;
  int nqb, nkb, causal;
};

__global__ __launch_bounds__(256) void pool_lists_kernel(PoolListArgs a) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < (int64_t)a.nqb * a.nkb) {
    const int qb = (int)(t / a.nkb), j = (int)(t - (int64_t)qb * a.nkb);
    a.idx[t] = j;
    a.slot[t] = (a.causal && j == qb) ? 0 : -1;
  }
  if (t < a.nqb) a.cnt[t] = a.causal ? min((int)t + 1, a.nkb) : a.nkb;
  if (t < kBlock) a.mask[t] = t == kBlock - 1 ? ~0ull : ((2ull << t) - 1ull);  // row t: keys 0..t
}

struct PoolReduceArgs {
  const float* r;  // [B*H][nqb][ncol_alloc][64]
  int nqb, ncol_alloc;
  int lpad;
  const float* lse;
  int L, bs, G, nd, ncol, causal, H;
  float* po;
  int64_t po_sb, po_sh, po_si;
  int64_t total;  // B * H * nd
};

// One workgroup per (bh, query block i); wave w takes key blocks j in [8w + 32t, 8w + 32t + 8);
// lane l the rows r0 + l and r0 + 64 + l of the block. Every load is issued at a clamped,
// in-bounds row and column, and entries outside the block or the causal lists are discarded
// by selects, so the eight loads of a step are in flight together. Dynamic LDS: nd floats.
__global__ __launch_bounds__(256) void pool_reduce_kernel(PoolReduceArgs a) {
  constexpr int kU = 8;
  extern __shared__ float row[];
  __shared__ float part[256];
  const int64_t w = blockIdx.x;
  if (w >= a.total) return;  // uniform over the workgroup
  const int64_t bh = w / a.nd;
  const int i = (int)(w - bh * a.nd);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r0 = i * a.bs, r1 = min(r0 + a.bs, a.L);
  const int ra = r0 + lane, rbw = r0 + 64 + lane;
  const int ra_c = min(ra, r1 - 1), rb_c = min(rbw, r1 - 1);  // rows read (always < L)
  const float* lb = a.lse + bh * a.lpad;
  const float lse_a = lb[ra_c];
  const float lse_b = lb[rb_c];
  // column 0 of rows ra_c / rb_c; column c is c * 64 floats further
  const float* pa = a.r + ((bh * a.nqb + ra_c / kBlock) * a.ncol_alloc) * kBlock + ra_c % kBlock;
  const float* pb = a.r + ((bh * a.nqb + rb_c / kBlock) * a.ncol_alloc) * kBlock + rb_c % kBlock;
  const int cpb = a.bs / a.G;                           // columns per key block: 1 or 2
  const int jend = a.causal ? min(i + 1, a.nd) : a.nd;  // blocks past jend are 0
  const bool two_rows = a.bs > kBlock;                  // block_size 128: two rows per lane
  for (int j0 = kU * wave; j0 < a.nd; j0 += 4 * kU) {
    // Phase 1: every load of the step (no branches between them).
    int cr[kU][2];
    bool ok[kU][2];
    float va[kU][2], vb[kU][2];
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int j = j0 + u, c = j * cpb + v;
        ok[u][v] = v < cpb && j < jend && c < a.ncol;
        cr[u][v] = ok[u][v] ? c : 0;
        va[u][v] = pa[cr[u][v] * kBlock];
      }
    if (two_rows) {
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v) vb[u][v] = pb[cr[u][v] * kBlock];
    }
    // Phase 2: probabilities, with entries outside the block or the causal lists discarded
    // (causal: column c was computed for row r only where its 64-key tile is in r's list).
    float x[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      float m = 0.f;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int ctile = cr[u][v] * a.G / kBlock;
        const float ea = __builtin_amdgcn_exp2f(va[u][v] - lse_a);
        m = fmaxf(m, (ok[u][v] && ra < r1 && !(a.causal && ctile > ra / kBlock)) ? ea : 0.f);
        if (two_rows) {
          const float eb = __builtin_amdgcn_exp2f(vb[u][v] - lse_b);
          m = fmaxf(m, (ok[u][v] && rbw < r1 && !(a.causal && ctile > rbw / kBlock)) ? eb : 0.f);
        }
      }
      x[u] = m;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) x[u] = fmaxf(x[u], __shfl_xor(x[u], o));
      if (lane == u && j0 + u < a.nd) row[j0 + u] = x[u];
    }
  }
  __syncthreads();
  float s = 0.f;
  for (int j = t; j < a.nd; j += 256) s += row[j];
  part[t] = s;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (t < st) part[t] += part[t + st];
    __syncthreads();
  }
  const float tot = part[0];
  const int b = (int)(bh / a.H), h = (int)(bh - (int64_t)b * a.H);
  float* dst = a.po + b * a.po_sb + h * a.po_sh + (int64_t)i * a.po_si;
  for (int j = t; j < a.nd; j += 256) dst[j] = row[j] / tot;
}

}  // namespace

extern "C" int sa_attn_pooling_workspace(int B, int H, int L, int block_size, int64_t* bytes) {
  const char* fn = "sa_attn_pooling_workspace";
  SA_REQUIRE(bytes, "%s: null bytes", fn);
  SA_REQUIRE(B > 0 && H > 0 && L > 0, "%s: bad shape B=%d H=%d L=%d", fn, B, H, L);
  SA_REQUIRE(block_size == 32 || block_size == 64 || block_size == 128, "%s: block_size %d not in {32, 64, 128}",
             fn, block_size);
  *bytes = (int64_t)pool_layout(B, H, L, block_size).total;
  return sa::ok();
}

namespace {

// Po from the stored row maxima and log-sum-exps (pool_reduce_kernel).
int launch_pool_reduce(const PoolLayout& p, const float* r, const float* lse, int B, int H, int L, int block_size,
                       int causal, float* po, const int64_t po_strides[3], hipStream_t s, const char* fn) {
  const int nd = sa::cdiv(L, block_size);
  PoolReduceArgs ra;
  ra.r = r; ra.nqb = p.nqb; ra.ncol_alloc = p.ncol_alloc; ra.lpad = p.lpad; ra.lse = lse;
  ra.L = L; ra.bs = block_size; ra.G = p.G; ra.nd = nd; ra.ncol = sa::cdiv(L, p.G); ra.causal = causal ? 1 : 0;
  ra.H = H; ra.po = po; ra.po_sb = po_strides[0]; ra.po_sh = po_strides[1]; ra.po_si = po_strides[2];
  ra.total = (int64_t)B * H * nd;
  SA_REQUIRE(ra.total < (1LL << 31), "%s: grid too large", fn);
  hipLaunchKernelGGL(pool_reduce_kernel, dim3((unsigned)ra.total), dim3(256), (unsigned)(nd * sizeof(float)), s, ra);
  return sa::check_launch(fn);
}

int attn_pooling(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k, const int64_t k_strides[3],
                 const uint16_t* v, const int64_t v_strides[3], uint16_t* out, const int64_t out_strides[3], int B,
                 int H, int H_kv, int L, int D, int causal, float sm_scale, int block_size, float* po,
                 const int64_t po_strides[3], void* workspace, int64_t workspace_bytes, void* stream, bool fp16,
                 const char* fn) {
  SA_REQUIRE(po && po_strides && workspace, "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && L > 0, "%s: bad shape B=%d H=%d L=%d", fn, B, H, L);
  SA_REQUIRE(H_kv > 0 && H % H_kv == 0, "%s: H_kv=%d must divide H=%d", fn, H_kv, H);
  SA_REQUIRE(block_size == 32 || block_size == 64 || block_size == 128, "%s: block_size %d not in {32, 64, 128}",
             fn, block_size);
  const PoolLayout p = pool_layout(B, H, L, block_size);
  const int nd = sa::cdiv(L, block_size);
  if (nd > kPoolMaxNd) return sa::fail(SA_ERR_UNSUPPORTED, "%s: %d blocks per row > %d", fn, nd, kPoolMaxNd);
  SA_REQUIRE(workspace_bytes >= (int64_t)p.total, "%s: workspace of %lld bytes < %lld", fn,
             (long long)workspace_bytes, (long long)p.total);
  SA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "%s: workspace not 256-byte aligned", fn);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  PoolListArgs la;
  la.idx = reinterpret_cast<int32_t*>(ws + p.idx);
  la.cnt = reinterpret_cast<int32_t*>(ws + p.cnt);
  la.slot = reinterpret_cast<int32_t*>(ws + p.slot);
  la.mask = reinterpret_cast<uint64_t*>(ws + p.mask);
  la.nqb = p.nqb; la.nkb = p.nkb; la.causal = causal ? 1 : 0;
  hipStream_t s = sa::as_stream(stream);
  const int64_t n_list = std::max<int64_t>((int64_t)p.nqb * p.nkb, kBlock);
  hipLaunchKernelGGL(pool_lists_kernel, dim3((unsigned)((n_list + 255) / 256)), dim3(256), 0, s, la);
  if (int rc = sa::check_launch(fn)) return rc;
  float* r = reinterpret_cast<float*>(ws + p.r);
  float* lse = reinterpret_cast<float*>(ws + p.lse);
  if (block_size == p.G) {
    // 32- or 64-token blocks: one wave's 64 query rows are one or two whole Po rows, so
    // the attention kernel forms them itself (no log-sum-exp buffer, no reduce launch).
    const PoolOut po_out{po, po_strides[0], po_strides[1], po_strides[2], nd, causal ? 1 : 0};
    return launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, L, L, D, la.idx, la.cnt,
                      p.nkb, true, causal ? la.slot : nullptr, causal ? la.mask : nullptr, nullptr, nullptr,
                      sm_scale, nullptr, 0, nullptr, 0, nullptr, 0, stream, fn, H / H_kv, p.G, r, nullptr, &po_out,
                      fp16);
  }
  if (int rc = launch_fwd(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, L, L, D, la.idx, la.cnt,
                          p.nkb, true, causal ? la.slot : nullptr, causal ? la.mask : nullptr, nullptr, nullptr,
                          sm_scale, nullptr, 0, nullptr, 0, nullptr, 0, stream, fn, H / H_kv, p.G, r, lse, nullptr,
                          fp16))
    return rc;
  return launch_pool_reduce(p, r, lse, B, H, L, block_size, causal, po, po_strides, s, fn);
}

// fp32 q, k, v (the reference's own arithmetic for attn_with_pooling, which computes in fp32):
// the fp32 kernel in pooling mode stores the row maxima and log-sum-exps, the reduce kernel
// forms Po for every block size.
int attn_pooling_f32(const float* q, const int64_t q_strides[3], const float* k, const int64_t k_strides[3],
                     const float* v, const int64_t v_strides[3], float* out, const int64_t out_strides[3], int B,
                     int H, int H_kv, int L, int D, int causal, float sm_scale, int block_size, float* po,
                     const int64_t po_strides[3], void* workspace, int64_t workspace_bytes, void* stream,
                     const char* fn) {
  SA_REQUIRE(po && po_strides && workspace, "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && L > 0, "%s: bad shape B=%d H=%d L=%d", fn, B, H, L);
  SA_REQUIRE(H_kv > 0 && H % H_kv == 0, "%s: H_kv=%d must divide H=%d", fn, H_kv, H);
  SA_REQUIRE(block_size == 32 || block_size == 64 || block_size == 128, "%s: block_size %d not in {32, 64, 128}",
             fn, block_size);
  const PoolLayout p = pool_layout(B, H, L, block_size);
  const int nd = sa::cdiv(L, block_size);
  if (nd > kPoolMaxNd) return sa::fail(SA_ERR_UNSUPPORTED, "%s: %d blocks per row > %d", fn, nd, kPoolMaxNd);
  SA_REQUIRE(workspace_bytes >= (int64_t)p.total, "%s: workspace of %lld bytes < %lld", fn,
             (long long)workspace_bytes, (long long)p.total);
  SA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "%s: workspace not 256-byte aligned", fn);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  PoolListArgs la;
  la.idx = reinterpret_cast<int32_t*>(ws + p.idx);
  la.cnt = reinterpret_cast<int32_t*>(ws + p.cnt);
  la.slot = reinterpret_cast<int32_t*>(ws + p.slot);
  la.mask = reinterpret_cast<uint64_t*>(ws + p.mask);
  la.nqb = p.nqb; la.nkb = p.nkb; la.causal = causal ? 1 : 0;
  hipStream_t s = sa::as_stream(stream);
  const int64_t n_list = std::max<int64_t>((int64_t)p.nqb * p.nkb, kBlock);
  hipLaunchKernelGGL(pool_lists_kernel, dim3((unsigned)((n_list + 255) / 256)), dim3(256), 0, s, la);
  if (int rc = sa::check_launch(fn)) return rc;
  float* r = reinterpret_cast<float*>(ws + p.r);
  float* lse = reinterpret_cast<float*>(ws + p.lse);
  if (int rc = sa::attn_f32_pooling(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, L, D, la.idx,
                                    la.cnt, p.nkb, H / H_kv, causal != 0, sm_scale, p.G, r, lse, stream, fn))
    return rc;
  return launch_pool_reduce(p, r, lse, B, H, L, block_size, causal, po, po_strides, s, fn);
}

}  // namespace

extern "C" int sa_attn_pooling_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                   const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                   uint16_t* out, const int64_t out_strides[3], int B, int H, int H_kv, int L, int D,
                                   int causal, float sm_scale, int block_size, float* po,
                                   const int64_t po_strides[3], void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  return attn_pooling(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, H_kv, L, D, causal, sm_scale,
                      block_size, po, po_strides, workspace, workspace_bytes, stream, false, "sa_attn_pooling_fwd");
}

extern "C" int sa_attn_pooling_fwd_f32(const float* q, const int64_t q_strides[3], const float* k,
                                       const int64_t k_strides[3], const float* v, const int64_t v_strides[3],
                                       float* out, const int64_t out_strides[3], int B, int H, int H_kv, int L, int D,
                                       int causal, float sm_scale, int block_size, float* po,
                                       const int64_t po_strides[3], void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  return attn_pooling_f32(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, H_kv, L, D, causal,
                          sm_scale, block_size, po, po_strides, workspace, workspace_bytes, stream,
                          "sa_attn_pooling_fwd_f32");
}

extern "C" int sa_attn_pooling_fwd_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                       const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                                       uint16_t* out, const int64_t out_strides[3], int B, int H, int H_kv, int L,
                                       int D, int causal, float sm_scale, int block_size, float* po,
                                       const int64_t po_strides[3], void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  return attn_pooling(q, q_strides, k, k_strides, v, v_strides, out, out_strides, B, H, H_kv, L, D, causal, sm_scale,
                      block_size, po, po_strides, workspace, workspace_bytes, stream, true, "sa_attn_pooling_fwd_f16");
}
