// Dense block mask -> compacted per-row kv lists (one wave per list row).
//
// Replaces the per-program scan of the boolean block mask inside the reference Triton
// kernel (special_attentions/utils/block_sparse_attn_kernel.py:69-70, 163-199): the list is
// built once per call and then drives the attention kernel's loads.
#include "sa_common.h"

namespace {

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

// Block masks of other block shapes (BLOCK_M x BLOCK_N, powers of two): one wave per 64-row
// tile row (b, h, m), lane over 64-key tiles. A 64 x 64 tile covers cr x cc mask cells (cr =
// 64 / BLOCK_M rows of cells when BLOCK_M < 64, else 1; likewise cc); cell (i, j) is
// mask[b, h, m0 + i, n0 + j] with m0 = m * 64 / BLOCK_M (cell rows of the tile) and n0 the
// same for keys. Cells whose first query row or key lies past Lq or Lk do not exist: they
// neither keep a tile nor cut it. A tile is listed when one of its existing cells is set;
// its slot is -1 when all of them are, else the pattern of set cells (bit i * cc + j), an
// index into the sa_cell_tile_masks table.
struct CellArgs {
  const uint8_t* mask;
  int64_t s0, s1, s2, s3;
  int H, Lq, Lk, bm, bn, nqb, nkb;
  int64_t rows;
  int32_t* kv_idx;
  int32_t* kv_slot;
  int max_cnt;
  int32_t* kv_cnt;
};

__global__ __launch_bounds__(256) void mask_cells_to_list_kernel(CellArgs a) {
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (row >= a.rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t bh = row / a.nqb;
  const int m = (int)(row - bh * a.nqb);
  const int64_t b = bh / a.H;
  const int64_t h = bh - b * a.H;
  const int cr = a.bm < 64 ? 64 / a.bm : 1, cc = a.bn < 64 ? 64 / a.bn : 1;
  const int m0 = (int)((int64_t)m * 64 / a.bm);
  const uint8_t* base = a.mask + b * a.s0 + h * a.s1;
  int32_t* out = a.kv_idx + row * a.max_cnt;
  int32_t* out_slot = a.kv_slot ? a.kv_slot + row * a.max_cnt : nullptr;
  int total = 0;
  for (int n0t = 0; n0t < a.nkb; n0t += 64) {
    const int n = n0t + lane;
    int bits = 0, exist = 0;
    if (n < a.nkb) {
      const int c0 = (int)((int64_t)n * 64 / a.bn);
      for (int i = 0; i < cr; ++i) {
        if ((int64_t)m * 64 + (int64_t)i * a.bm >= a.Lq) break;
        for (int j = 0; j < cc; ++j) {
          if ((int64_t)n * 64 + (int64_t)j * a.bn >= a.Lk) break;
          exist |= 1 << (i * cc + j);
          if (base[(int64_t)(m0 + i) * a.s2 + (int64_t)(c0 + j) * a.s3]) bits |= 1 << (i * cc + j);
        }
      }
    }
    const bool on = bits != 0;
    const uint64_t bal = __ballot(on);
    const int pre = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
    if (on) {
      out[total + pre] = n;
      if (out_slot) out_slot[total + pre] = bits == exist ? -1 : bits;
    }
    total += __popcll(bal);
  }
  if (lane == 0) a.kv_cnt[row] = total;
}

bool pow2_block(int x) { return x >= 16 && x <= 1024 && (x & (x - 1)) == 0; }

}  // namespace

extern "C" int sa_cell_tile_masks(int block_m, int block_n, uint64_t* masks, int64_t* n_patterns) {
  const char* fn = "sa_cell_tile_masks";
  SA_REQUIRE(n_patterns, "%s: null n_patterns", fn);
  SA_REQUIRE(pow2_block(block_m) && pow2_block(block_n), "%s: block sizes %d x %d (powers of two, 16..1024)", fn,
             block_m, block_n);
  const int bmc = block_m < 64 ? block_m : 64, bnc = block_n < 64 ? block_n : 64;
  const int cc = 64 / bnc, cells = (64 / bmc) * cc;
  *n_patterns = (int64_t)1 << cells;
  if (!masks) return sa::ok();
  for (int64_t p = 0; p < *n_patterns; ++p)
    for (int r = 0; r < 64; ++r) {
      uint64_t w = 0;
      for (int k = 0; k < 64; ++k)
        if ((p >> ((r / bmc) * cc + k / bnc)) & 1) w |= 1ull << k;
      masks[p * 64 + r] = w;
    }
  return sa::ok();
}

extern "C" int sa_mask_cells_to_kv_list(const uint8_t* mask, const int64_t mask_strides[4], int B, int H, int Lq,
                                        int Lk, int block_m, int block_n, int32_t* kv_idx, int32_t* kv_slot,
                                        int max_cnt, int32_t* kv_cnt, void* stream) {
  const char* fn = "sa_mask_cells_to_kv_list";
  SA_REQUIRE(mask && mask_strides && kv_idx && kv_cnt, "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && Lq > 0 && Lk > 0, "%s: bad shape B=%d H=%d Lq=%d Lk=%d", fn, B, H, Lq, Lk);
  SA_REQUIRE(pow2_block(block_m) && pow2_block(block_n), "%s: block sizes %d x %d (powers of two, 16..1024)", fn,
             block_m, block_n);
  SA_REQUIRE(kv_slot || (block_m >= 64 && block_n >= 64), "%s: kv_slot needed for blocks smaller than 64", fn);
  CellArgs a;
  a.mask = mask; a.s0 = mask_strides[0]; a.s1 = mask_strides[1]; a.s2 = mask_strides[2]; a.s3 = mask_strides[3];
  a.H = H; a.Lq = Lq; a.Lk = Lk; a.bm = block_m; a.bn = block_n;
  a.nqb = sa::cdiv(Lq, 64); a.nkb = sa::cdiv(Lk, 64);
  SA_REQUIRE(max_cnt >= a.nkb, "%s: max_cnt=%d < %d", fn, max_cnt, a.nkb);
  a.rows = (int64_t)B * H * a.nqb;
  a.kv_idx = kv_idx; a.kv_slot = kv_slot; a.max_cnt = max_cnt; a.kv_cnt = kv_cnt;
  const int64_t blocks = (a.rows + 3) / 4;
  SA_REQUIRE(blocks < (1LL << 31), "%s: too many rows", fn);
  hipLaunchKernelGGL(mask_cells_to_list_kernel, dim3((unsigned)blocks), dim3(256), 0, sa::as_stream(stream), a);
  return sa::check_launch(fn);
}

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
