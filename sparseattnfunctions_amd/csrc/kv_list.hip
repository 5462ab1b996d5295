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
