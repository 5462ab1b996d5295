// Frame-factored block masks of the reference's backup block-sparse path for gfx950.
//
// Replaces, in special_attentions/utils/mask_related.py:
//   get_inner_frame_mask (:344-395): the 64 x 64 cell sums of a frame's attention, here formed
//     from per-row key-block masses (the attention kernel's output with a 0/1 key-block
//     indicator V) by row_group_sums_kernel;
//   get_block_mask (:397-404): the Kronecker product of the frame-level mask with the
//     block-level inner-frame mask, padded with dense text blocks, by kron_mask_kernel.
// The energy cuts between them run in energy_list_kernel (estimator.hip).
//
// row_group_sums_kernel: one wave per (b*h, group of R rows); lane c adds column col0 + c of
// the group's rows in ascending row order (fp32), so a wave reads whole 128-byte rows.
// kron_mask_kernel: one thread per output element.
#include "sa_common.h"

namespace {

struct RowSumArgs {
  const uint16_t* x;
  int64_t sb, sh, sl;
  int H, L, R, groups, col0, ncols;
  float* out;  // [B*H][groups][ncols]
  int64_t total;  // B*H*groups
};

__global__ __launch_bounds__(64) void row_group_sums_kernel(RowSumArgs a) {
  const int64_t w = blockIdx.x;
  if (w >= a.total) return;
  const int lane = threadIdx.x;
  const int64_t bh = w / a.groups;
  const int g = (int)(w - bh * a.groups);
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int r0 = g * a.R, r1 = min(a.L, r0 + a.R);
  const bool active = lane < a.ncols;
  const uint16_t* base = a.x + b * a.sb + h * a.sh + a.col0 + (active ? lane : 0);
  float s = 0.f;
  for (int r = r0; r < r1; ++r) s += __uint_as_float((uint32_t)base[(int64_t)r * a.sl] << 16);
  if (active) a.out[w * a.ncols + lane] = s;
}

struct KronArgs {
  const uint8_t* frame;  // [BH][F][F]
  const uint8_t* inner;  // [BH][Ri][Ci]
  int F, Ri, Ci, pad;
  int rows, cols;  // F*Ri + pad, F*Ci + pad
  float* out;      // [BH][rows][cols]
  int64_t total;
};

__global__ __launch_bounds__(256) void kron_mask_kernel(KronArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int64_t per = (int64_t)a.rows * a.cols;
  const int64_t bh = i / per;
  const int64_t rc = i - bh * per;
  const int r = (int)(rc / a.cols), c = (int)(rc - (int64_t)r * a.cols);
  float v = 1.f;  // the padded (text) rows and columns are dense
  if (r < a.F * a.Ri && c < a.F * a.Ci) {
    const int fa = r / a.Ri, d = r - fa * a.Ri;
    const int fc = c / a.Ci, e = c - fc * a.Ci;
    const bool on = a.frame[(bh * a.F + fa) * a.F + fc] != 0 && a.inner[(bh * a.Ri + d) * a.Ci + e] != 0;
    v = on ? 1.f : 0.f;
  }
  a.out[i] = v;
}

}  // namespace

extern "C" int sa_row_group_sums(const uint16_t* x, const int64_t x_strides[3], int B, int H, int L,
                                 int rows_per_group, int col0, int ncols, float* out, void* stream) {
  const char* fn = "sa_row_group_sums";
  SA_REQUIRE(x && x_strides && out, "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && L > 0 && rows_per_group > 0, "%s: bad shape B=%d H=%d L=%d R=%d", fn, B, H, L,
             rows_per_group);
  SA_REQUIRE(col0 >= 0 && ncols >= 1 && ncols <= 64 && col0 + ncols <= 64, "%s: columns [%d, %d) outside [0, 64)",
             fn, col0, col0 + ncols);
  RowSumArgs a;
  a.x = x; a.sb = x_strides[0]; a.sh = x_strides[1]; a.sl = x_strides[2];
  a.H = H; a.L = L; a.R = rows_per_group; a.groups = sa::cdiv(L, rows_per_group);
  a.col0 = col0; a.ncols = ncols; a.out = out;
  a.total = (int64_t)B * H * a.groups;
  SA_REQUIRE(a.total < (1LL << 31), "%s: grid too large", fn);
  hipLaunchKernelGGL(row_group_sums_kernel, dim3((unsigned)a.total), dim3(64), 0, sa::as_stream(stream), a);
  return sa::check_launch(fn);
}

extern "C" int sa_kron_block_mask(const uint8_t* frame_mask, const uint8_t* inner_mask, int BH, int F, int Ri,
                                  int Ci, int pad, float* out, void* stream) {
  const char* fn = "sa_kron_block_mask";
  SA_REQUIRE(frame_mask && inner_mask && out, "%s: null pointer", fn);
  SA_REQUIRE(BH > 0 && F > 0 && Ri > 0 && Ci > 0 && pad >= 0, "%s: bad shape BH=%d F=%d Ri=%d Ci=%d pad=%d", fn, BH,
             F, Ri, Ci, pad);
  KronArgs a;
  a.frame = frame_mask; a.inner = inner_mask;
  a.F = F; a.Ri = Ri; a.Ci = Ci; a.pad = pad;
  a.rows = F * Ri + pad; a.cols = F * Ci + pad;
  a.out = out;
  a.total = (int64_t)BH * a.rows * a.cols;
  SA_REQUIRE((a.total + 255) / 256 < (1LL << 31), "%s: grid too large", fn);
  hipLaunchKernelGGL(kron_mask_kernel, dim3((unsigned)((a.total + 255) / 256)), dim3(256), 0, sa::as_stream(stream),
                     a);
  return sa::check_launch(fn);
}
