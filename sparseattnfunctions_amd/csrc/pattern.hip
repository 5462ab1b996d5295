// Frame-pattern attention of the 1.5-5B geometry (ParternAttentionColVersion_V2,
// partern_attention.py:318-456) for gfx950: the small per-head planning kernels and the final
// combine. The attention-shaped parts (text rows, first-frame masses, sampled frame maps,
// video-to-text attention, per-frame attention) run in the block-sparse attention kernel; the
// per-segment probability masses come out of it by attending to a 0/1 segment-indicator V.
//
//   plan: maps_kernel      img2text_map[f] and img2img_map[f1][f2] from the sampled
//                          attention's segment masses (get_weight_for_patch, :321-358);
//         fstats_kernel    per head: sum, min and max of each column of the first-frame masses
//                          (text mass for modify_factor_text, frame-i mass for frame i);
//         select_kernel    constrained_mod_factor (:262-315) as a per-element affine map +
//                          clamp, with the cross-head "any head out of range" decision, and
//                          the case of every key frame (first-frame masses where
//                          img2img_map[0][i] >= 0.1, :435);
//         qidx_kernel      the per-head query-row gather table (query frame = argmax over the
//                          img2img_map column, or the first frame);
//   combine_kernel         out = sum_i img2img[f1][i] * scale_i(r) * O_i[r]
//                                + img2text[f1] * mft(r) * O_text[f1*S + r]   (:447-452).
#include "sa_common.h"

namespace {

constexpr int kD = 64;
constexpr int kMaxF = 16;  // frames handled (the reference uses 11)

__device__ inline float bf(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// ---------------------------------------------------------------------------------------
// maps_kernel: one wave per (bh, f1). Masses m[row][c] (bf16, column 0 = text, 1 + f2 =
// frame f2) of the ns sampled rows of frame f1: img2text[f1] = sum_rows m[.][0] / ns,
// img2img[f1][f2] = sum_rows m[.][1 + f2] / ns. Lane l adds rows l, l + 64, ... (16-byte
// loads of columns 0-15, and column 16 when F = 16); the lanes' sums are then added by a
// fixed butterfly.
struct MapsArgs {
  const uint16_t* m;
  int64_t m_sb, m_sh, m_sl;
  int H, F, ns;
  int vec_ok;       // rows 16-byte aligned
  float* img2text;  // [BH][F]
  float* img2img;   // [BH][F][F]
  int64_t total;    // BH * F
};

__global__ __launch_bounds__(64) void maps_kernel(MapsArgs a) {
  const int64_t w = blockIdx.x;
  if (w >= a.total) return;
  const int lane = threadIdx.x;
  const int64_t bh = w / a.F;
  const int f1 = (int)(w - bh * a.F);
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int ncol = a.F + 1;  // <= 17
  const uint16_t* base = a.m + b * a.m_sb + h * a.m_sh + (int64_t)f1 * a.ns * a.m_sl;
  float s[17];
#pragma unroll
  for (int c = 0; c < 17; ++c) s[c] = 0.f;
  for (int r = lane; r < a.ns; r += 64) {
    const uint16_t* row = base + (int64_t)r * a.m_sl;
    if (a.vec_ok) {
      const uint4 w0 = *reinterpret_cast<const uint4*>(row);
      const uint4 w1 = *reinterpret_cast<const uint4*>(row + 8);
      const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        s[2 * q] += __uint_as_float(u[q] << 16);
        s[2 * q + 1] += __uint_as_float(u[q] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 16; ++c) s[c] += c < ncol ? bf(row[c]) : 0.f;
    }
    if (ncol > 16) s[16] += bf(row[16]);
  }
#pragma unroll
  for (int c = 0; c < 17; ++c) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s[c] += __shfl_xor(s[c], o);
  }
  if (lane == 0) {
    const float inv = 1.f / (float)a.ns;
    a.img2text[bh * a.F + f1] = s[0] * inv;
#pragma unroll
    for (int c = 1; c < 17; ++c)
      if (c < ncol) a.img2img[(bh * a.F + f1) * a.F + (c - 1)] = s[c] * inv;
  }
}

// ---------------------------------------------------------------------------------------
// fstats_kernel: one workgroup of 256 per bh; x_j[r] = mass column j of first-frame row r
// (j = 0 text, 1 + i frame i). Writes sum, min, max of every x_j over r < S. Thread t takes
// rows t, t + 256, ... (16-byte loads of columns 0-15, column 16 when there are 17); the
// threads' partials are combined by a fixed butterfly per wave, then the 4 waves in order.
struct StatsArgs {
  const uint16_t* m;
  int64_t m_sb, m_sh, m_sl;
  int H, S, n_fac;
  int vec_ok;     // rows 16-byte aligned and at least 16 elements apart
  float* stats;   // [BH][n_fac][3]
  int64_t total;  // BH
};

__global__ __launch_bounds__(256) void fstats_kernel(StatsArgs a) {
  __shared__ float red[4][17][3];
  const int64_t bh = blockIdx.x;
  if (bh >= a.total) return;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const uint16_t* base = a.m + b * a.m_sb + h * a.m_sh;
  float su[17], mn[17], mx[17];
#pragma unroll
  for (int c = 0; c < 17; ++c) {
    su[c] = 0.f;
    mn[c] = INFINITY;
    mx[c] = -INFINITY;
  }
  for (int r = t; r < a.S; r += 256) {
    const uint16_t* row = base + (int64_t)r * a.m_sl;
    float x[17];
    if (a.vec_ok) {
      const uint4 w0 = *reinterpret_cast<const uint4*>(row);
      const uint4 w1 = *reinterpret_cast<const uint4*>(row + 8);
      const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        x[2 * q] = __uint_as_float(u[q] << 16);
        x[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 16; ++c) x[c] = c < a.n_fac ? bf(row[c]) : 0.f;
    }
    x[16] = a.n_fac > 16 ? bf(row[16]) : 0.f;
#pragma unroll
    for (int c = 0; c < 17; ++c) {
      su[c] += x[c];
      mn[c] = fminf(mn[c], x[c]);
      mx[c] = fmaxf(mx[c], x[c]);
    }
  }
#pragma unroll
  for (int c = 0; c < 17; ++c) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      su[c] += __shfl_xor(su[c], o);
      mn[c] = fminf(mn[c], __shfl_xor(mn[c], o));
      mx[c] = fmaxf(mx[c], __shfl_xor(mx[c], o));
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int c = 0; c < 17; ++c) {
      red[wave][c][0] = su[c];
      red[wave][c][1] = mn[c];
      red[wave][c][2] = mx[c];
    }
  }
  __syncthreads();
  if (t < a.n_fac) {
    float* o = a.stats + (bh * a.n_fac + t) * 3;
    o[0] = ((red[0][t][0] + red[1][t][0]) + red[2][t][0]) + red[3][t][0];
    o[1] = fminf(fminf(red[0][t][1], red[1][t][1]), fminf(red[2][t][1], red[3][t][1]));
    o[2] = fmaxf(fmaxf(red[0][t][2], red[1][t][2]), fmaxf(red[2][t][2], red[3][t][2]));
  }
}

// ---------------------------------------------------------------------------------------
// select_kernel: one thread per (bh, factor j) plus the per-head frame choices.
// Factor j of head bh maps a first-frame mass x to the modify factor
//   mf = x / mean_r(x)  then constrained_mod_factor(mf, lo_j, hi_j):
//   if no head has min(mf) < lo or max(mf) > hi: mf unchanged (mode 0);
//   else per head: range = max - min (a head with range < 1e-6 keeps mf, mode 1), otherwise
//   the affine map of [min, max] onto [max(min, lo), min(max, hi)] rescaled to keep sum(mf)
//   (mode 2); modes 1 and 2 are clamped to [lo, hi].
// fac[bh][j] = {1 / mean, alpha, beta, mode}: mf' = clamp(alpha * x / mean + beta) (mode 2).
struct SelectArgs {
  const float* stats;  // [BH][n_fac][3]
  const float* img2img;  // [BH][F][F]
  int BH, F, S, T, n_fac;
  float lo_text, hi_text, lo_frame, hi_frame, map_thr;
  float* fac;       // [BH][n_fac][4]
  int32_t* frame_case;  // [BH][F]: 0 = selected query frame, 1 = first-frame masses
  float* inv_map0;  // [BH][F]: 1 / img2img[0][i]
  int32_t* q_idx;   // [BH][F*S] query token of selected-frame row (i*S + r)
};

__global__ __launch_bounds__(256) void select_kernel(SelectArgs a) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int n1 = a.BH * a.n_fac;
  if (t < n1) {
    const int bh = t / a.n_fac, j = t - bh * a.n_fac;
    const float lo = j == 0 ? a.lo_text : a.lo_frame;
    const float hi = j == 0 ? a.hi_text : a.hi_frame;
    // The cross-head decision of constrained_mod_factor (one factor j, every head).
    bool adjust = false;
    for (int o = 0; o < a.BH; ++o) {
      const float* st = a.stats + ((int64_t)o * a.n_fac + j) * 3;
      const float mean = st[0] / (float)a.S;
      adjust |= (st[1] / mean < lo) || (st[2] / mean > hi);
    }
    const float* st = a.stats + ((int64_t)bh * a.n_fac + j) * 3;
    const float mean = st[0] / (float)a.S;
    const float inv = 1.f / mean;
    const float osum = st[0] * inv;  // sum of mf
    const float cmin = st[1] * inv, cmax = st[2] * inv;
    float alpha = 1.f, beta = 0.f, mode = 0.f;
    if (adjust) {
      const float range = cmax - cmin;
      if (range < 1e-6f) {
        mode = 1.f;
      } else {
        const float tmin = cmin < lo ? lo : cmin;
        const float tmax = cmax > hi ? hi : cmax;
        const float sl = (tmax - tmin) / range;
        // sum of the scaled values: sum((mf - cmin) * sl + tmin) over S rows
        const float nsum = (osum - (float)a.S * cmin) * sl + (float)a.S * tmin;
        const float g = osum / nsum;
        alpha = sl * g;
        beta = (tmin - cmin * sl) * g;
        mode = 2.f;
      }
    }
    float* o = a.fac + ((int64_t)bh * a.n_fac + j) * 4;
    o[0] = inv;
    o[1] = alpha;
    o[2] = beta;
    o[3] = mode;
  }
  // Per (bh, key frame i): query frame and case.
  const int t2 = t - n1;
  if (t2 >= 0 && t2 < a.BH * a.F) {
    const int bh = t2 / a.F, i = t2 - bh * a.F;
    const float* mp = a.img2img + (int64_t)bh * a.F * a.F;
    const float m0 = mp[i];  // img2img[0][i]
    const bool first = !(m0 < a.map_thr);
    a.frame_case[t2] = first ? 1 : 0;
    a.inv_map0[t2] = 1.f / m0;
  }
}

// The query row gathered for selected row i*S + r of head bh: T + sel(bh, i)*S + r, with
// sel = 0 when the first-frame masses are used for key frame i, else the argmax of column i.
__global__ __launch_bounds__(256) void qidx_kernel(SelectArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = (int64_t)a.F * a.S;
  if (e >= (int64_t)a.BH * per) return;
  const int64_t bh = e / per;
  const int j = (int)(e - bh * per);
  const int i = j / a.S, r = j - i * a.S;
  const float* mp = a.img2img + bh * a.F * a.F;
  int sel = 0;
  if (mp[i] < a.map_thr) {
    float best = mp[i];
    for (int f1 = 1; f1 < a.F; ++f1) {
      const float x = mp[f1 * a.F + i];
      if (x > best) {
        best = x;
        sel = f1;
      }
    }
  }
  a.q_idx[e] = a.T + sel * a.S + r;
}

__device__ inline float apply_fac(const float* f, float x, float lo, float hi) {
  const float mf = x * f[0];
  if (f[3] == 0.f) return mf;
  const float y = f[3] == 2.f ? fmaf(f[1], mf, f[2]) : mf;
  return fminf(fmaxf(y, lo), hi);
}

// ---------------------------------------------------------------------------------------
// combine_kernel: one workgroup of 256 per (bh, 32 first-frame rows r): lane = 8 rows x ...
// Thread (row ri = tid / 8, dims 8*(tid % 8) .. +7) accumulates all F output frames of its
// row: out[T + f1*S + r] = sum_i img2img[f1][i] * s_i(r) * O_i[r] + img2text[f1] * mft(r) *
// O_text[f1*S + r], where s_i(r) = mf_i(r) (case 0) or mass_i(r) / img2img[0][i] (case 1).
struct CombineArgs {
  const uint16_t* of;   // [B,H,F*S,64] per-frame attention outputs
  int64_t of_sb, of_sh, of_sl;
  const uint16_t* ot;   // [B,H,F*S,64] video-to-text attention
  int64_t ot_sb, ot_sh, ot_sl;
  const uint16_t* mass;  // [B,H,S,64] first-frame masses (col 0 text, 1 + i frame i)
  int64_t m_sb, m_sh, m_sl;
  const float* img2text;  // [BH][F]
  const float* img2img;   // [BH][F][F]
  const float* fac;       // [BH][1+F][4]
  const int32_t* frame_case;
  const float* inv_map0;
  uint16_t* out;          // [B,H,T+F*S,64] (rows >= T written)
  int64_t o_sb, o_sh, o_sl;
  int H, F, S, T;
  float lo_text, hi_text, lo_frame, hi_frame;
  int rows_per_wg;  // 32
  int64_t total;    // BH * ceil(S / 32)
};

__device__ inline uint32_t pack_bf16(float a, float b) {
  const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
  const uint32_t ra = (ua + 0x7fffu + ((ua >> 16) & 1u)) >> 16;  // round to nearest even
  const uint32_t rb = (ub + 0x7fffu + ((ub >> 16) & 1u)) >> 16;
  return ra | (rb << 16);
}

template <int F>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
  const int64_t w = blockIdx.x;
  if (w >= a.total) return;
  const int nrb = (a.S + 31) / 32;
  const int64_t bh = w / nrb;
  const int r = (int)(w - bh * nrb) * 32 + (threadIdx.x >> 3);
  if (r >= a.S) return;
  const int c8 = threadIdx.x & 7;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const float* fac = a.fac + (int64_t)bh * (1 + F) * 4;
  const uint16_t* mrow = a.mass + b * a.m_sb + h * a.m_sh + (int64_t)r * a.m_sl;
  // Per key frame i: s_i(r) * O_i[r][dims]
  float vs[F][8];
#pragma unroll
  for (int i = 0; i < F; ++i) {
    const float x = bf(mrow[1 + i]);
    const float s = a.frame_case[bh * F + i] ? x * a.inv_map0[bh * F + i]
                                             : apply_fac(fac + (1 + i) * 4, x, a.lo_frame, a.hi_frame);
    const uint4 o = *reinterpret_cast<const uint4*>(a.of + b * a.of_sb + h * a.of_sh +
                                                    ((int64_t)i * a.S + r) * a.of_sl + 8 * c8);
    const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vs[i][2 * e] = s * __uint_as_float(ow[e] << 16);
      vs[i][2 * e + 1] = s * __uint_as_float(ow[e] & 0xffff0000u);
    }
  }
  const float mft = apply_fac(fac, bf(mrow[0]), a.lo_text, a.hi_text);
  const float* mp = a.img2img + (int64_t)bh * F * F;
  for (int f1 = 0; f1 < F; ++f1) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < F; ++i) {
      const float wgt = mp[f1 * F + i];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(wgt, vs[i][e], acc[e]);
    }
    const float tw = a.img2text[bh * F + f1] * mft;
    const uint4 o = *reinterpret_cast<const uint4*>(a.ot + b * a.ot_sb + h * a.ot_sh +
                                                    ((int64_t)f1 * a.S + r) * a.ot_sl + 8 * c8);
    const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
    uint32_t res[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = fmaf(tw, __uint_as_float(ow[e] << 16), acc[2 * e]);
      const float hi = fmaf(tw, __uint_as_float(ow[e] & 0xffff0000u), acc[2 * e + 1]);
      res[e] = pack_bf16(lo, hi);
    }
    *reinterpret_cast<uint4*>(a.out + b * a.o_sb + h * a.o_sh + ((int64_t)a.T + (int64_t)f1 * a.S + r) * a.o_sl +
                              8 * c8) = make_uint4(res[0], res[1], res[2], res[3]);
  }
}

// ---------------------------------------------------------------------------------------
// Per-head token gather: out[b,h,j] = x[b,h, idx[(b*H + h)*L_out + j]] (zero row outside
// [0, L_in)).
__global__ __launch_bounds__(256) void gather_heads_kernel(const uint16_t* x, int64_t x_sb, int64_t x_sh,
                                                           int64_t x_sl, int L_in, const int32_t* idx, int L_out,
                                                           int H, int64_t rows, uint16_t* out, int64_t o_sb,
                                                           int64_t o_sh, int64_t o_sl) {
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
  if (row >= rows) return;
  const int c8 = threadIdx.x & 7;
  const int64_t bh = row / L_out;
  const int j = (int)(row - bh * L_out);
  const int64_t b = bh / H, h = bh - b * H;
  const int src = idx[row];
  uint4 w = make_uint4(0u, 0u, 0u, 0u);
  if ((unsigned)src < (unsigned)L_in)
    w = *reinterpret_cast<const uint4*>(x + b * x_sb + h * x_sh + (int64_t)src * x_sl + 8 * c8);
  *reinterpret_cast<uint4*>(out + b * o_sb + h * o_sh + (int64_t)j * o_sl + 8 * c8) = w;
}

int check_bf16_rows(const void* p, const int64_t s[3], const char* fn) {
  SA_REQUIRE(p && s, "%s: null tensor", fn);
  if (reinterpret_cast<uintptr_t>(p) % 16) return sa::fail(SA_ERR_UNSUPPORTED, "%s: base not 16-byte aligned", fn);
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8) return sa::fail(SA_ERR_UNSUPPORTED, "%s: strides must be multiples of 8", fn);
  return SA_OK;
}


// ---------------------------------------------------------------------------------------
// constrained_mod_factor (partern_attention.py:262-315) on a standalone factor tensor
// x [BH][L] fp32. modfac_stats_kernel: one workgroup per head, fixed-order sum (thread t adds
// entries t, t + 256, ... in order, then a tree over the 256 partials), min and max.
// modfac_apply_kernel: the "any head out of range" decision from every head's statistics
// (once per workgroup of 2048 elements), then per element the affine map of [min, max] onto [max(min, lo), min(max, hi)], the
// rescale to the original sum (the mapped sum in closed form, (sum - L min) / range *
// (tmax - tmin) + L tmin), heads with range < 1e-6 unchanged, and the clamp to [lo, hi].
struct ModStatsArgs {
  const float* x;
  int64_t L;
  float* stats;  // [BH][3]: sum, min, max
};

__global__ __launch_bounds__(256) void modfac_stats_kernel(ModStatsArgs a) {
  __shared__ float ps[256], pmn[256], pmx[256];
  const int64_t bh = blockIdx.x;
  const int t = threadIdx.x;
  const float* x = a.x + bh * a.L;
  float s = 0.f, mn = INFINITY, mx = -INFINITY;
  for (int64_t i = t; i < a.L; i += 256) {
    const float v = x[i];
    s += v;
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  ps[t] = s; pmn[t] = mn; pmx[t] = mx;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (t < st) {
      ps[t] += ps[t + st];
      pmn[t] = fminf(pmn[t], pmn[t + st]);
      pmx[t] = fmaxf(pmx[t], pmx[t + st]);
    }
    __syncthreads();
  }
  if (t == 0) {
    a.stats[bh * 3 + 0] = ps[0];
    a.stats[bh * 3 + 1] = pmn[0];
    a.stats[bh * 3 + 2] = pmx[0];
  }
}

struct ModApplyArgs {
  const float* x;
  const float* stats;
  int BH;
  int64_t L;
  float lo, hi;
  float* out;
};

constexpr int kModApplyPerBlock = 2048;  // elements per workgroup of modfac_apply_kernel

__global__ __launch_bounds__(256) void modfac_apply_kernel(ModApplyArgs a) {
  // The cross-head decision, once per workgroup: threads share the heads, then one barrier OR.
  bool any = false;
  for (int h = threadIdx.x; h < a.BH; h += 256) any |= a.stats[h * 3 + 1] < a.lo || a.stats[h * 3 + 2] > a.hi;
  const bool need = __syncthreads_or(any);
  const int64_t n_all = (int64_t)a.BH * a.L;
  const int64_t i0 = (int64_t)blockIdx.x * kModApplyPerBlock + threadIdx.x;
  for (int64_t i = i0; i < min(n_all, (int64_t)(blockIdx.x + 1) * kModApplyPerBlock); i += 256) {
    const float v = a.x[i];
    if (!need) {
      a.out[i] = v;
      continue;
    }
    const int64_t bh = i / a.L;
    const float sum = a.stats[bh * 3 + 0], cmin = a.stats[bh * 3 + 1], cmax = a.stats[bh * 3 + 2];
    const float tmin = cmin < a.lo ? a.lo : cmin;
    const float tmax = cmax > a.hi ? a.hi : cmax;
    const bool flat = (cmax - cmin) < 1e-6f;
    const float rng = flat ? 1.f : cmax - cmin;
    const float n = (float)a.L;
    const float new_sum = (sum - n * cmin) / rng * (tmax - tmin) + n * tmin;
    const float scaled = (v - cmin) / rng * (tmax - tmin) + tmin;
    const float f = flat ? v : scaled * (sum / new_sum);
    a.out[i] = fminf(fmaxf(f, a.lo), a.hi);
  }
}
}  // namespace

extern "C" int sa_constrained_mod_factor(const float* x, int BH, int64_t L, float lo, float hi, float* stats,
                                         float* out, void* stream) {
  const char* fn = "sa_constrained_mod_factor";
  SA_REQUIRE(x && stats && out, "%s: null pointer", fn);
  SA_REQUIRE(BH > 0 && BH <= 4096 && L > 0, "%s: bad shape BH=%d L=%lld", fn, BH, (long long)L);
  SA_REQUIRE(lo <= hi, "%s: lo %g > hi %g", fn, (double)lo, (double)hi);
  hipStream_t s = sa::as_stream(stream);
  ModStatsArgs sa_{x, L, stats};
  hipLaunchKernelGGL(modfac_stats_kernel, dim3((unsigned)BH), dim3(256), 0, s, sa_);
  if (int rc = sa::check_launch(fn)) return rc;
  ModApplyArgs aa{x, stats, BH, L, lo, hi, out};
  const int64_t n = (int64_t)BH * L;
  const int64_t blocks = (n + kModApplyPerBlock - 1) / kModApplyPerBlock;
  SA_REQUIRE(blocks < (1LL << 31), "%s: grid too large", fn);
  hipLaunchKernelGGL(modfac_apply_kernel, dim3((unsigned)blocks), dim3(256), 0, s, aa);
  return sa::check_launch(fn);
}

extern "C" int sa_gather_tokens_heads(const uint16_t* x, const int64_t x_strides[3], int B, int H, int L_in, int D,
                                      const int32_t* idx, int L_out, uint16_t* out, const int64_t out_strides[3],
                                      void* stream) {
  const char* fn = "sa_gather_tokens_heads";
  SA_REQUIRE(idx, "%s: null idx", fn);
  SA_REQUIRE(B > 0 && H > 0 && L_in > 0 && L_out > 0, "%s: bad shape", fn);
  if (D != kD) return sa::fail(SA_ERR_UNSUPPORTED, "%s: head_dim %d (only 64)", fn, D);
  int rc = check_bf16_rows(x, x_strides, fn);
  if (rc) return rc;
  if ((rc = check_bf16_rows(out, out_strides, fn))) return rc;
  const int64_t rows = (int64_t)B * H * L_out;
  hipLaunchKernelGGL(gather_heads_kernel, dim3((unsigned)((rows * 8 + 255) / 256)), dim3(256), 0,
                     sa::as_stream(stream), x, x_strides[0], x_strides[1], x_strides[2], L_in, idx, L_out, H, rows,
                     out, out_strides[0], out_strides[1], out_strides[2]);
  return sa::check_launch(fn);
}

extern "C" int sa_pattern_maps(const uint16_t* map_mass, const int64_t map_strides[3], int B, int H, int F, int ns,
                               float* img2text, float* img2img, void* stream) {
  const char* fn = "sa_pattern_maps";
  SA_REQUIRE(map_mass && map_strides && img2text && img2img, "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && ns > 0, "%s: bad shape", fn);
  SA_REQUIRE(F >= 1 && F <= kMaxF, "%s: frames %d outside [1, %d]", fn, F, kMaxF);
  MapsArgs ma;
  ma.m = map_mass; ma.m_sb = map_strides[0]; ma.m_sh = map_strides[1]; ma.m_sl = map_strides[2];
  ma.H = H; ma.F = F; ma.ns = ns; ma.img2text = img2text; ma.img2img = img2img; ma.total = (int64_t)B * H * F;
  // 16-byte loads of columns 0-15: rows aligned and at least 16 elements apart
  ma.vec_ok = (reinterpret_cast<uintptr_t>(map_mass) % 16 == 0 && ma.m_sl >= 16 && ma.m_sl % 8 == 0 &&
               ma.m_sb % 8 == 0 && ma.m_sh % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL(maps_kernel, dim3((unsigned)ma.total), dim3(64), 0, sa::as_stream(stream), ma);
  return sa::check_launch(fn);
}

extern "C" int sa_pattern_plan(const uint16_t* ff_mass, const int64_t ff_strides[3], const float* img2img, int B,
                               int H, int F, int S, int T, float lo_text, float hi_text, float lo_frame,
                               float hi_frame, float map_thr, float* stats, float* fac, int32_t* frame_case,
                               float* inv_map0, int32_t* q_idx, void* stream) {
  const char* fn = "sa_pattern_plan";
  SA_REQUIRE(ff_mass && ff_strides && img2img && stats && fac && frame_case && inv_map0 && q_idx, "%s: null pointer",
             fn);
  SA_REQUIRE(B > 0 && H > 0 && S > 0 && T >= 0, "%s: bad shape", fn);
  SA_REQUIRE(F >= 1 && F <= kMaxF, "%s: frames %d outside [1, %d]", fn, F, kMaxF);
  hipStream_t s = sa::as_stream(stream);
  const int BH = B * H;
  StatsArgs sa_;
  sa_.m = ff_mass; sa_.m_sb = ff_strides[0]; sa_.m_sh = ff_strides[1]; sa_.m_sl = ff_strides[2];
  sa_.H = H; sa_.S = S; sa_.n_fac = 1 + F; sa_.stats = stats; sa_.total = BH;
  sa_.vec_ok = (reinterpret_cast<uintptr_t>(ff_mass) % 16 == 0 && sa_.m_sl >= 16 && sa_.m_sl % 8 == 0 &&
                sa_.m_sb % 8 == 0 && sa_.m_sh % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL(fstats_kernel, dim3((unsigned)sa_.total), dim3(256), 0, s, sa_);
  SelectArgs se;
  se.stats = stats; se.img2img = img2img; se.BH = BH; se.F = F; se.S = S; se.T = T; se.n_fac = 1 + F;
  se.lo_text = lo_text; se.hi_text = hi_text; se.lo_frame = lo_frame; se.hi_frame = hi_frame; se.map_thr = map_thr;
  se.fac = fac; se.frame_case = frame_case; se.inv_map0 = inv_map0; se.q_idx = q_idx;
  const int n = BH * (1 + F) + BH * F;
  hipLaunchKernelGGL(select_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, se);
  const int64_t nq = (int64_t)BH * F * S;
  hipLaunchKernelGGL(qidx_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, se);
  return sa::check_launch(fn);
}

extern "C" int sa_pattern_combine(const uint16_t* o_frames, const int64_t of_strides[3], const uint16_t* o_text,
                                  const int64_t ot_strides[3], const uint16_t* ff_mass, const int64_t ff_strides[3],
                                  const float* img2text, const float* img2img, const float* fac,
                                  const int32_t* frame_case, const float* inv_map0, int B, int H, int F, int S,
                                  int T, float lo_text, float hi_text, float lo_frame, float hi_frame, uint16_t* out,
                                  const int64_t out_strides[3], void* stream) {
  const char* fn = "sa_pattern_combine";
  SA_REQUIRE(img2text && img2img && fac && frame_case && inv_map0 && ff_mass && ff_strides, "%s: null pointer", fn);
  SA_REQUIRE(B > 0 && H > 0 && S > 0 && T >= 0, "%s: bad shape", fn);
  SA_REQUIRE(F >= 1 && F <= kMaxF, "%s: frames %d outside [1, %d]", fn, F, kMaxF);
  int rc;
  if ((rc = check_bf16_rows(o_frames, of_strides, fn)) || (rc = check_bf16_rows(o_text, ot_strides, fn)) ||
      (rc = check_bf16_rows(out, out_strides, fn)))
    return rc;
  CombineArgs a;
  a.of = o_frames; a.of_sb = of_strides[0]; a.of_sh = of_strides[1]; a.of_sl = of_strides[2];
  a.ot = o_text; a.ot_sb = ot_strides[0]; a.ot_sh = ot_strides[1]; a.ot_sl = ot_strides[2];
  a.mass = ff_mass; a.m_sb = ff_strides[0]; a.m_sh = ff_strides[1]; a.m_sl = ff_strides[2];
  a.img2text = img2text; a.img2img = img2img; a.fac = fac; a.frame_case = frame_case; a.inv_map0 = inv_map0;
  a.out = out; a.o_sb = out_strides[0]; a.o_sh = out_strides[1]; a.o_sl = out_strides[2];
  a.H = H; a.F = F; a.S = S; a.T = T;
  a.lo_text = lo_text; a.hi_text = hi_text; a.lo_frame = lo_frame; a.hi_frame = hi_frame;
  a.rows_per_wg = 32;
  a.total = (int64_t)B * H * ((S + 31) / 32);
  const dim3 g((unsigned)a.total), blk(256);
  hipStream_t s = sa::as_stream(stream);
  switch (F) {
#define SA_COMBINE_CASE(n) \
  case n:                  \
    hipLaunchKernelGGL(combine_kernel<n>, g, blk, 0, s, a); \
    break;
    SA_COMBINE_CASE(1) SA_COMBINE_CASE(2) SA_COMBINE_CASE(3) SA_COMBINE_CASE(4) SA_COMBINE_CASE(5)
    SA_COMBINE_CASE(6) SA_COMBINE_CASE(7) SA_COMBINE_CASE(8) SA_COMBINE_CASE(9) SA_COMBINE_CASE(10)
    SA_COMBINE_CASE(11) SA_COMBINE_CASE(12) SA_COMBINE_CASE(13) SA_COMBINE_CASE(14) SA_COMBINE_CASE(15)
    SA_COMBINE_CASE(16)
#undef SA_COMBINE_CASE
  }
  return sa::check_launch(fn);
}
