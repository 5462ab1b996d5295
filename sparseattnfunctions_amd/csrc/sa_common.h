// Shared host/device helpers for libsa_hip.so: error reporting, vector types, launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "sa_api.h"

namespace sa {

// Per-thread last-error message behind sa_last_error().
std::string& last_error_slot();

inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error_slot() = buf;
  return code;
}

inline int ok() {
  last_error_slot().clear();
  return SA_OK;
}

// Checks the launch that was just enqueued.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// Workspace of the fp16-score attention (sa_block_sparse_fwd_k16): the fp16 copy of k,
// [B*H][Lk][D] contiguous (D = 64 or 128), then the largest squared row norm of each 64-row
// key block (fp32 bits), [B*H][ceil(Lk/64)]. Written by sa_block_sparse_fwd_k16_prepare or
// (D = 64) sa_block_pool_k16.
inline int64_t k16_bytes(int B, int H, int Lk, int D = 64) {
  return ((int64_t)B * H * Lk * D * 2 + 255) / 256 * 256;
}
inline int64_t k16_ws_bytes(int B, int H, int Lk, int D = 64) {
  return k16_bytes(B, H, Lk, D) + (int64_t)B * H * cdiv(Lk, 64) * 4;
}
// With a key bias (D = 64): then, 256-byte aligned, the bias times log2(e), fp32 [B*H][Lk] contiguous.
inline int64_t k16_bias_offset(int B, int H, int Lk) { return (k16_ws_bytes(B, H, Lk) + 255) / 256 * 256; }
inline int64_t k16_ws_bytes_bias(int B, int H, int Lk) { return k16_bias_offset(B, H, Lk) + (int64_t)B * H * Lk * 4; }

// fp32 attention in pooling mode (attn_f32.hip), for the pooled-map entry point.
int attn_f32_pooling(const float* q, const int64_t q_strides[3], const float* k, const int64_t k_strides[3],
                     const float* v, const int64_t v_strides[3], float* out, const int64_t out_strides[3], int B,
                     int H, int L, int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt, int kv_rep,
                     bool causal, float sm_scale, int pool_cols, float* pool_r, float* pool_lse, void* stream,
                     const char* fn);

}  // namespace sa

#define SA_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ::sa::fail(SA_ERR_INVALID, __VA_ARGS__); \
  } while (0)

typedef __bf16 sa_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 sa_bf16x4 __attribute__((ext_vector_type(4)));
typedef float sa_f32x16 __attribute__((ext_vector_type(16)));
typedef float sa_f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t sa_u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t sa_u16x4 __attribute__((ext_vector_type(4)));

// Bitonic sort, descending, of the 64 * E keys of one wave: element i = 64 e + lane sits in
// register e of lane `lane`. Partners in the same lane (i ^ j, j >= 64) are exchanged in
// registers, partners in other lanes (j < 64) through shuffles; afterwards sorted position p
// holds the p-th largest key. E is a power of two.
template <int E>
__device__ inline void sa_wave_bitonic_desc(uint64_t (&key)[E], int lane) {
  constexpr int N = 64 * E;
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
        const int je = j >> 6;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (e & je) continue;
          // pair (i, i + j) in one lane; descending block when (i & k) == 0 (k > 64 here)
          const bool desc = ((64 * e) & k) == 0;
          const uint64_t x = key[e], y = key[e | je];
          const bool first_x = (x > y) == desc;
          key[e] = first_x ? x : y;
          key[e | je] = first_x ? y : x;
        }
      } else {
        const bool lower = (lane & j) == 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const bool desc = (((64 * e) | lane) & k) == 0;
          const uint64_t x = key[e];
          const uint32_t ylo = (uint32_t)__shfl_xor((int)(uint32_t)x, j);
          const uint32_t yhi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), j);
          const uint64_t y = ((uint64_t)yhi << 32) | ylo;
          // the lower index of a descending pair (or the upper of an ascending one) takes the
          // larger key
          key[e] = (lower == desc) == (x > y) ? x : y;
        }
      }
    }
  }
}
