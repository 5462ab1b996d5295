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
