// Shared helpers for the gfx950 HIP kernels of the Maba v2 hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/maba_hip.h"

namespace maba {

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
// Compute units of the current device (cached per device; 256 when it cannot be queried).
int device_cu_count();

// ---------------------------------------------------------------- scalar types
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(4))) short i16x4;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// Hardware transcendentals (v_exp_f32, v_log_f32, v_rcp_f32, v_sqrt_f32: about one ulp,
// without the IEEE division sequence or the denormal range scaling of the library forms,
// which cost several times more instructions).  Results that leave fp32's normal range
// saturate (exp to 0 or inf, rcp(inf) = 0); the log is taken of arguments >= 1 here.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float fast_log(float x) { return __builtin_amdgcn_logf(x) * 0.6931471805599453f; }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_sqrt(float x) { return __builtin_amdgcn_sqrtf(x); }

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float load_elem(const void* p, int dt, int64_t i) {
  switch (dt) {
    case MABA_F32: return ((const float*)p)[i];
    case MABA_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    case MABA_F16: return __half2float(((const __half*)p)[i]);
    default: return 0.f;
  }
}

__device__ __forceinline__ void store_elem(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case MABA_F32: ((float*)p)[i] = v; break;
    case MABA_BF16: ((uint16_t*)p)[i] = f32_to_bf16_bits(v); break;
    case MABA_F16: ((__half*)p)[i] = __float2half(v); break;
    default: break;
  }
}

// Strided view passed to kernels (up to 4 dims, element strides).
struct View4 {
  const void* p;
  int dt;
  int64_t s0, s1, s2, s3;
  __device__ __forceinline__ float at(int64_t a, int64_t b, int64_t c, int64_t d) const {
    return load_elem(p, dt, a * s0 + b * s1 + c * s2 + d * s3);
  }
};

struct MView4 {
  void* p;
  int dt;
  int64_t s0, s1, s2, s3;
  __device__ __forceinline__ void put(int64_t a, int64_t b, int64_t c, int64_t d, float v) const {
    store_elem(p, dt, a * s0 + b * s1 + c * s2 + d * s3, v);
  }
};

// ---------------------------------------------------------------- host helpers
inline bool is_float_dt(int dt) { return dt == MABA_F32 || dt == MABA_F16 || dt == MABA_BF16; }

inline View4 view4(const maba_tensor* t) {
  View4 v;
  v.p = t ? t->data : nullptr;
  v.dt = t ? t->dtype : MABA_F32;
  v.s0 = t ? t->stride[0] : 0;
  v.s1 = t ? t->stride[1] : 0;
  v.s2 = t ? t->stride[2] : 0;
  v.s3 = t ? t->stride[3] : 0;
  return v;
}

inline MView4 mview4(maba_tensor* t) {
  MView4 v;
  v.p = t->data;
  v.dt = t->dtype;
  v.s0 = t->stride[0];
  v.s1 = t->stride[1];
  v.s2 = t->stride[2];
  v.s3 = t->stride[3];
  return v;
}

// Checks ndim and leading shape of a descriptor; returns false and sets the
// error message otherwise.
bool expect_shape(const maba_tensor* t, const char* name, int ndim, const int64_t* shape);
bool expect_float(const maba_tensor* t, const char* name);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace maba
