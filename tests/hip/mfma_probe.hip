// Test-only probes of gfx950 MFMA lane layouts and issue rates.
// Each probe runs one MFMA on per-lane operand registers loaded from global
// memory and stores the raw per-lane accumulator registers, so a test can
// check an assumed lane layout against a host matrix product.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(8))) short i16x8;

__global__ void k_16x16x16bf16(const short* a, const short* b, float* d) {
  const int l = threadIdx.x;
  i16x4 av, bv;
  for (int i = 0; i < 4; ++i) { av[i] = a[l * 4 + i]; bv[i] = b[l * 4 + i]; }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, acc, 0, 0, 0);
  for (int i = 0; i < 4; ++i) d[l * 4 + i] = acc[i];
}

__global__ void k_16x16x32bf16(const short* a, const short* b, float* d) {
  const int l = threadIdx.x;
  i16x8 sa, sb;
  for (int i = 0; i < 8; ++i) { sa[i] = a[l * 8 + i]; sb[i] = b[l * 8 + i]; }
  const bf16x8 av = __builtin_bit_cast(bf16x8, sa), bv = __builtin_bit_cast(bf16x8, sb);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
  for (int i = 0; i < 4; ++i) d[l * 4 + i] = acc[i];
}

__global__ void k_32x32x16bf16(const short* a, const short* b, float* d) {
  const int l = threadIdx.x;
  i16x8 sa, sb;
  for (int i = 0; i < 8; ++i) { sa[i] = a[l * 8 + i]; sb[i] = b[l * 8 + i]; }
  const bf16x8 av = __builtin_bit_cast(bf16x8, sa), bv = __builtin_bit_cast(bf16x8, sb);
  f32x16 acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
  for (int i = 0; i < 16; ++i) d[l * 16 + i] = acc[i];
}

extern "C" int probe_mfma(int kind, const void* a, const void* b, void* d, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (kind == 0) hipLaunchKernelGGL(k_16x16x16bf16, dim3(1), dim3(64), 0, s, (const short*)a, (const short*)b, (float*)d);
  else if (kind == 1) hipLaunchKernelGGL(k_16x16x32bf16, dim3(1), dim3(64), 0, s, (const short*)a, (const short*)b, (float*)d);
  else hipLaunchKernelGGL(k_32x32x16bf16, dim3(1), dim3(64), 0, s, (const short*)a, (const short*)b, (float*)d);
  return (int)hipGetLastError();
}

