// Shared device helpers for the DF-SSM decode kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DFSSM_WAVE 64
#define DFSSM_LORA_R 16

typedef _Float16 f16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) 16-byte loads/stores: weights and SSM state are touched once per step.
__device__ __forceinline__ u32x4 ld_nt(const void* p) { return __builtin_nontemporal_load((const u32x4*)p); }
__device__ __forceinline__ f32x4 ld_nt_f4(const float* p) { return __builtin_nontemporal_load((const f32x4*)p); }
__device__ __forceinline__ void st_nt_f4(float* p, f32x4 v) { __builtin_nontemporal_store(v, (f32x4*)p); }

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(f16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (f16)f); }  // RNE
__device__ __forceinline__ float r16(float f) { return (float)(f16)f; }  // round through fp16

// Wave64 sums (xor butterfly: every lane ends with the total).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, DFSSM_WAVE);
  return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, DFSSM_WAVE);
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, DFSSM_WAVE));
  return v;
}

// Block-wide sums / max for blockDim.x == NT (multiple of 64). `red` must hold NT/64 entries.
template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  const int w = threadIdx.x / DFSSM_WAVE;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < NT / DFSSM_WAVE; ++i) t += red[i];
  return t;
}
template <int NT>
__device__ __forceinline__ float block_max_f32(float v, float* red) {
  v = wave_max_f32(v);
  const int w = threadIdx.x / DFSSM_WAVE;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < NT / DFSSM_WAVE; ++i) t = fmaxf(t, red[i]);
  return t;
}
template <int NT>
__device__ __forceinline__ int block_sum_i32(int v, int* red) {
  v = wave_sum_i32(v);
  const int w = threadIdx.x / DFSSM_WAVE;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < NT / DFSSM_WAVE; ++i) t += red[i];
  return t;
}

// Activation quantizer of the reference (_quantize_to_int8, df_ssm_inference.py:147-152):
// scale = fp16(fp16(max(amax, 1e-4)) * (1/127)); q = clamp(rne(fp16(x / scale)), -128, 127).
__device__ __forceinline__ float quant_scale(float amax) {
  float c = r16(amax > 1e-4f ? amax : 1e-4f);
  return r16(c * (1.0f / 127.0f));
}
__device__ __forceinline__ int quant_i8(float x, float scale) {
  float t = __builtin_rintf(r16(x / scale));
  t = t > 127.0f ? 127.0f : t;
  t = t < -128.0f ? -128.0f : t;
  return (int)t;
}
