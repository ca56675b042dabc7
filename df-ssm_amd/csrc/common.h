// Shared device helpers for the DF-SSM decode kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DFSSM_WAVE 64
#define DFSSM_LORA_R 16

typedef _Float16 f16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) 16-byte loads/stores: weights and SSM state are touched once per step.
__device__ __forceinline__ u32x4 ld_nt(const void* p) { return __builtin_nontemporal_load((const u32x4*)p); }
__device__ __forceinline__ f32x4 ld_nt_f4(const float* p) { return __builtin_nontemporal_load((const f32x4*)p); }
__device__ __forceinline__ void st_nt_f4(float* p, f32x4 v) { __builtin_nontemporal_store(v, (f32x4*)p); }
// Device-scope (agent) coherent 32/64-bit accesses: they go past the L2 of the issuing XCD, so a
// word stored by a workgroup on one XCD is seen by a load on another without any cache flush.
template <class T>
__device__ __forceinline__ T ld_dev(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The tag of a launch whose workgroup launch count is `epoch`, derived where it is used: the empty
// asm keeps the compiler from deriving it at the kernel start, where it waited for the count's
// device-scope round trip (~1 us) before issuing any other load.
__device__ __forceinline__ uint32_t tag_of(uint32_t epoch) {
  asm volatile("" : "+v"(epoch));
  return (epoch + 1u) & 0xffffu;
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(f16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (f16)f); }  // RNE
__device__ __forceinline__ float r16(float f) { return (float)(f16)f; }  // round through fp16

// Correctly rounded fp32 square root. v_sqrt_f32 is accurate to 1 ulp only; the fp64 square root
// rounded to fp32 is the correctly rounded fp32 result (53 >= 2*24 + 2, so the double rounding is
// innocuous), which is what IEEE sqrtf on the host returns.
__device__ __forceinline__ float sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }

// exp and log1p of the decode step: the same operation sequence as the spec's CPU restatement,
// built from correctly rounded operations only (+ - * /, fma, rint, bit moves), so results are
// identical bit for bit on the host and the GPU.
//  exp: Cody & Waite reduction x = n ln2 + r (ln2 as 9-bit head + tail), |r| <= ln2/2, degree-7
//       Taylor polynomial of e^r in Horner form, e^x = p 2^n; e^x for x < -86 returns 0 (so
//       nonzero results are normal numbers), overflow returns +inf. Max error 0.91 ulp.
//  log1p (y >= 0): u = 1+y = m 2^e, m in [sqrt(1/2), sqrt(2)), log m = 2 atanh((m-1)/(m+1)) with
//       the atanh series to s^9, plus the correction (y - (u-1))/u for the rounding of 1+y.
//       Max error 2.3 ulp.
__device__ __forceinline__ float dev_expf(float x) {
  if (x != x) return x;
  if (x < -86.0f) return 0.0f;
  if (x > 89.0f) return __builtin_inff();
  const float n = __builtin_rintf(x * 1.44269502f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.42860677e-6f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  const float sc = __builtin_bit_cast(float, (uint32_t)(ni + 127) << 23);
  return p * sc;
}

__device__ __forceinline__ float dev_log_pos(float u) {  // finite u >= 1
  const uint32_t b = __builtin_bit_cast(uint32_t, u);
  int e = (int)(b >> 23) - 127;
  float m = __builtin_bit_cast(float, (b & 0x7fffffu) | 0x3f800000u);
  if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 0.111111111f;
  p = __builtin_fmaf(p, s2, 0.142857143f);
  p = __builtin_fmaf(p, s2, 0.2f);
  p = __builtin_fmaf(p, s2, 0.333333333f);
  p = p * s2;
  const float t = 2.0f * s;
  const float lm = __builtin_fmaf(t, p, t);
  const float ef = (float)e;
  return __builtin_fmaf(ef, 0.693145751953125f, __builtin_fmaf(ef, 1.42860677e-6f, lm));
}

__device__ __forceinline__ float dev_log1pf(float y) {  // y >= 0
  if (y != y || y == 0.0f || y == __builtin_inff()) return y;
  const float u = 1.0f + y;
  const float lg = dev_log_pos(u);
  return lg + (y - (u - 1.0f)) / u;
}


// Fast wave reductions on the DPP crossbar (a few cycles per step, against ~100 for the LDS
// permute behind __shfl_xor). gfx9 DPP controls: quad_perm [1,0,3,2] = 0xB1 and [2,3,0,1] = 0x4E
// (butterflies within 4 lanes), row_ror:4 = 0x124 and row_ror:8 = 0x128 (rotations within a row
// of 16 lanes). After the four steps every lane holds its row's total; the four row totals are
// then read from lanes 0, 16, 32, 48, so the result is uniform and the summation order is the
// same in every wave.
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) { return __builtin_bit_cast(float, dpp_i32<CTRL>(__builtin_bit_cast(int, v))); }
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)u);
  const uint32_t hi = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)(u >> 32));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double row_sum_f64(double v) {
  v += dpp_f64<0xB1>(v);
  v += dpp_f64<0x4E>(v);
  v += dpp_f64<0x124>(v);
  v += dpp_f64<0x128>(v);
  return v;
}
__device__ __forceinline__ int row_sum_i32(int v) {
  v += dpp_i32<0xB1>(v);
  v += dpp_i32<0x4E>(v);
  v += dpp_i32<0x124>(v);
  v += dpp_i32<0x128>(v);
  return v;
}
__device__ __forceinline__ double wave_sum_dpp_f64(double v) {
  v = row_sum_f64(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}
__device__ __forceinline__ int wave_sum_dpp_i32(int v) {
  v += dpp_i32<0xB1>(v);
  v += dpp_i32<0x4E>(v);
  v += dpp_i32<0x124>(v);
  v += dpp_i32<0x128>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
__device__ __forceinline__ float wave_max_dpp_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x124>(v));
  v = fmaxf(v, dpp_f32<0x128>(v));
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Workgroup barrier that orders LDS accesses only. __syncthreads() is also a release of global
// memory, so it first waits until every global store the wave has issued is acknowledged (0.6 to
// 1 us); where the barrier only hands LDS data between waves that wait is pure latency.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block-wide sums / max for blockDim.x == NT (multiple of 64). `red` must hold NT/64 entries.
// Every sum reduced this way in the decode kernels is exact (fp64 sums of exactly representable
// products, integer sums), so the reduction order does not change results.
template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_dpp_f64(v);
  const int w = threadIdx.x / DFSSM_WAVE;
  lds_barrier();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  lds_barrier();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < NT / DFSSM_WAVE; ++i) t += red[i];
  return t;
}
template <int NT>
__device__ __forceinline__ float block_max_f32(float v, float* red) {
  v = wave_max_dpp_f32(v);
  const int w = threadIdx.x / DFSSM_WAVE;
  lds_barrier();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  lds_barrier();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < NT / DFSSM_WAVE; ++i) t = fmaxf(t, red[i]);
  return t;
}
template <int NT>
__device__ __forceinline__ int block_sum_i32(int v, int* red) {
  v = wave_sum_dpp_i32(v);
  const int w = threadIdx.x / DFSSM_WAVE;
  lds_barrier();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  lds_barrier();
  int t = 0;
#pragma unroll
  for (int i = 0; i < NT / DFSSM_WAVE; ++i) t += red[i];
  return t;
}

// Activation quantizer of the reference (_quantize_to_int8, df_ssm_inference.py:147-152):
// scale = fp16(fp16(max(amax, 1e-4)) * (1/127)); q = clamp(rne(fp16(x / scale)), -128, 127), the
// quotient an IEEE fp32 division. Computed here as q = clamp(rne(fp16(x * r)), -128, 127) with
// r = fp32(1 / (double)scale) (quant_rcp, once per row): fp16(x * r) differs from fp16(x / scale)
// for 1495 of the 1.0e9 pairs of a finite fp16 |x| and a positive finite fp16 scale, never after
// rne and the clamp at 127 (x >= 0) or 128 (x < 0, the same magnitudes mirrored) -- q is
// identical for every pair, checked exhaustively by tests/test_quant_recip.py. Three fp32
// operations per value replace the ~12-instruction fp32 division sequence.
__device__ __forceinline__ float quant_scale(float amax) {
  float c = r16(amax > 1e-4f ? amax : 1e-4f);
  return r16(c * (1.0f / 127.0f));
}
__device__ __forceinline__ float quant_rcp(float scale) { return (float)(1.0 / (double)scale); }
__device__ __forceinline__ int quant_i8(float x, float r) {
  const float t = __builtin_rintf(r16(x * r));  // |x * r| may overflow fp16 to inf: clamped below
  return (int)__builtin_amdgcn_fmed3f(t, -128.0f, 127.0f);
}

// Bit planes of 64 int8 values, one per lane (q of element k0 + lane): w[b] = bit b of elements
// k0 .. k0 + 31, w[8 + b] = bit b of elements k0 + 32 .. k0 + 63 (one ballot per plane). The
// words are wave-uniform (scalar registers); one lane stores them (planes_store).
__device__ __forceinline__ void planes64(int q, uint32_t (&w)[16]) {
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const uint64_t mask = __ballot((q >> b) & 1);
    w[b] = (uint32_t)mask;
    w[8 + b] = (uint32_t)(mask >> 32);
  }
}
// The 16 words to dst[0..15] (16-byte aligned; LDS or global), from lane 0.
__device__ __forceinline__ void planes_store(uint32_t* dst, const uint32_t (&w)[16]) {
  if ((threadIdx.x & 63) == 0) {
    u32x4* d = (u32x4*)dst;
    d[0] = u32x4{w[0], w[1], w[2], w[3]};
    d[1] = u32x4{w[4], w[5], w[6], w[7]};
    d[2] = u32x4{w[8], w[9], w[10], w[11]};
    d[3] = u32x4{w[12], w[13], w[14], w[15]};
  }
}
