// Density-field quantization of the SSM state at a chunk boundary (gfx950).
//
// training/df_ssm_mamba2_distill_dfw.py:139-165 (df_ssd_scan) quantizes the running state after
// every block_len tokens, per (sequence, head, state row p) over its d_state values:
//   mean, std (unbiased, clamped to 1e-8); lo = mean - 3 std; range = max(6 std, 1e-8)
//   hs = clamp((h - lo) / range, 0, 1); hc = clamp(hs + e, 0, 1) with sigma-delta error e
//   q  = (number of bank thresholds below hc) / KK              (SprayBank.quantize, :88-91)
//   e  = round(clamp(hc - q, -1, 1) 2^(bits-1)) / 2^(bits-1)     (_quantize_error, :105-110)
//   h  = q range + lo
// One wave per row of 128 values (lane l: values 2l, 2l+1); the two row sums are fp64 sums of
// the lane pairs over the adjacent-pair tree (a butterfly: a + b is the same bits as b + a), so
// a sequential restatement with the same tree reproduces them exactly; every other operation is
// a single correctly rounded fp32 operation (no contraction).
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kDfRows = 4;  // rows (waves) per workgroup

__device__ __forceinline__ double tree_sum64(double v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const double o = __shfl_xor(v, m);
    v = v + o;
  }
  return v;
}

__global__ __launch_bounds__(64 * kDfRows) void state_df_kernel(StateDfArgs a) {
  __shared__ float R[kStateDfMaxKK];
  for (int i = threadIdx.x; i < a.kk; i += blockDim.x) R[i] = a.thresholds[i];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * kDfRows + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  float2* hp = (float2*)(a.h + row * 128) + lane;
  const float2 hv = *hp;
  const double S = tree_sum64((double)hv.x + (double)hv.y);
  const float mean = (float)(S / 128.0);
  const float d0 = hv.x - mean, d1 = hv.y - mean;
  const double SS = tree_sum64((double)d0 * (double)d0 + (double)d1 * (double)d1);
  float sd = sqrt_rn((float)(SS / 127.0));
  sd = sd > 1e-8f ? sd : 1e-8f;
  const float t3 = 3.0f * sd, t6 = 6.0f * sd;
  const float lo = mean - t3;
  const float range = t6 > 1e-8f ? t6 : 1e-8f;
  float2 ev = {0.0f, 0.0f};
  float2* ep = a.sd_error ? (float2*)(a.sd_error + row * 128) + lane : nullptr;
  if (ep) ev = *ep;
  const float scale = a.sd_bits < 32 ? (float)(1 << (a.sd_bits - 1)) : 1.0f;
  float out[2], err[2];
  const float hin[2] = {hv.x, hv.y}, ein[2] = {ev.x, ev.y};
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float hs = (hin[k] - lo) / range;
    hs = hs < 0.0f ? 0.0f : (hs > 1.0f ? 1.0f : hs);
    float hc = hs;
    if (ep) {
      hc = hs + ein[k];
      hc = hc < 0.0f ? 0.0f : (hc > 1.0f ? 1.0f : hc);
    }
    int first = 0, n = a.kk;  // first threshold >= hc (= number below hc)
    while (n > 0) {
      const int half = n >> 1;
      if (R[first + half] < hc) {
        first += half + 1;
        n -= half + 1;
      } else {
        n = half;
      }
    }
    const float q = (float)first / (float)a.kk;
    float e = hc - q;
    e = e < -1.0f ? -1.0f : (e > 1.0f ? 1.0f : e);
    if (a.sd_bits < 32) e = __builtin_rintf(e * scale) / scale;
    err[k] = e;
    const float qr = q * range;
    out[k] = qr + lo;
  }
  *hp = float2{out[0], out[1]};
  if (ep) *ep = float2{err[0], err[1]};
}

hipError_t launch_state_df(const StateDfArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const long long blocks = (a.rows + kDfRows - 1) / kDfRows;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(state_df_kernel, dim3((unsigned)blocks), dim3(64 * kDfRows), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
