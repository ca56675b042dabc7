// Density-field quantization of the SSM state at a chunk boundary (gfx950).
//
// training/df_ssm_mamba2_distill_dfw.py:139-165 (df_ssd_scan) quantizes the running state after
// every block_len tokens, per (sequence, head, state row p) over its d_state values:
//   mean, std (unbiased, clamped to 1e-8); lo = mean - 3 std; range = max(6 std, 1e-8)
//   hs = clamp((h - lo) / range, 0, 1); hc = clamp(hs + e, 0, 1) with sigma-delta error e
//   q  = (number of bank thresholds below hc) / KK              (SprayBank.quantize, :88-91)
//   e  = round(clamp(hc - q, -1, 1) 2^(bits-1)) / 2^(bits-1)     (_quantize_error, :105-110)
//   h  = q range + lo
// Two rows of 128 values per wave (half-wave h: row 2w + h; lane l of the half: values 4l .. 4l+3,
// one 16-byte access, so each access instruction of a wave covers 1 KiB contiguous). The two row
// sums are fp64 sums over the adjacent-pair tree: (v0 + v1) + (v2 + v3) in the lane, then a
// butterfly over the 32 lanes of the half (a + b is the same bits as b + a), so a sequential
// restatement with the same tree reproduces them exactly; every other operation is a single
// correctly rounded fp32 operation (no contraction).
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kDfRows = 8;  // rows per workgroup (4 waves x 2)

__device__ __forceinline__ double tree_sum32(double v) {
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) {
    const double o = __shfl_xor(v, m);
    v = v + o;
  }
  return v;
}

__global__ __launch_bounds__(32 * kDfRows) void state_df_kernel(StateDfArgs a) {
  __shared__ float R[kStateDfMaxKK];
  for (int i = threadIdx.x; i < a.kk; i += blockDim.x) R[i] = a.thresholds[i];
  __syncthreads();
  const int lane = threadIdx.x & 31;
  long long row = (long long)blockIdx.x * kDfRows + (threadIdx.x >> 5);
  const bool live = row < a.rows;
  if (!live) row = a.rows - 1;  // the half-wave still takes part in the exchanges; stores nothing
  float4* hp = (float4*)(a.h + row * 128) + lane;
  const float4 hv = *hp;
  const double S = tree_sum32(((double)hv.x + (double)hv.y) + ((double)hv.z + (double)hv.w));
  const float mean = (float)(S / 128.0);
  const float d0 = hv.x - mean, d1 = hv.y - mean, d2 = hv.z - mean, d3 = hv.w - mean;
  const double SS = tree_sum32(((double)d0 * (double)d0 + (double)d1 * (double)d1) +
                               ((double)d2 * (double)d2 + (double)d3 * (double)d3));
  float sd = sqrt_rn((float)(SS / 127.0));
  sd = sd > 1e-8f ? sd : 1e-8f;
  const float t3 = 3.0f * sd, t6 = 6.0f * sd;
  const float lo = mean - t3;
  const float range = t6 > 1e-8f ? t6 : 1e-8f;
  float4 ev = {0.0f, 0.0f, 0.0f, 0.0f};
  float4* ep = a.sd_error ? (float4*)(a.sd_error + row * 128) + lane : nullptr;
  if (ep) ev = *ep;
  const float scale = a.sd_bits < 32 ? (float)(1 << (a.sd_bits - 1)) : 1.0f;
  float out[4], err[4];
  const float hin[4] = {hv.x, hv.y, hv.z, hv.w}, ein[4] = {ev.x, ev.y, ev.z, ev.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
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
  if (!live) return;
  *hp = float4{out[0], out[1], out[2], out[3]};
  if (ep) *ep = float4{err[0], err[1], err[2], err[3]};
}

hipError_t launch_state_df(const StateDfArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const long long blocks = (a.rows + kDfRows - 1) / kDfRows;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(state_df_kernel, dim3((unsigned)blocks), dim3(32 * kDfRows), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
