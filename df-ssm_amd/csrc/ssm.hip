// Mamba-2 single-step SSM update (+ gate) and the stand-alone conv1d step (gfx950).
//
// SSM: one workgroup of 256 threads owns (sequence m, head, 16 rows p of the head's P) -- 8 KiB of
// fp32 state, read and written once. (Two 16-row blocks per workgroup, four state loads of a thread
// in flight together, measured 8% faster in a graph of 48 launches of this kernel alone but 1.7%
// slower per decode step at batch 32 and the 2.7B shape at batch 64, so one block it is.) Thread t owns the 4 state columns n = 4*(t%32) .. +3 of rows
// p0 = 16*blk + t/32 and p0 + 8, so each 16-byte load/store instruction of the workgroup covers
// 4 KiB contiguous (measured 5.7 TB/s on the state stream against 5.0 for 32 contiguous bytes per
// thread). The small operands (dt, x, B, C, z) are loaded before the state: loads complete in
// issue order, so dt, exp(dt A) and the gate are computed while the state streams in and nothing
// waits on a store acknowledgement. The C.h readout is reduced over the 32 lanes of a row (two DPP
// rows). Arithmetic (ssm_step_kernel, df_ssm_kernels.cu:77-101, with an fp32 state and
// P = d_inner/nheads):
//   dt = log1p(exp(dt_raw + dt_bias)); Abar = exp(dt * -exp(A_log))   (dev_expf, dev_log1pf)
//   h = fma(Abar, h, (x*dt) * B_n);   y = fp16(sum_n C_n h_n + x * D)
// and, with the gate (GATE), g = fp16(y * fp16(z * fp16(sigmoid(z)))) (df_ssm_inference.py
// :194-195) with sum(g^2) of the block written to a per-block slot for the gated RMSNorm.
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

template <bool GATE>
__global__ __launch_bounds__(256) void ssm_kernel(SsmArgs a) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int m = blockIdx.y;
  const int pblocks = a.P / 16;
  const int head = blockIdx.x / pblocks;
  const int pb = blockIdx.x % pblocks;
  const int DI = a.H * a.P;
  const int n0 = 4 * (tid & 31);
  const int p = pb * 16 + (tid >> 5);  // and p + 8
  // small operands first
  const uint16_t* xr = a.xbc + (size_t)m * a.ld_xbc;
  const uint16_t dtr = a.dt[(size_t)m * a.ld_dt + head];
  const uint16_t xr0 = xr[head * a.P + p], xr1 = xr[head * a.P + p + 8];
  uint16_t zr0 = 0, zr1 = 0;
  if (GATE) {
    const uint16_t* zp = a.z + (size_t)m * a.ld_z + head * a.P + p;
    zr0 = zp[0];
    zr1 = zp[8];
  }
  const uint2 b4 = *(const uint2*)(xr + DI + n0);
  const uint2 c4 = *(const uint2*)(xr + DI + a.N + n0);
  const float Dh = a.D[head], dtb = a.dt_bias[head], alog = a.A_log[head];
  // then the state: rows p and p + 8
  float* hp = a.h + (((size_t)m * a.H + head) * a.P + p) * a.N + n0;
  const f32x4 s0 = ld_nt_f4(hp);
  const f32x4 s1 = ld_nt_f4(hp + 8 * a.N);

  const float dt = dev_log1pf(dev_expf(h2f(dtr) + dtb));
  const float abar = dev_expf(dt * -dev_expf(alog));
  const float xv0 = h2f(xr0), xv1 = h2f(xr1);
  const float X0 = xv0 * dt, X1 = xv1 * dt;
  float sz0 = 0.0f, sz1 = 0.0f;
  if (GATE) {
    const float z0 = h2f(zr0), z1 = h2f(zr1);
    sz0 = r16(z0 * r16(1.0f / (1.0f + dev_expf(-z0))));
    sz1 = r16(z1 * r16(1.0f / (1.0f + dev_expf(-z1))));
  }
  const uint32_t bw[2] = {b4.x, b4.y}, cw[2] = {c4.x, c4.y};
  float h0[4] = {s0.x, s0.y, s0.z, s0.w}, h1[4] = {s1.x, s1.y, s1.z, s1.w};
  double acc0 = 0.0, acc1 = 0.0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float bn = h2f((uint16_t)(bw[j >> 1] >> (16 * (j & 1))));
    const float cn = h2f((uint16_t)(cw[j >> 1] >> (16 * (j & 1))));
    h0[j] = __builtin_fmaf(abar, h0[j], X0 * bn);
    h1[j] = __builtin_fmaf(abar, h1[j], X1 * bn);
    acc0 += (double)cn * (double)h0[j];
    acc1 += (double)cn * (double)h1[j];
  }
  st_nt_f4(hp, f32x4{h0[0], h0[1], h0[2], h0[3]});
  st_nt_f4(hp + 8 * a.N, f32x4{h1[0], h1[1], h1[2], h1[3]});
  // a row's 32 lanes are DPP rows 0+1 (p) or 2+3 (p, in the upper half-wave)
  acc0 = row_sum_f64(acc0);
  acc1 = row_sum_f64(acc1);
  const double t0a = readlane_f64(acc0, 0) + readlane_f64(acc0, 16);
  const double t0b = readlane_f64(acc0, 32) + readlane_f64(acc0, 48);
  const double t1a = readlane_f64(acc1, 0) + readlane_f64(acc1, 16);
  const double t1b = readlane_f64(acc1, 32) + readlane_f64(acc1, 48);
  double gsqd = 0.0;
  if ((tid & 31) == 0) {
    const bool hi = lane >= 32;
    const float y0 = r16((float)(hi ? t0b : t0a) + xv0 * Dh);
    const float y1 = r16((float)(hi ? t1b : t1a) + xv1 * Dh);
    float o0 = y0, o1 = y1;
    if (GATE) {
      o0 = r16(y0 * sz0);
      o1 = r16(y1 * sz1);
      gsqd = (double)o0 * (double)o0 + (double)o1 * (double)o1;
    }
    uint16_t* yp = a.y_out + (size_t)m * a.ld_y + head * a.P + p;
    yp[0] = f2h(o0);
    yp[8] = f2h(o1);
  }
  if (GATE) {
    __shared__ double part[4];
    // lanes 0 and 32 of each wave hold their two rows' g^2; the others hold 0
    const double s = wave_sum_dpp_f64(gsqd);
    if (lane == 0) part[tid >> 6] = s;
    lds_barrier();
    if (tid == 0) a.sumsq_slots[(size_t)m * a.n_slots + blockIdx.x] = part[0] + part[1] + part[2] + part[3];
  }
}

// conv_step_kernel semantics (df_ssm_kernels.cu:27-47), in place on x (row stride ld) and the
// (M, C, 3) fp16 shift-register state.
__global__ __launch_bounds__(256) void conv_kernel(ConvArgs a) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (ch >= a.C) return;
  uint16_t* cs = a.state + ((size_t)m * a.C + ch) * 3;
  uint16_t* xp = a.x + (size_t)m * a.ld + ch;
  const float s0 = h2f(cs[0]), s1 = h2f(cs[1]), s2 = h2f(cs[2]);
  const uint16_t xo = *xp;
  cs[0] = cs[1];
  cs[1] = cs[2];
  cs[2] = xo;
  const uint16_t* wc = a.w + (size_t)ch * 4;
  const float xv = h2f(xo);
  float o = s0 * h2f(wc[0]);
  o = o + s1 * h2f(wc[1]);
  o = o + s2 * h2f(wc[2]);
  o = o + xv * h2f(wc[3]);
  o = o + h2f(a.b[ch]);
  const float sig = 1.0f / (1.0f + dev_expf(-o));
  *xp = f2h(o * sig);
}

hipError_t launch_ssm(const SsmArgs& a, int M, hipStream_t s) {
  // the gate and the sum(g^2) slots come together (the decode layer); neither for dfssm_ssm_step
  if (a.z && a.sumsq_slots)
    hipLaunchKernelGGL(ssm_kernel<true>, dim3(a.H * (a.P / 16), M), dim3(256), 0, s, a);
  else if (!a.z && !a.sumsq_slots)
    hipLaunchKernelGGL(ssm_kernel<false>, dim3(a.H * (a.P / 16), M), dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_conv(const ConvArgs& a, int M, hipStream_t s) {
  hipLaunchKernelGGL(conv_kernel, dim3((a.C + 255) / 256, M), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
