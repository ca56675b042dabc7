// Mamba-2 single-step SSM update (+ gate) and the stand-alone conv1d step (gfx950).
//
// SSM: one workgroup of 256 threads owns (sequence m, head, 16 rows p of the head's P). Thread t
// owns row p = 16*blk + t/16 and the 8 consecutive state columns n = 8*(t%16) .. +7, so each
// thread streams 32 B of fp32 state and the workgroup 8 KiB contiguous; the C.h readout is
// reduced over the 16 lanes that share a row. Arithmetic (ssm_step_kernel,
// df_ssm_kernels.cu:77-101, with an fp32 state and P = d_inner/nheads):
//   dt = log1p(exp(dt_raw + dt_bias)); Abar = exp(dt * -exp(A_log))   (dev_expf, dev_log1pf)
//   h = fma(Abar, h, (x*dt) * B_n);   y = fp16(sum_n C_n h_n + x * D)
// and, when a gate is requested, g = fp16(y * fp16(z * fp16(sigmoid(z)))) (df_ssm_inference.py
// :194-195) with sum(g^2) of the block written to a per-block slot for the gated RMSNorm.
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

__global__ __launch_bounds__(256) void ssm_kernel(SsmArgs a) {
  const int tid = threadIdx.x;
  const int m = blockIdx.y;
  const int pblocks = a.P / 16;
  const int head = blockIdx.x / pblocks;
  const int pb = blockIdx.x % pblocks;
  const int pl = tid >> 4;
  const int p = pb * 16 + pl;
  const int n0 = (tid & 15) * 8;
  const int DI = a.H * a.P;

  float* hp = a.h + (((size_t)m * a.H + head) * a.P + p) * a.N + n0;
  // state first: it is the bulk of the traffic and does not depend on the projection
  const f32x4 h0 = ld_nt_f4(hp);
  const f32x4 h1 = ld_nt_f4(hp + 4);

  const uint16_t* xr = a.xbc + (size_t)m * a.ld_xbc;
  const float dt = dev_log1pf(dev_expf(h2f(a.dt[(size_t)m * a.ld_dt + head]) + a.dt_bias[head]));
  const float abar = dev_expf(dt * -dev_expf(a.A_log[head]));
  const float xv = h2f(xr[head * a.P + p]);
  const float X = xv * dt;
  const uint4 b8 = *(const uint4*)(xr + DI + n0);
  const uint4 c8 = *(const uint4*)(xr + DI + a.N + n0);
  const uint32_t bw[4] = {b8.x, b8.y, b8.z, b8.w};
  const uint32_t cw[4] = {c8.x, c8.y, c8.z, c8.w};
  float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float bn = h2f((uint16_t)(bw[j >> 1] >> (16 * (j & 1))));
    const float cn = h2f((uint16_t)(cw[j >> 1] >> (16 * (j & 1))));
    hv[j] = __builtin_fmaf(abar, hv[j], X * bn);
    acc += (double)cn * (double)hv[j];
  }
  st_nt_f4(hp, f32x4{hv[0], hv[1], hv[2], hv[3]});
  st_nt_f4(hp + 4, f32x4{hv[4], hv[5], hv[6], hv[7]});
  acc = row_sum_f64(acc);  // the 16 lanes of a row (one DPP row) share state row p
  const float y = r16((float)acc + xv * a.D[head]);
  double gsqd = 0.0;
  if ((tid & 15) == 0) {
    float outv = y;
    if (a.z) {
      const float z = h2f(a.z[(size_t)m * a.ld_z + head * a.P + p]);
      const float sg = r16(1.0f / (1.0f + dev_expf(-z)));
      const float sz = r16(z * sg);
      outv = r16(y * sz);
      gsqd = (double)outv * (double)outv;
    }
    a.y_out[(size_t)m * a.ld_y + head * a.P + p] = f2h(outv);
  }
  if (a.sumsq_slots) {
    __shared__ double part[4];
    // lanes 0,16,32,48 of each wave hold the 4 rows' g^2; others hold 0
    const double s = wave_sum_dpp_f64(gsqd);
    if ((tid & 63) == 0) part[tid >> 6] = s;
    __syncthreads();
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
  hipLaunchKernelGGL(ssm_kernel, dim3(a.H * (a.P / 16), M), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_conv(const ConvArgs& a, int M, hipStream_t s) {
  hipLaunchKernelGGL(conv_kernel, dim3((a.C + 255) / 256, M), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
