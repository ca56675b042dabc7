// Mamba-2 single-step SSM update (+ gate), the same fused with out_proj's gated-norm prologue
// (decode at batch >= 5), and the stand-alone conv1d step (gfx950).
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

// One (sequence m, head, 16-row block) of the step. TAGGED: g goes to gT as tagged words
// (tag << 16) | fp16 with device-scope stores, and no sum(g^2) slot is written.
template <bool GATE, bool TAGGED>
__device__ __forceinline__ void ssm_rows(const SsmArgs& a, int bx, int m, uint32_t* gT, uint32_t epoch) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int pblocks = a.P / 16;
  const int head = bx / pblocks;
  const int pb = bx % pblocks;
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
    if (TAGGED) {
      uint32_t* gp = gT + (size_t)m * DI + head * a.P + p;
      const uint32_t tag = tag_of(epoch);
      st_dev(gp, (tag << 16) | f2h(o0));
      st_dev(gp + 8, (tag << 16) | f2h(o1));
    } else {
      uint16_t* yp = a.y_out + (size_t)m * a.ld_y + head * a.P + p;
      yp[0] = f2h(o0);
      yp[8] = f2h(o1);
    }
  }
  if (GATE && !TAGGED) {
    __shared__ double part[4];
    // lanes 0 and 32 of each wave hold their two rows' g^2; the others hold 0
    const double s = wave_sum_dpp_f64(gsqd);
    if (lane == 0) part[tid >> 6] = s;
    lds_barrier();
    if (tid == 0) a.sumsq_slots[(size_t)m * a.n_slots + bx] = part[0] + part[1] + part[2] + part[3];
  }
}

template <bool GATE>
__global__ __launch_bounds__(256) void ssm_kernel(SsmArgs a) {
  ssm_rows<GATE, false>(a, blockIdx.x, blockIdx.y, nullptr, 0u);
}

// ------------------------------------------------------------------------------------------
// ssm_prep_kernel (decode, batch >= 5): the step above for every (sequence, head, 16-row block)
// and, in the same launch, the gated-norm prologue of out_proj -- prep_kernel<OUT, 1>'s outputs
// (q, scale, LoRA intermediates) -- so the prologue needs no launch of its own and the prologues
// of early sequences run while the state of the last ones streams. 1-D grid: the H P / 16 SSM
// blocks of sequence 0, of sequence 1, ..., then 16 prologue workgroups per sequence (one per
// LoRA rank r): each polls the whole row of g from the tagged words, computes the gated RMSNorm
// (sum of g^2 from g itself), the maximum, the scale and rank r's intermediate, and writes the q
// bytes of column slice r. Every sum is a sum of exact products in fp64 (prep_kernel's values).
// Tags: every workgroup keeps its own launch count (read at the start, written back at the end);
// all of them start at zero and every launch runs every workgroup once, so all workgroups of a
// launch derive the same tag, and a word of the previous launch carries another one.
// Waiting: the prologue workgroups come after every SSM block in dispatch order (each XCD
// dispatches its share of the grid in order), so when one is placed every block it waits for has
// been placed or is behind SSM blocks only, which never wait: every wait ends, whatever the
// occupancy. Placed last, they also find most rows finished (one poll round) instead of polling
// through a row's lifetime, which, with a row's prologue next to its SSM blocks, took 2 TB/s of
// poll reads from the state stream (26% more time per decode step at batch 32). Every wait is
// also bounded (bit 2 of err on a timeout).
// Measured per decode step against the separate SSM and prologue kernels: 2371 -> 2322 us at
// batch 32 (1.3B shape), 6856 -> 6801 us at the 2.7B shape and batch 64. Slower: a row's
// prologues placed 8-9 rows behind its SSM blocks (2399 us), two ranks per prologue workgroup,
// the LoRA-B bytes loaded after the wait (+0.7 us per layer: one more cache round trip at the
// end), a 64-register limit (spills at K = 5120).
// ------------------------------------------------------------------------------------------
constexpr int kSpMaxK = 5120;
constexpr uint32_t kSpSpin = 1u << 18;
__device__ __forceinline__ bool sp_tag_ok(uint64_t v, uint32_t tag) {
  return ((uint32_t)v >> 16) == tag && ((uint32_t)(v >> 32) >> 16) == tag;
}

// Sixteen prologue workgroups per row, one LoRA rank rr each.
template <int NJ>
__device__ __forceinline__ void gated_prologue(const SsmPrepArgs& a, int rr, int m, uint32_t epoch) {
  __shared__ __attribute__((aligned(16))) uint32_t xn2[kSpMaxK / 2];  // g, then xn, as fp16 pairs
  __shared__ double red_d[4], red_h[4];
  __shared__ float red_f[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  constexpr int K = 512 * NJ;
  // wave w owns the column pairs 64 NJ w .. 64 NJ (w + 1) - 1, lane l the pairs u = 64 (NJ w + j) + l
  // (columns 2u, 2u + 1): every wave-wide load below is contiguous, and the loads of one thread are
  // 512 bytes apart (immediate offsets of one address). Norm weights, LoRA-B bytes and scale
  // first (loaded after the wait, they cost a cache round trip at the end of the launch), then
  // the tagged g words. All of them unconditional and raw until the polls are done: a select or a
  // conversion of a loaded value before the poll loop made the workgroup wait for these loads
  // before its first poll (without LoRA the bytes come from the norm weights, scaled by zero).
  const int8_t* lb = a.lB ? a.lB + (size_t)rr * K : (const int8_t*)a.norm_w;
  const uint16_t* lbs = a.lB ? a.lBs + rr : (const uint16_t*)a.norm_w;
  float2 wv[NJ];
  uint32_t bv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int u = 64 * (NJ * w + j) + lane;
    wv[j] = *(const float2*)(a.norm_w + 2 * u);
    bv[j] = *(const uint16_t*)(lb + 2 * u);
  }
  const uint16_t bs_raw = *lbs;
  const uint64_t* gp = (const uint64_t*)(a.gT + (size_t)m * K) + 64 * NJ * w + lane;
  // every round reloads all NJ words (each round's values are new definitions, so the registers
  // of one copy suffice; the extra loads of a round are a few KiB)
  uint64_t gv[NJ];
#pragma nounroll
  for (uint32_t it = 0;; ++it) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) gv[j] = ld_dev(gp + 64 * j);
    const uint32_t tag = tag_of(epoch);  // after the loads: waits for the launch count only
    bool good = true;
#pragma unroll
    for (int j = 0; j < NJ; ++j) good = good && sp_tag_ok(gv[j], tag);
    if (good) break;
    if (it == kSpSpin) {
      atomicOr(a.err, DFSSM_ERR_WAIT_SSM_PROLOGUE);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  const float bs = a.lB ? h2f(bs_raw) : 0.0f;
  // g pairs to this thread's own LDS slots (read back, then overwritten with xn, by this thread
  // alone), so the g registers are free before the norm pass
  double part = 0.0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t gpair = (uint32_t)(gv[j] & 0xffffu) | ((uint32_t)(gv[j] >> 16) & 0xffff0000u);
    xn2[64 * (NJ * w + j) + lane] = gpair;
    const double g0 = (double)h2f((uint16_t)gpair), g1 = (double)h2f((uint16_t)(gpair >> 16));
    part += g0 * g0;
    part += g1 * g1;
  }
  {  // sum of squares (fp64: the sums are exact)
    const double pw = wave_sum_dpp_f64(part);
    if (lane == 0) red_d[w] = pw;
  }
  lds_barrier();
  const double ss = (red_d[0] + red_d[1]) + (red_d[2] + red_d[3]);
  const float var = (float)ss * (1.0f / (float)K);
  const float r = 1.0f / sqrt_rn(var + 1e-5f);
  float mx = 0.0f;
  double hacc = 0.0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t gpair = xn2[64 * (NJ * w + j) + lane];
    const float x0 = r16((h2f((uint16_t)gpair) * r) * wv[j].x);
    const float x1 = r16((h2f((uint16_t)(gpair >> 16)) * r) * wv[j].y);
    mx = fmaxf(mx, fmaxf(fabsf(x0), fabsf(x1)));
    xn2[64 * (NJ * w + j) + lane] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
    // fp16 x fp16 is exact in fp32
    const float b0 = r16((float)(int8_t)bv[j] * bs);
    const float b1 = r16((float)(int8_t)(bv[j] >> 8) * bs);
    hacc += (double)(x0 * b0);
    hacc += (double)(x1 * b1);
  }
  {  // LoRA sum and maximum in one exchange (after every wave has read the squares)
    const double hw = wave_sum_dpp_f64(hacc);
    const float mw = wave_max_dpp_f32(mx);
    lds_barrier();
    if (lane == 0) {
      red_h[w] = hw;
      red_f[w] = mw;
    }
  }
  lds_barrier();  // also publishes xn
  const float amax = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
  const float xs = quant_scale(amax);
  const float rinv = quant_rcp(xs);
  const uint16_t* xn = (const uint16_t*)xn2;
  const int lo = rr * (K / 16), hi = lo + K / 16;
  for (int k = lo + tid; k < hi; k += 256) a.q_out[(size_t)m * a.ld_q + k] = (int8_t)quant_i8(h2f(xn[k]), rinv);
  if (tid == 0) {
    if (a.lB) a.h_out[(size_t)m * DFSSM_LORA_R + rr] = r16((float)((red_h[0] + red_h[1]) + (red_h[2] + red_h[3])));
    if (rr == 0) a.xs_out[m] = xs;
  }
}

template <int NJ>
__global__ __launch_bounds__(256) void ssm_prep_kernel(SsmPrepArgs a, int M) {
  const int nsb = a.s.H * (a.s.P / 16), bx = blockIdx.x;
  uint32_t* cnt = a.launches + bx;
  const uint32_t epoch = ld_dev(cnt);  // the tag (tag_of) is derived where it is used
  if (bx < nsb * M) {
    const int m = bx / nsb;
    ssm_rows<true, true>(a.s, bx - m * nsb, m, a.gT, epoch);
  } else {
    const int j = bx - nsb * M;
    gated_prologue<NJ>(a, j % DFSSM_LORA_R, j / DFSSM_LORA_R, epoch);
  }
  lds_barrier();  // every wave has read the count (and used its tag) before it is advanced
  if (threadIdx.x == 0) *cnt = epoch + 1u;  // read by the next launch only: a plain store suffices
}

bool ssm_prep_supported(int M, int K, int P) { return M >= 1 && K <= kSpMaxK && K % 512 == 0 && P % 16 == 0; }

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

hipError_t launch_ssm_prep(const SsmPrepArgs& a, int M, hipStream_t s) {
  const int K = a.s.H * a.s.P;
  if (!a.s.z || !a.gT || !a.launches || !a.err || !a.norm_w || !a.q_out || !a.xs_out || !a.h_out ||
      a.ld_q < K || (a.lB && !a.lBs))
    return hipErrorInvalidValue;
  if (!ssm_prep_supported(M, K, a.s.P)) return hipErrorInvalidValue;
  const dim3 g((a.s.H * (a.s.P / 16) + DFSSM_LORA_R) * M);
#define DFSSM_SP_LAUNCH(NJ) hipLaunchKernelGGL(ssm_prep_kernel<NJ>, g, dim3(256), 0, s, a, M);
  switch (K / 512) {
    case 1: DFSSM_SP_LAUNCH(1) break;
    case 2: DFSSM_SP_LAUNCH(2) break;
    case 3: DFSSM_SP_LAUNCH(3) break;
    case 4: DFSSM_SP_LAUNCH(4) break;
    case 5: DFSSM_SP_LAUNCH(5) break;
    case 6: DFSSM_SP_LAUNCH(6) break;
    case 7: DFSSM_SP_LAUNCH(7) break;
    case 8: DFSSM_SP_LAUNCH(8) break;
    case 9: DFSSM_SP_LAUNCH(9) break;
    case 10: DFSSM_SP_LAUNCH(10) break;
    default: return hipErrorInvalidValue;
  }
#undef DFSSM_SP_LAUNCH
  return hipGetLastError();
}

hipError_t launch_conv(const ConvArgs& a, int M, hipStream_t s) {
  hipLaunchKernelGGL(conv_kernel, dim3((a.C + 255) / 256, M), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
