// Prompt prefill, layer-major (gfx950): the n prompt tokens of every sequence go through one
// layer together, then the next layer. The projections and their prologues are row-independent,
// so the decode kernels run them on all batch x n rows at once (prep_kernel, gemm_kernel); only
// the two recurrences walk the tokens in order, here:
//
//   conv_seq_kernel  one thread per (sequence, conv channel): the fp16 shift register stays in
//                    registers while the thread walks the tokens; out = s0 w0 + s1 w1 + s2 w2 +
//                    x w3 + b (left to right, fp32), x <- fp16(out sigmoid(out)), in place on the
//                    projection rows, whose raw values the in_proj GEMM wrote (no conv there).
//   ssm_scan_kernel  one workgroup per (sequence, head, up to 4 blocks of 16 state rows): the fp32
//                    state of the rows stays in registers for all n tokens (read and written
//                    once per layer instead of once per token). Per token the arithmetic, the
//                    thread -> state-element map and every reduction tree are those of
//                    ssm_kernel<true>, so state, g and the per-block sum(g^2) slots are bit-for-bit
//                    what n decode steps produce. The tokens' operands (B | C, x, z, dt) are staged
//                    in LDS kTT tokens at a time, double-buffered, with softplus dt, exp(dt A),
//                    the gate factor z sigma(z), B widened to fp32 and C to fp64 computed once per
//                    token (per row) while staging.
//
// Together with the row-wise kernels this makes the prefill equal, bit for bit, to n calls of the
// decode step (Mamba-2 recurrence of df_ssm_kernels.cu:53-103 / training/
// df_ssm_mamba2_distill_dfw.py:346-381, evaluated token by token as the reference's
// cpu_inference_driver.py:186-204 ingests a prompt).
#include <type_traits>

#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

__global__ __launch_bounds__(256) void conv_seq_kernel(ConvSeqArgs a) {
  const int ch = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (ch >= a.C) return;
  uint16_t* cs = a.state + ((size_t)b * a.C + ch) * 3;
  uint16_t s0 = cs[0], s1 = cs[1], s2 = cs[2];
  const uint16_t* wc = a.w + (size_t)ch * 4;
  const float w0 = h2f(wc[0]), w1 = h2f(wc[1]), w2 = h2f(wc[2]), w3 = h2f(wc[3]);
  const float cb = h2f(a.b[ch]);
  uint16_t* col = a.x + (size_t)b * a.T * a.ld + ch;  // token t of sequence b: col[t * ld]
  constexpr int U = 8;
  for (int t0 = 0; t0 < a.T; t0 += U) {
    uint16_t raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) raw[u] = col[(size_t)(t0 + u < a.T ? t0 + u : a.T - 1) * a.ld];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t0 + u >= a.T) break;
      const uint16_t xo = raw[u];
      float o = h2f(s0) * w0;
      o = o + h2f(s1) * w1;
      o = o + h2f(s2) * w2;
      o = o + h2f(xo) * w3;
      o = o + cb;
      const float sig = 1.0f / (1.0f + dev_expf(-o));
      col[(size_t)(t0 + u) * a.ld] = f2h(o * sig);
      s0 = s1;
      s1 = s2;
      s2 = xo;
    }
  }
  cs[0] = s0;
  cs[1] = s1;
  cs[2] = s2;
}

constexpr int kTT = 16;    // tokens staged per round
constexpr int kPGMax = 4;  // 16-row state blocks per workgroup
constexpr int kTG = 4;     // tokens whose reductions run together

struct ScanBuf {
  float bf[kTT][128];              // B of each token, widened once here (fp16 values)
  double cd[kTT][128];             // C of each token, widened to fp64 (fp16 values)
  uint16_t x[kTT][16 * kPGMax];    // x of the workgroup's rows
  float sz[kTT][16 * kPGMax];      // gate factor fp16(z sigma(z)) of the workgroup's rows
  float dt[kTT], abar[kTT];        // softplus dt and exp(dt A) of the head
  double gpart[kTT][4 * kPGMax];   // per-wave partial sum(g^2), reduced per block after the round
};

// Raw operands of one round, loaded into registers one round ahead.
template <int PG>
struct ScanRaw {
  static constexpr int KB = (kTT * 32 + 256 * PG - 1) / (256 * PG);
  u32x4 bc[KB];    // 8 halves of B | C: chunk i = tid + 256 PG k, token i / 32, halves 8 (i % 32) ..
  uint16_t x, z;   // token tid / (16 PG), row tid % (16 PG) (tid < kTT * 16 PG = blockDim)
  uint16_t dt;     // token tid (tid < kTT)
};

template <int PG>
__device__ __forceinline__ ScanRaw<PG> scan_load(const ScanArgs& a, int b, int head, int t0) {
  const int tid = threadIdx.x;
  constexpr int NT = 256 * PG, RW = 16 * PG;
  ScanRaw<PG> r{};
  const size_t row0 = (size_t)b * a.T;
  // clamped token indices: rows past the end re-read the last token (never consumed)
#pragma unroll
  for (int k = 0; k < ScanRaw<PG>::KB; ++k) {
    const int i = tid + NT * k;
    const int t = t0 + i / 32;
    const uint16_t* p = a.xbc + (row0 + (t < a.T ? t : a.T - 1)) * a.ld_xbc + a.H * a.P + 8 * (i % 32);
    if (i < kTT * 32) r.bc[k] = *(const u32x4*)p;
  }
  if (tid < kTT * RW) {
    const int t = t0 + tid / RW;
    const size_t row = row0 + (t < a.T ? t : a.T - 1);
    const int col = head * a.P + a.pb0 * 16 + tid % RW;
    r.x = a.xbc[row * a.ld_xbc + col];
    r.z = a.z[row * a.ld_z + col];
  }
  if (tid < kTT) {
    const int t = t0 + tid;
    r.dt = a.dt[(row0 + (t < a.T ? t : a.T - 1)) * a.ld_dt + head];
  }
  return r;
}

template <int PG>
__device__ __forceinline__ void scan_stage(ScanBuf& S, const ScanRaw<PG>& r, float dtb, float nA) {
  const int tid = threadIdx.x;
  constexpr int NT = 256 * PG, RW = 16 * PG;
#pragma unroll
  for (int k = 0; k < ScanRaw<PG>::KB; ++k) {
    const int i = tid + NT * k;
    if (i < kTT * 32) {
      const int t = i / 32, c = i % 32;  // halves 8 c .. 8 c + 7 of B | C
      const u32x4 v = r.bc[k];
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = h2f((uint16_t)(v[e >> 1] >> (16 * (e & 1))));
      if (c < 16) {
        *(f32x4*)&S.bf[t][8 * c] = f32x4{f[0], f[1], f[2], f[3]};
        *(f32x4*)&S.bf[t][8 * c + 4] = f32x4{f[4], f[5], f[6], f[7]};
      } else {
        double* d = &S.cd[t][8 * (c - 16)];
#pragma unroll
        for (int e = 0; e < 8; ++e) d[e] = (double)f[e];
      }
    }
  }
  if (tid < kTT * RW) {
    const int t = tid / RW, i = tid % RW;
    S.x[t][i] = r.x;
    const float z = h2f(r.z);
    S.sz[t][i] = r16(z * r16(1.0f / (1.0f + dev_expf(-z))));
  }
  if (tid < kTT) {
    const float dt = dev_log1pf(dev_expf(h2f(r.dt) + dtb));
    S.dt[tid] = dt;
    S.abar[tid] = dev_expf(dt * nA);
  }
}

// v of lane l + 16 in lanes 0..15 and 32..47, and of lane l + 32 in lanes 0..31, by the gfx950
// lane swaps (v_permlane16_swap between rows 0|1 and 2|3, v_permlane32_swap between the halves;
// with both operands v, the second result holds the partner row's value in rows 0 and 2).
__device__ __forceinline__ double lane_plus16(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_permlane16_swap((uint32_t)u, (uint32_t)u, false, false)[1];
  const uint32_t hi = __builtin_amdgcn_permlane16_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false)[1];
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double lane_plus32(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_permlane32_swap((uint32_t)u, (uint32_t)u, false, false)[1];
  const uint32_t hi = __builtin_amdgcn_permlane32_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false)[1];
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

template <int PG>
__global__ __launch_bounds__(256 * PG) void ssm_scan_kernel(ScanArgs a) {
  __shared__ ScanBuf buf[2];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int grp = tid >> 8;            // 16-row block of this thread within the workgroup
  const int gt = tid & 255;            // thread within its block: the ssm_kernel map
  const int b = blockIdx.y;
  const int wg_per_head = a.P / (16 * PG);
  const int head = blockIdx.x / wg_per_head;
  const int pb = (blockIdx.x % wg_per_head) * PG + grp;  // state block of this thread
  ScanArgs aa = a;
  aa.pb0 = (blockIdx.x % wg_per_head) * PG;
  const int n0 = 4 * (gt & 31);
  const int pr = gt >> 5;              // rows pr and pr + 8 of the block
  const int p = pb * 16 + pr;
  const int rl = grp * 16 + pr;        // row index within the workgroup's staged x / sz
  const float Dh = a.D[head], dtb = a.dt_bias[head];
  const float nA = -dev_expf(a.A_log[head]);

  ScanRaw<PG> raw = scan_load<PG>(aa, b, head, 0);
  float* hp = a.h + (((size_t)b * a.H + head) * a.P + p) * a.N + n0;
  const f32x4 s0 = ld_nt_f4(hp);
  const f32x4 s1 = ld_nt_f4(hp + 8 * a.N);
  float h0[4] = {s0.x, s0.y, s0.z, s0.w}, h1[4] = {s1.x, s1.y, s1.z, s1.w};
  scan_stage<PG>(buf[0], raw, dtb, nA);
  lds_barrier();

  const int rounds = (a.T + kTT - 1) / kTT;
  for (int rd = 0; rd < rounds; ++rd) {
    const int t0 = rd * kTT;
    ScanBuf& S = buf[rd & 1];
    if (rd + 1 < rounds) raw = scan_load<PG>(aa, b, head, t0 + kTT);
    const int nt = a.T - t0 < kTT ? a.T - t0 : kTT;
    // Tokens in groups of kTG: the state updates are a chain of fmas, but a token's readout and
    // sum(g^2) reductions feed nothing later, so a group's reductions are independent chains the
    // compiler interleaves. Slots of a group past nt update nothing and store nothing.
    for (int t = 0; t < nt; t += kTG) {
      double acc0[kTG], acc1[kTG];
      float xv0[kTG], xv1[kTG];
      // FULL: all kTG tokens of the group exist (every group but a prompt's last), no selects
      auto group = [&](auto full_t) {
        constexpr bool FULL = decltype(full_t)::value;
#pragma unroll
        for (int j = 0; j < kTG; ++j) {
          const int tt = FULL ? t + j : (t + j < nt ? t + j : t);
          const f32x4 b4 = *(const f32x4*)&S.bf[tt][n0];
          const float bq[4] = {b4.x, b4.y, b4.z, b4.w};
          const double* cp = &S.cd[tt][n0];
          const double cq[4] = {cp[0], cp[1], cp[2], cp[3]};
          const float dt = S.dt[tt], abar = S.abar[tt];
          xv0[j] = h2f(S.x[tt][rl]);
          xv1[j] = h2f(S.x[tt][rl + 8]);
          const float X0 = xv0[j] * dt, X1 = xv1[j] * dt;
          const bool valid = FULL || t + j < nt;
          acc0[j] = 0.0;
          acc1[j] = 0.0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float n0v = __builtin_fmaf(abar, h0[q], X0 * bq[q]);
            const float n1v = __builtin_fmaf(abar, h1[q], X1 * bq[q]);
            h0[q] = valid ? n0v : h0[q];
            h1[q] = valid ? n1v : h1[q];
            // C h is exact in fp64 (11 x 24 significant bits), so the fma rounds exactly as
            // ssm_kernel's multiply-then-add
            acc0[j] = __builtin_fma(cq[q], (double)h0[q], acc0[j]);
            acc1[j] = __builtin_fma(cq[q], (double)h1[q], acc1[j]);
          }
        }
      };
      if (t + kTG <= nt) group(std::true_type{});
      else group(std::false_type{});
#pragma unroll
      for (int j = 0; j < kTG; ++j) {
        acc0[j] = row_sum_f64(acc0[j]);
        acc1[j] = row_sum_f64(acc1[j]);
      }
      double gsqd[kTG];
#pragma unroll
      for (int j = 0; j < kTG; ++j) {
        // the two 16-lane row sums of each state row added as ssm_kernel's readlanes add them:
        // (lane 0) + (lane 16) in lane 0, (lane 32) + (lane 48) in lane 32
        const double s0 = acc0[j] + lane_plus16(acc0[j]);
        const double s1 = acc1[j] + lane_plus16(acc1[j]);
        gsqd[j] = 0.0;
        if ((gt & 31) == 0 && t + j < nt) {
          const float y0 = r16((float)s0 + xv0[j] * Dh);
          const float y1 = r16((float)s1 + xv1[j] * Dh);
          const float o0 = r16(y0 * S.sz[t + j][rl]);
          const float o1 = r16(y1 * S.sz[t + j][rl + 8]);
          gsqd[j] = (double)o0 * (double)o0 + (double)o1 * (double)o1;
          uint16_t* yp = a.y_out + ((size_t)b * a.T + t0 + t + j) * a.ld_y + head * a.P + p;
          yp[0] = f2h(o0);
          yp[8] = f2h(o1);
        }
      }
      // the wave's sum(g^2): only lanes 0 and 32 hold non-zero values, so ssm_kernel's
      // wave_sum_dpp_f64 adds exact zeros to them and equals (lane 0) + (lane 32)
#pragma unroll
      for (int j = 0; j < kTG; ++j) {
        const double s = gsqd[j] + lane_plus32(gsqd[j]);  // (lane 0) + (lane 32) in lane 0
        if (lane == 0 && t + j < nt) S.gpart[t + j][w] = s;
      }
    }
    if (rd + 1 < rounds) scan_stage<PG>(buf[(rd + 1) & 1], raw, dtb, nA);
    lds_barrier();
    // per-block sum(g^2) of this round's tokens, in ssm_kernel's order (waves 0 + 1 + 2 + 3)
    if (tid < nt * PG) {
      const int t = tid / PG, g = tid % PG;
      const double* gp = &S.gpart[t][4 * g];
      const int slot = head * (a.P / 16) + aa.pb0 + g;
      a.sumsq_slots[((size_t)b * a.T + t0 + t) * a.n_slots + slot] = gp[0] + gp[1] + gp[2] + gp[3];
    }
  }
  st_nt_f4(hp, f32x4{h0[0], h0[1], h0[2], h0[3]});
  st_nt_f4(hp + 8 * a.N, f32x4{h1[0], h1[1], h1[2], h1[3]});
}

// dst[b] = src[b * T + T - 1]: the last token's row of every sequence.
__global__ __launch_bounds__(256) void last_rows_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                        int T, int D) {
  const int b = blockIdx.x;
  const uint16_t* s = src + ((size_t)b * T + T - 1) * D;
  for (int k = threadIdx.x; k < D; k += 256) dst[(size_t)b * D + k] = s[k];
}

hipError_t launch_conv_seq(const ConvSeqArgs& a, int batch, hipStream_t s) {
  hipLaunchKernelGGL(conv_seq_kernel, dim3((a.C + 255) / 256, batch), dim3(256), 0, s, a);
  return hipGetLastError();
}

int scan_groups(int P) {
  const int pbs = P / 16;
  return pbs % 4 == 0 ? 4 : (pbs % 2 == 0 ? 2 : 1);
}

hipError_t launch_ssm_scan(const ScanArgs& a, int batch, hipStream_t s) {
  if (a.T < 1 || a.P % 16 || a.N != 128) return hipErrorInvalidValue;
  const int PG = scan_groups(a.P);
  const dim3 grid(a.H * (a.P / (16 * PG)), batch);
  switch (PG) {
    case 4: hipLaunchKernelGGL(ssm_scan_kernel<4>, grid, dim3(1024), 0, s, a); break;
    case 2: hipLaunchKernelGGL(ssm_scan_kernel<2>, grid, dim3(512), 0, s, a); break;
    default: hipLaunchKernelGGL(ssm_scan_kernel<1>, grid, dim3(256), 0, s, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_last_rows(const uint16_t* src, uint16_t* dst, int batch, int T, int D, hipStream_t s) {
  hipLaunchKernelGGL(last_rows_kernel, dim3(batch), dim3(256), 0, s, src, dst, T, D);
  return hipGetLastError();
}

}  // namespace dfssm
