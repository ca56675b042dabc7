// Scaffold projection kernels: 1-bit packed GEMV with fused prologue and epilogue (gfx950).
//
// One workgroup (256 threads, 4 waves) owns one group of 64 output rows. Lane l of every wave
// owns row 64*g + l; wave w streams a quarter of the K columns. The sign bits are stored
// re-tiled at load time as [row group][16-byte chunk][64 lanes][4 words] so that each wave-wide
// 16-byte load is one contiguous 1 KiB transaction (still 1 bit per weight).
//
// Arithmetic: with planes P_b[j] = bit b of the int8 activations of columns 32j..32j+31,
//   sum_{bit=1} q = sum_{b<7} 2^b popc(w & P_b) - 128 popc(w & P_7)
//   acc = sum_k q_k * (2 bit_k - 1) = 2 * sum_{bit=1} q - sum_k q_k          (exact int32)
// i.e. 16 VALU ops (and + bcnt-accumulate per plane) per 32 weights per activation row.
//
// Prologue (every workgroup recomputes it; the activation vector is 4-10 KiB and L2-resident):
//   MODE_IN : xn = RMSNorm(x) * ln_w             (df_ssm_inference.py:141-145,165)
//   MODE_OUT: yn = RMSNorm(g) * norm_w with sum(g^2) taken from the SSM kernel's per-block
//             partials                            (df_ssm_inference.py:194-196)
//   then the int8 quantizer (:147-152), the bit planes, sum q, and the rank-16 LoRA
//   intermediate h16 = fp16(xn @ B16^T)          (:173,204).
// Epilogue per row n: y = fp16(fp16(fp16(acc) * s_x) * s_w[n]) (:158), out = fp16(y + h16.A16[n])
// (:173,204); MODE_IN additionally applies the depthwise conv + SiLU to the xBC rows
// (df_ssm_kernels.cu:27-47) and writes z | xBC | dt_raw; MODE_OUT adds the residual (:207).
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kNT = 256;

template <int M>
struct ProjLds {
  uint32_t planes[M][8192 / 32][8];   // bit planes of q, per word (up to K = 8192)
  uint16_t xn[8192];                  // normalized activations of the current row
  double lora_part[DFSSM_LORA_R][16]; // LoRA-h partials [r][slice]
  float hl[M][DFSSM_LORA_R];          // h16 values (as float)
  int T[4][M][64];                    // per-wave partial sum_{bit=1} q
  double red_d[4];
  float red_f[4];
  int red_i[4];
  int S[M];
  float xs[M];
};

// Prologue for one activation row m: builds xn (LDS), scale, planes, S, h16.
template <int M, int MODE>
__device__ void proj_prologue_row(const ProjArgs& a, int m, ProjLds<M>& L) {
  const int K = a.K, tid = threadIdx.x;
  const uint16_t* src = a.act + (size_t)m * a.ld_act;
  // 1) sum of squares -> r
  double ss;
  if (MODE == DFSSM_MODE_IN) {
    double part = 0.0;
    for (int k = tid; k < K; k += kNT) { double v = (double)h2f(src[k]); part += v * v; }
    ss = block_sum_f64<kNT>(part, L.red_d);
  } else {
    const double* sl = a.sumsq_slots + (size_t)m * a.n_slots;
    double part = 0.0;
    for (int j = tid; j < a.n_slots; j += kNT) part += sl[j];
    ss = block_sum_f64<kNT>(part, L.red_d);
  }
  const float var = (float)ss * (1.0f / (float)K);
  const float r = 1.0f / sqrt_rn(var + 1e-5f);
  // 2) xn = fp16((x * r) * w), amax
  float amax = 0.0f;
  for (int k = tid; k < K; k += kNT) {
    float v = r16((h2f(src[k]) * r) * a.norm_w[k]);
    L.xn[k] = f2h(v);
    amax = fmaxf(amax, fabsf(v));
  }
  amax = block_max_f32<kNT>(amax, L.red_f);
  const float xs = quant_scale(amax);
  // 3) q, planes (ballot over 64 consecutive columns), S
  int qsum = 0;
  const int lane = tid & 63;
  for (int k0 = (tid & ~63); k0 < K; k0 += kNT) {
    const int k = k0 + lane;
    int q = quant_i8(h2f(L.xn[k]), xs);
    qsum += q;
    const uint32_t qb = (uint32_t)q & 0xffu;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t mask = __ballot((qb >> b) & 1u);
      if (lane == b) L.planes[m][k0 / 32][b] = (uint32_t)mask;
      if (lane == 8 + b) L.planes[m][k0 / 32 + 1][b] = (uint32_t)(mask >> 32);
    }
  }
  const int S = block_sum_i32<kNT>(qsum, L.red_i);
  // 4) LoRA intermediate: thread (r = tid % 16, slice = tid / 16) sums columns of its slice.
  if (a.lB) {
    const int rr = tid & 15, slice = tid >> 4;
    const int per = K / 16;
    const int8_t* brow = a.lB + (size_t)rr * K + slice * per;
    const uint16_t* xsl = L.xn + slice * per;
    const float bs = h2f(a.lBs[rr]);
    double acc = 0.0;
    for (int k = 0; k < per; k += 4) {
      const uint32_t b4 = *(const uint32_t*)(brow + k);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b16 = r16((float)(int8_t)(b4 >> (8 * j)) * bs);
        acc += (double)h2f(xsl[k + j]) * (double)b16;
      }
    }
    L.lora_part[rr][slice] = acc;
  }
  __syncthreads();
  if (tid < DFSSM_LORA_R) {
    double t = 0.0;
#pragma unroll
    for (int s = 0; s < 16; ++s) t += L.lora_part[tid][s];
    L.hl[m][tid] = r16((float)t);
  }
  if (tid == 0) { L.S[m] = S; L.xs[m] = xs; }
  __syncthreads();
}

template <int M, int MODE>
__global__ __launch_bounds__(kNT) void proj_kernel(ProjArgs a) {
  __shared__ ProjLds<M> L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  const int KW = a.K / 32;             // words per row
  const int CH = KW / 4;               // 16-byte chunks per row
  const int CPW = CH / 4;              // chunks per wave
  const uint4* bits = (const uint4*)a.bits + ((size_t)g * CH + wave * CPW) * 64 + lane;

  // Issue the first chunks' loads before the prologue: the weights do not depend on activations.
  constexpr int PRE = 4;
  u32x4 pre[PRE];
#pragma unroll
  for (int c = 0; c < PRE; ++c) if (c < CPW) pre[c] = ld_nt(bits + (size_t)c * 64);

  for (int m = 0; m < M; ++m) proj_prologue_row<M, MODE>(a, m, L);

  uint32_t cnt[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int b = 0; b < 8; ++b) cnt[m][b] = 0;

  for (int c = 0; c < CPW; ++c) {
    u32x4 w4;
    if (c < PRE) {
#pragma unroll
      for (int cc = 0; cc < PRE; ++cc) if (cc == c) w4 = pre[cc];
    } else {
      w4 = ld_nt(bits + (size_t)c * 64);
    }
    const int word0 = (wave * CPW + c) * 4;
    const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4 p0 = *(const uint4*)&L.planes[m][word0 + i][0];
        const uint4 p1 = *(const uint4*)&L.planes[m][word0 + i][4];
        cnt[m][0] += __builtin_popcount(ww[i] & p0.x);
        cnt[m][1] += __builtin_popcount(ww[i] & p0.y);
        cnt[m][2] += __builtin_popcount(ww[i] & p0.z);
        cnt[m][3] += __builtin_popcount(ww[i] & p0.w);
        cnt[m][4] += __builtin_popcount(ww[i] & p1.x);
        cnt[m][5] += __builtin_popcount(ww[i] & p1.y);
        cnt[m][6] += __builtin_popcount(ww[i] & p1.z);
        cnt[m][7] += __builtin_popcount(ww[i] & p1.w);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int t = 0;
#pragma unroll
    for (int b = 0; b < 7; ++b) t += (int)(cnt[m][b] << b);
    t -= (int)(cnt[m][7] << 7);
    L.T[wave][m][lane] = t;
  }
  __syncthreads();

  // Epilogue: thread (m = tid / 64, row lane) -- M <= 4 rows of 64.
  if (tid < M * 64) {
    const int m = tid >> 6;
    const int n = g * 64 + lane;
    if (n < a.N) {
      const int T = L.T[0][m][lane] + L.T[1][m][lane] + L.T[2][m][lane] + L.T[3][m][lane];
      const int acc = 2 * T - L.S[m];
      if (a.acc_out) a.acc_out[(size_t)m * a.N + n] = acc;
      const float y = r16(r16(r16((float)acc) * L.xs[m]) * h2f(a.wscale[n]));
      const uint4 a16 = *(const uint4*)(a.lA + (size_t)n * DFSSM_LORA_R);
      const uint32_t av[4] = {a16.x, a16.y, a16.z, a16.w};
      const float as = h2f(a.lAs[n]);
      double lo = 0.0;
#pragma unroll
      for (int rr = 0; rr < DFSSM_LORA_R; ++rr) {
        const float aq = r16((float)(int8_t)(av[rr >> 2] >> (8 * (rr & 3))) * as);
        lo += (double)L.hl[m][rr] * (double)aq;
      }
      float out = r16((float)lo + y);
      if (MODE == DFSSM_MODE_IN) {
        const int ch = n - a.conv_lo;
        if (ch >= 0 && ch < a.conv_c) {
          // depthwise conv (k=4) + SiLU on the xBC channel ch; state (M, C, 3) fp16
          uint16_t* cs = a.conv_state + ((size_t)m * a.conv_c + ch) * 3;
          const float s0 = h2f(cs[0]), s1 = h2f(cs[1]), s2 = h2f(cs[2]);
          const uint16_t xo = f2h(out);
          cs[0] = cs[1];
          cs[1] = cs[2];
          cs[2] = xo;
          const uint16_t* wc = a.conv_w + (size_t)ch * 4;
          const float xv = h2f(xo);
          float o = s0 * h2f(wc[0]);
          o = o + s1 * h2f(wc[1]);
          o = o + s2 * h2f(wc[2]);
          o = o + xv * h2f(wc[3]);
          o = o + h2f(a.conv_b[ch]);
          const float sig = 1.0f / (1.0f + dev_expf(-o));
          out = o * sig;
        }
        a.out[(size_t)m * a.ld_out + n] = f2h(out);
      } else {
        uint16_t* xp = a.out + (size_t)m * a.ld_out + n;
        *xp = f2h(h2f(*xp) + out);
      }
    }
  }
}

// Stand-alone RMSNorm + quantizer (one workgroup per activation row): writes xn, q and the scale.
__global__ __launch_bounds__(kNT) void prologue_kernel(ProjArgs a, uint16_t* xn_out, int8_t* q_out, uint16_t* s_out) {
  __shared__ ProjLds<1> L;
  const int m = blockIdx.x;
  ProjArgs b = a;
  b.act = a.act + (size_t)m * a.ld_act;
  proj_prologue_row<1, DFSSM_MODE_IN>(b, 0, L);
  const float xs = L.xs[0];
  for (int k = threadIdx.x; k < a.K; k += kNT) {
    const uint16_t v = L.xn[k];
    xn_out[(size_t)m * a.K + k] = v;
    q_out[(size_t)m * a.K + k] = (int8_t)quant_i8(h2f(v), xs);
  }
  if (threadIdx.x == 0) s_out[m] = f2h(xs);
}

// Stand-alone scaffold GEMM for given int8 activations (tests / microbench): acc and y only.
template <int M>
__global__ __launch_bounds__(kNT) void scaffold_kernel(ScaffoldArgs a) {
  __shared__ uint32_t planes[M][8192 / 32][8];
  __shared__ int T[4][M][64];
  __shared__ int S[M];
  __shared__ int red_i[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  const int K = a.K, KW = K / 32, CH = KW / 4, CPW = CH / 4;
  const uint4* bits = (const uint4*)a.bits + ((size_t)g * CH + wave * CPW) * 64 + lane;
  for (int m = 0; m < M; ++m) {
    int qsum = 0;
    for (int k0 = (tid & ~63); k0 < K; k0 += kNT) {
      const int k = k0 + lane;
      const int q = a.q[(size_t)m * K + k];
      qsum += q;
      const uint32_t qb = (uint32_t)q & 0xffu;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint64_t mask = __ballot((qb >> b) & 1u);
        if (lane == b) planes[m][k0 / 32][b] = (uint32_t)mask;
        if (lane == 8 + b) planes[m][k0 / 32 + 1][b] = (uint32_t)(mask >> 32);
      }
    }
    const int s = block_sum_i32<kNT>(qsum, red_i);
    if (tid == 0) S[m] = s;
  }
  __syncthreads();
  uint32_t cnt[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int b = 0; b < 8; ++b) cnt[m][b] = 0;
  for (int c = 0; c < CPW; ++c) {
    const u32x4 w4 = ld_nt(bits + (size_t)c * 64);
    const int word0 = (wave * CPW + c) * 4;
    const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int b = 0; b < 8; ++b) cnt[m][b] += __builtin_popcount(ww[i] & planes[m][word0 + i][b]);
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int t = 0;
#pragma unroll
    for (int b = 0; b < 7; ++b) t += (int)(cnt[m][b] << b);
    t -= (int)(cnt[m][7] << 7);
    T[wave][m][lane] = t;
  }
  __syncthreads();
  if (tid < M * 64) {
    const int m = tid >> 6;
    const int n = g * 64 + lane;
    if (n < a.N) {
      const int acc = 2 * (T[0][m][lane] + T[1][m][lane] + T[2][m][lane] + T[3][m][lane]) - S[m];
      if (a.acc_out) a.acc_out[(size_t)m * a.N + n] = acc;
      if (a.y_out)
        a.y_out[(size_t)m * a.N + n] = f2h(r16(r16((float)acc) * h2f(a.xscale[m])) * h2f(a.wscale[n]));
    }
  }
}

// Re-tile row-major (N, K/32) sign-bit words into [N_pad/64][K/128][64][4].
__global__ void tile_bits_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int N, int KW, int n_pad) {
  const size_t total = (size_t)n_pad * KW;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    // destination index decomposition
    const int w4 = (int)(i & 3);
    const int lane = (int)((i >> 2) & 63);
    const size_t rest = i >> 8;              // g * CH + c
    const int CH = KW / 4;
    const int c = (int)(rest % CH);
    const int g = (int)(rest / CH);
    const int row = g * 64 + lane;
    const int word = c * 4 + w4;
    dst[i] = row < N ? src[(size_t)row * KW + word] : 0u;
  }
}

template <int M>
static hipError_t launch_proj_m(const ProjArgs& a, int mode, hipStream_t s) {
  const int groups = (a.N + 63) / 64;
  if (mode == DFSSM_MODE_IN)
    hipLaunchKernelGGL((proj_kernel<M, DFSSM_MODE_IN>), dim3(groups), dim3(kNT), 0, s, a);
  else
    hipLaunchKernelGGL((proj_kernel<M, DFSSM_MODE_OUT>), dim3(groups), dim3(kNT), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_proj(const ProjArgs& a, int M, int mode, hipStream_t s) {
  switch (M) {
    case 1: return launch_proj_m<1>(a, mode, s);
    case 2: return launch_proj_m<2>(a, mode, s);
    case 3: return launch_proj_m<3>(a, mode, s);
    case 4: return launch_proj_m<4>(a, mode, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_scaffold(const ScaffoldArgs& a, int M, hipStream_t s) {
  const int groups = (a.N + 63) / 64;
  switch (M) {
    case 1: hipLaunchKernelGGL(scaffold_kernel<1>, dim3(groups), dim3(kNT), 0, s, a); break;
    case 2: hipLaunchKernelGGL(scaffold_kernel<2>, dim3(groups), dim3(kNT), 0, s, a); break;
    case 3: hipLaunchKernelGGL(scaffold_kernel<3>, dim3(groups), dim3(kNT), 0, s, a); break;
    case 4: hipLaunchKernelGGL(scaffold_kernel<4>, dim3(groups), dim3(kNT), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_prologue(const ProjArgs& a, int M, uint16_t* xn, int8_t* q, uint16_t* sc, hipStream_t s) {
  hipLaunchKernelGGL(prologue_kernel, dim3(M), dim3(kNT), 0, s, a, xn, q, sc);
  return hipGetLastError();
}

hipError_t launch_tile_bits(const uint32_t* src, uint32_t* dst, int N, int KW, hipStream_t s) {
  const int n_pad = (N + 63) / 64 * 64;
  const size_t total = (size_t)n_pad * KW;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(tile_bits_kernel, dim3(blocks), dim3(256), 0, s, src, dst, N, KW, n_pad);
  return hipGetLastError();
}

}  // namespace dfssm
