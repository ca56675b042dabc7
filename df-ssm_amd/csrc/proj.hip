// Scaffold projection kernels: 1-bit packed GEMV with fused prologue and epilogue (gfx950).
//
// One workgroup (1024 threads, 16 waves) owns one group of 64 output rows. Lane l of every wave
// owns row 64*g + l; wave w streams the 16-byte column chunks w, w+16, ... of those rows. The sign bits are stored
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

constexpr int kMaxK = 5120;          // largest d_model / d_inner supported

// Workgroup size: 1024 threads (16 waves) for one activation row, so the redundant prologue is
// spread over the whole CU; 512 for 2..4 rows, which need more registers per thread.
template <int M> struct ProjShape {
  static constexpr int NT = M == 1 ? 1024 : 512;
  static constexpr int NW = NT / 64;
  static constexpr int MaxCPW = (kMaxK / 128 + NW - 1) / NW;  // 16-byte bit chunks per lane
  static constexpr int MaxLB = 16 * kMaxK / NT / 8;            // 8-byte LoRA-B vectors per thread
  static constexpr int Slices = NT / 16;                        // LoRA-h column slices
};

template <int M>
struct ProjLds {
  uint32_t planes[M][kMaxK / 32][8];  // bit planes of q, per 32-column word
  uint16_t xn[M][kMaxK];              // normalized activations (fp16)
  double lora_part[M][DFSSM_LORA_R][ProjShape<M>::Slices];
  float hl[M][DFSSM_LORA_R];          // h16 values (as float)
  int T[ProjShape<M>::NW][M][64];     // per-wave partial sum_{bit=1} q
  double red_d[ProjShape<M>::NW][M];
  float red_f[ProjShape<M>::NW][M];
  int red_i[ProjShape<M>::NW][M];
  int S[M];
  float xs[M];
};

// Block reductions of M values at once (one pair of barriers for all rows).
template <int M, int kNW>
__device__ __forceinline__ void block_sum_f64_m(double (&v)[M], double (&red)[kNW][M]) {
#pragma unroll
  for (int m = 0; m < M; ++m) v[m] = wave_sum_f64(v[m]);
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int m = 0; m < M; ++m) red[threadIdx.x >> 6][m] = v[m];
  __syncthreads();
#pragma unroll
  for (int m = 0; m < M; ++m) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kNW; ++w) t += red[w][m];
    v[m] = t;
  }
}
template <int M, int kNW>
__device__ __forceinline__ void block_max_f32_m(float (&v)[M], float (&red)[kNW][M]) {
#pragma unroll
  for (int m = 0; m < M; ++m) v[m] = wave_max_f32(v[m]);
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int m = 0; m < M; ++m) red[threadIdx.x >> 6][m] = v[m];
  __syncthreads();
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float t = red[0][m];
#pragma unroll
    for (int w = 1; w < kNW; ++w) t = fmaxf(t, red[w][m]);
    v[m] = t;
  }
}
template <int M, int kNW>
__device__ __forceinline__ void block_sum_i32_m(int (&v)[M], int (&red)[kNW][M]) {
#pragma unroll
  for (int m = 0; m < M; ++m) v[m] = wave_sum_i32(v[m]);
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int m = 0; m < M; ++m) red[threadIdx.x >> 6][m] = v[m];
  __syncthreads();
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < kNW; ++w) t += red[w][m];
    v[m] = t;
  }
}

// Prologue for all M activation rows. av[m] is the 16-byte vector `tid` of row m (K <= 8 * kNT),
// lb the thread's LoRA-B slice (row tid % 16, columns (tid / 16) * K / 64 ..). Builds xn (LDS), the
// scales, the bit planes, sum q, and h16.
template <int M, int MODE>
__device__ __forceinline__ void proj_prologue(const ProjArgs& a, const u32x4 (&av)[M], const double (&slot_part)[M],
                                              const uint2 (&lb)[ProjShape<M>::MaxLB], ProjLds<M>& L) {
  constexpr int kNT = ProjShape<M>::NT, kNW = ProjShape<M>::NW, kMaxLB = ProjShape<M>::MaxLB;
  const int K = a.K, tid = threadIdx.x, lane = tid & 63;
  const bool has_v = tid < K / 8;
  // 1) sum of squares -> r (MODE_OUT: the SSM kernel's per-block partials)
  double ss[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (MODE == DFSSM_MODE_IN) {
      double part = 0.0;
      if (has_v) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const double xv = (double)h2f((uint16_t)(av[m][e >> 1] >> (16 * (e & 1))));
          part += xv * xv;
        }
      }
      ss[m] = part;
    } else {
      ss[m] = slot_part[m];
    }
  }
  block_sum_f64_m<M, kNW>(ss, L.red_d);
  // 2) xn = fp16((x * r) * w) into LDS, amax
  float amax[M];
  f32x4 w0 = {0.f, 0.f, 0.f, 0.f}, w1 = {0.f, 0.f, 0.f, 0.f};
  if (has_v) {
    w0 = *(const f32x4*)(a.norm_w + 8 * tid);
    w1 = *(const f32x4*)(a.norm_w + 8 * tid + 4);
  }
  const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float var = (float)ss[m] * (1.0f / (float)K);
    const float r = 1.0f / sqrt_rn(var + 1e-5f);
    float mx = 0.0f;
    if (has_v) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = r16((h2f((uint16_t)(av[m][e >> 1])) * r) * wv[e]);
        const float x1 = r16((h2f((uint16_t)(av[m][e >> 1] >> 16)) * r) * wv[e + 1]);
        mx = fmaxf(mx, fmaxf(fabsf(x0), fabsf(x1)));
        o[e >> 1] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
      }
      *(u32x4*)&L.xn[m][8 * tid] = u32x4{o[0], o[1], o[2], o[3]};
    }
    amax[m] = mx;
  }
  block_max_f32_m<M, kNW>(amax, L.red_f);  // also publishes xn to the block
  // 3) q, planes (ballot over 64 consecutive columns; lanes 0..15 collect the 16 words), sum q
  int qsum[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float xs = quant_scale(amax[m]);
    int acc = 0;
    for (int k0 = (tid & ~63); k0 < K; k0 += kNT) {
      const int q = quant_i8(h2f(L.xn[m][k0 + lane]), xs);
      acc += q;
      const uint32_t qb = (uint32_t)q & 0xffu;
      uint32_t pw = 0u;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint64_t mask = __ballot((qb >> b) & 1u);
        pw = lane == b ? (uint32_t)mask : pw;
        pw = lane == 8 + b ? (uint32_t)(mask >> 32) : pw;
      }
      if (lane < 16) L.planes[m][k0 / 32 + (lane >> 3)][lane & 7] = pw;
    }
    qsum[m] = acc;
    if (tid == 0) L.xs[m] = xs;
  }
  block_sum_i32_m<M, kNW>(qsum, L.red_i);
  // 4) LoRA intermediate h16[m][r] = fp16(sum_k xn_k * fp16(B_i8[r,k] * B_s[r])):
  //    thread (r = tid % 16, slice = tid / 16) covers K/64 columns from registers.
  if (a.lB) {
    const int rr = tid & 15, slice = tid >> 4, per = K / (kNT / 16), nlb = per / 8;
    const float bs = h2f(a.lBs[rr]);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      double acc[2] = {0.0, 0.0};
      const uint16_t* xr = &L.xn[m][slice * per];
#pragma unroll
      for (int i = 0; i < kMaxLB; ++i) {
        if (i < nlb) {
          const uint2 bv = lb[i];
          const u32x4 x8 = *(const u32x4*)(xr + 8 * i);
          const uint32_t bw[2] = {bv.x, bv.y};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float b16 = r16((float)(int8_t)(bw[e >> 2] >> (8 * (e & 3))) * bs);
            const float xv = h2f((uint16_t)(x8[e >> 1] >> (16 * (e & 1))));
            acc[e & 1] += (double)(xv * b16);   // fp16 x fp16 is exact in fp32
          }
        }
      }
      L.lora_part[m][rr][slice] = acc[0] + acc[1];
    }
    __syncthreads();
    if (tid < M * DFSSM_LORA_R) {
      const int m = tid >> 4, r = tid & 15;
      double t = 0.0;
#pragma unroll 8
      for (int s = 0; s < kNT / 16; ++s) t += L.lora_part[m][r][s];
      L.hl[m][r] = r16((float)t);
    }
  }
  if (tid < M) L.S[tid] = qsum[tid];
  __syncthreads();
}

template <int M, int MODE>
__global__ __launch_bounds__(ProjShape<M>::NT) void proj_kernel(ProjArgs a) {
  constexpr int kNT = ProjShape<M>::NT, kNW = ProjShape<M>::NW;
  constexpr int kMaxCPW = ProjShape<M>::MaxCPW, kMaxLB = ProjShape<M>::MaxLB;
  __shared__ ProjLds<M> L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  const int K = a.K, CH = K / 128;

  // ---- every load that does not depend on another workgroup's output, issued first ----
  u32x4 av[M];
#pragma unroll
  for (int m = 0; m < M; ++m)
    av[m] = tid < K / 8 ? *(const u32x4*)(a.act + (size_t)m * a.ld_act + 8 * tid) : u32x4{0u, 0u, 0u, 0u};
  double slot_part[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    double p = 0.0;
    if (MODE == DFSSM_MODE_OUT)
      for (int j = tid; j < a.n_slots; j += kNT) p += a.sumsq_slots[(size_t)m * a.n_slots + j];
    slot_part[m] = p;
  }
  // epilogue row data: thread (m = tid / 64, row n = 64 g + lane)
  const int n = g * 64 + lane;
  const bool erow = tid < M * 64 && n < a.N;
  const int em = tid >> 6;
  u32x4 la = {0u, 0u, 0u, 0u};
  float e_ws = 0.0f, e_as = 0.0f;
  uint16_t cs0 = 0, cs1 = 0, cs2 = 0, cb = 0, xres = 0;
  uint32_t cw01 = 0, cw23 = 0;
  const int ch = n - a.conv_lo;
  const bool conv_row = MODE == DFSSM_MODE_IN && erow && ch >= 0 && ch < a.conv_c;
  if (erow) {
    la = *(const u32x4*)(a.lA + (size_t)n * DFSSM_LORA_R);
    e_ws = h2f(a.wscale[n]);
    e_as = h2f(a.lAs[n]);
    if (conv_row) {
      const uint16_t* cs = a.conv_state + ((size_t)em * a.conv_c + ch) * 3;
      cs0 = cs[0]; cs1 = cs[1]; cs2 = cs[2];
      const uint32_t* wc = (const uint32_t*)(a.conv_w + (size_t)ch * 4);
      cw01 = wc[0]; cw23 = wc[1];
      cb = a.conv_b[ch];
    }
    if (MODE == DFSSM_MODE_OUT) xres = a.out[(size_t)em * a.ld_out + n];
  }
  // LoRA-B slice of this thread
  uint2 lb[kMaxLB];
  {
    const int rr = tid & 15, slice = tid >> 4, per = K / (kNT / 16), nlb = per / 8;
    const int8_t* src = a.lB ? a.lB + (size_t)rr * K + slice * per : nullptr;
#pragma unroll
    for (int i = 0; i < kMaxLB; ++i) lb[i] = (src && i < nlb) ? *(const uint2*)(src + 8 * i) : make_uint2(0u, 0u);
  }
  // this lane's sign-bit chunks: wave w takes chunks w, w + 16, ... of the row group
  const u32x4* bits = (const u32x4*)a.bits + (size_t)g * CH * 64 + lane;
  u32x4 wb[kMaxCPW];
#pragma unroll
  for (int j = 0; j < kMaxCPW; ++j) {
    const int c = wave + kNW * j;
    wb[j] = c < CH ? ld_nt(bits + (size_t)c * 64) : u32x4{0u, 0u, 0u, 0u};
  }

  proj_prologue<M, MODE>(a, av, slot_part, lb, L);

  uint32_t cnt[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int b = 0; b < 8; ++b) cnt[m][b] = 0;
#pragma unroll
  for (int j = 0; j < kMaxCPW; ++j) {
    const int c = wave + kNW * j;
    if (c < CH) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = wb[j][i];
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const u32x4 p0 = *(const u32x4*)&L.planes[m][c * 4 + i][0];
          const u32x4 p1 = *(const u32x4*)&L.planes[m][c * 4 + i][4];
          cnt[m][0] += __builtin_popcount(w & p0[0]);
          cnt[m][1] += __builtin_popcount(w & p0[1]);
          cnt[m][2] += __builtin_popcount(w & p0[2]);
          cnt[m][3] += __builtin_popcount(w & p0[3]);
          cnt[m][4] += __builtin_popcount(w & p1[0]);
          cnt[m][5] += __builtin_popcount(w & p1[1]);
          cnt[m][6] += __builtin_popcount(w & p1[2]);
          cnt[m][7] += __builtin_popcount(w & p1[3]);
        }
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

  // ---- epilogue: thread (m = tid / 64, row n) ----
  if (erow) {
    const int m = em;
    int T = 0;
#pragma unroll
    for (int w = 0; w < kNW; ++w) T += L.T[w][m][lane];
    const int acc = 2 * T - L.S[m];
    if (a.acc_out) a.acc_out[(size_t)m * a.N + n] = acc;
    const float y = r16(r16(r16((float)acc) * L.xs[m]) * e_ws);
    double lo = 0.0;
#pragma unroll
    for (int rr = 0; rr < DFSSM_LORA_R; ++rr) {
      const float aq = r16((float)(int8_t)(la[rr >> 2] >> (8 * (rr & 3))) * e_as);
      lo += (double)L.hl[m][rr] * (double)aq;
    }
    float out = r16((float)lo + y);
    if (MODE == DFSSM_MODE_IN) {
      if (conv_row) {
        // depthwise conv (k=4) + SiLU on xBC channel ch; state (M, C, 3) fp16 shifts left
        uint16_t* cs = a.conv_state + ((size_t)m * a.conv_c + ch) * 3;
        const uint16_t xo = f2h(out);
        cs[0] = cs1;
        cs[1] = cs2;
        cs[2] = xo;
        const float xv = h2f(xo);
        float o = h2f(cs0) * h2f((uint16_t)cw01);
        o = o + h2f(cs1) * h2f((uint16_t)(cw01 >> 16));
        o = o + h2f(cs2) * h2f((uint16_t)cw23);
        o = o + xv * h2f((uint16_t)(cw23 >> 16));
        o = o + h2f(cb);
        const float sig = 1.0f / (1.0f + dev_expf(-o));
        out = o * sig;
      }
      a.out[(size_t)m * a.ld_out + n] = f2h(out);
    } else {
      a.out[(size_t)m * a.ld_out + n] = f2h(h2f(xres) + out);
    }
  }
}

// Stand-alone RMSNorm + quantizer (one workgroup per activation row): writes xn, q and the scale.
__global__ __launch_bounds__(ProjShape<1>::NT) void prologue_kernel(ProjArgs a, uint16_t* xn_out, int8_t* q_out, uint16_t* s_out) {
  constexpr int kNT = ProjShape<1>::NT, kMaxLB = ProjShape<1>::MaxLB;
  __shared__ ProjLds<1> L;
  const int m = blockIdx.x, tid = threadIdx.x;
  ProjArgs b = a;
  b.act = a.act + (size_t)m * a.ld_act;
  b.lB = nullptr;
  u32x4 av[1];
  av[0] = tid < a.K / 8 ? *(const u32x4*)(b.act + 8 * tid) : u32x4{0u, 0u, 0u, 0u};
  const double slot_part[1] = {0.0};
  uint2 lb[kMaxLB];
#pragma unroll
  for (int i = 0; i < kMaxLB; ++i) lb[i] = make_uint2(0u, 0u);
  proj_prologue<1, DFSSM_MODE_IN>(b, av, slot_part, lb, L);
  const float xs = L.xs[0];
  for (int k = tid; k < a.K; k += kNT) {
    const uint16_t v = L.xn[0][k];
    xn_out[(size_t)m * a.K + k] = v;
    q_out[(size_t)m * a.K + k] = (int8_t)quant_i8(h2f(v), xs);
  }
  if (tid == 0) s_out[m] = f2h(xs);
}

// Stand-alone scaffold GEMM for given int8 activations (tests / microbench): acc and y only.
constexpr int kNTs = 256;  // scaffold_kernel: 4 waves, each a quarter of K

template <int M>
__global__ __launch_bounds__(kNTs) void scaffold_kernel(ScaffoldArgs a) {
  __shared__ uint32_t planes[M][kMaxK / 32][8];
  __shared__ int T[4][M][64];
  __shared__ int S[M];
  __shared__ int red_i[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  const int K = a.K, KW = K / 32, CH = KW / 4, CPW = CH / 4;
  const uint4* bits = (const uint4*)a.bits + ((size_t)g * CH + wave * CPW) * 64 + lane;
  for (int m = 0; m < M; ++m) {
    int qsum = 0;
    for (int k0 = (tid & ~63); k0 < K; k0 += kNTs) {
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
    const int s = block_sum_i32<kNTs>(qsum, red_i);
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
    hipLaunchKernelGGL((proj_kernel<M, DFSSM_MODE_IN>), dim3(groups), dim3(ProjShape<M>::NT), 0, s, a);
  else
    hipLaunchKernelGGL((proj_kernel<M, DFSSM_MODE_OUT>), dim3(groups), dim3(ProjShape<M>::NT), 0, s, a);
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
    case 1: hipLaunchKernelGGL(scaffold_kernel<1>, dim3(groups), dim3(kNTs), 0, s, a); break;
    case 2: hipLaunchKernelGGL(scaffold_kernel<2>, dim3(groups), dim3(kNTs), 0, s, a); break;
    case 3: hipLaunchKernelGGL(scaffold_kernel<3>, dim3(groups), dim3(kNTs), 0, s, a); break;
    case 4: hipLaunchKernelGGL(scaffold_kernel<4>, dim3(groups), dim3(kNTs), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_prologue(const ProjArgs& a, int M, uint16_t* xn, int8_t* q, uint16_t* sc, hipStream_t s) {
  hipLaunchKernelGGL(prologue_kernel, dim3(M), dim3(ProjShape<1>::NT), 0, s, a, xn, q, sc);
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
