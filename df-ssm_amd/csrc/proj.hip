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
// The prologue of a projection (RMSNorm, int8 quantizer, bit planes, sum q, rank-16 LoRA
// intermediate) runs once per sequence in prep_kernel; the GEMV kernels read its results.
// Epilogue per row n: y = fp16(fp16(fp16(acc) * s_x) * s_w[n]) (:158), out = fp16(y + h16.A16[n])
// (:173,204); MODE_IN additionally applies the depthwise conv + SiLU to the xBC rows
// (df_ssm_kernels.cu:27-47) and writes z | xBC | dt_raw; MODE_OUT adds the residual (:207).
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kMaxK = 5120;          // largest d_model / d_inner supported

// ------------------------------------------------------------------------------------------
// prep_kernel: the per-projection prologue, computed once per sequence (16 workgroups of K/8
// threads per activation row m):
//   MODE_IN : xn = fp16((x * r) * ln_w), r = 1/sqrt(sum(x^2)/K + 1e-5)  (df_ssm_inference.py:141-145)
//   MODE_OUT: the same on the gated g with sum(g^2) from the SSM kernel's per-block partials
//   s = fp16(fp16(max(amax, 1e-4)) / 127), q = clamp(rne(fp16(xn / s)))     (:147-152)
//   planes[m][word][b] = bit b of q for the 32 columns of `word`; S = sum q
//   h[m][r] = fp16(sum_k xn_k * fp16(B_i8[r,k] * B_s[r]))                   (:83,173,204)
// ------------------------------------------------------------------------------------------
constexpr int kPT = 1024;       // threads per workgroup at most (K / 8 for K <= 5120)
constexpr int kPW = kPT / 64;

struct PrepLds {
  uint16_t xn[kMaxK];
  double red_d[kPW];
  double red_h[2][kPW];  // per-wave LoRA sums of the workgroup's ranks
  float red_f[kPW];
  int red_i[kPW];
};

// 16 M / R workgroups (more when M is not a multiple of 8) x K/8 threads (8 columns each; K is a
// multiple of 512, so whole waves): workgroup (r, m) recomputes the normalization and quantization
// of row m, writes the q bytes (and for the bit-plane GEMV the planes) of column slice r (R K/16
// columns) and the LoRA intermediates h[m][R r .. R r + R - 1]; workgroup (0, m) also writes sum q
// (when asked) and the scale. R = 1, or 2 when 16 workgroups per row would not all be resident at
// once. Three LDS reductions: the sum of squares, then the LoRA sums and the maximum together,
// then (workgroup 0, when asked) sum q.
template <int MODE, int R>
__global__ __launch_bounds__(kPT) void prep_kernel(PrepArgs a, int M) {
  __shared__ PrepLds L;
  constexpr int NR = DFSSM_LORA_R / R;  // workgroups per row
  // workgroup -> (rank group, row m): workgroups are dealt to the 8 XCDs in turn, and XCD x takes
  // the rows m = x (mod 8) with all rank groups of each, so a row (read by all of its
  // workgroups) is fetched into one XCD's L2 rather than into all eight
  const int x8 = (int)blockIdx.x & 7, j8 = (int)blockIdx.x >> 3;
  const int m = 8 * (j8 / NR) + x8, rg = j8 % NR, rr = R * rg;
  if (m >= M) return;  // uniform over the workgroup
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int K = a.K, NT = (int)blockDim.x, nw = NT >> 6;
  const uint16_t* act = a.act + (size_t)m * a.ld_act;
  // Loads first, in the order they are needed (loads complete in issue order, so waiting for one
  // waits for all issued before it): the sum-of-squares partials (MODE_OUT, n_slots < K / 8), the
  // activation vector, norm weights, LoRA-B row r and its scale (from a valid stand-in address
  // when there is no LoRA). Raw values are converted where used.
  double slot = 0.0;
  if (MODE == DFSSM_MODE_OUT) slot = a.sumsq_slots[(size_t)m * a.n_slots + (tid < a.n_slots ? tid : a.n_slots - 1)];
  const u32x4 av = *(const u32x4*)(act + 8 * tid);
  const f32x4 w0 = *(const f32x4*)(a.norm_w + 8 * tid);
  const f32x4 w1 = *(const f32x4*)(a.norm_w + 8 * tid + 4);
  uint2 b8[R];
  uint16_t bs_raw[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    b8[q] = *(const uint2*)((a.lB ? a.lB + (size_t)(rr + q) * K : (const int8_t*)act) + 8 * tid);
    bs_raw[q] = *(a.lB ? a.lBs + rr + q : act);
  }
  double part = 0.0;
  if (MODE == DFSSM_MODE_IN) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const double xv = (double)h2f((uint16_t)(av[e >> 1] >> (16 * (e & 1))));
      part += xv * xv;
    }
  } else {
    part = tid < a.n_slots ? slot : 0.0;
  }
  {  // sum of squares (fp64: the sums are exact)
    const double pw = wave_sum_dpp_f64(part);
    if (lane == 0) L.red_d[w] = pw;
  }
  lds_barrier();
  double ss = 0.0;
  for (int i = 0; i < nw; ++i) ss += L.red_d[i];
  // xn into LDS, this thread's max |xn| and LoRA partial
  const float var = (float)ss * (1.0f / (float)K);
  const float r = 1.0f / sqrt_rn(var + 1e-5f);
  const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
  float mx = 0.0f;
  double hacc[R];
  uint32_t o[4];
  {
#pragma unroll
    for (int q = 0; q < R; ++q) hacc[q] = 0.0;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float x0 = r16((h2f((uint16_t)(av[e >> 1])) * r) * wv[e]);
      const float x1 = r16((h2f((uint16_t)(av[e >> 1] >> 16)) * r) * wv[e + 1]);
      mx = fmaxf(mx, fmaxf(fabsf(x0), fabsf(x1)));
      o[e >> 1] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
      // LoRA intermediates of ranks rr .. rr + R - 1 over this thread's 8 columns (fp16 x fp16 is
      // exact in fp32)
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const float bs = a.lB ? h2f(bs_raw[q]) : 0.0f;
        const uint32_t bw[2] = {b8[q].x, b8[q].y};
        const float b0 = r16((float)(int8_t)(bw[e >> 2] >> (8 * (e & 3))) * bs);
        const float b1 = r16((float)(int8_t)(bw[(e + 1) >> 2] >> (8 * ((e + 1) & 3))) * bs);
        hacc[q] += (double)(x0 * b0);
        hacc[q] += (double)(x1 * b1);
      }
    }
    *(u32x4*)&L.xn[8 * tid] = u32x4{o[0], o[1], o[2], o[3]};
  }
  {  // LoRA sums and maximum in one exchange (the first barrier: every wave has read the squares)
    double hw[R];
#pragma unroll
    for (int q = 0; q < R; ++q) hw[q] = wave_sum_dpp_f64(hacc[q]);
    const float mw = wave_max_dpp_f32(mx);
    lds_barrier();
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < R; ++q) L.red_h[q][w] = hw[q];
      L.red_f[w] = mw;
    }
  }
  lds_barrier();  // also publishes xn
  double ht[R];
#pragma unroll
  for (int q = 0; q < R; ++q) ht[q] = 0.0;
  float amax = L.red_f[0];
  for (int i = 0; i < nw; ++i) {
#pragma unroll
    for (int q = 0; q < R; ++q) ht[q] += L.red_h[q][i];
    amax = fmaxf(amax, L.red_f[i]);
  }
  const float xs = quant_scale(amax);
  const float rinv = quant_rcp(xs);
  // q over all columns when sum q is wanted, else only where written: the bytes and bit planes
  // of the 64-column wave blocks that start in slice rr (slices narrower than 64 columns, K < 1024,
  // leave every other workgroup nothing to write). Global stores come last: a wave with a store
  // outstanding waits for its acknowledgement wherever a later load must be complete.
  const int lo = rr * (K / 16), hi = lo + R * (K / 16);
  const bool want_sum = a.s_out != nullptr;
  int qsum = 0;
  for (int k0 = 64 * w; k0 < K; k0 += NT) {
    const bool mine = k0 >= lo && k0 < hi;  // wave-uniform
    if (!want_sum && !mine) continue;
    const int q = quant_i8(h2f(L.xn[k0 + lane]), rinv);
    qsum += q;
    if (mine) {
      if (a.q_out) a.q_out[(size_t)m * a.ld_q + k0 + lane] = (int8_t)q;
      if (a.planes_out) {
        uint32_t pw[16];
        planes64(q, pw);
        planes_store(a.planes_out + ((size_t)m * (a.ld_q / 32) + k0 / 32) * 8, pw);
      }
    }
  }
  if (a.xn_out && rr == 0) *(u32x4*)(a.xn_out + (size_t)m * K + 8 * tid) = u32x4{o[0], o[1], o[2], o[3]};
  if (a.lB && tid == 0) {
#pragma unroll
    for (int q = 0; q < R; ++q) a.h_out[(size_t)m * DFSSM_LORA_R + rr + q] = r16((float)ht[q]);
  }
  if (rr == 0) {
    int S = 0;
    if (want_sum) {
      const int qw = wave_sum_dpp_i32(qsum);
      lds_barrier();  // every wave has read the LoRA sums
      if (lane == 0) L.red_i[w] = qw;
      lds_barrier();
      for (int i = 0; i < nw; ++i) S += L.red_i[i];
    }
    if (tid == 0) {
      if (a.s_out) a.s_out[m] = S;
      if (a.xs_out) a.xs_out[m] = xs;
      if (a.xs16_out) a.xs16_out[m] = f2h(xs);
    }
  }
}

// prep_rows_kernel: the same prologue for many rows (the prompt prefill runs thousands), one
// workgroup of K/8 threads per kPrepRows consecutive rows. The norm weights and the fp16 LoRA-B
// values of a thread's 8 columns (16 ranks) stay in registers across the rows, and each row's
// RMSNorm, quantizer and 16 LoRA intermediates are computed once (prep_kernel's 16 workgroups per
// row each recompute the norm). The thread -> column map, the per-thread order of the fp64 sums
// and the reduction trees are prep_kernel's, so every output is identical. Writes q_out (row-major
// or, with q_tiled, in the wide GEMM's tiled layout), xs_out, h_out and s_out; the decode-only
// outputs (planes_out, xn_out, xs16_out) are not supported.
constexpr int kPrepRows = 16;
constexpr int kPrepRowsT = kMaxK / 8;  // threads per workgroup at most

template <int MODE>
__global__ __launch_bounds__(kPrepRowsT) void prep_rows_kernel(PrepArgs a, int M) {
  __shared__ double red_d[kPrepRowsT / 64];
  __shared__ double red_h[kPrepRowsT / 64][DFSSM_LORA_R];
  __shared__ float red_f[kPrepRowsT / 64];
  __shared__ int red_i[kPrepRowsT / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int K = a.K, nw = (int)blockDim.x >> 6;
  const int m0 = (int)blockIdx.x * kPrepRows, m1 = m0 + kPrepRows < M ? m0 + kPrepRows : M;
  const bool want_sum = a.s_out != nullptr;
  // this row's activations (and its sum-of-squares slot) are loaded one row ahead
  auto load_row = [&](int m, u32x4& av, double& slot) {
    const int mm = m < m1 ? m : m1 - 1;
    av = *(const u32x4*)(a.act + (size_t)mm * a.ld_act + 8 * tid);
    if (MODE == DFSSM_MODE_OUT) slot = a.sumsq_slots[(size_t)mm * a.n_slots + (tid < a.n_slots ? tid : a.n_slots - 1)];
  };
  u32x4 av;
  double slot = 0.0;
  load_row(m0, av, slot);
  const f32x4 w0 = *(const f32x4*)(a.norm_w + 8 * tid);
  const f32x4 w1 = *(const f32x4*)(a.norm_w + 8 * tid + 4);
  const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
  // fp16(B_i8 * B_s) of the 8 columns for every rank, as fp16 pairs (prep_kernel's b0, b1)
  uint32_t bp[DFSSM_LORA_R][4];
#pragma unroll
  for (int rr = 0; rr < DFSSM_LORA_R; ++rr) {
    uint2 b8 = {0u, 0u};
    float bs = 0.0f;
    if (a.lB) {
      b8 = *(const uint2*)(a.lB + (size_t)rr * K + 8 * tid);
      bs = h2f(a.lBs[rr]);
    }
    const uint32_t bw[2] = {b8.x, b8.y};
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float b0 = r16((float)(int8_t)(bw[e >> 2] >> (8 * (e & 3))) * bs);
      const float b1 = r16((float)(int8_t)(bw[(e + 1) >> 2] >> (8 * ((e + 1) & 3))) * bs);
      bp[rr][e >> 1] = (uint32_t)f2h(b0) | ((uint32_t)f2h(b1) << 16);
    }
  }
  for (int m = m0; m < m1; ++m) {
    // opaque per row: keeps the 128 conversions of bp to fp32 inside the loop (hoisted, they
    // would not fit the registers)
#pragma unroll
    for (int rr = 0; rr < DFSSM_LORA_R; ++rr)
#pragma unroll
      for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(bp[rr][j]));
    const u32x4 cur = av;
    const double cslot = slot;
    if (m + 1 < m1) load_row(m + 1, av, slot);
    double part = 0.0;
    if (MODE == DFSSM_MODE_IN) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double xv = (double)h2f((uint16_t)(cur[e >> 1] >> (16 * (e & 1))));
        part += xv * xv;
      }
    } else {
      part = tid < a.n_slots ? cslot : 0.0;
    }
    {
      const double pw = wave_sum_dpp_f64(part);
      if (lane == 0) red_d[w] = pw;
    }
    lds_barrier();
    double ss = 0.0;
    for (int i = 0; i < nw; ++i) ss += red_d[i];
    const float var = (float)ss * (1.0f / (float)K);
    const float r = 1.0f / sqrt_rn(var + 1e-5f);
    float xn[8];
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      xn[e] = r16((h2f((uint16_t)(cur[e >> 1])) * r) * wv[e]);
      xn[e + 1] = r16((h2f((uint16_t)(cur[e >> 1] >> 16)) * r) * wv[e + 1]);
      mx = fmaxf(mx, fmaxf(fabsf(xn[e]), fabsf(xn[e + 1])));
    }
    {
      const float mw = wave_max_dpp_f32(mx);
      if (lane == 0) red_f[w] = mw;
    }
#pragma unroll
    for (int rr = 0; rr < DFSSM_LORA_R; ++rr) {  // one rank at a time: columns in order, as prep_kernel
      double hacc = 0.0;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {  // fp16 x fp16 is exact in fp32
        hacc += (double)(xn[e] * h2f((uint16_t)bp[rr][e >> 1]));
        hacc += (double)(xn[e + 1] * h2f((uint16_t)(bp[rr][e >> 1] >> 16)));
      }
      const double hw = wave_sum_dpp_f64(hacc);
      if (lane == 0) red_h[w][rr] = hw;
    }
    lds_barrier();  // (every wave has also read red_d: the next row may rewrite it)
    float amax = red_f[0];
    for (int i = 0; i < nw; ++i) amax = fmaxf(amax, red_f[i]);
    if (a.lB && tid < DFSSM_LORA_R) {
      double ht = 0.0;
      for (int i = 0; i < nw; ++i) ht += red_h[i][tid];
      a.h_out[(size_t)m * DFSSM_LORA_R + tid] = r16((float)ht);
    }
    const float xs = quant_scale(amax);
    const float rinv = quant_rcp(xs);
    uint32_t qw[2] = {0u, 0u};
    int qsum = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int q = quant_i8(xn[e], rinv);
      qsum += q;
      qw[e >> 2] |= (uint32_t)(q & 0xff) << (8 * (e & 3));
    }
    if (a.q_out) {
      int8_t* qp = a.q_tiled ? a.q_out + wide_tiled_offset(m, 8 * tid, K) : a.q_out + (size_t)m * a.ld_q + 8 * tid;
      *(uint2*)qp = uint2{qw[0], qw[1]};
    }
    int S = 0;
    if (want_sum) {  // uniform
      const int qs = wave_sum_dpp_i32(qsum);
      if (lane == 0) red_i[w] = qs;
      lds_barrier();
      for (int i = 0; i < nw; ++i) S += red_i[i];
    }
    if (tid == 0) {
      if (a.s_out) a.s_out[m] = S;
      if (a.xs_out) a.xs_out[m] = xs;
    }
    // red_f and red_h are rewritten only after the next row's first barrier, red_i after its
    // second: every wave has read them by then
  }
}

// ------------------------------------------------------------------------------------------
// proj_kernel: 1-bit scaffold GEMV for M <= 4 activation rows + fused epilogue.
// One workgroup (1024 threads, 16 waves) owns 64 output rows; lane l of every wave owns row
// 64 g + l and wave w streams the 16-byte column chunks w, w + 16, ... of those rows. The bit
// planes, sum q, scale and LoRA intermediate come from prep_kernel.
// ------------------------------------------------------------------------------------------
constexpr int kNT = 1024;
constexpr int kNW = kNT / 64;
constexpr int kMaxCPW = (kMaxK / 128 + kNW - 1) / kNW;
constexpr uint32_t kScafSpinMax = 1u << 18;  // polls of the intermediates before giving up

template <int M>
struct ProjLds {
  uint32_t planes[M][kMaxK / 32][8];
  int T[kNW][M][64];
  float hl[M][DFSSM_LORA_R];
  int S[M];
  float xs[M];
};

template <int M, int MODE>
__global__ __launch_bounds__(kNT) void proj_kernel(ProjArgs a) {
  __shared__ ProjLds<M> L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  const int K = a.K, CH = K / 128, KW = K / 32;

  // ---- loads: this lane's sign-bit chunks (independent of the activations) first ----
  const u32x4* bits = (const u32x4*)a.bits + (size_t)g * CH * 64 + lane;
  u32x4 wb[kMaxCPW];
#pragma unroll
  for (int j = 0; j < kMaxCPW; ++j) {
    const int c = wave + kNW * j;
    wb[j] = c < CH ? ld_nt(bits + (size_t)c * 64) : u32x4{0u, 0u, 0u, 0u};
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
  // prep results: planes (M * K bytes), scale, sum q, LoRA intermediate
  const int pv = M * KW * 8 / 4;  // 16-byte vectors of planes
  for (int i = tid; i < pv; i += kNT) {
    const int m = i / (KW * 2), r = i % (KW * 2);
    *((u32x4*)&L.planes[m][0][0] + r) = *((const u32x4*)(a.planes + (size_t)m * (a.ld_q / 32) * 8) + r);
  }
  if (tid < M * DFSSM_LORA_R) L.hl[tid >> 4][tid & 15] = a.h[(size_t)(tid >> 4) * DFSSM_LORA_R + (tid & 15)];
  if (tid < M) {
    L.S[tid] = a.qsum[tid];
    L.xs[tid] = a.xs[tid];
  }
  __syncthreads();

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

// Stand-alone scaffold op on many output rows (N >= 4096) at M <= 4 (dfssm_scaffold_gemm), and
// with LoRA at M = 1 in one launch (dfssm_scaffold_lora_gemm): proj_kernel's GEMV for given int8
// activations. (With fewer output rows, N / 64 workgroups leave most CUs idle and with LoRA at
// M >= 2 the intermediates cost M x 16 K fp64 products per workgroup: the GEMM path is faster.) One
// workgroup (1024 threads) owns 64 output rows. The small operands are loaded first (q bytes,
// the LoRA inputs), then the sign-bit chunks, so that building the bit planes and sum q (every
// workgroup for itself: M K values, two ballots' worth per thread) and the LoRA intermediates
// overlaps the bit stream. LoRA: wave r computes h[m][r] = fp16(sum_k xn[m][k] lBq[r][k]), each
// lane summing its K / 64 columns in fp64, then one wave sum per row; the fp16 x fp16 products
// are exact in fp32, so this is lora_h_kernel's sum in another order (fp64 sums of exact products:
// the same value while they stay exact, the assumption the one-launch layer's LoRA split makes
// too). Workgroup 0 writes the intermediates out.
template <int M, bool LORA, int KB>
__global__ __launch_bounds__(kNT) void scaffold_fused_kernel(ScaffoldArgs a) {
  constexpr int K = 512 * KB, CH = K / 128, NB = K / 64;
  constexpr int CPW = (CH + kNW - 1) / kNW;  // sign-bit chunks per wave
  constexpr int QB = (NB + kNW - 1) / kNW;   // 64-value q blocks per wave and row
  constexpr int XI = (K / 8 + kNT - 1) / kNT;  // xn vectors per thread and row
  __shared__ ProjLds<M> L;
  __shared__ __attribute__((aligned(16))) uint16_t xns[LORA ? M : 1][LORA ? K : 8];
  __shared__ int Sred[kNW][M];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  // ---- small operands first: q bytes of this wave's 64-value blocks, the xn rows (to LDS) and
  // this wave's LoRA-B row (rank = wave). Every load is unconditional: a load in a branch makes the
  // compiler wait for every outstanding load where the paths join. Indices past the operand (only
  // where K / 64 or K / 128 is not a multiple of the 16 waves) re-read its last block. ----
  int8_t qv[M][QB];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      const int b = wave + kNW * j;
      const int bc = (NB % kNW == 0 || b < NB) ? b : NB - 1;
      qv[m][j] = a.q[(size_t)m * K + 64 * bc + lane];
    }
  u32x4 bq[KB], xv8[LORA ? M : 1][XI];
  if (LORA) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int i = 0; i < XI; ++i) {
        const int c = tid + kNT * i;  // 8-column vector of row m (stored to LDS below)
        xv8[m][i] = *(const u32x4*)(a.xn + (size_t)m * K + 8 * (c < K / 8 ? c : K / 8 - 1));
      }
#pragma unroll
    for (int v = 0; v < KB; ++v)
      bq[v] = *(const u32x4*)(a.lBq + (size_t)wave * K + 512 * v + 8 * lane);
  }
  __builtin_amdgcn_sched_barrier(0);  // the small loads stay ahead of the bit stream
  // ---- the sign-bit chunks and the epilogue row data ----
  const u32x4* bits = (const u32x4*)a.bits + (size_t)g * CH * 64 + lane;
  u32x4 wb[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = wave + kNW * j;
    wb[j] = ld_nt(bits + (size_t)((CH % kNW == 0 || c < CH) ? c : CH - 1) * 64);
  }
  const int n = g * 64 + lane;
  const bool erow = tid < M * 64 && n < a.N;
  const int em = tid >> 6;
  const int nc = n < a.N ? n : a.N - 1, mc = em < M ? em : M - 1;
  // the scales are optional when y is not written: a valid stand-in address then (the sign bits
  // hold N K / 8 >= 2 N bytes, q M K >= 2 M bytes)
  const uint16_t* wsp = a.wscale ? a.wscale : (const uint16_t*)a.bits;
  const uint16_t* xsp = a.xscale ? a.xscale : (const uint16_t*)a.q;
  const uint16_t ws_raw = wsp[nc], xs_raw = xsp[mc];
  u32x4 la = {0u, 0u, 0u, 0u};
  uint16_t as_raw = 0;
  if (LORA) {
    la = *(const u32x4*)(a.lA + (size_t)nc * DFSSM_LORA_R);
    as_raw = a.lAs[nc];
  }
  __builtin_amdgcn_sched_barrier(0);
  if (LORA) {  // the xn rows to LDS (waits for the small loads only: they were issued first);
               // threads past the row rewrite its last vector with the same data
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int i = 0; i < XI; ++i) {
        const int c = tid + kNT * i;
        *(u32x4*)&xns[m][8 * (c < K / 8 ? c : K / 8 - 1)] = xv8[m][i];
      }
  }
  // ---- bit planes and sum q ----
  int qsum[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    qsum[m] = 0;
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      const int b = wave + kNW * j;
      if (b < NB) {  // wave-uniform
        const int q = qv[m][j];
        qsum[m] += q;
        uint32_t pw[16];
        planes64(q, pw);
        planes_store(&L.planes[m][2 * b][0], pw);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int s = wave_sum_dpp_i32(qsum[m]);
    if (lane == 0) Sred[wave][m] = s;
  }
  // ---- LoRA intermediates (wave r = rank r) ----
  if (LORA) {
    lds_barrier();  // xn in LDS (stored above)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;  // this lane's columns 512 v + 8 lane .. + 7, then one wave sum
#pragma unroll
      for (int v = 0; v < KB; ++v) {
        const u32x4 xv = *(const u32x4*)&xns[m][512 * v + 8 * lane];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = h2f((uint16_t)(xv[e >> 1] >> (16 * (e & 1))));
          const float b = h2f((uint16_t)(bq[v][e >> 1] >> (16 * (e & 1))));
          acc += (double)(x * b);
        }
      }
      const double t = wave_sum_dpp_f64(acc);
      if (lane == 0) {
        const uint16_t hb = f2h((float)t);
        L.hl[m][wave] = h2f(hb);
        if (g == 0) a.h_out[(size_t)m * DFSSM_LORA_R + wave] = hb;
      }
    }
  }
  lds_barrier();  // planes, sum q partials, intermediates
  if (tid < M) {
    int S = 0;
    for (int w = 0; w < kNW; ++w) S += Sred[w][tid];
    L.S[tid] = S;
  }
  // ---- GEMV (proj_kernel's) ----
  uint32_t cnt[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int b = 0; b < 8; ++b) cnt[m][b] = 0;
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
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
  lds_barrier();
  // ---- epilogue: thread (m = tid / 64, row n) ----
  if (erow) {
    const int m = em;
    int T = 0;
#pragma unroll
    for (int w = 0; w < kNW; ++w) T += L.T[w][m][lane];
    const int acc = 2 * T - L.S[m];
    if (a.acc_out) a.acc_out[(size_t)m * a.N + n] = acc;
    if (a.y_out) {
      const float y = r16(r16(r16((float)acc) * h2f(xs_raw)) * h2f(ws_raw));
      float out = y;
      if (LORA) {
        const float as = h2f(as_raw);
        double lo = 0.0;
#pragma unroll
        for (int rr = 0; rr < DFSSM_LORA_R; ++rr) {
          const float aq = r16((float)(int8_t)(la[rr >> 2] >> (8 * (rr & 3))) * as);
          lo += (double)L.hl[m][rr] * (double)aq;
        }
        out = r16((float)lo + y);
      }
      a.y_out[(size_t)m * a.N + n] = f2h(out);
    }
  }
}

// The stand-alone scaffold op with LoRA in one launch, the intermediates computed once: workgroups
// 0..15 are rank workgroups (h[m][r] for every row m, published as tagged words in kScafRep copies),
// workgroups 16.. run the GEMV of 64 output rows each and poll the 16 M words of their copy before
// the epilogue. A rank workgroup never waits and is dispatched before every GEMV workgroup, so every
// wait ends. Every launch has kScafGrid workgroups (those past the output rows only count the call),
// and each workgroup index keeps its own call count in the workspace: all counts are equal at a
// launch's start, so the count + 1 is the tag of the launch's words, known to every workgroup
// without any exchange.
__device__ __forceinline__ uint32_t scaf_tag(uint32_t c) { return (c + 1u) & 0xffffu; }

template <int M, int KB>
__global__ __launch_bounds__(kNT) void scaffold_xchg_kernel(ScaffoldArgs a) {
  constexpr int K = 512 * KB, CH = K / 128, NB = K / 64;
  constexpr int CPW = (CH + kNW - 1) / kNW;
  __shared__ int Tred[kNW][M][64];  // per-wave row partials of the GEMV
  __shared__ int Sred[kNW][M];      // per-wave sums of q
  __shared__ float hl[M][DFSSM_LORA_R];
  __shared__ double Rred[M][kNW];   // rank workgroups: per-wave partial sums
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // An offset the compiler cannot see is zero: the count's address then looks per-lane, so the
  // count stays in a vector register, waited for where it is used (a uniform load goes to a scalar
  // register at once, which waits for it before the data loads are issued).
  uint32_t zoff = 0u;
  asm volatile("" : "+v"(zoff));
  // every argument into registers at once: the compiler otherwise loads the argument block in
  // three dependent pieces around the branches below, a scalar-memory round trip each
  asm volatile("" ::"s"(a.bits), "s"(a.q), "s"(a.xscale), "s"(a.wscale), "s"(a.acc_out), "s"(a.y_out),
               "s"(a.lA), "s"(a.lAs), "s"(a.xn), "s"(a.lBq), "s"(a.h_out), "s"(a.ws), "s"(a.N));
  uint32_t* ws = a.ws;
  uint32_t* cnt = ws + blockIdx.x + zoff;
  if (blockIdx.x < DFSSM_LORA_R) {
    // ---- rank workgroup r: h[m][r] for all rows; thread t < K / 8 owns columns 8t..8t+7 ----
    const int r = blockIdx.x;
    const int c = tid < K / 8 ? tid : K / 8 - 1;  // waves past the row re-read its last vector
    const uint32_t e = ld_dev(cnt);  // first: the tagged stores wait for it
    u32x4 xv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) xv[m] = *(const u32x4*)(a.xn + (size_t)m * K + 8 * c);
    const u32x4 bv = *(const u32x4*)(a.lBq + (size_t)r * K + 8 * c);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;
      if (wave < KB) {  // uniform
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float x = h2f((uint16_t)(xv[m][k >> 1] >> (16 * (k & 1))));
          const float b = h2f((uint16_t)(bv[k >> 1] >> (16 * (k & 1))));
          acc += (double)(x * b);
        }
      }
      const double s = wave_sum_dpp_f64(acc);
      if (lane == 0) Rred[m][wave] = s;
    }
    lds_barrier();
    if (tid < kScafRep) {  // one copy per thread
#pragma unroll
      for (int m = 0; m < M; ++m) {
        double t = 0.0;
#pragma unroll
        for (int w = 0; w < kNW; ++w) t += Rred[m][w];
        const uint16_t hb = f2h((float)t);
        st_dev(ws + kScafWords + tid * kScafStride + m * DFSSM_LORA_R + r, (scaf_tag(e) << 16) | hb);
        if (tid == 0) a.h_out[(size_t)m * DFSSM_LORA_R + r] = hb;
      }
    }
    if (tid == 0) *cnt = e + 1u;  // read by the next call only: a plain store suffices
    return;
  }
  const int g = blockIdx.x - DFSSM_LORA_R;
  if (g * 64 >= a.N) {  // past the output rows: count the call
    if (tid == 0) *cnt = ld_dev(cnt) + 1u;
    return;
  }
  // ---- GEMV workgroup: wave w owns the 128-column chunks c = w + 16 j of its 64 rows; it loads the
  // q bytes of exactly those columns and builds their bit planes itself (wave-uniform ballots, in
  // scalar registers), so the GEMV needs no exchange between waves. All loads unconditional. ----
  int8_t qv[M][CPW][2];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int c = wave + kNW * j;
      const int cc = (CH % kNW == 0 || c < CH) ? c : CH - 1;
      qv[m][j][0] = a.q[(size_t)m * K + 128 * cc + lane];
      qv[m][j][1] = a.q[(size_t)m * K + 128 * cc + 64 + lane];
    }
  __builtin_amdgcn_sched_barrier(0);
  const u32x4* bits = (const u32x4*)a.bits + (size_t)g * CH * 64 + lane;
  u32x4 wb[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = wave + kNW * j;
    wb[j] = ld_nt(bits + (size_t)((CH % kNW == 0 || c < CH) ? c : CH - 1) * 64);
  }
  const int n = g * 64 + lane;
  const bool erow = tid < M * 64 && n < a.N;
  const int em = tid >> 6;
  const int nc = n < a.N ? n : a.N - 1, mc = em < M ? em : M - 1;
  const uint16_t ws_raw = a.wscale[nc], xs_raw = a.xscale[mc];
  const u32x4 la = *(const u32x4*)(a.lA + (size_t)nc * DFSSM_LORA_R);
  const uint16_t as_raw = a.lAs[nc];
  const uint32_t e = ld_dev(cnt);
  __builtin_amdgcn_sched_barrier(0);
  // first poll of this workgroup's copy of the intermediates, completed after the GEMV
  const uint32_t* hsrc = ws + kScafWords + (g % kScafRep) * kScafStride;
  uint32_t hv = tid < M * DFSSM_LORA_R ? ld_dev(hsrc + tid) : 0u;
  // ---- planes and GEMV, chunk by chunk ----
  int qsum[M];
  uint32_t cntb[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    qsum[m] = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) cntb[m][b] = 0;
  }
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = wave + kNW * j;
    if (c < CH) {  // wave-uniform
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint32_t pl[2][16];
        planes64(qv[m][j][0], pl[0]);
        planes64(qv[m][j][1], pl[1]);
        qsum[m] += qv[m][j][0] + qv[m][j][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = wb[j][i];
#pragma unroll
          for (int b = 0; b < 8; ++b) cntb[m][b] += __builtin_popcount(w & pl[i >> 1][8 * (i & 1) + b]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int t = 0;
#pragma unroll
    for (int b = 0; b < 7; ++b) t += (int)(cntb[m][b] << b);
    t -= (int)(cntb[m][7] << 7);
    Tred[wave][m][lane] = t;
    const int s = wave_sum_dpp_i32(qsum[m]);
    if (lane == 0) Sred[wave][m] = s;
  }
  if (tid < M * DFSSM_LORA_R) {  // the intermediates (bounded wait)
    const uint32_t tag = scaf_tag(e);
    for (uint32_t it = 0; (hv >> 16) != tag; ++it) {
      if (it == kScafSpinMax) {
        atomicOr((int*)(ws + kScafErr), 1);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      hv = ld_dev(hsrc + tid);
    }
    hl[tid / DFSSM_LORA_R][tid % DFSSM_LORA_R] = h2f((uint16_t)hv);
  }
  lds_barrier();
  if (erow) {
    const int m = em;
    int T = 0, S = 0;
#pragma unroll
    for (int w = 0; w < kNW; ++w) {
      T += Tred[w][m][lane];
      S += Sred[w][m];
    }
    const int acc = 2 * T - S;
    if (a.acc_out) a.acc_out[(size_t)m * a.N + n] = acc;
    const float y = r16(r16(r16((float)acc) * h2f(xs_raw)) * h2f(ws_raw));
    const float as = h2f(as_raw);
    double lo = 0.0;
#pragma unroll
    for (int rr = 0; rr < DFSSM_LORA_R; ++rr) {
      const float aq = r16((float)(int8_t)(la[rr >> 2] >> (8 * (rr & 3))) * as);
      lo += (double)hl[m][rr] * (double)aq;
    }
    a.y_out[(size_t)m * a.N + n] = f2h(r16((float)lo + y));
  }
  if (tid == 0) *cnt = e + 1u;
}

template <int M>
static hipError_t launch_scaffold_x(const ScaffoldArgs& a, hipStream_t s) {
  const dim3 grid(kScafGrid);
  switch (a.K / 512) {
#define DFSSM_SCAF_KB(kb) \
  case kb: hipLaunchKernelGGL((scaffold_xchg_kernel<M, kb>), grid, dim3(kNT), 0, s, a); break;
    DFSSM_SCAF_KB(1) DFSSM_SCAF_KB(2) DFSSM_SCAF_KB(3) DFSSM_SCAF_KB(4) DFSSM_SCAF_KB(5)
    DFSSM_SCAF_KB(6) DFSSM_SCAF_KB(7) DFSSM_SCAF_KB(8) DFSSM_SCAF_KB(9) DFSSM_SCAF_KB(10)
#undef DFSSM_SCAF_KB
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_scaffold_xchg(const ScaffoldArgs& a, int M, hipStream_t s) {
  if (a.K > kMaxK || a.K % 512 || M < 1 || M > 4 || !a.ws || !a.xn || !a.lBq || !a.h_out || !a.lA ||
      !a.lAs || !a.y_out || !a.wscale || !a.xscale || a.N < 1 || (a.N + 63) / 64 > kScafMaxGroups)
    return hipErrorInvalidValue;
  switch (M) {
    case 1: return launch_scaffold_x<1>(a, s);
    case 2: return launch_scaffold_x<2>(a, s);
    case 3: return launch_scaffold_x<3>(a, s);
    default: return launch_scaffold_x<4>(a, s);
  }
}

// LoRA intermediates of the stand-alone scaffold op: workgroup (r, m) of K / 8 threads,
// h[m][r] = fp16(sum_k xn[m][k] * lBq[r][k]); fp16 x fp16 products are exact in fp32 and summed
// in fp64 (the sum of prep_kernel and the one-launch layer).
__global__ __launch_bounds__(kPT) void lora_h_kernel(LoraHArgs a) {
  __shared__ double red[kPW];
  const int r = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
  const u32x4 xv = *(const u32x4*)(a.xn + (size_t)m * a.K + 8 * tid);
  const u32x4 bv = *(const u32x4*)(a.lBq + (size_t)r * a.K + 8 * tid);
  double acc = 0.0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = h2f((uint16_t)(xv[e >> 1] >> (16 * (e & 1))));
    const float b = h2f((uint16_t)(bv[e >> 1] >> (16 * (e & 1))));
    acc += (double)(x * b);
  }
  const int nw = (int)blockDim.x >> 6;
  acc = wave_sum_dpp_f64(acc);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    double t = 0.0;
    for (int i = 0; i < nw; ++i) t += red[i];
    a.h[(size_t)m * DFSSM_LORA_R + r] = f2h((float)t);
  }
}

hipError_t launch_lora_h(const LoraHArgs& a, int M, hipStream_t s) {
  if (a.K > kMaxK || a.K % 512) return hipErrorInvalidValue;  // K / 8 threads: whole waves
  hipLaunchKernelGGL(lora_h_kernel, dim3(DFSSM_LORA_R, M), dim3(a.K / 8), 0, s, a);
  return hipGetLastError();
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

hipError_t launch_prep(const PrepArgs& a, int M, int mode, hipStream_t s) {
  // the kernel reads one sum-of-squares slot per thread and the LoRA scale with its table
  if (mode == DFSSM_MODE_OUT && (!a.sumsq_slots || a.n_slots < 1 || a.n_slots > a.K / 8)) return hipErrorInvalidValue;
  if (a.lB && !a.lBs) return hipErrorInvalidValue;
  if (a.K > kMaxK || a.K % 512) return hipErrorInvalidValue;  // K / 8 threads: whole waves
  const bool rows_path = M > 64 && !a.planes_out && !a.xn_out && !a.xs16_out && (a.h_out || !a.lB);
  if (a.q_tiled && !rows_path) return hipErrorInvalidValue;
  if (rows_path) {  // many rows: one pass each
    const dim3 g((M + kPrepRows - 1) / kPrepRows);
    if (mode == DFSSM_MODE_IN)
      hipLaunchKernelGGL(prep_rows_kernel<DFSSM_MODE_IN>, g, dim3(a.K / 8), 0, s, a, M);
    else
      hipLaunchKernelGGL(prep_rows_kernel<DFSSM_MODE_OUT>, g, dim3(a.K / 8), 0, s, a, M);
    return hipGetLastError();
  }
  // 16 workgroups of K / 8 threads per row while they are all resident at once (at most 32 waves
  // per CU: 1024 workgroups of 640 threads at batch 64 and K = 5120 would take 1.3 rounds of the
  // CUs), else 2 ranks per workgroup
  int cus = 256;
  {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                 hipSuccess)
      cus = 256;
  }
  const long long waves = 16LL * ((M + 7) / 8 * 8) * (a.K / 512);
  const bool two = waves > 32LL * cus;
  const dim3 g(8 * (two ? DFSSM_LORA_R / 2 : DFSSM_LORA_R) * ((M + 7) / 8));
  if (mode == DFSSM_MODE_IN) {
    if (two) hipLaunchKernelGGL((prep_kernel<DFSSM_MODE_IN, 2>), g, dim3(a.K / 8), 0, s, a, M);
    else hipLaunchKernelGGL((prep_kernel<DFSSM_MODE_IN, 1>), g, dim3(a.K / 8), 0, s, a, M);
  } else {
    if (two) hipLaunchKernelGGL((prep_kernel<DFSSM_MODE_OUT, 2>), g, dim3(a.K / 8), 0, s, a, M);
    else hipLaunchKernelGGL((prep_kernel<DFSSM_MODE_OUT, 1>), g, dim3(a.K / 8), 0, s, a, M);
  }
  return hipGetLastError();
}

template <int M, bool LORA>
static hipError_t launch_scaffold_k(const ScaffoldArgs& a, int groups, hipStream_t s) {
  switch (a.K / 512) {
#define DFSSM_SCAF_KB(kb) \
  case kb: hipLaunchKernelGGL((scaffold_fused_kernel<M, LORA, kb>), dim3(groups), dim3(kNT), 0, s, a); break;
    DFSSM_SCAF_KB(1) DFSSM_SCAF_KB(2) DFSSM_SCAF_KB(3) DFSSM_SCAF_KB(4) DFSSM_SCAF_KB(5)
    DFSSM_SCAF_KB(6) DFSSM_SCAF_KB(7) DFSSM_SCAF_KB(8) DFSSM_SCAF_KB(9) DFSSM_SCAF_KB(10)
#undef DFSSM_SCAF_KB
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_scaffold(const ScaffoldArgs& a, int M, hipStream_t s) {
  const int groups = (a.N + 63) / 64;
  if (a.K > kMaxK || a.K % 512 || M < 1 || M > 4) return hipErrorInvalidValue;
  if (a.xn) {  // LoRA with the intermediates computed in the same launch (M = 1)
    if (M != 1 || !a.lBq || !a.h_out || !a.lA || !a.lAs || !a.y_out) return hipErrorInvalidValue;
    return launch_scaffold_k<1, true>(a, groups, s);
  }
  if (a.lA) return hipErrorInvalidValue;  // LoRA without xn: the GEMM path
  switch (M) {
    case 1: return launch_scaffold_k<1, false>(a, groups, s);
    case 2: return launch_scaffold_k<2, false>(a, groups, s);
    case 3: return launch_scaffold_k<3, false>(a, groups, s);
    default: return launch_scaffold_k<4, false>(a, groups, s);
  }
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
