/*
 * dfssm_oracle.c -- CPU restatement of the DF-SSM per-token decode step.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP path; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The product path never
 * links or calls it.
 *
 * Two families of functions:
 *
 *  or_*    the GPU-reference numerics: the dataflow and fp16 rounding points of
 *          inference/gpu/df_ssm_inference.py:141-224 and the conv/SSM arithmetic of
 *          inference/gpu/df_ssm_kernels.cu:27-103, with two deliberate changes the benchmark
 *          configuration asks for: the SSM state is fp32 (reference: fp16) and the SSM head
 *          dimension is d_inner/nheads (reference: hard-coded 32). Activations are fp16 bit
 *          patterns (uint16_t); weights are passed exactly as stored in the .dfssm file.
 *
 *  or_c_*  the CPU-reference numerics of inference/cpu/cpu_inference.c (fp32 activations,
 *          asymmetric uint8 activation quantizer with a popcount row-sum correction). These
 *          exist so that the restated dataflow can be compared with the compiled reference
 *          layer_forward (cpu_inference.c:303-376) built with HEADDIM=64.
 *
 * exp / log1p are this file's own or_expf / or_log1pf (see there), shared bit-for-bit with the
 * HIP kernels. Sums over a vector are accumulated in double and rounded once to fp32; the reference sums in
 * fp32 in an order that no reference test fixes, so sums carry a tolerance, not bit-exactness.
 * Integer work (bit unpack, scaffold accumulators, quantized values) is exact.
 *
 * fp32 -> fp16 conversion is round-to-nearest-even with IEEE overflow to inf, the behaviour
 * of __float2half and of torch's Half conversion; it is checked exhaustively against numpy.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LORA_R 16

/* ---------------------------------------------------------------- fp16 <-> fp32 ------------ */

float or_h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
  if (e == 0) {
    float f = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
    memcpy(&bits, &f, 4);
    bits |= sign;
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t or_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* >= 65520 -> inf */
  if (ax < 0x38800000u) {                                            /* below 2^-14 */
    float af;
    memcpy(&af, &ax, 4);
    return (uint16_t)(sign | (uint32_t)rintf(af * 16777216.0f));     /* units of 2^-24, RNE */
  }
  uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static inline uint16_t r16(double v) { return or_f2h((float)v); }
static inline float hf(uint16_t h) { return or_h2f(h); }

void or_f2h_array(const float* in, uint16_t* out, long n) { for (long i = 0; i < n; ++i) out[i] = or_f2h(in[i]); }
void or_h2f_array(const uint16_t* in, float* out, long n) { for (long i = 0; i < n; ++i) out[i] = or_h2f(in[i]); }

/* ---------------------------------------------------------------- exp / log1p -------------- */

/* exp and log1p of the decode step. The reference calls CUDA's expf/log1pf
 * (df_ssm_kernels.cu:45,78-79), whose results no reference test fixes; this build defines its
 * own, written with correctly rounded operations only (+ - * /, fmaf, rintf, bit moves) so that
 * the HIP kernels, which spell out the same sequence, produce the same bits:
 *
 * exp: Cody & Waite argument reduction x = n ln2 + r with ln2 split into a 9-bit head and a tail,
 *      |r| <= ln2/2, then the degree-7 Taylor polynomial of e^r in Horner form; e^x = p 2^n with
 *      2^n assembled from exponent bits. Results below e^-86 are returned as 0, so every nonzero
 *      output is a normal number; overflow gives +inf.
 * log: u = m 2^e with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s), s = (m-1)/(m+1), with the
 *      atanh series to s^9; log1p(y) = log(1+y) + (y - ((1+y) - 1)) / (1+y) (the standard
 *      correction for the rounding of 1+y).
 * Accuracy (checked against fp64 libm in tests): exp <= 2 ulp, log1p <= 3 ulp. */
float or_expf(float x) {
  if (x != x) return x;
  if (x < -86.0f) return 0.0f;
  if (x > 89.0f) return INFINITY;
  const float n = rintf(x * 1.44269502f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.42860677e-6f, r);
  float p = 1.98412698e-4f;
  p = fmaf(p, r, 1.38888889e-3f);
  p = fmaf(p, r, 8.33333333e-3f);
  p = fmaf(p, r, 4.16666667e-2f);
  p = fmaf(p, r, 1.66666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  const uint32_t eb = (uint32_t)(ni + 127) << 23;
  float sc;
  memcpy(&sc, &eb, 4);
  return p * sc;
}

static float or_log_pos(float u) { /* finite u >= 1 */
  uint32_t b;
  memcpy(&b, &u, 4);
  int e = (int)(b >> 23) - 127;
  const uint32_t mb = (b & 0x7fffffu) | 0x3f800000u;
  float m;
  memcpy(&m, &mb, 4);
  if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 0.111111111f;
  p = fmaf(p, s2, 0.142857143f);
  p = fmaf(p, s2, 0.2f);
  p = fmaf(p, s2, 0.333333333f);
  p = p * s2;
  const float t = 2.0f * s;
  const float lm = fmaf(t, p, t);
  const float ef = (float)e;
  return fmaf(ef, 0.693145751953125f, fmaf(ef, 1.42860677e-6f, lm));
}

float or_log1pf(float y) { /* y >= 0 (softplus argument) */
  if (y != y || y == 0.0f || y == INFINITY) return y;
  const float u = 1.0f + y;
  const float lg = or_log_pos(u);
  return lg + (y - (u - 1.0f)) / u;
}

void or_expf_array(const float* x, float* out, long n) { for (long i = 0; i < n; ++i) out[i] = or_expf(x[i]); }
void or_log1pf_array(const float* x, float* out, long n) { for (long i = 0; i < n; ++i) out[i] = or_log1pf(x[i]); }

/* ---------------------------------------------------------------- bits (row a2) ------------ */

/* Word j, bit b of row n is column 32j+b; bit 1 -> +1, bit 0 -> -1.
 * export_dfssm.py:34-42 (pack), df_ssm_inference.py:23-29 (unpack), cpu_inference.c:126-128. */
void or_unpack_bits(const uint32_t* packed, int rows, int kwords, int8_t* out) {
  for (long r = 0; r < rows; ++r)
    for (int j = 0; j < kwords; ++j) {
      uint32_t w = packed[r * kwords + j];
      for (int b = 0; b < 32; ++b) out[r * kwords * 32 + j * 32 + b] = ((w >> b) & 1u) ? 1 : -1;
    }
}

/* ---------------------------------------------------------------- scaffold (row a5) -------- */

/* byte -> its 8 signs (bit i of the byte -> element i), the unpack of or_unpack_bits 8 at a time */
static int8_t sign_lut[256][8];
static void init_sign_lut(void) {
  for (int v = 0; v < 256; ++v)
    for (int i = 0; i < 8; ++i) sign_lut[v][i] = ((v >> i) & 1) ? 1 : -1;
}

/* acc[m][n] = sum_k q[m][k] * w[n][k], exact int32 (torch._int_mm, df_ssm_inference.py:157). */
void or_scaffold_acc(const uint32_t* bits, const int8_t* q, int M, int N, int K, int32_t* acc) {
  const int kw = K / 32;
  if (sign_lut[0][0] == 0) init_sign_lut();
#pragma omp parallel
  {
    int8_t* w = (int8_t*)malloc((size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      const uint8_t* rb = (const uint8_t*)(bits + (size_t)n * kw); /* little-endian words */
      for (int j = 0; j < K / 8; ++j) memcpy(w + 8 * j, sign_lut[rb[j]], 8);
      for (int m = 0; m < M; ++m) {
        const int8_t* qm = q + (size_t)m * K;
        int32_t s = 0;
        for (int k = 0; k < K; ++k) s += (int32_t)qm[k] * (int32_t)w[k];
        acc[(size_t)m * N + n] = s;
      }
    }
    free(w);
  }
}

/* ---------------------------------------------------------------- norms (rows a3, a9) ------ */

/* out = fp16((fp32(x) * r) * w), r = 1/sqrt(sum(x^2) * (1/K) + 1e-5) in fp32.
 * _rms_norm, df_ssm_inference.py:141-145, followed by copy_ into an fp16 buffer (:165,196,210).
 * The mean is sum * (1/K) as ATen's mean reduction computes it. */
void or_rmsnorm(const uint16_t* x, const float* w, int M, int K, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    const uint16_t* xm = x + (size_t)m * K;
    double ss = 0.0;
    for (int k = 0; k < K; ++k) { double v = hf(xm[k]); ss += v * v; }
    float var = (float)ss * (1.0f / (float)K);
    float r = 1.0f / sqrtf(var + 1e-5f);
    for (int k = 0; k < K; ++k) out[(size_t)m * K + k] = or_f2h((hf(xm[k]) * r) * w[k]);
  }
}

/* ---------------------------------------------------------------- quantizer (row a4) ------- */

/* _quantize_to_int8, df_ssm_inference.py:147-152:
 *   s = fp16(fp16(max(amax|x|, 1e-4)) * (1/127))   (ATen divides a tensor by a CPU scalar
 *                                                     by multiplying with its fp32 reciprocal)
 *   q = clamp(rne(fp16(x / s)), -128, 127)          (tensor/tensor division is IEEE fp32) */
void or_quantize(const uint16_t* xn, int M, int K, int8_t* q, uint16_t* s) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    const uint16_t* xm = xn + (size_t)m * K;
    float amax = 0.0f;
    for (int k = 0; k < K; ++k) { float a = fabsf(hf(xm[k])); if (a > amax) amax = a; }
    float c = hf(or_f2h(amax > 1e-4f ? amax : 1e-4f));
    uint16_t sh = or_f2h(c * (1.0f / 127.0f));
    s[m] = sh;
    float sf = hf(sh);
    for (int k = 0; k < K; ++k) {
      float t = rintf(hf(or_f2h(hf(xm[k]) / sf)));
      if (t > 127.0f) t = 127.0f;
      if (t < -128.0f) t = -128.0f;
      q[(size_t)m * K + k] = (int8_t)t;
    }
  }
}

/* ---------------------------------------------------------------- LoRA + dequant (a5, a6) -- */

/* h16[m][r] = fp16(sum_k xn[m][k] * B16[r][k]) with B16 = fp16(B_i8 * B_s[r]) (the load-time
 * dequant of df_ssm_inference.py:83, then the fp16 GEMM x_norm @ lora_B.T of :173). */
void or_lora_h(const uint16_t* xn, const int8_t* lB, const uint16_t* lBs, int M, int K, uint16_t* h16) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m)
    for (int r = 0; r < LORA_R; ++r) {
      float bs = hf(lBs[r]);
      double s = 0.0;
      for (int k = 0; k < K; ++k) {
        float b16 = hf(or_f2h((float)lB[(size_t)r * K + k] * bs));
        s += (double)hf(xn[(size_t)m * K + k]) * (double)b16;
      }
      h16[m * LORA_R + r] = r16(s);
    }
}

/* out[m][n] = fp16(y + sum_r h16[m][r] * A16[n][r]) where
 *   y   = fp16(fp16(fp16(acc) * xs[m]) * ws[n])   (_scaffold_matmul, df_ssm_inference.py:158)
 *   A16 = fp16(A_i8 * A_s[n])                       (load-time dequant, :82)
 * and the sum is the fp32 addmm_ of :173 / :204. */
void or_dequant_lora(const int32_t* acc, const uint16_t* xs, const uint16_t* ws, const uint16_t* h16,
                     const int8_t* lA, const uint16_t* lAs, int M, int N, uint16_t* out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      float a16 = hf(or_f2h((float)acc[(size_t)m * N + n]));
      float y = hf(or_f2h(hf(or_f2h(a16 * hf(xs[m]))) * hf(ws[n])));
      float as = hf(lAs[n]);
      double s = 0.0;
      for (int r = 0; r < LORA_R; ++r) {
        float a = hf(or_f2h((float)lA[(size_t)n * LORA_R + r] * as));
        s += (double)hf(h16[m * LORA_R + r]) * (double)a;
      }
      out[(size_t)m * N + n] = or_f2h((float)s + y);
    }
}

/* ---------------------------------------------------------------- conv (row a7) ------------ */

/* conv_step_kernel, df_ssm_kernels.cu:27-47: out = s0*w0 + s1*w1 + s2*w2 + x*w3 + b (fp32,
 * left to right), state <- (s1, s2, x), x <- fp16(out * 1/(1+exp(-out))). Products of two fp16
 * values are exact in fp32, so the order of additions is the only rounding choice. */
void or_conv_step(uint16_t* state, uint16_t* xbc, int ld, const uint16_t* w, const uint16_t* b, int M, int C) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m)
    for (int ch = 0; ch < C; ++ch) {
      uint16_t* cs = state + ((size_t)m * C + ch) * 3;
      uint16_t* xp = xbc + (size_t)m * ld + ch;
      float s0 = hf(cs[0]), s1 = hf(cs[1]), s2 = hf(cs[2]), xv = hf(*xp);
      cs[0] = cs[1];
      cs[1] = cs[2];
      cs[2] = *xp;
      const uint16_t* wc = w + (size_t)ch * 4;
      float o = s0 * hf(wc[0]);
      o = o + s1 * hf(wc[1]);
      o = o + s2 * hf(wc[2]);
      o = o + xv * hf(wc[3]);
      o = o + hf(b[ch]);
      float sig = 1.0f / (1.0f + or_expf(-o));
      *xp = or_f2h(o * sig);
    }
}

/* ---------------------------------------------------------------- SSM (row a8) ------------- */

/* ssm_step_kernel, df_ssm_kernels.cu:53-103, with an fp32 state and P = d_inner/nheads:
 *   dt = log1p(exp(dt_raw + dt_bias)); Abar = exp(dt * -exp(A_log))   (or_expf / or_log1pf)
 *   h[p][n] = fma(Abar, h[p][n], (x_p * dt) * B_n)
 *   y_p = fp16(sum_n C_n * h[p][n] + x_p * D)
 * x = xbc[0:DI], B = xbc[DI:DI+N], C = xbc[DI+N:DI+2N] (ngroups = 1: B and C shared by all heads,
 * df_ssm_inference.py:185-187). */
void or_ssm_step(float* h, const uint16_t* xbc, int ld_xbc, const uint16_t* dt_raw, int ld_dt,
                 const float* dt_bias, const float* A_log, const float* Dp,
                 int M, int H, int P, int N, uint16_t* y) {
  const int DI = H * P;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m)
    for (int hd = 0; hd < H; ++hd) {
      const uint16_t* xr = xbc + (size_t)m * ld_xbc;
      float dt = or_log1pf(or_expf(hf(dt_raw[(size_t)m * ld_dt + hd]) + dt_bias[hd]));
      float abar = or_expf(dt * -or_expf(A_log[hd]));
      float Bf[512], Cf[512]; /* N <= 512: B and C of this sequence, converted once */
      for (int n = 0; n < N; ++n) {
        Bf[n] = hf(xr[DI + n]);
        Cf[n] = hf(xr[DI + N + n]);
      }
      for (int p = 0; p < P; ++p) {
        float xv = hf(xr[hd * P + p]);
        float X = xv * dt;
        float* hp = h + (((size_t)m * H + hd) * P + p) * N;
        double acc = 0.0;
        for (int n = 0; n < N; ++n) {
          float hn = fmaf(abar, hp[n], X * Bf[n]);
          hp[n] = hn;
          acc += (double)Cf[n] * (double)hn;
        }
        y[(size_t)m * DI + hd * P + p] = or_f2h((float)acc + xv * Dp[hd]);
      }
    }
}

/* ---------------------------------------------------------------- gate (row a9) ------------ */

/* g = fp16(y * fp16(z * fp16(sigmoid(z)))) -- the three fp16 tensor ops of
 * df_ssm_inference.py:194-195; the gated RMSNorm is or_rmsnorm on g. */
void or_gate(const uint16_t* y, const uint16_t* z, int ld_z, int M, int DI, uint16_t* g) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m)
    for (int k = 0; k < DI; ++k) {
      float zv = hf(z[(size_t)m * ld_z + k]);
      float sg = hf(or_f2h(1.0f / (1.0f + or_expf(-zv))));
      float sz = hf(or_f2h(zv * sg));
      g[(size_t)m * DI + k] = or_f2h(hf(y[(size_t)m * DI + k]) * sz);
    }
}

/* ---------------------------------------------------------------- residual (row a10) ------- */

void or_residual(uint16_t* x, const uint16_t* o, int M, int D) {
  for (long i = 0; i < (long)M * D; ++i) x[i] = or_f2h(hf(x[i]) + hf(o[i]));
}

/* ---------------------------------------------------------------- embedding, head (a11) ---- */

/* x0 = E16[tok] with E16 = fp16(E_i8 * s_E) for the int8 table (emb_code 1) or the stored fp16
 * table (emb_code 0); df_ssm_inference.py:220. */
void or_embed(const int8_t* E8, const uint16_t* sE, const uint16_t* E16, int emb_code,
              const int64_t* tok, int M, int D, uint16_t* x) {
  for (int m = 0; m < M; ++m) {
    long t = (long)tok[m];
    for (int k = 0; k < D; ++k)
      x[(size_t)m * D + k] = emb_code ? or_f2h((float)E8[t * D + k] * hf(sE[t])) : E16[t * D + k];
  }
}

/* logits[m][v] = fp16(sum_k xf[m][k] * E[v][k]) (tied head, df_ssm_inference.py:224). For the
 * int8 table the row scale is applied after the dot product: fp16(fp32(dot) * s_E[v]).
 * next[m] = first index of the maximum fp16 logit (torch.argmax, :236). */
void or_lm_head(const uint16_t* xf, const int8_t* E8, const uint16_t* sE, const uint16_t* E16, int emb_code,
                int M, int V, int D, uint16_t* logits, int64_t* next) {
  double* xd = (double*)malloc(sizeof(double) * (size_t)M * D);
  for (long i = 0; i < (long)M * D; ++i) xd[i] = hf(xf[i]);
#pragma omp parallel for schedule(static)
  for (int v = 0; v < V; ++v)
    for (int m = 0; m < M; ++m) {
      double s = 0.0;
      const double* xm = xd + (size_t)m * D;
      if (emb_code) {
        const int8_t* e = E8 + (size_t)v * D;
        for (int k = 0; k < D; ++k) s += xm[k] * (double)e[k];
        logits[(size_t)m * V + v] = or_f2h((float)s * hf(sE[v]));
      } else {
        const uint16_t* e = E16 + (size_t)v * D;
        for (int k = 0; k < D; ++k) s += xm[k] * (double)hf(e[k]);
        logits[(size_t)m * V + v] = r16(s);
      }
    }
  free(xd);
  for (int m = 0; m < M; ++m) {
    int64_t best = 0;
    float bv = hf(logits[(size_t)m * V]);
    for (int v = 1; v < V; ++v) {
      float lv = hf(logits[(size_t)m * V + v]);
      if (lv > bv) { bv = lv; best = v; }
    }
    next[m] = best;
  }
}

/* ================================================================ CPU-reference numerics ==== */

/* rms_norm, cpu_inference.c:34-52: out = (x * w) * (1/sqrt(ss/dim + 1e-5)). */
void or_c_rms_norm(const float* x, const float* w, float* out, int M, int dim) {
  for (int m = 0; m < M; ++m) {
    const float* xm = x + (size_t)m * dim;
    double ss = 0.0;
    for (int i = 0; i < dim; ++i) ss += (double)xm[i] * xm[i];
    float inv = 1.0f / sqrtf((float)ss / dim + 1e-5f);
    for (int i = 0; i < dim; ++i) out[(size_t)m * dim + i] = xm[i] * w[i] * inv;
  }
}

/* quantize_input_uint8, cpu_inference.c:65-97: s = 255/(2 max(amax, 1e-8)),
 * q = rne(clamp(x*s + 128, 0, 255)), x_scale = 1/s. x*s + 128 is one fused multiply-add: gcc
 * contracts the _mm512_add_ps(_mm512_mul_ps(..)) of :86-87 at its default -ffp-contract=fast, and
 * the compiled reference rounds e.g. fma(x, s, 128) = 0.50000006 (product -127.49999994) to 1
 * where the unfused sum would be 0.5 -> 0. */
void or_c_quantize_u8(const float* x, int K, uint8_t* q, float* x_scale) {
  float amax = 0.0f;
  for (int i = 0; i < K; ++i) { float a = fabsf(x[i]); if (a > amax) amax = a; }
  if (amax < 1e-8f) amax = 1e-8f;
  float s = 255.0f / (2.0f * amax);
  *x_scale = 1.0f / s;
  for (int i = 0; i < K; ++i) {
    float v = fmaf(x[i], s, 128.0f);
    if (v < 0.0f) v = 0.0f;
    if (v > 255.0f) v = 255.0f;
    q[i] = (uint8_t)rintf(v);
  }
}

/* scaffold_matvec_avx512, cpu_inference.c:99-151, with precompute_row_sums (:286-299):
 * out = fp32(dot(u8, +-1) - 128 * rowsum) * x_scale * scale. */
void or_c_scaffold(const uint32_t* bits, const float* x, const float* scale, int M, int N, int K, float* out) {
  const int kw = K / 32;
  uint8_t* q = (uint8_t*)malloc((size_t)K);
  for (int m = 0; m < M; ++m) {
    float xs;
    or_c_quantize_u8(x + (size_t)m * K, K, q, &xs);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
      const uint32_t* row = bits + (size_t)n * kw;
      int32_t dot = 0, pop = 0;
      for (int j = 0; j < kw; ++j) {
        pop += __builtin_popcount(row[j]);
        for (int b = 0; b < 32; ++b) dot += ((row[j] >> b) & 1u) ? (int32_t)q[j * 32 + b] : -(int32_t)q[j * 32 + b];
      }
      int32_t rowsum = 2 * pop - K;
      out[(size_t)m * N + n] = (float)(dot - 128 * rowsum) * xs * scale[n];
    }
  }
  free(q);
}

/* lora_matvec, cpu_inference.c:155-194: h[r] = (B[r].x) * Bs[r]; out[n] += (A[n].h) * As[n]. */
void or_c_lora(const int8_t* A, const float* As, const int8_t* B, const float* Bs, const float* x,
               float* out, int M, int N, int K) {
  for (int m = 0; m < M; ++m) {
    float hr[LORA_R];
    for (int r = 0; r < LORA_R; ++r) {
      double s = 0.0;
      for (int k = 0; k < K; ++k) s += (double)B[(size_t)r * K + k] * x[(size_t)m * K + k];
      hr[r] = (float)s * Bs[r];
    }
    for (int n = 0; n < N; ++n) {
      float s = 0.0f;
      for (int r = 0; r < LORA_R; ++r) s += (float)A[(size_t)n * LORA_R + r] * hr[r];
      out[(size_t)m * N + n] += s * As[n];
    }
  }
}

/* conv_step, cpu_inference.c:204-227 (fp32 state). */
void or_c_conv(float* state, float* xbc, int ld, const float* w, const float* b, int M, int C) {
  for (int m = 0; m < M; ++m)
    for (int ch = 0; ch < C; ++ch) {
      float* cs = state + ((size_t)m * C + ch) * 3;
      float* xp = xbc + (size_t)m * ld + ch;
      float s0 = cs[0], s1 = cs[1], s2 = cs[2], xv = *xp;
      cs[0] = s1; cs[1] = s2; cs[2] = xv;
      float o = s0 * w[ch * 4 + 0] + s1 * w[ch * 4 + 1] + s2 * w[ch * 4 + 2] + xv * w[ch * 4 + 3] + b[ch];
      *xp = o / (1.0f + expf(-o));
    }
}

/* softplus in layer_forward (cpu_inference.c:352-355) + ssm_step (:231-262). */
void or_c_ssm(float* h, const float* xbc, int ld, const float* dt_raw, int ld_dt, const float* dt_bias,
              const float* A_log, const float* Dp, int M, int H, int P, int N, float* y) {
  const int DI = H * P;
  for (int m = 0; m < M; ++m)
    for (int hd = 0; hd < H; ++hd) {
      const float* xr = xbc + (size_t)m * ld;
      float dt = log1pf(expf(dt_raw[(size_t)m * ld_dt + hd] + dt_bias[hd]));
      float abar = expf(dt * -expf(A_log[hd]));
      for (int p = 0; p < P; ++p) {
        float xv = xr[hd * P + p], X = xv * dt;
        float* hp = h + (((size_t)m * H + hd) * P + p) * N;
        double acc = 0.0;
        for (int n = 0; n < N; ++n) {
          float hn = abar * hp[n] + X * xr[DI + n];
          hp[n] = hn;
          acc += (double)xr[DI + N + n] * hn;
        }
        y[(size_t)m * DI + hd * P + p] = (float)acc + xv * Dp[hd];
      }
    }
}

/* gate_norm, cpu_inference.c:266-278: g = y * silu(z); out = g * inv_rms * w. */
void or_c_gate_norm(const float* y, const float* z, int ld_z, const float* w, float* out, int M, int DI) {
  for (int m = 0; m < M; ++m) {
    double ss = 0.0;
    for (int i = 0; i < DI; ++i) {
      float zv = z[(size_t)m * ld_z + i];
      float g = y[(size_t)m * DI + i] * (zv / (1.0f + expf(-zv)));
      out[(size_t)m * DI + i] = g;
      ss += (double)g * g;
    }
    float inv = 1.0f / sqrtf((float)ss / DI + 1e-5f);
    for (int i = 0; i < DI; ++i) out[(size_t)m * DI + i] = out[(size_t)m * DI + i] * inv * w[i];
  }
}

/* ---------------------------------------------------------------- sampling ---------------- */
/* The sampling head's definition (dfssm_sample), restated by its definition rather than by the
 * kernel's radix select and slab scan: penalty + temperature per eval/gen_test.py:71-74 (mode 0)
 * or training/df_ssm_mamba2_distill_dfw.py:1069-1073 (mode 1); e = exp(z - max z),
 * E = floor(e 2^40); tokens ranked by e descending, index ascending (a full sort here); a token is
 * kept iff the E mass ranked above it is <= floor(top_p * Z) -- the reference's
 * `(cumsum - p) > top_p` drop rule (gen_test.py:77-80) on exact masses; the draw is the first
 * kept index (index order) whose cumulative kept mass exceeds R = floor(h S / 2^64), S the kept
 * mass and h = splitmix64 (Steele, Lea, Flood 2014) of seed ^ (sequence << 40 | step << 17 | 0x1ffff). */
static uint64_t or_splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

static float or_penalized(float l, int cnt, float T, float r, int mode) {
  if (mode == 0) {
    float z = l / T;
    return cnt > 0 ? z / r : z;
  }
  float z = l;
  for (int k = 0; k < cnt; ++k) z = z > 0.0f ? z / r : z * r;
  return z / T;
}

typedef struct { uint32_t key; int idx; } or_rank_t;
static int or_rank_cmp(const void* pa, const void* pb) {
  const or_rank_t* a = (const or_rank_t*)pa;
  const or_rank_t* b = (const or_rank_t*)pb;
  if (a->key != b->key) return a->key > b->key ? -1 : 1;
  return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

/* logits (M, V) fp16, counts (M, V) and step (M) updated as the kernel does; kept (M, V) optional
 * output of the kept set (1/0). */
void or_sample(const uint16_t* logits, int32_t* counts, uint32_t* step, int M, int V, float T, float top_p,
               float r, int mode, uint64_t seed, int64_t* next, uint8_t* kept_out) {
  float* z = (float*)malloc(sizeof(float) * V);
  uint64_t* E = (uint64_t*)malloc(sizeof(uint64_t) * V);
  or_rank_t* rk = (or_rank_t*)malloc(sizeof(or_rank_t) * V);
  uint8_t* kept = (uint8_t*)malloc(V);
  for (int b = 0; b < M; ++b) {
    const uint16_t* lg = logits + (size_t)b * V;
    int32_t* cn = counts + (size_t)b * V;
    float m = -INFINITY;
    for (int i = 0; i < V; ++i) {
      z[i] = or_penalized(or_h2f(lg[i]), cn[i], T, r, mode);
      m = fmaxf(m, z[i]);
    }
    uint64_t Z = 0;
    for (int i = 0; i < V; ++i) {
      float e = or_expf(z[i] - m);
      memcpy(&rk[i].key, &e, 4);
      rk[i].idx = i;
      E[i] = (uint64_t)(e * 1099511627776.0f);
      Z += E[i];
    }
    uint64_t thr = (uint64_t)((double)top_p * (double)Z);
    if (top_p >= 1.0f || thr >= Z) {
      memset(kept, 1, V);
    } else {
      qsort(rk, V, sizeof(or_rank_t), or_rank_cmp);
      uint64_t S = 0;
      for (int k = 0; k < V; ++k) {
        kept[rk[k].idx] = S <= thr;
        S += E[rk[k].idx];
      }
    }
    uint64_t S = 0;
    for (int i = 0; i < V; ++i) if (kept[i]) S += E[i];
    uint64_t h = or_splitmix64(seed ^ (((uint64_t)b << 40) | ((uint64_t)(step[b] & 0x7fffffu) << 17) | 0x1ffffull));
    uint64_t R = (uint64_t)(((unsigned __int128)h * S) >> 64);
    uint64_t acc = 0;
    int bi = V;
    for (int i = 0; i < V; ++i) {
      if (!kept[i]) continue;
      acc += E[i];
      if (acc > R) { bi = i; break; }
    }
    int tok = bi < V ? bi : 0;
    next[b] = tok;
    cn[tok] += 1;
    step[b] += 1u;
    if (kept_out) memcpy(kept_out + (size_t)b * V, kept, V);
  }
  free(z); free(E); free(rk); free(kept);
}

/* Density-field state quantization at a chunk boundary, training/df_ssm_mamba2_distill_dfw.py:
 * 139-165 (df_ssd_scan: mean/std scaling, sigma-delta), :88-91 (SprayBank.quantize: searchsorted
 * count / KK), :105-110 (_quantize_error). Rows of 128 values. The two row sums are fp64 sums of
 * the value pairs (2l, 2l+1) over the adjacent-pair tree; std is unbiased (torch.std). */
static double or_tree_sum64(double* v) {
  for (int w = 1; w < 64; w *= 2)
    for (int l = 0; l < 64; l += 2 * w) v[l] = v[l] + v[l + w];
  return v[0];
}
void or_state_df(float* h, float* sd_error, long rows, const float* R, int kk, int sd_bits) {
  for (long r = 0; r < rows; ++r) {
    float* x = h + r * 128;
    float* e = sd_error ? sd_error + r * 128 : NULL;
    double v[64];
    for (int l = 0; l < 64; ++l) v[l] = (double)x[2 * l] + (double)x[2 * l + 1];
    const float mean = (float)(or_tree_sum64(v) / 128.0);
    for (int l = 0; l < 64; ++l) {
      const float d0 = x[2 * l] - mean, d1 = x[2 * l + 1] - mean;
      v[l] = (double)d0 * (double)d0 + (double)d1 * (double)d1;
    }
    float sd = sqrtf((float)(or_tree_sum64(v) / 127.0));
    if (!(sd > 1e-8f)) sd = 1e-8f;
    const float t3 = 3.0f * sd, t6 = 6.0f * sd;
    const float lo = mean - t3;
    const float range = t6 > 1e-8f ? t6 : 1e-8f;
    const float scale = sd_bits < 32 ? (float)(1 << (sd_bits - 1)) : 1.0f;
    for (int k = 0; k < 128; ++k) {
      float hs = (x[k] - lo) / range;
      hs = hs < 0.0f ? 0.0f : (hs > 1.0f ? 1.0f : hs);
      float hc = hs;
      if (e) {
        hc = hs + e[k];
        hc = hc < 0.0f ? 0.0f : (hc > 1.0f ? 1.0f : hc);
      }
      int cnt = 0;
      while (cnt < kk && R[cnt] < hc) ++cnt;  /* sorted: the number of thresholds below hc */
      const float q = (float)cnt / (float)kk;
      if (e) {
        float d = hc - q;
        d = d < -1.0f ? -1.0f : (d > 1.0f ? 1.0f : d);
        if (sd_bits < 32) d = rintf(d * scale) / scale;
        e[k] = d;
      }
      const float qr = q * range;
      x[k] = qr + lo;
    }
  }
}
