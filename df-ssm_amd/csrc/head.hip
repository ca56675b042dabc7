// Embedding gather, final RMSNorm + tied LM head + greedy argmax (gfx950).
//
// The table -- int8 with an fp16 row scale (format embedding code 1), or fp16 as the exporter
// writes it (code 0) -- is stored re-tiled at load time as [V_pad/64][row bytes/16][64 lanes]
// [16 B]: lane l of a wave owns vocabulary row 64*g + l and each wave-wide 16-byte load is one
// contiguous 1 KiB transaction. Wave w of the 256-thread workgroup covers a quarter of D.
//
// Logits (df_ssm_inference.py:210,224): xf = fp16(RMSNorm(x) * norm_f); int8 table:
// logit_v = fp16(fp32(sum_k xf_k * E_i8[v,k]) * s_E[v]); fp16 table: logit_v = fp16(fp32(sum_k
// xf_k * E_16[v,k])). The dot product is accumulated in fp64, where the products (fp16 x int8,
// fp16 x fp16) are exact, so the result does not depend on the summation order. Greedy token = first index of the maximum fp16 logit (torch.argmax, :236):
// every workgroup writes its (max, first index) pair; the last workgroup to finish (ticket
// counter, reset by that workgroup) reduces the pairs and may write the next token's embedding.
#include "common.h"
#include "dfssm_kernels.h"

#include <type_traits>

namespace dfssm {

// Vocabulary limit of the heads: at most 1024 table groups of 64 rows (V <= 65536), so that the
// last workgroup's argmax holds every per-workgroup pair in registers; k slices of 512 per row.
constexpr int kHeadMaxGroups = 1024;
constexpr int kHeadMaxKP = 10;  // D <= 5120

// Element j of a 16-byte table chunk, widened: 16 int8 or 8 fp16 per chunk.
template <bool F16>
__device__ __forceinline__ double emb_elem(const u32x4& e4, int j) {
  if (F16) return (double)h2f((uint16_t)(e4[j >> 1] >> (16 * (j & 1))));
  return (double)(int)(int8_t)(e4[j >> 2] >> (8 * (j & 3)));
}
// Embedding value of row t (tile group tg = t / 64, lane tl = t % 64), column k, as fp16 bits.
template <bool F16>
__device__ __forceinline__ uint16_t emb_value(const uint8_t* emb, const uint16_t* scale, int CH, int tg, int tl, int k) {
  if (F16) return ((const uint16_t*)(emb + (((size_t)tg * CH + (k >> 3)) * 64 + tl) * 16))[k & 7];
  return f2h((float)(int8_t)emb[(((size_t)tg * CH + (k >> 4)) * 64 + tl) * 16 + (k & 15)] * h2f(scale[tg * 64 + tl]));
}

// (value, index) pair reductions of the argmax: the larger value wins, on equal values the
// smaller index. Candidates enter through `>` comparisons against -inf, so no NaN is ever a best:
// a total order, and the result does not depend on the order of the reduction. DPP steps move the
// pairs between lanes in the VALU (an LDS shuffle costs a round trip per step).
__device__ __forceinline__ void argmax_take(float& b, int& bi, float ob, int oi) {
  if (ob > b || (ob == b && oi < bi)) { b = ob; bi = oi; }
}
template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float& b, int& bi) {
  argmax_take(b, bi, dpp_f32<CTRL>(b), dpp_i32<CTRL>(bi));
}
// over the 16 lanes of every DPP row: each lane ends with its row's pair
__device__ __forceinline__ void row_argmax_dpp(float& b, int& bi) {
  argmax_dpp_step<0xB1>(b, bi);   // quad_perm 1,0,3,2
  argmax_dpp_step<0x4E>(b, bi);   // quad_perm 2,3,0,1
  argmax_dpp_step<0x124>(b, bi);  // row_ror 4
  argmax_dpp_step<0x128>(b, bi);  // row_ror 8
}
// over the wave: each lane ends with the wave's pair
__device__ __forceinline__ void wave_argmax_dpp(float& b, int& bi) {
  row_argmax_dpp(b, bi);
  float rb[4];
  int ri[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    rb[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, b), 16 * r));
    ri[r] = __builtin_amdgcn_readlane(bi, 16 * r);
  }
  b = rb[0];
  bi = ri[0];
#pragma unroll
  for (int r = 1; r < 4; ++r) argmax_take(b, bi, rb[r], ri[r]);
}

// The last workgroup's argmax over the NG per-workgroup (max, first index) pairs of every row
// (part_val/part_idx, row-major by row): wave w takes rows w + NWV (r0 + r), r < RW, and every
// lane loads all its pairs of all those rows (at most K each, clamped in-bounds addresses) before
// comparing any, so the reduction costs one memory round trip. Writes a.next and toks.
template <int NWV, int RW, int K>
__device__ __forceinline__ void argmax_pairs(const HeadArgs& a, int M, int NG, int* toks, int r0 = 0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float pv[RW][K];
  int pi[RW][K];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int m = wave + NWV * (r0 + r) < M ? wave + NWV * (r0 + r) : M - 1;
#pragma unroll
    for (int q = 0; q < K; ++q) {
      const int j = lane + 64 * q < NG ? lane + 64 * q : NG - 1;
      pv[r][q] = __hip_atomic_load(a.part_val + (size_t)m * NG + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pi[r][q] = __hip_atomic_load(a.part_idx + (size_t)m * NG + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int m = wave + NWV * (r0 + r);
    float b = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < K; ++q)
      if (lane + 64 * q < NG && (pv[r][q] > b || (pv[r][q] == b && pi[r][q] < bi))) {
        b = pv[r][q];
        bi = pi[r][q];
      }
    wave_argmax_dpp(b, bi);
    if (lane == 0 && m < M) {
      // no comparable logit (all NaN): report token 0 rather than an index outside the table
      if (bi < 0 || bi >= a.V) bi = 0;
      a.next[m] = (int64_t)bi;
      toks[m] = bi;
    }
  }
}

// x_next[m] = the embedding of token toks[m], m < M, by NT threads in 16-byte table chunks (16
// int8 or 8 fp16 values), KB chunks per thread loaded before any is converted and stored.
template <bool F16, int NT, int KB = 8>
__device__ __forceinline__ void embed_next(const HeadArgs& a, const int* toks, int M, int D) {
  const int CH = F16 ? D / 8 : D / 16, n = M * CH;
  for (int c0 = (int)threadIdx.x; c0 < n; c0 += NT * KB) {
    u32x4 ch[KB];
    uint16_t sc[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const int c = c0 + NT * i < n ? c0 + NT * i : n - 1;
      const int m = c / CH, k = c - m * CH, t = toks[m];
      ch[i] = *(const u32x4*)(a.emb + (((size_t)(t >> 6) * CH + k) * 64 + (t & 63)) * 16);
      sc[i] = F16 ? (uint16_t)0 : a.emb_scale[t];
    }
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const int c = c0 + NT * i;
      if (c < n) {
        const int m = c / CH, k = c - m * CH;
        if (F16) {
          *(u32x4*)(a.x_next + (size_t)m * D + 8 * k) = ch[i];
        } else {
          const float sv = h2f(sc[i]);
          uint32_t o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = ch[i][e >> 1];
            const int sh = 16 * (e & 1);
            const float v0 = (float)(int8_t)(w >> sh) * sv, v1 = (float)(int8_t)(w >> (sh + 8)) * sv;
            o[e] = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
          }
          u32x4* dst = (u32x4*)(a.x_next + (size_t)m * D + 16 * k);
          dst[0] = u32x4{o[0], o[1], o[2], o[3]};
          dst[1] = u32x4{o[4], o[5], o[6], o[7]};
        }
      }
    }
  }
}

template <int M, bool F16>
__global__ __launch_bounds__(256) void head_kernel(HeadArgs a) {
  extern __shared__ double xf[];  // [M][D] final-normed activations as fp64
  __shared__ double part[4][M][64];
  __shared__ double red_d[4];
  __shared__ bool is_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  constexpr int EPC = F16 ? 8 : 16;  // table elements per 16-byte chunk
  const int D = a.D, CH = D / EPC, CPW = CH / 4;
  const u32x4* E = (const u32x4*)a.emb + ((size_t)g * CH + wave * CPW) * 64 + lane;

  // first group of chunks in flight before the prologue (the table does not depend on x)
  constexpr int G = 8;  // chunks per group; D is a multiple of 512, so CPW is a multiple of 8
  u32x4 cur[G], nxt[G];
#pragma unroll
  for (int c = 0; c < G; ++c) cur[c] = ld_nt(E + (size_t)c * 64);

  for (int m = 0; m < M; ++m) {
    const uint16_t* xm = a.x + (size_t)m * D;
    double ps = 0.0;
    for (int k = tid; k < D; k += 256) { double v = (double)h2f(xm[k]); ps += v * v; }
    const double ss = block_sum_f64<256>(ps, red_d);
    const float var = (float)ss * (1.0f / (float)D);
    const float r = 1.0f / sqrt_rn(var + 1e-5f);
    for (int k = tid; k < D; k += 256) xf[m * D + k] = (double)r16((h2f(xm[k]) * r) * a.norm_f[k]);
  }
  __syncthreads();

  double acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0;
  for (int c0 = 0; c0 < CPW; c0 += G) {
    if (c0 + G < CPW) {
#pragma unroll
      for (int c = 0; c < G; ++c) nxt[c] = ld_nt(E + (size_t)(c0 + G + c) * 64);
    }
#pragma unroll
    for (int c = 0; c < G; ++c) {
      const u32x4 e4 = cur[c];
      const int k0 = (wave * CPW + c0 + c) * EPC;
#pragma unroll
      for (int j = 0; j < EPC; ++j) {
        const double e = emb_elem<F16>(e4, j);
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = __builtin_fma(xf[m * D + k0 + j], e, acc[m]);
      }
    }
#pragma unroll
    for (int c = 0; c < G; ++c) cur[c] = nxt[c];
  }
#pragma unroll
  for (int m = 0; m < M; ++m) part[wave][m][lane] = acc[m];
  __syncthreads();

  if (wave < M) {
    const int m = wave;
    const int v = g * 64 + lane;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    if (v < a.V) {
      const double s = part[0][m][lane] + part[1][m][lane] + part[2][m][lane] + part[3][m][lane];
      const uint16_t lh = F16 ? f2h((float)s) : f2h((float)s * h2f(a.emb_scale[v]));
      if (a.logits) a.logits[(size_t)m * a.V + v] = lh;
      best = h2f(lh);
      bidx = v;
    }
    wave_argmax_dpp(best, bidx);
    if (lane == 0) {
      a.part_val[(size_t)m * gridDim.x + g] = best;
      a.part_idx[(size_t)m * gridDim.x + g] = bidx;
    }
  }
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const unsigned t = atomicAdd(a.ticket, 1u);
    is_last = (t == gridDim.x - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  __shared__ int next_tok[M];
  argmax_pairs<4, 1, kHeadMaxGroups / 64>(a, M, (int)gridDim.x, next_tok);
  if (tid == 0) *a.ticket = 0u;
  __syncthreads();
  if (a.x_next) embed_next<F16, 256>(a, next_tok, M, D);
}

__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
  const int m = blockIdx.x;
  const int64_t t64 = a.tok_tc > 0 ? a.tokens[(size_t)(m / a.tok_tc) * a.tok_ld + a.tok_t0 + m % a.tok_tc] : a.tokens[m];
  const int t = (t64 < 0 || t64 >= a.V) ? 0 : (int)t64;
  if (t64 < 0 || t64 >= a.V) {
    if (threadIdx.x == 0) atomicOr(a.err_flag, DFSSM_ERR_TOKEN_RANGE);
  }
  for (int k = threadIdx.x; k < a.D; k += 256)
    a.x[(size_t)m * a.D + k] = a.f16 ? emb_value<true>(a.emb, a.emb_scale, a.D / 8, t >> 6, t & 63, k)
                                     : emb_value<false>(a.emb, a.emb_scale, a.D / 16, t >> 6, t & 63, k);
}

// Re-tile a row-major (V, D) table of D bytes per row into [V_pad/64][D/16][64][16].
__global__ void tile_emb_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int V, int D, int v_pad) {
  const size_t total = (size_t)v_pad * D / 4;  // in 4-byte units
  const int CH = D / 16;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int w = (int)(i & 3);              // which 4-byte word of the 16-byte chunk
    const int lane = (int)((i >> 2) & 63);
    const size_t rest = i >> 8;              // g * CH + c
    const int c = (int)(rest % CH);
    const int g = (int)(rest / CH);
    const int row = g * 64 + lane;
    uint32_t v = 0;
    if (row < V) v = *(const uint32_t*)(src + (size_t)row * D + c * 16 + w * 4);
    ((uint32_t*)dst)[i] = v;
  }
}

// ---------------------------------------------------------------------------------------------
// Exact int8 head for 1..4 rows on the int8 matrix cores (int8 table). An fp16 value xf is
// X 2^-24 with X an integer, |X| < 2^40, written as six signed base-256 digits d_b in [-128, 127]
// (X = sum_b d_b 256^b); v_mfma_i32_16x16x64_i8 gives exact int32 sums S_b[v] = sum_k d_b[k] E[v][k],
// and T = sum_b S_b 256^b (int64) = sum_k X_k E[v][k] exactly. The logit is fp16(fp32(T 2^-24) *
// s_E[v]): the fp64 kernel's value whenever that one's sum is exact, and exact without condition.
//
// MFMA layout (per 64-wide k step, two MFMAs): B = the table (lane l: row l % 16 of the wave's
// 16 rows, tiled 16-byte chunk l / 16 of the step), A = the digit rows (lane l: row l % 16 of the
// A tile, the same k block); tile 0 holds digits 0..3 of sequence m at A-rows 4 m + b, tile 1
// digits 4, 5 at A-rows 4 m, 4 m + 1, so lane group m = l / 16 ends with all six sums of
// (m, row l % 16) (the output layout is D[4 (l / 16) + e][l % 16]).
// ---------------------------------------------------------------------------------------------
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr int kHKS = 512;  // k slice per workgroup

// fp16 value * 2^24 as an integer (exact for finite values).
__device__ __forceinline__ long long fx24(uint16_t hb) {
  const int e = (hb >> 10) & 31, mant = hb & 1023;
  const long long X = e ? (long long)(1024 | mant) << (e - 1) : (long long)mant;
  return (hb & 0x8000) ? -X : X;
}

// ---------------------------------------------------------------------------------------------
// Work unit: each 1024-thread workgroup (one per CU) owns kHgGroups consecutive 64-row table
// groups over the whole k range (KP = D / 512 slices of 512, a template parameter so that the
// slice loop unrolls), so no partial sum leaves the workgroup. Wave w takes table rows
// 16 (w % 4) .. + 15 of group kHgGroups blockIdx + w / 4 and streams them through a two-slice
// register ring: slice kp + 2 is issued as soon as slice kp has gone through the MFMAs. The
// workgroup computes the final norm and the six digit planes of the whole rows once, into LDS
// (M * 6 * D bytes), two columns per thread; the int32 accumulators hold the sums over all of k
// (at most 5120 * 128 * 127 < 2^31 in magnitude), recombined in int64. Then the logits, the
// workgroup's (max, first index) pair per sequence, and the last workgroup (ticket) reduces the
// pairs and may write the next embedding. Measured at batch 1, 1.3B shape, per head: 25.3 us for
// the earlier form (256-thread workgroups on 64 rows x a 512-wide slice, partial sums combined by
// the last slice of each group through a per-group counter); 23.5 us for 256-thread workgroups on
// one group over all of k (each of the 786 workgroups computed the whole rows' digit planes with
// four waves, which held back the ring's refill); 20.1 us for this form.
// ---------------------------------------------------------------------------------------------
constexpr int kHgThreads = 1024, kHgWaves = kHgThreads / 64, kHgGroups = kHgWaves / 4;

template <int M, int KP>
__global__ __launch_bounds__(kHgThreads) void head_i8g_kernel(HeadArgs a, int NG) {
  extern __shared__ __attribute__((aligned(16))) int8_t hg_dg[];  // [M * 6][D] digit planes
  __shared__ double red[kHgWaves][M];
  __shared__ float pv[kHgWaves][M];
  __shared__ int pix[kHgWaves][M];
  __shared__ int next_tok[M];
  __shared__ bool is_last;
  constexpr int D = KP * kHKS, CH = D / 16, PH = D / 2;
  constexpr int PJ = (PH + kHgThreads - 1) / kHgThreads;  // column pairs per thread (tid + 1024 j)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int jg = lane >> 4, rl = lane & 15;
  const int G = gridDim.x, wg = blockIdx.x;
  const int g = kHgGroups * wg + (wave >> 2);           // this wave's table group (may be >= NG)
  const int gc = g < NG ? g : NG - 1;                    // clamped for the loads
  const int row = 16 * (wave & 3) + rl, v = g * 64 + row;

  // loads: x and norm_f of this thread's column pairs (unconditional, from clamped pairs: a load in
  // a branch makes the compiler wait for every load at the join), the row scale, then the table's
  // first two slices. Loads complete in issue order, and the scheduler would otherwise move the
  // table loads ahead of norm_f (the digit planes then waited for the table); sched_barrier pins
  // each group where it is issued.
  uint32_t xp[M][PJ];
  float2 nf[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int p = tid + kHgThreads * j, pc = p < PH ? p : 0;
#pragma unroll
    for (int m = 0; m < M; ++m) xp[m][j] = *(const uint32_t*)(a.x + (size_t)m * D + 2 * pc);
    nf[j] = *(const float2*)(a.norm_f + 2 * pc);
  }
  const uint16_t es = a.emb_scale[v < a.V ? v : a.V - 1];
  __builtin_amdgcn_sched_barrier(0);
  const u32x4* E = (const u32x4*)a.emb + ((size_t)gc * CH + jg) * 64 + 16 * (wave & 3) + rl;
  u32x4 b0[8], b1[8];
  auto load_slice = [&](u32x4 (&bf)[8], int kp) {
#pragma unroll
    for (int s = 0; s < 8; ++s) bf[s] = ld_nt(E + (size_t)(kp * (kHKS / 16) + 4 * s) * 64);
    __builtin_amdgcn_sched_barrier(0);
  };
  // the second slice before the digit planes at M = 1, after them for more rows (whose digit
  // registers and a second slice in flight together spilled; at M = 3 so did the first slice)
  if constexpr (M != 3) load_slice(b0, 0);
  if constexpr (KP > 1 && M == 1) load_slice(b1, 1);

  // final RMSNorm scale of each row (fp64 sum of squares: exact)
#pragma unroll
  for (int m = 0; m < M; ++m) {
    double ps = 0.0;
#pragma unroll
    for (int j = 0; j < PJ; ++j)
      if (tid + kHgThreads * j < PH) {
        const double x0 = (double)h2f((uint16_t)xp[m][j]), x1 = (double)h2f((uint16_t)(xp[m][j] >> 16));
        ps += x0 * x0;
        ps += x1 * x1;
      }
    ps = wave_sum_dpp_f64(ps);
    if (lane == 0) red[wave][m] = ps;
  }
  // barriers that order LDS only: a full barrier would first wait for every load of the wave,
  // the table slices in flight included
  lds_barrier();
  // digit planes of xf 2^24 (xf = fp16(x r norm_f), an integer below 2^41 in magnitude): six
  // signed base-256 digits, the pair's two columns of a plane per 2-byte store
#pragma unroll
  for (int m = 0; m < M; ++m) {
    double ss = 0.0;
#pragma unroll
    for (int q = 0; q < kHgWaves; ++q) ss += red[q][m];
    const float r = 1.0f / sqrt_rn((float)ss * (1.0f / (float)D) + 1e-5f);
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int p = tid + kHgThreads * j;
      if (p < PH) {
        uint32_t pk[6] = {0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          long long X = fx24(f2h(r16((h2f((uint16_t)(xp[m][j] >> (16 * h))) * r) * (h ? nf[j].y : nf[j].x))));
#pragma unroll
          for (int b = 0; b < 5; ++b) {
            const int d = (int)(int8_t)(X & 0xff);
            X = (X - d) >> 8;
            pk[b] |= (uint32_t)(d & 0xff) << (8 * h);
          }
          pk[5] |= (uint32_t)((int)X & 0xff) << (8 * h);
        }
#pragma unroll
        for (int b = 0; b < 6; ++b) *(uint16_t*)(hg_dg + (size_t)(m * 6 + b) * D + 2 * p) = (uint16_t)pk[b];
      }
    }
  }
  if constexpr (M == 3) load_slice(b0, 0);
  if constexpr (KP > 1 && M > 1) load_slice(b1, 1);
  lds_barrier();

  // the k steps: two MFMAs each (A = digit rows 4 m + b of tile 0 and 4 m + 4 + b of tile 1, zero
  // where there is no such digit; rows without a digit read plane 0 and are zeroed by a select)
  const int ma = rl >> 2, ba = rl & 3;
  const bool a0ok = ma < M, a1ok = ma < M && ba < 2;
  const int8_t* A0p = hg_dg + (size_t)(a0ok ? ma * 6 + ba : 0) * D + 16 * jg;
  const int8_t* A1p = hg_dg + (size_t)(a1ok ? ma * 6 + 4 + ba : 0) * D + 16 * jg;
  const i32x4 z4 = {0, 0, 0, 0};
  i32x4 acc0 = z4, acc1 = z4;
  auto mfma_slice = [&](const u32x4 (&bf)[8], int kp) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const i32x4 Bv = __builtin_bit_cast(i32x4, bf[s]);
      const i32x4 A0r = *(const i32x4*)(A0p + kp * kHKS + 64 * s);
      const i32x4 A1r = *(const i32x4*)(A1p + kp * kHKS + 64 * s);
      acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0ok ? A0r : z4, Bv, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1ok ? A1r : z4, Bv, acc1, 0, 0, 0);
    }
  };
#pragma unroll
  for (int kp = 0; kp < KP; ++kp) {
    if (kp % 2 == 0) {
      mfma_slice(b0, kp);
      if (kp + 2 < KP) load_slice(b0, kp + 2);
    } else {
      mfma_slice(b1, kp);
      if (kp + 2 < KP) load_slice(b1, kp + 2);
    }
  }

  // logits of the workgroup's rows, its (max, first index) pair per sequence, and the last
  // workgroup (ticket) reduces the pairs
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  if (jg < M && v < a.V) {
    const long long T = (long long)acc0[0] + ((long long)acc0[1] << 8) + ((long long)acc0[2] << 16) +
                        ((long long)acc0[3] << 24) + ((long long)acc1[0] << 32) + ((long long)acc1[1] << 40);
    const uint16_t lh = f2h((float)((double)T * 0x1p-24) * h2f(es));
    if (a.logits) a.logits[(size_t)jg * a.V + v] = lh;
    best = h2f(lh);
    bidx = v;
  }
  row_argmax_dpp(best, bidx);  // the 16 lanes of the sequence's row group
  if (rl == 0 && jg < M) {
    pv[wave][jg] = best;
    pix[wave][jg] = bidx;
  }
  lds_barrier();
  if (tid < M) {
    float b = pv[0][tid];
    int bi = pix[0][tid];
#pragma unroll
    for (int q = 1; q < kHgWaves; ++q) argmax_take(b, bi, pv[q][tid], pix[q][tid]);
    __hip_atomic_store(a.part_val + (size_t)tid * G + wg, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.part_idx + (size_t)tid * G + wg, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the pair has reached the device-coherent level
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(a.ticket, 1u) == (unsigned)(G - 1);
  __syncthreads();
  if (!is_last) return;
  argmax_pairs<kHgWaves, 1, kHeadMaxGroups / kHgGroups / 64>(a, M, G, next_tok);
  if (tid == 0) *a.ticket = 0u;
  __syncthreads();
  if (a.x_next) embed_next<false, kHgThreads>(a, next_tok, M, D);
}

template <int M, int KP>
static hipError_t launch_head_i8g_kp(const HeadArgs& a, int groups, hipStream_t s) {
  const size_t shm = (size_t)M * 6 * a.D;  // at most 120 KiB (M = 4, D = 5120)
  if (shm > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&head_i8g_kernel<M, KP>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  // the pair arrays hold `groups` pairs per row, the workgroups fewer
  hipLaunchKernelGGL((head_i8g_kernel<M, KP>), dim3((groups + kHgGroups - 1) / kHgGroups), dim3(kHgThreads), shm,
                     s, a, groups);
  return hipGetLastError();
}
template <int M>
static hipError_t launch_head_i8g(const HeadArgs& a, int groups, hipStream_t s) {
  if (a.D % kHKS) return hipErrorInvalidValue;  // whole 512-wide slices (the kernel's D is KP * 512)
  switch (a.D / kHKS) {
    case 1: return launch_head_i8g_kp<M, 1>(a, groups, s);
    case 2: return launch_head_i8g_kp<M, 2>(a, groups, s);
    case 3: return launch_head_i8g_kp<M, 3>(a, groups, s);
    case 4: return launch_head_i8g_kp<M, 4>(a, groups, s);
    case 5: return launch_head_i8g_kp<M, 5>(a, groups, s);
    case 6: return launch_head_i8g_kp<M, 6>(a, groups, s);
    case 7: return launch_head_i8g_kp<M, 7>(a, groups, s);
    case 8: return launch_head_i8g_kp<M, 8>(a, groups, s);
    case 9: return launch_head_i8g_kp<M, 9>(a, groups, s);
    case 10: return launch_head_i8g_kp<M, 10>(a, groups, s);
    default: return hipErrorInvalidValue;
  }
}

template <int M, bool F16>
static hipError_t launch_head_mf(const HeadArgs& a, int groups, size_t shm, hipStream_t s) {
  // dynamic LDS above 64 KiB needs an explicit opt-in (gfx950 has 160 KiB per workgroup)
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&head_kernel<M, F16>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((head_kernel<M, F16>), dim3(groups), dim3(256), shm, s, a);
  return hipGetLastError();
}

hipError_t launch_head(const HeadArgs& a, int M, hipStream_t s) {
  const int groups = (a.V + 63) / 64;
  if (M < 1 || M > 4 || groups > kHeadMaxGroups || a.D > 512 * kHeadMaxKP) return hipErrorInvalidValue;
  if (!a.f16) {
    switch (M) {
      case 1: return launch_head_i8g<1>(a, groups, s);
      case 2: return launch_head_i8g<2>(a, groups, s);
      case 3: return launch_head_i8g<3>(a, groups, s);
      default: return launch_head_i8g<4>(a, groups, s);
    }
  }
  // fp16 table: the rows' final-normed values sit in LDS as fp64 (8 D bytes per row, at most
  // 120 KiB), so wide models run the rows in launches of fewer rows, one after the other
  const size_t per_row = (size_t)a.D * sizeof(double);
  const int fit = (int)((120 * 1024) / per_row);
  if (fit < 1) return hipErrorInvalidValue;
  for (int r0 = 0; r0 < M; r0 += fit) {
    const int mr = M - r0 < fit ? M - r0 : fit;
    HeadArgs b = a;
    b.x = a.x + (size_t)r0 * a.D;
    b.logits = a.logits ? a.logits + (size_t)r0 * a.V : nullptr;
    b.next = a.next + r0;
    b.x_next = a.x_next ? a.x_next + (size_t)r0 * a.D : nullptr;
    hipError_t e;
    switch (mr) {
      case 1: e = launch_head_mf<1, true>(b, groups, per_row, s); break;
      case 2: e = launch_head_mf<2, true>(b, groups, 2 * per_row, s); break;
      case 3: e = launch_head_mf<3, true>(b, groups, 3 * per_row, s); break;
      default: e = launch_head_mf<4, true>(b, groups, 4 * per_row, s); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_embed(const EmbedArgs& a, int M, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_tile_emb(const uint8_t* src, uint8_t* dst, int V, int D, hipStream_t s) {
  const int v_pad = (V + 63) / 64 * 64;
  const size_t total = (size_t)v_pad * D / 4;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(tile_emb_kernel, dim3(blocks), dim3(256), 0, s, src, dst, V, D, v_pad);
  return hipGetLastError();
}


// ---------------------------------------------------------------------------------------------
// Exact int8 head for 5..64 rows (int8 table): the digit decomposition of the 1..4-row kernel as
// a tiled GEMM. head_digits_kernel computes the final RMSNorm of every row once and writes the
// six base-256 digit planes of X = xf 2^24, tiled for the A operand: tile t = b NH + h holds
// digit b of rows 16 h .. 16 h + 15, laid out [tile][16-byte k chunk][16 rows][16 bytes]
// (NH = ceil(M / 16); rows M .. 16 NH - 1 and the chunks past D are zero). head_i8s_kernel (below)
// multiplies them with the table on the int8 matrix cores: the accumulator layout
// D[4 (l / 16) + e][l % 16] of v_mfma_i32_16x16x64_i8 leaves lane l with all six digit sums S_b of
// (m = 16 h + 4 (l / 16) + e, v = 16 fragment + l % 16) in its own registers, T = sum_b S_b 256^b
// (int64) = sum_k X_k E[v][k] exactly, and the logit is fp16(fp32(T 2^-24) * s_E[v]) as in the
// 1..4-row kernel. The table streams from HBM once; the digit planes (6 * 16 NH * D bytes) from L2
// into each workgroup's LDS.
// ---------------------------------------------------------------------------------------------
// 16-byte k chunks per digit-plane row: D / 16 rounded up to whole groups of four 64-wide k steps
// (the rings run four steps per iteration without a tail; the padding is zero)
__host__ __device__ inline int digit_chunks(int D) { return (D / 64 + 3) / 4 * 4 * 4; }
size_t head_digit_bytes(int M, int D) { return (size_t)6 * 16 * ((M + 15) / 16) * digit_chunks(D) * 16; }

__global__ __launch_bounds__(256) void head_digits_kernel(const uint16_t* __restrict__ x,
                                                         const float* __restrict__ norm_f,
                                                         int8_t* __restrict__ dig, int M, int NH, int D) {
  __shared__ double red[4];
  const int m = blockIdx.x, tid = threadIdx.x;  // grid: 16 NH rows
  const int CH = D / 16, h = m >> 4, rr = m & 15;
  const int CHp = digit_chunks(D);  // the planes are zero past column D
  const uint16_t* xm = x + (size_t)(m < M ? m : 0) * D;
  // the first digit chunk of this thread (x and norm_f), loaded with the sum-of-squares pass so
  // that the digits need no second memory round trip (clamped in-bounds; chunks past D are zero)
  const int c0 = tid < CH ? tid : CH - 1;
  const u32x4 x00 = *(const u32x4*)(xm + 16 * c0), x01 = *(const u32x4*)(xm + 16 * c0 + 8);
  const f32x4* nfp0 = (const f32x4*)(norm_f + 16 * c0);
  const f32x4 n00 = nfp0[0], n01 = nfp0[1], n02 = nfp0[2], n03 = nfp0[3];
  float r = 0.0f;
  if (m < M) {  // uniform over the workgroup
    double ps = 0.0;
    for (int k = 8 * tid; k < D; k += 8 * 256) {
      const u32x4 xv = *(const u32x4*)(xm + k);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double v = (double)h2f((uint16_t)(xv[e >> 1] >> (16 * (e & 1))));
        ps += v * v;
      }
    }
    const double ss = block_sum_f64<256>(ps, red);
    r = 1.0f / sqrt_rn((float)ss * (1.0f / (float)D) + 1e-5f);
  }
  for (int c = tid; c < CHp; c += 256) {  // one 16-column chunk per thread
    uint32_t pk[6][4];
#pragma unroll
    for (int b = 0; b < 6; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) pk[b][j] = 0u;
    if (m < M && c < CH) {
      u32x4 x0 = x00, x1 = x01;
      f32x4 n4[4] = {n00, n01, n02, n03};
      if (c != tid) {  // the second and later chunks of a thread (D > 4096)
        x0 = *(const u32x4*)(xm + 16 * c);
        x1 = *(const u32x4*)(xm + 16 * c + 8);
        const f32x4* nfp = (const f32x4*)(norm_f + 16 * c);
        n4[0] = nfp[0]; n4[1] = nfp[1]; n4[2] = nfp[2]; n4[3] = nfp[3];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t w = i < 8 ? x0[i >> 1] : x1[(i - 8) >> 1];
        const float xv = h2f((uint16_t)(w >> (16 * (i & 1))));
        long long X = fx24(f2h(r16((xv * r) * n4[i >> 2][i & 3])));
#pragma unroll
        for (int b = 0; b < 5; ++b) {
          const int d = (int)(int8_t)(X & 0xff);
          X = (X - d) >> 8;
          pk[b][i >> 2] |= (uint32_t)(d & 0xff) << (8 * (i & 3));
        }
        pk[5][i >> 2] |= (uint32_t)((int)X & 0xff) << (8 * (i & 3));
      }
    }
#pragma unroll
    for (int b = 0; b < 6; ++b)
      *(u32x4*)(dig + (((size_t)(b * NH + h) * CHp + c) * 16 + rr) * 16) = u32x4{pk[b][0], pk[b][1], pk[b][2], pk[b][3]};
  }
}

// ---------------------------------------------------------------------------------------------
// head_i8s_kernel<NH>: the digit-plane GEMM of the batched exact head with the digit tiles staged
// in LDS. A workgroup of 8 waves owns a run of fragments (16 vocabulary rows each). The 16 NH
// activation rows are split into NRG row groups of NHW = NH / NRG row blocks (NRG = 2 at 64 rows,
// else 1); wave w computes row group w / (8 / NRG) against F fragments, so that each wave reads
// 6 NHW digit tiles per 64-wide k step from LDS for 6 NHW F MFMAs (at 64 rows in one group the
// 24-tile reads bound the loop). The digit tiles of CK k steps (all row blocks, 6 NH CK KiB) are
// copied into LDS by the whole workgroup one chunk ahead (double buffer, one barrier per chunk),
// so the waves read them through the LDS queue (lgkmcnt) instead of re-reading L2 through the
// vector-memory queue, where loads complete in issue order and a digit-tile wait was also a wait
// for the table loads issued before it. The table fragments (HBM) stream through a register ring
// kHsDB steps deep; between table loads the queue holds one batch of staging loads per chunk,
// issued a chunk before its use. Logits, argmax and the next embedding as in the other heads.
// ---------------------------------------------------------------------------------------------
constexpr int kHsWaves = 8, kHsThreads = 64 * kHsWaves, kHsDB = 4;  // steps per loop turn = kHsDB

__host__ __device__ constexpr int hs_nrg(int NH) { return NH == 4 ? 2 : 1; }                   // row groups
__host__ __device__ constexpr int hs_frags(int NH) { return NH / hs_nrg(NH) <= 2 ? 2 : 1; }    // fragments per wave
__host__ __device__ constexpr int hs_ck(int NH) { return NH <= 2 ? 4 : 2; }                    // k steps per chunk
__host__ __device__ constexpr int hs_wg_frags(int NH) { return kHsWaves / hs_nrg(NH) * hs_frags(NH); }
__host__ __device__ constexpr size_t hs_lds_bytes(int NH) { return (size_t)2 * 6 * NH * hs_ck(NH) * 1024; }

template <int NH>
__global__ __launch_bounds__(kHsThreads) __attribute__((amdgpu_waves_per_eu(2))) void head_i8s_kernel(HeadArgs a, int M) {
  constexpr int NRG = hs_nrg(NH), NHW = NH / NRG, WPG = kHsWaves / NRG;
  constexpr int F = hs_frags(NH), CK = hs_ck(NH);
  constexpr int NT = 6 * NH;                      // staged digit tiles per k step: tile t = b NH + h
  constexpr int NTW = 6 * NHW;                    // tiles of a wave's row group
  constexpr int AG = NTW <= 12 ? NTW : NTW / 2;   // tiles read from LDS at a time
  constexpr int CHUNK = NT * CK * 64;             // 16-byte vectors per staged chunk
  constexpr int SV = (CHUNK + kHsThreads - 1) / kHsThreads;
  constexpr int MP = 16 * NH;
  extern __shared__ __attribute__((aligned(16))) u32x4 abuf[];  // [2][NT][CK][64]
  __shared__ float wbest[kHsWaves][16 * NHW];
  __shared__ int widx[kHsWaves][16 * NHW];
  __shared__ bool is_last;
  __shared__ int next_tok[MP];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave / WPG, wf = wave % WPG;     // row group, fragment slot
  const int jg = lane >> 4, rl = lane & 15;
  const int D = a.D, CH = D / 16, KS = D / 64;
  const int nfr = (a.V + 15) / 16;                // fragments of 16 rows (the table has 64-row groups)
  const int CHp = digit_chunks(D);
  const int fb0 = (int)blockIdx.x * WPG * F + wf * F;  // this wave's first fragment
  // the wave's fragments (clamped into the table: past it a wave recomputes the last one and
  // discards the result) and their row scales (loaded first, used at the end)
  int fr[F];
  uint16_t sc[F];
#pragma unroll
  for (int f = 0; f < F; ++f) {
    fr[f] = fb0 + f < nfr ? fb0 + f : nfr - 1;
    const int v = 16 * fr[f] + rl;
    sc[f] = a.emb_scale[v < a.V ? v : a.V - 1];
  }
  // table fragment f at k step s: group g = fr / 4, rows 16 (fr % 4) + rl, 16-byte chunk 4 s + jg
  const char* Eb = (const char*)a.emb;
  auto tab = [&](int f, int s) -> const u32x4* {
    const int g = fr[f] >> 2;
    return (const u32x4*)(Eb + ((size_t)g * CH + 4 * s + jg) * 1024 + (size_t)((fr[f] & 3) * 16 + rl) * 16);
  };
  // staging: vector v of chunk c is tile t = v / (CK 64), step c CK + (v / 64) % CK, lane v % 64
  const char* Ab = (const char*)a.hdig;
  auto stage_load = [&](u32x4* sv, int c) {
#pragma unroll
    for (int i = 0; i < SV; ++i) {
      const int v0 = tid + kHsThreads * i, v = v0 < CHUNK ? v0 : CHUNK - 1;
      const int t = v / (CK * 64), r = v - t * (CK * 64);
      sv[i] = *(const u32x4*)(Ab + ((size_t)t * CHp + 4 * c * CK) * 256 + (size_t)r * 16);
    }
  };
  auto stage_store = [&](const u32x4* sv, int buf) {
#pragma unroll
    for (int i = 0; i < SV; ++i) {
      const int v = tid + kHsThreads * i;
      if (CHUNK % kHsThreads == 0 || v < CHUNK) abuf[buf * CHUNK + v] = sv[i];
    }
  };
  // accumulators: wave tile j = b NHW + hh is digit b of row block rg NHW + hh (LDS tile b NH + rg NHW + hh)
  i32x4 acc[NTW][F];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int f = 0; f < F; ++f) acc[t][f] = i32x4{0, 0, 0, 0};
  u32x4 Bf[kHsDB][F];
  u32x4 sv[SV];
  // prologue: chunk 0 staged (its loads first), the table steps 0 .. DB - 1 in flight
  stage_load(sv, 0);
#pragma unroll
  for (int d = 0; d < kHsDB; ++d)
#pragma unroll
    for (int f = 0; f < F; ++f) Bf[d][f] = ld_nt(tab(f, d < KS ? d : KS - 1));
  stage_store(sv, 0);
  lds_barrier();
  const int NC = KS / CK;
  // one loop turn = kHsDB k steps; the last turn issues no table loads (there is no step after
  // it: loads there would only delay the epilogue, and loads in a branch would make every chunk's
  // staging wait count on the fewest loads in flight, draining the ring)
  auto turn = [&](int it, auto last) {
    constexpr bool LAST = decltype(last)::value;
#pragma unroll
    for (int u = 0; u < kHsDB; ++u) {
      const int step = kHsDB * it + u;
      const int c = step / CK, buf = c & 1;
      if (u % CK == 0) {
        stage_load(sv, c + 1 < NC ? c + 1 : NC - 1);  // the next chunk
        // sched_barrier pins the loads where they are issued: the scheduler would otherwise sink
        // them to the end of the unrolled steps, and the next step's table wait would then
        // expose the whole load latency
        __builtin_amdgcn_sched_barrier(0);
      }
      const u32x4* At = abuf + buf * CHUNK + (step - c * CK) * 64 + lane;
#pragma unroll
      for (int j0 = 0; j0 < NTW; j0 += AG) {
        u32x4 A[AG];
#pragma unroll
        for (int j = 0; j < AG; ++j) {
          const int b = (j0 + j) / NHW, hh = (j0 + j) % NHW;
          A[j] = At[((b * NH + rg * NHW + hh) * CK) * 64];
        }
        // every read of the group issued before its MFMAs (the scheduler would otherwise reuse
        // two registers and wait an LDS round trip for every four MFMAs)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < AG; ++j)
#pragma unroll
          for (int f = 0; f < F; ++f)
            acc[j0 + j][f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, A[j]),
                                                                 __builtin_bit_cast(i32x4, Bf[u][f]), acc[j0 + j][f], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (!LAST) {
#pragma unroll
        for (int f = 0; f < F; ++f) Bf[u][f] = ld_nt(tab(f, step + kHsDB));
      }
      __builtin_amdgcn_sched_barrier(0);
      if (u % CK == CK - 1) {  // end of chunk c: the next chunk into the other buffer
        stage_store(sv, buf ^ 1);
        lds_barrier();
      }
    }
  };
#pragma nounroll
  for (int it = 0; it < KS / kHsDB - 1; ++it) turn(it, std::false_type{});
  turn(KS / kHsDB - 1, std::true_type{});

  // exact dot products: lane l holds activation rows 16 (rg NHW + hh) + 4 jg + e of vocabulary
  // rows 16 fr[f] + rl; T = sum_b S_b 256^b (int64)
  float best[NHW][4];
  int bidx[NHW][4];
#pragma unroll
  for (int hh = 0; hh < NHW; ++hh)
#pragma unroll
    for (int e = 0; e < 4; ++e) { best[hh][e] = -INFINITY; bidx[hh][e] = 0x7fffffff; }
#pragma unroll
  for (int f = 0; f < F; ++f) {
    const int v = 16 * (fb0 + f) + rl;
    const float svv = h2f(sc[f]);
#pragma unroll
    for (int hh = 0; hh < NHW; ++hh)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        long long T = 0;
#pragma unroll
        for (int b = 0; b < 6; ++b) T += (long long)acc[b * NHW + hh][f][e] << (8 * b);
        const int m = 16 * (rg * NHW + hh) + 4 * jg + e;
        if (fb0 + f < nfr && m < M && v < a.V) {
          const uint16_t lh = f2h((float)((double)T * 0x1p-24) * svv);
          if (a.logits) a.logits[(size_t)m * a.V + v] = lh;
          const float lv = h2f(lh);
          if (lv > best[hh][e]) { best[hh][e] = lv; bidx[hh][e] = v; }  // v increases with f
        }
      }
  }
#pragma unroll
  for (int hh = 0; hh < NHW; ++hh)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      row_argmax_dpp(best[hh][e], bidx[hh][e]);  // the 16 lanes of row group jg
      if (rl == 0) {
        wbest[wave][16 * hh + 4 * jg + e] = best[hh][e];
        widx[wave][16 * hh + 4 * jg + e] = bidx[hh][e];
      }
    }
  __syncthreads();
  const int NGW = (int)gridDim.x;
  if (tid < M) {  // row tid: the waves of its row group
    const int g = tid / (16 * NHW), rw = tid % (16 * NHW);
    float vb[WPG];
    int vi[WPG];
#pragma unroll
    for (int w = 0; w < WPG; ++w) { vb[w] = wbest[g * WPG + w][rw]; vi[w] = widx[g * WPG + w][rw]; }
    float b = vb[0];
    int bi = vi[0];
#pragma unroll
    for (int w = 1; w < WPG; ++w) argmax_take(b, bi, vb[w], vi[w]);
    __hip_atomic_store(a.part_val + (size_t)tid * NGW + blockIdx.x, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.part_idx + (size_t)tid * NGW + blockIdx.x, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the pairs have reached the device-coherent level
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(a.ticket, 1u) == (unsigned)(NGW - 1);
  __syncthreads();
  if (!is_last) return;
  argmax_pairs<kHsWaves, (MP + kHsWaves - 1) / kHsWaves, kHeadMaxGroups / 128>(a, M, NGW, next_tok);
  if (tid == 0) *a.ticket = 0u;
  __syncthreads();
  // the embedding in one round of loads up to 20 chunks per thread (64 rows of 2560 bytes)
  constexpr int KBE = (MP * 320 + kHsThreads - 1) / kHsThreads < 20 ? (MP * 320 + kHsThreads - 1) / kHsThreads : 20;
  if (a.x_next) embed_next<false, kHsThreads, KBE>(a, next_tok, M, D);
}

template <int NH>
static hipError_t launch_head_i8s(const HeadArgs& a, int M, hipStream_t s) {
  const size_t shm = hs_lds_bytes(NH);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&head_i8s_kernel<NH>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
  if (e != hipSuccess) return e;
  const int nfr = (a.V + 15) / 16, per = hs_wg_frags(NH);
  hipLaunchKernelGGL((head_i8s_kernel<NH>), dim3((nfr + per - 1) / per), dim3(kHsThreads), shm, s, a, M);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Batched head (M = 5..64): logits on the fp16 matrix cores, v_mfma_f32_16x16x32_f16. A = xf
// (fp16, 16 rows x 32 k), B = 16 vocabulary rows of the int8 table converted exactly to fp16 in
// registers. Products are exact; the sum is accumulated in fp32 (not exact -- the 1..4-row kernel
// above is). One workgroup (4 waves) owns 256 vocabulary rows (each wave 4 tiles of 16); xf is
// staged in LDS 512 columns at a time. Argmax as above: per-workgroup pairs, then the last
// workgroup to finish reduces them.
// ---------------------------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4m __attribute__((ext_vector_type(4)));

constexpr int kHT = 256;
constexpr int kHV = 256;   // vocabulary rows per workgroup
constexpr int kHK = 512;   // k chunk
constexpr int kHS = kHK + 8;  // LDS row stride of the xf tile (halves)

// xf[m] = fp16((x * r) * norm_f) for the batched head (one workgroup per row).
__global__ __launch_bounds__(256) void final_norm_kernel(const uint16_t* __restrict__ x, const float* __restrict__ norm_f,
                                                        uint16_t* __restrict__ xf, int D) {
  __shared__ double red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  const uint16_t* xm = x + (size_t)m * D;
  double ps = 0.0;
  for (int k = tid; k < D; k += 256) { const double v = (double)h2f(xm[k]); ps += v * v; }
  const double ss = block_sum_f64<256>(ps, red);
  const float var = (float)ss * (1.0f / (float)D);
  const float r = 1.0f / sqrt_rn(var + 1e-5f);
  for (int k = tid; k < D; k += 256) xf[(size_t)m * D + k] = f2h((h2f(xm[k]) * r) * norm_f[k]);
}

template <int MI, bool F16>
__global__ __launch_bounds__(kHT) void head_mfma_kernel(HeadArgs a, int M) {
  constexpr int MP = MI * 16;
  __shared__ __attribute__((aligned(16))) uint16_t xs[MP][kHS];
  __shared__ float wbest[4][MP];
  __shared__ int widx[4][MP];
  __shared__ bool is_last;
  __shared__ int next_tok[MP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int D = a.D, CH = F16 ? D / 8 : D / 16;
  const int v0 = blockIdx.x * kHV + wave * 64;
  const int vpad = (a.V + 63) / 64 * 64;

  f32x4m acc[4][MI];
#pragma unroll
  for (int vt = 0; vt < 4; ++vt)
#pragma unroll
    for (int ib = 0; ib < MI; ++ib) acc[vt][ib] = f32x4m{0.f, 0.f, 0.f, 0.f};

  for (int t = 0; t < D / kHK; ++t) {
    __syncthreads();
    for (int i = tid; i < MP * (kHK / 8); i += kHT) {  // 16-byte vectors of the xf chunk
      const int row = i / (kHK / 8), c8 = i % (kHK / 8);
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row < M) v = *(const u32x4*)(a.xf + (size_t)row * D + t * kHK + c8 * 8);
      *(u32x4*)&xs[row][c8 * 8] = v;
    }
    __syncthreads();
#pragma unroll 2
    for (int ks = 0; ks < kHK / 32; ++ks) {
      const int kl = ks * 32 + 8 * (lane >> 4);
      const int k = t * kHK + kl;
      f16x8 A[MI];
#pragma unroll
      for (int ib = 0; ib < MI; ++ib) A[ib] = *(const f16x8*)&xs[ib * 16 + (lane & 15)][kl];
#pragma unroll
      for (int vt = 0; vt < 4; ++vt) {
        const int v = v0 + vt * 16 + (lane & 15);
        // the tiled table holds V rounded up to 64 rows (zero padded); the last tile may pass it
        f16x8 B;
        if (F16) {
          const u32x4 e16 = v < vpad ? *(const u32x4*)(a.emb + (((size_t)(v >> 6) * CH + (k >> 3)) * 64 + (v & 63)) * 16)
                                     : u32x4{0u, 0u, 0u, 0u};
          B = __builtin_bit_cast(f16x8, e16);
        } else {
          const uint2 e8 = v < vpad ? *(const uint2*)(a.emb + (((size_t)(v >> 6) * CH + (k >> 4)) * 64 + (v & 63)) * 16 + (k & 15))
                                    : make_uint2(0u, 0u);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = e < 4 ? e8.x : e8.y;
            B[e] = (_Float16)(float)(int8_t)(w >> (8 * (e & 3)));
          }
        }
#pragma unroll
        for (int ib = 0; ib < MI; ++ib) acc[vt][ib] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[ib], B, acc[vt][ib], 0, 0, 0);
      }
    }
  }

  // logits and per-row best of this wave: element (vt, ib, j) is row m = 16 ib + 4 (lane/16) + j,
  // vocabulary v = v0 + 16 vt + lane % 16
  float best[MI][4];
  int bidx[MI][4];
#pragma unroll
  for (int ib = 0; ib < MI; ++ib)
#pragma unroll
    for (int j = 0; j < 4; ++j) { best[ib][j] = -INFINITY; bidx[ib][j] = 0x7fffffff; }
#pragma unroll
  for (int vt = 0; vt < 4; ++vt) {
    const int v = v0 + vt * 16 + (lane & 15);
    if (v >= a.V) continue;
    const float sc = F16 ? 1.0f : h2f(a.emb_scale[v]);
#pragma unroll
    for (int ib = 0; ib < MI; ++ib)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = ib * 16 + 4 * (lane >> 4) + j;
        if (m >= M) continue;
        const uint16_t lh = F16 ? f2h(acc[vt][ib][j]) : f2h(acc[vt][ib][j] * sc);
        if (a.logits) a.logits[(size_t)m * a.V + v] = lh;
        const float lv = h2f(lh);
        if (lv > best[ib][j]) { best[ib][j] = lv; bidx[ib][j] = v; }  // v increases with vt
      }
  }
  // reduce over the 16 lanes that share (lane / 16), then over the 4 waves
#pragma unroll
  for (int ib = 0; ib < MI; ++ib)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float b = best[ib][j];
      int bi = bidx[ib][j];
      row_argmax_dpp(b, bi);  // the 16 lanes of the row group
      if ((lane & 15) == 0) {
        const int m = ib * 16 + 4 * (lane >> 4) + j;
        wbest[wave][m] = b;
        widx[wave][m] = bi;
      }
    }
  __syncthreads();
  if (tid < M) {
    float b = wbest[0][tid];
    int bi = widx[0][tid];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float ob = wbest[w][tid];
      const int oi = widx[w][tid];
      if (ob > b || (ob == b && oi < bi)) { b = ob; bi = oi; }
    }
    a.part_val[(size_t)tid * gridDim.x + blockIdx.x] = b;
    a.part_idx[(size_t)tid * gridDim.x + blockIdx.x] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const unsigned tk = atomicAdd(a.ticket, 1u);
    is_last = (tk == gridDim.x - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int r0 = 0; r0 < MI * 4; r0 += 4)  // four rows per wave at a time (registers)
    argmax_pairs<4, 4, kHeadMaxGroups / 256>(a, M, (int)gridDim.x, next_tok, r0);
  if (tid == 0) *a.ticket = 0u;
  __syncthreads();
  if (a.x_next) embed_next<F16, kHT>(a, next_tok, M, D);
}

hipError_t launch_head_batched(const HeadArgs& a, int M, hipStream_t s) {
  if (M < 1 || M > 64 || a.D % kHK || (a.V + 63) / 64 > kHeadMaxGroups) return hipErrorInvalidValue;
  if (!a.f16) {  // int8 table: exact digit-plane GEMM
    if (!a.hdig) return hipErrorInvalidValue;
    const int nh = (M + 15) / 16;
    hipLaunchKernelGGL(head_digits_kernel, dim3(16 * nh), dim3(256), 0, s, a.x, a.norm_f, (int8_t*)a.hdig, M, nh, a.D);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (nh) {
      case 1: return launch_head_i8s<1>(a, M, s);
      case 2: return launch_head_i8s<2>(a, M, s);
      case 3: return launch_head_i8s<3>(a, M, s);
      default: return launch_head_i8s<4>(a, M, s);
    }
  }
  if (!a.xf) return hipErrorInvalidValue;
  hipLaunchKernelGGL(final_norm_kernel, dim3(M), dim3(256), 0, s, a.x, a.norm_f, (uint16_t*)a.xf, a.D);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int groups = (a.V + kHV - 1) / kHV;
  const int mi = (M + 15) / 16;
#define DFSSM_HEAD_MFMA(MI)                                                                        \
  if (mi == MI) {                                                                                 \
    if (a.f16) hipLaunchKernelGGL((head_mfma_kernel<MI, true>), dim3(groups), dim3(kHT), 0, s, a, M); \
    else hipLaunchKernelGGL((head_mfma_kernel<MI, false>), dim3(groups), dim3(kHT), 0, s, a, M);      \
  }
  DFSSM_HEAD_MFMA(1)
  DFSSM_HEAD_MFMA(2)
  DFSSM_HEAD_MFMA(3)
  DFSSM_HEAD_MFMA(4)
#undef DFSSM_HEAD_MFMA
  return hipGetLastError();
}

}  // namespace dfssm
