// Sampling head (gfx950): temperature, repetition penalty and top-p (nucleus) sampling of the
// next token from the fp16 logits, one workgroup of 1024 threads per sequence, with the chosen
// token counted in the sequence's occurrence counts and, optionally, embedded as the next input.
//
// Reference semantics: eval/gen_test.py:54-95 (logits / T, then logits[seen] / r for every token
// seen so far, softmax, sort descending, drop a token when the probability mass ranked above it
// exceeds top_p, renormalize, multinomial) and training/df_ssm_mamba2_distill_dfw.py:1066-1078
// (for every earlier occurrence: positive logits / r, others * r; then softmax(logits / T); the
// same top-p rule). torch's multinomial RNG cannot be reproduced, so the draw is defined here,
// deterministically, and the oracle restates it:
//   z_i      the penalized, tempered logit (mode 0: gen_test order; mode 1: training order), fp32
//   e_i      = exp(z_i - max z) (this build's exp), E_i = floor(e_i 2^40) as an integer, so the
//            normalizer Z = sum E_i and every partial sum are exact, whatever the order
//   rank     by e_i descending, index ascending; token i is kept iff the sum of E over the tokens
//            ranked above it is <= floor(top_p Z) (top_p >= 1: all kept)
//   draw     inverse CDF in index order on the exact masses: S = sum of E over the kept tokens,
//            R = floor(h S / 2^64) with h = splitmix64 (Steele, Lea, Flood 2014) of
//            (seed, sequence, step); the token is the first kept index whose cumulative kept
//            mass exceeds R -- a draw from the renormalized top-p distribution (as
//            torch.multinomial on the renormalized sorted probabilities, gen_test.py:81-85),
//            with one random number per draw.
// The kept set is found without sorting: a 4-pass radix select (8 bits per pass, MSB first) over
// the fp32 bit patterns of e_i (positive floats order as integers) with exact 64-bit bin sums of
// E_i in LDS, then the tied tokens at the boundary key are kept in index order as far as the
// mass allows. z and e live in two workspace rows of the sequence (L2-resident between passes),
// read wave-contiguously: thread t owns the 16-byte vectors t, t + 1024, ...
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kST = 1024;                  // threads per sequence

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ float penalized(float l, int cnt, const SampleArgs& a) {
  if (a.mode == 0) {  // gen_test.py:71-74: logits / T, then seen tokens / r
    float z = l / a.temperature;
    return cnt > 0 ? z / a.penalty : z;
  }
  float z = l;  // distill_dfw.py:1069-1072: once per occurrence, by sign; then / T (:1073)
  for (int k = 0; k < cnt; ++k) z = z > 0.0f ? z / a.penalty : z * a.penalty;
  return z / a.temperature;
}

// floor(e 2^40) for 0 <= e <= 1, from the bits (e 2^40 is exact; the integer part is the shifted
// significand)
__device__ __forceinline__ uint64_t fixed40(float e) {
  const uint32_t b = __builtin_bit_cast(uint32_t, e);
  const int ex = (int)(b >> 23);
  const uint64_t mant = (uint64_t)((b & 0x7fffffu) | 0x800000u);
  const int sh = ex - 110;  // e 2^40 = mant 2^(ex - 127 - 23 + 40)
  if (ex == 0 || sh <= -24) return 0ull;
  return sh >= 0 ? mant << sh : mant >> (-sh);
}

// Element j of a thread's vector k is token 4 (tid + kST k) + j: every wave-wide access to a
// scratch row (stride ld floats, a multiple of 4) covers 1 KiB contiguous. A thread holds
// nv4 = ceil(ld / (4 kST)) vectors; chunks of four are loaded before any is used (vectors past
// the row re-read its last one; their elements are excluded by index).
__device__ __forceinline__ void load4(const float* row, int ld, int c, float (&v)[16]) {
  const int tid = threadIdx.x, last = ld / 4 - 1;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int q = tid + kST * (c + k);
    const f32x4 x = *(const f32x4*)(row + 4 * (q < last ? q : last));
    v[4 * k] = x[0]; v[4 * k + 1] = x[1]; v[4 * k + 2] = x[2]; v[4 * k + 3] = x[3];
  }
}
__device__ __forceinline__ int tok_of(int c, int j) { return 4 * ((int)threadIdx.x + kST * (c + j / 4)) + (j & 3); }

template <int NT>
__device__ __forceinline__ long long block_sum_ll(long long v, long long* red) {
  for (int off = 32; off > 0; off >>= 1) {
    const int lo = __shfl_xor((int)(uint32_t)v, off, 64);
    const int hi = __shfl_xor((int)(uint32_t)((unsigned long long)v >> 32), off, 64);
    v += (long long)(((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo);
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  long long t = 0;
  for (int k = 0; k < NT / 64; ++k) t += red[k];
  return t;
}

__global__ __launch_bounds__(kST) void sample_kernel(SampleArgs a) {
  __shared__ unsigned long long hist[kST / 64][256];  // one histogram per wave: fewer colliding atomics
  __shared__ float redf[kST / 64];
  __shared__ long long redl[kST / 64];
  __shared__ unsigned long long sel[2];  // radix prefix, mass above it
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int b = blockIdx.x, V = a.V;
  const int ld = (V + 3) / 4 * 4;
  const int nv4 = (ld / 4 + kST - 1) / kST;  // vectors per thread
  const uint16_t* lg = a.logits + (size_t)b * V;
  const int* cn = a.counts + (size_t)b * V;
  float* zr = a.escratch + (size_t)b * 2 * ld;  // z, and e = exp(z - max z)
  float* er = zr + ld;

  // z (padding: -inf) to the z row, and its maximum
  float m = -INFINITY;
#pragma unroll 1
  for (int c = 0; c < nv4; c += 4) {
    uint16_t l16[16];
    int cc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = tok_of(c, j);
      l16[j] = lg[i < V ? i : V - 1];
      cc[j] = cn[i < V ? i : V - 1];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float z4[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int i = tok_of(c, 4 * k + t);
        z4[t] = (c + k < nv4 && i < V) ? penalized(h2f(l16[4 * k + t]), cc[4 * k + t], a) : -INFINITY;
        m = fmaxf(m, z4[t]);
      }
      const int q = tid + kST * (c + k);
      if (c + k < nv4 && 4 * q < ld) *(f32x4*)(zr + 4 * q) = f32x4{z4[0], z4[1], z4[2], z4[3]};
    }
  }
  {
    const float wm = wave_max_dpp_f32(m);
    if (lane == 0) redf[w] = wm;
    __syncthreads();
    m = redf[0];
    for (int k = 1; k < kST / 64; ++k) m = fmaxf(m, redf[k]);
  }
  // e = exp(z - max z) to the e row (padding 0), and the exact normalizer
  long long zs = 0;
#pragma unroll 1
  for (int c = 0; c < nv4; c += 4) {
    float v[16];
    load4(zr, ld, c, v);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float e4[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        e4[t] = dev_expf(v[4 * k + t] - m);
        zs += (c + k < nv4 && tok_of(c, 4 * k + t) < V) ? (long long)fixed40(e4[t]) : 0ll;
      }
      const int q = tid + kST * (c + k);
      if (c + k < nv4 && 4 * q < ld) *(f32x4*)(er + 4 * q) = f32x4{e4[0], e4[1], e4[2], e4[3]};
    }
  }
  const unsigned long long Z = (unsigned long long)block_sum_ll<kST>(zs, redl);
  const unsigned long long thr = (unsigned long long)((double)a.top_p * (double)Z);
  uint32_t kb = 0;  // boundary key and last kept index among its ties; all kept: 0 and V
  int ib = V;
  if (a.top_p < 1.0f && thr < Z) {
    uint32_t prefix = 0, pmask = 0;
    unsigned long long above = 0;
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      for (int q = tid; q < (kST / 64) * 256; q += kST) (&hist[0][0])[q] = 0ull;
      __syncthreads();
#pragma unroll 1
      for (int c = 0; c < nv4; c += 4) {
        float v[16];
        load4(er, ld, c, v);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t key = __builtin_bit_cast(uint32_t, v[j]);
          const unsigned long long E = fixed40(v[j]);
          if (c + j / 4 < nv4 && tok_of(c, j) < V && (key & pmask) == prefix && E != 0ull)
            atomicAdd(&hist[w][(key >> shift) & 255u], E);
        }
      }
      __syncthreads();
      if (tid < 256) {  // the waves' histograms summed into histogram 0
        unsigned long long t = hist[0][tid];
        for (int k = 1; k < kST / 64; ++k) t += hist[k][tid];
        hist[0][tid] = t;
      }
      __syncthreads();
      if (tid == 0) {  // the digit whose bin holds the first token past the mass limit
        unsigned long long R = above;
        int d = 255;
        for (; d > 0; --d) {
          if (R + hist[0][d] > thr) break;
          R += hist[0][d];
        }
        sel[0] = prefix | ((uint32_t)d << shift);
        sel[1] = R;
      }
      __syncthreads();
      prefix = (uint32_t)sel[0];
      above = sel[1];
      pmask |= 255u << shift;
    }
    kb = prefix;
    // the tokens with key kb, in index order, stay while the mass above them is <= thr: all of
    // them unless more tie than the mass allows; then the nkeep-th smallest index among them by
    // bisection over the index (rare: equal fp32 probabilities at the cut)
    const unsigned long long eb = fixed40(__builtin_bit_cast(float, kb));
    const long long nkeep = eb ? (long long)((thr - above) / eb) + 1 : (long long)V;  // eb > 0 by construction
    int lo_i = 0, hi_i = V - 1;  // invariant: the answer is in [lo_i, hi_i]
    for (int it = 0; it < 32; ++it) {
      const int mid = it == 0 ? V - 1 : (lo_i + hi_i) / 2;
      long long cnt = 0;
#pragma unroll 1
      for (int c = 0; c < nv4; c += 4) {
        float v[16];
        load4(er, ld, c, v);
#pragma unroll
        for (int j = 0; j < 16; ++j)
          cnt += (c + j / 4 < nv4 && tok_of(c, j) <= mid && tok_of(c, j) < V &&
                  __builtin_bit_cast(uint32_t, v[j]) == kb) ? 1 : 0;
      }
      cnt = block_sum_ll<kST>(cnt, redl);  // ties with index <= mid
      if (it == 0) {
        if (cnt <= nkeep) break;  // every tie is kept: ib = V
        continue;
      }
      if (cnt >= nkeep) hi_i = mid; else lo_i = mid + 1;
      if (lo_i == hi_i) {
        ib = lo_i;
        break;
      }
    }
  }
  // inverse-CDF draw in index order (slab k = tokens 4096 k .. 4096 k + 4095, then thread, then
  // element): kept mass per slab (exact in fp64: slab sums < 2^53), the slab, the thread by a
  // scan of the slab's per-thread masses, the token within the thread
  constexpr int kSlabs = kSampleMaxVocab / (4 * kST);
  double slab[kSlabs];
#pragma unroll
  for (int k = 0; k < kSlabs; ++k) slab[k] = 0.0;
#pragma unroll
  for (int c = 0; c < kSlabs; c += 4) {
    if (c < nv4) {
      float v[16];
      load4(er, ld, c, v);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int i = tok_of(c, j);
        const uint32_t key = __builtin_bit_cast(uint32_t, v[j]);
        if (c + j / 4 < nv4 && i < V && (key > kb || (key == kb && i <= ib))) slab[c + j / 4] += (double)fixed40(v[j]);
      }
    }
  }
  __shared__ double slab_w[kST / 64][kSlabs];
  __shared__ unsigned long long slab_t[kSlabs];
  __shared__ int pick[2];  // slab, thread
  __shared__ unsigned long long rem_s;
#pragma unroll
  for (int k = 0; k < kSlabs; ++k) {
    const double ws = wave_sum_dpp_f64(slab[k]);
    if (lane == 0) slab_w[w][k] = ws;
  }
  __syncthreads();
  if (tid < kSlabs) {
    double t = 0.0;
    for (int k = 0; k < kST / 64; ++k) t += slab_w[k][tid];
    slab_t[tid] = (unsigned long long)t;
  }
  __syncthreads();
  if (tid == 0) {
    unsigned long long S = 0;
    for (int k = 0; k < kSlabs; ++k) S += slab_t[k];
    const uint64_t h = splitmix64(a.seed ^ (((uint64_t)b << 40) | ((uint64_t)(a.step[b] & 0x7fffffu) << 17) | 0x1ffffull));
    unsigned long long R = __umul64hi(h, S);  // uniform in [0, S)
    int k = 0;
    while (k < kSlabs - 1 && R >= slab_t[k]) R -= slab_t[k++];
    pick[0] = k;
    rem_s = R;
  }
  __syncthreads();
  const int ks = pick[0];
  // this thread's kept masses in slab ks, and the exclusive scan over the threads
  unsigned long long em[4];
  unsigned long long mine = 0;
  {
    const int q = tid + kST * ks, last = ld / 4 - 1;
    const f32x4 x = *(const f32x4*)(er + 4 * (q < last ? q : last));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int i = 4 * q + t;
      // through a scalar: hipcc 7.2 bit-casts an element of an ext_vector_type as element 0
      const float xt = x[t];
      const uint32_t key = __builtin_bit_cast(uint32_t, xt);
      em[t] = (ks < nv4 && i < V && (key > kb || (key == kb && i <= ib))) ? fixed40(xt) : 0ull;
      mine += em[t];
    }
  }
  double incl = (double)mine;  // < 2^53: exact
  for (int off = 1; off < 64; off <<= 1) {
    const double t = __shfl_up(incl, off, 64);
    if (lane >= off) incl += t;
  }
  if (lane == 63) slab_w[w][0] = incl;
  __syncthreads();
  double wbase = 0.0;
  for (int k = 0; k < w; ++k) wbase += slab_w[k][0];
  const unsigned long long excl = (unsigned long long)(wbase + incl) - mine;
  const unsigned long long R = rem_s;
  if (mine > 0 && excl <= R && R < excl + mine) {  // exactly one thread
    unsigned long long acc = excl;
    int tok = 4 * (tid + kST * ks);
#pragma unroll
    for (int t = 0; t < 4; ++t) {  // the first token whose cumulative mass exceeds R
      if (R < acc + em[t]) {
        tok = 4 * (tid + kST * ks) + t;
        break;
      }
      acc += em[t];
    }
    a.next[b] = tok;
    a.counts[(size_t)b * V + tok] += 1;
    a.step[b] += 1u;
  }
}

hipError_t launch_sample(const SampleArgs& a, int batch, hipStream_t s) {
  if (a.V < 1 || a.V > kSampleMaxVocab) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_kernel, dim3(batch), dim3(kST), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
