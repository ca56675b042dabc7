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
// E_i, then the tied tokens at the boundary key are kept in index order as far as the mass allows.
// Three kernels: sample_slice_kernel<0> and <1> split each sequence's vocabulary over NW
// workgroups (contiguous slices): the maxima of z, then e (to the sequence's e row), the exact
// partial normalizers and the partial first-pass histograms (the pass over every token, whose
// few populated bins make the per-wave atomics collide most); sample_kernel (one workgroup of
// 1024 threads per sequence) adds the partials and runs passes 2..4, the ties and the draw over
// the e row (L2-resident), read wave-contiguously: thread t owns the 16-byte vectors t, t + 1024,
// ... The partials occupy the sequence's first scratch row.
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kST = 1024;                  // threads per sequence (selection and draw)
constexpr int kSW = 256;                   // threads per slice workgroup
constexpr int kMaxSlices = 64;             // slice workgroups per sequence

// Slice workgroups per sequence: at most kMaxSlices, and the partials (maxima, normalizers and
// 256-bin histograms) must fit the first scratch row of rs = sample_row_floats(V) floats.
__host__ __device__ inline int sample_slices(int rs) {
  const int n = (rs * 4 - 1024) / 2048;
  return n < 1 ? 1 : (n > kMaxSlices ? kMaxSlices : n);
}
// partials in the first row: maxima (float[NW]) at byte 0, normalizers (u64[NW]) at byte 256,
// histograms (u64[NW][256]) at byte 1024
__device__ __forceinline__ float* part_max(float* row0) { return row0; }
__device__ __forceinline__ unsigned long long* part_z(float* row0) { return (unsigned long long*)((char*)row0 + 256); }
__device__ __forceinline__ unsigned long long* part_hist(float* row0) {
  return (unsigned long long*)((char*)row0 + 1024);
}

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

// PHASE 0: the maximum of z over the slice; PHASE 1: e = exp(z - max z) of the slice to the e row
// (the last slice also zeroes the padding up to ld), its exact normalizer and first-pass histogram.
// Slice w of NW: tokens [w SL, min(V, (w + 1) SL)), SL = ceil(V / NW).
template <int PHASE>
__global__ __launch_bounds__(kSW) void sample_slice_kernel(SampleArgs a) {
  __shared__ unsigned long long hist[kSW / 64][256];
  __shared__ float redf[kSW / 64];
  __shared__ long long redl[kSW / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sw = blockIdx.x, b = blockIdx.y, V = a.V;
  const int ld = (V + 3) / 4 * 4, rs = sample_row_floats(V);
  const int NW = sample_slices(rs), SL = (V + NW - 1) / NW;
  const int lo = sw * SL, hi = lo + SL < V ? lo + SL : V;
  const uint16_t* lg = a.logits + (size_t)b * V;
  const int* cn = a.counts + (size_t)b * V;
  float* row0 = a.escratch + (size_t)b * 2 * rs;
  float* er = row0 + rs;
  if (PHASE == 0) {
    float m = -INFINITY;
    for (int i = lo + tid; i < hi; i += kSW) m = fmaxf(m, penalized(h2f(lg[i]), cn[i], a));
    const float wm = wave_max_dpp_f32(m);
    if (lane == 0) redf[w] = wm;
    __syncthreads();
    if (tid == 0) {
      float t = redf[0];
      for (int k = 1; k < kSW / 64; ++k) t = fmaxf(t, redf[k]);
      part_max(row0)[sw] = t;
    }
    return;
  }
  for (int q = tid; q < (kSW / 64) * 256; q += kSW) (&hist[0][0])[q] = 0ull;
  float m = part_max(row0)[0];
  for (int k = 1; k < NW; ++k) m = fmaxf(m, part_max(row0)[k]);
  __syncthreads();
  long long zs = 0;
  for (int i = lo + tid; i < hi; i += kSW) {
    const float e = dev_expf(penalized(h2f(lg[i]), cn[i], a) - m);
    er[i] = e;
    const unsigned long long E = fixed40(e);
    zs += (long long)E;
    if (E != 0ull) atomicAdd(&hist[w][__builtin_bit_cast(uint32_t, e) >> 24], E);
  }
  if (sw == NW - 1)
    for (int i = V + tid; i < ld; i += kSW) er[i] = 0.0f;
  const long long Zw = block_sum_ll<kSW>(zs, redl);  // (its barriers also publish hist)
  if (tid == 0) part_z(row0)[sw] = (unsigned long long)Zw;
  if (tid < 256) {  // 256 bins, one per thread
    unsigned long long t = 0;
    for (int k = 0; k < kSW / 64; ++k) t += hist[k][tid];
    part_hist(row0)[(size_t)sw * 256 + tid] = t;
  }
}

__global__ __launch_bounds__(kST) void sample_kernel(SampleArgs a) {
  __shared__ unsigned long long hist[kST / 64][256];  // one histogram per wave: fewer colliding atomics
  __shared__ long long redl[kST / 64];
  __shared__ unsigned long long sel[2];  // mass above the chosen bin (d > 0), (d = 0)
  __shared__ unsigned long long wtot[4];
  __shared__ int dsel;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int b = blockIdx.x, V = a.V;
  const int ld = (V + 3) / 4 * 4;
  const int nv4 = (ld / 4 + kST - 1) / kST;  // vectors per thread
  const int rs = sample_row_floats(V), NW = sample_slices(rs);
  float* row0 = a.escratch + (size_t)b * 2 * rs;  // the slices' partials
  float* er = row0 + rs;                          // e = exp(z - max z)
  // the exact normalizer, the sum of the slices' (every partial is an integer: any order)
  __shared__ unsigned long long zsum, hsum[4][256];
  if (w == 0) {
    unsigned long long zp = lane < NW ? part_z(row0)[lane] : 0ull;
    for (int off = 32; off > 0; off >>= 1) {
      const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)zp, off, 64);
      const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(zp >> 32), off, 64);
      zp += ((unsigned long long)hi << 32) | lo;
    }
    if (lane == 0) zsum = zp;
  }
  {  // the first pass's histogram: thread t adds bin t % 256 over slices t / 256, + 4, ...
    unsigned long long hp = 0;
    for (int k = tid >> 8; k < NW; k += 4) hp += part_hist(row0)[(size_t)k * 256 + (tid & 255)];
    hsum[tid >> 8][tid & 255] = hp;
  }
  __syncthreads();
  const unsigned long long Z = zsum;
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
      if (pass == 0 && tid < 256)  // the first pass's histogram: the slices' partials, summed above
        hist[0][tid] = (hsum[0][tid] + hsum[1][tid]) + (hsum[2][tid] + hsum[3][tid]);
#pragma unroll 1
      for (int c = 0; c < (pass == 0 ? 0 : nv4); c += 4) {
        float v[16];
        load4(er, ld, c, v);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t key = __builtin_bit_cast(uint32_t, v[j]);
          if (c + j / 4 < nv4 && tok_of(c, j) < V && (key & pmask) == prefix) {  // few match past pass 1
            const unsigned long long E = fixed40(v[j]);
            if (E != 0ull) atomicAdd(&hist[w][(key >> shift) & 255u], E);
          }
        }
      }
      __syncthreads();
      // the digit d whose bin holds the first token past the mass limit, scanning bins from 255
      // down: the largest d >= 1 with above + (mass of bins >= d) > thr, else 0; the new mass
      // above = above + (mass of bins > d). Thread t < 256 holds bin t: the waves' histograms
      // summed, then suffix sums within each wave (shuffles) and across the four waves (LDS).
      unsigned long long h = 0, incl = 0;
      if (tid < 256) {
        for (int k = 0; k < kST / 64; ++k) h += hist[k][tid];
        incl = h;
        for (int off = 1; off < 64; off <<= 1) {
          const uint32_t lo = (uint32_t)__shfl_down((int)(uint32_t)incl, off, 64);
          const uint32_t hi = (uint32_t)__shfl_down((int)(uint32_t)(incl >> 32), off, 64);
          if (lane + off < 64) incl += ((unsigned long long)hi << 32) | lo;
        }
        if (lane == 0) wtot[w] = incl;  // bins 64 w .. 64 w + 63
        if (tid == 0) dsel = 0;
      }
      __syncthreads();
      if (tid < 256) {
        for (int k = w + 1; k < 4; ++k) incl += wtot[k];
        const unsigned long long in = above + incl, ex = in - h;  // bins >= tid, bins > tid
        if (tid == 0) sel[1] = ex;                                // the d = 0 case
        if (tid >= 1 && in > thr && ex <= thr) {                  // at most one such bin
          dsel = tid;
          sel[0] = ex;
        }
      }
      __syncthreads();
      const int d = dsel;
      above = d > 0 ? sel[0] : sel[1];
      prefix |= (uint32_t)d << shift;
      pmask |= 255u << shift;
      __syncthreads();  // sel and dsel are rewritten by the next pass
    }
    kb = prefix;
    // the tokens with key kb, in index order, stay while the mass above them is <= thr: all of
    // them unless more tie than the mass allows; then ib = the index of the nkeep-th of them
    // (ties are common: fp16 logits take few distinct values). Index order is slab order, then
    // thread order within a slab: one pass counts each thread's ties per slab, the slab totals
    // give the slab holding the nkeep-th tie, a scan over that slab's threads the thread, and the
    // thread its token.
    const unsigned long long eb = fixed40(__builtin_bit_cast(float, kb));
    const long long nkeep = eb ? (long long)((thr - above) / eb) + 1 : (long long)V;  // eb > 0 by construction
    constexpr int kSl = kSampleMaxVocab / (4 * kST);
    int tcnt[kSl];
#pragma unroll
    for (int k = 0; k < kSl; ++k) tcnt[k] = 0;
#pragma unroll
    for (int c = 0; c < kSl; c += 4) {
      if (c < nv4) {
        float v[16];
        load4(er, ld, c, v);
#pragma unroll
        for (int j = 0; j < 16; ++j)
          tcnt[c + j / 4] += (c + j / 4 < nv4 && tok_of(c, j) < V && __builtin_bit_cast(uint32_t, v[j]) == kb) ? 1 : 0;
      }
    }
    __shared__ int slab_ties[kST / 64][kSl];
    __shared__ int tie_pick[2];  // slab, rank of the wanted tie within it (1-based)
#pragma unroll
    for (int k = 0; k < kSl; ++k) {
      const int ws = wave_sum_dpp_i32(tcnt[k]);
      if (lane == 0) slab_ties[w][k] = ws;
    }
    __shared__ int slab_tot[kSl];
    __syncthreads();
    if (tid < kSl) {
      int t = 0;
      for (int q = 0; q < kST / 64; ++q) t += slab_ties[q][tid];
      slab_tot[tid] = t;
    }
    __syncthreads();
    if (tid == 0) {
      long long cum = 0;
      int ks = -1;
      long long rank = 0;
      for (int k = 0; k < kSl && ks < 0; ++k) {
        if (cum + slab_tot[k] >= nkeep) {
          ks = k;
          rank = nkeep - cum;
        }
        cum += slab_tot[k];
      }
      tie_pick[0] = ks;  // -1: no more ties than nkeep, every tie is kept
      tie_pick[1] = (int)rank;
    }
    __syncthreads();
    const int ks = tie_pick[0], rank = tie_pick[1];
    if (ks >= 0) {  // exclusive scan of the threads' ties in slab ks (thread order = index order)
      int mine = 0;
#pragma unroll
      for (int k = 0; k < kSl; ++k)
        if (k == ks) mine = tcnt[k];
      int incl = mine;
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
      }
      if (lane == 63) slab_ties[w][0] = incl;
      __syncthreads();
      int base = 0;
      for (int q = 0; q < w; ++q) base += slab_ties[q][0];
      const int excl = base + incl - mine;
      if (mine > 0 && excl < rank && rank <= excl + mine) {  // exactly one thread
        const int q = tid + kST * ks, last = ld / 4 - 1;
        const f32x4 x = *(const f32x4*)(er + 4 * (q < last ? q : last));
        int seen = excl;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float xt = x[t];  // through a scalar (see the draw below)
          if (4 * q + t < V && __builtin_bit_cast(uint32_t, xt) == kb && ++seen == rank) tie_pick[1] = -(4 * q + t) - 1;
        }
      }
      __syncthreads();
      ib = -tie_pick[1] - 1;
    }
  }
  // inverse-CDF draw in index order (slab k = tokens 4096 k .. 4096 k + 4095, then thread, then
  // element): kept mass per slab (exact in fp64: slab sums < 2^53), the slab, the thread by a
  // scan of the slab's per-thread masses, the token within the thread
  constexpr int kSlabs = kSampleMaxVocab / (4 * kST);
  __shared__ double slab_w[kST / 64][kSlabs];
  __shared__ unsigned long long slab_t[kSlabs];
  __shared__ int pick[2];  // slab, thread
  __shared__ unsigned long long rem_s;
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
  const int NW = sample_slices(sample_row_floats(a.V));
  hipLaunchKernelGGL(sample_slice_kernel<0>, dim3(NW, batch), dim3(kSW), 0, s, a);
  hipLaunchKernelGGL(sample_slice_kernel<1>, dim3(NW, batch), dim3(kSW), 0, s, a);
  hipLaunchKernelGGL(sample_kernel, dim3(batch), dim3(kST), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
