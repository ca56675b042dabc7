// Sampling head (gfx950): temperature, repetition penalty and top-p (nucleus) sampling of the
// next token from the fp16 logits, with the chosen token counted in the sequence's occurrence
// counts.
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
// E_i; the tokens tied at the boundary key kb are kept in index order as far as the mass allows.
//
// Every pass over the vocabulary runs on NW slice workgroups per sequence (contiguous slices of at
// most 1024 tokens), one launch per pass, so that no pass is bound by one CU's VALU issue:
//   max    the slice maxima of z; slice 0 clears the sequence's global sums
//   exp    e_i to the sequence's e row, the normalizer Z and the histogram of the keys' top byte,
//          summed into global memory with 64-bit atomics (integers: any order)
//   pass p = 1..3: digit p - 1 from the global histogram of pass p - 1 and the selection the
//          previous launch stored (computed alike by every workgroup, stored by the first), then
//          the histogram of byte p of the keys that match the selection
//   mass   the last digit, i.e. kb; per slice the exact mass of the keys above kb and the count
//          of keys equal to kb
//   draw   one workgroup per sequence: the ties kept per slice (in slice order, i.e. index
//          order), the kept masses per slice, the slice holding R, and within it the token by
//          block scans of its tied and kept tokens.
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kSW = 256;          // threads per slice workgroup (and per draw workgroup)
constexpr int kMaxSlices = 64;    // slice workgroups per sequence
constexpr int kSliceMin = 512;    // fewer slices for small vocabularies: at least this many tokens each

// Slices per sequence: ceil(V / 512), at most 64, so a slice holds at most 1024 tokens (V <= 65536).
__host__ __device__ inline int sample_slices(int V) {
  const int n = (V + kSliceMin - 1) / kSliceMin;
  return n < 1 ? 1 : (n > kMaxSlices ? kMaxSlices : n);
}

// The selection so far: the key prefix of the digits chosen, its mask, and the exact mass of the
// tokens whose keys rank above the prefix.
struct Sel {
  uint32_t prefix, pmask;
  unsigned long long above;
};

// The sequence's first scratch row (byte offsets): slice maxima float[64] at 0, the normalizer Z
// (u64) at 256, the four pass histograms u64[4][256] at 512, the slices' masses above kb u64[64]
// at 8704, their counts of keys equal to kb int[64] at 9216, and the selections after k digits
// Sel[k - 1], k = 1..4, at 9472 (9536 bytes; a row has at least 2560 floats). A launch reads the
// slot the previous one wrote and writes the next: its workgroups never read what it writes.
struct SampleRow {
  float* maxs;
  unsigned long long* Z;
  unsigned long long* hist;  // [4][256]
  unsigned long long* mass;
  int* ties;
  Sel* sel;  // [4]: after 1, 2, 3, 4 digits
};
__device__ __forceinline__ SampleRow sample_row(float* row0) {
  char* c = (char*)row0;
  return SampleRow{(float*)c, (unsigned long long*)(c + 256), (unsigned long long*)(c + 512),
                   (unsigned long long*)(c + 8704), (int*)(c + 9216), (Sel*)(c + 9472)};
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

// One radix digit (a 256-thread workgroup; every workgroup of a launch computes the same): from
// the global histogram `hist` of pass p over the keys matching the selection `r` of passes
// 0 .. p - 1, with thread t holding bin t, the digit is the largest d >= 1 with
// r.above + (mass of bins >= d) > thr, else 0; the new mass above is r.above + (mass of bins > d).
struct SelLds {
  unsigned long long wtot[kSW / 64];
  unsigned long long sel;
  int dsel;
};
__device__ Sel select_digit(const unsigned long long* hist, Sel r, int p, unsigned long long thr, SelLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int shift = 24 - 8 * p;
  const unsigned long long h = hist[tid];
  unsigned long long incl = h;  // suffix sums: bins >= tid within the wave
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_down((int)(uint32_t)incl, off, 64);
    const uint32_t hi = (uint32_t)__shfl_down((int)(uint32_t)(incl >> 32), off, 64);
    if (lane + off < 64) incl += ((unsigned long long)hi << 32) | lo;
  }
  if (lane == 0) L.wtot[w] = incl;  // bins 64 w .. 64 w + 63
  if (tid == 0) L.dsel = 0;
  __syncthreads();
  for (int k = w + 1; k < kSW / 64; ++k) incl += L.wtot[k];
  const unsigned long long in = r.above + incl, ex = in - h;  // bins >= tid, bins > tid
  if (tid == 0) L.sel = ex;                                   // the d = 0 case
  __syncthreads();
  if (tid >= 1 && in > thr && ex <= thr) {                    // at most one such bin
    L.dsel = tid;
    L.sel = ex;
  }
  __syncthreads();
  const int d = L.dsel;
  r.above = L.sel;
  r.prefix |= (uint32_t)d << shift;
  r.pmask |= 255u << shift;
  return r;
}

// The selection threshold floor(top_p Z); false when every token is kept.
__device__ __forceinline__ bool selecting(const SampleArgs& a, unsigned long long Z, unsigned long long& thr) {
  thr = (unsigned long long)((double)a.top_p * (double)Z);
  return a.top_p < 1.0f && thr < Z;
}

// The slice of workgroup sw: tokens [lo, hi).
__device__ __forceinline__ void slice_of(int V, int sw, int& lo, int& hi) {
  const int NW = sample_slices(V), SL = (V + NW - 1) / NW;
  lo = sw * SL;
  hi = lo + SL < V ? lo + SL : V;
}

// Adds this workgroup's per-wave LDS histograms (every wave has passed a barrier since its last
// atomic) into the global histogram: the non-zero bins only.
__device__ __forceinline__ void flush_hist(unsigned long long (&hist)[kSW / 64][256], unsigned long long* g) {
  const int tid = threadIdx.x;
  unsigned long long t = 0;
#pragma unroll
  for (int k = 0; k < kSW / 64; ++k) t += hist[k][tid];
  if (t != 0ull) atomicAdd(g + tid, t);
}

// The maxima of z per slice; slice 0 also clears the sequence's global sums (Z and histograms).
__global__ __launch_bounds__(kSW) void sample_max_kernel(SampleArgs a) {
  __shared__ float redf[kSW / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sw = blockIdx.x, b = blockIdx.y, V = a.V;
  int lo, hi;
  slice_of(V, sw, lo, hi);
  const uint16_t* lg = a.logits + (size_t)b * V;
  const int* cn = a.counts + (size_t)b * V;
  const SampleRow R = sample_row(a.escratch + (size_t)b * 2 * sample_row_floats(V));
  float m = -INFINITY;
  for (int i = lo + tid; i < hi; i += kSW) m = fmaxf(m, penalized(h2f(lg[i]), cn[i], a));
  if (sw == 0) {
    for (int q = tid; q < 4 * 256; q += kSW) R.hist[q] = 0ull;
    if (tid == 0) *R.Z = 0ull;
  }
  const float wm = wave_max_dpp_f32(m);
  if (lane == 0) redf[w] = wm;
  __syncthreads();
  if (tid == 0) {
    float t = redf[0];
    for (int k = 1; k < kSW / 64; ++k) t = fmaxf(t, redf[k]);
    R.maxs[sw] = t;
  }
}

// e = exp(z - max z) of the slice to the e row, its exact normalizer and top-byte histogram into
// the global sums.
__global__ __launch_bounds__(kSW) void sample_exp_kernel(SampleArgs a) {
  __shared__ unsigned long long hist[kSW / 64][256];
  __shared__ long long redl[kSW / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sw = blockIdx.x, b = blockIdx.y, V = a.V, NW = sample_slices(V);
  const int rs = sample_row_floats(V);
  int lo, hi;
  slice_of(V, sw, lo, hi);
  const uint16_t* lg = a.logits + (size_t)b * V;
  const int* cn = a.counts + (size_t)b * V;
  float* row0 = a.escratch + (size_t)b * 2 * rs;
  float* er = row0 + rs;
  const SampleRow R = sample_row(row0);
  __shared__ float mx;
  if (tid < 64) {  // the slice maxima, all loaded at once (wave 0; NW <= 64)
    const float wm = wave_max_dpp_f32(tid < NW ? R.maxs[tid] : -INFINITY);
    if (tid == 0) mx = wm;
  }
  for (int q = tid; q < (kSW / 64) * 256; q += kSW) (&hist[0][0])[q] = 0ull;
  __syncthreads();
  const float m = mx;
  unsigned long long zs = 0;
  for (int i = lo + tid; i < hi; i += kSW) {
    const float e = dev_expf(penalized(h2f(lg[i]), cn[i], a) - m);
    er[i] = e;
    const unsigned long long E = fixed40(e);
    zs += E;
    if (E != 0ull) atomicAdd(&hist[w][__builtin_bit_cast(uint32_t, e) >> 24], E);
  }
  const long long Zw = block_sum_ll<kSW>((long long)zs, redl);  // (its barriers also publish hist)
  if (tid == 0) atomicAdd(R.Z, (unsigned long long)Zw);
  flush_hist(hist, R.hist);
}

// Radix pass p (1..3): the digits of passes 0 .. p - 1, then the histogram of byte p of the
// slice's keys that match them (skipped when every token is kept).
__global__ __launch_bounds__(kSW) void sample_pass_kernel(SampleArgs a, int p) {
  __shared__ unsigned long long hist[kSW / 64][256];
  __shared__ SelLds sl;
  const int tid = threadIdx.x, w = tid >> 6;
  const int sw = blockIdx.x, b = blockIdx.y, V = a.V, rs = sample_row_floats(V);
  int lo, hi;
  slice_of(V, sw, lo, hi);
  float* row0 = a.escratch + (size_t)b * 2 * rs;
  const float* er = row0 + rs;
  const SampleRow R = sample_row(row0);
  float ev[4];  // the slice's e values (at most 1024 tokens), loaded ahead of the selection
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = lo + tid + kSW * j;
    ev[j] = i < hi ? er[i] : 0.0f;
  }
  unsigned long long thr;
  if (!selecting(a, *R.Z, thr)) return;  // uniform over the grid
  const Sel prev = p > 1 ? R.sel[p - 2] : Sel{0u, 0u, 0ull};
  for (int q = tid; q < (kSW / 64) * 256; q += kSW) (&hist[0][0])[q] = 0ull;
  // digit p - 1 (its barriers also publish the cleared hist); the next launch starts from it
  const Sel s = select_digit(R.hist + 256 * (p - 1), prev, p - 1, thr, sl);
  if (sw == 0 && tid == 0) R.sel[p - 1] = s;
  const int shift = 24 - 8 * p;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t key = __builtin_bit_cast(uint32_t, ev[j]);
    if (lo + tid + kSW * j < hi && (key & s.pmask) == s.prefix) {
      const unsigned long long E = fixed40(ev[j]);
      if (E != 0ull) atomicAdd(&hist[w][(key >> shift) & 255u], E);
    }
  }
  __syncthreads();
  flush_hist(hist, R.hist + 256 * p);
}

// The boundary key kb from the four histograms (0 when every token is kept); per slice the exact
// mass of the keys above kb and the count of keys equal to kb.
__global__ __launch_bounds__(kSW) void sample_mass_kernel(SampleArgs a) {
  __shared__ SelLds sl;
  __shared__ long long redl[kSW / 64];
  const int tid = threadIdx.x;
  const int sw = blockIdx.x, b = blockIdx.y, V = a.V, rs = sample_row_floats(V);
  int lo, hi;
  slice_of(V, sw, lo, hi);
  float* row0 = a.escratch + (size_t)b * 2 * rs;
  const float* er = row0 + rs;
  const SampleRow R = sample_row(row0);
  float ev[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = lo + tid + kSW * j;
    ev[j] = i < hi ? er[i] : 0.0f;
  }
  unsigned long long thr;
  uint32_t kb = 0;
  if (selecting(a, *R.Z, thr)) {  // uniform over the grid
    const Sel s = select_digit(R.hist + 256 * 3, R.sel[2], 3, thr, sl);  // the last digit
    if (sw == 0 && tid == 0) R.sel[3] = s;                               // the draw starts from it
    kb = s.prefix;
  }
  unsigned long long mg = 0;
  int nt = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t key = __builtin_bit_cast(uint32_t, ev[j]);
    if (lo + tid + kSW * j < hi) {
      if (key > kb) mg += fixed40(ev[j]);
      nt += key == kb ? 1 : 0;
    }
  }
  const long long M = block_sum_ll<kSW>((long long)mg, redl);
  const long long T = block_sum_ll<kSW>((long long)nt, redl);
  if (tid == 0) {
    R.mass[sw] = (unsigned long long)M;
    R.ties[sw] = (int)T;
  }
}

// Inclusive block scan of 64-bit values over the kSW threads (v < 2^63).
__device__ __forceinline__ unsigned long long block_scan_u64(unsigned long long v, unsigned long long* red) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, off, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(v >> 32), off, 64);
    if (lane >= off) v += ((unsigned long long)hi << 32) | lo;
  }
  __syncthreads();
  if (lane == 63) red[w] = v;
  __syncthreads();
  for (int k = 0; k < w; ++k) v += red[k];
  return v;
}

// One workgroup per sequence: ties kept per slice, kept masses, the slice holding R and the token.
__global__ __launch_bounds__(kSW) void sample_draw_kernel(SampleArgs a) {
  __shared__ unsigned long long red[kSW / 64];
  __shared__ unsigned long long pick_r;
  __shared__ int pick_s, pick_kt;
  const int tid = threadIdx.x, lane = tid & 63;
  const int b = blockIdx.x, V = a.V, NW = sample_slices(V), rs = sample_row_floats(V);
  float* row0 = a.escratch + (size_t)b * 2 * rs;
  const float* er = row0 + rs;
  const SampleRow R = sample_row(row0);
  const unsigned long long mass = tid < NW ? R.mass[tid] : 0ull;
  const int ties = tid < NW ? R.ties[tid] : 0;
  unsigned long long thr;
  uint32_t kb = 0;
  long long nkeep = (long long)V;  // ties kept in index order (all when every token is kept)
  if (selecting(a, *R.Z, thr)) {
    const Sel s = R.sel[3];  // after all four digits
    kb = s.prefix;
    const unsigned long long eb = fixed40(__builtin_bit_cast(float, kb));  // > 0 by construction
    nkeep = eb ? (long long)((thr - s.above) / eb) + 1 : (long long)V;
  }
  const unsigned long long eb = fixed40(__builtin_bit_cast(float, kb));
  if (tid < 64) {  // wave 0: slice lanes (NW <= 64)
    if (tid == 0) {  // (overwritten below by the one picking lane, later in the same wave)
      pick_s = 0;
      pick_r = 0ull;
      pick_kt = 0;
    }
    int tin = ties;  // ties in slices <= lane
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(tin, off, 64);
      if (lane >= off) tin += t;
    }
    const long long before = tin - ties;
    long long kt = nkeep - before;
    kt = kt < 0 ? 0 : (kt > ties ? ties : kt);
    const unsigned long long kept = mass + eb * (unsigned long long)kt;
    unsigned long long incl = kept;
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)incl, off, 64);
      const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(incl >> 32), off, 64);
      if (lane >= off) incl += ((unsigned long long)hi << 32) | lo;
    }
    const unsigned long long S = ((unsigned long long)(uint32_t)__shfl((int)(uint32_t)(incl >> 32), 63, 64) << 32) |
                                 (uint32_t)__shfl((int)(uint32_t)incl, 63, 64);
    const uint64_t h = splitmix64(a.seed ^ (((uint64_t)b << 40) | ((uint64_t)(a.step[b] & 0x7fffffu) << 17) | 0x1ffffull));
    const unsigned long long Rd = __umul64hi(h, S);  // uniform in [0, S)
    const unsigned long long ex = incl - kept;
    if (lane < NW && ex <= Rd && Rd < incl) {  // exactly one slice
      pick_s = lane;
      pick_r = Rd - ex;
      pick_kt = (int)kt;
    }
  }
  __syncthreads();
  const int ps = pick_s, kt = pick_kt;
  const unsigned long long Rr = pick_r;
  int lo, hi;
  slice_of(V, ps, lo, hi);
  // thread t owns tokens lo + 4 t .. lo + 4 t + 3 of the slice (index order = thread order)
  float ev[4];
  int ntie = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = lo + 4 * tid + j;
    ev[j] = i < hi ? er[i] : 0.0f;
    ntie += (i < hi && __builtin_bit_cast(uint32_t, ev[j]) == kb) ? 1 : 0;
  }
  const int trank = (int)(block_scan_u64((unsigned long long)ntie, red) - (unsigned long long)ntie);  // ties before
  unsigned long long em[4], mine = 0;
  {
    int r = trank;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = lo + 4 * tid + j;
      const uint32_t key = __builtin_bit_cast(uint32_t, ev[j]);
      bool keep = i < hi && key > kb;
      if (i < hi && key == kb) keep = r++ < kt;
      em[j] = keep ? fixed40(ev[j]) : 0ull;
      mine += em[j];
    }
  }
  const unsigned long long incl = block_scan_u64(mine, red), excl = incl - mine;
  if (mine > 0 && excl <= Rr && Rr < incl) {  // exactly one thread
    unsigned long long acc = excl;
    int tok = lo + 4 * tid;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // the first token whose cumulative mass exceeds R
      if (Rr < acc + em[j]) {
        tok = lo + 4 * tid + j;
        break;
      }
      acc += em[j];
    }
    a.next[b] = tok;
    a.counts[(size_t)b * V + tok] += 1;
    a.step[b] += 1u;
  }
}

hipError_t launch_sample(const SampleArgs& a, int batch, hipStream_t s) {
  if (a.V < 1 || a.V > kSampleMaxVocab) return hipErrorInvalidValue;
  const dim3 g(sample_slices(a.V), batch);
  hipLaunchKernelGGL(sample_max_kernel, g, dim3(kSW), 0, s, a);
  hipLaunchKernelGGL(sample_exp_kernel, g, dim3(kSW), 0, s, a);
  for (int p = 1; p < 4; ++p) hipLaunchKernelGGL(sample_pass_kernel, g, dim3(kSW), 0, s, a, p);
  hipLaunchKernelGGL(sample_mass_kernel, g, dim3(kSW), 0, s, a);
  hipLaunchKernelGGL(sample_draw_kernel, dim3(batch), dim3(kSW), 0, s, a);
  return hipGetLastError();
}

}  // namespace dfssm
