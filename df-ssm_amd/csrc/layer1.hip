// One decode layer for 1..4 sequences in a single launch, organised by SSM item (gfx950).
//
// Grid: one workgroup per SSM item (head, 16-row block of the head's P rows), all co-resident
// (NI = H * P / 16 items, NI a power of two <= 256 and <= the CU count). Workgroup w computes
// everything its item needs that no other item needs, so the only data that crosses
// workgroups are the values every item shares:
//   in_proj: the item's 16 z rows, 16 x rows and its head's dt row (the dt row is recomputed by
//     the P / 16 workgroups of a head), plus 2 d_state / NI of the B | C rows, which it publishes;
//   LoRA intermediates of in_proj (16 ranks x d_model columns): workgroup w computes the exact
//     partial sum of rank w % 16 over column slice w / 16 and publishes it; every workgroup polls
//     the NI partials and adds them in a fixed order (the sums are exact fp64 sums of exactly
//     representable products, so any split gives the same value);
//   conv + SiLU of its x rows and B | C rows (it owns those channels' conv state), gate of its z
//     rows, softplus dt and exp(dt A) of its head; polls the B | C values of the other
//     workgroups; SSM update of its 16 state rows; publishes its 16 gated outputs g;
//   out_proj (workgroups w < D / 32): polls all g, gated RMSNorm, quantizer, bit planes, LoRA
//     partial of rank w % 16 over a slice of d_inner (published and polled like in_proj's), GEMV
//     of its 32 rows, residual into x.
// So a layer has three exchanges: LoRA partials (overlapping the in_proj GEMV), B | C, and g.
//
// Waves have fixed roles, because loads complete in issue order (waiting for one waits for every
// load the wave issued before it): waves 0..7 (control) load the activations and norm weights at
// the start and afterwards only poll and reduce; waves 8..15 (stream) issue every bulk load at the
// start -- the in_proj and out_proj sign bits of the workgroup, the epilogue rows, the SSM state
// -- and run the GEMVs, epilogues and the SSM update. All waves quantize and build bit planes.
//
// Exchanged values travel as tagged words written and polled with device-scope (sc1) accesses:
// (tag << 16) | fp16 in 32-bit words, (tag << 48) | payload in 64-bit words; the tag is the
// launch's epoch (each workgroup keeps its launch count in the workspace, so all derive the same
// tag without a shared counter). Words polled by every workgroup are written in kXRep copies and
// workgroup w polls copy w % kXRep, so that the polls spread over memory channels. Every poll is
// bounded: a timeout sets bit 2 of the workspace error flag and the grid still drains.
//
// Arithmetic is that of the one-launch layer in fused.hip (and of prep/proj/ssm): integer scaffold
// sums, exact fp64 sums for the norms, LoRA and readout, the same fp16 rounding points.
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

#ifdef DFSSM_TIMELINE
constexpr int kTl1Slots = 64, kTl1Wg = 256, kTl1Stamps = 32;
__device__ unsigned long long dfssm_timeline1[kTl1Slots][kTl1Wg][kTl1Stamps];
#define TL1_DECL __shared__ unsigned long long tl1_s[kTl1Stamps]
#define TL1(k)                                                                   \
  do {                                                                           \
    if (ltix() == 0) tl1_s[k] = __builtin_amdgcn_s_memrealtime();                \
  } while (0)
#else
#define TL1_DECL
#define TL1(k) do {} while (0)
#endif

namespace {

constexpr int kT = 1024;                  // threads per workgroup (16 waves)
constexpr int kCT = 512;                  // control threads: waves 0..7
constexpr int kST = kT - kCT;             // stream threads: waves 8..15
constexpr int kMaxK = 4096;               // d_model and d_inner at most
constexpr int kMaxCH = kMaxK / 128;       // 16-byte chunks (128 columns) of a row
constexpr int kMaxRowsA = 33 + 8;         // in_proj rows of a workgroup: z16, x16, dt, <= 8 B|C rows
constexpr int kUA = (kMaxRowsA * kMaxCH + kST - 1) / kST;  // in_proj GEMV units per stream thread
constexpr int kRC = 32;                   // out_proj rows of a phase-C workgroup
constexpr int kUC = (kRC * kMaxCH + kST - 1) / kST;        // out_proj GEMV units per stream thread
constexpr int kMaxSlice = 1024;           // LoRA partial: columns of one (rank, slice)
constexpr int kMaxNI = 256;               // items (= workgroups)
constexpr uint32_t kSpin = 1u << 18;

__device__ __forceinline__ int ltix() {
  int t = __builtin_amdgcn_workitem_id_x();
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int lbix() {
  int t = __builtin_amdgcn_workgroup_id_x();
  asm volatile("" : "+s"(t));
  return t;
}
// Marks v as changed here: the compiler can neither move computations on a loaded value above this
// point nor merge them with earlier code, so the wave waits for that load only where it is used.
template <class T>
__device__ __forceinline__ void opaque(T& v) {
  asm volatile("" : "+v"(v));
}
__device__ __forceinline__ uint32_t tag_of(uint32_t epoch_raw) {
  opaque(epoch_raw);
  return (epoch_raw + 1u) & 0xffffu;
}
template <class T>
__device__ __forceinline__ T lds_dev(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void sts_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int M>
struct ItemLds {  // every member 16-byte aligned: read and written as 16-byte vectors
  alignas(16) uint32_t planes[M][kMaxK / 32][8];     // bit planes of the quantized activations
  alignas(16) int T[M][kMaxRowsA][kMaxCH + 4];       // GEMV partial counts per (row, chunk)
  alignas(16) uint16_t xn[M][kMaxK];                 // normalized activations (phase C: first the polled g)
  alignas(16) double rd[M][8];                       // control-wave partial sums
  alignas(16) float rf[M][8];                        // control-wave partial maxima
  alignas(16) int qs[M][16];                         // per-wave partial sums of q
  alignas(16) double hp[M][kMaxNI];                  // polled LoRA partials
  alignas(16) float hl[M][DFSSM_LORA_R];             // LoRA intermediates (fp16 values)
  alignas(16) uint16_t bc[M][256];                   // B | C after the conv
  alignas(16) uint16_t xv[M][16];                    // the item's conv'd x
  alignas(16) uint16_t gate[M][16];                  // its gate z sigma(z)
  alignas(16) uint16_t gl[M][16];                    // its output g
  alignas(16) float dt[M];
  alignas(16) float abar[M];
};

// in_proj row of slot i of workgroup w: 0..15 z rows, 16..31 x rows, 32 the head's dt row,
// 33 .. 33 + nbc - 1 the workgroup's B | C rows.
__device__ __forceinline__ int row_a(int i, int head, int pb, int P, int DI, int N2, int w, int nbc) {
  return i < 16 ? head * P + pb * 16 + i
                : (i < 32 ? DI + head * P + pb * 16 + (i - 16) : (i == 32 ? 2 * DI + N2 + head : 2 * DI + w * nbc + (i - 33)));
}

__device__ __forceinline__ const u32x4* tiled(const uint32_t* bits, int n, int c, int CH) {
  return (const u32x4*)bits + ((size_t)(n >> 6) * CH + c) * 64 + (n & 63);
}

// Poll 32-bit words (tag << 16) | fp16 pairs: N 64-bit loads at p + 2 j in flight together; out[j]
// = the two fp16 values low | high. Bounded: a timeout sets bit 2 of err.
template <int N>
__device__ __forceinline__ void poll_pairs(const uint32_t* p, uint32_t tag, uint32_t (&out)[N], int* err,
                                           unsigned long long* t_issue = nullptr) {
  uint64_t v[N];
  if (t_issue) *t_issue = __builtin_amdgcn_s_memrealtime();
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = lds_dev((const uint64_t*)p + j);
  auto good = [&](uint64_t x) { return ((uint32_t)x >> 16) == tag && ((uint32_t)(x >> 32) >> 16) == tag; };
  for (uint32_t it = 0;; ++it) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok = ok && good(v[j]);
    if (ok) break;
    if (it == kSpin) {
      atomicOr(err, 4);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    if (t_issue) *t_issue = __builtin_amdgcn_s_memrealtime();
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = lds_dev((const uint64_t*)p + j);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) out[j] = ((uint32_t)v[j] & 0xffffu) | ((uint32_t)(v[j] >> 32) << 16);
}

// Poll 64-bit words tagged in bits 48..63: up to N words p[i0 + stride j] (j < n), in flight
// together. Bounded as above.
template <int N>
__device__ __forceinline__ void poll_w64(const uint64_t* p, int i0, int stride, int n, uint32_t tag, uint64_t (&v)[N],
                                         int* err, unsigned long long* t_issue = nullptr) {
  if (t_issue) *t_issue = __builtin_amdgcn_s_memrealtime();
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = j < n ? lds_dev(p + i0 + (size_t)stride * j) : ((uint64_t)tag << 48);
  for (uint32_t it = 0;; ++it) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok = ok && (uint32_t)(v[j] >> 48) == tag;
    if (ok) break;
    if (it == kSpin) {
      atomicOr(err, 4);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    if (t_issue) *t_issue = __builtin_amdgcn_s_memrealtime();
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (j < n) v[j] = lds_dev(p + i0 + (size_t)stride * j);
  }
}

// Bit planes of 64 int8 values (q of value k0 + lane) into the 16 words at dst (LDS): word 2b + h =
// bit b of values k0 + 32h .. k0 + 32h + 31, each plane's 64-bit ballot stored whole by lane 0.
__device__ __forceinline__ void planes64_store(uint32_t* dst, int q, int lane) {
  uint64_t b64[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) b64[b] = __ballot((q >> b) & 1);
  if (lane == 0) {
    uint64_t* d = (uint64_t*)dst;
#pragma unroll
    for (int b = 0; b < 8; ++b) d[b] = b64[b];
  }
}

// Sum of bit-plane popcounts of one 16-byte chunk c (128 columns) of a row against activation
// row m: sum_{bit=1} q over those columns.
template <int M>
__device__ __forceinline__ int chunk_dot(const ItemLds<M>& L, int m, int c, const u32x4& wb) {
  uint32_t cnt[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
  for (int sh = 0; sh < 2; ++sh) {
    const u32x4* ps = (const u32x4*)&L.planes[m][c * 4 + 2 * sh][0];
    const u32x4 d0 = ps[0], d1 = ps[1], d2 = ps[2], d3 = ps[3];
    const uint32_t pl[16] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3],
                             d2[0], d2[1], d2[2], d2[3], d3[0], d3[1], d3[2], d3[3]};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t w = wb[2 * sh + h];
#pragma unroll
      for (int b = 0; b < 8; ++b) cnt[b] += __builtin_popcount(w & pl[2 * b + h]);
    }
  }
  int t = 0;
#pragma unroll
  for (int b = 0; b < 7; ++b) t += (int)(cnt[b] << b);
  return t - (int)(cnt[7] << 7);
}

// Control waves: RMSNorm of M rows of K values (8 consecutive values per thread t < K / 8,
// v[m]: one 16-byte vector of fp16) into L.xn, with per-wave partial maxima in L.rf. Two
// barriers (the stream waves pass the same two).
template <int M>
__device__ __forceinline__ void norm_control(ItemLds<M>& L, const u32x4 (&v)[M], const f32x4 (&wv)[2], int K,
                                             unsigned long long* tl, int s0, int s1, int s2) {
  const int tid = ltix(), lane = tid & 63, wave = tid >> 6;
  const bool has = tid < K / 8;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    double part = 0.0;
    if (has) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double x = (double)h2f((uint16_t)(v[m][e >> 1] >> (16 * (e & 1))));
        part += x * x;
      }
    }
    part = wave_sum_dpp_f64(part);
    if (lane == 0) L.rd[m][wave] = part;
  }
  lds_barrier();
  if (tl && tid == 0) tl[s0] = __builtin_amdgcn_s_memrealtime();
  f32x4 w0 = wv[0], w1 = wv[1];
  opaque(w0);
  opaque(w1);
  const float w8[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
#pragma unroll
  for (int m = 0; m < M; ++m) {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += L.rd[m][i];
    const float var = (float)ss * (1.0f / (float)K);
    const float r = 1.0f / sqrt_rn(var + 1e-5f);
    float mx = 0.0f;
    if (has) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t pair = v[m][e >> 1];
        const float x0 = r16((h2f((uint16_t)pair) * r) * w8[e]);
        const float x1 = r16((h2f((uint16_t)(pair >> 16)) * r) * w8[e + 1]);
        mx = fmaxf(mx, fmaxf(fabsf(x0), fabsf(x1)));
        o[e >> 1] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
      }
      *(u32x4*)&L.xn[m][8 * tid] = u32x4{o[0], o[1], o[2], o[3]};
    }
    mx = wave_max_dpp_f32(mx);
    if (lane == 0) L.rf[m][wave] = mx;
  }
  if (tl && tid == 0) tl[s1] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();
  if (tl && tid == 0) tl[s2] = __builtin_amdgcn_s_memrealtime();
}

// Quantization scale and its fp64 reciprocal of every row (after norm_control's second barrier).
template <int M>
__device__ __forceinline__ void row_scales(const ItemLds<M>& L, float (&rinv)[M], float (&xs)[M]) {
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float amax = L.rf[m][0];
#pragma unroll
    for (int i = 1; i < 8; ++i) amax = fmaxf(amax, L.rf[m][i]);
    xs[m] = quant_scale(amax);
    rinv[m] = quant_rcp(xs[m]);
  }
}

// Every wave: q, bit planes and the wave's sum q of the 64-value blocks 64 (wave + 16 j) of K.
template <int M>
__device__ __forceinline__ void quantize_waves(ItemLds<M>& L, int K, const float (&rinv)[M]) {
  const int lane = ltix() & 63, wave = ltix() >> 6;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int qsum = 0;
    int q[kMaxK / 1024];
#pragma unroll
    for (int j = 0; j < kMaxK / 1024; ++j) {  // all of this wave's blocks, for instruction overlap
      const int k0 = 64 * wave + 1024 * j;
      q[j] = k0 < K ? quant_i8(h2f(L.xn[m][k0 + lane]), rinv[m]) : 0;
    }
#pragma unroll
    for (int j = 0; j < kMaxK / 1024; ++j) {
      const int k0 = 64 * wave + 1024 * j;
      if (k0 < K) {
        qsum += q[j];
        planes64_store(&L.planes[m][k0 / 32][0], q[j], lane);
      }
    }
    qsum = wave_sum_dpp_i32(qsum);
    if (lane == 0) L.qs[m][wave] = qsum;
  }
}

// Control threads t < NP poll the NP exchanged partials of every row m (two words each, from this
// workgroup's copy: words 2 (m NP + t), 2 (m NP + t) + 1) into L.hp.
template <int M>
__device__ __forceinline__ void poll_partials(ItemLds<M>& L, const uint64_t* base, int NP, uint32_t tag, int* err) {
  const int tid = ltix();
  if (tid >= NP) return;
  uint64_t v[2 * M];
#pragma unroll
  for (int j = 0; j < 2 * M; ++j) v[j] = lds_dev(base + 2 * ((j >> 1) * NP + tid) + (j & 1));
  for (uint32_t it = 0;; ++it) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 2 * M; ++j) ok = ok && (uint32_t)(v[j] >> 48) == tag;
    if (ok) break;
    if (it == kSpin) {
      atomicOr(err, 4);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < 2 * M; ++j) v[j] = lds_dev(base + 2 * ((j >> 1) * NP + tid) + (j & 1));
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
    L.hp[m][tid] = __builtin_bit_cast(double, (uint64_t)((v[2 * m] & 0xffffffffu) | ((v[2 * m + 1] & 0xffffffffu) << 32)));
}

// Threads t < 16 M: h[m][r] = fp16(sum over slices s of hp[m][16 s + r]), in slice order.
template <int M>
__device__ __forceinline__ void sum_partials(ItemLds<M>& L, int NP) {
  const int tid = ltix();
  if (tid < DFSSM_LORA_R * M) {
    const int m = tid / DFSSM_LORA_R, r = tid % DFSSM_LORA_R;
    double s = 0.0;
    for (int sl = 0; sl < NP / DFSSM_LORA_R; ++sl) s += L.hp[m][sl * DFSSM_LORA_R + r];
    L.hl[m][r] = r16((float)s);
  }
}

// Sum of the GEMV partial counts of row i of sequence m over its CH chunks (CH a multiple of 4).
template <int M>
__device__ __forceinline__ int t_sum(const ItemLds<M>& L, int m, int i, int CH) {
  int t = 0;
#pragma unroll
  for (int c4 = 0; c4 < kMaxCH; c4 += 4) {
    if (c4 < CH) {
      const i32x4 v = *(const i32x4*)&L.T[m][i][c4];
      t += (v[0] + v[1]) + (v[2] + v[3]);
    }
  }
  return t;
}

// Exact partial LoRA intermediate of one rank over `width` columns starting at col0 (one wave):
// sum_k xn[m][col0 + k] * bq[k] (bq: the slice of the fp16 LoRA-B row in LDS; fp16 x fp16
// products exact in fp32, summed in fp64). Lane l takes columns 16 l .. 16 l + 15. Result uniform
// across the wave.
template <int M>
__device__ __forceinline__ double lora_partial(const ItemLds<M>& L, int m, int col0, int width, const u32x4 (&bq)[2]) {
  const int lane = ltix() & 63;
  double acc = 0.0;
  if (16 * lane < width) {
    const u32x4 x0 = *(const u32x4*)&L.xn[m][col0 + 16 * lane];
    const u32x4 x1 = *(const u32x4*)&L.xn[m][col0 + 16 * lane + 8];
    u32x4 b0 = bq[0], b1 = bq[1];
    opaque(b0);
    opaque(b1);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t xw = (e < 8 ? x0 : x1)[(e & 7) >> 1], bw = (e < 8 ? b0 : b1)[(e & 7) >> 1];
      const float xv = h2f((uint16_t)(xw >> (16 * (e & 1))));
      const float bv = h2f((uint16_t)(bw >> (16 * (e & 1))));
      acc += (double)(xv * bv);
    }
  }
  return wave_sum_dpp_f64(acc);
}

// Publish an fp64 partial as two 64-bit words (tag << 48) | 32 bits, in every copy (lanes c <
// kXRep write copy c).
__device__ __forceinline__ void publish_partial(uint64_t* base, int idx, double v, uint32_t tag) {
  const int lane = ltix() & 63;
  if (lane < kXRep) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    uint64_t* d = base + (size_t)lane * kLpStride + 2 * idx;
    sts_dev<uint64_t>(d, ((uint64_t)tag << 48) | (uint64_t)(u & 0xffffffffu));
    sts_dev<uint64_t>(d + 1, ((uint64_t)tag << 48) | (uint64_t)(u >> 32));
  }
}

}  // namespace

// Indices of a workgroup, shared by both wave roles.
struct ItemCtx {
  int G, w, D, DI, N2, P, PB, head, pb, nbc, NR, CHA, CHC, S, WA, gC, SC, WC, rA, sA, sC;
  bool cwg;
};

__device__ __forceinline__ ItemCtx item_ctx(const FusedArgs& a) {
  ItemCtx c;
  c.G = gridDim.x;
  c.w = lbix();
  c.D = a.D; c.DI = a.DI; c.N2 = 2 * a.N; c.P = a.P; c.PB = a.P / 16;
  c.head = c.w / c.PB; c.pb = c.w % c.PB;
  c.nbc = c.N2 / c.G; c.NR = 33 + c.nbc;
  c.CHA = c.D / 128; c.CHC = c.DI / 128;
  c.S = c.G / DFSSM_LORA_R; c.WA = c.D / c.S;          // LoRA slices of d_model and their width
  c.gC = c.D / kRC; c.SC = c.gC / DFSSM_LORA_R; c.WC = c.DI / c.SC;
  c.rA = c.w % DFSSM_LORA_R; c.sA = c.w / DFSSM_LORA_R; c.sC = c.w / DFSSM_LORA_R;
  c.cwg = c.w < c.gC;
  return c;
}

// Waves 0..7: activation loads, norms, LoRA partials, every poll and publication of g. Barrier
// sequence B1..B14 as in stream_path.
template <int M>
__device__ void control_path(ItemLds<M>& L, const FusedArgs& a, const ItemCtx& c, uint32_t epoch_raw,
                             unsigned long long* tl) {
  const int tid = ltix(), wave = tid >> 6, lane = tid & 63;
  // loads in the order of use (they complete in issue order): x and the in_proj norm weights of
  // this thread's 8 values, the in_proj LoRA-B slice (wave 0), the out_proj norm weights and
  // LoRA-B slice (wave 1; phase C), all held in registers until used
  u32x4 xa[M];
  f32x4 lw[2], nw[2];
  u32x4 bA[2], bC[2];
  {
    const int t = tid < c.D / 8 ? tid : 0;
#pragma unroll
    for (int m = 0; m < M; ++m) xa[m] = *(const u32x4*)(a.x + (size_t)m * c.D + 8 * t);
    lw[0] = *(const f32x4*)(a.ln_w + 8 * t);
    lw[1] = *(const f32x4*)(a.ln_w + 8 * t + 4);
    const uint16_t* pa = a.in_lBq + (size_t)c.rA * c.D + c.sA * c.WA + (16 * lane < c.WA ? 16 * lane : 0);
    bA[0] = *(const u32x4*)pa;
    bA[1] = *(const u32x4*)(pa + 8);
    const int tc = tid < c.DI / 8 ? tid : 0;
    nw[0] = *(const f32x4*)(a.norm_w + 8 * tc);
    nw[1] = *(const f32x4*)(a.norm_w + 8 * tc + 4);
    const uint16_t* pc =
        a.out_lBq + (size_t)c.rA * c.DI + (c.cwg ? c.sC : 0) * c.WC + (16 * lane < c.WC ? 16 * lane : 0);
    bC[0] = *(const u32x4*)pc;
    bC[1] = *(const u32x4*)(pc + 8);
  }
  if (tl) {
#pragma unroll
    for (int m = 0; m < M; ++m) opaque(xa[m]);
    if (tid == 0) tl[16] = __builtin_amdgcn_s_memrealtime();
  }
  norm_control<M>(L, xa, lw, c.D, tl, 14, 18, 15);  // B1, B2
  float rinv[M];
  float xs[M];
  row_scales<M>(L, rinv, xs);
  const uint32_t tag = tag_of(epoch_raw);
  if (wave == 0) {  // this workgroup's LoRA partial (rank rA, slice sA) of every sequence
#pragma unroll
    for (int m = 0; m < M; ++m)
      publish_partial(a.lpA, m * c.G + c.w, lora_partial<M>(L, m, c.sA * c.WA, c.WA, bA), tag);
  }
  quantize_waves<M>(L, c.D, rinv);
  if (tl && tid == 0) tl[20] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();  // B3
  if (tl && tid == 0) tl[1] = __builtin_amdgcn_s_memrealtime();
  poll_partials<M>(L, a.lpA + (size_t)(c.w % kXRep) * kLpStride, c.G, tag, a.err);
  if (tl && tid == 0) tl[23] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();  // B4
  if (tl && tid == 0) tl[2] = __builtin_amdgcn_s_memrealtime();
  sum_partials<M>(L, c.G);
  lds_barrier();  // B5
  if (tl && tid == 0) tl[3] = __builtin_amdgcn_s_memrealtime();
  // B | C of every sequence from this workgroup's copy: thread t < 64 M, values 4 (t % 64) .. + 3
  if (tid < 64 * M) {
    const int m = tid / 64, l = tid % 64;
    uint32_t v2[2];
    unsigned long long t_is = 0;
    poll_pairs<2>(a.bcT + (c.w % kXRep) * kBcStride + m * c.N2 + 4 * l, tag, v2, a.err, tl ? &t_is : nullptr);
    *(uint2*)&L.bc[m][4 * l] = uint2{v2[0], v2[1]};
    if (tl && tid == 0) tl[19] = t_is;
  }
  if (tl && tid == 0) tl[4] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();  // B6
  if (tl && tid == 0) tl[5] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();  // B7: the SSM outputs g are in L.gl
  if (tid < 6 * M * kXRep) {  // the item's g: three values and the tag per 64-bit word (m, item, q),
                              // thread group cp writing copy cp
    const int cp = tid / (6 * M), m = (tid % (6 * M)) / 6, q = tid % 6;
    uint64_t word = (uint64_t)tag << 48;
#pragma unroll
    for (int e = 0; e < 3; ++e)
      if (3 * q + e < 16) word |= (uint64_t)L.gl[m][3 * q + e] << (16 * e);
    sts_dev(a.gP + (size_t)cp * kGStride + ((size_t)m * c.G + c.w) * 6 + q, word);
  }
  if (tl && tid == 0) tl[6] = __builtin_amdgcn_s_memrealtime();
  if (c.cwg) {
    {  // all g of every sequence into L.xn (words t + 512 j)
      constexpr int kGW = (M * kMaxNI * 6 + kCT - 1) / kCT;
      const int NW = M * c.G * 6;
      uint64_t v[kGW];
      unsigned long long t_is = 0;
      poll_w64<kGW>(a.gP + (size_t)(c.w % kXRep) * kGStride, tid, kCT, (NW - tid + kCT - 1) / kCT, tag, v, a.err,
                    tl ? &t_is : nullptr);
      if (tl && tid == 0) tl[22] = t_is;
#pragma unroll
      for (int j = 0; j < kGW; ++j) {
        const int wd = tid + kCT * j;
        if (wd < NW) {
          const int q = wd % 6, it = (wd / 6) % c.G, m = wd / (6 * c.G);
          const int base = (it / c.PB) * c.P + (it % c.PB) * 16 + 3 * q;
#pragma unroll
          for (int e = 0; e < 3; ++e)
            if (3 * q + e < 16) L.xn[m][base + e] = (uint16_t)(v[j] >> (16 * e));
        }
      }
    }
    if (tl && tid == 0) tl[11] = __builtin_amdgcn_s_memrealtime();
    lds_barrier();  // B8
    if (tl && tid == 0) tl[7] = __builtin_amdgcn_s_memrealtime();
    u32x4 ga[M];
    {
      const int t = tid < c.DI / 8 ? tid : 0;
#pragma unroll
      for (int m = 0; m < M; ++m) ga[m] = *(const u32x4*)&L.xn[m][8 * t];
    }
    if (tl && tid == 0) tl[25] = __builtin_amdgcn_s_memrealtime();
    norm_control<M>(L, ga, nw, c.DI, tl, 26, 31, 27);  // B9, B10
    row_scales<M>(L, rinv, xs);
    if (wave == 1) {  // LoRA partial of out_proj (rank rA, slice sC) of every sequence
#pragma unroll
      for (int m = 0; m < M; ++m)
        publish_partial(a.lpC, m * c.gC + c.w, lora_partial<M>(L, m, c.sC * c.WC, c.WC, bC), tag);
    }
    quantize_waves<M>(L, c.DI, rinv);
    if (tl && (tid == 0 || tid == 64)) tl[tid ? 28 : 29] = __builtin_amdgcn_s_memrealtime();
    lds_barrier();  // B11
    if (tl && tid == 0) tl[8] = __builtin_amdgcn_s_memrealtime();
    poll_partials<M>(L, a.lpC + (size_t)(c.w % kXRep) * kLpStride, c.gC, tag, a.err);
    lds_barrier();  // B12
    if (tl && tid == 0) tl[9] = __builtin_amdgcn_s_memrealtime();
    sum_partials<M>(L, c.gC);
    lds_barrier();  // B13
    if (tl && tid == 0) tl[10] = __builtin_amdgcn_s_memrealtime();
  }
}

// Waves 8..15: every bulk load at the start (sign bits, epilogue rows, SSM state), the GEMVs,
// the epilogues and the SSM update.
template <int M>
__device__ void stream_path(ItemLds<M>& L, const FusedArgs& a, const ItemCtx& c, uint32_t epoch_raw,
                            unsigned long long* tl) {
  const int st = ltix() - kCT, lane = ltix() & 63;
  // epilogue slot of this thread, one kind of row per wave so that no wave runs two branches:
  // stream wave 0 the z rows, 1 the x rows, 2 the dt rows, 3 the B | C rows (sequence em)
  const int sw = st >> 6;
  int ei = 0, em = 0;
  bool ev = false;
  if (sw == 0 || sw == 1) {
    ev = lane < 16 * M;
    ei = 16 * sw + (lane & 15);
    em = lane >> 4;
  } else if (sw == 2) {
    ev = lane < M;
    ei = 32;
    em = lane;
  } else if (sw == 3) {
    ev = lane < c.nbc * M;
    ei = 33 + lane % c.nbc;
    em = lane / c.nbc;
  }
  if (!ev) ei = em = 0;
  if (tl && st == 0) tl[17] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();  // B1
  // bulk loads, staged so that they do not crowd out the activation loads at the start: in_proj
  // bits and epilogue rows now, the state after B4, out_proj bits and rows after B7
  // in_proj sign bits of the workgroup's rows: units u = st + 512 j, chunk u / NR of slot u % NR
  u32x4 wa[kUA];
#pragma unroll
  for (int j = 0; j < kUA; ++j) {
    int u = st + kST * j;
    u = u < c.NR * c.CHA ? u : 0;
    wa[j] = ld_nt(tiled(a.in_bits, row_a(u % c.NR, c.head, c.pb, c.P, c.DI, c.N2, c.w, c.nbc), u / c.NR, c.CHA));
  }
  // epilogue row of this thread
  const int en = row_a(ei, c.head, c.pb, c.P, c.DI, c.N2, c.w, c.nbc);
  const int ech = en - c.DI < 0 ? 0 : (en - c.DI >= a.C ? a.C - 1 : en - c.DI);
  const u32x4 la = *(const u32x4*)(a.in_lA + (size_t)en * DFSSM_LORA_R);
  const uint32_t e_ws = a.in_ws[en], e_as = a.in_lAs[en];
  uint16_t* const cs = a.conv + ((size_t)em * a.C + ech) * 3;
  uint32_t e_cs01;
  __builtin_memcpy(&e_cs01, cs, 4);
  const uint32_t e_cs2 = cs[2];
  const uint32_t e_cw01 = ((const uint32_t*)(a.conv_w + (size_t)ech * 4))[0];
  const uint32_t e_cw23 = ((const uint32_t*)(a.conv_w + (size_t)ech * 4))[1];
  const uint32_t e_cb = a.conv_b[ech];
  const float e_bias = a.dt_bias[c.head], e_alog = a.A_log[c.head];
  lds_barrier();  // B2
  float rinv[M];
  float xs[M];
  row_scales<M>(L, rinv, xs);
  quantize_waves<M>(L, c.D, rinv);
  lds_barrier();  // B3
  // GEMV partial counts of the workgroup's rows
#pragma unroll
  for (int j = 0; j < kUA; ++j) opaque(wa[j]);
#pragma unroll
  for (int j = 0; j < kUA; ++j) {
    const int u = st + kST * j;
    if (u < c.NR * c.CHA) {
      const int ch = u / c.NR, i = u % c.NR;
#pragma unroll
      for (int m = 0; m < M; ++m) L.T[m][i][ch] = chunk_dot<M>(L, m, ch, wa[j]);
    }
  }
  if (tl && st == 0) tl[24] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();  // B4
  // SSM state: row r = st / 32 of the item, columns 4 (st % 32) .. + 3, every sequence
  const int sr = st / 32, c4 = 4 * (st % 32);
  f32x4 hs[M];
#pragma unroll
  for (int m = 0; m < M; ++m)
    hs[m] = ld_nt_f4(a.h + (((size_t)m * a.H + c.head) * c.P + c.pb * 16 + sr) * a.N + c4);
  const float Dh = a.Dp[c.head];
  lds_barrier();  // B5: the LoRA intermediates are in L.hl
  // epilogue of in_proj slot ei, sequence em (its row data are used from here on)
  u32x4 lae = la;
  uint32_t ews = e_ws, eas = e_as, ecs01 = e_cs01, ecs2 = e_cs2, ecw01 = e_cw01, ecw23 = e_cw23, ecb = e_cb;
  float ebias = e_bias, ealog = e_alog;
  opaque(lae); opaque(ews); opaque(eas); opaque(ecs01); opaque(ecs2); opaque(ecw01); opaque(ecw23);
  opaque(ecb); opaque(ebias); opaque(ealog);
  const uint32_t tag = tag_of(epoch_raw);
  bool conv_pending = false;
  uint16_t cv0 = 0, cv1 = 0, cv2 = 0;
  if (ev) {
    int qsum = 0;
#pragma unroll
    for (int v = 0; v < 16; ++v) qsum += L.qs[em][v];
    const int T = t_sum<M>(L, em, ei, c.CHA);
    const int acc = 2 * T - qsum;
    const float as = h2f((uint16_t)eas);
    double lo = 0.0;
#pragma unroll
    for (int r = 0; r < DFSSM_LORA_R; ++r) {
      const float aq = r16((float)(int8_t)(lae[r >> 2] >> (8 * (r & 3))) * as);
      lo += (double)L.hl[em][r] * (double)aq;
    }
    const float y = r16(r16(r16((float)acc) * xs[em]) * h2f((uint16_t)ews));
    const float out = r16((float)lo + y);
    if (ei < 16) {  // z row: gate z sigma(z)
      const float sg = r16(1.0f / (1.0f + dev_expf(-out)));
      L.gate[em][ei] = f2h(r16(out * sg));
    } else if (ei == 32) {  // the head's dt row
      const float dt = dev_log1pf(dev_expf(out + ebias));
      L.dt[em] = dt;
      L.abar[em] = dev_expf(dt * -dev_expf(ealog));
    } else {  // x or B|C channel: depthwise conv (k = 4) + SiLU, the state shifted left
      const uint16_t xo = f2h(out);
      conv_pending = true;
      cv0 = (uint16_t)(ecs01 >> 16);
      cv1 = (uint16_t)ecs2;
      cv2 = xo;
      const float xv = h2f(xo);
      float o = h2f((uint16_t)ecs01) * h2f((uint16_t)ecw01);
      o = o + h2f((uint16_t)(ecs01 >> 16)) * h2f((uint16_t)(ecw01 >> 16));
      o = o + h2f((uint16_t)ecs2) * h2f((uint16_t)ecw23);
      o = o + xv * h2f((uint16_t)(ecw23 >> 16));
      o = o + h2f((uint16_t)ecb);
      const float sig = 1.0f / (1.0f + dev_expf(-o));
      const uint16_t conv_out = f2h(o * sig);
      if (ei < 32) {
        L.xv[em][ei - 16] = conv_out;
      } else {  // B|C channel j: to every copy of the polled words
        const uint32_t word = ((uint32_t)tag << 16) | conv_out;
        const int j = ech - c.DI;
#pragma unroll
        for (int cp = 0; cp < kXRep; ++cp) sts_dev(a.bcT + cp * kBcStride + em * c.N2 + j, word);
      }
    }
  }
  if (tl && (st == 0 || st == 192)) tl[st ? 21 : 12] = __builtin_amdgcn_s_memrealtime();
  lds_barrier();  // B6: B | C of every workgroup are in L.bc
  if (conv_pending) {  // this thread read the channel's state at the start; nobody else touches it
    cs[0] = cv0;
    cs[1] = cv1;
    cs[2] = cv2;
  }
  // SSM update of the item's 16 rows (row sr, columns c4 .. c4 + 3)
  float Dhe = Dh;
  opaque(Dhe);
#pragma unroll
  for (int m = 0; m < M; ++m) opaque(hs[m]);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float xv = h2f(L.xv[m][sr]);
    const float X = xv * L.dt[m], ab = L.abar[m];
    const uint2 bw = *(const uint2*)&L.bc[m][c4];
    const uint2 cw = *(const uint2*)&L.bc[m][a.N + c4];
    const float Bv[4] = {h2f((uint16_t)bw.x), h2f((uint16_t)(bw.x >> 16)), h2f((uint16_t)bw.y), h2f((uint16_t)(bw.y >> 16))};
    const float Cv[4] = {h2f((uint16_t)cw.x), h2f((uint16_t)(cw.x >> 16)), h2f((uint16_t)cw.y), h2f((uint16_t)(cw.y >> 16))};
    f32x4 hv;
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      hv[k] = __builtin_fmaf(ab, hs[m][k], X * Bv[k]);
      acc += (double)Cv[k] * (double)hv[k];
    }
    st_nt_f4(a.h + (((size_t)m * a.H + c.head) * c.P + c.pb * 16 + sr) * a.N + c4, hv);
    // a row's 32 lanes are DPP rows 0 + 1 (even rows) or 2 + 3 (odd rows); readlane takes a
    // uniform lane, so both totals are read and the half-wave picks its own
    acc = row_sum_f64(acc);
    const double lo_rows = readlane_f64(acc, 0) + readlane_f64(acc, 16);
    const double hi_rows = readlane_f64(acc, 32) + readlane_f64(acc, 48);
    if ((lane & 31) == 0) {
      const float y = r16((float)(lane >= 32 ? hi_rows : lo_rows) + xv * Dhe);
      L.gl[m][sr] = f2h(r16(y * h2f(L.gate[m][sr])));
    }
  }
  lds_barrier();  // B7
  // out_proj sign bits (phase-C workgroups; the others load a valid stand-in) and epilogue row
  const int wcg = c.cwg ? c.w : 0;
  u32x4 wcb[kUC];
#pragma unroll
  for (int j = 0; j < kUC; ++j) {
    int u = st + kST * j;
    u = u < kRC * c.CHC ? u : 0;
    wcb[j] = ld_nt(tiled(a.out_bits, wcg * kRC + u % kRC, u / kRC, c.CHC));
  }
  const int ce = st < kRC * M ? st : 0;
  const int cn = wcg * kRC + ce % kRC, cm = ce / kRC;
  const u32x4 lc = *(const u32x4*)(a.out_lA + (size_t)cn * DFSSM_LORA_R);
  const uint32_t c_ws = a.out_ws[cn], c_as = a.out_lAs[cn], c_xres = a.x[(size_t)cm * c.D + cn];
  if (c.cwg) {
    lds_barrier();  // B8: all g in L.xn
    lds_barrier();  // B9
    lds_barrier();  // B10: normalized, maxima in L.rf
    row_scales<M>(L, rinv, xs);
    quantize_waves<M>(L, c.DI, rinv);
    if (tl && st == 0) tl[30] = __builtin_amdgcn_s_memrealtime();
    lds_barrier();  // B11
#pragma unroll
    for (int j = 0; j < kUC; ++j) opaque(wcb[j]);
#pragma unroll
    for (int j = 0; j < kUC; ++j) {
      const int u = st + kST * j;
      if (u < kRC * c.CHC) {
        const int ch = u / kRC, i = u % kRC;
#pragma unroll
        for (int m = 0; m < M; ++m) L.T[m][i][ch] = chunk_dot<M>(L, m, ch, wcb[j]);
      }
    }
    lds_barrier();  // B12
    lds_barrier();  // B13: the LoRA intermediates are in L.hl
    u32x4 lce = lc;
    uint32_t cws = c_ws, cas = c_as, cxres = c_xres;
    opaque(lce); opaque(cws); opaque(cas); opaque(cxres);
    if (st < kRC * M) {  // residual of out_proj row cn = 32 w + i of sequence cm
      const int i = st % kRC;
      int qsum = 0;
#pragma unroll
      for (int v = 0; v < 16; ++v) qsum += L.qs[cm][v];
      const int T = t_sum<M>(L, cm, i, c.CHC);
      const int acc = 2 * T - qsum;
      const float as = h2f((uint16_t)cas);
      double lo = 0.0;
#pragma unroll
      for (int r = 0; r < DFSSM_LORA_R; ++r) {
        const float aq = r16((float)(int8_t)(lce[r >> 2] >> (8 * (r & 3))) * as);
        lo += (double)L.hl[cm][r] * (double)aq;
      }
      const float y = r16(r16(r16((float)acc) * xs[cm]) * h2f((uint16_t)cws));
      const float out = r16((float)lo + y);
      a.x[(size_t)cm * c.D + cn] = f2h(h2f((uint16_t)cxres) + out);
    }
  }
}

template <int M>
__global__ __launch_bounds__(kT) void layer_item_kernel(FusedArgs a) {
  __shared__ ItemLds<M> L;
  TL1_DECL;
#ifdef DFSSM_TIMELINE
  if (ltix() < kTl1Stamps) tl1_s[ltix()] = 0ull;
  __syncthreads();
  unsigned long long* tl = tl1_s;
#else
  unsigned long long* tl = nullptr;
#endif
  TL1(0);
  const ItemCtx c = item_ctx(a);
  const uint32_t epoch_raw = lds_dev(a.launches + c.w);  // used (tag_of) only after the first phase
  if (ltix() < kCT) control_path<M>(L, a, c, epoch_raw, tl);
  else stream_path<M>(L, a, c, epoch_raw, tl);
  __syncthreads();  // B14: every wave of this workgroup has read its launch count
  if (ltix() == 0) sts_dev(a.launches + c.w, epoch_raw + 1u);
  TL1(13);
#ifdef DFSSM_TIMELINE
  __syncthreads();
  if (ltix() < kTl1Stamps && c.w < kTl1Wg) dfssm_timeline1[epoch_raw % kTl1Slots][c.w][ltix()] = tl1_s[ltix()];
#endif
}

// Grid for the shapes this kernel takes: NI = H P / 16 items, a power of two in [32, 256] that
// divides 2 d_state (B | C rows per workgroup) and fits the device (one workgroup per CU, each
// fitting at least once); 16 LoRA ranks x NI / 16 slices of d_model of at most kMaxSlice columns;
// D / 32 phase-C workgroups (a multiple of 16, at most NI) whose LoRA slices of d_inner are at
// most kMaxSlice wide; d_model and d_inner multiples of 512 up to 4096.
int item_plan(int cus, int per_cu, int M, int D, int DI, int H, int P) {
  if (M < 1 || M > 4 || P % 16 || D % 512 || DI % 512 || D > kMaxK || DI > kMaxK) return 0;
  const int NI = H * (P / 16);
  if (NI < 32 || NI > kMaxNI || (NI & (NI - 1)) || 256 % NI) return 0;
  if (per_cu < 1 || NI > cus) return 0;
  if (D / (NI / DFSSM_LORA_R) > kMaxSlice) return 0;
  const int gC = D / kRC;
  if (gC % DFSSM_LORA_R || gC > NI || DI / (gC / DFSSM_LORA_R) > kMaxSlice) return 0;
  if (33 + 256 / NI > kMaxRowsA) return 0;
  return NI;
}

template <int M>
static int item_occupancy() {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&layer_item_kernel<M>),
                                                   kT, 0) != hipSuccess)
    return 0;
  return per_cu;
}

int item_layer_grid(int M, int D, int DI, int H, int P) {
  static int cus_of[16] = {0};
  static int occ[16][5] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16 || M < 1 || M > 4) return 0;
  if (cus_of[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    occ[dev][1] = item_occupancy<1>();
    occ[dev][2] = item_occupancy<2>();
    occ[dev][3] = item_occupancy<3>();
    occ[dev][4] = item_occupancy<4>();
    cus_of[dev] = cus > 0 ? cus : -1;
  }
  if (cus_of[dev] < 0) return 0;
  return item_plan(cus_of[dev], occ[dev][M], M, D, DI, H, P);
}

hipError_t launch_item_layer(const FusedArgs& a, int M, hipStream_t s) {
  const int G = item_layer_grid(M, a.D, a.DI, a.H, a.P);
  if (G < 1) return hipErrorNotSupported;
  switch (M) {
    case 1: hipLaunchKernelGGL(layer_item_kernel<1>, dim3(G), dim3(kT), 0, s, a); break;
    case 2: hipLaunchKernelGGL(layer_item_kernel<2>, dim3(G), dim3(kT), 0, s, a); break;
    case 3: hipLaunchKernelGGL(layer_item_kernel<3>, dim3(G), dim3(kT), 0, s, a); break;
    case 4: hipLaunchKernelGGL(layer_item_kernel<4>, dim3(G), dim3(kT), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace dfssm

#ifdef DFSSM_TIMELINE
// Copies the item layer's stamp array (kTl1Slots x kTl1Wg x kTl1Stamps u64) to host memory.
extern "C" int dfssm_timeline1_read(void* host, size_t bytes) {
  if (bytes < sizeof(dfssm::dfssm_timeline1)) return -5;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(dfssm::dfssm_timeline1), sizeof(dfssm::dfssm_timeline1));
}
#endif
