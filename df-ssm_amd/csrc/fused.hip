// One decode layer for 1..4 sequences in a single launch (gfx950).
//
// At batch <= 4 a layer moves ~7.8 MB, and the five-kernel form spends most of its time in
// launch gaps and per-kernel ramp-up. Here one grid of G workgroups (1024 threads, one per CU,
// all co-resident) runs the layer in three phases:
//   A  in_proj: workgroup w < gA = ceil(IPO/64) owns output rows 64w..64w+63: RMSNorm, int8
//      quantizer and the activation bit planes of its own GEMV chunks (the inputs are 4 KiB of
//      x, L2-resident), the packed-bit GEMV, dequantization, LoRA, and per row type: the gate
//      z sigma(z) (z rows), conv + SiLU (x, B, C rows), softplus dt and exp(dt A) (dt rows).
//      Workgroups gA..gA+15 compute the 16 LoRA intermediates (one rank each); the GEMV
//      workgroups pick them up just before their epilogue. (Slice partials published by the
//      GEMV workgroups themselves, as the item-organised layer does, measured slower here: the
//      GEMV workgroups reach their RMSNorm ~2 us after the LoRA workgroups would.)
//   B  SSM + gate: item (sequence, head, 16-row block); two waves per item poll the words the
//      item needs (gate, x, B, C, dt) into LDS, then every wave updates one fp32 state row and
//      writes its g.
//   C  out_proj: workgroup w < gC = D/RC (RC = 32 rows per group, 64 when D/32 + 16 groups do
//      not fit the grid) reads all of g, runs the gated RMSNorm prologue and the GEMV of its rows
//      and adds the residual into x; workgroups gC..gC+15 compute the out_proj LoRA
//      intermediates as in phase A.
// The prologues and GEMVs are bound by VALU issue (16 waves share the CU's four 16-lane SIMDs):
// the quantizer's bit planes are built once per 64 values with 8 ballots, stored whole.
// The weights and the state do not depend on the activations, so each workgroup issues those
// loads first.
//
// Workgroup barriers order LDS only (lds_barrier): waves of a workgroup never hand each other
// data through global memory, and a full barrier would first wait for every global store of the
// wave to be acknowledged.
//
// Data passed between workgroups of one launch travels as 32-bit words (tag << 16) | fp16 value,
// stored and loaded with device-scope (agent) coherent accesses, which do not hit stale lines of
// another XCD's L2. The tag is the launch's epoch mod 2^16; workgroup w keeps its own launch count
// in the workspace (read at the start, written back at the end, by w alone), so every workgroup
// of a launch derives the same epoch without any shared counter. A consumer polls the data words
// it needs until they carry the current tag: one memory round trip, no flags, no clearing (every
// word is rewritten by every launch). A 32-bit store
// is single-copy atomic, so tag and value always arrive together. Every poll is bounded: on a
// timeout the thread sets bit 2 of the workspace error flag and goes on, so the grid always
// drains (the host reports the error).
//
// Arithmetic is that of prep_kernel + proj_kernel + ssm_kernel; every sum that the kernels
// split differently (sum of squares, LoRA intermediate and LoRA term, C.h readout) is a sum of
// exactly representable products accumulated in fp64, and integer sums are exact.
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

constexpr int kFT = 1024;
constexpr int kFW = kFT / 64;
constexpr int kFMaxK = 5120;
constexpr int kFMaxCPW = (kFMaxK / 128 + kFW - 1) / kFW;
// out_proj in RG-row groups (RG = 16 or 32): thread t owns row t % RG and half-chunks
// u = t / RG + (1024 / RG) j
template <int RG>
constexpr int kCR = (2 * (kFMaxK / 128) + kFT / RG - 1) / (kFT / RG);
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
constexpr uint32_t kSpinMax = 1u << 18;
constexpr int kMaxItems = kFW / 2;  // SSM items per workgroup (two polling waves each)
// at batch M: at most 2 M items per workgroup (the plan checks it), so that the per-item
// registers held through phase B's polls scale with the batch
template <int M>
constexpr int kItemsOf = 2 * M < kMaxItems ? 2 * M : kMaxItems;
// Multi-layer launch: whether a workgroup issues its loads of the next layer's weights before it
// waits for that layer's input (true), or only after (false: measured the same per step at batch
// 1, with less memory traffic while the previous layer's phase C runs).
constexpr bool kPrefetchNextLayer = false;

// Thread and workgroup index, opaque to the optimizer: addresses derived from them are computed
// where they are used instead of being hoisted to the kernel start and kept live (in registers)
// across all three phases.
__device__ __forceinline__ int tix() {
  int t = __builtin_amdgcn_workitem_id_x();
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int bix() {
  int t = __builtin_amdgcn_workgroup_id_x();
  asm volatile("" : "+s"(t));
  return t;
}

// Profiling builds (-DDFSSM_TIMELINE, libdfssm_hip_timeline.so): wall-clock stamps
// (s_memrealtime, 100 MHz) of the phases of every workgroup, kept in LDS by thread 0 and written
// at the end of the launch to dfssm_timeline[launch % kTlSlots][workgroup][stamp]; read on the host
// with dfssm_timeline_read. Product builds compile TL(k) to nothing.
#ifdef DFSSM_TIMELINE
constexpr int kTlSlots = 64, kTlWg = 256, kTlStamps = 16;
__device__ unsigned long long dfssm_timeline[kTlSlots][kTlWg][kTlStamps];
__shared__ unsigned long long tl_s[kTlStamps];
#define TL_DECL
#define TL(k)                                                                   \
  do {                                                                          \
    if (tix() == 0) tl_s[k] = __builtin_amdgcn_s_memrealtime();                 \
  } while (0)
#define TL_FLUSH(slot)                                                          \
  do {                                                                          \
    if (tix() < kTlStamps && bix() < kTlWg)                                     \
      dfssm_timeline[(slot) % kTlSlots][bix()][tix()] = tl_s[tix()];            \
  } while (0)
#else
#define TL_DECL
#define TL(k) do {} while (0)
#define TL_FLUSH(slot) do {} while (0)
#endif

// XCD-scope exchange (between workgroups of one XCD, which share its L2): a plain store goes to
// the L2 (the per-CU L1 is write-through), and a non-temporal load neither allocates in nor hits
// the per-CU L1, so it reads the L2. Measured two-workgroup round trip 0.5 us, against 0.9 us on
// one XCD and 1.2 us across XCDs for device-scope (sc1) accesses, which go past the L2. Valid only
// for words that no CU reads with a plain load in the same launch (a plain load would allocate the
// line in that CU's L1).
template <class T>
__device__ __forceinline__ T ld_xcd(const T* p) {
  asm volatile("" ::: "memory");  // a fresh load at every call (polls)
  return __builtin_nontemporal_load(p);
}
template <class T>
__device__ __forceinline__ void st_xcd(T* p, T v) {
  // a relaxed atomic store of wavefront scope is a plain global store (no cache-policy bits; the
  // workgroup scope would add sc0), and unlike a plain C++ store it is neither merged nor dropped
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
// Exchange of the one-launch layers: device scope (XL false) or XCD scope (XL true).
template <bool XL, class T>
__device__ __forceinline__ T ld_x(const T* p) {
  if constexpr (XL) return ld_xcd(p);
  else return ld_dev(p);
}
template <bool XL, class T>
__device__ __forceinline__ void st_x(T* p, T v) {
  if constexpr (XL) st_xcd(p, v);
  else st_dev(p, v);
}

// Words of one SSM item, polled by two waves and shared through LDS.
struct ItemLds {
  uint32_t bc[DFSSM_WAVE * 2];  // B (pairs 0..63) and C (pairs 64..127), fp16 pairs
  uint16_t x[16], gate[16];     // x and z sigma(z) of the item's 16 rows
  float dt, abar;               // softplus dt and exp(dt A) of the item's head
};

template <int M>
struct FusedLds {
  uint32_t planes[M][kFMaxK / 32][8];
  int T[M][64][kFW + 1];  // per-wave GEMV partials of each row (padded against bank conflicts)
  uint16_t xn[kFMaxK];
  double rd[M][kFW];   // per-wave partial sums (squares; LoRA rank)
  double rq[M][4][kFW];  // per-wave LoRA sums of up to 4 ranks (XCD-partitioned layer)
  float rf[M][kFW];    // per-wave partial amax
  int ri[M][kFW];      // per-wave partial sum q
  float hl[M][DFSSM_LORA_R];
  float xs[M];
  ItemLds item[kMaxItems];
};

// Epilogue inputs of one output row, loaded ahead of the GEMV. Thread t works on row t / 16 of
// the group with wave partial / LoRA rank s = t % 16; threads s < M also finalize sequence s.
// Every field is a raw load (each in its own register), made unconditionally from clamped
// indices and used only in the epilogue: loads complete in issue order, so converting or
// packing a loaded value here (or a load inside a branch, whose join waits for all loads) would
// make the workgroup wait for the weight stream before its prologue starts.
struct EpiRow {
  uint32_t cw01, cw23;
  float bias, alog;          // dt rows: dt_bias and A_log of the head (A = -exp(A_log) later)
  int la;                    // LoRA A[n][s]
  uint32_t ws, as, cs01, cs2, cb, xres;  // cs01: conv state words 0 | 1 << 16, one (unaligned) load
};

// Conv-state update of one row, stored after the row group's outputs.
struct ConvPend {
  uint16_t* p;
  uint16_t v0, v1, v2;
};

// Columns of the activation values that thread t < K / 8 holds in the norm and the prologue (K is a
// multiple of 512, checked with the model dims). Contiguous map (IL false): columns 8 t .. 8 t + 7.
// Interleaved map (IL true, used where the values are polled): wave w covers columns 512 w ..
// 512 w + 511 as 256 adjacent pairs, lane l the pairs l, l + 64, l + 128, l + 192, so that each
// wave-wide poll of one pair is one contiguous 512 bytes of tagged words: a poll round of a
// workgroup then touches each cache line of the polled words once (with the contiguous map, four
// times). Threads >= K / 8 map as thread 0 (their values are never used).
template <bool IL>
struct PairMap {
  int base;  // pair j at column base + 128 j (IL) or base + 2 j
  __device__ __forceinline__ int col(int j) const { return base + (IL ? 128 : 2) * j; }
};
template <bool IL>
__device__ __forceinline__ PairMap<IL> pair_map(int K) {
  const int t = tix() < K / 8 ? tix() : 0;
  return PairMap<IL>{IL ? 512 * (t >> 6) + 2 * (t & 63) : 8 * t};
}

// Activations (IN only) and their norm weights, 4 pairs at pair_map's columns.
template <int M>
struct PIn {
  u32x4 av[M];
  f32x4 w0, w1;  // weights of values 0..3 and 4..7 (pairs 0, 1 and 2, 3)
};

template <int M, bool OUT, bool IL>
__device__ __forceinline__ void load_pin(PIn<M>& pi, const uint16_t* act, int K, const float* norm_w) {
  // unconditional loads from a clamped column: a load inside a branch makes the compiler wait for
  // all loads at the join
  const PairMap<IL> pm = pair_map<IL>(K);
  if (IL) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) pi.av[m][j] = OUT ? 0u : *(const uint32_t*)(act + (size_t)m * K + pm.col(j));
    f32x2 w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = *(const f32x2*)(norm_w + pm.col(j));
    pi.w0 = f32x4{w[0][0], w[0][1], w[1][0], w[1][1]};
    pi.w1 = f32x4{w[2][0], w[2][1], w[3][0], w[3][1]};
  } else {
#pragma unroll
    for (int m = 0; m < M; ++m)
      pi.av[m] = OUT ? u32x4{0u, 0u, 0u, 0u} : *(const u32x4*)(act + (size_t)m * K + pm.base);
    pi.w0 = *(const f32x4*)(norm_w + pm.base);
    pi.w1 = *(const f32x4*)(norm_w + pm.base + 4);
  }
}

// The 4 pairs of this thread at pair_map's columns of an fp16 row in LDS or memory.
template <bool IL>
__device__ __forceinline__ u32x4 load_pairs(const uint16_t* row, const PairMap<IL>& pm) {
  if (!IL) return *(const u32x4*)(row + pm.base);
  u32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = *(const uint32_t*)(row + pm.col(j));
  return v;
}
template <bool IL>
__device__ __forceinline__ void store_pairs(uint16_t* row, const PairMap<IL>& pm, const uint32_t (&o)[4]) {
  if (!IL) {
    *(u32x4*)(row + pm.base) = u32x4{o[0], o[1], o[2], o[3]};
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) *(uint32_t*)(row + pm.col(j)) = o[j];
}

__device__ __forceinline__ void load_bits(u32x4 (&wb)[kFMaxCPW], const uint32_t* bits, int grp, int K) {
  const int lane = tix() & 63, wave = tix() >> 6, CH = K / 128;
  const u32x4* b = (const u32x4*)bits + (size_t)grp * CH * 64 + lane;
#pragma unroll
  for (int j = 0; j < kFMaxCPW; ++j) {
    const int c = wave + kFW * j;
    wb[j] = c < CH ? ld_nt(b + (size_t)c * 64) : u32x4{0u, 0u, 0u, 0u};
  }
}

// RG-row group `grp` (rows RG grp .. RG grp + RG - 1 of the 64-row tiles): thread (row
// r = lane % RG, u = (64 / RG) wave + lane / RG + (1024 / RG) j) loads words 2h, 2h + 1 of chunk c,
// cu = u = 2c + h.
template <int RG>
__device__ __forceinline__ void load_bits_rg(u32x2 (&wb)[kCR<RG>], const uint32_t* bits, int grp, int K) {
  const int lane = tix() & 63, wave = tix() >> 6, CH = K / 128;
  const u32x4* b = (const u32x4*)bits + (size_t)(grp / (64 / RG)) * CH * 64 + (grp % (64 / RG)) * RG + lane % RG;
#pragma unroll
  for (int j = 0; j < kCR<RG>; ++j) {
    const int cu = (64 / RG) * wave + lane / RG + (kFT / RG) * j;
    wb[j] = cu < 2 * CH ? __builtin_nontemporal_load((const u32x2*)(b + (size_t)(cu >> 1) * 64) + (cu & 1))
                        : u32x2{0u, 0u};
  }
}

// Row n = RG grp + tid / 16; the sequence-specific inputs for m = tid % 16 < M (threads
// s >= M and rows past N load row / sequence 0's values, never used).
template <int M, bool IN, int RG = 64>
__device__ __forceinline__ EpiRow load_epi(const FusedArgs& a, int grp) {
  EpiRow e;
  const int tid = tix(), s = tid & 15, n0 = grp * RG + (tid >> 4);
  const int N = IN ? a.IPO : a.D;
  const int n = n0 < N ? n0 : N - 1;
  const int m = s < M ? s : 0;
  e.la = (IN ? a.in_lA : a.out_lA)[(size_t)n * DFSSM_LORA_R + s];
  e.as = (IN ? a.in_lAs : a.out_lAs)[n];
  e.ws = (IN ? a.in_ws : a.out_ws)[n];
  if (IN) {
    int ch = n - a.DI, dtr = n - (2 * a.DI + 2 * a.N);
    ch = ch < 0 ? 0 : (ch >= a.C ? a.C - 1 : ch);
    dtr = dtr < 0 ? 0 : dtr;
    const uint16_t* cs = a.conv + ((size_t)m * a.C + ch) * 3;
    __builtin_memcpy(&e.cs01, cs, 4);
    e.cs2 = cs[2];
    const uint32_t* wc = (const uint32_t*)(a.conv_w + (size_t)ch * 4);
    e.cw01 = wc[0]; e.cw23 = wc[1];
    e.cb = a.conv_b[ch];
    e.bias = a.dt_bias[dtr];
    e.alog = a.A_log[dtr];
    e.xres = 0u;
  } else {
    e.xres = a.x[(size_t)m * a.D + n];
    e.cs01 = e.cs2 = e.cw01 = e.cw23 = e.cb = 0u;
    e.bias = e.alog = 0.0f;
  }
  return e;
}

__device__ __forceinline__ uint32_t tagged(uint32_t tag, uint16_t v) { return (tag << 16) | v; }

// Poll a tagged word until it carries `tag`; returns its fp16 bits. After a timeout (`ok`
// false) polls return at once. One load in flight per poll: keeping two in flight (staggered)
// made the phase hand-offs slower, the extra poll traffic delaying the producers' stores, and
// sleeping 64 or 256 clocks between polls measured the same as 64.
__device__ __forceinline__ void poll_timeout(bool& ok, int* err) {
  ok = false;
  atomicOr(err, 4);
}
template <bool XL = false>
__device__ __forceinline__ uint32_t poll1(const uint32_t* p, uint32_t tag, bool& ok, int* err) {
  uint32_t v = ld_x<XL>(p);
  for (uint32_t it = 0; ok && (v >> 16) != tag; ++it) {
    if (it == kSpinMax) {
      poll_timeout(ok, err);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    v = ld_x<XL>(p);
  }
  return v & 0xffffu;
}
__device__ __forceinline__ bool tag_ok2(uint64_t v, uint32_t tag) {
  return ((uint32_t)v >> 16) == tag && ((uint32_t)(v >> 32) >> 16) == tag;
}
__device__ __forceinline__ uint32_t pack2(uint64_t v) { return ((uint32_t)v & 0xffffu) | ((uint32_t)(v >> 32) << 16); }

// N pairs of adjacent tagged words at p + 2 S j (8-byte aligned), all loads in flight together;
// out[j] = the pair's two fp16 values packed low | high.
template <int N, int S, bool XL = false>
__device__ __forceinline__ void pollv(const uint32_t* p, uint32_t tag, uint32_t (&out)[N], bool& ok, int* err) {
  uint64_t v[N];
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = ld_x<XL>((const uint64_t*)p + S * j);
  for (uint32_t it = 0; ok; ++it) {
    bool good = true;
#pragma unroll
    for (int j = 0; j < N; ++j) good = good && tag_ok2(v[j], tag);
    if (good) break;
    if (it == kSpinMax) {
      poll_timeout(ok, err);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (!tag_ok2(v[j], tag)) v[j] = ld_x<XL>((const uint64_t*)p + S * j);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) out[j] = pack2(v[j]);
}

// RMSNorm of the M activation rows (K columns) into L.xn, one row at a time, with `body(m, mx)`
// run after each row's normalized values are in LDS (mx = this thread's max |xn|). IN: x loaded
// ahead (pi.av); OUT: the gated g of this launch, polled from its tagged words (gT).
template <int M, bool OUT, bool IL, class Body>
__device__ __forceinline__ void norm_rows(FusedLds<M>& L, const PIn<M>& pi, const uint32_t* gT, int K,
                                          uint32_t tag, int* err, Body body) {
  const int tid = tix(), lane = tid & 63, wave = tid >> 6;
  const bool has_v = tid < K / 8;
  const float wv[8] = {pi.w0[0], pi.w0[1], pi.w0[2], pi.w0[3], pi.w1[0], pi.w1[1], pi.w1[2], pi.w1[3]};
  bool ok = true;
  for (int m = 0; m < M; ++m) {
    u32x4 av = {0u, 0u, 0u, 0u};
    double part = 0.0;
    if (has_v) {
      if (OUT) {
        uint32_t w4[4];
        const PairMap<IL> pm = pair_map<IL>(K);
        pollv<4, IL ? 64 : 1>(gT + (size_t)m * K + pm.base, tag, w4, ok, err);
        av = u32x4{w4[0], w4[1], w4[2], w4[3]};
      } else {
        av = pi.av[m];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double xv = (double)h2f((uint16_t)(av[e >> 1] >> (16 * (e & 1))));
        part += xv * xv;
      }
    }
    const double wsum = wave_sum_dpp_f64(part);
    if (lane == 0) L.rd[m][wave] = wsum;
    lds_barrier();  // also: every wave is done with the previous row's xn
    if (OUT && m == 0) TL(14);
    double ss = 0.0;
#pragma unroll
    for (int w = 0; w < kFW; ++w) ss += L.rd[m][w];
    const float var = (float)ss * (1.0f / (float)K);
    const float r = 1.0f / sqrt_rn(var + 1e-5f);
    float mx = 0.0f;
    if (has_v) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = r16((h2f((uint16_t)(av[e >> 1])) * r) * wv[e]);
        const float x1 = r16((h2f((uint16_t)(av[e >> 1] >> 16)) * r) * wv[e + 1]);
        mx = fmaxf(mx, fmaxf(fabsf(x0), fabsf(x1)));
        o[e >> 1] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
      }
      store_pairs<IL>(L.xn, pair_map<IL>(K), o);
    }
    body(m, mx);
  }
}

// Bit planes of 64 int8 values (q of value k0 + lane) into the 16 words at dst (LDS, 16-byte
// aligned), from lane 0: word 2b + h = bit b of values k0 + 32h .. k0 + 32h + 31, i.e. each
// plane's 64-bit ballot stored whole (one 64-bit register move per plane).
__device__ __forceinline__ void planes_store64(uint32_t* dst, int q, int lane) {
  uint64_t b64[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) b64[b] = __ballot((q >> b) & 1);
  if (lane == 0) {
    uint64_t* d = (uint64_t*)dst;
#pragma unroll
    for (int b = 0; b < 8; ++b) d[b] = b64[b];
  }
}

// Projection prologue (GEMV workgroups): per row the amax, the quantization scale, and each
// wave's bit planes of its own GEMV chunks (no barrier before the GEMV) with their sum q.
// CW: the wave's chunks are CW consecutive ones per round of CW * 16 (those its GEMV reads).
template <int M, bool OUT, bool IL, int CW = 1>
__device__ void prologue(FusedLds<M>& L, const PIn<M>& pi, const uint32_t* gT, int K, uint32_t tag, int* err) {
  const int tid = tix(), lane = tid & 63, wave = tid >> 6;
  const int CH = K / 128;
  norm_rows<M, OUT, IL>(L, pi, gT, K, tag, err, [&](int m, float mx) {
    const float wmax = wave_max_dpp_f32(mx);
    if (lane == 0) L.rf[m][wave] = wmax;
    lds_barrier();  // publishes xn and the partial maxima
    if (OUT && m == 0) TL(15);
    float amax = L.rf[m][0];
#pragma unroll
    for (int w = 1; w < kFW; ++w) amax = fmaxf(amax, L.rf[m][w]);
    const float xs = quant_scale(amax);
    const float rinv = quant_rcp(xs);
    if (tid == 0) L.xs[m] = xs;
    int qsum = 0;
    for (int c = CW * wave; c < CH; c += (c % CW == CW - 1) ? CW * (kFW - 1) + 1 : 1) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int k0 = 128 * c + 64 * hh;
        const int q = quant_i8(h2f(L.xn[k0 + lane]), rinv);
        qsum += q;
        planes_store64(&L.planes[m][k0 / 32][0], q, lane);
      }
    }
    const int wq = wave_sum_dpp_i32(qsum);
    if (lane == 0) L.ri[m][wave] = wq;
  });
}

// LoRA intermediate of rank r for every row (LoRA workgroups): h[m][r] =
// fp16(sum_k xn_k * Bq[r][k]), fp16 x fp16 products exact in fp32, summed in fp64, stored as a
// tagged word hout[m * 16 + r] with `tag`. OUT (or a polled x): the activations are polled from
// gT until they carry `ptag`.
template <int M, bool OUT, bool IL>
__device__ void lora_rank(FusedLds<M>& L, const uint16_t* x, const uint32_t* gT, int K, const float* norm_w,
                          const uint16_t* lBq, int r, uint32_t* hout, uint32_t tag, int* err, uint32_t ptag) {
  const int tid = tix(), lane = tid & 63, wave = tid >> 6;
  const bool has_v = tid < K / 8;
  PIn<M> pi;
  load_pin<M, OUT, IL>(pi, x, K, norm_w);
  const u32x4 b8 = load_pairs<IL>(lBq + (size_t)r * K, pair_map<IL>(K));
  norm_rows<M, OUT, IL>(L, pi, gT, K, ptag, err, [&](int m, float) {
    double hacc = 0.0;
    if (has_v) {
      const u32x4 xv8 = load_pairs<IL>(L.xn, pair_map<IL>(K));  // this thread's own columns
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xv = h2f((uint16_t)(xv8[e >> 1] >> (16 * (e & 1))));
        const float bv = h2f((uint16_t)(b8[e >> 1] >> (16 * (e & 1))));
        hacc += (double)(xv * bv);
      }
    }
    const double hw = wave_sum_dpp_f64(hacc);
    lds_barrier();  // the sum-of-squares partials of this row have been read by every wave
    if (lane == 0) L.rd[m][wave] = hw;
    lds_barrier();
    if (tid < kXRep) {  // one copy per thread
      double t = 0.0;
#pragma unroll
      for (int w = 0; w < kFW; ++w) t += L.rd[m][w];
      st_dev(hout + tid * kHStride + m * DFSSM_LORA_R + r, tagged(tag, f2h((float)t)));
    }
  });
}

// Packed-bit GEMV of one 64-row group: per-wave partials into L.T (no barrier).
template <int M>
__device__ __forceinline__ void gemv_partials(FusedLds<M>& L, const u32x4 (&wb)[kFMaxCPW], int K) {
  const int lane = tix() & 63, wave = tix() >> 6;
  const int CH = K / 128;
  uint32_t cnt[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int b = 0; b < 8; ++b) cnt[m][b] = 0u;
#pragma unroll
  for (int j = 0; j < kFMaxCPW; ++j) {
    const int c = wave + kFW * j;
    if (c < CH) {
#pragma unroll
      for (int sh = 0; sh < 2; ++sh) {  // the two 64-value sets of the chunk
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const u32x4* ps = (const u32x4*)&L.planes[m][c * 4 + 2 * sh][0];
          const u32x4 d0 = ps[0], d1 = ps[1], d2 = ps[2], d3 = ps[3];
          const uint32_t pl[16] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3],
                                   d2[0], d2[1], d2[2], d2[3], d3[0], d3[1], d3[2], d3[3]};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t w = wb[j][2 * sh + h];
#pragma unroll
            for (int b = 0; b < 8; ++b) cnt[m][b] += __builtin_popcount(w & pl[2 * b + h]);
          }
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
    L.T[m][lane][wave] = t;
  }
}

// Packed-bit GEMV of one RG-row group: each thread two words of one row per half-chunk, the
// threads of a wave that share a row summed by lane exchange; per-wave partials into L.T rows
// 0..RG-1.
template <int M, int RG>
__device__ __forceinline__ void gemv_partials_rg(FusedLds<M>& L, const u32x2 (&wb)[kCR<RG>], int K) {
  const int lane = tix() & 63, wave = tix() >> 6;
  const int CH = K / 128;
  uint32_t cnt[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int b = 0; b < 8; ++b) cnt[m][b] = 0u;
#pragma unroll
  for (int j = 0; j < kCR<RG>; ++j) {
    const int cu = (64 / RG) * wave + lane / RG + (kFT / RG) * j;
    if (cu < 2 * CH) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        // the words 2 cu, 2 cu + 1 are the halves of 64-value set cu
        const u32x4* ps = (const u32x4*)&L.planes[m][2 * cu][0];
        const u32x4 d0 = ps[0], d1 = ps[1], d2 = ps[2], d3 = ps[3];
        const uint32_t pl[16] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3],
                                 d2[0], d2[1], d2[2], d2[3], d3[0], d3[1], d3[2], d3[3]};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const uint32_t w = wb[j][i];
#pragma unroll
          for (int b = 0; b < 8; ++b) cnt[m][b] += __builtin_popcount(w & pl[2 * b + i]);
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
    if (RG == 16) t += __shfl_xor(t, 16);
    t += __shfl_xor(t, 32);
    if (lane < RG) L.T[m][lane][wave] = t;
  }
}

// LoRA intermediates of this phase (threads < 16 M): the first load is issued before the GEMV
// (lora_issue), the poll completes after it (lora_finish) into L.hl; the caller then passes a
// barrier. (A second load issued halfway through the GEMV measured no earlier: a device-scope store
// takes ~1 us to become visible, and the producers store the words shortly before the GEMV starts.)
template <bool XL = false>
__device__ __forceinline__ uint32_t lora_issue(const uint32_t* hsrc, int M) {
  return tix() < M * DFSSM_LORA_R ? ld_x<XL>(hsrc + tix()) : 0u;
}
template <int M, bool XL = false>
__device__ __forceinline__ void lora_finish(FusedLds<M>& L, const uint32_t* hsrc, uint32_t v, uint32_t tag, int* err) {
  const int tid = tix();
  if (tid < M * DFSSM_LORA_R) {
    bool ok = true;
    if ((v >> 16) != tag) v = poll1<XL>(hsrc + tid, tag, ok, err);
    L.hl[tid / DFSSM_LORA_R][tid % DFSSM_LORA_R] = h2f((uint16_t)v);
  }
}

// Epilogue of one 64-row group (after the barrier that publishes L.T and L.hl), 16 threads per
// row: acc = sum over waves s of (2 T_s - sum q_s) and the LoRA term sum_r h_r aq_r as DPP row
// sums (exact: integers, and exactly representable products in fp64); thread s = m then
// finalizes sequence m. IN: z rows store the gate z sigma(z), x/B/C rows conv + SiLU, dt rows
// softplus dt and exp(dt A) (as tagged fp32 words); OUT: the residual add into x (also kept in
// *xkeep and, for a next layer of the same launch, published to every copy at xpub).
// XL (XCD-partitioned layer): the words go to this XCD's copies with XCD-scope stores.
template <int M, bool IN, int RG = 64, bool XL = false>
__device__ ConvPend epilogue(FusedLds<M>& L, const FusedArgs& a, const EpiRow& er, int grp, uint32_t tag,
                             uint32_t* xpub = nullptr, uint32_t* xkeep = nullptr, int xcd = 0) {
  ConvPend cp{nullptr, 0, 0, 0};
  const int tid = tix(), s = tid & 15, j = tid >> 4;
  const int N = IN ? a.IPO : a.D;
  const int n = grp * RG + j;
  const float aq = r16((float)(int8_t)er.la * h2f((uint16_t)er.as));
  int accm = 0;
  double lom = 0.0;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int part = row_sum_i32(2 * L.T[m][j][s] - L.ri[m][s]);
    const double lo = row_sum_f64((double)L.hl[m][s] * (double)aq);
    if (s == m) {
      accm = part;
      lom = lo;
    }
  }
  if (s >= M || j >= RG || n >= N) return cp;
  const int m = s;
  const float y = r16(r16(r16((float)accm) * L.xs[m]) * h2f((uint16_t)er.ws));
  float out = r16((float)lom + y);
  if (IN) {
    const int ch = n - a.DI, dtr = n - (2 * a.DI + 2 * a.N);
    if (ch < 0) {  // z row: the gate z sigma(z)
      const float sg = r16(1.0f / (1.0f + dev_expf(-out)));
      out = r16(out * sg);
    } else if (ch < a.C) {
      // depthwise conv (k = 4) + SiLU; the (M, C, 3) fp16 state shifts left (stored later); the B
      // and C channels go to the polled copies (bcT), the x channels to projT
      const uint16_t xo = f2h(out);
      cp = ConvPend{a.conv + ((size_t)m * a.C + ch) * 3, (uint16_t)(er.cs01 >> 16), (uint16_t)er.cs2, xo};
      const float xv = h2f(xo);
      float o = h2f((uint16_t)er.cs01) * h2f((uint16_t)er.cw01);
      o = o + h2f((uint16_t)(er.cs01 >> 16)) * h2f((uint16_t)(er.cw01 >> 16));
      o = o + h2f((uint16_t)er.cs2) * h2f((uint16_t)er.cw23);
      o = o + xv * h2f((uint16_t)(er.cw23 >> 16));
      o = o + h2f((uint16_t)er.cb);
      const float sig = 1.0f / (1.0f + dev_expf(-o));
      out = o * sig;
    } else {  // dt row of head dtr
      const float dt = dev_log1pf(dev_expf(out + er.bias));
      const float abar = dev_expf(dt * -dev_expf(er.alog));
      uint64_t* w = a.dtT + (XL ? (size_t)xcd * kDtStride : 0) + ((size_t)m * a.H + dtr) * 2;
      st_x<XL>(w, ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, dt));
      st_x<XL>(w + 1, ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, abar));
      return cp;
    }
    const uint32_t word = tagged(tag, f2h(out));
    const int bc = ch - a.DI;  // B | C channel index, or < 0
    if (bc >= 0) {
      if (XL) {
        st_xcd(a.bcT + xcd * kBcStride + m * 2 * a.N + bc, word);
      } else {
#pragma unroll
        for (int c = 0; c < kXRep; ++c) st_dev(a.bcT + c * kBcStride + m * 2 * a.N + bc, word);
      }
    } else {
      st_x<XL>(a.projT + (size_t)m * a.IPO + n, word);
    }
  } else {
    const uint16_t xv = f2h(h2f((uint16_t)er.xres) + out);
    a.x[(size_t)m * a.D + n] = xv;
    if (xkeep) *xkeep = xv;
    if (xpub) {  // the next layer's input, to every copy
#pragma unroll
      for (int c = 0; c < kXRep; ++c) st_dev(xpub + (size_t)c * kXStride + (size_t)m * a.D + n, tagged(tag, xv));
    }
  }
  return cp;
}

__device__ __forceinline__ void store_conv(const ConvPend& cp) {
  if (cp.p) {
    cp.p[0] = cp.v0;
    cp.p[1] = cp.v1;
    cp.p[2] = cp.v2;
  }
}

// Item `it` = (sequence m, head, 16-row block pb); NI = H * P / 16 items per sequence.
struct Item {
  int m, head, pb;
};
__device__ __forceinline__ Item item_of(const FusedArgs& a, int it) {
  const int PB = a.P / 16, NI = a.H * PB;
  const int m = it / NI, rem = it % NI;
  return Item{m, rem / PB, rem % PB};
}

// This thread's two state columns of the item's row p = 16 pb + wave.
__device__ __forceinline__ float* state_row(const FusedArgs& a, const Item& t) {
  const int lane = tix() & 63, wave = tix() >> 6;
  return a.h + (((size_t)t.m * a.H + t.head) * a.P + t.pb * 16 + wave) * a.N + 2 * lane;
}

// Poll the words of item k (waves 2k and 2k + 1) into L.item[k]. Wave 2k: B and C (lane l:
// pairs l and 64 + l of the 128); wave 2k + 1: lanes 0..15 x, 16..31 the gate of the 16 rows,
// lanes 32 and 33 dt and exp(dt A).
// XL: from this XCD's copies (xcd), with XCD-scope loads.
template <int M, bool XL = false>
__device__ void poll_item(FusedLds<M>& L, const FusedArgs& a, int k, const Item& t, uint32_t tag, int xcd = 0) {
  const int lane = tix() & 63, wave = tix() >> 6;
  const uint32_t* pr = a.projT + (size_t)t.m * a.IPO;
  bool ok = true;
  if (wave == 2 * k) {
    uint32_t w[2];  // pairs lane (B) and 64 + lane (C): each wave-wide load one contiguous 512 bytes
    pollv<2, 64, XL>(a.bcT + (XL ? xcd : bix() % kXRep) * kBcStride + t.m * 2 * a.N + 2 * lane, tag, w, ok, a.err);
    L.item[k].bc[lane] = w[0];
    L.item[k].bc[DFSSM_WAVE + lane] = w[1];
  } else if (wave == 2 * k + 1 && lane < 34) {
    // lanes 0..31 poll 32-bit words (tag in the high half), lanes 32 and 33 64-bit words (tag in
    // the high word), all in one loop so that neither set waits for the other's round trips
    const int r0 = t.head * a.P + 16 * t.pb;
    const bool w32 = lane < 32;
    // every lane loads both kinds (from valid addresses): no divergent loads inside the loop
    const uint32_t* p32 = (lane & 31) < 16 ? pr + a.DI + r0 + (lane & 15) : pr + r0 + (lane & 15);
    const uint64_t* p64 = a.dtT + (XL ? (size_t)xcd * kDtStride : 0) + ((size_t)t.m * a.H + t.head) * 2 + (lane & 1);
    auto ready = [&](uint32_t x, uint64_t y) { return w32 ? (x >> 16) == tag : (uint32_t)(y >> 32) == tag; };
    uint32_t va = ld_x<XL>(p32);
    uint64_t vb = ld_x<XL>(p64);
    for (uint32_t it = 0; ok && !ready(va, vb); ++it) {
      if (it == kSpinMax) {
        poll_timeout(ok, a.err);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      va = ld_x<XL>(p32);
      vb = ld_x<XL>(p64);
    }
    const uint64_t r = w32 ? (uint64_t)va : vb;
    if (lane < 16) L.item[k].x[lane] = (uint16_t)r;
    else if (lane < 32) L.item[k].gate[lane - 16] = (uint16_t)r;
    else if (lane == 32) L.item[k].dt = __builtin_bit_cast(float, (uint32_t)r);
    else L.item[k].abar = __builtin_bit_cast(float, (uint32_t)r);
  }
}

// SSM + gate of item k (after the barrier that publishes L.item[k]): wave w owns state row
// p = 16 pb + w, lane l the state columns 2l, 2l+1.
template <int M>
__device__ __forceinline__ void ssm_item(FusedLds<M>& L, const FusedArgs& a, int k, const Item& t, f32x2 h0,
                                         float Dh, uint32_t tag) {
  const int lane = tix() & 63, wave = tix() >> 6;
  const int p = t.pb * 16 + wave;
  const ItemLds& I = L.item[k];
  const uint32_t bp = I.bc[lane], cp = I.bc[DFSSM_WAVE + lane];
  const float xv = h2f(I.x[wave]);
  const float X = xv * I.dt;
  f32x2 hv;
  hv.x = __builtin_fmaf(I.abar, h0.x, X * h2f((uint16_t)bp));
  hv.y = __builtin_fmaf(I.abar, h0.y, X * h2f((uint16_t)(bp >> 16)));
  double acc = (double)h2f((uint16_t)cp) * (double)hv.x + (double)h2f((uint16_t)(cp >> 16)) * (double)hv.y;
  st_dev((uint64_t*)state_row(a, t), __builtin_bit_cast(uint64_t, hv));
  acc = wave_sum_dpp_f64(acc);
  if (lane == 0) {
    const float y = r16((float)acc + xv * Dh);
    const float gv = r16(y * h2f(I.gate[wave]));
    st_dev(a.gT + (size_t)t.m * a.DI + t.head * a.P + p, tagged(tag, f2h(gv)));
  }
}

// Multi-layer launch, start of layer l > first: wave 0 waits until the first x word of every
// out_proj group (row RC g of every sequence) of the previous layer carries `tag`, polling one
// word per group (the whole of x is polled afterwards, by the threads that use it). This keeps the
// workgroups that are done early from flooding memory with polls of all of x (or of their SSM
// items' words) while the previous layer's phase C runs. The caller passes a barrier next.
template <int M, int RC>
__device__ __forceinline__ void wait_prev_layer(const uint32_t* xsrc, int D, uint32_t tag, int* err) {
  if (tix() >= 64) return;
  const int lane = tix(), gC = D / RC;
  constexpr int kW = (M * (kFMaxK / 32) + 63) / 64;  // words per lane
  for (int j = 0; j < kW; ++j) {
    const int idx = lane + 64 * j;
    if (idx >= M * gC) break;
    const uint32_t* p = xsrc + (size_t)(idx / gC) * D + (size_t)(idx % gC) * RC;
    uint32_t v = ld_dev(p);
    for (uint32_t it = 0; (v >> 16) != tag; ++it) {
      if (it == kSpinMax) {
        atomicOr(err, 4);
        break;
      }
      __builtin_amdgcn_s_sleep(4);
      v = ld_dev(p);
    }
  }
}

// Layer l of a multi-layer launch: every per-layer pointer advanced by l strides.
__device__ __forceinline__ FusedArgs at_layer(const FusedArgs& a, const FusedStrides& st, int l) {
  FusedArgs b = a;
  const long long k = l;
#define DFSSM_ADV(f) b.f = (decltype(b.f))((const char*)a.f + st.f * k)
  DFSSM_ADV(in_bits); DFSSM_ADV(in_ws); DFSSM_ADV(in_lA); DFSSM_ADV(in_lAs); DFSSM_ADV(in_lBq);
  DFSSM_ADV(out_bits); DFSSM_ADV(out_ws); DFSSM_ADV(out_lA); DFSSM_ADV(out_lAs); DFSSM_ADV(out_lBq);
  DFSSM_ADV(conv_w); DFSSM_ADV(conv_b); DFSSM_ADV(A_log); DFSSM_ADV(Dp); DFSSM_ADV(dt_bias);
  DFSSM_ADV(norm_w); DFSSM_ADV(ln_w); DFSSM_ADV(h); DFSSM_ADV(conv);
#undef DFSSM_ADV
  b.layer = l;
  return b;
}

// The arguments of every layer of a multi-layer launch, written to device memory (thread l:
// layer l) so that the launch loads each layer's from there instead of keeping the strides and
// the base pointers live in registers through all layers.
__global__ void layer_table_kernel(FusedArgs a0, FusedStrides st, FusedArgs* tab) {
  const int l = blockIdx.x * blockDim.x + threadIdx.x;
  if (l < a0.n_layer) tab[l] = at_layer(a0, st, l);
}

// RC: rows per out_proj group (32, or 64 when D / 32 + 16 groups do not fit the grid).
// MULTI: layers a0.layer .. a0.n_layer - 1 in one launch. A workgroup goes on to the next layer
// as soon as its own part of a layer is done (its weight and state loads for that layer then
// overlap the end of the previous one); phase A of layer l > a0.layer polls x from the tagged
// words that phase C of layer l - 1 publishes (buffer (l - 1) % 2 of xT). Every word a layer
// writes for other workgroups is read by them before the writes of the next layer can start:
// those all wait for the next layer's x, which phase C publishes only after every SSM item of
// the layer is done, and every workgroup that reads x or LoRA words in phase A owns an item.
// The out_proj group of a workgroup (at most one, as the plan requires) keeps its x rows in
// registers from one layer to the next instead of reading them back.
template <int M, int RC, bool MULTI>
__global__ __launch_bounds__(kFT) void layer_fused_kernel(FusedArgs a0, const FusedArgs* __restrict__ tab) {
  __shared__ FusedLds<M> L;
  TL_DECL;
  // The launch's epoch is the first load; its tags are derived where they are used (tag_now):
  // the empty asm keeps the compiler from computing them right after a branch join near the
  // kernel start, where it can only wait for every load issued so far (the weight stream
  // included).
  const uint32_t epoch_raw = ld_dev(a0.launches + bix());
  const int l_end = MULTI ? a0.n_layer : a0.layer + 1;
  uint32_t xkeep = 0u;  // MULTI: this thread's x value of its out_proj row, from the last layer
  for (int l = a0.layer; l < l_end; ++l) {
  // indices re-derived in every layer (opaque, so not hoisted and kept live across layers)
  const int tid = tix(), lane = tid & 63, wave = tid >> 6;
  const int G = gridDim.x, wg = bix();
  const FusedArgs a = MULTI ? tab[l] : a0;  // (scalar loads of this layer's arguments)
  auto tag_of_layer = [&](int layer) {
    uint32_t v = epoch_raw;
    asm volatile("" : "+v"(v));
    return (v * (uint32_t)a0.n_layer + (uint32_t)layer + 1u) & 0xffffu;
  };
  auto tag_now = [&]() { return tag_of_layer(l); };
  const bool poll_x = MULTI && l > a0.layer;  // x of this layer from the previous one's words
  const uint32_t* x_src = a0.xT + (size_t)(((l - 1) & 1) * kXRep + wg % kXRep) * kXStride;
  uint32_t* x_pub = MULTI && l + 1 < l_end ? a0.xT + (size_t)((l & 1) * kXRep) * kXStride : nullptr;
#ifdef DFSSM_TIMELINE
  if (tix() < kTlStamps) tl_s[tix()] = 0ull;
  lds_barrier();
#endif
  TL(0);
  if constexpr (MULTI && !kPrefetchNextLayer) {
    if (poll_x) {
      wait_prev_layer<M, RC>(x_src, a.D, tag_of_layer(l - 1), a.err);
      lds_barrier();
    }
  }
  const int gA = (a.IPO + 63) / 64, gC = a.D / RC;
  const int NI = a.H * (a.P / 16), items = M * NI;
  uint32_t* hA = a.hT;                       // copy 0 (the LoRA workgroups write every copy)
  uint32_t* hC = a.hT + M * DFSSM_LORA_R;
  const uint32_t* hA_mine = hA + (wg % kXRep) * kHStride;  // the copy this workgroup polls
  const uint32_t* hC_mine = hC + (wg % kXRep) * kHStride;

  // ---- loads that do not depend on the activations ----
  u32x4 wa[kFMaxCPW];
  EpiRow ea = {};
  PIn<M> pa;
  if (wg < gA) {  // x first: the prologue needs it before the weights
    load_pin<M, false, MULTI>(pa, a.x, a.D, a.ln_w);
    load_bits(wa, a.in_bits, wg, a.D);
    ea = load_epi<M, true>(a, wg);
  }
  // state row of this workgroup's first SSM item (the other items' rows load before phase B's polls)
  // (unconditional, from a clamped item: see load_pin). Issuing these and the weights only once x
  // is in measured slower (the prologue waits as long for x, and then for the weights).
  const f32x2 h0 = __builtin_nontemporal_load((const f32x2*)state_row(a, item_of(a, wg < items ? wg : items - 1)));
  if constexpr (MULTI && kPrefetchNextLayer) {
    if (poll_x) {
      wait_prev_layer<M, RC>(x_src, a.D, tag_of_layer(l - 1), a.err);
      lds_barrier();
    }
  }

  // ---- phase A: in_proj (workgroups < gA), LoRA ranks (gA .. gA + 15) ----
  if (wg < gA) {
    if (poll_x) prologue<M, true, MULTI>(L, pa, x_src, a.D, tag_of_layer(l - 1), a.err);
    else prologue<M, false, MULTI>(L, pa, nullptr, a.D, 0u, a.err);  // x loaded ahead, no polls
    TL(1);
    for (int grp = wg; grp < gA; grp += G) {
      if (grp != wg) {
        load_bits(wa, a.in_bits, grp, a.D);
        ea = load_epi<M, true>(a, grp);
      }
      const uint32_t hv = lora_issue(hA_mine, M);
      gemv_partials<M>(L, wa, a.D);
      TL(2);
      const uint32_t tag = tag_now();
      lora_finish<M>(L, hA_mine, hv, tag, a.err);
      lds_barrier();
      TL(3);
      store_conv(epilogue<M, true>(L, a, ea, grp, tag));
      TL(4);
      lds_barrier();
    }
  } else if (wg < gA + DFSSM_LORA_R) {
    if (poll_x)
      lora_rank<M, true, MULTI>(L, nullptr, x_src, a.D, a.ln_w, a.in_lBq, wg - gA, hA, tag_now(), a.err,
                         tag_of_layer(l - 1));
    else
      lora_rank<M, false, MULTI>(L, a.x, nullptr, a.D, a.ln_w, a.in_lBq, wg - gA, hA, tag_now(), a.err, 0u);
    TL(4);
  }
  // ---- phase B: SSM + gate ----
  u32x4 wc[RC < 64 ? 1 : kFMaxCPW];
  u32x2 wcr[kCR<RC < 64 ? RC : 16>];
  EpiRow ec = {};
  if (wg < gC) {  // phase-C weights, loaded while phase B runs
    if constexpr (RC < 64) load_bits_rg<RC>(wcr, a.out_bits, wg, a.DI);
    else load_bits(wc, a.out_bits, wg, a.DI);
    ec = load_epi<M, false, RC>(a, wg);
    if (poll_x) ec.xres = xkeep;  // written by this thread in the previous layer
  }
  const int nk = wg < items ? (items - 1 - wg) / G + 1 : 0;  // <= kItemsOf<M>
  if (nk > 0) {
    f32x2 hk[kItemsOf<M>];
    float dk[kItemsOf<M>];
    hk[0] = h0;
#pragma unroll
    for (int k = 0; k < kItemsOf<M>; ++k) {
      if (k < nk) {
        const Item t = item_of(a, wg + k * G);
        if (k > 0) hk[k] = __builtin_nontemporal_load((const f32x2*)state_row(a, t));
        dk[k] = a.Dp[t.head];
      }
    }
    const uint32_t tag = tag_now();
    TL(5);
    for (int k = 0; k < nk; ++k) poll_item<M>(L, a, k, item_of(a, wg + k * G), tag);
    lds_barrier();
    TL(6);
#pragma unroll
    for (int k = 0; k < kItemsOf<M>; ++k)
      if (k < nk) ssm_item<M>(L, a, k, item_of(a, wg + k * G), hk[k], dk[k], tag);
  }
  // ---- phase C: out_proj + residual (workgroups < gC), LoRA ranks (gC .. gC + 15) ----
  TL(7);
  if (wg < gC) {
    lds_barrier();  // LDS reuse after phase A
    PIn<M> pc;
    load_pin<M, true, true>(pc, nullptr, a.DI, a.norm_w);
    const uint32_t tag = tag_now();
    TL(8);
    prologue<M, true, true, RC == 16 ? 2 : 1>(L, pc, a.gT, a.DI, tag, a.err);  // the chunks of the wave's GEMV
    TL(9);
    for (int grp = wg; grp < gC; grp += G) {
      if (grp != wg) {
        if constexpr (RC < 64) load_bits_rg<RC>(wcr, a.out_bits, grp, a.DI);
        else load_bits(wc, a.out_bits, grp, a.DI);
        ec = load_epi<M, false, RC>(a, grp);
      }
      const uint32_t hv = lora_issue(hC_mine, M);
      if constexpr (RC < 64) gemv_partials_rg<M, RC>(L, wcr, a.DI);
      else gemv_partials<M>(L, wc, a.DI);
      TL(10);
      lora_finish<M>(L, hC_mine, hv, tag, a.err);
      lds_barrier();
      TL(11);
      (void)epilogue<M, false, RC>(L, a, ec, grp, tag, x_pub, MULTI ? &xkeep : nullptr);
      TL(12);
      lds_barrier();
    }
  } else if (wg < gC + DFSSM_LORA_R) {
    lds_barrier();
    lora_rank<M, true, true>(L, nullptr, a.gT, a.DI, a.norm_w, a.out_lBq, wg - gC, hC, tag_now(), a.err, tag_now());
    TL(12);
  }
  lds_barrier();  // LDS reuse by the next layer; every wave has read the launch count
  TL(13);
#ifdef DFSSM_TIMELINE
  lds_barrier();
  TL_FLUSH(epoch_raw * (uint32_t)a0.n_layer + (uint32_t)l);
#endif
  }
  if (tix() == 0) st_dev(a0.launches + bix(), epoch_raw + 1u);
}

// ---------------------------------------------------------------------------------------------
// XCD-partitioned one-launch layer (batch <= 4). Grid: 8 XCDs x 32 workgroups, one per CU;
// workgroup w runs on XCD x (its XCC_ID register; w % 8 up to a rotation that varies by dispatch)
// with local index i = w / 8. XCD x owns the SSM heads x H/8 .. (x + 1) H/8 - 1 and every word its
// items need is produced on x itself and exchanged through x's L2 (XCD-scope stores and
// non-temporal loads, ~2x faster than device scope); only g crosses XCDs (device scope).
//   A  i < 2 gz: the z and x row groups of x's heads (gz = H/8 P / 64 groups each); then the
//      gbc = 4 B | C groups and the dt groups holding x's heads (computed on every XCD), then
//      4..16 LoRA-rank workgroups (16 / their number ranks each). The B | C conv state is updated
//      by XCD 0 only, in phase C, once all of g is in: every item's g needs its XCD's B | C rows,
//      so by then every XCD's B | C workgroups have read the old state.
//   B  local item j (sequence, head, 16-row block of x's heads) on workgroup j % 32.
//   C  i < gc = D / 256: out_proj rows 32 (x gc + i) .. + 31 (g polled device-scope); the last 4
//      workgroups of the XCD: the out_proj LoRA intermediates, 4 ranks each.
constexpr int kXRankC = 4;  // out_proj LoRA-rank workgroups per XCD (4 ranks each)

__device__ __forceinline__ int xcc_id() {
  return (int)(__builtin_amdgcn_s_getreg(20 | ((4 - 1) << 11)) & 0xfu);  // HW_REG_XCC_ID bits 3:0
}

// Local SSM item j of XCD x: (sequence, head, 16-row block) over x's heads.
__device__ __forceinline__ Item xcd_item(const FusedArgs& a, int xcd, int j) {
  const int hx = a.H / kXcd, PB = a.P / 16, per = hx * PB;
  const int m = j / per, rem = j - m * per;
  return Item{m, xcd * hx + rem / PB, rem % PB};
}

// LoRA intermediates of ranks r0 .. r0 + nr - 1 (nr <= 4) for every row, as lora_rank, stored once
// (to this XCD's words) with XCD scope.
template <int M, bool OUT, bool IL>
__device__ void lora_ranks(FusedLds<M>& L, const uint16_t* x, const uint32_t* gT, int K, const float* norm_w,
                           const uint16_t* lBq, int r0, int nr, uint32_t* hout, uint32_t tag, int* err,
                           uint32_t ptag) {
  const int tid = tix(), lane = tid & 63, wave = tid >> 6;
  const bool has_v = tid < K / 8;
  PIn<M> pi;
  load_pin<M, OUT, IL>(pi, x, K, norm_w);
  u32x4 b8[4];  // ranks past nr re-read rank r0 (unused)
#pragma unroll
  for (int q = 0; q < 4; ++q) b8[q] = load_pairs<IL>(lBq + (size_t)(r0 + (q < nr ? q : 0)) * K, pair_map<IL>(K));
  norm_rows<M, OUT, IL>(L, pi, gT, K, ptag, err, [&](int m, float) {
    double hacc[4] = {0.0, 0.0, 0.0, 0.0};
    if (has_v) {
      const u32x4 xv8 = load_pairs<IL>(L.xn, pair_map<IL>(K));  // this thread's own columns
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xv = h2f((uint16_t)(xv8[e >> 1] >> (16 * (e & 1))));
#pragma unroll
        for (int q = 0; q < 4; ++q) hacc[q] += (double)(xv * h2f((uint16_t)(b8[q][e >> 1] >> (16 * (e & 1)))));
      }
    }
    double hw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) hw[q] = q < nr ? wave_sum_dpp_f64(hacc[q]) : 0.0;
    lds_barrier();  // the sum-of-squares partials of this row have been read by every wave
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) L.rq[m][q][wave] = hw[q];
    }
    lds_barrier();
    if (tid < nr) {
      double t = 0.0;
#pragma unroll
      for (int w = 0; w < kFW; ++w) t += L.rq[m][tid][w];
      st_xcd(hout + m * DFSSM_LORA_R + r0 + tid, tagged(tag, f2h((float)t)));
    }
  });
}

template <int M>
__global__ __launch_bounds__(kFT) void layer_xcd_kernel(FusedArgs a) {
  __shared__ FusedLds<M> L;
  TL_DECL;
  const uint32_t epoch_raw = ld_dev(a.launches + bix());
  auto tag_now = [&]() {  // derived where used (see layer_fused_kernel)
    uint32_t v = epoch_raw;
    asm volatile("" : "+v"(v));
    return (v * (uint32_t)a.n_layer + (uint32_t)a.layer + 1u) & 0xffffu;
  };
  // XCD from the hardware: workgroups go to the XCDs round robin, but the first one's XCD varies
  // from dispatch to dispatch (under graph replay workgroup 0 ran on XCD 7), so workgroup w runs on
  // XCD (w + c) % 8 for some c; (XCC_ID, w / 8) is then one (XCD, local index) pair per workgroup.
  // (Another placement would leave a role without a workgroup: its consumers' waits time out.)
  const int wg = bix(), xcd = xcc_id(), li = wg / kXcd;
#ifdef DFSSM_TIMELINE
  if (tix() < kTlStamps) tl_s[tix()] = 0ull;
  lds_barrier();
#endif
  TL(0);
  const int hx = a.H / kXcd, PB = a.P / 16;
  const int gz = hx * a.P / 64, gbc = 2 * a.N / 64;
  const int dt0 = xcd * hx / 64, gdt = ((xcd + 1) * hx - 1) / 64 - dt0 + 1;  // dt groups of x's heads
  const int nga = 2 * gz + gbc + gdt;
  const int nra = nga + 16 <= kXcdWg ? 16 : (nga + 8 <= kXcdWg ? 8 : 4), rpa = DFSSM_LORA_R / nra;
  const int gc = a.D / (kXcd * 32);
  int grpA = -1;
  if (li < gz) grpA = xcd * gz + li;
  else if (li < 2 * gz) grpA = a.DI / 64 + xcd * gz + (li - gz);
  else if (li < 2 * gz + gbc) grpA = 2 * a.DI / 64 + (li - 2 * gz);
  else if (li < nga) grpA = (2 * a.DI + 2 * a.N) / 64 + dt0 + (li - 2 * gz - gbc);
  const bool bcA = li >= 2 * gz && li < 2 * gz + gbc;
  uint32_t* hA = a.hT + xcd * kHStride;  // this XCD's LoRA words: in_proj (M, 16), then out_proj
  uint32_t* hC = hA + M * DFSSM_LORA_R;
  const int nloc = M * hx * PB;
  const int nk = li < nloc ? (nloc - 1 - li) / kXcdWg + 1 : 0;  // <= kItemsOf<M> (the plan checks it)

  // ---- loads that do not depend on the activations ----
  u32x4 wa[kFMaxCPW];
  EpiRow ea = {};
  PIn<M> pa;
  if (grpA >= 0) {  // x first: the prologue needs it before the weights
    load_pin<M, false, false>(pa, a.x, a.D, a.ln_w);
    load_bits(wa, a.in_bits, grpA, a.D);
    ea = load_epi<M, true>(a, grpA);
  }
  const f32x2 h0 = __builtin_nontemporal_load((const f32x2*)state_row(a, xcd_item(a, xcd, li < nloc ? li : 0)));

  // ---- phase A: in_proj row groups, LoRA ranks ----
  ConvPend cpA{nullptr, 0, 0, 0};  // XCD 0: this thread's B | C conv-state update, stored in phase C
  if (grpA >= 0) {
    prologue<M, false, false>(L, pa, nullptr, a.D, 0u, a.err);
    TL(1);
    const uint32_t hv = lora_issue<true>(hA, M);
    gemv_partials<M>(L, wa, a.D);
    TL(2);
    const uint32_t tag = tag_now();
    lora_finish<M, true>(L, hA, hv, tag, a.err);
    lds_barrier();
    TL(3);
    const ConvPend cp = epilogue<M, true, 64, true>(L, a, ea, grpA, tag, nullptr, nullptr, xcd);
    if (!bcA) store_conv(cp);
    else if (xcd == 0) cpA = cp;
    TL(4);
    lds_barrier();
  } else if (li < nga + nra) {
    lora_ranks<M, false, false>(L, a.x, nullptr, a.D, a.ln_w, a.in_lBq, (li - nga) * rpa, rpa, hA, tag_now(), a.err,
                                0u);
    TL(4);
  }
  // ---- phase B: SSM + gate of this XCD's items ----
  const int grpC = li < gc ? xcd * gc + li : -1;
  u32x2 wcr[kCR<32>];
  EpiRow ec = {};
  if (grpC >= 0) {  // phase-C weights, loaded while phase B runs
    load_bits_rg<32>(wcr, a.out_bits, grpC, a.DI);
    ec = load_epi<M, false, 32>(a, grpC);
  }
  if (nk > 0) {
    f32x2 hk[kItemsOf<M>];
    float dk[kItemsOf<M>];
    hk[0] = h0;
#pragma unroll
    for (int k = 0; k < kItemsOf<M>; ++k) {
      if (k < nk) {
        const Item t = xcd_item(a, xcd, li + k * kXcdWg);
        if (k > 0) hk[k] = __builtin_nontemporal_load((const f32x2*)state_row(a, t));
        dk[k] = a.Dp[t.head];
      }
    }
    const uint32_t tag = tag_now();
    TL(5);
    for (int k = 0; k < nk; ++k) poll_item<M, true>(L, a, k, xcd_item(a, xcd, li + k * kXcdWg), tag, xcd);
    lds_barrier();
    TL(6);
#pragma unroll
    for (int k = 0; k < kItemsOf<M>; ++k)
      if (k < nk) ssm_item<M>(L, a, k, xcd_item(a, xcd, li + k * kXcdWg), hk[k], dk[k], tag);
  }
  TL(7);
  // ---- phase C: out_proj + residual, LoRA ranks ----
  if (grpC >= 0) {
    lds_barrier();  // LDS reuse after phases A and B
    PIn<M> pc;
    load_pin<M, true, true>(pc, nullptr, a.DI, a.norm_w);
    const uint32_t tag = tag_now();
    TL(8);
    prologue<M, true, true, 1>(L, pc, a.gT, a.DI, tag, a.err);
    TL(9);
    if (xcd == 0 && li == 0 && tix() == 0) st_xcd(a.xflag, tagged(tag, 0));  // every g word is in
    const uint32_t hv = lora_issue<true>(hC, M);
    gemv_partials_rg<M, 32>(L, wcr, a.DI);
    TL(10);
    lora_finish<M, true>(L, hC, hv, tag, a.err);
    lds_barrier();
    TL(11);
    (void)epilogue<M, false, 32, true>(L, a, ec, grpC, tag);
    TL(12);
    lds_barrier();
  } else if (li >= kXcdWg - kXRankC) {
    lds_barrier();
    lora_ranks<M, true, true>(L, nullptr, a.gT, a.DI, a.norm_w, a.out_lBq, (li - (kXcdWg - kXRankC)) * 4, 4, hC,
                              tag_now(), a.err, tag_now());
    TL(12);
  } else if (cpA.p) {  // XCD 0's B | C workgroups (idle in phase C: the plan checks it)
    bool ok = true;
    (void)poll1<true>(a.xflag, tag_now(), ok, a.err);
    store_conv(cpA);
  }
  lds_barrier();
  TL(13);
#ifdef DFSSM_TIMELINE
  if (tix() == 0) tl_s[15] = 1000ull + xcc_id();  // profiling builds: the XCD this workgroup ran on
  lds_barrier();
  TL_FLUSH(epoch_raw * (uint32_t)a.n_layer + (uint32_t)a.layer);
#endif
  if (tix() == 0) st_dev(a.launches + bix(), epoch_raw + 1u);
}

// Grid of the XCD-partitioned layer, or 0: the device must have exactly 8 x 32 CUs with the
// instantiation resident once per CU; per XCD the phase-A row groups plus at least 4 LoRA-rank
// workgroups fit in 32, the out_proj groups (D / 256 of 32 rows) come before the B | C workgroups
// and those before the last 4 (the phase-C rank workgroups), so that the B | C workgroups are idle
// in phase C; a workgroup polls at most 2 M (and kMaxItems) items.
int xcd_plan(int cus, int per_cu, int M, int D, int DI, int H, int P, int N) {
  if (cus != kXcdGrid || per_cu < 1 || M < 1 || M > 4 || N != 128) return 0;
  if (D > kFMaxK || DI > kFMaxK || H % kXcd || P % 16 || D % (kXcd * 32)) return 0;
  const int hx = H / kXcd;
  if ((hx * P) % 64) return 0;
  const int gz = hx * P / 64, gbc = 2 * N / 64;
  int gdt = 1;
  for (int x = 0; x < kXcd; ++x) {
    const int g = ((x + 1) * hx - 1) / 64 - x * hx / 64 + 1;
    gdt = g > gdt ? g : gdt;
  }
  const int nga = 2 * gz + gbc + gdt, gc = D / (kXcd * 32);
  if (nga + 4 > kXcdWg || gc > 2 * gz || 2 * gz + gbc > kXcdWg - kXRankC) return 0;
  const int per_wg = (M * hx * (P / 16) + kXcdWg - 1) / kXcdWg;
  if (per_wg > (2 * M < kMaxItems ? 2 * M : kMaxItems)) return 0;
  return kXcdGrid;
}


// The one-launch layer waits between its workgroups, so all G of them must be resident at once:
// G = one workgroup per CU (at most kFusedMaxGrid), which holds only if the launched
// instantiation fits at least once per CU (per_cu >= 1, from the occupancy query of that exact
// kernel). The grid must also hold the phase-A and phase-C workgroups plus their 16 LoRA
// workgroups, and every workgroup that reads x in phase A must also own an SSM item: phase C
// overwrites x once it has seen every item's output, which then implies that all reads of x are
// done. A workgroup polls at most 2 M (and kMaxItems) items (two waves each). The state width
// (d_state 128 = two columns per lane) and P % 16 == 0 are checked with the model dims.
// Rows per out_proj group (RC): 32 when D / 32 groups and the 16 LoRA workgroups fit the grid,
// else 64 (16-row groups measured 1% slower per step at batch 1: 128 pollers of the gated words).
// Returns G, or 0 when the layer must run as five kernels.
int fused_plan(int cus, int per_cu32, int per_cu64, int M, int IPO, int D, int DI, int H, int P, int* rc_out) {
  const int G = cus < kFusedMaxGrid ? cus : kFusedMaxGrid;
  if (G < 1 || M < 1 || M > 4) return 0;
  const int rc = D / 32 + DFSSM_LORA_R <= G ? 32 : 64;
  const int per_cu = rc == 32 ? per_cu32 : per_cu64;
  if (per_cu < 1 || (long long)per_cu * cus < G) return 0;  // not all workgroups co-resident
  const int gA = (IPO + 63) / 64, gC = D / rc, items = M * H * (P / 16);
  if (gA > kFusedMaxGroups || D > kFMaxK || DI > kFMaxK || G < gA + DFSSM_LORA_R || G < gC + DFSSM_LORA_R ||
      items < gA + DFSSM_LORA_R || items > 2 * M * G || items > kMaxItems * G)
    return 0;
  if (rc_out) *rc_out = rc;
  return G;
}

template <int M, int RC, bool MULTI>
static int occupancy_of() {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void*>(&layer_fused_kernel<M, RC, MULTI>), kFT, 0) != hipSuccess)
    return 0;
  return per_cu;
}

template <int M>
static int xcd_occupancy() {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&layer_xcd_kernel<M>), kFT,
                                                   0) != hipSuccess)
    return 0;
  return per_cu;
}

// Device facts for the plan, queried once per device: CU count and, per batch M = 1..4, the
// occupancy of both row-group instantiations, single-layer [0] and multi-layer [1].
struct FusedDev {
  int cus = -1;
  int per_cu[5][2][2] = {};
  int xcd_per_cu[5] = {};  // layer_xcd_kernel<M>
};

static const FusedDev* fused_dev() {
  static FusedDev devs[16];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return nullptr;
  FusedDev& d = devs[dev];
  if (d.cus < 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
#define DFSSM_OCC(MM)                                                                     \
  d.per_cu[MM][0][0] = occupancy_of<MM, 32, false>(); d.per_cu[MM][1][0] = occupancy_of<MM, 64, false>(); \
  d.per_cu[MM][0][1] = occupancy_of<MM, 32, true>(); d.per_cu[MM][1][1] = occupancy_of<MM, 64, true>();
    DFSSM_OCC(1) DFSSM_OCC(2) DFSSM_OCC(3) DFSSM_OCC(4)
#undef DFSSM_OCC
    d.xcd_per_cu[1] = xcd_occupancy<1>(); d.xcd_per_cu[2] = xcd_occupancy<2>();
    d.xcd_per_cu[3] = xcd_occupancy<3>(); d.xcd_per_cu[4] = xcd_occupancy<4>();
    d.cus = cus;
  }
  return &d;
}

static int fused_grid(int M, int IPO, int D, int DI, int H, int P, int* rc, bool multi = false) {
  const FusedDev* d = fused_dev();
  if (!d || M < 1 || M > 4) return 0;
  return fused_plan(d->cus, d->per_cu[M][0][multi], d->per_cu[M][1][multi], M, IPO, D, DI, H, P, rc);
}

bool fused_layer_supported(int M, int IPO, int D, int DI, int H, int P, bool multi) {
  return fused_grid(M, IPO, D, DI, H, P, nullptr, multi) > 0;
}

static int xcd_grid(int M, int D, int DI, int H, int P, int N) {
  const FusedDev* d = fused_dev();
  if (!d || M < 1 || M > 4) return 0;
  return xcd_plan(d->cus, d->xcd_per_cu[M], M, D, DI, H, P, N);
}

bool xcd_layer_supported(int M, int D, int DI, int H, int P, int N) { return xcd_grid(M, D, DI, H, P, N) > 0; }

hipError_t launch_xcd_layer(const FusedArgs& a, int M, hipStream_t s) {
  const int G = xcd_grid(M, a.D, a.DI, a.H, a.P, a.N);
  if (G < 1 || a.xflag == nullptr) return hipErrorNotSupported;
  switch (M) {
    case 1: hipLaunchKernelGGL(layer_xcd_kernel<1>, dim3(G), dim3(kFT), 0, s, a); break;
    case 2: hipLaunchKernelGGL(layer_xcd_kernel<2>, dim3(G), dim3(kFT), 0, s, a); break;
    case 3: hipLaunchKernelGGL(layer_xcd_kernel<3>, dim3(G), dim3(kFT), 0, s, a); break;
    case 4: hipLaunchKernelGGL(layer_xcd_kernel<4>, dim3(G), dim3(kFT), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// out[r][k] = fp16(B[r][k] * Bs[r]), the load-time LoRA-B dequantization.
__global__ void dequant_lora_b_kernel(const int8_t* __restrict__ B, const uint16_t* __restrict__ Bs, int K,
                                      uint16_t* __restrict__ out) {
  const int i = bix() * blockDim.x + tix();
  if (i < DFSSM_LORA_R * K) out[i] = f2h((float)B[i] * h2f(Bs[i / K]));
}

hipError_t launch_dequant_lora_b(const int8_t* B, const uint16_t* Bs, int K, uint16_t* out, hipStream_t s) {
  const int n = DFSSM_LORA_R * K;
  hipLaunchKernelGGL(dequant_lora_b_kernel, dim3((n + 255) / 256), dim3(256), 0, s, B, Bs, K, out);
  return hipGetLastError();
}

hipError_t launch_fused_layer(const FusedArgs& a, int M, hipStream_t s) {
  int rc = 0;
  const int G = fused_grid(M, a.IPO, a.D, a.DI, a.H, a.P, &rc);
  if (G < 1) return hipErrorNotSupported;
  const FusedArgs* none = nullptr;
#define DFSSM_FUSED(MM)                                                                              \
  case MM:                                                                                           \
    if (rc == 32) hipLaunchKernelGGL((layer_fused_kernel<MM, 32, false>), dim3(G), dim3(kFT), 0, s, a, none); \
    else hipLaunchKernelGGL((layer_fused_kernel<MM, 64, false>), dim3(G), dim3(kFT), 0, s, a, none);        \
    break;
  switch (M) {
    DFSSM_FUSED(1)
    DFSSM_FUSED(2)
    DFSSM_FUSED(3)
    DFSSM_FUSED(4)
    default: return hipErrorInvalidValue;
  }
#undef DFSSM_FUSED
  return hipGetLastError();
}

hipError_t launch_fused_layers(const FusedArgs& a, const FusedStrides& st, FusedArgs* tab, int M, hipStream_t s) {
  int rc = 0;
  const int G = fused_grid(M, a.IPO, a.D, a.DI, a.H, a.P, &rc, true);
  if (G < 1 || a.xT == nullptr || tab == nullptr || a.layer < 0 || a.layer >= a.n_layer || a.n_layer > kMaxLayers)
    return hipErrorNotSupported;
  hipLaunchKernelGGL(layer_table_kernel, dim3(1), dim3(kMaxLayers), 0, s, a, st, tab);
#define DFSSM_FUSED(MM)                                                                              \
  case MM:                                                                                           \
    if (rc == 32) hipLaunchKernelGGL((layer_fused_kernel<MM, 32, true>), dim3(G), dim3(kFT), 0, s, a, tab); \
    else hipLaunchKernelGGL((layer_fused_kernel<MM, 64, true>), dim3(G), dim3(kFT), 0, s, a, tab);        \
    break;
  switch (M) {
    DFSSM_FUSED(1)
    DFSSM_FUSED(2)
    DFSSM_FUSED(3)
    DFSSM_FUSED(4)
    default: return hipErrorInvalidValue;
  }
#undef DFSSM_FUSED
  return hipGetLastError();
}

}  // namespace dfssm

#ifdef DFSSM_TIMELINE
// Copies the whole stamp array (kTlSlots x kTlWg x kTlStamps u64) to host memory.
extern "C" int dfssm_timeline_read(void* host, size_t bytes) {
  if (bytes < sizeof(dfssm::dfssm_timeline)) return -5;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(dfssm::dfssm_timeline), sizeof(dfssm::dfssm_timeline));
}
#endif
