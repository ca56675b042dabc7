// One decode layer for 1..4 sequences in a single launch (gfx950).
//
// At batch <= 4 a layer moves ~7.8 MB, and the five-kernel form spends most of its time in
// launch gaps and per-kernel ramp-up. Here one grid of G workgroups (1024 threads, one per CU,
// all co-resident) runs the layer in three phases:
//   A  in_proj: workgroup w < gA = ceil(IPO/64) owns output rows 64w..64w+63: RMSNorm and int8
//      quantizer of x (4 KiB, L2-resident) into LDS, the packed-bit GEMV on v_dot4, dequantization,
//      LoRA, and per row type: the gate z sigma(z) (z rows), conv + SiLU (x, B, C rows), softplus
//      dt and exp(dt A) (dt rows). Workgroups gA..gA+15 compute the 16 LoRA intermediates (one rank
//      each); the GEMV workgroups pick them up just before their epilogue.
//   B  SSM + gate: item (sequence, head, 16-row block); two waves per item poll the words the
//      item needs (gate, x, B, C, dt) into LDS, then every wave updates one fp32 state row and
//      writes its g.
//   C  out_proj: workgroup w < gC = D/RC (RC = 32 rows per group, 64 when D/32 + 16 groups do
//      not fit the grid) reads all of g, runs the gated RMSNorm prologue and the GEMV of its rows
//      and adds the residual into x; workgroups gC..gC+15 compute the out_proj LoRA
//      intermediates as in phase A.
// The weights and the state do not depend on the activations, so each workgroup issues those
// loads first.
//
// Prologues (RMSNorm + quantizer) run on the "data waves" only: thread t < K/8 holds columns
// 8t..8t+7 of every row, so K/512 waves carry the activations and the others just pass the
// workgroup barriers (a wave64 VALU instruction occupies a 16-lane SIMD for 4 cycles, so VALU work
// that every wave repeats costs 4x what it costs on one wave per SIMD). The int8 activations go to
// LDS as bytes in the order the GEMV's dot products read them (quantize_rows), and the GEMV multiplies
// them with the sign bits on v_dot4_i32_i8: for a 32-bit weight word w (columns 32j..32j+31,
// bit i = column 32j+i), w & (0x01010101 << s) has byte b = 2^s (bit set) or 0 for column
// 32j+8b+s, so dot4(q dword s, that mask) = 2^s * (sum of q over the set bits among those four
// columns); s = 7 gives the byte 0x80 = -128, i.e. -128 times the sum. Eight accumulators per
// sequence, rescaled once at the end (exact), give T = sum of q over the set bits, and the
// scaffold accumulator is 2T - sum(q).
//
// Workgroup barriers order LDS only (lds_barrier): waves of a workgroup never hand each other
// data through global memory, and a full barrier would first wait for every global store of the
// wave to be acknowledged.
//
// Data passed between workgroups of one launch travels as 32-bit words (tag << 16) | fp16 value,
// stored and loaded with device-scope (agent) coherent accesses, which do not hit stale lines of
// another XCD's L2. The tag is derived from the launch's epoch mod 2^16; workgroup w keeps its own
// launch count in the workspace (read at the start, written back at the end, by w alone), so every
// workgroup of a launch derives the same epoch without any shared counter. A consumer polls the
// data words it needs until they carry the current tag: one memory round trip, no flags, no
// clearing (every word is rewritten by every launch). A 32-bit store is single-copy atomic, so tag
// and value always arrive together. Every poll is bounded: on a timeout the thread sets
// ERR_WAIT_LAYER in the workspace error flag and goes on, so the grid always drains (the host
// reports the error).
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
// out_proj in RG-row groups (RG = 32): thread t owns row t % RG and half-chunks
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
constexpr int kTlSlots = 64, kTlWg = 256, kTlStamps = 24;
__device__ unsigned long long dfssm_timeline[kTlSlots][kTlWg][kTlStamps];
__shared__ unsigned long long tl_s[kTlStamps];
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
#define TL(k) do {} while (0)
#define TL_FLUSH(slot) do {} while (0)
#endif

// Words of one SSM item, polled by two waves and shared through LDS.
struct ItemLds {
  uint32_t bc[DFSSM_WAVE * 2];  // B (pairs 0..63) and C (pairs 64..127), fp16 pairs
  uint16_t x[16], gate[16];     // x and z sigma(z) of the item's 16 rows
  float dt, abar;               // softplus dt and exp(dt A) of the item's head
};

template <int M>
struct FusedLds {
  // int8 activations of each row, 4 per dword: for the 32 columns 32j..32j+31, dword
  // 8j + 2 (s % 4) + s / 4 holds the columns 32j + s + 8b in its bytes b = 0..3 (s = 0..7)
  uint32_t q[M][kFMaxK / 4];
  int T[M][64][kFW + 1];  // per-wave GEMV partials of each row (padded against bank conflicts)
  double rd[M][kFW];   // per-wave partial sums of squares (0 for waves without activations)
  double rh[M][kFW];   // per-wave partial LoRA sums (likewise)
  float rf[M][kFW];    // per-wave partial amax (likewise)
  int ri[M][kFW];      // per-wave partial sum q (0 for waves without activations)
  float hl[M][DFSSM_LORA_R];
  float xs[M];
  ItemLds item[kMaxItems];
};

// Epilogue inputs of one output row, loaded ahead of the GEMV. Thread t works on row t / 16 of
// the group with wave partial / LoRA rank s = t % 16; threads s < M also finalize sequence s.
// Every field is a raw load (each in its own register), made unconditionally from clamped
// indices and used only in the epilogue: loads complete in issue order, so converting or
// packing a loaded value here (or a load inside a branch, whose join waits for all loads) would
// make the workgroup wait for the weight stream before its prologue starts. The epilogue makes
// the fields opaque before it converts them, so that the compiler cannot move the conversions
// up to the loads.
struct EpiRow {
  u32x2 cw;  // conv weights 0 | 1 << 16, 2 | 3 << 16: one 64-bit load, kept as one register pair
  float bias, alog;          // dt rows: dt_bias and A_log of the head (A = -exp(A_log) later)
  int la;                    // LoRA A[n][s]
  uint32_t ws, as, cs01, cs2, cb, xres;  // cs01: conv state words 0 | 1 << 16, one (unaligned) load
};

// Conv-state update of one row, stored after the row group's outputs.
struct ConvPend {
  uint16_t* p;
  uint16_t v0, v1, v2;
};

// Position of column c of the gated output g among its tagged words (K = d_inner): the thread
// that holds column c in the phase-C prologue (t = c / 8, columns 8t..8t+7) polls its 8 words as
// 4 adjacent pairs, pair p at 64-bit index p K / 8 + t, so that each wave-wide poll of one pair
// is one contiguous 512 bytes. The words are written in kGRep copies kGStride words apart (phase-C
// workgroup w polls copy w % kGRep): 64 workgroups polling one 16 KiB block queue on the few
// memory channels it maps to (one copy: 736 us per decode step at batch 1, eight: 722 us).
__device__ __forceinline__ int gpos(int c, int K) {
  const int t = c >> 3, i = c & 7;
  return 2 * ((i >> 1) * (K >> 3) + t) + (i & 1);
}

// Activations (phase A: x, 8 fp16 values of columns 8t..8t+7 per row) and their norm weights.
template <int M>
struct PIn {
  u32x4 av[M];
  f32x4 w0, w1;  // weights of columns 8t..8t+3 and 8t+4..8t+7
};

template <int M, bool OUT>
__device__ __forceinline__ void load_pin(PIn<M>& pi, const uint16_t* act, int K, const float* norm_w) {
  // unconditional loads from a clamped column: a load inside a branch makes the compiler wait for
  // all loads at the join
  const int t = tix() < K / 8 ? tix() : 0;
#pragma unroll
  for (int m = 0; m < M; ++m)
    pi.av[m] = OUT ? u32x4{0u, 0u, 0u, 0u} : *(const u32x4*)(act + (size_t)m * K + 8 * t);
  pi.w0 = *(const f32x4*)(norm_w + 8 * t);
  pi.w1 = *(const f32x4*)(norm_w + 8 * t + 4);
}

__device__ __forceinline__ void load_bits(u32x4 (&wb)[kFMaxCPW], const uint32_t* bits, int grp, int K) {
  const int lane = tix() & 63, wave = tix() >> 6, CH = K / 128;
  const u32x4* b = (const u32x4*)bits + (size_t)grp * CH * 64 + lane;
  // chunks past the row's end are left unset (the GEMV skips them): with a zero default the
  // compiler may copy a loaded value at the branch join, waiting there for every load
#pragma unroll
  for (int j = 0; j < kFMaxCPW; ++j) {
    const int c = wave + kFW * j;
    if (c < CH) wb[j] = ld_nt(b + (size_t)c * 64);
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
    // unconditional, from a clamped half-chunk (the GEMV skips cu >= 2 CH): no branch join
    const int cu = (64 / RG) * wave + lane / RG + (kFT / RG) * j, cc = cu < 2 * CH ? cu : 2 * CH - 1;
    wb[j] = __builtin_nontemporal_load((const u32x2*)(b + (size_t)(cc >> 1) * 64) + (cc & 1));
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
    e.cw = *(const u32x2*)wc;
    e.cb = a.conv_b[ch];
    e.bias = a.dt_bias[dtr];
    e.alog = a.A_log[dtr];
    e.xres = 0u;
  } else {
    e.xres = a.x[(size_t)m * a.D + n];
    e.cs01 = e.cs2 = e.cb = 0u;
    e.cw = u32x2{0u, 0u};
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
  atomicOr(err, DFSSM_ERR_WAIT_LAYER);
}
__device__ __forceinline__ uint32_t poll1(const uint32_t* p, uint32_t tag, bool& ok, int* err) {
  uint32_t v = ld_dev(p);
  for (uint32_t it = 0; ok && (v >> 16) != tag; ++it) {
    if (it == kSpinMax) {
      poll_timeout(ok, err);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    v = ld_dev(p);
  }
  return v & 0xffffu;
}
__device__ __forceinline__ bool tag_ok2(uint64_t v, uint32_t tag) {
  return ((uint32_t)v >> 16) == tag && ((uint32_t)(v >> 32) >> 16) == tag;
}
__device__ __forceinline__ uint32_t pack2(uint64_t v) { return ((uint32_t)v & 0xffffu) | ((uint32_t)(v >> 32) << 16); }

// N pairs of adjacent tagged words at p + 2 S j (8-byte aligned), all loads in flight together;
// out[j] = the pair's two fp16 values packed low | high.
template <int N>
__device__ __forceinline__ void pollv(const uint32_t* p, int S, uint32_t tag, uint32_t (&out)[N], bool& ok, int* err) {
  uint64_t v[N];
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = ld_dev((const uint64_t*)p + (size_t)S * j);
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
      if (!tag_ok2(v[j], tag)) v[j] = ld_dev((const uint64_t*)p + (size_t)S * j);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) out[j] = pack2(v[j]);
}

// RMSNorm of the M activation rows (K columns) on the data waves (wave < K / 512): xn[m] = the
// fp16 normalized values of this thread's columns 8t..8t+7 (pairs packed low | high) and mx[m]
// their largest magnitude. IN: x loaded ahead (pi.av); OUT: the gated g of this launch, polled
// from its tagged words (gT, in gpos order). One workgroup barrier.
template <int M, bool OUT>
__device__ __forceinline__ void norm_rows(FusedLds<M>& L, const PIn<M>& pi, const uint32_t* gT, int K, uint32_t tag,
                                          int* err, u32x4 (&xn)[M], float (&mx)[M]) {
  const int tid = tix(), lane = tid & 63, wave = tid >> 6, nd = K >> 9;
  const bool dw = wave < nd;
  u32x4 av[M];
  if (dw) {
    bool ok = true;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (OUT) {
        uint32_t w4[4];
        pollv<4>(gT + (size_t)m * K + 2 * tid, K >> 3, tag, w4, ok, err);
        av[m] = u32x4{w4[0], w4[1], w4[2], w4[3]};
      } else {
        av[m] = pi.av[m];
      }
    }
    TL(OUT ? 17 : 16);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      double part = 0.0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double xv = (double)h2f((uint16_t)(av[m][e >> 1] >> (16 * (e & 1))));
        part += xv * xv;
      }
      const double wsum = wave_sum_dpp_f64(part);
      if (lane == 0) L.rd[m][wave] = wsum;
    }
  } else if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) L.rd[m][wave] = 0.0;
  }
  lds_barrier();
  TL(OUT ? 19 : 18);
  if (dw) {
    const float wv[8] = {pi.w0[0], pi.w0[1], pi.w0[2], pi.w0[3], pi.w1[0], pi.w1[1], pi.w1[2], pi.w1[3]};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      double ss = 0.0;  // every wave's partial, all loads in flight together (0 from the other waves)
#pragma unroll
      for (int w = 0; w < kFW; ++w) ss += L.rd[m][w];
      const float var = (float)ss * (1.0f / (float)K);
      const float r = 1.0f / sqrt_rn(var + 1e-5f);
      float mxm = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = r16((h2f((uint16_t)(av[m][e >> 1])) * r) * wv[e]);
        const float x1 = r16((h2f((uint16_t)(av[m][e >> 1] >> 16)) * r) * wv[e + 1]);
        mxm = fmaxf(mxm, fmaxf(fabsf(x0), fabsf(x1)));
        xn[m][e >> 1] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
      }
      mx[m] = mxm;
    }
  }
}

// Within each quad of lanes (4i..4i+3, quad lane b = lane % 4): byte j of the result of lane b is
// byte b of lane j's a (a 4 x 4 byte transpose: two DPP quad permutations and two byte selects).
// v_perm_b32 (src0, src1, sel): byte k of the result is byte sel_k of the 8 bytes
// {src1 bytes 0..3, src0 bytes 0..3}.
__device__ __forceinline__ uint32_t quad_transpose_bytes(uint32_t a, int b) {
  const uint32_t p = (uint32_t)dpp_i32<0x4E>((int)a);  // lane b ^ 2
  const uint32_t u = __builtin_amdgcn_perm(p, a, (b & 2) ? 0x03020706u : 0x05040100u);
  const uint32_t q = (uint32_t)dpp_i32<0xB1>((int)u);  // lane b ^ 1
  return __builtin_amdgcn_perm(q, u, (b & 1) ? 0x03070105u : 0x06020400u);
}

// The int8 quantizer of the M rows (after norm_rows) on the data waves: the scale from the row's
// amax, q into L.q in the GEMV's order, sum q into L.ri (0 from the other waves), the scale into
// L.xs. One workgroup barrier; the caller passes another before the GEMV reads L.q.
// Thread t = 4j + b holds q of columns 32j + 8b + s (s = 0..7) as the bytes b of the dwords s of
// block j; after the quad transpose it holds the dwords s = b and s = b + 4 and stores them as one
// 64-bit word at dword 8j + 2b (each wave-wide store 512 contiguous bytes).
template <int M, int TLI>  // TLI: timeline stamp after the barrier (profiling builds)
__device__ __forceinline__ void quantize_rows(FusedLds<M>& L, const u32x4 (&xn)[M], const float (&mx)[M], int K) {
  const int tid = tix(), lane = tid & 63, wave = tid >> 6, nd = K >> 9;
  const bool dw = wave < nd;
  if (dw) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float wmax = wave_max_dpp_f32(mx[m]);
      if (lane == 0) L.rf[m][wave] = wmax;
    }
  } else if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) L.rf[m][wave] = 0.0f;
  }
  lds_barrier();
  TL(TLI);
  if (dw) {
    const int b = tid & 3;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float amax = L.rf[m][0];
#pragma unroll
      for (int w = 1; w < kFW; ++w) amax = fmaxf(amax, L.rf[m][w]);
      const float xs = quant_scale(amax);
      const float rinv = quant_rcp(xs);
      if (tid == 0) L.xs[m] = xs;
      int qsum = 0;
      uint32_t wd[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t d = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int s = 4 * h + e;
          const int q = quant_i8(h2f((uint16_t)(xn[m][s >> 1] >> (16 * (s & 1)))), rinv);
          qsum += q;
          d |= ((uint32_t)q & 0xffu) << (8 * e);
        }
        wd[h] = quad_transpose_bytes(d, b);
      }
      *(u32x2*)&L.q[m][8 * (tid >> 2) + 2 * b] = u32x2{wd[0], wd[1]};
      const int wq = wave_sum_dpp_i32(qsum);
      if (lane == 0) L.ri[m][wave] = wq;
    }
  } else if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) L.ri[m][wave] = 0;
  }
}

// sum of q over the set bits of one 32-bit weight word (block jb) into the 8 accumulators of each
// sequence (acc[m][s] collects 2^s times the sum of the columns 32 jb + 8b + s; s = 7: -128 times)
template <int M>
__device__ __forceinline__ void dot_word(const FusedLds<M>& L, uint32_t w, int jb, int (&acc)[M][8]) {
  uint32_t mk[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) mk[s] = w & (0x01010101u << s);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const u32x4 qa = *(const u32x4*)&L.q[m][8 * jb];      // dwords s = 0, 4, 1, 5
    const u32x4 qb = *(const u32x4*)&L.q[m][8 * jb + 4];  // dwords s = 2, 6, 3, 7
    acc[m][0] = __builtin_amdgcn_sdot4((int)qa[0], (int)mk[0], acc[m][0], false);
    acc[m][4] = __builtin_amdgcn_sdot4((int)qa[1], (int)mk[4], acc[m][4], false);
    acc[m][1] = __builtin_amdgcn_sdot4((int)qa[2], (int)mk[1], acc[m][1], false);
    acc[m][5] = __builtin_amdgcn_sdot4((int)qa[3], (int)mk[5], acc[m][5], false);
    acc[m][2] = __builtin_amdgcn_sdot4((int)qb[0], (int)mk[2], acc[m][2], false);
    acc[m][6] = __builtin_amdgcn_sdot4((int)qb[1], (int)mk[6], acc[m][6], false);
    acc[m][3] = __builtin_amdgcn_sdot4((int)qb[2], (int)mk[3], acc[m][3], false);
    acc[m][7] = __builtin_amdgcn_sdot4((int)qb[3], (int)mk[7], acc[m][7], false);
  }
}
// T = sum of q over the set bits, from the 8 scaled accumulators (every shift is exact)
__device__ __forceinline__ int dot_total(const int (&acc)[8]) {
  int t = 0;
#pragma unroll
  for (int s = 0; s < 7; ++s) t += acc[s] >> s;
  return t - (acc[7] >> 7);
}

// Packed-bit GEMV of one 64-row group: per-wave partials T into L.T (no barrier). Lane l = row,
// wave w the chunks (128 columns) w, w + 16, ...
template <int M>
__device__ __forceinline__ void gemv_partials(FusedLds<M>& L, const u32x4 (&wb)[kFMaxCPW], int K) {
  const int lane = tix() & 63, wave = tix() >> 6;
  const int CH = K / 128;
  int acc[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[m][s] = 0;
#pragma unroll
  for (int j = 0; j < kFMaxCPW; ++j) {
    const int c = wave + kFW * j;
    if (c < CH) {
#pragma unroll
      for (int h = 0; h < 4; ++h) dot_word<M>(L, wb[j][h], 4 * c + h, acc);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) L.T[m][lane][wave] = dot_total(acc[m]);
}

// Packed-bit GEMV of one RG-row group (RG = 32): each thread two words of one row per half-chunk,
// the two threads of a wave that share a row summed by a lane swap; per-wave partials into L.T rows
// 0..RG-1.
template <int M, int RG>
__device__ __forceinline__ void gemv_partials_rg(FusedLds<M>& L, const u32x2 (&wb)[kCR<RG>], int K) {
  static_assert(RG == 32, "half-wave row groups only");
  const int lane = tix() & 63, wave = tix() >> 6;
  const int CH = K / 128;
  int acc[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[m][s] = 0;
#pragma unroll
  for (int j = 0; j < kCR<RG>; ++j) {
    const int cu = (64 / RG) * wave + lane / RG + (kFT / RG) * j;
    if (cu < 2 * CH) {
      // the words 0, 1 of half-chunk cu are the blocks 2 cu, 2 cu + 1
      dot_word<M>(L, wb[j][0], 2 * cu, acc);
      dot_word<M>(L, wb[j][1], 2 * cu + 1, acc);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    int t = dot_total(acc[m]);
    t += (int)__builtin_amdgcn_permlane32_swap((uint32_t)t, (uint32_t)t, false, false)[1];  // lane + 32
    if (lane < RG) L.T[m][lane][wave] = t;
  }
}

// LoRA intermediate of rank r for every row (LoRA workgroups): h[m][r] =
// fp16(sum_k xn_k * Bq[r][k]), fp16 x fp16 products exact in fp32, summed in fp64, stored as a
// tagged word in kXRep copies of hout[m * 16 + r] with `tag`. OUT: the activations are polled from
// gT until they carry `ptag`.
template <int M, bool OUT>
__device__ __forceinline__ void lora_rank(FusedLds<M>& L, const uint16_t* x, const uint32_t* gT, int K, const float* norm_w,
                          const uint16_t* lBq, int r, uint32_t* hout, uint32_t tag, int* err, uint32_t ptag) {
  const int tid = tix(), lane = tid & 63, wave = tid >> 6, nd = K >> 9;
  PIn<M> pi;
  load_pin<M, OUT>(pi, x, K, norm_w);
  const u32x4 b8 = *(const u32x4*)(lBq + (size_t)r * K + 8 * (tid < K / 8 ? tid : 0));
  u32x4 xn[M];
  float mx[M];
  norm_rows<M, OUT>(L, pi, gT, K, ptag, err, xn, mx);
  if (wave < nd) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      double hacc = 0.0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xv = h2f((uint16_t)(xn[m][e >> 1] >> (16 * (e & 1))));
        const float bv = h2f((uint16_t)(b8[e >> 1] >> (16 * (e & 1))));
        hacc += (double)(xv * bv);
      }
      const double hw = wave_sum_dpp_f64(hacc);
      if (lane == 0) L.rh[m][wave] = hw;
    }
  } else if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) L.rh[m][wave] = 0.0;
  }
  lds_barrier();
  if (tid < kXRep) {  // one copy per thread
#pragma unroll
    for (int m = 0; m < M; ++m) {
      double t = 0.0;
#pragma unroll
      for (int w = 0; w < kFW; ++w) t += L.rh[m][w];
      st_dev(hout + tid * kHStride + m * DFSSM_LORA_R + r, tagged(tag, f2h((float)t)));
    }
  }
}

// LoRA intermediates of this phase (threads < 16 M): the first load is issued before the GEMV
// (lora_issue), the poll completes after it (lora_finish) into L.hl; the caller then passes a
// barrier. (A second load issued halfway through the GEMV measured no earlier: a device-scope store
// takes ~1 us to become visible, and the producers store the words shortly before the GEMV starts.)
__device__ __forceinline__ uint32_t lora_issue(const uint32_t* hsrc, int M) {
  return tix() < M * DFSSM_LORA_R ? ld_dev(hsrc + tix()) : 0u;
}
template <int M>
__device__ __forceinline__ void lora_finish(FusedLds<M>& L, const uint32_t* hsrc, uint32_t v, uint32_t tag, int* err) {
  const int tid = tix();
  if (tid < M * DFSSM_LORA_R) {
    bool ok = true;
    if ((v >> 16) != tag) v = poll1(hsrc + tid, tag, ok, err);
    L.hl[tid / DFSSM_LORA_R][tid % DFSSM_LORA_R] = h2f((uint16_t)v);
  }
}

// Epilogue of one 64-row group (after the barrier that publishes L.T and L.hl), 16 threads per
// row: acc = sum over waves s of (2 T_s - sum q_s) and the LoRA term sum_r h_r aq_r as DPP row
// sums (exact: integers, and exactly representable products in fp64); thread s = m then
// finalizes sequence m. IN: z rows store the gate z sigma(z), x/B/C rows conv + SiLU, dt rows
// softplus dt and exp(dt A) (as tagged fp32 words); OUT: the residual add into x.
template <int M, bool IN, int RG = 64>
__device__ ConvPend epilogue(FusedLds<M>& L, const FusedArgs& a, const EpiRow& er_in, int grp, uint32_t tag) {
  // the inputs, opaque from here on: the compiler otherwise hoists their conversions to right
  // after the loads at the kernel start and waits there for them
  EpiRow er = er_in;
  asm volatile("" : "+v"(er.cw), "+v"(er.bias), "+v"(er.alog), "+v"(er.la), "+v"(er.ws),
               "+v"(er.as), "+v"(er.cs01), "+v"(er.cs2), "+v"(er.cb), "+v"(er.xres));
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
      float o = h2f((uint16_t)er.cs01) * h2f((uint16_t)er.cw[0]);
      o = o + h2f((uint16_t)(er.cs01 >> 16)) * h2f((uint16_t)(er.cw[0] >> 16));
      o = o + h2f((uint16_t)er.cs2) * h2f((uint16_t)er.cw[1]);
      o = o + xv * h2f((uint16_t)(er.cw[1] >> 16));
      o = o + h2f((uint16_t)er.cb);
      const float sig = 1.0f / (1.0f + dev_expf(-o));
      out = o * sig;
    } else {  // dt row of head dtr
      const float dt = dev_log1pf(dev_expf(out + er.bias));
      const float abar = dev_expf(dt * -dev_expf(er.alog));
      uint64_t* w = a.dtT + ((size_t)m * a.H + dtr) * 2;
      st_dev(w, ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, dt));
      st_dev(w + 1, ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, abar));
      return cp;
    }
    const uint32_t word = tagged(tag, f2h(out));
    const int bc = ch - a.DI;  // B | C channel index, or < 0
    if (bc >= 0) {
#pragma unroll
      for (int c = 0; c < kXRep; ++c) st_dev(a.bcT + c * kBcStride + m * 2 * a.N + bc, word);
    } else {
      st_dev(a.projT + (size_t)m * a.IPO + n, word);
    }
  } else {
    a.x[(size_t)m * a.D + n] = f2h(h2f((uint16_t)er.xres) + out);
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
template <int M>
__device__ void poll_item(FusedLds<M>& L, const FusedArgs& a, int k, const Item& t, uint32_t tag) {
  const int lane = tix() & 63, wave = tix() >> 6;
  const uint32_t* pr = a.projT + (size_t)t.m * a.IPO;
  bool ok = true;
  if (wave == 2 * k) {
    uint32_t w[2];  // pairs lane (B) and 64 + lane (C): each wave-wide load one contiguous 512 bytes
    pollv<2>(a.bcT + (bix() % kXRep) * kBcStride + t.m * 2 * a.N + 2 * lane, 64, tag, w, ok, a.err);
    L.item[k].bc[lane] = w[0];
    L.item[k].bc[DFSSM_WAVE + lane] = w[1];
  } else if (wave == 2 * k + 1 && lane < 34) {
    // lanes 0..31 poll 32-bit words (tag in the high half), lanes 32 and 33 64-bit words (tag in
    // the high word), all in one loop so that neither set waits for the other's round trips
    const int r0 = t.head * a.P + 16 * t.pb;
    const bool w32 = lane < 32;
    // every lane loads both kinds (from valid addresses): no divergent loads inside the loop
    const uint32_t* p32 = (lane & 31) < 16 ? pr + a.DI + r0 + (lane & 15) : pr + r0 + (lane & 15);
    const uint64_t* p64 = a.dtT + ((size_t)t.m * a.H + t.head) * 2 + (lane & 1);
    auto ready = [&](uint32_t x, uint64_t y) { return w32 ? (x >> 16) == tag : (uint32_t)(y >> 32) == tag; };
    uint32_t va = ld_dev(p32);
    uint64_t vb = ld_dev(p64);
    for (uint32_t it = 0; ok && !ready(va, vb); ++it) {
      if (it == kSpinMax) {
        poll_timeout(ok, a.err);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      va = ld_dev(p32);
      vb = ld_dev(p64);
    }
    const uint64_t r = w32 ? (uint64_t)va : vb;
    if (lane < 16) L.item[k].x[lane] = (uint16_t)r;
    else if (lane < 32) L.item[k].gate[lane - 16] = (uint16_t)r;
    else if (lane == 32) L.item[k].dt = __builtin_bit_cast(float, (uint32_t)r);
    else L.item[k].abar = __builtin_bit_cast(float, (uint32_t)r);
  }
}

// SSM + gate of item k (after the barrier that publishes L.item[k]): wave w owns state row
// p = 16 pb + w, lane l the state columns 2l, 2l+1; g goes to its tagged word in gpos order.
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
  acc = wave_sum_dpp_f64(acc);  // the same value in every lane
  if (lane < kGRep) {            // lane c writes copy c (one store instruction for all copies)
    const float y = r16((float)acc + xv * Dh);
    const float gv = r16(y * h2f(I.gate[wave]));
    st_dev(a.gT + (size_t)lane * kGStride + (size_t)t.m * a.DI + gpos(t.head * a.P + p, a.DI), tagged(tag, f2h(gv)));
  }
}

// RC: rows per out_proj group (32, or 64 when D / 32 + 16 groups do not fit the grid).
template <int M, int RC>
__global__ __launch_bounds__(kFT) void layer_fused_kernel(FusedArgs a) {
  __shared__ FusedLds<M> L;
  // The launch's epoch is the first load; its tags are derived where they are used (tag_now):
  // the empty asm keeps the compiler from computing them right after a branch join near the
  // kernel start, where it can only wait for every load issued so far (the weight stream
  // included). Tag of layer l at epoch e: e L + l + 1 (mod 2^16); every launch of a workgroup
  // index advances its epoch, so a word left by the previous launch never carries the tag a poll
  // waits for.
  // every argument into registers at once: the compiler otherwise loads the launch-count pointer
  // first and waits for it before loading the rest of the argument block (one more scalar-memory
  // round trip before the first data load)
  asm volatile("" ::"s"(a.in_bits), "s"(a.in_ws), "s"(a.in_lA), "s"(a.in_lAs), "s"(a.in_lBq), "s"(a.out_bits),
               "s"(a.out_ws), "s"(a.out_lA), "s"(a.out_lAs), "s"(a.out_lBq), "s"(a.conv_w), "s"(a.conv_b));
  asm volatile("" ::"s"(a.A_log), "s"(a.Dp), "s"(a.dt_bias), "s"(a.norm_w), "s"(a.ln_w), "s"(a.h), "s"(a.conv),
               "s"(a.x), "s"(a.projT), "s"(a.gT), "s"(a.hT), "s"(a.bcT), "s"(a.dtT), "s"(a.launches), "s"(a.err));
  asm volatile("" ::"s"(a.layer), "s"(a.n_layer), "s"(a.D), "s"(a.DI), "s"(a.N), "s"(a.H), "s"(a.P), "s"(a.IPO),
               "s"(a.C));
  const uint32_t epoch_raw = ld_dev(a.launches + bix());
  const int G = gridDim.x, wg = bix();
  auto tag_now = [&]() {
    uint32_t v = epoch_raw;
    asm volatile("" : "+v"(v));
    return (v * (uint32_t)a.n_layer + (uint32_t)a.layer + 1u) & 0xffffu;
  };
#ifdef DFSSM_TIMELINE
  if (tix() < kTlStamps) tl_s[tix()] = 0ull;
  lds_barrier();
#endif
  TL(0);
  const int gA = (a.IPO + 63) / 64, gC = a.D / RC;
  const int NI = a.H * (a.P / 16), items = M * NI;
  uint32_t* hA = a.hT;                       // copy 0 (the LoRA workgroups write every copy)
  uint32_t* hC = a.hT + M * DFSSM_LORA_R;
  const uint32_t* hA_mine = hA + (wg % kXRep) * kHStride;  // the copy this workgroup polls
  const uint32_t* hC_mine = hC + (wg % kXRep) * kHStride;

  // ---- loads that do not depend on the activations ----
  // Set and used on the phase-A path only: no default value, which the compiler would merge with
  // the loaded values at the branch join (folding the epilogue's conversions into the join, right
  // after the loads, and waiting there for them).
  u32x4 wa[kFMaxCPW];
  EpiRow ea;
  PIn<M> pa;
  if (wg < gA) {  // x first: the prologue needs it before the weights
    load_pin<M, false>(pa, a.x, a.D, a.ln_w);
    load_bits(wa, a.in_bits, wg, a.D);
    ea = load_epi<M, true>(a, wg);
  }
  // state row of this workgroup's first SSM item (the other items' rows load before phase B's polls)
  // (unconditional, from a clamped item: see load_pin). Issuing these and the weights only once x
  // is in measured slower (the prologue waits as long for x, and then for the weights).
  const f32x2 h0 = __builtin_nontemporal_load((const f32x2*)state_row(a, item_of(a, wg < items ? wg : items - 1)));

  // ---- phase A: in_proj (workgroups < gA), LoRA ranks (gA .. gA + 15) ----
  // The launch's tag, derived once on every path (after its first polls' loads on the GEMV path):
  // a tag derived after the paths join made the compiler wait for the epoch load there, on the
  // path that had already waited for it too, i.e. for phase A's device-scope stores.
  uint32_t tag;
  if (wg < gA) {
    {
      u32x4 xn[M];
      float mx[M];
      norm_rows<M, false>(L, pa, nullptr, a.D, 0u, a.err, xn, mx);  // x loaded ahead, no polls
      TL(14);
      quantize_rows<M, 20>(L, xn, mx, a.D);
    }
    lds_barrier();  // q published
    TL(1);
    {  // one 64-row group per workgroup (the plan keeps gA + 16 <= G)
      const uint32_t hv = lora_issue(hA_mine, M);
      gemv_partials<M>(L, wa, a.D);
      TL(2);
      tag = tag_now();
      lora_finish<M>(L, hA_mine, hv, tag, a.err);
      lds_barrier();
      TL(3);
      store_conv(epilogue<M, true>(L, a, ea, wg, tag));
      TL(4);
      lds_barrier();
    }
  } else if (wg < gA + DFSSM_LORA_R) {
    tag = tag_now();
    lora_rank<M, false>(L, a.x, nullptr, a.D, a.ln_w, a.in_lBq, wg - gA, hA, tag, a.err, 0u);
    TL(4);
  } else {
    tag = tag_now();
  }
  // ---- phase B: SSM + gate ----
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
    TL(5);
    int k = 0;
    do poll_item<M>(L, a, k, item_of(a, wg + k * G), tag);
    while (++k < nk);
    // Every wave waits here for its own loads and stores (the polling waves already have): the
    // compiler's accounting then holds nothing pending past phase B, and no later register reuse
    // waits on the state rows of items this workgroup does not own (loaded only when it does),
    // which would also wait for phase B's device-scope stores. The barrier below waits for the
    // polling waves, which see phase A's stores acknowledged first.
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
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
    // The weights, issued once this workgroup's SSM items are done: loads and stores complete in
    // issue order, so a load issued before a poll holds back the poll's result (issued at phase B's
    // start, their HBM round trip delayed the items' inputs). The gated output g arrives a poll
    // round trip after the last item, about as long as these loads take. The epilogue inputs
    // follow the polls of g: with them here, the compiler's wait before the polls (at most 10
    // memory operations in flight) also waited for the SSM's state stores.
    u32x4 wc[RC < 64 ? 1 : kFMaxCPW];
    u32x2 wcr[kCR<32>];
    if constexpr (RC < 64) load_bits_rg<RC>(wcr, a.out_bits, wg, a.DI);
    else load_bits(wc, a.out_bits, wg, a.DI);
    PIn<M> pc;
    EpiRow ec;
    load_pin<M, true>(pc, nullptr, a.DI, a.norm_w);
    TL(8);
    {
      u32x4 xn[M];
      float mx[M];
      norm_rows<M, true>(L, pc, a.gT + (size_t)(wg % kGRep) * kGStride, a.DI, tag, a.err, xn, mx);
      ec = load_epi<M, false, RC>(a, wg);
      TL(15);
      quantize_rows<M, 21>(L, xn, mx, a.DI);
    }
    lds_barrier();  // q published
    TL(9);
    {  // one RC-row group per workgroup (the plan keeps gC + 16 <= G)
      const uint32_t hv = lora_issue(hC_mine, M);
      if constexpr (RC < 64) gemv_partials_rg<M, RC>(L, wcr, a.DI);
      else gemv_partials<M>(L, wc, a.DI);
      TL(10);
      lora_finish<M>(L, hC_mine, hv, tag, a.err);
      lds_barrier();
      TL(11);
      (void)epilogue<M, false, RC>(L, a, ec, wg, tag);
      TL(12);
      lds_barrier();
    }
  } else if (wg < gC + DFSSM_LORA_R) {
    lds_barrier();
    lora_rank<M, true>(L, nullptr, a.gT + (size_t)(wg % kGRep) * kGStride, a.DI, a.norm_w, a.out_lBq, wg - gC, hC,
                       tag, a.err, tag);
    TL(12);
  }
  lds_barrier();  // every wave has read the launch count
  TL(13);
#ifdef DFSSM_TIMELINE
  lds_barrier();
  TL_FLUSH(epoch_raw * (uint32_t)a.n_layer + (uint32_t)a.layer);
#endif
  // a plain store: the count is read only by the next launch, after the kernel boundary has made
  // it visible; a device-scope store here held the launch's end for its write-through to memory
  // (~0.85 us per layer at batch 1: 697 -> 657 us per decode step)
  if (tix() == 0) a.launches[bix()] = epoch_raw + 1u;
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

template <int M, int RC>
static int occupancy_of() {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void*>(&layer_fused_kernel<M, RC>), kFT, 0) != hipSuccess)
    return 0;
  return per_cu;
}

// Device facts for the plan, queried once per device: CU count and, per batch M = 1..4, the
// occupancy of both row-group instantiations.
struct FusedDev {
  int cus = -1;
  int per_cu[5][2] = {};
};

static const FusedDev* fused_dev() {
  static FusedDev devs[16];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return nullptr;
  FusedDev& d = devs[dev];
  if (d.cus < 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
#define DFSSM_OCC(MM) d.per_cu[MM][0] = occupancy_of<MM, 32>(); d.per_cu[MM][1] = occupancy_of<MM, 64>();
    DFSSM_OCC(1) DFSSM_OCC(2) DFSSM_OCC(3) DFSSM_OCC(4)
#undef DFSSM_OCC
    d.cus = cus;
  }
  return &d;
}

static int fused_grid(int M, int IPO, int D, int DI, int H, int P, int* rc) {
  const FusedDev* d = fused_dev();
  if (!d || M < 1 || M > 4) return 0;
  return fused_plan(d->cus, d->per_cu[M][0], d->per_cu[M][1], M, IPO, D, DI, H, P, rc);
}

bool fused_layer_supported(int M, int IPO, int D, int DI, int H, int P) {
  return fused_grid(M, IPO, D, DI, H, P, nullptr) > 0;
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
#define DFSSM_FUSED(MM)                                                                   \
  case MM:                                                                                \
    if (rc == 32) hipLaunchKernelGGL((layer_fused_kernel<MM, 32>), dim3(G), dim3(kFT), 0, s, a); \
    else hipLaunchKernelGGL((layer_fused_kernel<MM, 64>), dim3(G), dim3(kFT), 0, s, a);        \
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
