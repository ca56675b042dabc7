// Batched scaffold projection (M = 5..64 activation rows) on the int8 matrix cores (gfx950).
//
// acc[m][n] = sum_k q[m][k] * (2 bit[n][k] - 1) (exact int32) is computed with
// v_mfma_i32_16x16x64_i8: A = q (16 rows x 64 k, int8), B = the sign bits of 16 output rows
// expanded in registers to +-1 bytes, so that the MFMA sums are acc itself. Expansion of a nibble
// to four 0/1 bytes is one multiply and one mask: (nib * 0x00204081) & 0x01010101 -- the four
// shifted copies of the nibble occupy disjoint bit ranges, so the product has no carries -- and
// v_perm_b32 then looks each byte up in a word holding 0xff at byte 0 and 0x01 at byte 1 (a zero
// word for the chunks past K, whose bytes then contribute nothing): four full-rate instructions
// per four bytes, no branches. (Earlier forms: ~(x * 0xfe) for the +-1 bytes, a quarter-rate
// 32-bit multiply, with the compiler branching around every nibble for the chunks past K; or 0/1
// bytes with acc = 2 T - sum q and the row sums taken from the q tile in LDS, alone 0.7 us per
// launch. The lookup took the decode step from 2318 to 2260 us at batch 32 and from 6776 to
// 6507 us at the 2.7B shape and batch 64.)
//
// One workgroup (1024 threads = 16 waves) owns 16 RT output rows (RT = 1, 2 or 4 row tiles: the
// fewest that keep the grid within one workgroup per CU); it keeps their bits in registers and walks the activation
// rows in blocks of 32 (16 when K > 4096). Wave w = (row tile rt = w % RT, k slot kq = w / RT),
// KQ = 16 / RT k slots. The 16-byte bit chunks c of a row tile (128 columns each) are dealt out as
// c = kq + KQ j + 4 KQ sb to lane group j = lane / 16 of wave slot kq, block sb: every lane keeps
// its chunks in registers, loaded once, fully coalesced. Within an MFMA step lane group j
// supplies columns 128 c + 16 s .. +15 of both operands; a consistent permutation of the k index
// between A and B leaves the dot product unchanged. The q tile of all rows sits in LDS (one
// batch of loads); the k slots' int32 partials are added through LDS (exact), and the epilogue
// is shared by the waves (element i of a lane's 4 MI accumulators by wave slot i % KQ). The
// rank-16 LoRA term runs on the fp64 matrix cores (v_mfma_f64_16x16x4f64, exact products of fp32
// and fp16 values, exact sums) between the MFMA loop and the epilogue: measured 0.9% less time per
// decode step at batch 32 than the 16 fp64 FMAs per element it replaces.
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef double v4d __attribute__((ext_vector_type(4)));

constexpr int kGT = 1024;

// Dynamic LDS of gemm_kernel: a block's q tile, later reused for the int32 k-slot partials
// [KQ][RT][MI][4][64] followed by the fp64 LoRA partials [min(KQ / MI, 4)][RT][MI][4][64].
__host__ __device__ constexpr size_t gemm_part_bytes(int MI, int RT) { return (size_t)16 * MI * 4 * 64 * 4; }
__host__ __device__ constexpr size_t gemm_lora_bytes(int MI, int RT) {
  return (size_t)((16 / RT) / MI < 4 ? (16 / RT) / MI : 4) * RT * MI * 4 * 64 * 8;
}

// ---- the next layer's in_proj prologue in the out_proj launch (PRO; decode, batch >= 5) ----
// Four workgroups (16 waves) per sequence m, placed after every GEMM workgroup; workgroup k polls
// the row of the new x (D = N columns) from the tagged words the GEMM epilogues publish, computes
// RMSNorm (fp64 sum of squares), the maximum and the scale, writes the q bytes of columns
// k D / 4 .. (k + 1) D / 4 - 1, and computes the LoRA intermediates of ranks 4 k .. 4 k + 3: wave w
// sums rank 4 k + w / 4 over column quarter w % 4 (lane l: 8-column blocks 64 i + l of the quarter)
// from the normalized row in LDS -- prep_kernel<IN>'s outputs; every sum is a sum of exact
// products in fp64. (One workgroup per sequence, all 16 ranks, took 3.8 us more per layer: these
// workgroups inherit the GEMM's LDS, one per CU, so a row's 16 dot products ran on one CU.)
// Waiting: every GEMM workgroup comes before them in dispatch order and never waits, so every
// wait ends; every wait is also bounded (bit 2 of err on a timeout).
constexpr int kProPW = 4;   // prologue workgroups per sequence
constexpr int kProPJ = 3;   // column pairs per thread at most (N / 2 <= 2560 over 1024 threads)
constexpr int kProBI = 3;   // 8-column blocks per lane of a quarter at most (N / 32 <= 160 over 64 lanes)
constexpr int kProPF = 4;   // 16-byte prefetch vectors per thread of the next layer's prologue weights
__device__ __forceinline__ bool pro_tag_ok(uint64_t v, uint32_t tag) {
  return ((uint32_t)v >> 16) == tag && ((uint32_t)(v >> 32) >> 16) == tag;
}
__device__ __forceinline__ void gemm_in_prologue(const GemmPro& p, int D, int m, int k, uint32_t epoch, uint32_t* xn2) {
  __shared__ double pr_d[16];
  __shared__ float pr_f[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int np = D / 2, nbq = D / 32;  // column pairs; 8-column blocks per quarter
  const int rr = kProPW * k + (w >> 2), c0 = (w & 3) * (D / 4);
  // norm weights of this thread's pairs u = tid + 1024 j and the LoRA-B bytes of rank rr over the
  // wave's quarter first, then x. Unconditional (clamped pairs and blocks, unused past the end;
  // without LoRA the bytes come from the norm weights, scaled by zero) and raw until the polls are
  // done: a select or a conversion of a loaded value before the poll loop made the workgroup wait
  // for these loads before its first poll.
  float2 wv[kProPJ];
#pragma unroll
  for (int j = 0; j < kProPJ; ++j) {
    const int u = tid + 1024 * j;
    wv[j] = *(const float2*)(p.norm_w + 2 * (u < np ? u : np - 1));
  }
  const int8_t* lb = p.lB ? p.lB + (size_t)rr * D + c0 : (const int8_t*)p.norm_w;
  uint2 bq[kProBI];
#pragma unroll
  for (int i = 0; i < kProBI; ++i) {
    const int b = 64 * i + lane;
    bq[i] = *(const uint2*)(lb + 8 * (b < nbq ? b : nbq - 1));
  }
  const uint16_t bs_raw = *(p.lB ? p.lBs + rr : (const uint16_t*)p.norm_w);
  const uint64_t* xp = (const uint64_t*)(p.xT + (size_t)m * D) + tid;
  uint64_t xv[kProPJ];
#pragma nounroll
  for (uint32_t it = 0;; ++it) {
#pragma unroll
    for (int j = 0; j < kProPJ; ++j) xv[j] = tid + 1024 * j < np ? ld_dev(xp + 1024 * j) : 0ull;
    const uint32_t tag = tag_of(epoch);  // after the loads: waits for the launch count only
    bool good = true;
#pragma unroll
    for (int j = 0; j < kProPJ; ++j) good = good && (tid + 1024 * j >= np || pro_tag_ok(xv[j], tag));
    if (good) break;
    if (it == (1u << 18)) {
      atomicOr(p.err, DFSSM_ERR_WAIT_OUT_PROLOGUE);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  const float bs = p.lB ? h2f(bs_raw) : 0.0f;
  double part = 0.0;
#pragma unroll
  for (int j = 0; j < kProPJ; ++j) {
    if (tid + 1024 * j >= np) break;
    const double x0 = (double)h2f((uint16_t)xv[j]), x1 = (double)h2f((uint16_t)(xv[j] >> 32));
    part += x0 * x0;
    part += x1 * x1;
  }
  {  // sum of squares (fp64: the sums are exact)
    const double pw = wave_sum_dpp_f64(part);
    if (lane == 0) pr_d[w] = pw;
  }
  lds_barrier();
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 16; ++i) ss += pr_d[i];
  const float r = 1.0f / sqrt_rn((float)ss * (1.0f / (float)D) + 1e-5f);
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < kProPJ; ++j) {
    const int u = tid + 1024 * j;
    if (u >= np) break;
    const float x0 = r16((h2f((uint16_t)xv[j]) * r) * wv[j].x);
    const float x1 = r16((h2f((uint16_t)(xv[j] >> 32)) * r) * wv[j].y);
    mx = fmaxf(mx, fmaxf(fabsf(x0), fabsf(x1)));
    xn2[u] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
  }
  {
    const float mw = wave_max_dpp_f32(mx);
    if (lane == 0) pr_f[w] = mw;
  }
  lds_barrier();  // publishes xn and the maxima (every wave has read the squares before it)
  float amax = pr_f[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) amax = fmaxf(amax, pr_f[i]);
  const float xs = quant_scale(amax);
  const float rinv = quant_rcp(xs);
  // rank rr over this wave's quarter (fp16 x fp16 is exact in fp32)
  double hacc = 0.0;
#pragma unroll
  for (int i = 0; i < kProBI; ++i) {
    const int b = 64 * i + lane;
    if (b >= nbq) break;
    const u32x4 x8 = *(const u32x4*)&xn2[(c0 >> 1) + 4 * b];
    const uint32_t bw[2] = {bq[i].x, bq[i].y};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = h2f((uint16_t)(x8[e >> 1] >> (16 * (e & 1))));
      const float bv = r16((float)(int8_t)(bw[e >> 2] >> (8 * (e & 3))) * bs);
      hacc += (double)(x * bv);
    }
  }
  {  // per-wave partials into pr_d (its sums of squares were read before the last barrier)
    const double hw = wave_sum_dpp_f64(hacc);
    if (lane == 0) pr_d[w] = hw;
  }
  const uint16_t* xn = (const uint16_t*)xn2;
  for (int c = k * (D / 4) + tid; c < (k + 1) * (D / 4); c += kGT)
    p.q_out[(size_t)m * p.ld_q + c] = (int8_t)quant_i8(h2f(xn[c]), rinv);
  lds_barrier();  // publishes the partials
  if (tid < kProPW && p.lB)
    p.h_out[(size_t)m * DFSSM_LORA_R + kProPW * k + tid] =
        r16((float)((pr_d[4 * tid] + pr_d[4 * tid + 1]) + (pr_d[4 * tid + 2] + pr_d[4 * tid + 3])));
  if (tid == 0 && k == 0) p.xs_out[m] = xs;
}

template <int MI, int RT, int MODE, bool PRO>
__device__ __forceinline__ void gemm_body(const GemmArgs& a, const GemmPro& p) {
  constexpr int MP = MI * 16;  // activation rows per block
  constexpr int KQ = 16 / RT;  // k slots
  constexpr int kKMax = MI == 2 ? 4096 : 5120;  // the host picks MI = 2 only for K <= 4096
  constexpr int kSB = (kKMax / 128 + 4 * KQ - 1) / (4 * KQ);  // bit-chunk blocks per lane
  // LoRA term: the four rank steps of a (row tile, block tile) split over min(KQ / MI, 4) waves
  constexpr int kLoraSlots = KQ / MI < 4 ? KQ / MI : 4;
  extern __shared__ __attribute__((aligned(16))) int8_t qs[];  // MP rows x QS bytes; then partials
  __shared__ float hl[MP][DFSSM_LORA_R];
  __shared__ float xsl[MP];
  __shared__ uint32_t tag_s;  // PRO: this launch's tag
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // PRO: launch count of this workgroup (read at the start, advanced once its tag is known)
  uint32_t* cnt = nullptr;
  uint32_t epoch = 0;
  if constexpr (PRO) {
    cnt = p.launches + (size_t)blockIdx.y * gridDim.x + blockIdx.x;
    // Every thread, from a per-lane (vector) address, on both paths: loaded by thread 0 alone,
    // the value was moved at the branch join right after the load, and the workgroup waited there
    // for the count's device-scope round trip before loading its tile (a uniform address becomes a
    // scalar load, which the first LDS access would wait for); one load for both paths also keeps
    // the GEMM path from reusing its register while it is pending (a wait amid the tile's loads).
    int z = 0;
    asm volatile("" : "+v"(z));
    epoch = ld_dev(cnt + z);
    if ((int)blockIdx.y >= p.gy) {  // prologue workgroups
      const int pi = ((int)blockIdx.y - p.gy) * (int)gridDim.x + (int)blockIdx.x;
      if (pi < kProPW * a.M) gemm_in_prologue(p, a.N, pi / kProPW, pi % kProPW, epoch, (uint32_t*)qs);
      lds_barrier();  // every wave has used its tag before the count is advanced
      if (tid == 0) *cnt = epoch + 1u;  // read by the next launch only: a plain store suffices
      return;
    }
  }
  const int rt = wave % RT, kq = wave / RT, j = lane >> 4;
  const int g = blockIdx.x;
  const int K = a.K, CH = K / 128;
  const int QS = K + 16;  // padded LDS row stride
  // rows of this workgroup: blocks [blockIdx.y * bpw, +bpw) of the activation rows (one range
  // in decode; the prompt prefill spreads its thousands of rows over gridDim.y ranges)
  // (PRO: the grid rows past p.gy hold the prologue workgroups, not row ranges)
  const int grows = PRO ? p.gy : (int)gridDim.y;
  const int nblk = (a.M + MP - 1) / MP, bpw = (nblk + grows - 1) / grows;
  const int m_begin = (int)blockIdx.y * bpw * MP;
  if (m_begin >= a.M) return;
  const int m_end = m_begin + bpw * MP < a.M ? m_begin + bpw * MP : a.M;
  const int M = m_end - m_begin;  // rows of this workgroup, from m_begin

  // ---- the first row block's q tile, issued before the bits (loads complete in issue order, so
  // the tile does not wait for the weight stream from HBM) ----
  // Wave w copies rows w + 16 jr, lane l the 16-byte vectors l + 64 i of a row: no index division,
  // row addresses are scalar. Loads are unconditional from clamped indices (a load inside a branch
  // makes the compiler wait for all loads where the paths join); staging selects.
  constexpr int kQI = kKMax / 16 / 64;  // vectors per lane and row, K at most
  const int MB0 = M < MP ? M : MP;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  u32x4 qv[MI][kQI];
#pragma unroll
  for (int jr = 0; jr < MI; ++jr) {
    const int row = wv + 16 * jr;
    const int8_t* qrow = a.q + (size_t)(m_begin + (row < MB0 ? row : MB0 - 1)) * a.ld_q;
#pragma unroll
    for (int i = 0; i < kQI; ++i) {
      const int c16 = lane + 64 * i;  // lanes past the row load nothing (exec-masked)
      qv[jr][i] = c16 < K / 16 ? *(const u32x4*)(qrow + c16 * 16) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  // its LoRA intermediates and activation scales: unconditional loads from clamped indices,
  // selected when staged (using a loaded value waits for every load issued before it)
  const int hi0 = tid < MB0 * DFSSM_LORA_R ? tid : MB0 * DFSSM_LORA_R - 1;
  const int xi0 = tid < MB0 ? tid : MB0 - 1;
  float hv0 = 0.0f, xsv0 = 0.0f;
  uint16_t xsh0 = 0;
  if (MODE != DFSSM_MODE_SCAFFOLD) {
    hv0 = a.h[(size_t)m_begin * DFSSM_LORA_R + hi0];
    xsv0 = a.xs[m_begin + xi0];
  } else {
    if (a.xs16) xsh0 = a.xs16[m_begin + xi0];  // absent when only the accumulators are written
    if (a.h16) hv0 = h2f(a.h16[(size_t)m_begin * DFSSM_LORA_R + hi0]);  // stand-alone op with LoRA
  }

  // ---- this workgroup's bits (registers, loaded once for every row block) and epilogue rows,
  // kept raw until the epilogue ----
  const int r = rt * 16 + (lane & 15);  // output row within the workgroup's 16 RT
  // the bits are tiled in groups of 64 rows: [group][chunk][64 rows][16 bytes]
  const int g64 = g * RT / 4, r64 = (g * RT % 4) * 16 + r;
  u32x4 wb[kSB];
#pragma unroll
  for (int sb = 0; sb < kSB; ++sb) {
    const int c = kq + KQ * j + 4 * KQ * sb;
    // chunks past CH re-read the last one; the MFMA loop zeroes their operands
    wb[sb] = ld_nt((const u32x4*)a.bits + ((size_t)g64 * CH + (c < CH ? c : CH - 1)) * 64 + r64);
  }
  {  // the first block's q tile into LDS (waits only for the loads issued before the bits)
#pragma unroll
    for (int jr = 0; jr < MI; ++jr) {
      const int row = wv + 16 * jr;
#pragma unroll
      for (int i = 0; i < kQI; ++i) {
        const int c16 = lane + 64 * i;
        if (c16 < K / 16) *(u32x4*)(qs + (size_t)row * QS + c16 * 16) = row < MB0 ? qv[jr][i] : u32x4{0u, 0u, 0u, 0u};
      }
    }
    if (tid < MP * DFSSM_LORA_R) hl[tid >> 4][tid & 15] = tid < MB0 * DFSSM_LORA_R ? hv0 : 0.0f;
    if (tid < MP) xsl[tid] = tid < MB0 ? (MODE != DFSSM_MODE_SCAFFOLD ? xsv0 : h2f(xsh0)) : 0.0f;
  }
  const int n = g * 16 * RT + r;
  const bool nrow = n < a.N;
  u32x4 la = {0u, 0u, 0u, 0u};
  uint16_t ws_raw = 0, as_raw = 0;
  uint32_t cw01 = 0, cw23 = 0;
  uint16_t cb = 0;
  const int ch = n - a.conv_lo;
  const bool conv_row = MODE == DFSSM_MODE_IN && a.conv_state && nrow && ch >= 0 && ch < a.conv_c;
  if (nrow) {
    if (a.wscale) ws_raw = a.wscale[n];
    if (MODE != DFSSM_MODE_SCAFFOLD || a.lA) {
      la = *(const u32x4*)(a.lA + (size_t)n * DFSSM_LORA_R);
      as_raw = a.lAs[n];
    }
    if (conv_row) {
      const uint32_t* wc = (const uint32_t*)(a.conv_w + (size_t)ch * 4);
      cw01 = wc[0]; cw23 = wc[1];
      cb = a.conv_b[ch];
    }
  }
  constexpr int kEI = (4 * MI + KQ - 1) / KQ;  // epilogue elements per lane
  const bool lora = MODE != DFSSM_MODE_SCAFFOLD || a.lA;
  // partial LoRA terms [slot][rt][ib][e][lane] (fp64), after the int32 partials in the dynamic LDS
  double* lod = (double*)(qs + gemm_part_bytes(MI, RT));
  if (PRO && tid == 0) {  // read by every thread after the loop's barriers
    tag_s = (epoch + 1u) & 0xffffu;
    *cnt = epoch + 1u;  // read by the next launch only: a plain store suffices
  }
  // PRO: the next layer's prologue weights (norm weights and LoRA-B table, 20 N bytes, the first
  // 64 KiB of them) into every XCD's L2 -- workgroups 0..7 are dealt one to each XCD -- so the
  // prologue workgroups, which start only as GEMM workgroups end, do not wait on HBM for them;
  // the values are consumed (a register dependency) only after the last row block
  u32x4 pf[kProPF];
  const bool pf_on = PRO && (int)(blockIdx.y * gridDim.x + blockIdx.x) < 8;
  if (pf_on) {
    const int nw4 = a.N / 4;  // 16-byte vectors of the norm weights; the table's follow
#pragma unroll
    for (int i = 0; i < kProPF; ++i) {
      const int v = tid + kGT * i;
      pf[i] = v < nw4 ? *(const u32x4*)(p.norm_w + 4 * v)
                      : (v < nw4 + a.N && p.lB ? *(const u32x4*)(p.lB + 16 * (size_t)(v - nw4)) : u32x4{0u, 0u, 0u, 0u});
    }
    asm volatile("" ::: "memory");  // issued here, not sunk to their use
  }
#pragma nounroll
  for (int m0 = m_begin; m0 < m_end; m0 += MP) {
    const int MB = m_end - m0 < MP ? m_end - m0 : MP;  // rows in this block
    // ---- q tile, LoRA intermediates and scales of rows m0 .. m0 + MB - 1 (the first block's
    // were staged before the loop): every load is issued before the first LDS store, from
    // clamped rows, so the tile costs one memory round trip, overlapping the barrier ----
    if (RT == 4 && MI == 1 && m0 > m_begin) {
      // in_proj at 64 output rows with 16-row blocks reaches here only for d_model > 4096; the
      // unrolled copy below would raise this variant's peak registers past 128, so it copies
      // with a loop (a load round trip per vector)
      lds_barrier();  // the previous block's partials (in qs) have been read
      for (int c16 = lane; c16 < K / 16; c16 += 64) {
        u32x4 x = {0u, 0u, 0u, 0u};
        if (wv < MB) x = *(const u32x4*)(a.q + (size_t)(m0 + wv) * a.ld_q + c16 * 16);
        *(u32x4*)(qs + (size_t)wv * QS + c16 * 16) = x;
      }
      if (tid < MP * DFSSM_LORA_R) {
        const int m = tid >> 4;
        const size_t hidx = (size_t)(m0 + m) * DFSSM_LORA_R + (tid & 15);
        hl[m][tid & 15] = m >= MB ? 0.0f : (a.h ? a.h[hidx] : (a.h16 ? h2f(a.h16[hidx]) : 0.0f));
      }
      if (tid < MP) xsl[tid] = tid < MB ? (a.xs ? a.xs[m0 + tid] : (a.xs16 ? h2f(a.xs16[m0 + tid]) : 0.0f)) : 0.0f;
    } else if (m0 > m_begin) {
      // at most 4 vectors per lane and row in flight (a fifth, K > 4096, in a second round)
      constexpr int kQR = kQI > 4 ? 4 : kQI;
      const int hi = tid < MB * DFSSM_LORA_R ? tid : MB * DFSSM_LORA_R - 1;
      const int xi = tid < MB ? tid : MB - 1;
      float hv = 0.0f, xsv = 0.0f;
#pragma unroll
      for (int i0 = 0; i0 < kQI; i0 += kQR) {
        u32x4 qn[MI][kQR];
#pragma unroll
        for (int jr = 0; jr < MI; ++jr) {
          const int row = wv + 16 * jr;
          const int8_t* qrow = a.q + (size_t)(m0 + (row < MB ? row : MB - 1)) * a.ld_q;
#pragma unroll
          for (int i = 0; i < kQR; ++i) {
            const int c16 = lane + 64 * (i0 + i);
            qn[jr][i] = (i0 + i < kQI && c16 < K / 16) ? *(const u32x4*)(qrow + c16 * 16) : u32x4{0u, 0u, 0u, 0u};
          }
        }
        if (i0 == 0) {
          if (a.h) hv = a.h[(size_t)m0 * DFSSM_LORA_R + hi];
          else if (a.h16) hv = h2f(a.h16[(size_t)m0 * DFSSM_LORA_R + hi]);
          if (a.xs) xsv = a.xs[m0 + xi];
          else if (a.xs16) xsv = h2f(a.xs16[m0 + xi]);
          lds_barrier();  // the previous block's partials (in qs) have been read
        }
#pragma unroll
        for (int jr = 0; jr < MI; ++jr) {
          const int row = wv + 16 * jr;
#pragma unroll
          for (int i = 0; i < kQR; ++i) {
            const int c16 = lane + 64 * (i0 + i);
            if (i0 + i < kQI && c16 < K / 16)
              *(u32x4*)(qs + (size_t)row * QS + c16 * 16) = row < MB ? qn[jr][i] : u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
      if (tid < MP * DFSSM_LORA_R) hl[tid >> 4][tid & 15] = tid < MB * DFSSM_LORA_R ? hv : 0.0f;
      if (tid < MP) xsl[tid] = tid < MB ? xsv : 0.0f;
    }
    // the epilogue's old values -- conv state (in_proj) or residual row (out_proj) of this lane's
    // accumulator elements -- issued now and used after the MFMA loop and the LoRA term:
    // unconditional loads from clamped in-bounds indices (a load in a branch makes the compiler
    // wait for it where the paths join, before the MFMA loop)
    uint16_t pold[kEI][3];
    if constexpr (MODE == DFSSM_MODE_IN || MODE == DFSSM_MODE_OUT) {
#pragma unroll
      for (int ii = 0; ii < kEI; ++ii) {
        const int i0 = kq + KQ * ii;
        const int i = i0 < 4 * MI ? i0 : 4 * MI - 1;
        const int mb0 = (i >> 2) * 16 + 4 * j + (i & 3);
        const int mm = m0 + (mb0 < MB ? mb0 : MB - 1);
        if (MODE == DFSSM_MODE_IN) {
          const int chc = ch < 0 ? 0 : (ch < a.conv_c ? ch : a.conv_c - 1);
          const uint16_t* cs = a.conv_state ? a.conv_state + ((size_t)mm * a.conv_c + chc) * 3 : a.out;
          pold[ii][0] = cs[0];
          pold[ii][1] = cs[1];
          pold[ii][2] = cs[2];
        } else {
          pold[ii][0] = a.out[(size_t)mm * a.ld_out + (nrow ? n : a.N - 1)];
        }
      }
    }
    lds_barrier();

    // ---- MFMA over this wave's chunks ----
    // The byte expansion of the bits does not change between row blocks; a zero the compiler
    // cannot see through keeps it from hoisting all 24 expanded operands (96 registers) out of
    // the loop. (A volatile LDS word read through a generic pointer is a FLAT load, whose wait
    // is vmcnt(0): it held the MFMA loop until every earlier load, the epilogue's, had landed.)
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    v4i acc[MI];
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[i] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb) {
      if (kq + 4 * KQ * sb < CH) {  // wave-uniform: some lane group has a chunk in this block
        const int c = kq + KQ * j + 4 * KQ * sb;
        const bool valid = c < CH;
        const uint32_t lut = valid ? 0x000001ffu : 0u;  // byte 0: -1, byte 1: +1 (zero past K)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const uint32_t w = wb[sb][s >> 1] ^ zero;
          const uint32_t b16 = (s & 1) ? (w >> 16) : (w & 0xffffu);
          v4i B;
#pragma unroll
          for (int nib = 0; nib < 4; ++nib) {
            const uint32_t x = (((b16 >> (4 * nib)) & 0xfu) * 0x00204081u) & 0x01010101u;  // 0/1 bytes
            B[nib] = (int)__builtin_amdgcn_perm(0u, lut, x);                                // +-1 bytes
          }
          const int k = valid ? 128 * c + 16 * s : 0;
#pragma unroll
          for (int ib = 0; ib < MI; ++ib) {
            const v4i A = *(const v4i*)(qs + (size_t)(ib * 16 + (lane & 15)) * QS + k);
            acc[ib] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, acc[ib], 0, 0, 0);
          }
        }
      }
    }
    lds_barrier();  // q tile no longer needed: reuse it for the partials
    int* part = (int*)qs;  // [kq][rt][ib][e][lane]
#pragma unroll
    for (int ib = 0; ib < MI; ++ib)
#pragma unroll
      for (int e = 0; e < 4; ++e) part[(((kq * RT + rt) * MI + ib) * 4 + e) * 64 + lane] = acc[ib][e];
    // ---- LoRA term lo[m][n] = sum_r h[m][r] aq[n][r] on the fp64 matrix cores: per (row tile rt,
    // block tile ib) four v_mfma_f64_16x16x4f64 steps of 4 ranks (A = h, B = aq = fp16(A_i8 A_s) of
    // the lane's own output row, both exact in fp64), split over the KQ / MI waves of that tile;
    // the f64 D holds row l / 16 + 4 i of lane l in register i, the int8 accumulators row
    // 4 (l / 16) + i, so A row a carries activation row 4 (a % 4) + a / 4 and each lane then adds
    // up the partial D of its own accumulator elements. The products are exact and their sum is
    // exact in fp64 (as for the VALU sums it replaces), so the order does not matter ----
    if (lora) {
      const int ib = kq % MI, kk = kq / MI;
      if (kk < kLoraSlots) {
        v4d d = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          if (st % kLoraSlots != kk) continue;
          const int rr = 4 * st + (lane >> 4);
          const double av = (double)hl[ib * 16 + 4 * (lane & 3) + ((lane >> 2) & 3)][rr];
          const float aq = r16((float)(int8_t)((la[rr >> 2] ^ zero) >> (8 * (rr & 3))) * h2f(as_raw ^ (uint16_t)zero));
          d = __builtin_amdgcn_mfma_f64_16x16x4f64(av, (double)aq, d, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) lod[(((kk * RT + rt) * MI + ib) * 4 + i) * 64 + lane] = d[i];
      }
    }
    lds_barrier();
    // the old values are waited for here, on every path: consumed only inside the lanes'
    // branches below, they would stay pending (as far as the compiler can tell) into the next
    // row block, whose q-tile loads would then wait for them
    if constexpr (MODE == DFSSM_MODE_IN) {
#pragma unroll
      for (int ii = 0; ii < kEI; ++ii) asm volatile("" ::"v"(pold[ii][0]), "v"(pold[ii][1]), "v"(pold[ii][2]));
    } else if constexpr (MODE == DFSSM_MODE_OUT) {
#pragma unroll
      for (int ii = 0; ii < kEI; ++ii) asm volatile("" ::"v"(pold[ii][0]));
    }

    // ---- epilogue: wave (rt, kq) finishes accumulator elements i = kq, kq + KQ, ... < 4 MI ----
    if (nrow && kq < 4 * MI) {
#pragma unroll
      for (int ii = 0; ii < kEI; ++ii) {
        const int i = kq + KQ * ii;
        if (i >= 4 * MI) break;
        const int ib = i >> 2, e = i & 3;
        const int mb = ib * 16 + 4 * j + e;  // row within the block
        if (mb >= MB) continue;
        const int m = m0 + mb;
        int T = 0;
#pragma unroll
        for (int q = 0; q < KQ; ++q) T += part[(((q * RT + rt) * MI + ib) * 4 + e) * 64 + lane];
        const int accv = T;
        if (a.acc_out) a.acc_out[(size_t)m * a.N + n] = accv;
        const float y = r16(r16(r16((float)accv) * xsl[mb]) * h2f(ws_raw ^ (uint16_t)zero));
        if (MODE == DFSSM_MODE_SCAFFOLD && !a.lA) {
          if (a.out) a.out[(size_t)m * a.ld_out + n] = f2h(y);
          continue;
        }
        double lo = 0.0;
#pragma unroll
        for (int q = 0; q < kLoraSlots; ++q) lo += lod[(((q * RT + rt) * MI + ib) * 4 + e) * 64 + lane];
        float out = r16((float)lo + y);
        if (MODE == DFSSM_MODE_SCAFFOLD) {  // stand-alone op with LoRA: y + LoRA term
          if (a.out) a.out[(size_t)m * a.ld_out + n] = f2h(out);
          continue;
        }
        uint16_t* op = a.out + (size_t)m * a.ld_out + n;
        if (MODE == DFSSM_MODE_IN) {
          if (conv_row) {
            uint16_t* cs = a.conv_state + ((size_t)m * a.conv_c + ch) * 3;
            const uint16_t s0 = pold[ii][0], s1 = pold[ii][1], s2 = pold[ii][2];
            const uint16_t xo = f2h(out);
            cs[0] = s1;
            cs[1] = s2;
            cs[2] = xo;
            const float xv = h2f(xo);
            const uint32_t c01 = cw01 ^ zero, c23 = cw23 ^ zero;
            float o = h2f(s0) * h2f((uint16_t)c01);
            o = o + h2f(s1) * h2f((uint16_t)(c01 >> 16));
            o = o + h2f(s2) * h2f((uint16_t)c23);
            o = o + xv * h2f((uint16_t)(c23 >> 16));
            o = o + h2f(cb ^ (uint16_t)zero);
            const float sig = 1.0f / (1.0f + dev_expf(-o));
            out = o * sig;
          }
          *op = f2h(out);
        } else {
          const uint16_t xv = f2h(h2f(pold[ii][0]) + out);
          *op = xv;
          if (PRO) st_dev(p.xT + (size_t)m * a.N + n, (tag_s << 16) | xv);
        }
      }
    }
  }
  if (pf_on) {
#pragma unroll
    for (int i = 0; i < kProPF; ++i) asm volatile("" ::"v"(pf[i][0]));
  }
}

// The kernels: the GEMM alone, and out_proj with the next layer's prologue (separate entry points,
// so that the GEMM alone keeps its own argument block and LDS)
template <int MI, int RT, int MODE>
__global__ __launch_bounds__(kGT) void gemm_kernel(GemmArgs a) {
  gemm_body<MI, RT, MODE, false>(a, GemmPro{});
}
template <int MI, int RT>
__global__ __launch_bounds__(kGT) void gemm_pro_kernel(GemmArgs a, GemmPro p) {
  gemm_body<MI, RT, DFSSM_MODE_OUT, true>(a, p);
}

static size_t gemm_lds_bytes(int MI, int RT, int K) {
  const size_t tile = (size_t)MI * 16 * (K + 16);
  const size_t part = gemm_part_bytes(MI, RT) + gemm_lora_bytes(MI, RT);
  return tile > part ? tile : part;
}

template <int MI, int RT, int MODE, bool PRO>
static hipError_t launch_gemm_mi(const GemmArgs& a, const GemmPro* pro, hipStream_t s) {
  const size_t shm = gemm_lds_bytes(MI, RT, a.K);
  // one workgroup per CU (registers and LDS). Decode batches: with 16 output rows per workgroup
  // (N <= 4096: 128..256 workgroups) one row block per workgroup, the blocks in a second grid
  // dimension (a further round of workgroups starts as CUs free up, where a workgroup walking its
  // blocks pays each block's q-tile round trip and epilogue in turn: out_proj 7.0 -> 6.3 us at
  // batch 32, 18.5 -> 16.2 us at the 2.7B shape and batch 64); with 32 or 64 output rows per
  // workgroup (133..166 workgroups) the blocks stay in one workgroup (a second round measured
  // slower). Many rows (prefill) are split into ranges so that the grid fills about two rounds.
  const int gx = (a.N + 16 * RT - 1) / (16 * RT);
  const int nblk = (a.M + MI * 16 - 1) / (MI * 16);
  int gy = a.M > 64 ? (512 + gx / 2) / gx : (RT == 1 ? nblk : 1);
  gy = gy < 1 ? 1 : (gy > nblk ? nblk : gy);
  int cus = 0;
  if (PRO) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                 hipSuccess)
      return hipErrorNotSupported;
  }
  // PRO: every GEMM grid row must hold rows (each workgroup advances its launch count once), the
  // prologue's normalized row lives in the dynamic LDS, the counts in kGemmProMaxWg words; a
  // shape outside these is refused before anything is set or launched
  const int gyp = gy + (kProPW * a.M + gx - 1) / gx;
  if (PRO && ((gy - 1) * ((nblk + gy - 1) / gy) >= nblk || shm < (size_t)2 * a.N ||
              (long long)gx * gyp > kGemmProMaxWg))
    return hipErrorNotSupported;
  // The prologue workgroups inherit the GEMM's registers and LDS (one workgroup per CU), so they
  // run on CUs the GEMM's last round leaves free, or after it. A GEMM of whole rounds leaves none:
  // then the prologue's tail cost what its own launch does (batch 32, 256 workgroups: 2322 ->
  // 2338 us per decode step), against 6783 -> 6738 us at the 2.7B shape and batch 64 (640
  // workgroups). Refused for whole rounds. (One GEMM grid row instead, each workgroup walking the
  // row blocks so that the prologue runs beside the GEMM on the free half of the CUs, was slower
  // still: 2322 -> 2514 us.)
  if (PRO && cus > 0 && (gx * gy) % cus == 0) return hipErrorNotSupported;
  if constexpr (PRO) {
    static_assert(MODE == DFSSM_MODE_OUT, "the prologue follows out_proj");
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_pro_kernel<MI, RT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
    GemmPro p = *pro;
    p.gy = gy;
    hipLaunchKernelGGL((gemm_pro_kernel<MI, RT>), dim3(gx, gyp), dim3(kGT), shm, s, a, p);
  } else {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<MI, RT, MODE>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_kernel<MI, RT, MODE>), dim3(gx, gy), dim3(kGT), shm, s, a);
  }
  return hipGetLastError();
}

template <int MI, int MODE, bool PRO>
static hipError_t launch_gemm_rt(const GemmArgs& a, const GemmPro* pro, hipStream_t s) {
  // the fewest output rows per workgroup (16, 32 or 64) that keep the grid within one workgroup
  // per CU (256): a workgroup fills its CU, so a grid beyond 256 runs a second round
  if (a.N <= 256 * 16) return launch_gemm_mi<MI, 1, MODE, PRO>(a, pro, s);
  if (a.N <= 256 * 32) return launch_gemm_mi<MI, 2, MODE, PRO>(a, pro, s);
  return launch_gemm_mi<MI, 4, MODE, PRO>(a, pro, s);
}

template <int MODE, bool PRO>
static hipError_t launch_gemm_mode(const GemmArgs& a, const GemmPro* pro, hipStream_t s) {
  // one launch for all rows, in blocks whose q tile (rows x (K + 16) bytes) fits the 160 KiB of
  // LDS: 32 rows up to K = 4096, 16 above; 16 also for N <= 4096 (one row block per workgroup,
  // see launch_gemm_mi: more, smaller blocks spread over more CUs)
  return (a.M > 16 && a.K <= 4096 && a.N > 4096) ? launch_gemm_rt<2, MODE, PRO>(a, pro, s)
                                                  : launch_gemm_rt<1, MODE, PRO>(a, pro, s);
}

// ---------------------------------------------------------------------------------------------
// Wide GEMM for the prompt prefill (thousands of activation rows). The sign bits are expanded once
// per projection to int8 +-1 (expand_bits_kernel: W8 row-major (N, K)), then a plain MFMA GEMM:
// a workgroup of 4 waves owns a 128 x 128 tile (activation rows x output rows), wave w the 64 x 64
// quarter (rows 64 (w & 1), outputs 64 (w >> 1)) as 4 x 4 tiles of v_mfma_i32_16x16x64_i8, its A
// (q) and B (W8) operands loaded straight into registers two k steps ahead (three-stage ring; loads
// complete in issue order). Both operands are stored in 16-row tiles (wide_tiled_offset), so the
// MFMA lane layout (lane l: row l % 16, 16 bytes of k block l / 16) is one contiguous 1 KiB per
// wave-wide load; row-major rows K bytes apart put every lane on its own cache line. acc = sum_k q[m][k] W8[n][k] is exact (int32), i.e. gemm_kernel's
// acc; the epilogue is gemm_kernel's, operation for operation (scales, LoRA term in fp64, proj
// rows or residual add). Workgroup -> tile: workgroups are dealt to the 8 XCDs in turn, so XCD x
// takes the row tiles m = x (mod 8) (each activation tile is read by one XCD's L2) and walks the
// output tiles of one row tile after another.
// ---------------------------------------------------------------------------------------------
// W8 = bit k of row n ? +1 : -1 in the wide tiled layout; one thread per (row, 128-column chunk)
// of the tiled bits.
__global__ __launch_bounds__(256) void expand_bits_kernel(const uint32_t* __restrict__ bits, int8_t* __restrict__ w8,
                                                          int N, int K) {
  const int CH = K / 128;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= N * CH) return;
  const int n = i / CH, c = i - n * CH;
  const u32x4 b = ld_nt(bits + (((size_t)(n >> 6) * CH + c) * 64 + (n & 63)) * 4);
#pragma unroll
  for (int q = 0; q < 8; ++q) {  // 16 columns 128 c + 16 q .. + 15: bits 16 q .. of the chunk
    const uint32_t h16 = (b[q >> 1] >> (16 * (q & 1))) & 0xffffu;
    uint32_t o[4];
#pragma unroll
    for (int nib = 0; nib < 4; ++nib) {
      const uint32_t x = (((h16 >> (4 * nib)) & 0xfu) * 0x00204081u) & 0x01010101u;  // 0/1 bytes
      o[nib] = __builtin_amdgcn_perm(0u, 0x000001ffu, x);                             // -> -1/+1
    }
    *(u32x4*)(w8 + wide_tiled_offset(n, 128 * c + 16 * q, K)) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

constexpr int kWT = 128;  // tile edge (rows and outputs)

template <int MODE>
__global__ __launch_bounds__(256) void gemm_wide_kernel(GemmArgs a, const int8_t* __restrict__ w8, int TN) {
  __shared__ float hl[kWT][DFSSM_LORA_R];
  __shared__ float xsl[kWT];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int L = (int)blockIdx.x, xcd = L & 7, j = L >> 3;
  const int tm = 8 * (j / TN) + xcd, tn = j % TN;
  const int TM = (a.M + kWT - 1) / kWT;
  if (tm >= TM) return;  // uniform over the workgroup
  const int m0 = tm * kWT, n0 = tn * kWT, K = a.K, KS = K / 64;
  const int lr = lane & 15;
  // operand bases: 16-row tiles of the tiled layouts, lane l at byte 16 l of a (tile, k step)
  // (tiles past the last one are clamped to it: their results are discarded)
  const int lastA = (a.M + 15) / 16 - 1, lastB = (a.N + 15) / 16 - 1;
  uint32_t ao[4], bo[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int ta = (m0 + 64 * wm + 16 * t) >> 4, tb = (n0 + 64 * wn + 16 * t) >> 4;
    ao[t] = (uint32_t)((ta < lastA ? ta : lastA) * KS * 1024 + 16 * lane);
    bo[t] = (uint32_t)((tb < lastB ? tb : lastB) * KS * 1024 + 16 * lane);
  }
  v4i acc[4][4];
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) acc[ti][tj] = v4i{0, 0, 0, 0};
  v4i A[3][4], B[3][4];
  auto load = [&](int st, int step) {
    const uint32_t ko = (uint32_t)(1024 * (step < KS ? step : KS - 1));  // the ring's overrun re-reads
#pragma unroll
    for (int t = 0; t < 4; ++t) A[st][t] = *(const v4i*)(a.q + ao[t] + ko);
#pragma unroll
    for (int t = 0; t < 4; ++t) B[st][t] = *(const v4i*)(w8 + bo[t] + ko);
  };
  auto mma = [&](int st) {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < 4; ++tj) acc[ti][tj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[st][ti], B[st][tj], acc[ti][tj], 0, 0, 0);
  };
  load(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load(1, 1);
  __builtin_amdgcn_sched_barrier(0);
  // whole groups of three steps (K / 64 = 8, 16, ... 80: the last group may run past KS; those
  // steps multiply a re-read of step KS - 1 and are skipped)
  for (int s = 0; s < KS; s += 3) {
    load(2, s + 2);
    __builtin_amdgcn_sched_barrier(0);
    mma(0);
    load(0, s + 3);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < KS) mma(1);
    load(1, s + 4);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 2 < KS) mma(2);
  }

  // ---- epilogue (gemm_kernel's): the tile's LoRA intermediates and activation scales in LDS ----
  for (int i = tid; i < kWT * DFSSM_LORA_R; i += 256) {
    const int m = m0 + i / DFSSM_LORA_R;
    (&hl[0][0])[i] = m < a.M ? a.h[(size_t)m * DFSSM_LORA_R + i % DFSSM_LORA_R] : 0.0f;
  }
  if (tid < kWT) xsl[tid] = m0 + tid < a.M ? a.xs[m0 + tid] : 0.0f;
  __syncthreads();
#pragma unroll  // (a runtime tj would index the accumulators dynamically: scratch memory)
  for (int tj = 0; tj < 4; ++tj) {
    const int n = n0 + 64 * wn + 16 * tj + lr;
    if (n >= a.N) continue;
    const u32x4 la = *(const u32x4*)(a.lA + (size_t)n * DFSSM_LORA_R);
    const float as = h2f(a.lAs[n]), ws = h2f(a.wscale[n]);
    double aqd[DFSSM_LORA_R];
#pragma unroll
    for (int rr = 0; rr < DFSSM_LORA_R; ++rr) aqd[rr] = (double)r16((float)(int8_t)(la[rr >> 2] >> (8 * (rr & 3))) * as);
    uint16_t old[4][4];
    if (MODE == DFSSM_MODE_OUT) {  // the residual rows, all loaded before any is used
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + 64 * wm + 16 * ti + 4 * (lane >> 4) + e;
          old[ti][e] = a.out[(size_t)(m < a.M ? m : a.M - 1) * a.ld_out + n];
        }
    }
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int mb = 64 * wm + 16 * ti + 4 * (lane >> 4) + e, m = m0 + mb;
        if (m >= a.M) continue;
        const int accv = acc[ti][tj][e];
        const float y = r16(r16(r16((float)accv) * xsl[mb]) * ws);
        double lo = 0.0;
#pragma unroll
        for (int rr = 0; rr < DFSSM_LORA_R; ++rr) lo += (double)hl[mb][rr] * aqd[rr];
        const float out = r16((float)lo + y);
        uint16_t* op = a.out + (size_t)m * a.ld_out + n;
        if (MODE == DFSSM_MODE_IN) *op = f2h(out);
        else *op = f2h(h2f(old[ti][e]) + out);
      }
  }
}

size_t gemm_wide_w8_bytes(int N, int K) { return (size_t)(N + 15) / 16 * 16 * K; }

hipError_t launch_gemm_wide(const GemmArgs& a, int mode, int8_t* w8, hipStream_t s) {
  if (a.M < 1 || a.K % 512 || a.K > 5120 || !a.h || !a.xs || !a.lA || !a.lAs || !a.wscale || a.conv_state ||
      a.acc_out || (mode != DFSSM_MODE_IN && mode != DFSSM_MODE_OUT))
    return hipErrorInvalidValue;
  const int CH = a.K / 128;
  hipLaunchKernelGGL(expand_bits_kernel, dim3((a.N * CH + 255) / 256), dim3(256), 0, s, a.bits, w8, a.N, a.K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int TM = (a.M + kWT - 1) / kWT, TN = (a.N + kWT - 1) / kWT;
  const dim3 g(8 * ((TM + 7) / 8) * TN);
  if (mode == DFSSM_MODE_IN) hipLaunchKernelGGL(gemm_wide_kernel<DFSSM_MODE_IN>, g, dim3(256), 0, s, a, w8, TN);
  else hipLaunchKernelGGL(gemm_wide_kernel<DFSSM_MODE_OUT>, g, dim3(256), 0, s, a, w8, TN);
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs& a, int mode, hipStream_t s) {
  if (a.M < 1 || a.M > kGemmMaxRows || a.K % 512 || a.K > 5120) return hipErrorInvalidValue;
  switch (mode) {
    case DFSSM_MODE_IN: return launch_gemm_mode<DFSSM_MODE_IN, false>(a, nullptr, s);
    case DFSSM_MODE_OUT: return launch_gemm_mode<DFSSM_MODE_OUT, false>(a, nullptr, s);
    case DFSSM_MODE_SCAFFOLD: return launch_gemm_mode<DFSSM_MODE_SCAFFOLD, false>(a, nullptr, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_out_pro(const GemmArgs& a, const GemmPro& p, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || a.K % 512 || a.K > 5120 || a.N % 512 || a.N > 5120) return hipErrorNotSupported;
  if (!a.out || !a.lA || !a.lAs) return hipErrorInvalidValue;
  if (!p.xT || !p.launches || !p.err || !p.norm_w || !p.q_out || !p.xs_out || !p.h_out || p.ld_q < a.N ||
      (p.lB && !p.lBs))
    return hipErrorInvalidValue;
  return launch_gemm_mode<DFSSM_MODE_OUT, true>(a, &p, s);
}

}  // namespace dfssm
