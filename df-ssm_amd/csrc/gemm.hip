// Batched scaffold projection (M = 5..64 activation rows) on the int8 matrix cores (gfx950).
//
// T[m][n] = sum_k q[m][k] * bit[n][k] is computed with v_mfma_i32_16x16x64_i8: A = q (16 rows x
// 64 k, int8), B = the sign bits of 16 output rows expanded in registers to 0/1 bytes, and
// acc = 2 T - sum_k q[m][k] (exact int32; acc = sum_k q * (2 bit - 1)). Expansion of a nibble to
// four 0/1 bytes is one multiply and one mask: (nib * 0x00204081) & 0x01010101 -- the four
// shifted copies of the nibble occupy disjoint bit ranges, so the product has no carries.
//
// One workgroup (256 threads, 4 waves) owns a group of 64 output rows; wave w owns rows 16w..16w+15
// of it for all MI*16 activation rows (MI accumulator tiles per wave). K is walked in 512-column
// chunks: the chunk's q tile (MI*16 x 512 bytes, LDS rows padded to avoid bank conflicts) and
// the group's 4 KiB of sign bits are staged in LDS while the next chunk is already loading into
// registers. Epilogues are those of the GEMV path (dequant, LoRA, conv + SiLU or residual).
#include "common.h"
#include "dfssm_kernels.h"

namespace dfssm {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGT = 256;
constexpr int kKC = 512;        // K chunk
constexpr int kQS = kKC + 16;   // LDS row stride of the q tile (bytes)

template <int MI, int MODE>
__global__ __launch_bounds__(kGT) void gemm_kernel(GemmArgs a) {
  constexpr int MP = MI * 16;
  __shared__ __attribute__((aligned(16))) int8_t qs[MP][kQS];
  __shared__ __attribute__((aligned(16))) uint32_t bsm[kKC / 128][64][4];
  __shared__ int Ssum[MP];
  __shared__ float hl[MP][DFSSM_LORA_R];
  __shared__ float xsl[MP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x;
  const int K = a.K, CH = K / 128, nchunks = K / kKC, M = a.M;

  for (int i = tid; i < MP * DFSSM_LORA_R; i += kGT) {
    const int m = i >> 4;
    hl[m][i & 15] = (a.h && m < M) ? a.h[i] : 0.0f;
  }
  if (tid < MP) {
    Ssum[tid] = 0;
    xsl[tid] = tid < M ? (a.xs ? a.xs[tid] : (a.xs16 ? h2f(a.xs16[tid]) : 0.0f)) : 0.0f;
  }

  // epilogue row data: lane's output row n (same for all its accumulator elements)
  const int n = g * 64 + wave * 16 + (lane & 15);
  const bool nrow = n < a.N;
  u32x4 la = {0u, 0u, 0u, 0u};
  float e_ws = 0.0f, e_as = 0.0f;
  uint32_t cw01 = 0, cw23 = 0;
  uint16_t cb = 0;
  const int ch = n - a.conv_lo;
  const bool conv_row = MODE == DFSSM_MODE_IN && nrow && ch >= 0 && ch < a.conv_c;
  if (nrow) {
    if (a.wscale) e_ws = h2f(a.wscale[n]);
    if (MODE != DFSSM_MODE_SCAFFOLD) {
      la = *(const u32x4*)(a.lA + (size_t)n * DFSSM_LORA_R);
      e_as = h2f(a.lAs[n]);
    }
    if (conv_row) {
      const uint32_t* wc = (const uint32_t*)(a.conv_w + (size_t)ch * 4);
      cw01 = wc[0]; cw23 = wc[1];
      cb = a.conv_b[ch];
    }
  }

  // chunk loads: q tile vectors (row, 16-byte column) and this thread's 16 bytes of bits
  u32x4 qreg[2 * MI];
  u32x4 breg;
  const u32x4* bits = (const u32x4*)a.bits + (size_t)g * CH * 64 + tid;
  auto load_chunk = [&](int t) {
#pragma unroll
    for (int p = 0; p < 2 * MI; ++p) {
      const int v = tid + kGT * p, row = v >> 5, c16 = v & 31;
      qreg[p] = row < M ? *(const u32x4*)(a.q + (size_t)row * a.ld_q + t * kKC + c16 * 16) : u32x4{0u, 0u, 0u, 0u};
    }
    breg = ld_nt(bits + (size_t)t * 4 * 64);
  };

  v4i acc[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) acc[i] = v4i{0, 0, 0, 0};
  load_chunk(0);
  for (int t = 0; t < nchunks; ++t) {
    __syncthreads();  // previous chunk's readers are done
#pragma unroll
    for (int p = 0; p < 2 * MI; ++p) {
      const int v = tid + kGT * p, row = v >> 5, c16 = v & 31;
      *(u32x4*)&qs[row][c16 * 16] = qreg[p];
      if (row < M) {
        int s = 0;
#pragma unroll
        for (int e = 0; e < 16; ++e) s += (int)(int8_t)(qreg[p][e >> 2] >> (8 * (e & 3)));
        atomicAdd(&Ssum[row], s);
      }
    }
    ((u32x4*)&bsm[0][0][0])[tid] = breg;
    __syncthreads();
    if (t + 1 < nchunks) load_chunk(t + 1);
#pragma unroll
    for (int s = 0; s < kKC / 64; ++s) {
      const int r = wave * 16 + (lane & 15);
      const int kl = 64 * s + 16 * (lane >> 4);
      const uint32_t w = bsm[kl >> 7][r][(kl & 127) >> 5];
      const uint32_t b16 = (kl & 16) ? (w >> 16) : (w & 0xffffu);
      v4i B;
#pragma unroll
      for (int nib = 0; nib < 4; ++nib) B[nib] = (int)((((b16 >> (4 * nib)) & 0xfu) * 0x00204081u) & 0x01010101u);
#pragma unroll
      for (int ib = 0; ib < MI; ++ib) {
        const v4i A = *(const v4i*)&qs[ib * 16 + (lane & 15)][kl];
        acc[ib] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, acc[ib], 0, 0, 0);
      }
    }
  }
  __syncthreads();

  // epilogue: accumulator element (ib, v) is T[m = 16 ib + 4 (lane / 16) + v][n]
  if (!nrow) return;
#pragma unroll
  for (int ib = 0; ib < MI; ++ib) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = ib * 16 + 4 * (lane >> 4) + v;
      if (m >= M) continue;
      const int accv = 2 * acc[ib][v] - Ssum[m];
      if (a.acc_out) a.acc_out[(size_t)m * a.N + n] = accv;
      const float y = r16(r16(r16((float)accv) * xsl[m]) * e_ws);
      if (MODE == DFSSM_MODE_SCAFFOLD) {
        if (a.out) a.out[(size_t)m * a.ld_out + n] = f2h(y);
        continue;
      }
      double lo = 0.0;
#pragma unroll
      for (int rr = 0; rr < DFSSM_LORA_R; ++rr) {
        const float aq = r16((float)(int8_t)(la[rr >> 2] >> (8 * (rr & 3))) * e_as);
        lo += (double)hl[m][rr] * (double)aq;
      }
      float out = r16((float)lo + y);
      uint16_t* op = a.out + (size_t)m * a.ld_out + n;
      if (MODE == DFSSM_MODE_IN) {
        if (conv_row) {
          uint16_t* cs = a.conv_state + ((size_t)m * a.conv_c + ch) * 3;
          const uint16_t s0 = cs[0], s1 = cs[1], s2 = cs[2];
          const uint16_t xo = f2h(out);
          cs[0] = s1;
          cs[1] = s2;
          cs[2] = xo;
          const float xv = h2f(xo);
          float o = h2f(s0) * h2f((uint16_t)cw01);
          o = o + h2f(s1) * h2f((uint16_t)(cw01 >> 16));
          o = o + h2f(s2) * h2f((uint16_t)cw23);
          o = o + xv * h2f((uint16_t)(cw23 >> 16));
          o = o + h2f(cb);
          const float sig = 1.0f / (1.0f + dev_expf(-o));
          out = o * sig;
        }
        *op = f2h(out);
      } else {
        *op = f2h(h2f(*op) + out);
      }
    }
  }
}

template <int MODE>
static hipError_t launch_gemm_mode(const GemmArgs& a, hipStream_t s) {
  const int groups = (a.N + 63) / 64;
  const int MI = (a.M + 15) / 16;
  switch (MI) {
    case 1: hipLaunchKernelGGL((gemm_kernel<1, MODE>), dim3(groups), dim3(kGT), 0, s, a); break;
    case 2: hipLaunchKernelGGL((gemm_kernel<2, MODE>), dim3(groups), dim3(kGT), 0, s, a); break;
    case 3: hipLaunchKernelGGL((gemm_kernel<3, MODE>), dim3(groups), dim3(kGT), 0, s, a); break;
    case 4: hipLaunchKernelGGL((gemm_kernel<4, MODE>), dim3(groups), dim3(kGT), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs& a, int mode, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || a.K % kKC) return hipErrorInvalidValue;
  switch (mode) {
    case DFSSM_MODE_IN: return launch_gemm_mode<DFSSM_MODE_IN>(a, s);
    case DFSSM_MODE_OUT: return launch_gemm_mode<DFSSM_MODE_OUT>(a, s);
    case DFSSM_MODE_SCAFFOLD: return launch_gemm_mode<DFSSM_MODE_SCAFFOLD>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dfssm
