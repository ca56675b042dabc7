// Internal kernel argument blocks and launchers (not part of the C-ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dfssm.h"  // DFSSM_ERR_* bits of the workspace error flag

#define DFSSM_MODE_IN 0
#define DFSSM_MODE_OUT 1
#define DFSSM_MODE_SCAFFOLD 2

namespace dfssm {

// Prologue of a projection, once per activation row (prep_kernel).
struct PrepArgs {
  const uint16_t* act;       // activation rows (M, ld_act) fp16: x (IN) or gated g (OUT)
  int ld_act;
  const float* norm_w;       // (K) fp32 RMSNorm weight: ln_w (IN) or norm_w (OUT)
  const double* sumsq_slots; // OUT: (M, n_slots) per-block sum(g^2) from the SSM kernel
  int n_slots;
  const int8_t* lB;          // (16, K) LoRA B, int8 (null: no LoRA intermediate)
  const uint16_t* lBs;       // (16) fp16
  int8_t* q_out;             // (M, ld_q) int8 activations, or null
  uint32_t* planes_out;      // (M, ld_q/32, 8) bit planes of q, or null
  int ld_q;
  int* s_out;                // (M) sum of q
  float* xs_out;             // (M) activation scale (an fp16 value)
  float* h_out;              // (M, 16) LoRA intermediate (fp16 values)
  uint16_t* xn_out;          // (M, K) normalized activations, or null
  uint16_t* xs16_out;        // (M) activation scale as fp16 bits, or null
  int K;
  int q_tiled;               // q_out in the 16-row tiled layout of the wide GEMM (many-row path only)
};
// The wide GEMM's operand layout (activations q and expanded weights): 16-row tiles of 64-column
// k steps, [row / 16][k / 64][(k / 16) % 4][row % 16][k % 16], so that lane l of a wave reading
// (row tile, k step) takes bytes 16 l .. 16 l + 15: one contiguous 1 KiB per wave-wide load.
// K is a multiple of 64; the rows are padded to a multiple of 16.
__host__ __device__ inline size_t wide_tiled_offset(int row, int k, int K) {
  return (((size_t)(row >> 4) * (K >> 6) + (k >> 6)) * 4 + ((k >> 4) & 3)) * 256 + (row & 15) * 16 + (k & 15);
}

struct ProjArgs {
  const uint32_t* bits;      // tiled sign bits [N_pad/64][K/128][64][4]
  const uint16_t* wscale;    // (N) fp16 per-row scale
  const int8_t* lA;          // (N, 16) LoRA A, int8
  const uint16_t* lAs;       // (N) fp16
  const uint32_t* planes;    // prep: (M, ld_q/32, 8) bit planes
  int ld_q;
  const int* qsum;           // prep: (M)
  const float* xs;           // prep: (M)
  const float* h;            // prep: (M, 16)
  uint16_t* out;             // IN: proj (M, ld_out); OUT: residual x (M, ld_out), updated in place
  int ld_out;
  int32_t* acc_out;          // optional (M, N) int32 scaffold accumulators
  // IN only: conv1d applied to rows [conv_lo, conv_lo + conv_c)
  uint16_t* conv_state;      // (M, conv_c, 3) fp16
  const uint16_t* conv_w;    // (conv_c, 4) fp16
  const uint16_t* conv_b;    // (conv_c) fp16
  int conv_lo, conv_c;
  int N, K;
};

// Batched projection on the int8 matrix cores (M = 1..64 rows; used for M >= 5).
struct GemmArgs {
  const uint32_t* bits;      // tiled sign bits
  const uint16_t* wscale;    // (N) fp16
  const int8_t* lA;          // (N, 16) (IN / OUT)
  const uint16_t* lAs;       // (N) (IN / OUT)
  const int8_t* q;           // (M, ld_q) int8 activations
  int ld_q, M;
  const float* xs;           // (M) activation scales (fp16 values) or null
  const uint16_t* xs16;      // (M) fp16 activation scales (SCAFFOLD), used when xs is null
  const float* h;            // (M, 16) LoRA intermediate (IN / OUT)
  const uint16_t* h16;       // SCAFFOLD with LoRA (lA non-null): (M, 16) fp16 intermediates
  uint16_t* out;             // IN: proj; OUT: residual x (in place); SCAFFOLD: y (may be null)
  int ld_out;
  int32_t* acc_out;          // optional (M, N) accumulators
  uint16_t* conv_state;      // IN: (M, conv_c, 3); null: the conv rows are written raw (prefill)
  const uint16_t* conv_w;
  const uint16_t* conv_b;
  int conv_lo, conv_c;
  int N, K;
};
constexpr int kGemmMaxRows = 32768;
// Decode at batch >= 5: the next layer's in_proj prologue (prep_kernel<IN>'s outputs) computed
// by M extra workgroups of the out_proj launch, after every GEMM workgroup, from the new x rows
// handed over as tagged words (tag << 16) | fp16.
struct GemmPro {
  uint32_t* xT;              // (M, N) tagged words of the new x, rewritten by every launch
  uint32_t* launches;        // per-workgroup launch counts (kGemmProMaxWg), zeroed at init
  int* err;                  // DFSSM_ERR_WAIT_OUT_PROLOGUE: a wait timed out
  const float* norm_w;       // (N) fp32 RMSNorm weight of the next layer
  const int8_t* lB;          // (16, N) its LoRA B, int8 (null: no LoRA intermediate)
  const uint16_t* lBs;       // (16) fp16
  int8_t* q_out;             // (M, ld_q) int8 activations
  int ld_q;
  float* xs_out;             // (M) activation scale (an fp16 value)
  float* h_out;              // (M, 16) LoRA intermediate (fp16 values)
  int gy;                    // set by the launch: grid rows of GEMM workgroups (prologues follow)
};
constexpr int kGemmProMaxWg = 4096;  // workgroups of one out_proj launch with the prologue
// out_proj (MODE_OUT) with the next layer's prologue; hipErrorNotSupported (nothing launched) for
// a shape it does not take (M > 64, N not a multiple of 512 or above 5120, a grid beyond
// kGemmProMaxWg), so the caller runs the two kernels instead
hipError_t launch_gemm_out_pro(const GemmArgs& a, const GemmPro& p, hipStream_t s);
  // activation rows of one gemm_kernel launch (prefill)

struct ScaffoldArgs {
  const uint32_t* bits;      // tiled sign bits
  const int8_t* q;           // (M, K) int8 activations
  const uint16_t* xscale;    // (M) fp16 (needed only with y_out)
  const uint16_t* wscale;    // (N) fp16 (needed only with y_out)
  int32_t* acc_out;          // (M, N) or null
  uint16_t* y_out;           // (M, N) fp16(fp16(fp16(acc) * xs) * ws) [+ LoRA term] or null
  const int8_t* lA;          // optional LoRA: (N, 16) int8 A, (N) fp16 scales, (M, 16) fp16 h
  const uint16_t* lAs;
  const uint16_t* h16;
  int N, K;
  // M <= 4 with LoRA (one launch): the intermediates are computed in the kernel from xn and the
  // fp16 LoRA-B table, and written to h_out
  const uint16_t* xn;        // (M, K) fp16
  const uint16_t* lBq;       // (16, K) fp16(B_i8 * B_s)
  uint16_t* h_out;           // (M, 16) fp16
  // exchange workspace of the one-launch LoRA form (rank workgroups hand the intermediates to the
  // GEMV workgroups as tagged words): per-workgroup call counts, an error word, then kScafRep
  // copies of the 16 M tagged words; null: the intermediates are computed in every workgroup
  uint32_t* ws;
};
constexpr int kScafGrid = 256;                    // workgroups of every exchange launch
constexpr int kScafMaxGroups = kScafGrid - 16;    // 64-row output groups after the 16 rank workgroups
constexpr int kScafErr = kScafGrid, kScafWords = kScafGrid + 64;
constexpr int kScafRep = 8, kScafStride = 1024;  // copies of the tagged intermediates, words apart
constexpr size_t kScafWsBytes = (size_t)(kScafWords + kScafRep * kScafStride) * 4;
static_assert(kScafWsBytes <= DFSSM_SCAFFOLD_WORKSPACE_BYTES, "scaffold exchange workspace");
static_assert(kScafErr * 4 == DFSSM_SCAFFOLD_ERROR_OFFSET, "scaffold exchange error word");

// LoRA intermediates of the stand-alone scaffold op: h[m][r] = fp16(sum_k xn[m][k] * lBq[r][k]).
struct LoraHArgs {
  const uint16_t* xn;        // (M, K) fp16
  const uint16_t* lBq;       // (16, K) fp16(B_i8 * B_s)
  uint16_t* h;               // (M, 16) fp16
  int K;
};
hipError_t launch_lora_h(const LoraHArgs& a, int M, hipStream_t s);

struct SsmArgs {
  float* h;                  // (M, H, P, N) fp32 state, updated in place
  const uint16_t* xbc;       // (M, ld_xbc) fp16 rows x | B | C (after the conv)
  int ld_xbc;
  const uint16_t* dt;        // (M, ld_dt) fp16 raw dt
  int ld_dt;
  const uint16_t* z;         // (M, ld_z) fp16 gate input, or null for plain y
  int ld_z;
  const float* dt_bias;
  const float* A_log;
  const float* D;
  uint16_t* y_out;           // (M, ld_y) fp16: g (gated) or y
  int ld_y;
  double* sumsq_slots;       // (M, n_slots) per-block sum(g^2), or null
  int n_slots;
  int H, P, N;
};

// Decode at batch >= 5: the SSM step + gate (SsmArgs, whose y_out and sumsq_slots are unused) and
// the gated-norm prologue of out_proj (prep_kernel<OUT>'s outputs) in one launch. The gated g
// travels between the launch's workgroups as tagged words (tag << 16) | fp16 in gT.
struct SsmPrepArgs {
  SsmArgs s;
  uint32_t* gT;              // (M, H P) tagged words, rewritten by every launch
  uint32_t* launches;        // ((H P / 16 + 16) M) per-workgroup launch counts, zeroed at init
  int* err;                  // DFSSM_ERR_WAIT_SSM_PROLOGUE: a wait timed out
  const float* norm_w;       // (H P) fp32 gated-RMSNorm weight
  const int8_t* lB;          // (16, H P) LoRA B, int8 (null: no LoRA intermediate)
  const uint16_t* lBs;       // (16) fp16
  int8_t* q_out;             // (M, ld_q) int8 activations
  int ld_q;
  float* xs_out;             // (M) activation scale (an fp16 value)
  float* h_out;              // (M, 16) LoRA intermediate (fp16 values)
};
// Whether launch_ssm_prep takes these dimensions (K = H P <= 5120, a multiple of 512; P % 16 == 0).
bool ssm_prep_supported(int M, int K, int P);
hipError_t launch_ssm_prep(const SsmPrepArgs& a, int M, hipStream_t s);

struct ConvArgs {
  uint16_t* state;           // (M, C, 3) fp16
  uint16_t* x;               // (M, ld) fp16, in place
  const uint16_t* w;         // (C, 4)
  const uint16_t* b;         // (C)
  int ld, C;
};

// Prompt prefill (prefill.hip): conv over the tokens of each sequence, rows (b, t) at b * T + t.
struct ConvSeqArgs {
  uint16_t* state;           // (batch, C, 3) fp16, advanced by T tokens
  uint16_t* x;               // rows (batch * T, ld): raw xBC in, conv'd + SiLU out (in place)
  int ld;
  const uint16_t* w;         // (C, 4)
  const uint16_t* b;         // (C)
  int C, T;
};

// Prompt prefill: SSM + gate over T tokens per sequence (rows (b, t) at b * T + t), state in
// registers; the fields mean what they mean in SsmArgs, with z and the slots required.
struct ScanArgs {
  float* h;                  // (batch, H, P, N) fp32 state, advanced by T tokens
  const uint16_t* xbc;       // rows x | B | C (after the conv)
  int ld_xbc;
  const uint16_t* dt;        // raw dt rows
  int ld_dt;
  const uint16_t* z;         // gate input rows
  int ld_z;
  const float* dt_bias;
  const float* A_log;
  const float* D;
  uint16_t* y_out;           // (batch * T, ld_y) gated g
  int ld_y;
  double* sumsq_slots;       // (batch * T, n_slots) per-block sum(g^2)
  int n_slots;
  int H, P, N, T;
  int pb0;                   // set by the kernel
};

// Sampling head (sample.hip): one workgroup per sequence.
constexpr int kSampleMaxVocab = 65536;
struct SampleArgs {
  const uint16_t* logits;    // (M, V) fp16
  int* counts;               // (M, V) occurrences of each token so far; the drawn token is counted
  uint32_t* step;            // (M) draw counter of each sequence (RNG stream position), advanced
  int64_t* next;             // (M) drawn tokens
  float temperature, top_p, penalty;
  int mode;                  // 0: gen_test.py order, 1: training-script order (see sample.hip)
  uint64_t seed;
  int V;
  float* escratch;           // (M, 2, sample_row_floats(V)) workspace rows: the sums of the slice
                             // workgroups (maxima, normalizer, histograms, masses), then
                             // e = exp(z - max z)
};
// Floats per sampler scratch row: V rounded up to 4, at least 2560 (the sums take 9472 bytes).
__host__ __device__ inline int sample_row_floats(int V) {
  const int ld = (V + 3) / 4 * 4;
  return ld > 2560 ? ld : 2560;
}

struct HeadArgs {
  const uint16_t* x;         // (M, D) fp16 residual
  const float* norm_f;       // (D) fp32
  const uint8_t* emb;        // tiled table: int8 (f16 = 0) or fp16 (f16 = 1)
  const uint16_t* emb_scale; // (V) fp16 row scales of the int8 table
  int f16;
  int V, D;
  uint16_t* logits;          // (M, V) fp16 or null
  float* part_val;           // (M, n_groups)
  int* part_idx;             // (M, n_groups)
  unsigned* ticket;          // zero before the first launch; left zero by every launch
  int64_t* next;             // (M) greedy tokens
  uint16_t* x_next;          // optional (M, D): embedding of the greedy tokens
  const uint16_t* xf;        // batched head: (M, D) scratch for the final-normed rows
  const int8_t* hdig;        // int8 head at M >= 5: digit planes, head_digit_bytes(M, D) bytes
};

struct EmbedArgs {
  const int64_t* tokens;     // (M)
  const uint8_t* emb;        // tiled table: int8 (f16 = 0) or fp16 (f16 = 1)
  const uint16_t* emb_scale; // (V) for the int8 table
  int f16;
  uint16_t* x;               // (M, D)
  int* err_flag;             // set to 1 if a token is out of range
  int V, D;
  // tok_tc > 0: row m reads tokens[(m / tok_tc) * tok_ld + tok_t0 + m % tok_tc] (a window of
  // tok_tc tokens of every sequence of a row-major (batch, tok_ld) prompt); else tokens[m]
  int tok_ld, tok_t0, tok_tc;
};

// One whole layer for 1..4 sequences in a single launch (fused.hip).
struct FusedArgs {
  const uint32_t* in_bits; const uint16_t* in_ws; const int8_t* in_lA; const uint16_t* in_lAs;
  const uint16_t* in_lBq;    // (16, D) fp16(B_i8 * B_s)
  const uint32_t* out_bits; const uint16_t* out_ws; const int8_t* out_lA; const uint16_t* out_lAs;
  const uint16_t* out_lBq;   // (16, DI)
  const uint16_t* conv_w; const uint16_t* conv_b;
  const float* A_log; const float* Dp; const float* dt_bias;
  const float* norm_w; const float* ln_w;
  float* h;                  // (M, H, P, N) fp32 state of this layer
  uint16_t* conv;            // (M, C, 3) fp16 conv state of this layer
  uint16_t* x;               // (M, D) residual, updated in place
  // words exchanged between workgroups of a launch: (tag << 16) | fp16 bits, tag = the launch's
  // epoch mod 2^16
  uint32_t* projT;           // (M, IPO): gate z sigma(z) | conv'd xBC (dt rows unused)
  uint32_t* gT;              // kGRep copies (stride kGStride words) of (M, DI): gated SSM output, in gpos order
  uint32_t* hT;              // kXRep copies (stride kHStride words) of (2, M, 16): LoRA intermediates of
                             // in_proj / out_proj; consumer workgroup w polls copy w % kXRep
  uint32_t* bcT;             // kXRep copies (stride kBcStride words) of (M, 2 d_state): conv'd B | C
  uint64_t* dtT;             // (M, H, 2): softplus dt and exp(dt A) per head, (tag << 32) | fp32 bits
  uint32_t* launches;        // (G) launch count of each workgroup
  int* err;                  // error flags (DFSSM_ERR_WAIT_LAYER: a wait timed out)
  // the launch's layer: every launch takes the tag epoch * n_layer + layer + 1 (mod 2^16), so
  // that no word left by the previous launch carries a tag a poll waits for
  int layer, n_layer;
  int D, DI, N, H, P, IPO, C;
};

// Words that many workgroups poll (the LoRA intermediates, B | C) are written in kXRep copies at
// different addresses, so that their polls spread over memory channels instead of queueing on one
// cache line.
constexpr int kXRep = 8;
constexpr int kHStride = 1024;   // words between copies of hT (>= 2 * 4 * 16)
constexpr int kBcStride = 1088;  // words between copies of bcT (>= 4 * 256)
constexpr int kGRep = 8;                   // copies of the gated output words of the one-launch layer
constexpr int kGStride = 4 * 5120 + 1088;  // words between them (>= 4 * d_inner)
constexpr int kFusedMaxGroups = 256;  // in_proj row groups of 64
constexpr int kFusedMaxGrid = 1024;   // workgroups of the one-launch layer
bool fused_layer_supported(int M, int IPO, int D, int DI, int H, int P);
// Grid of the one-launch layer on a device with `cus` CUs where per_cu32 / per_cu64 workgroups of
// the 32- / 64-row-group instantiations fit per CU; 0 = use the five-kernel form. *rc_out = RC.
int fused_plan(int cus, int per_cu32, int per_cu64, int M, int IPO, int D, int DI, int H, int P, int* rc_out);
hipError_t launch_fused_layer(const FusedArgs& a, int M, hipStream_t s);
hipError_t launch_dequant_lora_b(const int8_t* B, const uint16_t* Bs, int K, uint16_t* out, hipStream_t s);

hipError_t launch_proj(const ProjArgs& a, int M, int mode, hipStream_t s);
hipError_t launch_prep(const PrepArgs& a, int M, int mode, hipStream_t s);
hipError_t launch_gemm(const GemmArgs& a, int mode, hipStream_t s);
// Prefill GEMM for thousands of rows (IN without conv, OUT): q in the wide tiled layout (rows
// padded to 16); expands the bits to w8 (gemm_wide_w8_bytes of scratch, tiled likewise) and runs
// a tiled MFMA GEMM with gemm_kernel's epilogue.
size_t gemm_wide_w8_bytes(int N, int K);
hipError_t launch_gemm_wide(const GemmArgs& a, int mode, int8_t* w8, hipStream_t s);
hipError_t launch_scaffold(const ScaffoldArgs& a, int M, hipStream_t s);
hipError_t launch_scaffold_xchg(const ScaffoldArgs& a, int M, hipStream_t s);  // a.ws set, M <= 4
hipError_t launch_tile_bits(const uint32_t* src, uint32_t* dst, int N, int KW, hipStream_t s);
hipError_t launch_ssm(const SsmArgs& a, int M, hipStream_t s);
hipError_t launch_conv(const ConvArgs& a, int M, hipStream_t s);
hipError_t launch_head(const HeadArgs& a, int M, hipStream_t s);
hipError_t launch_head_batched(const HeadArgs& a, int M, hipStream_t s);
size_t head_digit_bytes(int M, int D);  // HeadArgs::hdig size for the batched int8 head
hipError_t launch_embed(const EmbedArgs& a, int M, hipStream_t s);
hipError_t launch_sample(const SampleArgs& a, int batch, hipStream_t s);

// Density-field state quantization at a chunk boundary: rows of 128 fp32 values.
constexpr int kStateDfMaxKK = 1024;
struct StateDfArgs {
  float* h;                 // (rows, 128) state, quantized in place
  float* sd_error;          // (rows, 128) sigma-delta error, updated in place; null = none
  const float* thresholds;  // (kk) sorted thresholds of the bank
  long long rows;
  int kk, sd_bits;          // sd_bits >= 32: the error is kept unquantized
};
hipError_t launch_state_df(const StateDfArgs& a, hipStream_t s);
hipError_t launch_conv_seq(const ConvSeqArgs& a, int batch, hipStream_t s);
hipError_t launch_ssm_scan(const ScanArgs& a, int batch, hipStream_t s);
hipError_t launch_last_rows(const uint16_t* src, uint16_t* dst, int batch, int T, int D, hipStream_t s);
hipError_t launch_tile_emb(const uint8_t* src, uint8_t* dst, int V, int row_bytes, hipStream_t s);

}  // namespace dfssm
