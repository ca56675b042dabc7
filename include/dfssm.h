/*
 * dfssm.h -- C ABI of libdfssm_hip.so, the MI355X (gfx950) DF-SSM decode-step library.
 *
 * Conventions
 *  - Every pointer argument is a device pointer (HBM) owned by the caller, unless marked "host".
 *  - fp16 tensors are passed as uint16_t bit patterns; fp32 as float; row-major, C-contiguous
 *    unless a leading dimension (ld_*) is given, in elements.
 *  - Every call is asynchronous on `stream` (a hipStream_t; NULL = the null stream), never
 *    allocates device memory, never synchronizes, and is therefore capturable into a HIP graph.
 *  - Every function returns 0 on success, a negative DFSSM_E* code when argument validation
 *    fails (nothing is launched), or a positive hipError_t from the launch.
 *  - The library keeps no state between calls; concurrent calls are safe when they touch
 *    disjoint buffers or are ordered on one stream.
 *
 * Model-specific constraints (checked by dfssm_check_dims): d_state = 128, ngroups = 1,
 * LoRA rank 16, d_conv = 4, P = d_inner / nheads a multiple of 16, d_model and d_inner multiples
 * of 512 and at most 5120, nheads a multiple of 8, vocab_size at most 65536, batch 1..64.
 */
#ifndef DFSSM_H
#define DFSSM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DFSSM_ABI_VERSION 7

#define DFSSM_OK 0
#define DFSSM_E_NULL (-1)        /* a required pointer is NULL */
#define DFSSM_E_DIMS (-2)        /* model dimensions not supported by the kernels */
#define DFSSM_E_BATCH (-3)       /* batch size not supported */
#define DFSSM_E_ALIGN (-4)       /* pointer or leading dimension misaligned */
#define DFSSM_E_RANGE (-5)       /* index (layer, token count, size) out of range */
#define DFSSM_E_SCRATCH (-6)     /* the static workspace is too small for these dimensions */
#define DFSSM_E_CAPTURE (-7)     /* the call must not run under stream capture */

/* Bits of the workspace error flag (dfssm_workspace_error_flag), set by the kernels and left set
 * until the caller clears the flag. No counterpart in the reference (its gather raises a device
 * assert on a bad token id, and its kernels never wait on each other). */
#define DFSSM_ERR_TOKEN_RANGE 1          /* a token id outside [0, vocab) reached the embedding gather
                                            (row 0 was used) */
#define DFSSM_ERR_WAIT_LAYER 4           /* a bounded wait between workgroups of the one-launch layer
                                            (batch <= 4) timed out: that layer's output is wrong */
#define DFSSM_ERR_WAIT_SSM_PROLOGUE 8    /* a bounded wait of the SSM + out_proj-prologue launch
                                            (batch >= 5, DFSSM_PHASE_SSM_PROLOGUE) timed out */
#define DFSSM_ERR_WAIT_OUT_PROLOGUE 16   /* a bounded wait of the out_proj + next-prologue launch
                                            (batch >= 5, DFSSM_PHASE_OUT_PROLOGUE) timed out */

typedef struct dfssm_dims {
  int32_t n_layer, d_model, d_inner, d_state, nheads, headdim, ngroups, vocab_size;
  int32_t batch;     /* sequences decoded together */
  int32_t emb_code;  /* 0 = fp16 table (as the exporter writes it), 1 = int8 table + fp16 row scale */
} dfssm_dims;

/* Device pointers of one layer, in .dfssm order (training/export_dfssm.py:135-185). The sign bits
 * are in the tiled layout produced by dfssm_tile_bits; everything else is as stored in the file,
 * except the two norm weights, which are fp32 (fp16 files are widened at load), and the two
 * derived LoRA-B tables at the end, fp16(B_i8 * B_s) (16, K) from dfssm_dequant_lora_b -- the
 * load-time dequantization of df_ssm_inference.py:82-83,96-97. */
typedef struct dfssm_layer {
  const uint32_t* in_bits;   const uint16_t* in_scale;
  const int8_t* in_lA;       const uint16_t* in_lA_s;
  const int8_t* in_lB;       const uint16_t* in_lB_s;
  const uint32_t* out_bits;  const uint16_t* out_scale;
  const int8_t* out_lA;      const uint16_t* out_lA_s;
  const int8_t* out_lB;      const uint16_t* out_lB_s;
  const uint16_t* conv_w;    const uint16_t* conv_b;
  const float* A_log;        const float* D;          const float* dt_bias;
  const float* norm_w;       const float* ln_w;
  const uint16_t* in_lBq;    const uint16_t* out_lBq;
} dfssm_layer;

typedef struct dfssm_model {
  dfssm_dims dims;
  const dfssm_layer* layers;     /* HOST array of n_layer descriptors (device pointers inside) */
  const void* emb;               /* table (int8 or fp16) in the tiled layout of dfssm_tile_embedding */
  const uint16_t* emb_scale;     /* (V) fp16 row scales of an int8 table; NULL for an fp16 table */
  const float* norm_f;           /* (D) fp32 */
} dfssm_model;

typedef struct dfssm_state {
  float* h;                      /* (n_layer, batch, nheads, P, d_state) fp32 SSM state */
  uint16_t* conv;                /* (n_layer, batch, d_xbc, 3) fp16 conv shift register */
} dfssm_state;

/* ---- library ---------------------------------------------------------------------------- */
int dfssm_version(void);
const char* dfssm_error_string(int code);
/* 0 if the kernels support `dims`, else DFSSM_E_DIMS / DFSSM_E_BATCH. */
int dfssm_check_dims(const dfssm_dims* dims);

/* Workgroups of the one-launch layer (batch <= 4) on a device with `cus` compute units where
 * `blocks_per_cu` of its 1024-thread workgroups fit at once, or 0 when a layer runs as five
 * kernels instead. The one-launch layer waits between its workgroups, so it is used only when all
 * of them are resident together (one per CU, blocks_per_cu >= 1 for the instantiation launched).
 * dfssm_layer_step makes this decision with the current device's values; exposed so that the
 * rule can be checked without a GPU. No counterpart in the reference (its layers are separate
 * kernel launches, df_ssm_inference.py:161-207). */
int dfssm_one_launch_plan(const dfssm_dims* dims, int cus, int blocks_per_cu);
/* Layer kernel selection for dfssm_layer_step / dfssm_decode_step (process-wide; returns the
 * previous setting, or DFSSM_E_RANGE). At batch <= 4, DFSSM_LAYER_AUTO (default) and
 * DFSSM_LAYER_FUSED run the one-launch layer where the device and the shape allow it, else five
 * kernels; DFSSM_LAYER_FIVE always runs five kernels per layer (and the five phases at batch >= 5).
 * All give bit-identical results; the setting exists to compare them. No counterpart in the
 * reference. */
#define DFSSM_LAYER_AUTO 0
#define DFSSM_LAYER_FUSED 1
#define DFSSM_LAYER_FIVE 2
int dfssm_set_layer_kernel(int which);

/* ---- load-time layout ------------------------------------------------------------------ */
/* Bytes of the tiled copy of a (rows, k/32) sign-bit matrix / of a (vocab, row_bytes) table
 * (row_bytes = d_model for int8, 2 * d_model for fp16). */
size_t dfssm_tiled_bits_bytes(int rows, int k);
size_t dfssm_tiled_emb_bytes(int vocab, int row_bytes);
/* Re-tile row-major packed sign bits (the .dfssm int32 words, export_dfssm.py:34-42) for the
 * scaffold kernels. Replaces the load-time unpack of df_ssm_inference.py:23-29,70-74: the copy
 * stays 1 bit per weight. k must be a multiple of 512. */
int dfssm_tile_bits(const uint32_t* src, uint32_t* dst, int rows, int k, void* stream);
/* LoRA-B dequantization at load: out[r][k] = fp16(B[r][k] * Bs[r]) for r < 16, k < K
 * (df_ssm_inference.py:82-83,96-97: B_deq = (B_i8.float() * B_s.float()).half()). */
int dfssm_dequant_lora_b(const int8_t* B, const uint16_t* Bs, int K, uint16_t* out, void* stream);
/* Re-tile the row-major embedding table (V rows of row_bytes bytes: int8 or fp16 values) for the
 * gather and the tied head (replaces the fp16 table kept by df_ssm_inference.py:63-64). */
int dfssm_tile_embedding(const void* src, void* dst, int vocab, int row_bytes, void* stream);

/* ---- single operators ------------------------------------------------------------------ */
/* Scaffold GEMM: acc[m][n] = sum_k q[m][k] * (bit ? +1 : -1) (exact int32) and, if y_out is
 * non-NULL, y = fp16(fp16(fp16(acc) * xscale[m]) * wscale[n]). Replaces torch._int_mm plus the
 * dequant of _scaffold_matmul, df_ssm_inference.py:154-158. M = 1..64 (1..4 on the packed-bit
 * VALU GEMV, 5..64 on the int8 matrix cores). */
int dfssm_scaffold_gemm(const uint32_t* tiled_bits, const int8_t* q, const uint16_t* xscale,
                        const uint16_t* wscale, int M, int N, int K, int32_t* acc_out,
                        uint16_t* y_out, void* stream);

/* Scaffold projection with its rank-16 LoRA correction (one projection of a layer, as an
 * operator): acc as dfssm_scaffold_gemm (exact int32, written if acc_out is non-NULL),
 *   lora_h[m][r] = fp16(sum_k xn[m][k] * lBq[r][k])                       (x_norm @ lora_B.T)
 *   y[m][n] = fp16(fp32(sum_r lora_h[m][r] * fp16(lA[n][r] * lA_s[n])) + fp16(fp16(fp16(acc) *
 *             xscale[m]) * wscale[n]))                                   (proj.addmm_(..., lora_A.T))
 * with the sums over exactly representable products in fp64. Replaces _scaffold_matmul plus the
 * LoRA addmm_ of df_ssm_inference.py:154-158,169-173 (in_proj) and :199-204 (out_proj). xn (M, K)
 * fp16 are the normalized activations the LoRA reads (q their int8 quantization with scales
 * xscale); lBq (16, K) is the load-time fp16 LoRA-B table (dfssm_dequant_lora_b); lA (N, 16) int8
 * and lA_s (N) fp16 as stored in the file. lora_h (M, 16) fp16 receives the intermediates.
 * M = 1..64 (1..4 on the packed-bit VALU GEMV, 5..64 on the int8 matrix cores).
 * workspace (no counterpart in the reference; NULL allowed): DFSSM_SCAFFOLD_WORKSPACE_BYTES of
 * device memory, 16-byte aligned and zeroed once before its first use. With it, M <= 4, M K <=
 * 8192 and N <= 15 360 run as one launch in which 16 workgroups compute the intermediates once and
 * hand them to the GEMV workgroups through the workspace (the same results as without it). Calls that share a
 * workspace must not overlap. The word at byte offset DFSSM_SCAFFOLD_ERROR_OFFSET is non-zero
 * after a call whose wait for the intermediates timed out (its y is then wrong); it stays set
 * until the caller clears it. */
#define DFSSM_SCAFFOLD_WORKSPACE_BYTES (64u << 10)
#define DFSSM_SCAFFOLD_ERROR_OFFSET 1024u
int dfssm_scaffold_lora_gemm(const uint32_t* tiled_bits, const uint16_t* wscale, const int8_t* q,
                             const uint16_t* xscale, const uint16_t* xn, const int8_t* lA, const uint16_t* lA_s,
                             const uint16_t* lBq, int M, int N, int K, uint16_t* lora_h, int32_t* acc_out,
                             uint16_t* y_out, void* workspace, void* stream);

/* RMSNorm + int8 quantization of M rows (the prologue of every projection):
 * xn = fp16((x * r) * w), q = int8 activations, s = fp16 scales.
 * Replaces _rms_norm + _quantize_to_int8, df_ssm_inference.py:141-152. */
int dfssm_rmsnorm_quantize(const uint16_t* x, const float* w, int M, int K, uint16_t* xn_out,
                           int8_t* q_out, uint16_t* s_out, void* stream);

/* conv1d shift-register step + SiLU, in place on xbc (rows of stride ld_xbc) and conv_state
 * (batch, channels, 3). Replaces df_ssm_kernels.conv_step (df_ssm_kernels.cu:109-125). */
int dfssm_conv_step(uint16_t* conv_state, uint16_t* xbc, int ld_xbc, const uint16_t* conv_w,
                    const uint16_t* conv_b, int batch, int channels, void* stream);

/* Mamba-2 SSM step with an fp32 state h (batch, nheads, headdim, d_state). xbc rows hold
 * x | B | C (after the conv), dt rows the raw dt. Writes y (batch, ld_y). Replaces
 * df_ssm_kernels.ssm_step (df_ssm_kernels.cu:127-151); the reference's fp16 state becomes fp32
 * and the caller need not zero y. */
int dfssm_ssm_step(float* h_state, const uint16_t* xbc, int ld_xbc, const uint16_t* dt, int ld_dt,
                   const float* dt_bias, const float* A_log, const float* D, uint16_t* y_out,
                   int ld_y, int batch, int nheads, int headdim, int d_state, void* stream);

/* ---- decode ----------------------------------------------------------------------------- */
/* Workspace for the layer/decode calls; init zeroes what must start at zero (once, before use). */
size_t dfssm_workspace_bytes(const dfssm_dims* dims);
int dfssm_workspace_init(const dfssm_dims* dims, void* workspace, void* stream);

/* x = embedding(tokens): x (batch, D) fp16. Out-of-range tokens read row 0 and set the
 * workspace error flag (dfssm_workspace_error_flag). Replaces df_ssm_inference.py:220. */
int dfssm_embed(const dfssm_model* model, const int64_t* tokens, uint16_t* x, void* workspace,
                void* stream);
/* Device address of the int error flag inside the workspace. */
int* dfssm_workspace_error_flag(const dfssm_dims* dims, void* workspace);

/* One residual block on x (batch, D) fp16, in place: RMSNorm, in_proj scaffold + LoRA, conv,
 * SSM, gate, gated RMSNorm, out_proj scaffold + LoRA, residual. Replaces one iteration of
 * _run_layers, df_ssm_inference.py:161-207. One launch at batch <= 4 (see
 * dfssm_set_layer_kernel); at batch >= 5 four (phases 0, 1, DFSSM_PHASE_SSM_PROLOGUE, 4);
 * with DFSSM_LAYER_FIVE the five phases below. */
int dfssm_layer_step(const dfssm_model* model, int layer, uint16_t* x, const dfssm_state* state,
                     void* workspace, void* stream);

/* One of the kernels of dfssm_layer_step, in order: 0 = RMSNorm + int8 quantization + LoRA
 * intermediate of x (df_ssm_inference.py:165-168,173), 1 = in_proj scaffold + LoRA + conv/SiLU
 * (:169-182), 2 = SSM step + gate (:185-195), 3 = gated RMSNorm + quantization + LoRA
 * intermediate (:196-199,204), 4 = out_proj scaffold + LoRA + residual (:200-207). Running the
 * phases in order equals dfssm_layer_step; exposed for per-kernel timing. */
#define DFSSM_LAYER_PHASES 5
/* Two more values of `phase`, the fused launches of the decode step at batch >= 5 (no counterpart
 * in the reference; exposed for per-launch timing): DFSSM_PHASE_SSM_PROLOGUE = phases 2 and 3 in
 * one launch; DFSSM_PHASE_OUT_PROLOGUE = phase 4 of `layer` and phase 0 of layer + 1 in one
 * launch (layer + 1 < n_layer). Both return DFSSM_E_DIMS, launching nothing, for a batch or shape
 * they do not take (batch <= 4; the second also where the out_proj grid fills whole rounds of the
 * CUs, which dfssm_decode_step then runs as two launches). */
#define DFSSM_PHASE_SSM_PROLOGUE 5
#define DFSSM_PHASE_OUT_PROLOGUE 6
int dfssm_layer_phase(const dfssm_model* model, int layer, int phase, uint16_t* x,
                      const dfssm_state* state, void* workspace, void* stream);

/* Final RMSNorm, tied int8 head and greedy argmax: logits (batch, V) fp16 (may be NULL),
 * next (batch) int64. If x_next is non-NULL the embedding of `next` is written there (it may
 * alias x). Replaces df_ssm_inference.py:210,224,236. */
int dfssm_lmhead_argmax(const dfssm_model* model, const uint16_t* x, void* workspace,
                        uint16_t* logits, int64_t* next, uint16_t* x_next, void* stream);

/* One whole decode step: if tokens != NULL, x = embedding(tokens) first; then every layer,
 * then the head. With fuse_next_embed != 0, x receives the embedding of the greedy tokens, so
 * the following step can pass tokens = NULL. Replaces forward() + argmax,
 * df_ssm_inference.py:219-224,236. At batch >= 5 a layer is three launches (in_proj,
 * DFSSM_PHASE_SSM_PROLOGUE, DFSSM_PHASE_OUT_PROLOGUE) where the shape takes them. */
int dfssm_decode_step(const dfssm_model* model, const int64_t* tokens, uint16_t* x,
                      const dfssm_state* state, void* workspace, uint16_t* logits, int64_t* next,
                      int fuse_next_embed, void* stream);

/* ---- decode step without a workspace argument (allocates nothing) ----------------------- */
/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): dfssm_decode_step with
 * its workspace in a library-owned static device array of DFSSM_STATIC_WORKSPACE_BYTES, which
 * each GPU the library runs on holds until the process ends. Dimensions whose
 * dfssm_workspace_bytes exceeds it are rejected with DFSSM_E_SCRATCH (24 MiB covers batch <= 32
 * at the 1.3B and 2.7B shapes). All calls on one GPU share that GPU's array: calls that overlap
 * on one GPU (other streams, other threads) race; calls ordered on one stream do not. The first
 * call on a device, and the first after the dimensions change, clears the array's counters with a
 * fill kernel on `stream` and must not be captured (else DFSSM_E_CAPTURE); later calls may be.
 * error_out (device int, may be NULL) receives the workspace error flag of this call (the
 * DFSSM_ERR_* bits), which is then cleared; this also happens when the step fails after queueing
 * some of its kernels, once the static workspace is set up. Every other argument is as in
 * dfssm_decode_step. */
#define DFSSM_STATIC_WORKSPACE_BYTES (24u << 20)
int dfssm_decode_step_static(const dfssm_model* model, const int64_t* tokens, uint16_t* x,
                             const dfssm_state* state, uint16_t* logits, int64_t* next, int fuse_next_embed,
                             int* error_out, void* stream);

/* ---- sampling ------------------------------------------------------------------------ */
typedef struct dfssm_sample_params {
  float temperature;   /* > 0 */
  float top_p;         /* >= 0; >= 1 keeps every token, 0 only the most probable */
  float penalty;       /* repetition penalty r > 0 (1 = none) */
  int32_t mode;        /* 0: z = logit / T, then / r if the token occurred (eval/gen_test.py:71-74);
                          1: per occurrence logit > 0 ? / r : * r, then / T
                          (training/df_ssm_mamba2_distill_dfw.py:1069-1073) */
  uint64_t seed;
} dfssm_sample_params;

/* Draw the next token of every sequence from fp16 logits (batch, V) with temperature, repetition
 * penalty and top-p, as eval/gen_test.py:54-95 and training/df_ssm_mamba2_distill_dfw.py:
 * 1066-1078 do with torch.sort / cumsum / multinomial. The top-p set is the reference's rule
 * (a token stays while the probability mass ranked above it is <= top_p) on exact fixed-point
 * masses E = floor(exp(z - max) 2^40); the draw is by inverse CDF over the kept tokens in index
 * order, at R = floor(h S / 2^64) (S the kept mass, h = splitmix64 of seed, sequence and step[b]),
 * deterministic for a given seed (torch's generator is not reproduced).
 * counts (batch, V) int32 holds each token's occurrences so far (the caller counts the prompt);
 * the drawn token is added, and step (batch) advances. next (batch) receives the tokens; if
 * x_next is non-NULL it receives their embedding (as dfssm_embed). workspace: the decode
 * workspace (scratch for the draw and the error flag). V <= 65536. */
int dfssm_sample(const dfssm_model* model, const uint16_t* logits, int32_t* counts, uint32_t* step,
                 const dfssm_sample_params* params, int64_t* next, uint16_t* x_next, void* workspace,
                 void* stream);

/* ---- prompt prefill ------------------------------------------------------------------- */
/* Workspace of dfssm_prefill for chunks of up to max_rows = batch x tokens-per-chunk rows
 * (batch <= max_rows <= 32768); 0 if the arguments are not supported. */
size_t dfssm_prefill_workspace_bytes(const dfssm_dims* dims, int max_rows);

/* Ingest a prompt of n_tokens tokens per sequence, tokens (batch, n_tokens) int64 row-major: the
 * result -- state, logits, next and x -- is bit-for-bit that of n_tokens dfssm_decode_step calls
 * with tokens[:, t] (the reference ingests prompts token by token, cpu_inference_driver.py:
 * 186-204; its GPU generate() has no prompt, df_ssm_inference.py:226-243). Layer-major: the
 * prompt rows of all sequences go through a layer together (prologues and scaffold GEMMs over
 * batch x n_tokens rows on the int8 matrix cores), the conv and the SSM recurrence walk the
 * tokens with their state in registers, so weights and state are read once per layer and chunk
 * instead of once per token. The prompt is processed in chunks of max_rows / batch tokens;
 * prefill_workspace holds dfssm_prefill_workspace_bytes(dims, max_rows) bytes, workspace is the
 * decode workspace (the head and the error flag). logits (batch, V) may be NULL; x receives the
 * embedding of `next` if fuse_next_embed, else the last token's residual row. */
int dfssm_prefill(const dfssm_model* model, const int64_t* tokens, int n_tokens, uint16_t* x,
                  const dfssm_state* state, void* workspace, void* prefill_workspace, int max_rows,
                  uint16_t* logits, int64_t* next, int fuse_next_embed, void* stream);

/* ---- density-field state (row f4) ------------------------------------------------------- */
/* Quantize SSM state rows at a chunk boundary as training/df_ssm_mamba2_distill_dfw.py:139-165
 * (df_ssd_scan) does after every block_len tokens. The reference applies it in training only.
 * Per row of d_state = 128 fp32 values:
 *   mean and unbiased std (clamped to 1e-8), lo = mean - 3 std, range = max(6 std, 1e-8),
 *   hs = clamp((h - lo) / range, 0, 1), hc = clamp(hs + e, 0, 1) (e = sd_error, if given),
 *   q = (number of thresholds[0..kk) below hc) / kk  (SprayBank.quantize, :88-91),
 *   e = round(clamp(hc - q, -1, 1) 2^(sd_bits-1)) / 2^(sd_bits-1)  (_quantize_error, :105-110;
 *       unquantized for sd_bits >= 32),
 *   h = q range + lo.
 * h and sd_error are (rows, 128), 16-byte aligned, updated in place; sd_error NULL = no sigma-delta.
 * thresholds: the kk sorted thresholds of the bank for this chunk (bank = chunk % num_banks),
 * 1 <= kk <= 1024. Both row sums are fp64 over a fixed adjacent-pair tree, so results are
 * deterministic. */
int dfssm_state_density_field(float* h, float* sd_error, int64_t rows, int d_state,
                              const float* thresholds, int kk, int sd_bits, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DFSSM_H */
