// C ABI of libdfssm_hip.so: argument validation, workspace layout and launch sequencing.
// Declarations and conventions: include/dfssm.h.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <mutex>

#include "dfssm.h"
#include "dfssm_kernels.h"

using namespace dfssm;

namespace {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

struct Derived {
  int B, L, D, DI, N, H, P, V, IPO, C, n_slots, head_groups;
};

Derived derive(const dfssm_dims* d) {
  Derived r;
  r.B = d->batch; r.L = d->n_layer; r.D = d->d_model; r.DI = d->d_inner; r.N = d->d_state;
  r.H = d->nheads; r.P = d->nheads > 0 ? d->d_inner / d->nheads : 0; r.V = d->vocab_size;
  r.C = r.DI + 2 * d->ngroups * r.N;
  r.IPO = 2 * r.DI + 2 * d->ngroups * r.N + r.H;
  r.n_slots = r.P > 0 ? r.H * (r.P / 16) : 0;
  r.head_groups = (r.V + 63) / 64;
  return r;
}

struct WsLayout {
  size_t proj, g, slots, q, planes, qsum, xs, h, xf, part_val, part_idx, hdig, samp, ticket, err, launches,
      proj_t, g_t, h_t, dt_t, bc_t, g_s, launches_s, x_s, launches_o, total;
};

WsLayout ws_layout(const dfssm_dims* d) {
  const Derived r = derive(d);
  WsLayout w;
  size_t off = 0;
  w.proj = off;     off = align_up(off + (size_t)r.B * r.IPO * 2);
  w.g = off;        off = align_up(off + (size_t)r.B * r.DI * 2);
  w.slots = off;    off = align_up(off + (size_t)r.B * r.n_slots * 8);
  const int kq = r.D > r.DI ? r.D : r.DI;  // row stride of the prep buffers
  w.q = off;        off = align_up(off + (size_t)r.B * kq);
  w.planes = off;   off = align_up(off + (size_t)r.B * kq);
  w.qsum = off;     off = align_up(off + (size_t)r.B * 4);
  w.xs = off;       off = align_up(off + (size_t)r.B * 4);
  w.h = off;        off = align_up(off + (size_t)r.B * 16 * 4);
  w.xf = off;       off = align_up(off + (size_t)r.B * r.D * 2);
  w.part_val = off; off = align_up(off + (size_t)r.B * r.head_groups * 4);
  w.part_idx = off; off = align_up(off + (size_t)r.B * r.head_groups * 4);
  w.hdig = off;     off = align_up(off + (r.B > 4 ? head_digit_bytes(r.B, r.D) : 0));  // batched int8 head
  w.samp = off;     off = align_up(off + (size_t)r.B * 2 * sample_row_floats(r.V) * 4);  // sampler rows
  w.ticket = off;   off = align_up(off + 4);
  w.err = off;      off = align_up(off + 4);
  // one-launch layer: per-workgroup launch counts and the tagged exchange words (zeroed by
  // dfssm_workspace_init together with the head's ticket and the error flag)
  w.launches = off; off = align_up(off + (size_t)kFusedMaxGrid * 4);
  w.proj_t = off;   off = align_up(off + (size_t)r.B * r.IPO * 4);
  w.g_t = off;      off = align_up(off + (size_t)kGRep * kGStride * 4);
  w.h_t = off;      off = align_up(off + (size_t)kXRep * kHStride * 4);
  w.dt_t = off;     off = align_up(off + 2 * (size_t)r.B * r.H * 8);
  w.bc_t = off;     off = align_up(off + (size_t)kXRep * kBcStride * 4);
  // batch >= 5: the SSM + gated-norm prologue launch's tagged g words and launch counts
  w.g_s = off;      off = align_up(off + (size_t)r.B * r.DI * 4);
  w.launches_s = off; off = align_up(off + (size_t)(r.DI / 16 + 16) * r.B * 4);  // 16 LoRA ranks
  // batch >= 5: the out_proj launch with the next layer's prologue, its tagged x words and counts
  w.x_s = off;      off = align_up(off + (size_t)r.B * r.D * 4);
  w.launches_o = off; off = align_up(off + (size_t)kGemmProMaxWg * 4);
  w.total = off;
  return w;
}

// Prompt prefill workspace for up to `rows` = batch x tokens-per-chunk activation rows: the
// residual stream of every row, the projection rows, g, the sum(g^2) slots and the prologue
// outputs (q, scale, LoRA intermediate).
struct PfLayout {
  size_t x, proj, g, slots, q, xs, h, w8, total;
};
// Prefill chunks of at least this many rows run the projections on the wide GEMM (weights
// expanded to int8 in the prefill workspace), smaller ones on gemm_kernel.
constexpr int kWideGemmRows = 256;

PfLayout pf_layout(const Derived& r, int rows) {
  PfLayout w;
  size_t off = 0;
  const int kq = r.D > r.DI ? r.D : r.DI;
  w.x = off;     off = align_up(off + (size_t)rows * r.D * 2);
  w.proj = off;  off = align_up(off + (size_t)rows * r.IPO * 2);
  w.g = off;     off = align_up(off + (size_t)rows * r.DI * 2);
  w.slots = off; off = align_up(off + (size_t)rows * r.n_slots * 8);
  w.q = off;     off = align_up(off + (size_t)(rows + 15) / 16 * 16 * kq);  // rows padded to 16 (tiled)
  w.xs = off;    off = align_up(off + (size_t)rows * 4);
  w.h = off;     off = align_up(off + (size_t)rows * 16 * 4);
  w.w8 = off;
  if (rows >= kWideGemmRows) {  // the larger projection's expanded weights
    const size_t a = gemm_wide_w8_bytes(r.IPO, r.D), b = gemm_wide_w8_bytes(r.D, r.DI);
    off = align_up(off + (a > b ? a : b));
  }
  w.total = off;
  return w;
}

inline int hip_status(hipError_t e) { return e == hipSuccess ? DFSSM_OK : (int)e; }

// Which layer kernel dfssm_layer_step uses (dfssm_set_layer_kernel). DFSSM_LAYER_AUTO and
// DFSSM_LAYER_FUSED run the one-launch layer at batch <= 4 where the device and shape take it.
int g_layer_kernel = DFSSM_LAYER_AUTO;

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

bool kdim_ok(int k) { return k > 0 && k % 512 == 0 && k <= 5120; }

__global__ void zero_u32_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace

extern "C" {

int dfssm_version(void) { return DFSSM_ABI_VERSION; }

const char* dfssm_error_string(int code) {
  switch (code) {
    case DFSSM_OK: return "ok";
    case DFSSM_E_NULL: return "required pointer is NULL";
    case DFSSM_E_DIMS: return "model dimensions not supported by the kernels";
    case DFSSM_E_BATCH: return "batch size not supported (1..64)";
    case DFSSM_E_ALIGN: return "pointer or leading dimension misaligned (16-byte rows required)";
    case DFSSM_E_RANGE: return "index out of range";
    case DFSSM_E_SCRATCH:
      return "the decode workspace of these dimensions exceeds the static workspace (DFSSM_STATIC_WORKSPACE_BYTES)";
    case DFSSM_E_CAPTURE:
      return "the first call for these dimensions on a device must not be captured (it clears the static workspace)";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

int dfssm_check_dims(const dfssm_dims* d) {
  if (!d) return DFSSM_E_NULL;
  if (d->n_layer <= 0 || d->vocab_size <= 0 || d->vocab_size > 65536 || d->nheads <= 0) return DFSSM_E_DIMS;
  if (!kdim_ok(d->d_model) || !kdim_ok(d->d_inner)) return DFSSM_E_DIMS;
  if (d->d_state != 128 || d->ngroups != 1 || (d->emb_code != 0 && d->emb_code != 1)) return DFSSM_E_DIMS;
  if (d->d_inner % d->nheads) return DFSSM_E_DIMS;
  const int P = d->d_inner / d->nheads;
  if (P % 16 || d->nheads % 8) return DFSSM_E_DIMS;
  if (d->batch < 1 || d->batch > 64) return DFSSM_E_BATCH;
  return DFSSM_OK;
}

int dfssm_one_launch_plan(const dfssm_dims* d, int cus, int blocks_per_cu) {
  if (!d || dfssm_check_dims(d) != DFSSM_OK) return 0;
  const Derived r = derive(d);
  return fused_plan(cus, blocks_per_cu, blocks_per_cu, r.B, r.IPO, r.D, r.DI, r.H, r.P, nullptr);
}

int dfssm_set_layer_kernel(int which) {
  if (which != DFSSM_LAYER_AUTO && which != DFSSM_LAYER_FUSED && which != DFSSM_LAYER_FIVE)
    return DFSSM_E_RANGE;
  const int prev = g_layer_kernel;
  g_layer_kernel = which;
  return prev;
}

size_t dfssm_tiled_bits_bytes(int rows, int k) {
  if (rows <= 0 || k <= 0) return 0;
  return (size_t)((rows + 63) / 64 * 64) * (size_t)(k / 32) * 4;
}

size_t dfssm_tiled_emb_bytes(int vocab, int row_bytes) {
  if (vocab <= 0 || row_bytes <= 0) return 0;
  return (size_t)((vocab + 63) / 64 * 64) * (size_t)row_bytes;
}

int dfssm_tile_bits(const uint32_t* src, uint32_t* dst, int rows, int k, void* stream) {
  if (!src || !dst) return DFSSM_E_NULL;
  if (rows <= 0 || !kdim_ok(k)) return DFSSM_E_DIMS;
  return hip_status(launch_tile_bits(src, dst, rows, k / 32, as_stream(stream)));
}

int dfssm_dequant_lora_b(const int8_t* B, const uint16_t* Bs, int K, uint16_t* out, void* stream) {
  if (!B || !Bs || !out) return DFSSM_E_NULL;
  if (K <= 0) return DFSSM_E_DIMS;
  return hip_status(launch_dequant_lora_b(B, Bs, K, out, as_stream(stream)));
}

int dfssm_tile_embedding(const void* src, void* dst, int vocab, int row_bytes, void* stream) {
  if (!src || !dst) return DFSSM_E_NULL;
  if (vocab <= 0 || row_bytes <= 0 || row_bytes % 64) return DFSSM_E_DIMS;
  if (((uintptr_t)src & 3u) || !aligned16(dst)) return DFSSM_E_ALIGN;
  return hip_status(launch_tile_emb((const uint8_t*)src, (uint8_t*)dst, vocab, row_bytes, as_stream(stream)));
}

// The stand-alone scaffold op runs the bit-plane GEMV (N / 64 workgroups) only with at least this
// many output rows; with fewer, the matrix-core GEMM (N / 16 workgroups) measured faster.
constexpr int kScaffoldGemvMinN = 4096;

int dfssm_scaffold_gemm(const uint32_t* tiled_bits, const int8_t* q, const uint16_t* xscale,
                        const uint16_t* wscale, int M, int N, int K, int32_t* acc_out,
                        uint16_t* y_out, void* stream) {
  if (!tiled_bits || !q || (!acc_out && !y_out)) return DFSSM_E_NULL;
  if (y_out && (!xscale || !wscale)) return DFSSM_E_NULL;
  if (M < 1 || M > 64) return DFSSM_E_BATCH;
  if (N <= 0 || !kdim_ok(K)) return DFSSM_E_DIMS;
  if (!aligned16(tiled_bits) || !aligned16(q)) return DFSSM_E_ALIGN;
  if (M <= 4 && N >= kScaffoldGemvMinN) {
    ScaffoldArgs a{tiled_bits, q, xscale, wscale, acc_out, y_out, nullptr, nullptr, nullptr, N, K};
    return hip_status(launch_scaffold(a, M, as_stream(stream)));
  }
  GemmArgs a{};
  a.bits = tiled_bits; a.wscale = y_out ? wscale : nullptr;
  a.q = q; a.ld_q = K; a.M = M;
  a.xs16 = xscale;
  a.out = y_out; a.ld_out = N; a.acc_out = acc_out;
  a.N = N; a.K = K;
  return hip_status(launch_gemm(a, DFSSM_MODE_SCAFFOLD, as_stream(stream)));
}

int dfssm_scaffold_lora_gemm(const uint32_t* tiled_bits, const uint16_t* wscale, const int8_t* q,
                             const uint16_t* xscale, const uint16_t* xn, const int8_t* lA, const uint16_t* lA_s,
                             const uint16_t* lBq, int M, int N, int K, uint16_t* lora_h, int32_t* acc_out,
                             uint16_t* y_out, void* workspace, void* stream) {
  if (!tiled_bits || !wscale || !q || !xscale || !xn || !lA || !lA_s || !lBq || !lora_h || !y_out)
    return DFSSM_E_NULL;
  if (M < 1 || M > 64) return DFSSM_E_BATCH;
  if (N <= 0 || !kdim_ok(K)) return DFSSM_E_DIMS;
  if (!aligned16(tiled_bits) || !aligned16(q) || !aligned16(xn) || !aligned16(lBq) || !aligned16(lA) ||
      !aligned16(workspace))
    return DFSSM_E_ALIGN;
  hipStream_t s = as_stream(stream);
  // one launch: rank workgroups compute the intermediates once and hand them over. Its GEMV runs on
  // the VALU, M K values per workgroup: at M K > 8192 (out_proj K = 4096 at M = 4: 10.8 us per call
  // against 8.5) the matrix-core GEMM below is faster.
  if (workspace && M <= 4 && M * K <= 8192 && (N + 63) / 64 <= kScafMaxGroups) {
    ScaffoldArgs a{tiled_bits, q, xscale, wscale, acc_out, y_out, lA, lA_s, nullptr, N, K, xn, lBq, lora_h,
                   (uint32_t*)workspace};
    return hip_status(launch_scaffold_xchg(a, M, s));
  }
  if (M == 1 && N >= kScaffoldGemvMinN) {  // one launch, the GEMV's workgroups compute the intermediates
    ScaffoldArgs a{tiled_bits, q, xscale, wscale, acc_out, y_out, lA, lA_s, nullptr, N, K, xn, lBq, lora_h};
    return hip_status(launch_scaffold(a, M, s));
  }
  // otherwise the intermediates once (lora_h_kernel), then the matrix-core GEMM
  LoraHArgs la{xn, lBq, lora_h, K};
  hipError_t e = launch_lora_h(la, M, s);
  if (e != hipSuccess) return hip_status(e);
  GemmArgs a{};
  a.bits = tiled_bits; a.wscale = wscale;
  a.q = q; a.ld_q = K; a.M = M;
  a.xs16 = xscale;
  a.lA = lA; a.lAs = lA_s; a.h16 = lora_h;
  a.out = y_out; a.ld_out = N; a.acc_out = acc_out;
  a.N = N; a.K = K;
  return hip_status(launch_gemm(a, DFSSM_MODE_SCAFFOLD, s));
}

int dfssm_rmsnorm_quantize(const uint16_t* x, const float* w, int M, int K, uint16_t* xn_out,
                           int8_t* q_out, uint16_t* s_out, void* stream) {
  if (!x || !w || !xn_out || !q_out || !s_out) return DFSSM_E_NULL;
  if (M < 1 || !kdim_ok(K)) return DFSSM_E_DIMS;
  PrepArgs a{};
  a.act = x; a.ld_act = K; a.norm_w = w;
  a.q_out = q_out; a.ld_q = K;
  a.xn_out = xn_out; a.xs16_out = s_out;
  a.K = K;
  return hip_status(launch_prep(a, M, DFSSM_MODE_IN, as_stream(stream)));
}

int dfssm_conv_step(uint16_t* conv_state, uint16_t* xbc, int ld_xbc, const uint16_t* conv_w,
                    const uint16_t* conv_b, int batch, int channels, void* stream) {
  if (!conv_state || !xbc || !conv_w || !conv_b) return DFSSM_E_NULL;
  if (batch < 1 || channels < 1 || ld_xbc < channels) return DFSSM_E_DIMS;
  ConvArgs a{conv_state, xbc, conv_w, conv_b, ld_xbc, channels};
  return hip_status(launch_conv(a, batch, as_stream(stream)));
}

int dfssm_ssm_step(float* h_state, const uint16_t* xbc, int ld_xbc, const uint16_t* dt, int ld_dt,
                   const float* dt_bias, const float* A_log, const float* D, uint16_t* y_out,
                   int ld_y, int batch, int nheads, int headdim, int d_state, void* stream) {
  if (!h_state || !xbc || !dt || !dt_bias || !A_log || !D || !y_out) return DFSSM_E_NULL;
  if (batch < 1 || nheads < 1 || headdim < 16 || headdim % 16 || d_state != 128) return DFSSM_E_DIMS;
  const int DI = nheads * headdim;
  if (ld_xbc < DI + 2 * d_state || ld_dt < nheads || ld_y < DI) return DFSSM_E_DIMS;
  if (!aligned16(h_state) || !aligned16(xbc) || (ld_xbc % 8) || (DI % 8)) return DFSSM_E_ALIGN;
  SsmArgs a{};
  a.h = h_state;
  a.xbc = xbc; a.ld_xbc = ld_xbc;
  a.dt = dt; a.ld_dt = ld_dt;
  a.z = nullptr; a.ld_z = 0;
  a.dt_bias = dt_bias; a.A_log = A_log; a.D = D;
  a.y_out = y_out; a.ld_y = ld_y;
  a.sumsq_slots = nullptr; a.n_slots = 0;
  a.H = nheads; a.P = headdim; a.N = d_state;
  return hip_status(launch_ssm(a, batch, as_stream(stream)));
}

size_t dfssm_workspace_bytes(const dfssm_dims* dims) {
  if (!dims || dfssm_check_dims(dims) != DFSSM_OK) return 0;
  return ws_layout(dims).total;
}

int dfssm_workspace_init(const dfssm_dims* dims, void* workspace, void* stream) {
  if (!dims || !workspace) return DFSSM_E_NULL;
  int rc = dfssm_check_dims(dims);
  if (rc) return rc;
  const WsLayout w = ws_layout(dims);
  // ticket, error flag and the fused-layer flags and epoch are the tail of the workspace; a fill
  // kernel clears them
  uint32_t* p = (uint32_t*)((char*)workspace + w.ticket);
  const int n = (int)((w.total - w.ticket) / 4);
  hipLaunchKernelGGL(zero_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), p, n);
  return hip_status(hipGetLastError());
}

int* dfssm_workspace_error_flag(const dfssm_dims* dims, void* workspace) {
  if (!dims || !workspace || dfssm_check_dims(dims) != DFSSM_OK) return nullptr;
  return (int*)((char*)workspace + ws_layout(dims).err);
}

static int check_model(const dfssm_model* model) {
  if (!model || !model->layers || !model->emb || !model->norm_f) return DFSSM_E_NULL;
  if (model->dims.emb_code == 1 && !model->emb_scale) return DFSSM_E_NULL;
  int rc = dfssm_check_dims(&model->dims);
  if (rc) return rc;
  if (!aligned16(model->emb)) return DFSSM_E_ALIGN;
  return DFSSM_OK;
}

int dfssm_embed(const dfssm_model* model, const int64_t* tokens, uint16_t* x, void* workspace,
                void* stream) {
  int rc = check_model(model);
  if (rc) return rc;
  if (!tokens || !x || !workspace) return DFSSM_E_NULL;
  const Derived r = derive(&model->dims);
  EmbedArgs a{tokens, (const uint8_t*)model->emb, model->emb_scale, model->dims.emb_code == 0 ? 1 : 0, x,
              (int*)((char*)workspace + ws_layout(&model->dims).err), r.V, r.D};
  return hip_status(launch_embed(a, r.B, as_stream(stream)));
}

static int check_layer_args(const dfssm_model* model, int layer, uint16_t* x, const dfssm_state* state,
                            void* workspace) {
  int rc = check_model(model);
  if (rc) return rc;
  if (!x || !state || !state->h || !state->conv || !workspace) return DFSSM_E_NULL;
  if (layer < 0 || layer >= model->dims.n_layer) return DFSSM_E_RANGE;
  const dfssm_layer& Lw = model->layers[layer];
  if (!Lw.in_bits || !Lw.in_scale || !Lw.in_lA || !Lw.in_lA_s || !Lw.in_lB || !Lw.in_lB_s ||
      !Lw.out_bits || !Lw.out_scale || !Lw.out_lA || !Lw.out_lA_s || !Lw.out_lB || !Lw.out_lB_s ||
      !Lw.conv_w || !Lw.conv_b || !Lw.A_log || !Lw.D || !Lw.dt_bias || !Lw.norm_w || !Lw.ln_w ||
      !Lw.in_lBq || !Lw.out_lBq)
    return DFSSM_E_NULL;
  if (!aligned16(Lw.in_lBq) || !aligned16(Lw.out_lBq)) return DFSSM_E_ALIGN;
  if (!aligned16(Lw.in_bits) || !aligned16(Lw.out_bits) || !aligned16(Lw.in_lA) ||
      !aligned16(Lw.out_lA) || !aligned16(state->h) || ((uintptr_t)Lw.in_lB & 7u) ||
      ((uintptr_t)Lw.out_lB & 7u) || !aligned16(workspace) || !aligned16(Lw.ln_w) || !aligned16(Lw.norm_w) ||
      !aligned16(x))
    return DFSSM_E_ALIGN;
  return DFSSM_OK;
}

// The whole layer in one launch (batch <= 4).
static FusedArgs fused_args(const dfssm_model* model, int layer, uint16_t* x, const dfssm_state* state,
                            void* workspace) {
  const Derived r = derive(&model->dims);
  const dfssm_layer& Lw = model->layers[layer];
  const WsLayout w = ws_layout(&model->dims);
  char* ws = (char*)workspace;
  FusedArgs a{};
  a.in_bits = Lw.in_bits; a.in_ws = Lw.in_scale; a.in_lA = Lw.in_lA; a.in_lAs = Lw.in_lA_s;
  a.in_lBq = Lw.in_lBq;
  a.out_bits = Lw.out_bits; a.out_ws = Lw.out_scale; a.out_lA = Lw.out_lA; a.out_lAs = Lw.out_lA_s;
  a.out_lBq = Lw.out_lBq;
  a.conv_w = Lw.conv_w; a.conv_b = Lw.conv_b;
  a.A_log = Lw.A_log; a.Dp = Lw.D; a.dt_bias = Lw.dt_bias;
  a.norm_w = Lw.norm_w; a.ln_w = Lw.ln_w;
  a.h = state->h + (size_t)layer * r.B * r.H * r.P * r.N;
  a.conv = state->conv + (size_t)layer * r.B * r.C * 3;
  a.x = x;
  a.projT = (uint32_t*)(ws + w.proj_t);
  a.gT = (uint32_t*)(ws + w.g_t);
  a.hT = (uint32_t*)(ws + w.h_t);
  a.bcT = (uint32_t*)(ws + w.bc_t);
  a.dtT = (uint64_t*)(ws + w.dt_t);
  a.launches = (uint32_t*)(ws + w.launches);
  a.err = (int*)(ws + w.err);
  a.layer = layer;
  a.n_layer = r.L;
  a.D = r.D; a.DI = r.DI; a.N = r.N; a.H = r.H; a.P = r.P; a.IPO = r.IPO; a.C = r.C;
  return a;
}

// The whole layer in one launch (batch <= 4).
static int fused_layer(const dfssm_model* model, int layer, uint16_t* x, const dfssm_state* state,
                       void* workspace, void* stream) {
  const Derived r = derive(&model->dims);
  const FusedArgs a = fused_args(model, layer, x, state, workspace);
  return hip_status(launch_fused_layer(a, r.B, as_stream(stream)));
}

// Arguments of the matrix-core in_proj (in) or out_proj GEMM of `layer` (batch >= 5).
static GemmArgs batched_gemm_args(const dfssm_model* model, int layer, bool in, uint16_t* x, const dfssm_state* state,
                                  void* workspace) {
  const Derived r = derive(&model->dims);
  const dfssm_layer& Lw = model->layers[layer];
  const WsLayout w = ws_layout(&model->dims);
  char* ws = (char*)workspace;
  GemmArgs a{};
  a.q = (const int8_t*)(ws + w.q); a.ld_q = r.D > r.DI ? r.D : r.DI; a.M = r.B;
  a.xs = (const float*)(ws + w.xs);
  a.h = (const float*)(ws + w.h);
  if (in) {
    a.bits = Lw.in_bits; a.wscale = Lw.in_scale; a.lA = Lw.in_lA; a.lAs = Lw.in_lA_s;
    a.out = (uint16_t*)(ws + w.proj); a.ld_out = r.IPO;
    a.conv_state = state->conv + (size_t)layer * r.B * r.C * 3;
    a.conv_w = Lw.conv_w; a.conv_b = Lw.conv_b;
    a.conv_lo = r.DI; a.conv_c = r.C;
    a.N = r.IPO; a.K = r.D;
  } else {
    a.bits = Lw.out_bits; a.wscale = Lw.out_scale; a.lA = Lw.out_lA; a.lAs = Lw.out_lA_s;
    a.out = x; a.ld_out = r.D;
    a.N = r.D; a.K = r.DI;
  }
  return a;
}

// Phases 2 and 3 of dfssm_layer_phase in one launch (batch >= 5): the SSM step + gate, with the
// gated-norm prologue of out_proj computed by workgroups of the same launch.
static int ssm_prep_layer(const dfssm_model* model, int layer, const dfssm_state* state, void* workspace,
                          void* stream) {
  const Derived r = derive(&model->dims);
  const dfssm_layer& Lw = model->layers[layer];
  const WsLayout w = ws_layout(&model->dims);
  char* ws = (char*)workspace;
  uint16_t* proj = (uint16_t*)(ws + w.proj);
  SsmPrepArgs a{};
  a.s.h = state->h + (size_t)layer * r.B * r.H * r.P * r.N;
  a.s.xbc = proj + r.DI; a.s.ld_xbc = r.IPO;
  a.s.dt = proj + r.DI + r.C; a.s.ld_dt = r.IPO;
  a.s.z = proj; a.s.ld_z = r.IPO;
  a.s.dt_bias = Lw.dt_bias; a.s.A_log = Lw.A_log; a.s.D = Lw.D;
  a.s.H = r.H; a.s.P = r.P; a.s.N = r.N;
  a.gT = (uint32_t*)(ws + w.g_s);
  a.launches = (uint32_t*)(ws + w.launches_s);
  a.err = (int*)(ws + w.err);
  a.norm_w = Lw.norm_w;
  a.lB = Lw.out_lB; a.lBs = Lw.out_lB_s;
  a.q_out = (int8_t*)(ws + w.q); a.ld_q = r.D > r.DI ? r.D : r.DI;
  a.xs_out = (float*)(ws + w.xs);
  a.h_out = (float*)(ws + w.h);
  return hip_status(launch_ssm_prep(a, r.B, as_stream(stream)));
}

// Phase 4 of `layer` and phase 0 of layer + 1 in one launch (batch >= 5): out_proj with the next
// layer's in_proj prologue computed by workgroups of the same launch. DFSSM_E_DIMS (nothing
// launched) where the out_proj grid does not take them.
static int out_prep_layer(const dfssm_model* model, int layer, uint16_t* x, const dfssm_state* state,
                          void* workspace, void* stream) {
  const Derived r = derive(&model->dims);
  const WsLayout w = ws_layout(&model->dims);
  char* ws = (char*)workspace;
  const dfssm_layer& Ln = model->layers[layer + 1];
  GemmPro p{};
  p.xT = (uint32_t*)(ws + w.x_s);
  p.launches = (uint32_t*)(ws + w.launches_o);
  p.err = (int*)(ws + w.err);
  p.norm_w = Ln.ln_w;
  p.lB = Ln.in_lB; p.lBs = Ln.in_lB_s;
  p.q_out = (int8_t*)(ws + w.q); p.ld_q = r.D > r.DI ? r.D : r.DI;
  p.xs_out = (float*)(ws + w.xs);
  p.h_out = (float*)(ws + w.h);
  const hipError_t e = launch_gemm_out_pro(batched_gemm_args(model, layer, false, x, state, workspace), p,
                                           as_stream(stream));
  return e == hipErrorNotSupported ? DFSSM_E_DIMS : hip_status(e);
}

int dfssm_layer_phase(const dfssm_model* model, int layer, int phase, uint16_t* x,
                      const dfssm_state* state, void* workspace, void* stream) {
  int rc = check_layer_args(model, layer, x, state, workspace);
  if (rc) return rc;
  if (phase < 0 || phase > DFSSM_PHASE_OUT_PROLOGUE) return DFSSM_E_RANGE;
  const Derived r = derive(&model->dims);
  if (phase == DFSSM_PHASE_SSM_PROLOGUE) {
    if (r.B <= 4 || !ssm_prep_supported(r.B, r.DI, r.P)) return DFSSM_E_DIMS;
    return ssm_prep_layer(model, layer, state, workspace, stream);
  }
  if (phase == DFSSM_PHASE_OUT_PROLOGUE) {
    if (r.B <= 4 || layer + 1 >= r.L) return DFSSM_E_DIMS;
    return out_prep_layer(model, layer, x, state, workspace, stream);
  }
  const dfssm_layer& Lw = model->layers[layer];
  const WsLayout w = ws_layout(&model->dims);
  char* ws = (char*)workspace;
  uint16_t* proj = (uint16_t*)(ws + w.proj);
  uint16_t* g = (uint16_t*)(ws + w.g);
  double* slots = (double*)(ws + w.slots);
  const int kq = r.D > r.DI ? r.D : r.DI;
  hipStream_t s = as_stream(stream);

  if (phase == 0 || phase == 3) {  // prologue of in_proj (x) / out_proj (gated g)
    PrepArgs p{};
    const bool in = phase == 0;
    p.act = in ? x : g;
    p.ld_act = in ? r.D : r.DI;
    p.norm_w = in ? Lw.ln_w : Lw.norm_w;
    p.sumsq_slots = in ? nullptr : slots;
    p.n_slots = in ? 0 : r.n_slots;
    p.lB = in ? Lw.in_lB : Lw.out_lB;
    p.lBs = in ? Lw.in_lB_s : Lw.out_lB_s;
    p.q_out = (int8_t*)(ws + w.q);
    p.ld_q = kq;
    if (r.B <= 4) {  // the bit-plane GEMV reads planes and sum q; the matrix-core GEMM neither
      p.planes_out = (uint32_t*)(ws + w.planes);
      p.s_out = (int*)(ws + w.qsum);
    }
    p.xs_out = (float*)(ws + w.xs);
    p.h_out = (float*)(ws + w.h);
    p.K = in ? r.D : r.DI;
    return hip_status(launch_prep(p, r.B, in ? DFSSM_MODE_IN : DFSSM_MODE_OUT, s));
  }
  if (phase == 2) {  // SSM step + gate -> g, per-block sum(g^2)
    SsmArgs as{};
    as.h = state->h + (size_t)layer * r.B * r.H * r.P * r.N;
    as.xbc = proj + r.DI; as.ld_xbc = r.IPO;
    as.dt = proj + r.DI + r.C; as.ld_dt = r.IPO;
    as.z = proj; as.ld_z = r.IPO;
    as.dt_bias = Lw.dt_bias; as.A_log = Lw.A_log; as.D = Lw.D;
    as.y_out = g; as.ld_y = r.DI;
    as.sumsq_slots = slots; as.n_slots = r.n_slots;
    as.H = r.H; as.P = r.P; as.N = r.N;
    return hip_status(launch_ssm(as, r.B, s));
  }
  const bool in = phase == 1;
  if (r.B > 4) {  // int8 matrix-core path
    const GemmArgs a = batched_gemm_args(model, layer, in, x, state, workspace);
    return hip_status(launch_gemm(a, in ? DFSSM_MODE_IN : DFSSM_MODE_OUT, s));
  }
  ProjArgs a{};
  a.planes = (const uint32_t*)(ws + w.planes);
  a.ld_q = kq;
  a.qsum = (const int*)(ws + w.qsum);
  a.xs = (const float*)(ws + w.xs);
  a.h = (const float*)(ws + w.h);
  if (in) {  // in_proj scaffold + LoRA + conv/SiLU -> proj
    a.bits = Lw.in_bits; a.wscale = Lw.in_scale; a.lA = Lw.in_lA; a.lAs = Lw.in_lA_s;
    a.out = proj; a.ld_out = r.IPO;
    a.conv_state = state->conv + (size_t)layer * r.B * r.C * 3;
    a.conv_w = Lw.conv_w; a.conv_b = Lw.conv_b;
    a.conv_lo = r.DI; a.conv_c = r.C;
    a.N = r.IPO; a.K = r.D;
    return hip_status(launch_proj(a, r.B, DFSSM_MODE_IN, s));
  }
  // phase 4: out_proj scaffold + LoRA + residual -> x
  a.bits = Lw.out_bits; a.wscale = Lw.out_scale; a.lA = Lw.out_lA; a.lAs = Lw.out_lA_s;
  a.out = x; a.ld_out = r.D;
  a.N = r.D; a.K = r.DI;
  return hip_status(launch_proj(a, r.B, DFSSM_MODE_OUT, s));
}

int dfssm_layer_step(const dfssm_model* model, int layer, uint16_t* x, const dfssm_state* state,
                     void* workspace, void* stream) {
  int rc = check_layer_args(model, layer, x, state, workspace);
  if (rc) return rc;
  const Derived r = derive(&model->dims);
  const bool one_launch = g_layer_kernel != DFSSM_LAYER_FIVE && fused_layer_supported(r.B, r.IPO, r.D, r.DI, r.H, r.P);
  if (one_launch) return fused_layer(model, layer, x, state, workspace, stream);
  if (r.B > 4 && g_layer_kernel != DFSSM_LAYER_FIVE && ssm_prep_supported(r.B, r.DI, r.P)) {
    // four launches: prologue + in_proj, SSM with the out_proj prologue, out_proj
    for (int phase : {0, 1}) {
      rc = dfssm_layer_phase(model, layer, phase, x, state, workspace, stream);
      if (rc) return rc;
    }
    rc = ssm_prep_layer(model, layer, state, workspace, stream);
    if (rc) return rc;
    return dfssm_layer_phase(model, layer, 4, x, state, workspace, stream);
  }
  for (int phase = 0; phase < DFSSM_LAYER_PHASES; ++phase) {
    const int rc = dfssm_layer_phase(model, layer, phase, x, state, workspace, stream);
    if (rc) return rc;
  }
  return DFSSM_OK;
}

int dfssm_lmhead_argmax(const dfssm_model* model, const uint16_t* x, void* workspace,
                        uint16_t* logits, int64_t* next, uint16_t* x_next, void* stream) {
  int rc = check_model(model);
  if (rc) return rc;
  if (!x || !workspace || !next) return DFSSM_E_NULL;
  const Derived r = derive(&model->dims);
  const WsLayout w = ws_layout(&model->dims);
  char* ws = (char*)workspace;
  if (r.B > 4) {  // matrix-core head: exact on the int8 table, fp32 accumulation on an fp16 table
    HeadArgs a{};
    a.x = x; a.norm_f = model->norm_f; a.emb = (const uint8_t*)model->emb; a.emb_scale = model->emb_scale;
    a.f16 = model->dims.emb_code == 0 ? 1 : 0;
    a.V = r.V; a.D = r.D; a.logits = logits;
    a.part_val = (float*)(ws + w.part_val); a.part_idx = (int*)(ws + w.part_idx);
    a.ticket = (unsigned*)(ws + w.ticket);
    a.next = next; a.x_next = x_next;
    a.xf = (const uint16_t*)(ws + w.xf);
    a.hdig = (const int8_t*)(ws + w.hdig);
    return hip_status(launch_head_batched(a, r.B, as_stream(stream)));
  }
  HeadArgs a{};
  a.x = x; a.norm_f = model->norm_f; a.emb = (const uint8_t*)model->emb; a.emb_scale = model->emb_scale;
    a.f16 = model->dims.emb_code == 0 ? 1 : 0;
  a.V = r.V; a.D = r.D; a.logits = logits;
  a.part_val = (float*)(ws + w.part_val); a.part_idx = (int*)(ws + w.part_idx);
  a.ticket = (unsigned*)(ws + w.ticket);
  a.next = next; a.x_next = x_next;
  rc = hip_status(launch_head(a, r.B, as_stream(stream)));
  if (rc) return rc;
  return DFSSM_OK;
}

// The layers of a decode step, launch by launch. Batch >= 5 (unless DFSSM_LAYER_FIVE): per layer
// the in_proj GEMM, the SSM launch with out_proj's prologue, and the out_proj launch with the
// next layer's in_proj prologue where the shape takes it (else out_proj, and the next layer's
// prologue on its own), three launches instead of five; other batches layer by layer as
// dfssm_layer_step.
static int decode_layers(const dfssm_model* model, uint16_t* x, const dfssm_state* state, void* workspace,
                         void* stream) {
  const Derived r = derive(&model->dims);
  int rc = DFSSM_OK;
  if (r.B <= 4 || g_layer_kernel == DFSSM_LAYER_FIVE || !ssm_prep_supported(r.B, r.DI, r.P)) {
    for (int l = 0; l < r.L && !rc; ++l) rc = dfssm_layer_step(model, l, x, state, workspace, stream);
    return rc;
  }
  bool prepped = false;  // the q, scale and LoRA intermediates of this layer's in_proj are written
  for (int l = 0; l < r.L; ++l) {
    if (!prepped && (rc = dfssm_layer_phase(model, l, 0, x, state, workspace, stream))) return rc;
    if ((rc = dfssm_layer_phase(model, l, 1, x, state, workspace, stream))) return rc;
    if ((rc = dfssm_layer_phase(model, l, DFSSM_PHASE_SSM_PROLOGUE, x, state, workspace, stream))) return rc;
    rc = dfssm_layer_phase(model, l, DFSSM_PHASE_OUT_PROLOGUE, x, state, workspace, stream);
    prepped = rc == DFSSM_OK;
    if (rc == DFSSM_E_DIMS && (rc = dfssm_layer_phase(model, l, 4, x, state, workspace, stream))) return rc;
    if (rc) return rc;
  }
  return DFSSM_OK;
}

int dfssm_decode_step(const dfssm_model* model, const int64_t* tokens, uint16_t* x,
                      const dfssm_state* state, void* workspace, uint16_t* logits, int64_t* next,
                      int fuse_next_embed, void* stream) {
  int rc = check_model(model);
  if (rc) return rc;
  if (!x || !state || !workspace || !next) return DFSSM_E_NULL;
  if (tokens) {
    rc = dfssm_embed(model, tokens, x, workspace, stream);
    if (rc) return rc;
  }
  rc = decode_layers(model, x, state, workspace, stream);
  if (rc) return rc;
  return dfssm_lmhead_argmax(model, x, workspace, logits, next, fuse_next_embed ? x : nullptr, stream);
}

int dfssm_sample(const dfssm_model* model, const uint16_t* logits, int32_t* counts, uint32_t* step,
                 const dfssm_sample_params* params, int64_t* next, uint16_t* x_next, void* workspace,
                 void* stream) {
  int rc = check_model(model);
  if (rc) return rc;
  if (!logits || !counts || !step || !params || !next) return DFSSM_E_NULL;
  const Derived r = derive(&model->dims);
  if (r.V > kSampleMaxVocab) return DFSSM_E_DIMS;
  const dfssm_sample_params& p = *params;
  if (!(p.temperature > 0.0f) || !(p.penalty > 0.0f) || !(p.top_p >= 0.0f) || (p.mode != 0 && p.mode != 1))
    return DFSSM_E_RANGE;
  SampleArgs a{};
  a.logits = logits; a.counts = counts; a.step = step; a.next = next;
  a.temperature = p.temperature; a.top_p = p.top_p; a.penalty = p.penalty; a.mode = p.mode; a.seed = p.seed;
  a.V = r.V;
  if (!workspace) return DFSSM_E_NULL;
  a.escratch = (float*)((char*)workspace + ws_layout(&model->dims).samp);
  hipStream_t s = as_stream(stream);
  rc = hip_status(launch_sample(a, r.B, s));
  if (rc || !x_next) return rc;
  return dfssm_embed(model, next, x_next, workspace, stream);
}

size_t dfssm_prefill_workspace_bytes(const dfssm_dims* dims, int max_rows) {
  if (!dims || dfssm_check_dims(dims) != DFSSM_OK) return 0;
  if (max_rows < dims->batch || max_rows > kGemmMaxRows) return 0;
  return pf_layout(derive(dims), max_rows).total;
}

// One chunk of the prefill: tokens t0 .. t0 + tc - 1 of every sequence through all layers.
static int prefill_chunk(const dfssm_model* model, const int64_t* tokens, int n_tokens, int t0, int tc,
                         const dfssm_state* state, void* workspace, char* pw, hipStream_t s) {
  const Derived r = derive(&model->dims);
  const PfLayout w = pf_layout(r, r.B * tc);
  const int R = r.B * tc;
  const int kq = r.D > r.DI ? r.D : r.DI;
  uint16_t* xr = (uint16_t*)(pw + w.x);
  uint16_t* proj = (uint16_t*)(pw + w.proj);
  uint16_t* g = (uint16_t*)(pw + w.g);
  double* slots = (double*)(pw + w.slots);
  EmbedArgs e{tokens, (const uint8_t*)model->emb, model->emb_scale, model->dims.emb_code == 0 ? 1 : 0, xr,
              (int*)((char*)workspace + ws_layout(&model->dims).err), r.V, r.D, n_tokens, t0, tc};
  hipError_t st = launch_embed(e, R, s);
  if (st != hipSuccess) return hip_status(st);
  for (int l = 0; l < r.L; ++l) {
    const dfssm_layer& Lw = model->layers[l];
    float* h = state->h + (size_t)l * r.B * r.H * r.P * r.N;
    uint16_t* conv = state->conv + (size_t)l * r.B * r.C * 3;
    for (int ph = 0; ph < 2; ++ph) {  // in_proj, then out_proj
      const bool in = ph == 0;
      PrepArgs p{};
      p.act = in ? xr : g;
      p.ld_act = in ? r.D : r.DI;
      p.norm_w = in ? Lw.ln_w : Lw.norm_w;
      p.sumsq_slots = in ? nullptr : slots;
      p.n_slots = in ? 0 : r.n_slots;
      p.lB = in ? Lw.in_lB : Lw.out_lB;
      p.lBs = in ? Lw.in_lB_s : Lw.out_lB_s;
      p.q_out = (int8_t*)(pw + w.q);
      p.ld_q = kq;
      p.xs_out = (float*)(pw + w.xs);
      p.h_out = (float*)(pw + w.h);
      p.K = in ? r.D : r.DI;
      p.q_tiled = R >= kWideGemmRows;  // the wide GEMM reads q tiled
      st = launch_prep(p, R, in ? DFSSM_MODE_IN : DFSSM_MODE_OUT, s);
      if (st != hipSuccess) return hip_status(st);
      GemmArgs a{};
      a.q = (const int8_t*)(pw + w.q); a.ld_q = kq; a.M = R;
      a.xs = (const float*)(pw + w.xs);
      a.h = (const float*)(pw + w.h);
      if (in) {  // raw projection rows: the conv runs over the tokens below
        a.bits = Lw.in_bits; a.wscale = Lw.in_scale; a.lA = Lw.in_lA; a.lAs = Lw.in_lA_s;
        a.out = proj; a.ld_out = r.IPO;
        a.N = r.IPO; a.K = r.D;
      } else {
        a.bits = Lw.out_bits; a.wscale = Lw.out_scale; a.lA = Lw.out_lA; a.lAs = Lw.out_lA_s;
        a.out = xr; a.ld_out = r.D;
        a.N = r.D; a.K = r.DI;
      }
      st = R >= kWideGemmRows ? launch_gemm_wide(a, in ? DFSSM_MODE_IN : DFSSM_MODE_OUT, (int8_t*)(pw + w.w8), s)
                              : launch_gemm(a, in ? DFSSM_MODE_IN : DFSSM_MODE_OUT, s);
      if (st != hipSuccess) return hip_status(st);
      if (!in) break;
      ConvSeqArgs c{conv, proj + r.DI, r.IPO, Lw.conv_w, Lw.conv_b, r.C, tc};
      st = launch_conv_seq(c, r.B, s);
      if (st != hipSuccess) return hip_status(st);
      ScanArgs sc{};
      sc.h = h;
      sc.xbc = proj + r.DI; sc.ld_xbc = r.IPO;
      sc.dt = proj + r.DI + r.C; sc.ld_dt = r.IPO;
      sc.z = proj; sc.ld_z = r.IPO;
      sc.dt_bias = Lw.dt_bias; sc.A_log = Lw.A_log; sc.D = Lw.D;
      sc.y_out = g; sc.ld_y = r.DI;
      sc.sumsq_slots = slots; sc.n_slots = r.n_slots;
      sc.H = r.H; sc.P = r.P; sc.N = r.N; sc.T = tc;
      st = launch_ssm_scan(sc, r.B, s);
      if (st != hipSuccess) return hip_status(st);
    }
  }
  return DFSSM_OK;
}

int dfssm_prefill(const dfssm_model* model, const int64_t* tokens, int n_tokens, uint16_t* x,
                  const dfssm_state* state, void* workspace, void* prefill_workspace, int max_rows,
                  uint16_t* logits, int64_t* next, int fuse_next_embed, void* stream) {
  int rc = check_model(model);
  if (rc) return rc;
  if (!tokens || !x || !state || !state->h || !state->conv || !workspace || !prefill_workspace || !next)
    return DFSSM_E_NULL;
  const Derived r = derive(&model->dims);
  if (n_tokens < 1 || max_rows < r.B || max_rows > kGemmMaxRows) return DFSSM_E_RANGE;
  if (!aligned16(prefill_workspace) || !aligned16(workspace) || !aligned16(x) || !aligned16(state->h))
    return DFSSM_E_ALIGN;
  for (int l = 0; l < r.L; ++l) {
    rc = check_layer_args(model, l, x, state, workspace);
    if (rc) return rc;
  }
  hipStream_t s = as_stream(stream);
  char* pw = (char*)prefill_workspace;
  const int T = max_rows / r.B;  // tokens per chunk
  int tc = 0;
  for (int t0 = 0; t0 < n_tokens; t0 += tc) {
    tc = n_tokens - t0 < T ? n_tokens - t0 : T;
    rc = prefill_chunk(model, tokens, n_tokens, t0, tc, state, workspace, pw, s);
    if (rc) return rc;
  }
  // the last token's residual row of every sequence, then the head as after a decode step
  rc = hip_status(launch_last_rows((const uint16_t*)(pw + pf_layout(r, r.B * tc).x), x, r.B, tc, r.D, s));
  if (rc) return rc;
  return dfssm_lmhead_argmax(model, x, workspace, logits, next, fuse_next_embed ? x : nullptr, stream);
}

}  // extern "C"

// ---- decode step without a caller workspace (no allocation) ---------------------------------
// The decode workspace lives in `scratch`, a file-scope device array of
// DFSSM_STATIC_WORKSPACE_BYTES that every GPU the library runs on holds until the process ends.
// Host code never passes `scratch` itself (its name is a host-side stand-in, not a device
// address): the device address comes from hipGetSymbolAddress, once per device, and is kept per
// device. The part of the workspace that must start at zero (tickets, error flag, launch counts
// and exchange words of the one-launch layer) is cleared by a fill kernel when a device is first
// used and whenever the model dimensions change (the layout depends on them); nothing is cleared
// on later calls with the same dimensions, which share the array's contents in stream order.
static __device__ __align__(256) unsigned char scratch[DFSSM_STATIC_WORKSPACE_BYTES];

namespace {

constexpr int kStaticMaxDevices = 64;
struct StaticWs {
  void* ptr = nullptr;
  bool cleared = false;
  dfssm_dims dims{};
};
StaticWs g_static[kStaticMaxDevices];
std::mutex g_static_mu;

__global__ void take_flag_kernel(int* flag, int* out) {
  if (threadIdx.x == 0) {
    *out = *flag;
    *flag = 0;
  }
}

// Device address of this device's static workspace, cleared for `dims` if it was last used with
// other dimensions (or never). Returns a DFSSM code.
int static_workspace(const dfssm_dims* dims, hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  if (dev < 0 || dev >= kStaticMaxDevices) return DFSSM_E_RANGE;
  std::lock_guard<std::mutex> lock(g_static_mu);
  StaticWs& st = g_static[dev];
  if (!st.ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e);
    if (!p) return DFSSM_E_NULL;
    st.ptr = p;
  }
  if (!st.cleared || memcmp(&st.dims, dims, sizeof(dfssm_dims)) != 0) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return hip_status(e);
    if (cs != hipStreamCaptureStatusNone) return DFSSM_E_CAPTURE;
    const int rc = dfssm_workspace_init(dims, st.ptr, stream);  // a fill kernel, no memset
    if (rc) return rc;
    st.dims = *dims;
    st.cleared = true;
  }
  *out = st.ptr;
  return DFSSM_OK;
}

}  // namespace

extern "C" {

int dfssm_decode_step_static(const dfssm_model* model, const int64_t* tokens, uint16_t* x,
                             const dfssm_state* state, uint16_t* logits, int64_t* next, int fuse_next_embed,
                             int* error_out, void* stream) {
  int rc = check_model(model);
  if (rc) return rc;
  if (!x || !state || !next) return DFSSM_E_NULL;
  const size_t need = dfssm_workspace_bytes(&model->dims);
  if (need == 0) return DFSSM_E_DIMS;
  if (need > (size_t)DFSSM_STATIC_WORKSPACE_BYTES) return DFSSM_E_SCRATCH;
  hipStream_t s = as_stream(stream);
  void* ws = nullptr;
  rc = static_workspace(&model->dims, s, &ws);
  if (rc) return rc;
  rc = dfssm_decode_step(model, tokens, x, state, ws, logits, next, fuse_next_embed, stream);
  if (!error_out) return rc;
  // also when the step failed after queueing some of its kernels: their flag bits belong to this call
  hipLaunchKernelGGL(take_flag_kernel, dim3(1), dim3(64), 0, s, dfssm_workspace_error_flag(&model->dims, ws), error_out);
  const int rc2 = hip_status(hipGetLastError());
  return rc ? rc : rc2;
}

int dfssm_state_density_field(float* h, float* sd_error, int64_t rows, int d_state, const float* thresholds,
                              int kk, int sd_bits, void* stream) {
  if (!h || !thresholds) return DFSSM_E_NULL;
  if (d_state != 128) return DFSSM_E_DIMS;
  if (rows < 0 || kk < 1 || kk > kStateDfMaxKK || sd_bits < 1) return DFSSM_E_RANGE;
  if (((uintptr_t)h & 15u) || ((uintptr_t)sd_error & 15u) || ((uintptr_t)thresholds & 3u)) return DFSSM_E_ALIGN;
  StateDfArgs a{};
  a.h = h; a.sd_error = sd_error; a.thresholds = thresholds; a.rows = rows; a.kk = kk; a.sd_bits = sd_bits;
  return hip_status(launch_state_df(a, as_stream(stream)));
}

}  // extern "C"
