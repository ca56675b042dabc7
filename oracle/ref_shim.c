/*
 * ref_shim.c -- TEST INFRASTRUCTURE ONLY. Appended (by build_ref.sh) to the translation unit of
 * the reference inference/cpu/cpu_inference.c so that its file-static step functions can be
 * called from tests through ctypes. Each wrapper forwards its arguments unchanged.
 */
void ref_rms_norm(const float* x, const float* w, float* out, int dim) { rms_norm(x, w, out, dim); }
void ref_quantize_u8(const float* x, uint8_t* q, float* scale_out, int n) { quantize_input_uint8(x, q, scale_out, n); }
void ref_scaffold_matvec(const uint32_t* packed_w, const float* x, const float* scale, const int* row_sums,
                         float* out, int out_features, int packed_cols) {
  scaffold_matvec_avx512(packed_w, x, scale, row_sums, out, out_features, packed_cols);
}
void ref_lora_matvec(const int8_t* A, const float* As, const int8_t* B, const float* Bs, const float* x,
                     float* out, int out_features, int in_features, int rank) {
  lora_matvec(A, As, B, Bs, x, out, out_features, in_features, rank);
}
void ref_conv_step(float* conv_state, float* xBC, const float* conv_w, const float* conv_b) {
  conv_step(conv_state, xBC, conv_w, conv_b);
}
void ref_ssm_step(float* h_state, const float* x_ssm, const float* B_param, const float* C_param, const float* dt,
                  const float* A_log, const float* D_param, float* y_out) {
  ssm_step(h_state, x_ssm, B_param, C_param, dt, A_log, D_param, y_out);
}
void ref_gate_norm(const float* y, const float* z, const float* w, float* out, int dim) { gate_norm(y, z, w, out, dim); }
int ref_headdim(void) { return HEADDIM; }
