/*
 * Exported op wrappers and capability markers (reference src/host/op_export.c:6-48).
 */
#include "htp_ops/op_export.h"

int htp_ops_rpc_rms_norm_f32(int dst_fd, int dst_offset, int src_fd, int src_offset, int ne0, int ne1) {
  return htp_ops_rms_norm_f32(get_global_handle(), dst_fd, dst_offset, src_fd, src_offset, ne0, ne1);
}

int htp_ops_rpc_rms_norm_f32_session(htp_ops_session *session, int dst_fd, int dst_offset, int src_fd,
                                     int src_offset, int ne0, int ne1) {
  return htp_ops_rms_norm_f32(htp_ops_session_handle(session), dst_fd, dst_offset, src_fd, src_offset, ne0, ne1);
}

int htp_ops_rpc_mat_mul_permuted_w16a32(int output_fd, int output_offset, int activation_fd,
                                        int activation_offset, int weight_fd, int weight_offset, int m, int k,
                                        int n) {
  return htp_ops_mat_mul_permuted_w16a32(get_global_handle(), output_fd, output_offset, activation_fd,
                                         activation_offset, weight_fd, weight_offset, m, k, n);
}

int htp_ops_rpc_mat_mul_permuted_w16a32_session(htp_ops_session *session, int output_fd, int output_offset,
                                                int activation_fd, int activation_offset, int weight_fd,
                                                int weight_offset, int m, int k, int n) {
  return htp_ops_mat_mul_permuted_w16a32(htp_ops_session_handle(session), output_fd, output_offset, activation_fd,
                                         activation_offset, weight_fd, weight_offset, m, k, n);
}

int htp_ops_rpc_mat_mul_permuted_w16a32_trace_session(htp_ops_session *session, int output_fd,
                                                      int output_offset, int activation_fd,
                                                      int activation_offset, int weight_fd, int weight_offset,
                                                      int m, int k, int n, uint64_t *activation_hash,
                                                      uint64_t *output_hash, uint64_t *output_hash_after_remap) {
  return htp_ops_mat_mul_permuted_w16a32_trace(htp_ops_session_handle(session), output_fd, output_offset,
                                               activation_fd, activation_offset, weight_fd, weight_offset, m, k, n,
                                               activation_hash, output_hash, output_hash_after_remap);
}

/* Opcode 16 (shared-message F16 GEMM with fused epilogue) is implemented. */
int htp_ops_f16_epilogue_version(void) { return 1; }

/* Opcode 19's DiT modes (9 LayerNorm + modulation, 10 gated residual, 11
 * matrix RoPE, 12 strided SwiGLU, 13 SwiGLU beside the attention output) are
 * implemented, so both DiT markers advertise them (reference
 * src/host/op_export.c:45-48).  Opcodes 17 and 18 (native conv / attention)
 * are not: the native-model marker stays 0. */
int htp_ops_native_model_version(void) { return 0; }
int htp_ops_dit_aux_version(void) { return 1; }
int htp_ops_dit_concat_version(void) { return 1; }
