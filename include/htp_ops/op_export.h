/*
 * Exported op wrappers and capability markers.
 *   htp_ops_rpc_*               reference include/host/op_export.h:1-17, src/host/op_export.c:6-38
 *   htp_ops_f16_epilogue_version reference src/host/op_export.c:41 (returns 1: opcode 16 supported)
 *   native_model / dit_aux / dit_concat markers: reference src/host/op_export.c:43-48.  Those
 *     advertise opcodes 17-19 which this library does not implement, so they return 0.
 */
#ifndef HTP_OPS_OP_EXPORT_H
#define HTP_OPS_OP_EXPORT_H

#include <stdint.h>

#include "session.h"

#ifdef __cplusplus
extern "C" {
#endif

int htp_ops_rpc_rms_norm_f32(int dst_fd, int dst_offset, int src_fd, int src_offset, int ne0, int ne1);
int htp_ops_rpc_rms_norm_f32_session(htp_ops_session *session, int dst_fd, int dst_offset, int src_fd,
                                     int src_offset, int ne0, int ne1);
int htp_ops_rpc_mat_mul_permuted_w16a32(int output_fd, int output_offset, int activation_fd,
                                        int activation_offset, int weight_fd, int weight_offset, int m, int k,
                                        int n);
int htp_ops_rpc_mat_mul_permuted_w16a32_session(htp_ops_session *session, int output_fd, int output_offset,
                                                int activation_fd, int activation_offset, int weight_fd,
                                                int weight_offset, int m, int k, int n);
int htp_ops_rpc_mat_mul_permuted_w16a32_trace_session(htp_ops_session *session, int output_fd,
                                                      int output_offset, int activation_fd,
                                                      int activation_offset, int weight_fd, int weight_offset,
                                                      int m, int k, int n, uint64_t *activation_hash,
                                                      uint64_t *output_hash, uint64_t *output_hash_after_remap);

int htp_ops_f16_epilogue_version(void);
int htp_ops_native_model_version(void);
int htp_ops_dit_aux_version(void);
int htp_ops_dit_concat_version(void);

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_OP_EXPORT_H */
