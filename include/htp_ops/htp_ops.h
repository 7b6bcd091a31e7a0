/*
 * Backend lifecycle entry points.  The reference declares these in its FastRPC
 * IDL (reference include/htp_ops.idl:9-28) and the host calls them through the
 * generated stub; here they are plain C functions of the same names,
 * argument meanings and AEE return codes, backed by one MI355X.
 *
 *   htp_ops_open / htp_ops_close           reference src/dsp/commu.c:369-409
 *   htp_ops_init_backend[_fraction]        reference src/dsp/commu.c:412-467, 507-549
 *   htp_ops_init_mapping_backend           reference src/dsp/commu.c:469-480
 *   htp_ops_release_backend                reference src/dsp/commu.c:482-505
 *   htp_ops_create_channel[_with_token]    reference src/dsp/commu.c:551-572
 *   htp_ops_destroy_channel                reference src/dsp/commu.c:574-576
 *   htp_ops_mat_mul_permuted_w16a32[_trace] reference src/dsp/commu.c:637-797
 *   htp_ops_test_ops                       reference src/dsp/commu.c:813-827
 */
#ifndef HTP_OPS_HTP_OPS_H
#define HTP_OPS_HTP_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef HTP_OPS_REMOTE_HANDLE64_DEFINED
#define HTP_OPS_REMOTE_HANDLE64_DEFINED
typedef uint64_t remote_handle64;
#endif

typedef int AEEResult;

/* AEE result codes used by this interface (Hexagon SDK AEEStdErr.h values). */
#define AEE_SUCCESS 0
#define AEE_EFAILED 1
#define AEE_ENOMEMORY 2
#define AEE_EBADSTATE 13
#define AEE_EBADPARM 14
#define AEE_EUNSUPPORTED 20
#define AEE_EALREADY 26

AEEResult htp_ops_open(const char *uri, remote_handle64 *handle);
AEEResult htp_ops_close(remote_handle64 handle);
AEEResult htp_ops_init_backend(remote_handle64 handle);
AEEResult htp_ops_init_backend_fraction(remote_handle64 handle, uint32_t numerator, uint32_t denominator);
AEEResult htp_ops_init_mapping_backend(remote_handle64 handle);
AEEResult htp_ops_release_backend(remote_handle64 handle);
AEEResult htp_ops_create_channel(remote_handle64 handle, int32_t fd, uint32_t size);
AEEResult htp_ops_create_channel_with_token(remote_handle64 handle, uint64_t session_token, int32_t fd,
                                            uint32_t size);
AEEResult htp_ops_destroy_channel(remote_handle64 handle);

/* Opcode 0 is outside this library: returns AEE_EUNSUPPORTED. */
AEEResult htp_ops_rms_norm_f32(remote_handle64 handle, int32_t fd0, int32_t offset0, int32_t fd1,
                               int32_t offset1, int32_t ne0, int32_t ne1);
/* Direct (non-mailbox) opcode-1 GEMM: output f32 [m][n] = fp16(act) x permuted W. */
AEEResult htp_ops_mat_mul_permuted_w16a32(remote_handle64 handle, int32_t output_fd, int32_t output_offset,
                                          int32_t activation_fd, int32_t activation_offset, int32_t weight_fd,
                                          int32_t weight_offset, int32_t m, int32_t k, int32_t n);
/* Same GEMM; also returns FNV-1a 64 hashes of the activation and output bytes. */
AEEResult htp_ops_mat_mul_permuted_w16a32_trace(remote_handle64 handle, int32_t output_fd, int32_t output_offset,
                                                int32_t activation_fd, int32_t activation_offset,
                                                int32_t weight_fd, int32_t weight_offset, int32_t m, int32_t k,
                                                int32_t n, uint64_t *activation_hash, uint64_t *output_hash,
                                                uint64_t *output_hash_after_remap);
/* Runs the library's built-in host contract tests; *userdma_scope = 1. */
AEEResult htp_ops_test_ops(remote_handle64 handle, int32_t *userdma_scope);

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_HTP_OPS_H */
