/*
 * Host-side weight packers producing the reference's weight formats.
 *
 * The reference consumes W8A8 constants blobs and permuted FP16 weights but
 * does not contain their producers (the W8A8 packer lives in sd.cpp, which is
 * absent; the FP16 writer appears only inside the reference's host test,
 * src/host/test.c:547-558).  These functions write the formats exactly as the
 * reference's consumers read them:
 *   blob header / offsets   reference include/op_reg.h:80-85, src/dsp/op_executor.cc:321-335
 *   W(n,k) deep tile address reference src/dsp/ops/linear_w8a8.c:453,482,486-488,
 *                            tests/hmx-probe/study_dsp.c:82-84
 *   permuted FP16 (k,n)      reference src/host/test.c:551-556
 */
#ifndef HTP_OPS_PACK_H
#define HTP_OPS_PACK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 128 + k*n + 8*n + 4*k */
size_t htp_ops_w8a8_constants_bytes(int k, int n);

/*
 * Writes a W8A8 constants blob.  w: int8 [n][k] (row n = output channel);
 * sw: f32[n] per-column scale; sums: i32[n] or NULL (then sum_k w[n][k]);
 * inv: f32[k] smoothing vector or NULL (then 1.0).  Requires k % 32 == 0,
 * n % 64 == 0 and blob_bytes >= htp_ops_w8a8_constants_bytes(k, n).
 * Returns 0, or -1 on a bad argument.
 */
int htp_ops_w8a8_pack_constants(uint8_t *blob, size_t blob_bytes, const int8_t *w, const float *sw,
                                const int32_t *sums, const float *inv, int k, int n, uint64_t signature);

/*
 * Symmetric per-output-channel quantization of f32 weights w [n][k] (after
 * dividing each input channel by inv[k], NULL = 1): sw[n] = max_k |w/inv| / 127
 * (1 when the row is zero) and q = rne(w/inv / sw) clamped to [-127, 127].
 * Design of this library (the reference's producer is absent).
 */
int htp_ops_w8a8_quantize_weights(int8_t *q, float *sw, const float *w, const float *inv, int k, int n);

/*
 * FP16 source weights -> W8A8 constants blob in one call (the sd.cpp-side
 * producer the reference's blob header is designed for: op_reg.h:80-85 keeps
 * an original_f16_signature of the weights the blob was made from).
 * w_f16: fp16 bits [n][k] (row n = output channel), converted to f32 exactly;
 * inv: f32[k] smoothing vector or NULL (then 1.0, stored as such).  The
 * weights are quantized by htp_ops_w8a8_quantize_weights (w / inv, per
 * output channel), sums are sum_k q, and original_f16_signature is
 * htp_ops_fnv1a64 of the k*n*2 fp16 bytes.  Same shape and size rules as
 * htp_ops_w8a8_pack_constants.  Returns 0, or -1 on a bad argument or when
 * scratch memory cannot be allocated.
 */
int htp_ops_w8a8_pack_f16(uint8_t *blob, size_t blob_bytes, const uint16_t *w_f16, const float *inv, int k, int n);

/* FNV-1a 64 of a byte range (the value stored as original_f16_signature by callers that want one). */
uint64_t htp_ops_fnv1a64(const void *data, size_t bytes);

/* Logical fp16 weight w [k][n] (row-major, fp16 bits) -> reference permuted layout. */
int htp_ops_f16_permute_weights(uint16_t *permuted, const uint16_t *w_kn, int k, int n);

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_PACK_H */
