/*
 * CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.
 *
 * A portable C11 restatement of the reference's arithmetic for opcodes 15, 16
 * and 1.  It is linked only by tests/, __graft_entry__.smoke() (as the checker)
 * and bench.py's cpu_baseline leg; the product library never calls it.
 *
 * Floating point is IEEE-754 binary32 with round-to-nearest-even on every
 * operation and no contraction (build with -ffp-contract=off, no fast-math).
 * The reference performs the same steps in Hexagon QFloat followed by IEEE
 * conversion; the bit-level QFloat rounding is not observable from the
 * reference's own tests, so the reference contract is defined as IEEE per
 * operation (see the per-function notes in htp_oracle.c).
 *
 * Parity status of each function (what pins it; tests/test_oracle.py,
 * tests/test_abi.py, tests/test_golden.py):
 *   f32<->f16                 pinned: exhaustive against numpy's binary16.
 *   blob pack/unpack/offset,  pinned: the reference's address formula
 *   check_header                (linear_w8a8.c:453,482,486-488, study_dsp.c:82-84),
 *                               bijection, one-hot and round-trip tests, the
 *                               header rule of op_executor.cc:331-335.
 *   accumulate                pinned: int64 brute force, one-hot, the boundary
 *                               targets of integer_tests.c:97, the study data
 *                               expectation of study_host.c:11-15.
 *   quantize_value(s),        pinned to the IEEE-per-operation definition:
 *   quantize, output, linear    closed forms, ties-to-even and clamp special
 *                               cases, exhaustive rintf comparison, numpy float32
 *                               restatements.  Parity unpinned against the
 *                               reference hardware's QFloat rounding (no test of
 *                               the reference observes it).
 *   planes                    pinned: reassembly of the byte planes into the
 *                               accumulator (layout of linear_w8a8.c:209-227).
 *   gelu_tanh, quick_gelu     pinned to the closed forms in double within the
 *                               2e-3 bound; parity unpinned against the
 *                               reference's HVX exp2 polynomial (hvx_math.h:526-613).
 *   f16_permute/_index        pinned: the writer formula of test.c:551-556, one-hot.
 *   f16_gemm_epilogue         pinned: float64 brute force, all-ones gives K,
 *                               one-hot; parity unpinned against the HMX FP16
 *                               accumulation order and precision (mat_mul.c:724-748).
 *   qk0_value/_dequant        pinned: a model of the HVX instructions the
 *                               reference uses, run through the reference's
 *                               single-group path, reproduces ggml's published
 *                               Q4_0/Q8_0/IQ4_NL group order; the same model run
 *                               through the super-block path equals this
 *                               restatement; scale-one blocks give the codes
 *                               exactly.  Parity unpinned against the sd.cpp
 *                               packer (absent) and the qf16 product rounding.
 *   qkv_index                 pinned: a model of the HVX instructions of the
 *                               packing steps (wsf_to_vhf interleave, vdeal,
 *                               vshuff, vscatter byte offsets) run on a matrix
 *                               of distinct values equals these positions.
 *   qkv_rsqrt                 pinned: within 2 ulp of 1/sqrt in double over
 *                               the normal range, and the magic-constant start
 *                               (three Newton steps from 0x5f3759df, each an
 *                               IEEE operation); parity unpinned against the
 *                               QFloat steps of mat_mul.c:1137-1165.
 *   qkv_post                  pinned: float64 closed forms (normalized rows
 *                               have RMS gamma within the fp16 bound, bias
 *                               only shifts V, identity rotary matrices keep
 *                               Q/K, rotations keep pair norms); parity unpinned
 *                               against the QFloat rounding of the bias add,
 *                               sum of squares and scaling.
 */
#ifndef HTP_ORACLE_H
#define HTP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- binary16 ------------------------------------------------------------ */
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
void oracle_f32_to_f16_array(uint16_t *dst, const float *src, size_t count);
void oracle_f16_to_f32_array(float *dst, const uint16_t *src, size_t count);

/* ---- W8A8 constants blob ---------------------------------------------------- */
size_t oracle_w8a8_blob_bytes(int k, int n);
size_t oracle_w8a8_weight_offset(int k, int n_idx, int k_idx);
/* w: int8 [n][k]; sums == NULL -> sum_k w; inv == NULL -> 1.0f. */
void oracle_w8a8_pack_blob(uint8_t *blob, const int8_t *w, const float *sw, const int32_t *sums,
                           const float *inv, int k, int n, uint64_t signature);
void oracle_w8a8_unpack_weights(int8_t *w, const uint8_t *blob, int k, int n);
int oracle_w8a8_check_header(const uint8_t *blob, int k, int n);

/* ---- W8A8 arithmetic -------------------------------------------------------- */
uint8_t oracle_w8a8_quantize_value(float v);
void oracle_w8a8_quantize_values(uint8_t *dst, const float *v, size_t count);
void oracle_w8a8_quantize(uint8_t *u, float *s, const float *x, const float *inv, int m, int k, int nthreads);
void oracle_w8a8_accumulate(int32_t *acc, const uint8_t *u, const uint8_t *blob, int m, int k, int n,
                            int nthreads);
void oracle_w8a8_output(float *y, const int32_t *acc, const float *s, const uint8_t *blob, int m, int k, int n,
                        int nthreads);
void oracle_w8a8_linear(float *y, const float *x, const uint8_t *blob, int m, int k, int n, int nthreads);
void oracle_w8a8_planes(uint8_t *out, const int32_t *acc, int m, int n);

/* ---- epilogues ----------------------------------------------------------- */
float oracle_gelu_tanh(float z);
float oracle_quick_gelu(float z);
void oracle_gelu_tanh_inplace(float *y, size_t count);
float oracle_silu(float z);

/* ---- opcode 19 model auxiliary ops ---------------------------------------- */
int oracle_model_aux(float *y, const float *x, const float *w, const float *b, int mode, int count, int width,
                     int channels, int spatial, int groups, int batch, int other_count, int activation, float eps);

/* ---- packed F16 GEMM -------------------------------------------------------- */
size_t oracle_f16_permuted_index(int k_total, int k_idx, int n_idx);
/* Dequantizing GEMM (opcodes 2/3/4); types are ggml's (reference
 * include/dsp/quants.h:33-54). */
enum { ORACLE_GGML_Q4_0 = 2, ORACLE_GGML_Q8_0 = 8, ORACLE_GGML_IQ4_NL = 20 };
size_t oracle_qk0_block_bytes(int type);
uint16_t oracle_qk0_value(const uint8_t *block, int j, int type);
int oracle_qk0_dequant(uint16_t *permuted, const uint8_t *blocks, int k, int n, int type);
void oracle_f16_permute(uint16_t *permuted, const uint16_t *w_kn, int k, int n);
void oracle_f16_gemm_epilogue(float *y, const float *x, const uint16_t *permuted, const float *bias, int m, int k,
                              int n, int channels, int mode, int nthreads);

/* ---- fused QKV + RMS + RoPE packing (opcodes 8/10/11/12) -------------------- */
/* which: 0 = Q, 1 = K, 2 = V; halfword index inside one head's region. */
size_t oracle_qkv_index(int which, int token_tiles, int head_dim, int tt, int r, int c);
float oracle_qkv_rsqrt(float x);
void oracle_qkv_post(uint16_t *q, uint16_t *k, uint16_t *v, const float *raw, const float *bias, const float *q_norm,
                     const float *k_norm, const float *pe, int rope_token_offset, int rope_token_count, int tokens,
                     int n_heads, int head_dim, int output_token_tiles, int output_token_offset);

/* ---- deterministic inputs --------------------------------------------------- */
uint64_t oracle_splitmix64(uint64_t *state);
void oracle_fill_normal(float *dst, size_t count, float mean, float stddev, uint64_t seed);
void oracle_fill_uniform(float *dst, size_t count, float lo, float hi, uint64_t seed);
void oracle_fill_int8(int8_t *dst, size_t count, int lo, int hi, uint64_t seed);

int oracle_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* HTP_ORACLE_H */
