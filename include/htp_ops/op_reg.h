/*
 * Operator registry: opcode numbering and request payloads of the quantized
 * linear path.  The numbering and every payload below are wire ABI shared with
 * existing callers, so they are laid out exactly like the reference:
 *   opcode enum                 reference include/op_reg.h:41-66
 *   RpcmemBufAddr               reference include/op_reg.h:68-71
 *   W8A8 blob header / payloads reference include/op_reg.h:80-149
 *   MatMulParams (opcode 1)     reference include/op_reg.h:151-181
 *   F16EpilogueParams (op 16)   reference include/op_reg.h:477-489
 *   QKV payloads (ops 8/10-12)  reference include/op_reg.h:183-285
 *   NativeAuxParams (op 19)     reference include/op_reg.h:503-507
 *
 * Opcodes 1-4, 8, 10-12, 15, 16 and 19 are executed by this library; every
 * other opcode is answered with HTP_OPS_E_UNSUPPORTED instead of a silent
 * success.
 */
#ifndef HTP_OPS_OP_REG_H
#define HTP_OPS_OP_REG_H

#include <stddef.h>
#include <stdint.h>

#include "message.h"

#ifdef __cplusplus
extern "C" {
#endif

enum HtpOpsIndex {
  HTP_OPS_RMS_NORM_F32 = 0,
  HTP_OPS_MAT_MUL_PERMUTED_W16A32 = 1,
  HTP_OPS_MAT_MUL_PERMUTED_W4D16A32 = 2,
  HTP_OPS_MAT_MUL_PERMUTED_W8D16A32 = 3,
  HTP_OPS_MAT_MUL_PERMUTED_W4D16A32_IQ4_NL = 4,
  HTP_OPS_FLASH_ATTN_QO_F32_KV_F16 = 5,
  HTP_OPS_BLOCK_SPARSE_ATTN_QO_F32_KV_F16 = 6,
  HTP_OPS_BLOCK_SPARSE_SCORE_QO_F32_KM_F16 = 7,
  HTP_OPS_QKV_MUL_RMS_PACKED_W16A32 = 8,
  HTP_OPS_BLOCK_SPARSE_ATTN_QKV_PACKED_F16 = 9,
  HTP_OPS_QKV_MUL_RMS_PACKED_DUAL_W16A32 = 10,
  HTP_OPS_QKV_MUL_RMS_PACKED_ROPE_W16A32 = 11,
  HTP_OPS_QKV_MUL_RMS_PACKED_DUAL_ROPE_W16A32 = 12,
  HTP_OPS_FUSED_ANCHOR_ATTN_QO_F32_KV_F16 = 13,
  HTP_OPS_ATTN_REARRANGE_BENCH = 14,
  HTP_OPS_MAT_MUL_NATIVE_W8A8 = 15,
  HTP_OPS_MAT_MUL_F16_EPILOGUE = 16,
  HTP_OPS_CONV2D_NCHW_F16 = 17,
  HTP_OPS_ATTENTION_F32 = 18,
  HTP_OPS_MODEL_AUX_F32 = 19,
  HTP_OPS_COUNT = 20,
};

/* Return code for opcodes this library does not implement (reference: 0). */
#define HTP_OPS_E_UNSUPPORTED (-95)

/* A tensor is named by the rpcmem fd that owns it and a byte offset in it. */
struct RpcmemBufAddr {
  int32_t fd;
  int32_t offset;
} __attribute__((packed));

/* ---- opcode 15: W8A8 linear ------------------------------------------- */

#define W8A8_BLOB_MAGIC 0x38574d48u /* "HMW8" little-endian */
#define W8A8_BLOB_VERSION 1u
#define W8A8_BLOB_HEADER_BYTES 128u

/*
 * Constants blob = header | int8 weights (HMX deep tiles, k*n bytes) |
 * per-column scale f32[n] | per-column weight sum i32[n] | smoothing f32[k].
 * Weight element W(n,k) lives at byte
 *   128 + (n/64)*64*k + (k/32)*2048 + ((n%64)/32)*1024 + ((k%32)/4)*128 + (n%32)*4 + k%4.
 */
struct W8A8Header {
  uint32_t magic, version, k, n;
  uint32_t weight_offset, scale_offset, sum_offset, inverse_offset, bytes, reserved;
  uint64_t original_f16_signature;
  uint8_t padding[80];
};

struct NativeW8A8Params {
  struct RpcmemBufAddr output, activation, constants;
  int32_t m, k, n, elapsed_us;
} __attribute__((packed));

/* Optional diagnostic trailer (payload 104 bytes). mode 1/2/3 as documented
 * in the executor; ticks are 19.2 MHz units. */
struct NativeW8A8Profile {
  uint32_t mode, reserved;
  uint64_t setup_ticks, activation_ticks, weight_ticks, hmx_ticks, output_ticks;
  uint64_t mac_ticks, readout_ticks;
};
struct NativeW8A8ProfileParams {
  struct NativeW8A8Params base;
  struct NativeW8A8Profile profile;
} __attribute__((packed));

/* CPU-epilogue variant (payload 48 bytes): raw int32 accumulator byte planes
 * are written into the output tensor and progress is published in a control
 * buffer. */
#define W8A8_CPU_MAX_BATCHES 64
#define W8A8_CONTROL_WEIGHT_FIRST 1u
struct W8A8CpuBatch {
  int32_t m0, rows, n0, columns;
};
struct W8A8CpuControl {
  uint32_t produced;
  uint32_t flags;
  uint32_t vtcm_bytes, activation_rows, weight_columns, weight_loads;
  uint64_t weight_loaded_bytes;
  uint32_t resident_batch_rows;
  uint8_t padding[92];
  float scales[4096];
  struct W8A8CpuBatch batches[W8A8_CPU_MAX_BATCHES];
};
struct NativeW8A8CpuParams {
  struct NativeW8A8Params base;
  struct RpcmemBufAddr control;
} __attribute__((packed));

HTP_OPS_STATIC_ASSERT(sizeof(struct W8A8Header) == 128, "W8A8 constants ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct NativeW8A8Params) == 40, "W8A8 message ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct NativeW8A8CpuParams) == 48, "W8A8 CPU message ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct W8A8CpuControl) == 17536, "W8A8 CPU control ABI");
HTP_OPS_STATIC_ASSERT(offsetof(struct W8A8CpuControl, scales) == 128, "W8A8 scale offset");
HTP_OPS_STATIC_ASSERT(offsetof(struct W8A8CpuControl, batches) == 16512, "W8A8 batch offset");
HTP_OPS_STATIC_ASSERT(sizeof(struct NativeW8A8Profile) == 64, "W8A8 profile ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct NativeW8A8ProfileParams) == 104, "W8A8 profile request ABI");

/* ---- opcode 1: packed-F16 GEMM ------------------------------------------ */

/*
 * Permuted FP16 weight: element (k, n) of the logical [k][n] weight is at fp16
 * index ((n/32)*(k_total/32) + k/32)*1024 + ((k%32)/2)*64 + (n%32)*2 + k%2.
 */
struct MatMulParams {
  struct RpcmemBufAddr output;
  struct RpcmemBufAddr activation; /* m * k f32 */
  struct RpcmemBufAddr weight;     /* k * n permuted f16 */
  int32_t m;
  int32_t k;
  int32_t n;
  uint64_t debug_vtcm_base;
  uint32_t debug_vtcm_size;
  int32_t debug_vtcm_ctx;
  int32_t debug_hmx_ctx;
  uint64_t debug_worker_pool;
  int32_t debug_hmx_lock_result;
  uint64_t debug_dsp_activation_hash;
  uint64_t debug_dsp_output_hash;
  uint64_t debug_dsp_output_hash_after_invalidate;
} __attribute__((packed));

struct MatMulProfileParams {
  struct MatMulParams matmul;
  int32_t elapsed_us;
} __attribute__((packed));

HTP_OPS_STATIC_ASSERT(sizeof(struct MatMulParams) == 92, "MatMulParams ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct MatMulProfileParams) == 96, "MatMulProfileParams ABI");

/* ---- opcode 16: packed-F16 GEMM with fused epilogue ---------------------- */

/* mode: 0 = bias, 1 = bias + GELU(tanh form), 2 = bias + QuickGELU,
 *       3 = bias + channel-major store (output [channels][m]). */
enum F16EpilogueMode {
  F16_EPILOGUE_BIAS = 0,
  F16_EPILOGUE_GELU = 1,
  F16_EPILOGUE_QUICK_GELU = 2,
  F16_EPILOGUE_CHANNEL_MAJOR = 3,
};

struct F16EpilogueParams {
  struct RpcmemBufAddr output, activation, weight, bias; /* bias.fd < 0: no bias */
  int32_t m, k, n, channels, mode, elapsed_us;
} __attribute__((packed));

HTP_OPS_STATIC_ASSERT(sizeof(struct F16EpilogueParams) == 56, "F16 epilogue ABI");

/* Opcode 19 payload (reference include/op_reg.h:503-507): model auxiliary f32
 * ops.  weight.fd / bias.fd < 0 mean "absent".  Modes 0-13 as in
 * src/dsp/ops/mat_mul.c:2356-2486 (see hb_model_aux in hb.h). */
struct NativeAuxParams {
  struct RpcmemBufAddr output, input, weight, bias;
  int32_t mode, count, width, channels, spatial, groups, batch, other_count, activation;
  float eps;
  int32_t elapsed_us;
} __attribute__((packed));

HTP_OPS_STATIC_ASSERT(sizeof(struct NativeAuxParams) == 76, "native auxiliary ABI");

/* ---- opcodes 8/10/11/12: fused QKV projection + RMS norm (+ RoPE) ----------
 * (reference include/op_reg.h:23-39 shape rule, :183-285 payloads)
 * The weight is opcode 1's permuted fp16 layout with 3 * n_heads * head_dim
 * columns (Q | K | V); bias has as many floats (fd < 0: none, except for
 * opcode 8), q_norm / k_norm head_dim floats; outputs are fp16 packed tiles
 * of n_heads * ceil(tokens/32) * head_dim * 32 halfwords each. */
static inline int htp_packed_head_count_supported(int n_heads) {
  return n_heads == 24 || n_heads == 30 || n_heads == 38;
}
static inline int htp_packed_head_dim_supported(int head_dim) { return head_dim == 64 || head_dim == 128; }
static inline int htp_packed_shape_supported(int n_heads, int n_kv_heads, int head_dim, int require_equal_kv) {
  return n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && htp_packed_head_count_supported(n_heads) &&
         htp_packed_head_dim_supported(head_dim) && (n_heads != 38 || head_dim == 64) &&
         (!require_equal_kv || (n_heads == n_kv_heads && htp_packed_head_count_supported(n_kv_heads)));
}

struct QkvMulRmsPackedParams {
  struct RpcmemBufAddr q, k_out, v, activation, weight, bias, q_norm, k_norm;
  int32_t tokens, input_dim, n_heads, head_dim, elapsed_us;
} __attribute__((packed));

struct QkvMulRmsPackedDualParams {
  struct RpcmemBufAddr q, k_out, v;
  struct RpcmemBufAddr image_activation, image_weight, image_bias, image_q_norm, image_k_norm;
  struct RpcmemBufAddr text_activation, text_weight, text_bias, text_q_norm, text_k_norm;
  int32_t image_tokens, text_tokens, input_dim, n_heads, head_dim, elapsed_us;
} __attribute__((packed));

/* rope_pe: rope_token_count tokens x head_dim/2 2x2 matrices (4 floats each). */
struct QkvMulRmsPackedRopeParams {
  struct RpcmemBufAddr q, k_out, v, activation, weight, bias, q_norm, k_norm, rope_pe;
  int32_t tokens, input_dim, n_heads, head_dim, rope_token_offset, rope_token_count, elapsed_us;
} __attribute__((packed));

struct QkvMulRmsPackedDualRopeParams {
  struct RpcmemBufAddr q, k_out, v;
  struct RpcmemBufAddr image_activation, image_weight, image_bias, image_q_norm, image_k_norm;
  struct RpcmemBufAddr text_activation, text_weight, text_bias, text_q_norm, text_k_norm;
  struct RpcmemBufAddr rope_pe;
  int32_t image_tokens, text_tokens, input_dim, n_heads, head_dim, image_rope_token_offset, text_rope_token_offset,
      elapsed_us;
} __attribute__((packed));

HTP_OPS_STATIC_ASSERT(sizeof(struct QkvMulRmsPackedParams) == 84, "QKV payload ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct QkvMulRmsPackedDualParams) == 128, "QKV dual payload ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct QkvMulRmsPackedRopeParams) == 100, "QKV RoPE payload ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct QkvMulRmsPackedDualRopeParams) == 144, "QKV dual RoPE payload ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct RpcmemBufAddr) == 8, "RpcmemBufAddr ABI");

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_OP_REG_H */
