/* Compiled by tests/test_abi.py against include/htp_ops: reports this
 * library's wire-ABI sizes and offsets with the same numbering as
 * oracle/ref_abi.c reports the reference's. */
#include <stddef.h>
#include <stdint.h>

#include "htp_ops/message.h"
#include "htp_ops/op_reg.h"

size_t own_abi_size(int which) {
  switch (which) {
    case 0: return sizeof(struct MessageHeader);
    case 1: return sizeof(struct RequestHeader);
    case 2: return sizeof(struct OpComputeRequest);
    case 3: return sizeof(struct RpcmemBufAddr);
    case 4: return sizeof(struct W8A8Header);
    case 5: return sizeof(struct NativeW8A8Params);
    case 6: return sizeof(struct NativeW8A8Profile);
    case 7: return sizeof(struct NativeW8A8ProfileParams);
    case 8: return sizeof(struct W8A8CpuControl);
    case 9: return sizeof(struct NativeW8A8CpuParams);
    case 10: return sizeof(struct MatMulParams);
    case 11: return sizeof(struct F16EpilogueParams);
    case 12: return sizeof(struct RpcmemMapRequest);
    case 13: return sizeof(struct RpcmemMapEntryV2);
    case 14: return sizeof(struct RpcmemMapRequestV2);
    case 15: return sizeof(struct W8A8CpuBatch);
    case 16: return sizeof(struct NativeAuxParams);
    case 17: return sizeof(struct QkvMulRmsPackedParams);
    case 18: return sizeof(struct QkvMulRmsPackedDualParams);
    case 19: return sizeof(struct QkvMulRmsPackedRopeParams);
    case 20: return sizeof(struct QkvMulRmsPackedDualRopeParams);
    default: return 0;
  }
}

size_t own_abi_offset(int which) {
  switch (which) {
    case 0: return offsetof(struct NativeW8A8Params, m);
    case 1: return offsetof(struct NativeW8A8Params, elapsed_us);
    case 2: return offsetof(struct F16EpilogueParams, m);
    case 3: return offsetof(struct F16EpilogueParams, mode);
    case 4: return offsetof(struct F16EpilogueParams, elapsed_us);
    case 5: return offsetof(struct MatMulParams, m);
    case 6: return offsetof(struct MatMulParams, debug_dsp_output_hash_after_invalidate);
    case 7: return offsetof(struct W8A8Header, original_f16_signature);
    case 8: return offsetof(struct W8A8CpuControl, scales);
    case 9: return offsetof(struct W8A8CpuControl, batches);
    case 10: return offsetof(struct W8A8CpuControl, resident_batch_rows);
    case 11: return offsetof(struct NativeW8A8CpuParams, control);
    case 12: return offsetof(struct RpcmemMapRequestV2, entries);
    case 13: return offsetof(struct W8A8Header, inverse_offset);
    case 14: return offsetof(struct NativeAuxParams, mode);
    case 15: return offsetof(struct NativeAuxParams, eps);
    case 16: return offsetof(struct NativeAuxParams, elapsed_us);
    case 17: return offsetof(struct QkvMulRmsPackedParams, tokens);
    case 18: return offsetof(struct QkvMulRmsPackedParams, elapsed_us);
    case 19: return offsetof(struct QkvMulRmsPackedDualParams, text_activation);
    case 20: return offsetof(struct QkvMulRmsPackedDualParams, elapsed_us);
    case 21: return offsetof(struct QkvMulRmsPackedRopeParams, rope_pe);
    case 22: return offsetof(struct QkvMulRmsPackedRopeParams, rope_token_count);
    case 23: return offsetof(struct QkvMulRmsPackedDualRopeParams, rope_pe);
    case 24: return offsetof(struct QkvMulRmsPackedDualRopeParams, text_rope_token_offset);
    default: return (size_t)-1;
  }
}

int own_opcode(int which) {
  switch (which) {
    case 0: return HTP_OPS_MAT_MUL_PERMUTED_W16A32;
    case 1: return HTP_OPS_MAT_MUL_NATIVE_W8A8;
    case 2: return HTP_OPS_MAT_MUL_F16_EPILOGUE;
    case 3: return HTP_OPS_COUNT;
    case 4: return REQUEST_TYPE_OP_COMPUTE;
    case 5: return REQUEST_TYPE_RPCMEM_MAP;
    case 6: return HTP_OPS_MODEL_AUX_F32;
    case 7: return HTP_OPS_QKV_MUL_RMS_PACKED_W16A32;
    case 8: return HTP_OPS_QKV_MUL_RMS_PACKED_DUAL_W16A32;
    case 9: return HTP_OPS_QKV_MUL_RMS_PACKED_ROPE_W16A32;
    case 10: return HTP_OPS_QKV_MUL_RMS_PACKED_DUAL_ROPE_W16A32;
    default: return -1;
  }
}

/* The packed QKV opcodes' head-shape rule. */
int own_packed_shape_supported(int n_heads, int n_kv_heads, int head_dim, int require_equal_kv) {
  return htp_packed_shape_supported(n_heads, n_kv_heads, head_dim, require_equal_kv) ? 1 : 0;
}

int own_message_header_validate_layout(const void *h, size_t capacity, size_t *total_size) {
  return message_header_validate_layout((const struct MessageHeader *)h, capacity, total_size);
}
