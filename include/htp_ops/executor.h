/*
 * Request executor: the in-process counterpart of the reference's DSP-side
 * dispatcher, same entry point and return codes.
 *
 *   execute_op_simple   reference include/dsp/op_executor.h:32, src/dsp/op_executor.cc:274-1118
 *     opcode 15 (W8A8)  reference src/dsp/op_executor.cc:314-353
 *     opcode 16 (F16+epilogue) reference src/dsp/op_executor.cc:446-471
 *     opcode 1  (F16)   reference src/dsp/op_executor.cc:473-540
 *     opcode 19 (model auxiliary f32 ops) reference src/dsp/op_executor.cc:371-404
 *     opcodes 2/3/4 (Q4_0 / Q8_0 / IQ4_NL weights, F16 GEMM)
 *                       reference src/dsp/op_executor.cc:771-800
 *     opcodes 8/10/11/12 (fused QKV + RMS norm (+ RoPE), packed fp16 outputs)
 *                       reference src/dsp/op_executor.cc:542-770
 *
 * Return codes (unchanged from the reference):
 *   opcode 15: -1 payload size / shape / profile mode, -2 unmapped buffer,
 *              -3 constants header mismatch, -10 kernel argument error,
 *              -12 CPU-control batch overflow.
 *   opcode 16: -1 validation or unmapped buffer, -10/-11/-12 kernel argument errors.
 *   opcode 1:  -1 short payload, -2 unmapped buffer, -3 misaligned buffer (128 B).
 *   opcodes 2/3/4: -1 short payload, unmapped buffer, zero dimension, k or n
 *              not a multiple of 32, misaligned buffer (128 B).
 *   opcode 19: -1 payload size / validation / unmapped buffer, -40 a norm with
 *              no whole row (the reference's empty worker pool).
 *   opcodes 8/10/11/12: -1 payload size, unsupported shape (heads 24/30/38,
 *              head_dim 64/128, 38 heads only with 64), input_dim not a multiple of
 *              32, a required buffer unmapped, q/k/v/activation/weight not 128-byte
 *              aligned, dual requests with image_tokens not a multiple of 32 or no
 *              text tokens, negative rotary offsets or count.
 *   other opcodes: HTP_OPS_E_UNSUPPORTED (the reference silently returns 0).
 *   A GPU runtime failure while executing a valid request returns -5.
 * All argument checks happen before any GPU work is queued.
 */
#ifndef HTP_OPS_EXECUTOR_H
#define HTP_OPS_EXECUTOR_H

#include <stddef.h>
#include <stdint.h>

#include "message.h"
#include "op_reg.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Executes one compute request in place: req points at the OpComputeRequest,
 * req_size counts the opcode word plus the payload.  Output tensors are
 * host-visible when this returns. */
int execute_op_simple(struct OpComputeRequest *req, size_t req_size);

/* Executes every request of a mailbox message in order, exactly as the
 * channel thread does, without touching the state word.  Returns 0 when the
 * layout is valid (per-request codes are in each RequestHeader.state) and -1
 * when the layout is invalid (nothing executed). */
int htp_ops_execute_message(struct MessageHeader *msg, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_EXECUTOR_H */
