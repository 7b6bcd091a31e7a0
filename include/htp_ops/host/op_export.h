/* Include-path shim: reference callers write #include "host/op_export.h"
 * (reference src/host/op_export.c:1); with -I include/htp_ops that line
 * resolves here. */
#ifndef HTP_OPS_HOST_OP_EXPORT_SHIM_H
#define HTP_OPS_HOST_OP_EXPORT_SHIM_H
#include "../op_export.h"
#endif
