/* Include-path shim: reference callers write #include "host/session.h"
 * (reference src/host/test.c:11, src/host/op_export.c:3); with
 * -I include/htp_ops that line resolves here. */
#ifndef HTP_OPS_HOST_SESSION_SHIM_H
#define HTP_OPS_HOST_SESSION_SHIM_H
#include "../session.h"
#endif
