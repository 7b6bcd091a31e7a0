/* Include-path shim for the Hexagon SDK's <remote.h> (reference
 * src/host/test.c:2): remote_handle64 and fastrpc_mmap/munmap, as this
 * library defines them (htp_ops.h, rpcmem.h). */
#ifndef HTP_OPS_REMOTE_SHIM_H
#define HTP_OPS_REMOTE_SHIM_H
#include "htp_ops.h"
#include "rpcmem.h"
#endif
