/*
 * A caller written against the reference's headers, include lines unchanged
 * (reference src/host/test.c:2-14): it compiles with -I include/htp_ops and
 * links against libhtp_ops.so alone.  Run on the CPU it exercises only calls
 * that need no GPU.
 */
#include <remote.h>
#include <rpcmem.h>
#include <stdio.h>
#include <string.h>

#include "host/op_export.h"
#include "host/session.h"
#include "htp_ops.h"
#include "message.h"
#include "op_reg.h"

int main(void) {
  struct NativeW8A8Params p;
  memset(&p, 0, sizeof(p));
  remote_handle64 h = 0;
  (void)h;
  printf("%d %d %d %d\n", (int)sizeof(p), (int)sizeof(struct F16EpilogueParams), HTP_OPS_MAT_MUL_NATIVE_W8A8,
         htp_ops_f16_epilogue_version());
  return 0;
}
