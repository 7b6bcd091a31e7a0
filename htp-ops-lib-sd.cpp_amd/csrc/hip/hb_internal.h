// Internal helpers shared by the hb_* translation units (not installed).
#ifndef HB_INTERNAL_H
#define HB_INTERNAL_H

#include <hip/hip_runtime.h>

#include "htp_ops/hb.h"

int hb_fail(hipError_t err, const char *what);
int hb_invalid(const char *what);
hipStream_t hb_resolve_stream(hb_stream s);

// Returns the launch status of the last kernel as an hb status code.
static inline int hb_check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? HB_OK : hb_fail(err, what);
}

typedef int hb_i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int hb_u32x4 __attribute__((ext_vector_type(4)));
typedef float hb_f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 hb_f16x8 __attribute__((ext_vector_type(8)));

static inline size_t hb_round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

#endif  // HB_INTERNAL_H
