/*
 * Backend lifecycle (the reference's FastRPC skeleton entry points, here plain
 * C functions on the host).  Each htp_ops_open creates a backend instance; the
 * returned handle names it.  State machine and return codes follow reference
 * src/dsp/commu.c:369-576 (open/close, init_backend[_fraction],
 * init_mapping_backend, release_backend, create/destroy_channel); the direct
 * W16 GEMM entry points follow reference src/dsp/commu.c:637-797 and
 * htp_ops_test_ops reference src/dsp/commu.c:813-827.
 */
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "host_internal.h"
#include "htp_ops/executor.h"
#include "htp_ops/htp_ops.h"
#include "htp_ops/op_reg.h"

int htp_exec_matmul_w16a32(const struct MatMulParams *p, int32_t *elapsed_us, uint64_t *act_hash,
                           uint64_t *out_hash);

struct htp_backend {
  int initialized;
  int mapping_only;
  htp_channel *channel;
};

#define MAX_BACKENDS 64
static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static htp_backend *g_live[MAX_BACKENDS];

int htp_backend_device(void) {
  const char *v = getenv("HTP_OPS_AMD_DEVICE");
  return v && *v ? atoi(v) : 0;
}

htp_backend *htp_backend_from_handle(remote_handle64 handle) {
  htp_backend *found = NULL;
  pthread_mutex_lock(&g_lock);
  for (int i = 0; i < MAX_BACKENDS; ++i)
    if (g_live[i] && (remote_handle64)(uintptr_t)g_live[i] == handle) found = g_live[i];
  pthread_mutex_unlock(&g_lock);
  return found;
}

int htp_backend_compute_allowed(const htp_backend *b) { return b && !b->mapping_only; }

static AEEResult require_initialized(htp_backend *b) {
  return b && b->initialized ? AEE_SUCCESS : AEE_EBADSTATE;
}

AEEResult htp_ops_open(const char *uri, remote_handle64 *handle) {
  (void)uri;
  if (!handle) return AEE_EBADPARM;
  htp_backend *b = (htp_backend *)calloc(1, sizeof(*b));
  if (!b) return AEE_ENOMEMORY;
  pthread_mutex_lock(&g_lock);
  int slot = -1;
  for (int i = 0; i < MAX_BACKENDS && slot < 0; ++i)
    if (!g_live[i]) slot = i;
  if (slot >= 0) g_live[slot] = b;
  pthread_mutex_unlock(&g_lock);
  if (slot < 0) {
    free(b);
    return AEE_ENOMEMORY;
  }
  *handle = (remote_handle64)(uintptr_t)b;
  return AEE_SUCCESS;
}

AEEResult htp_ops_close(remote_handle64 handle) {
  htp_backend *b = htp_backend_from_handle(handle);
  if (!b) return AEE_EBADSTATE;
  htp_channel_stop(b->channel);
  pthread_mutex_lock(&g_lock);
  for (int i = 0; i < MAX_BACKENDS; ++i)
    if (g_live[i] == b) g_live[i] = NULL;
  pthread_mutex_unlock(&g_lock);
  free(b);
  return AEE_SUCCESS;
}

static AEEResult bring_up(htp_backend *b) {
  if (htp_executor_ensure_device() != 0) return AEE_EFAILED;
  b->initialized = 1;
  b->mapping_only = 0;
  return AEE_SUCCESS;
}

AEEResult htp_ops_init_backend(remote_handle64 handle) {
  htp_backend *b = htp_backend_from_handle(handle);
  if (!b) return AEE_EBADSTATE;
  if (b->initialized && !b->mapping_only) return AEE_SUCCESS;
  b->initialized = 0;
  return bring_up(b);
}

AEEResult htp_ops_init_backend_fraction(remote_handle64 handle, uint32_t numerator, uint32_t denominator) {
  htp_backend *b = htp_backend_from_handle(handle);
  if (!b) return AEE_EBADSTATE;
  if (b->initialized) return AEE_SUCCESS;
  if (numerator == 0 || denominator == 0 || numerator > denominator) return AEE_EBADPARM;
  /* The fraction sized the DSP scratchpad share; HBM needs no partitioning. */
  return bring_up(b);
}

AEEResult htp_ops_init_mapping_backend(remote_handle64 handle) {
  htp_backend *b = htp_backend_from_handle(handle);
  if (!b) return AEE_EBADSTATE;
  if (b->initialized) return AEE_SUCCESS;
  b->initialized = 1;
  b->mapping_only = 1;
  return AEE_SUCCESS;
}

AEEResult htp_ops_release_backend(remote_handle64 handle) {
  htp_backend *b = htp_backend_from_handle(handle);
  if (!b) return AEE_EBADSTATE;
  b->initialized = 0;
  b->mapping_only = 1;
  return AEE_SUCCESS;
}

static AEEResult create_channel(remote_handle64 handle, int32_t fd, uint32_t size, uint64_t token) {
  htp_backend *b = htp_backend_from_handle(handle);
  if (require_initialized(b) != AEE_SUCCESS) return AEE_EBADSTATE;
  if (b->channel) return AEE_EALREADY;
  htp_view v;
  if (size < sizeof(struct MessageHeader) + sizeof(int32_t) || htp_registry_host_view(fd, 0, size, &v) != 0 ||
      !v.host)
    return -1;
  htp_channel *c = NULL;
  if (htp_channel_start(&c, b, v.host, size, token) != 0) return -1;
  b->channel = c;
  return AEE_SUCCESS;
}

AEEResult htp_ops_create_channel(remote_handle64 handle, int32_t fd, uint32_t size) {
  return create_channel(handle, fd, size, 0);
}

AEEResult htp_ops_create_channel_with_token(remote_handle64 handle, uint64_t session_token, int32_t fd,
                                            uint32_t size) {
  return create_channel(handle, fd, size, session_token);
}

AEEResult htp_ops_destroy_channel(remote_handle64 handle) {
  htp_backend *b = htp_backend_from_handle(handle);
  if (!b || !b->channel) return AEE_SUCCESS;
  htp_channel_stop(b->channel);
  b->channel = NULL;
  return AEE_SUCCESS;
}

AEEResult htp_ops_rms_norm_f32(remote_handle64 handle, int32_t fd0, int32_t offset0, int32_t fd1, int32_t offset1,
                               int32_t ne0, int32_t ne1) {
  (void)fd0;
  (void)offset0;
  (void)fd1;
  (void)offset1;
  (void)ne0;
  (void)ne1;
  if (require_initialized(htp_backend_from_handle(handle)) != AEE_SUCCESS) return AEE_EBADSTATE;
  return AEE_EUNSUPPORTED;
}

static struct MatMulParams matmul_params(int32_t output_fd, int32_t output_offset, int32_t activation_fd,
                                         int32_t activation_offset, int32_t weight_fd, int32_t weight_offset,
                                         int32_t m, int32_t k, int32_t n) {
  struct MatMulParams p;
  memset(&p, 0, sizeof(p));
  p.output.fd = output_fd;
  p.output.offset = output_offset;
  p.activation.fd = activation_fd;
  p.activation.offset = activation_offset;
  p.weight.fd = weight_fd;
  p.weight.offset = weight_offset;
  p.m = m;
  p.k = k;
  p.n = n;
  return p;
}

AEEResult htp_ops_mat_mul_permuted_w16a32(remote_handle64 handle, int32_t output_fd, int32_t output_offset,
                                          int32_t activation_fd, int32_t activation_offset, int32_t weight_fd,
                                          int32_t weight_offset, int32_t m, int32_t k, int32_t n) {
  if (require_initialized(htp_backend_from_handle(handle)) != AEE_SUCCESS) return AEE_EBADSTATE;
  const struct MatMulParams p =
      matmul_params(output_fd, output_offset, activation_fd, activation_offset, weight_fd, weight_offset, m, k, n);
  return htp_exec_matmul_w16a32(&p, NULL, NULL, NULL);
}

AEEResult htp_ops_mat_mul_permuted_w16a32_trace(remote_handle64 handle, int32_t output_fd, int32_t output_offset,
                                                int32_t activation_fd, int32_t activation_offset,
                                                int32_t weight_fd, int32_t weight_offset, int32_t m, int32_t k,
                                                int32_t n, uint64_t *activation_hash, uint64_t *output_hash,
                                                uint64_t *output_hash_after_remap) {
  if (require_initialized(htp_backend_from_handle(handle)) != AEE_SUCCESS) return AEE_EBADSTATE;
  if (activation_hash) *activation_hash = 0;
  if (output_hash) *output_hash = 0;
  if (output_hash_after_remap) *output_hash_after_remap = 0;
  const struct MatMulParams p =
      matmul_params(output_fd, output_offset, activation_fd, activation_offset, weight_fd, weight_offset, m, k, n);
  uint64_t ah = 0, oh = 0;
  const int rc = htp_exec_matmul_w16a32(&p, NULL, &ah, &oh);
  if (activation_hash) *activation_hash = ah;
  if (output_hash) *output_hash = oh;
  if (rc == 0 && output_hash_after_remap) {
    /* Re-resolve the output after dropping the fd's device state: the bytes
     * the host sees must be unchanged. */
    htp_view v;
    if (htp_registry_host_view(output_fd, output_offset, (size_t)m * n * 4u, &v) == 0 && v.host)
      *output_hash_after_remap = htp_fnv1a64(v.host, v.bytes);
  }
  return rc;
}

/* Host-side contract checks run by htp_ops_test_ops, on the model of the
 * reference's DSP self-tests (reference src/dsp/op_tests.cc:158-361, 606-649). */
static int self_tests(void) {
  int failures = 0;
  /* Mailbox layout validation cases. */
  uint8_t storage[128] __attribute__((aligned(8)));
  struct MessageHeader *msg = (struct MessageHeader *)storage;
  size_t total = 0;
#define SET_VALID()                                                             \
  do {                                                                          \
    memset(storage, 0, sizeof(storage));                                        \
    msg->n_reqs = 2;                                                            \
    msg->req_offsets[0] = (int32_t)message_header_size(msg);                    \
    msg->req_offsets[1] = msg->req_offsets[0] + (int32_t)sizeof(struct RequestHeader); \
    msg->req_offsets[2] = msg->req_offsets[1] + (int32_t)sizeof(struct RequestHeader); \
  } while (0)
  SET_VALID();
  failures += !message_header_validate_layout(msg, sizeof(storage), &total);
  failures += total != (size_t)msg->req_offsets[2];
  SET_VALID();
  msg->n_reqs = -1;
  failures += message_header_validate_layout(msg, sizeof(storage), &total);
  SET_VALID();
  msg->n_reqs = INT32_MAX;
  failures += message_header_validate_layout(msg, sizeof(storage), &total);
  SET_VALID();
  msg->req_offsets[0] = (int32_t)message_header_size(msg) - 1;
  failures += message_header_validate_layout(msg, sizeof(storage), &total);
  SET_VALID();
  msg->req_offsets[1] = msg->req_offsets[0] - 1;
  failures += message_header_validate_layout(msg, sizeof(storage), &total);
  SET_VALID();
  msg->req_offsets[1] = msg->req_offsets[0] + (int32_t)sizeof(struct RequestHeader) - 1;
  failures += message_header_validate_layout(msg, sizeof(storage), &total);
  SET_VALID();
  msg->req_offsets[2] = (int32_t)sizeof(storage) + 1;
  failures += message_header_validate_layout(msg, sizeof(storage), &total);
#undef SET_VALID
  /* Payload boundaries: malformed requests are rejected without writing past
   * the payload (canary bytes stay intact). */
  struct {
    uint8_t request[sizeof(struct OpComputeRequest) + sizeof(struct NativeW8A8ProfileParams)];
    uint8_t canary[64];
  } req;
  const size_t sizes[] = {0, 39, 41, 47, 55, 103};
  const uint32_t ops[] = {HTP_OPS_MAT_MUL_NATIVE_W8A8, HTP_OPS_MAT_MUL_F16_EPILOGUE};
  for (size_t o = 0; o < 2; ++o) {
    for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); ++i) {
      memset(&req, 0xa5, sizeof(req));
      memcpy(req.request, &ops[o], sizeof(ops[o]));
      const size_t len = sizeof(struct OpComputeRequest) + sizes[i];
      failures += execute_op_simple((struct OpComputeRequest *)req.request, len) != -1;
      for (size_t j = 0; j < sizeof(req.canary); ++j) failures += req.canary[j] != 0xa5;
    }
  }
  return failures;
}

AEEResult htp_ops_test_ops(remote_handle64 handle, int32_t *userdma_scope) {
  if (require_initialized(htp_backend_from_handle(handle)) != AEE_SUCCESS) return AEE_EBADSTATE;
  if (!userdma_scope) return AEE_EBADPARM;
  if (self_tests() != 0) return AEE_EFAILED;
  *userdma_scope = 1; /* no shared DMA engine: scope is per worker */
  return AEE_SUCCESS;
}
