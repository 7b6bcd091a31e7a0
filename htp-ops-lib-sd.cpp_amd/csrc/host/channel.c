/*
 * Mailbox channel: a receiver thread polls the shared message buffer, runs
 * every request of a posted message in order and publishes completion.
 *
 * Protocol and request handling follow reference src/dsp/commu.c:99-268:
 *   - the state word is loaded with acquire semantics; a message is pending
 *     when v[0] != 0 and v[1] == 0;
 *   - an invalid layout executes nothing but still completes;
 *   - OP_COMPUTE requests return AEE_EBADSTATE while the backend is
 *     mapping-only, else execute_op_simple's code;
 *   - RPCMEM_MAP V1 releases n_puts fds; V2 checks the session token, then
 *     releases n_puts and resolves n_gets views (any failure -> -1);
 *   - completion stores v[0] | 1 << 8 into the state word with release
 *     semantics, after every output is host-visible; requests on HBM
 *     tensors are synchronised once per message, not once each.
 */
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "host_internal.h"
#include "htp_ops/executor.h"

struct htp_channel {
  pthread_t thread;
  htp_backend *backend;
  uint8_t *msg;
  size_t capacity;
  uint64_t token;
  atomic_int stop;
};

static void set_state(struct RequestHeader *r, int32_t v) { memcpy(&r->state, &v, sizeof(v)); }

static void process_map(struct RequestHeader *r, size_t data_size, uint64_t token) {
  if (data_size < sizeof(struct RpcmemMapRequest)) {
    set_state(r, -1);
    return;
  }
  int32_t state = 0;
  /* a put frees device mirrors and cached weight images that queued work of
   * earlier requests in this message may still read */
  if (htp_executor_flush() != 0) {
    set_state(r, -1);
    return;
  }
  const struct RpcmemMapRequestV2 *v2 = (const struct RpcmemMapRequestV2 *)r->data;
  const int is_v2 = data_size >= sizeof(struct RpcmemMapRequestV2) && v2->magic == RPCMEM_MAP_REQUEST_SESSION_MAGIC &&
                    v2->version == RPCMEM_MAP_REQUEST_VERSION_SESSION;
  if (is_v2) {
    const size_t available = (data_size - sizeof(*v2)) / sizeof(struct RpcmemMapEntryV2);
    if (v2->header_size < sizeof(*v2) || v2->n_puts < 0 || v2->n_gets < 0 || v2->session_token != token ||
        (size_t)v2->n_puts + (size_t)v2->n_gets > available) {
      set_state(r, -1);
      return;
    }
    for (int32_t j = 0; j < v2->n_puts && state == 0; ++j) {
      struct RpcmemMapEntryV2 e;
      memcpy(&e, &v2->entries[j], sizeof(e));
      if (htp_registry_put(e.fd) != 0) state = -1;
    }
    for (int32_t j = 0; j < v2->n_gets && state == 0; ++j) {
      struct RpcmemMapEntryV2 e;
      memcpy(&e, &v2->entries[v2->n_puts + j], sizeof(e));
      htp_view v;
      if (e.offset > (uint64_t)INT64_MAX || htp_registry_host_view(e.fd, (int64_t)e.offset, (size_t)e.size, &v) != 0)
        state = -1;
    }
  } else {
    const struct RpcmemMapRequest *v1 = (const struct RpcmemMapRequest *)r->data;
    const size_t available = (data_size - sizeof(*v1)) / sizeof(int32_t);
    if (v1->n_puts < 0 || v1->n_gets < 0 || (size_t)v1->n_puts > available ||
        (size_t)v1->n_gets > available - (size_t)v1->n_puts) {
      set_state(r, -1);
      return;
    }
    for (int32_t j = 0; j < v1->n_puts; ++j) {
      int32_t fd;
      memcpy(&fd, &v1->fds[j], sizeof(fd));
      (void)htp_registry_put(fd); /* unknown fds are ignored, as a repeated put is */
    }
  }
  set_state(r, state);
}

void htp_channel_process(htp_backend *backend, struct MessageHeader *msg, size_t capacity, uint64_t token) {
  size_t used = 0;
  if (!message_header_validate_layout(msg, capacity, &used)) return;
  htp_executor_message_begin();
  for (int32_t i = 0; i < msg->n_reqs; ++i) {
    const size_t wire = (size_t)msg->req_offsets[i + 1] - (size_t)msg->req_offsets[i];
    const size_t data_size = wire - sizeof(struct RequestHeader);
    struct RequestHeader *r = message_header_get_request_ptr(msg, i);
    int32_t type;
    memcpy(&type, &r->type, sizeof(type));
    switch (type) {
      case REQUEST_TYPE_OP_COMPUTE:
        if (backend && !htp_backend_compute_allowed(backend)) {
          set_state(r, AEE_EBADSTATE);
        } else {
          set_state(r, htp_executor_message_request((struct OpComputeRequest *)r->data, data_size, &r->state));
        }
        break;
      case REQUEST_TYPE_RPCMEM_MAP: process_map(r, data_size, token); break;
      default: break;
    }
  }
  /* one synchronisation for the message: every output is host-visible
   * before the caller sees the completion flag */
  (void)htp_executor_message_end();
}

static void backoff(unsigned *idle) {
  if (*idle < 4096) {
    ++*idle;
    sched_yield();
    return;
  }
  struct timespec ts = {0, *idle < 65536 ? 2000 : 20000};
  if (*idle < 65536) ++*idle;
  nanosleep(&ts, NULL);
}

static void *receiver_loop(void *arg) {
  htp_channel *c = (htp_channel *)arg;
  (void)htp_executor_ensure_device(); /* compute requests report -5 if this failed */
  uint64_t *word = (uint64_t *)(void *)c->msg;
  unsigned idle = 0;
  while (!atomic_load_explicit(&c->stop, memory_order_acquire)) {
    const uint64_t d = __atomic_load_n(word, __ATOMIC_ACQUIRE);
    const uint8_t v0 = (uint8_t)(d & 0xffu), v1 = (uint8_t)((d >> 8) & 0xffu);
    if (v0 == 0 || v1 != 0) {
      backoff(&idle);
      continue;
    }
    idle = 0;
    htp_channel_process(c->backend, (struct MessageHeader *)c->msg, c->capacity, c->token);
    __atomic_store_n(word, (uint64_t)v0 | (1ull << 8), __ATOMIC_RELEASE);
  }
  return NULL;
}

int htp_channel_start(htp_channel **out, htp_backend *backend, uint8_t *msg, size_t capacity, uint64_t token) {
  htp_channel *c = (htp_channel *)calloc(1, sizeof(*c));
  if (!c) return -1;
  c->backend = backend;
  c->msg = msg;
  c->capacity = capacity;
  c->token = token;
  atomic_init(&c->stop, 0);
  memset(msg, 0, capacity);
  if (pthread_create(&c->thread, NULL, receiver_loop, c) != 0) {
    free(c);
    return -1;
  }
  *out = c;
  return 0;
}

void htp_channel_stop(htp_channel *c) {
  if (!c) return;
  atomic_store_explicit(&c->stop, 1, memory_order_release);
  pthread_join(c->thread, NULL);
  free(c);
}
