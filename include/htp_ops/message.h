/*
 * Shared-memory mailbox wire format between a host process and the executor.
 *
 * Byte-for-byte the same layout as the reference mailbox so that an existing
 * caller (sd.cpp HTP backend, the reference host test) can drive this
 * implementation unchanged:
 *   reference include/message.h:6-66   (structs, request types, map requests)
 *   reference include/message.h:68-113 (layout validation)
 *
 * Protocol (reference src/dsp/commu.c:99-268, src/host/test.c:1121-1144):
 *   host:     state.d = 0; fill n_reqs, req_offsets[], requests; state.v[0] = 1
 *   executor: sees v[0] != 0 && v[1] == 0 (acquire), validates the layout,
 *             runs requests in order writing RequestHeader.state,
 *             then publishes v[1] = 1 (release)
 *   host:     waits for v[1] == 1, reads return codes and in-payload outputs.
 */
#ifndef HTP_OPS_MESSAGE_H
#define HTP_OPS_MESSAGE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
#define HTP_OPS_STATIC_ASSERT(c, m) static_assert(c, m)
extern "C" {
#else
#define HTP_OPS_STATIC_ASSERT(c, m) _Static_assert(c, m)
#endif

/* 8-byte state word: v[0] = request posted by host, v[1] = done by executor. */
struct MessageState {
  union {
    volatile uint8_t v[8];
    volatile uint64_t d;
  };
} __attribute__((packed));

struct MessageHeader {
  struct MessageState state;
  uint32_t checksum;      /* unused by the protocol, kept for layout */
  int32_t n_reqs;
  int32_t req_offsets[]; /* n_reqs + 1 byte offsets from the header start */
} __attribute__((packed));

struct RequestHeader {
  int32_t state; /* executor writes the request's return code here */
  int32_t type;  /* enum RequestType */
  uint8_t data[];
} __attribute__((packed));

enum RequestType {
  REQUEST_TYPE_NO_OP = 0,
  REQUEST_TYPE_RPCMEM_MAP = 1,
  REQUEST_TYPE_OP_COMPUTE = 2,
  REQUEST_TYPE_COUNT = 3,
};

/* Legacy map request: n_puts fds to release, then n_gets fds. */
struct RpcmemMapRequest {
  int32_t n_puts;
  int32_t n_gets;
  int32_t fds[];
} __attribute__((packed));

enum {
  RPCMEM_MAP_REQUEST_VERSION_LEGACY = 1,
  RPCMEM_MAP_REQUEST_VERSION_SESSION = 2,
  RPCMEM_MAP_REQUEST_SESSION_MAGIC = 0x32504d52u, /* "RMP2" */
};

struct RpcmemMapEntryV2 {
  int32_t fd;
  uint32_t role;
  uint64_t offset;
  uint64_t size;
  uint64_t producer_epoch;
} __attribute__((packed));

struct RpcmemMapRequestV2 {
  uint32_t magic;
  uint16_t version;
  uint16_t header_size;
  uint64_t session_token;
  int32_t n_puts;
  int32_t n_gets;
  struct RpcmemMapEntryV2 entries[];
} __attribute__((packed));

struct OpComputeRequest {
  uint32_t op; /* enum HtpOpsIndex */
  uint8_t payload[];
} __attribute__((packed));

HTP_OPS_STATIC_ASSERT(sizeof(struct MessageState) == 8, "MessageState ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct MessageHeader) == 16, "MessageHeader ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct RequestHeader) == 8, "RequestHeader ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct RpcmemMapRequest) == 8, "RpcmemMapRequest ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct RpcmemMapEntryV2) == 32, "RpcmemMapEntryV2 ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct RpcmemMapRequestV2) == 24, "RpcmemMapRequestV2 ABI");
HTP_OPS_STATIC_ASSERT(sizeof(struct OpComputeRequest) == 4, "OpComputeRequest ABI");

/*
 * Returns 1 and the byte size used by the message when every offset lies
 * inside `capacity`, offsets are non-decreasing, the first request starts
 * after the offset table and each request holds at least a RequestHeader.
 * Returns 0 otherwise (the executor then runs nothing but still completes).
 * Same acceptance rule as reference include/message.h:68-113.
 */
static inline int message_header_validate_layout(const struct MessageHeader *h, size_t capacity,
                                                 size_t *total_size) {
  if (h == NULL || total_size == NULL || capacity < sizeof(struct MessageHeader) + sizeof(int32_t)) {
    return 0;
  }
  const int32_t n = h->n_reqs;
  if (n < 0) {
    return 0;
  }
  const size_t table_entries = (size_t)n + 1u;
  if (table_entries > (capacity - sizeof(struct MessageHeader)) / sizeof(int32_t)) {
    return 0;
  }
  const size_t table_end = sizeof(struct MessageHeader) + table_entries * sizeof(int32_t);
  if (h->req_offsets[0] < 0) {
    return 0;
  }
  size_t cursor = (size_t)h->req_offsets[0];
  if (cursor < table_end || cursor > capacity) {
    return 0;
  }
  for (int32_t i = 1; i <= n; ++i) {
    const int32_t wire = h->req_offsets[i];
    if (wire < 0) {
      return 0;
    }
    const size_t next = (size_t)wire;
    if (next < cursor || next > capacity || next - cursor < sizeof(struct RequestHeader)) {
      return 0;
    }
    cursor = next;
  }
  *total_size = cursor;
  return 1;
}

static inline size_t message_header_size(const struct MessageHeader *h) {
  return sizeof(struct MessageHeader) + ((size_t)h->n_reqs + 1u) * sizeof(int32_t);
}

static inline size_t message_total_size(const struct MessageHeader *h) {
  return (size_t)h->req_offsets[h->n_reqs];
}

static inline size_t message_header_get_request_size(const struct MessageHeader *h, int req_idx) {
  return (size_t)(h->req_offsets[req_idx + 1] - h->req_offsets[req_idx]);
}

static inline struct RequestHeader *message_header_get_request_ptr(struct MessageHeader *h, int req_idx) {
  return (struct RequestHeader *)((uintptr_t)h + (uintptr_t)h->req_offsets[req_idx]);
}

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_MESSAGE_H */
