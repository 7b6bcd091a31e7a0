/* Internal declarations shared by the C host library (not installed). */
#ifndef HTP_HOST_INTERNAL_H
#define HTP_HOST_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "htp_ops/hb.h"
#include "htp_ops/htp_ops.h"
#include "htp_ops/message.h"

/* ---- buffer registry (registry.c) --------------------------------------- */

/* A resolved tensor view: host address (NULL for HBM-resident fds) and the
 * device address of the same bytes (HBM storage or the host buffer's mirror). */
typedef struct {
  int fd;
  size_t offset;
  size_t bytes;
  uint8_t *host;
  uint8_t *dev;
  int is_device;
  uint64_t generation;
} htp_view;

/* Resolves [offset, offset+bytes) of a mapped fd; creates the device mirror
 * of a host buffer on first use.  Returns 0, or -1 when the fd is unknown,
 * not mapped, or the range does not fit; -5 when the mirror cannot be made. */
int htp_registry_view(int fd, int64_t offset, size_t bytes, htp_view *out);
/* Same lookup without creating a mirror (host pointer only). */
int htp_registry_host_view(int fd, int64_t offset, size_t bytes, htp_view *out);
/* Drops the device mirror and every cached prepacked weight of an fd (map "put"). */
int htp_registry_put(int fd);
int htp_registry_known(int fd);
/* Records a library write of [offset, offset + bytes) of fd: cached weight
 * images built from overlapping bytes become stale. */
void htp_registry_touch(int fd, size_t offset, size_t bytes);

/* ---- prepacked weight cache (registry.c) -------------------------------- */

enum {
  HTP_WEIGHT_W8A8 = 1,
  HTP_WEIGHT_F16 = 2,
  /* quantized super-blocks of opcodes 2/3/4, dequantized into the F16 image */
  HTP_WEIGHT_Q4_0 = 3,
  HTP_WEIGHT_Q8_0 = 4,
  HTP_WEIGHT_IQ4_NL = 5,
  /* a device copy of host-resident quantized super-blocks (few-row calls) */
  HTP_WEIGHT_QK0_RAW = 6
};

/* Returns the device image of a prepacked weight for the given source view,
 * building it on a miss.  `sig` identifies the source contents (header bytes /
 * sampled hash).  *built is set when a prepack ran. */
int htp_weight_cache_get(int kind, const htp_view *src, int k, int n, uint64_t sig, void **packed, int *built,
                         hb_stream s);
/* 1 when a valid image for the source view is cached (what
 * htp_weight_cache_get would return without building), else 0. */
int htp_weight_cache_peek(int kind, const htp_view *src, int k, int n, uint64_t sig);
int htp_weight_cache_drop_fd(int fd);
int htp_weight_cache_enabled(void);

/* ---- executor scratch (executor.c) --------------------------------------- */

/* Device scratch owned by the executor, grown on demand (slot 0..4). */
void *htp_executor_scratch(int slot, size_t bytes);
hb_stream htp_executor_stream(void);
int htp_executor_ensure_device(void);

/* Mailbox messages: between begin and end, requests whose tensors all live
 * in HBM complete without a stream synchronisation each; end (or flush)
 * synchronises once, writes their elapsed_us fields, and on a GPU failure
 * overwrites their return codes (`state`, an int32 in the request header)
 * with -5. */
void htp_executor_message_begin(void);
int htp_executor_message_request(struct OpComputeRequest *req, size_t req_size, void *state);
int htp_executor_flush(void);
int htp_executor_message_end(void);

/* ---- backend (backend.c) ------------------------------------------------- */

typedef struct htp_backend htp_backend;
htp_backend *htp_backend_from_handle(remote_handle64 handle);
int htp_backend_compute_allowed(const htp_backend *b);
int htp_backend_device(void);

/* ---- channel (channel.c) ------------------------------------------------- */

typedef struct htp_channel htp_channel;
int htp_channel_start(htp_channel **out, htp_backend *backend, uint8_t *msg, size_t capacity, uint64_t token);
void htp_channel_stop(htp_channel *chan);
void htp_channel_process(htp_backend *backend, struct MessageHeader *msg, size_t capacity, uint64_t token);

/* ---- misc ----------------------------------------------------------------- */

uint64_t htp_fnv1a64(const void *data, size_t bytes);

#endif /* HTP_HOST_INTERNAL_H */
