/*
 * Host session API with the reference's semantics (reference
 * src/host/session.c:14-382): explicit sessions, a process-wide default
 * session with legacy global wrappers, an active-session selector and the
 * channel token derived from a reserved session's index.  A session owns one
 * backend instance (htp_ops_open) instead of a FastRPC process domain.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "htp_ops/session.h"

struct htp_ops_session {
  remote_handle64 handle;
  uint32_t session_id;
  uint32_t session_index; /* reserved-session ordinal (0 = default session) */
  uint32_t effective_domain_id;
  int base_domain_id;
  int reserved;
  int backend_initialized;
  int channel_initialized;
};

#define INVALID_HANDLE ((remote_handle64)-1)
#define MAX_RESERVED_SESSIONS 32

static htp_ops_session *default_session = NULL;
static htp_ops_session *active_session = NULL;
static remote_handle64 legacy_handle = INVALID_HANDLE;
static int reserved_in_use[MAX_RESERVED_SESSIONS];

static uint32_t alloc_reserved_index(void) {
  for (uint32_t i = 1; i < MAX_RESERVED_SESSIONS; ++i) {
    if (!reserved_in_use[i]) {
      reserved_in_use[i] = 1;
      return i;
    }
  }
  return 0;
}

static void free_reserved_index(uint32_t i) {
  if (i > 0 && i < MAX_RESERVED_SESSIONS) reserved_in_use[i] = 0;
}

static uint64_t channel_token(const htp_ops_session *s) {
  if (!s || !s->reserved) return 0;
  return ((uint64_t)s->session_index << 32) | s->effective_domain_id;
}

int htp_ops_session_open(htp_ops_session **out, int base_domain, const char *name, int reserve_new) {
  if (!out) return -1;
  *out = NULL;
  htp_ops_session *s = (htp_ops_session *)calloc(1, sizeof(*s));
  if (!s) return -1;
  s->handle = INVALID_HANDLE;
  s->base_domain_id = base_domain;
  s->effective_domain_id = (uint32_t)base_domain;
  s->reserved = reserve_new != 0;
  if (s->reserved) {
    s->session_index = alloc_reserved_index();
    if (s->session_index == 0) {
      fprintf(stderr, "htp_ops: no free reserved session index (max %d)\n", MAX_RESERVED_SESSIONS - 1);
      free(s);
      return -1;
    }
    s->session_id = s->session_index;
  }
  if (htp_ops_open(name, &s->handle) != AEE_SUCCESS) {
    free_reserved_index(s->session_index);
    free(s);
    return -1;
  }
  *out = s;
  return 0;
}

htp_ops_session *htp_ops_default_session(void) { return default_session; }

int htp_ops_session_init_backend(htp_ops_session *s) {
  if (!s || s->handle == INVALID_HANDLE) return -1;
  const char *multi = getenv("SD_HTP_MULTI_SESSION");
  int err;
  if (s->reserved && multi && multi[0] != '0') {
    err = htp_ops_init_mapping_backend(s->handle);
  } else {
    err = htp_ops_init_backend(s->handle);
  }
  if (err == AEE_SUCCESS) s->backend_initialized = 1;
  return err;
}

int htp_ops_session_acquire_backend(htp_ops_session *s) {
  if (!s || s->handle == INVALID_HANDLE) return -1;
  const int err = htp_ops_init_backend(s->handle);
  if (err == AEE_SUCCESS) s->backend_initialized = 1;
  return err;
}

int htp_ops_session_release_backend(htp_ops_session *s) {
  if (!s || s->handle == INVALID_HANDLE) return -1;
  const int err = htp_ops_release_backend(s->handle);
  if (err == AEE_SUCCESS) s->backend_initialized = 0;
  return err;
}

int htp_ops_session_create_channel(htp_ops_session *s, int fd, unsigned int max_msg_size) {
  if (!s || s->handle == INVALID_HANDLE) return -1;
  const int err = htp_ops_create_channel(s->handle, fd, max_msg_size);
  if (err == AEE_SUCCESS) s->channel_initialized = 1;
  return err;
}

int htp_ops_session_create_channel_with_token(htp_ops_session *s, int fd, unsigned int max_msg_size) {
  if (!s || s->handle == INVALID_HANDLE) return -1;
  const int err = htp_ops_create_channel_with_token(s->handle, channel_token(s), fd, max_msg_size);
  if (err == AEE_SUCCESS) s->channel_initialized = 1;
  return err;
}

int htp_ops_session_destroy_channel(htp_ops_session *s) {
  if (!s || s->handle == INVALID_HANDLE) return -1;
  const int err = htp_ops_destroy_channel(s->handle);
  if (err == AEE_SUCCESS) s->channel_initialized = 0;
  return err;
}

remote_handle64 htp_ops_session_handle(const htp_ops_session *s) { return s ? s->handle : INVALID_HANDLE; }

int htp_ops_set_active_session(htp_ops_session *s) {
  if (!s || s->handle == INVALID_HANDLE) return -1;
  active_session = s;
  return 0;
}

int htp_ops_set_default_session(void) {
  if (!default_session || default_session->handle == INVALID_HANDLE) return -1;
  active_session = default_session;
  return 0;
}

uint32_t htp_ops_session_id(const htp_ops_session *s) { return s ? s->session_id : 0; }
uint32_t htp_ops_session_domain(const htp_ops_session *s) { return s ? s->effective_domain_id : 0; }
int htp_ops_session_is_reserved(const htp_ops_session *s) { return s && s->reserved; }
int htp_ops_session_is_initialized(const htp_ops_session *s) { return s && s->backend_initialized; }
int htp_ops_session_has_channel(const htp_ops_session *s) { return s && s->channel_initialized; }

void htp_ops_session_close(htp_ops_session *s) {
  if (!s) return;
  if (s->handle != INVALID_HANDLE) {
    if (s->channel_initialized) (void)htp_ops_destroy_channel(s->handle);
    htp_ops_close(s->handle);
  }
  if (s->reserved) free_reserved_index(s->session_index);
  if (active_session == s) active_session = default_session == s ? NULL : default_session;
  free(s);
}

remote_handle64 get_global_handle(void) {
  if (active_session) return active_session->handle;
  return default_session ? default_session->handle : legacy_handle;
}

int open_dsp_session(int domain_id, int unsigned_pd_enabled) {
  (void)unsigned_pd_enabled;
  if (default_session) return 0;
  const int err = htp_ops_session_open(&default_session, domain_id, NULL, 0);
  if (err == 0) {
    legacy_handle = default_session->handle;
    active_session = default_session;
  }
  return err;
}

void close_dsp_session(void) {
  htp_ops_session_close(default_session);
  default_session = NULL;
  active_session = NULL;
  legacy_handle = INVALID_HANDLE;
}

void init_htp_backend(void) {
  if (default_session) (void)htp_ops_session_init_backend(default_session);
}

int release_htp_backend(void) { return htp_ops_session_release_backend(default_session); }

int create_htp_message_channel(int fd, unsigned int max_msg_size) {
  return htp_ops_session_create_channel(default_session, fd, max_msg_size);
}

int destroy_htp_message_channel(void) { return htp_ops_session_destroy_channel(default_session); }
