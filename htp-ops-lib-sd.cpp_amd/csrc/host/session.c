/*
 * Host session API (contract: reference include/host/session.h:13-49).
 *
 * A session here is a thin record around one backend instance of this
 * library (htp_ops_open): the backend holds the GPU state, the session only
 * remembers which instance it owns, the caller's domain number, whether it
 * took a reserved ordinal, and which lifecycle steps succeeded.
 *
 * Process-wide state is one registry: the legacy session that
 * open_dsp_session() creates, the session selected for the legacy op
 * wrappers (NULL selects the legacy session), and a bitmask of reserved
 * ordinals.  A reserved session's ordinal is its id and names it in the
 * channel token (ordinal << 32 | domain) that V2 map requests carry.
 */
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "htp_ops/session.h"

enum { SESSION_BACKEND_UP = 1u << 0, SESSION_CHANNEL_UP = 1u << 1 };

struct htp_ops_session {
  remote_handle64 backend; /* the backend instance this session owns */
  int domain;              /* domain number given at open */
  uint32_t ordinal;        /* reserved ordinal (1..31), 0 when not reserved */
  unsigned flags;          /* SESSION_* */
};

#define NO_BACKEND ((remote_handle64)-1)

static struct {
  pthread_mutex_t lock;
  htp_ops_session *legacy;   /* opened by open_dsp_session() */
  htp_ops_session *selected; /* backs the legacy wrappers; NULL = legacy */
  uint32_t ordinals;         /* bit i set: reserved ordinal i is taken (bit 0 never) */
} g_sessions = {PTHREAD_MUTEX_INITIALIZER, NULL, NULL, 0u};

static uint32_t take_ordinal(void) {
  pthread_mutex_lock(&g_sessions.lock);
  const uint32_t free_bits = ~g_sessions.ordinals & ~1u;
  uint32_t ordinal = 0;
  if (free_bits) {
    ordinal = (uint32_t)__builtin_ctz(free_bits);
    g_sessions.ordinals |= 1u << ordinal;
  }
  pthread_mutex_unlock(&g_sessions.lock);
  return ordinal;
}

static void give_back_ordinal(uint32_t ordinal) {
  if (ordinal == 0 || ordinal >= 32) return;
  pthread_mutex_lock(&g_sessions.lock);
  g_sessions.ordinals &= ~(1u << ordinal);
  pthread_mutex_unlock(&g_sessions.lock);
}

static int usable(const htp_ops_session *s) { return s && s->backend != NO_BACKEND; }

/* Runs one backend lifecycle call and records its outcome in the session's flags. */
static int step(htp_ops_session *s, int err, unsigned flag, int set_on_success) {
  if (err == AEE_SUCCESS) s->flags = set_on_success ? (s->flags | flag) : (s->flags & ~flag);
  return err;
}

int htp_ops_session_open(htp_ops_session **out, int base_domain, const char *name, int reserve_new) {
  if (!out) return -1;
  *out = NULL;
  htp_ops_session *s = (htp_ops_session *)calloc(1, sizeof(*s));
  if (!s) return -1;
  s->backend = NO_BACKEND;
  s->domain = base_domain;
  if (reserve_new) {
    s->ordinal = take_ordinal();
    if (!s->ordinal) {
      fprintf(stderr, "htp_ops: all 31 reserved session ordinals are taken\n");
      free(s);
      return -1;
    }
  }
  if (htp_ops_open(name, &s->backend) != AEE_SUCCESS) {
    give_back_ordinal(s->ordinal);
    free(s);
    return -1;
  }
  *out = s;
  return 0;
}

htp_ops_session *htp_ops_default_session(void) { return g_sessions.legacy; }

int htp_ops_session_init_backend(htp_ops_session *s) {
  if (!usable(s)) return -1;
  /* Reserved sessions of a multi-session process only map buffers. */
  const char *multi = getenv("SD_HTP_MULTI_SESSION");
  const int mapping_only = s->ordinal && multi && multi[0] != '0';
  return step(s, mapping_only ? htp_ops_init_mapping_backend(s->backend) : htp_ops_init_backend(s->backend),
              SESSION_BACKEND_UP, 1);
}

int htp_ops_session_acquire_backend(htp_ops_session *s) {
  if (!usable(s)) return -1;
  return step(s, htp_ops_init_backend(s->backend), SESSION_BACKEND_UP, 1);
}

int htp_ops_session_release_backend(htp_ops_session *s) {
  if (!usable(s)) return -1;
  return step(s, htp_ops_release_backend(s->backend), SESSION_BACKEND_UP, 0);
}

int htp_ops_session_create_channel(htp_ops_session *s, int fd, unsigned int max_msg_size) {
  if (!usable(s)) return -1;
  return step(s, htp_ops_create_channel(s->backend, fd, max_msg_size), SESSION_CHANNEL_UP, 1);
}

int htp_ops_session_create_channel_with_token(htp_ops_session *s, int fd, unsigned int max_msg_size) {
  if (!usable(s)) return -1;
  const uint64_t token = s->ordinal ? ((uint64_t)s->ordinal << 32) | (uint32_t)s->domain : 0u;
  return step(s, htp_ops_create_channel_with_token(s->backend, token, fd, max_msg_size), SESSION_CHANNEL_UP, 1);
}

int htp_ops_session_destroy_channel(htp_ops_session *s) {
  if (!usable(s)) return -1;
  return step(s, htp_ops_destroy_channel(s->backend), SESSION_CHANNEL_UP, 0);
}

remote_handle64 htp_ops_session_handle(const htp_ops_session *s) { return s ? s->backend : NO_BACKEND; }

int htp_ops_set_active_session(htp_ops_session *s) {
  if (!usable(s)) return -1;
  g_sessions.selected = s;
  return 0;
}

int htp_ops_set_default_session(void) {
  if (!usable(g_sessions.legacy)) return -1;
  g_sessions.selected = NULL;
  return 0;
}

uint32_t htp_ops_session_id(const htp_ops_session *s) { return s ? s->ordinal : 0u; }
uint32_t htp_ops_session_domain(const htp_ops_session *s) { return s ? (uint32_t)s->domain : 0u; }
int htp_ops_session_is_reserved(const htp_ops_session *s) { return s && s->ordinal != 0; }
int htp_ops_session_is_initialized(const htp_ops_session *s) { return s && (s->flags & SESSION_BACKEND_UP); }
int htp_ops_session_has_channel(const htp_ops_session *s) { return s && (s->flags & SESSION_CHANNEL_UP); }

void htp_ops_session_close(htp_ops_session *s) {
  if (!s) return;
  if (s->backend != NO_BACKEND) {
    /* closing the backend stops its channel as well */
    (void)htp_ops_close(s->backend);
  }
  give_back_ordinal(s->ordinal);
  /* a closed session can no longer back the legacy wrappers */
  if (g_sessions.selected == s) g_sessions.selected = NULL;
  if (g_sessions.legacy == s) g_sessions.legacy = NULL;
  free(s);
}

remote_handle64 get_global_handle(void) {
  const htp_ops_session *s = g_sessions.selected ? g_sessions.selected : g_sessions.legacy;
  return s ? s->backend : NO_BACKEND;
}

int open_dsp_session(int domain_id, int unsigned_pd_enabled) {
  (void)unsigned_pd_enabled; /* no protection domains on the GPU */
  if (g_sessions.legacy) return 0;
  htp_ops_session *s = NULL;
  const int err = htp_ops_session_open(&s, domain_id, NULL, 0);
  if (err == 0) {
    g_sessions.legacy = s;
    g_sessions.selected = NULL;
  }
  return err;
}

void close_dsp_session(void) {
  htp_ops_session_close(g_sessions.legacy);
  g_sessions.legacy = NULL;
  g_sessions.selected = NULL;
}

void init_htp_backend(void) {
  if (g_sessions.legacy) (void)htp_ops_session_init_backend(g_sessions.legacy);
}

int release_htp_backend(void) { return htp_ops_session_release_backend(g_sessions.legacy); }

int create_htp_message_channel(int fd, unsigned int max_msg_size) {
  return htp_ops_session_create_channel(g_sessions.legacy, fd, max_msg_size);
}

int destroy_htp_message_channel(void) { return htp_ops_session_destroy_channel(g_sessions.legacy); }
