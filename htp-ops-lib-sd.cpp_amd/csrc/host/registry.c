/*
 * Tensor buffer registry (rpcmem / fastrpc_mmap shim) and the prepacked
 * weight cache.
 *
 * The reference keeps an fd -> address map on the DSP side, filled lazily and
 * released by map "put" requests (reference src/dsp/mmap_mgr.cc:32-139,
 * src/dsp/commu.c:187-243).  Here every rpcmem allocation gets a registry
 * entry with its host storage (pinned) or HBM storage, plus a lazily created
 * device mirror for host buffers.  Prepacked weights derived from an fd are
 * cached and dropped together with the fd's mapping.
 */
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "host_internal.h"
#include "htp_ops/rpcmem.h"

typedef struct {
  int fd;
  uint8_t *host; /* NULL for HBM-resident buffers */
  uint8_t *dev;  /* HBM storage, or the host buffer's device mirror (lazy) */
  size_t size;
  int is_device;
  int pinned;    /* host storage from hipHostMalloc (else aligned_alloc) */
  int mapped;    /* fastrpc_mmap called */
  uint64_t generation;
} reg_entry;

typedef struct {
  int kind;
  int fd;
  size_t offset, bytes;
  int k, n;
  uint64_t sig, generation;
  void *packed;
} cache_entry;

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static reg_entry *g_entries;
static size_t g_count, g_cap;
static int g_next_fd = 0x4000;
static uint64_t g_generation = 1;
static cache_entry *g_cache;
static size_t g_cache_count, g_cache_cap;

uint64_t htp_fnv1a64(const void *data, size_t bytes) {
  const uint8_t *p = (const uint8_t *)data;
  uint64_t h = 14695981039346656037ull;
  for (size_t i = 0; i < bytes; ++i) {
    h ^= p[i];
    h *= 1099511628211ull;
  }
  return h;
}

static reg_entry *find_fd_locked(int fd) {
  for (size_t i = 0; i < g_count; ++i)
    if (g_entries[i].fd == fd) return &g_entries[i];
  return NULL;
}

static reg_entry *find_ptr_locked(const void *p) {
  for (size_t i = 0; i < g_count; ++i) {
    const void *base = g_entries[i].is_device ? (const void *)g_entries[i].dev : (const void *)g_entries[i].host;
    if (base == p) return &g_entries[i];
  }
  return NULL;
}

static void drop_cache_fd_locked(int fd) {
  size_t w = 0;
  for (size_t i = 0; i < g_cache_count; ++i) {
    if (g_cache[i].fd == fd) {
      hb_free(g_cache[i].packed);
    } else {
      g_cache[w++] = g_cache[i];
    }
  }
  g_cache_count = w;
}

static void drop_mirror_locked(reg_entry *e) {
  if (!e->is_device && e->dev) {
    hb_free(e->dev);
    e->dev = NULL;
  }
}

void rpcmem_init(void) {}

void rpcmem_deinit(void) {}

void *rpcmem_alloc2(int heapid, uint32_t flags, size_t size) {
  (void)heapid;
  if (size == 0) return NULL;
  reg_entry e;
  memset(&e, 0, sizeof(e));
  e.size = size;
  if (flags & RPCMEM_FLAG_AMD_DEVICE) {
    if (htp_executor_ensure_device() != 0) return NULL;
    void *d = NULL;
    if (hb_malloc(&d, size) != HB_OK) return NULL;
    e.dev = (uint8_t *)d;
    e.is_device = 1;
  } else {
    void *h = NULL;
    if (hb_device_count() > 0 && hb_host_malloc(&h, size) == HB_OK) {
      e.pinned = 1;
    } else {
      /* No GPU visible: plain page-aligned memory so host-side validation
       * paths stay usable; any compute request still needs the GPU. */
      h = aligned_alloc(4096, (size + 4095) / 4096 * 4096);
      if (!h) return NULL;
    }
    e.host = (uint8_t *)h;
  }
  pthread_mutex_lock(&g_lock);
  if (g_count == g_cap) {
    size_t cap = g_cap ? g_cap * 2 : 64;
    reg_entry *grown = (reg_entry *)realloc(g_entries, cap * sizeof(reg_entry));
    if (!grown) {
      pthread_mutex_unlock(&g_lock);
      if (e.is_device) hb_free(e.dev);
      else if (e.pinned) hb_host_free(e.host);
      else free(e.host);
      return NULL;
    }
    g_entries = grown;
    g_cap = cap;
  }
  e.fd = g_next_fd++;
  e.generation = g_generation++;
  g_entries[g_count++] = e;
  pthread_mutex_unlock(&g_lock);
  return e.is_device ? (void *)e.dev : (void *)e.host;
}

void *rpcmem_alloc(int heapid, uint32_t flags, int size) {
  if (size <= 0) return NULL;
  return rpcmem_alloc2(heapid, flags, (size_t)size);
}

void rpcmem_free(void *po) {
  if (!po) return;
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_ptr_locked(po);
  if (!e) {
    pthread_mutex_unlock(&g_lock);
    return;
  }
  reg_entry copy = *e;
  drop_cache_fd_locked(copy.fd);
  *e = g_entries[--g_count];
  pthread_mutex_unlock(&g_lock);
  if (copy.is_device) {
    hb_free(copy.dev);
  } else {
    if (copy.dev) hb_free(copy.dev);
    if (copy.pinned) hb_host_free(copy.host);
    else free(copy.host);
  }
}

int rpcmem_to_fd(void *po) {
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_ptr_locked(po);
  const int fd = e ? e->fd : -1;
  pthread_mutex_unlock(&g_lock);
  return fd;
}

int fastrpc_mmap(int domain, int fd, void *addr, int offset, size_t length, int flags) {
  (void)domain;
  (void)addr;
  (void)flags;
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  int rc = AEE_EBADPARM;
  if (e && offset >= 0 && (size_t)offset <= e->size && length <= e->size - (size_t)offset) {
    e->mapped = 1;
    rc = 0;
  }
  pthread_mutex_unlock(&g_lock);
  return rc;
}

int fastrpc_munmap(int domain, int fd, void *addr, size_t length) {
  (void)domain;
  (void)addr;
  (void)length;
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  int rc = AEE_EBADPARM;
  if (e) {
    e->mapped = 0;
    drop_cache_fd_locked(fd);
    drop_mirror_locked(e);
    rc = 0;
  }
  pthread_mutex_unlock(&g_lock);
  return rc;
}

static int view_locked(int fd, int64_t offset, size_t bytes, htp_view *out, int want_dev) {
  reg_entry *e = find_fd_locked(fd);
  if (!e || !e->mapped || offset < 0 || (size_t)offset > e->size || bytes > e->size - (size_t)offset) return -1;
  if (want_dev && !e->is_device && !e->dev) {
    void *d = NULL;
    if (hb_malloc(&d, e->size) != HB_OK) return -5;
    e->dev = (uint8_t *)d;
  }
  out->fd = fd;
  out->offset = (size_t)offset;
  out->bytes = bytes;
  out->host = e->host ? e->host + offset : NULL;
  out->dev = e->dev ? e->dev + offset : NULL;
  out->is_device = e->is_device;
  out->generation = e->generation;
  return 0;
}

int htp_registry_view(int fd, int64_t offset, size_t bytes, htp_view *out) {
  pthread_mutex_lock(&g_lock);
  const int rc = view_locked(fd, offset, bytes, out, 1);
  pthread_mutex_unlock(&g_lock);
  return rc;
}

int htp_registry_host_view(int fd, int64_t offset, size_t bytes, htp_view *out) {
  pthread_mutex_lock(&g_lock);
  const int rc = view_locked(fd, offset, bytes, out, 0);
  pthread_mutex_unlock(&g_lock);
  return rc;
}

int htp_registry_put(int fd) {
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  int rc = -1;
  if (e) {
    drop_cache_fd_locked(fd);
    drop_mirror_locked(e);
    e->generation = g_generation++;
    rc = 0;
  }
  pthread_mutex_unlock(&g_lock);
  return rc;
}

int htp_registry_known(int fd) {
  pthread_mutex_lock(&g_lock);
  const int known = find_fd_locked(fd) != NULL;
  pthread_mutex_unlock(&g_lock);
  return known;
}

/* Marks stale every cached image built from bytes of fd that overlap
 * [offset, offset + bytes): their next lookup rebuilds them.  Images of the
 * fd's other ranges stay valid, so one buffer may hold weights, activations
 * and outputs (as the reference's own tests lay them out) without a rebuild
 * per call. */
static void stale_range_locked(int fd, size_t offset, size_t bytes) {
  for (size_t i = 0; i < g_cache_count; ++i) {
    cache_entry *c = &g_cache[i];
    if (c->fd == fd && c->offset < offset + bytes && offset < c->offset + c->bytes) c->generation = 0;
  }
}

void htp_registry_touch(int fd, size_t offset, size_t bytes) {
  pthread_mutex_lock(&g_lock);
  stale_range_locked(fd, offset, bytes);
  pthread_mutex_unlock(&g_lock);
}

/* ---- MI355X extensions ---------------------------------------------------- */

int64_t htp_ops_amd_buffer_size(int fd) {
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  const int64_t size = e ? (int64_t)e->size : -1;
  pthread_mutex_unlock(&g_lock);
  return size;
}

int htp_ops_amd_buffer_is_device(int fd) {
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  const int r = e ? e->is_device : -1;
  pthread_mutex_unlock(&g_lock);
  return r;
}

void *htp_ops_amd_buffer_device_ptr(int fd) {
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  void *p = NULL;
  if (e) {
    if (!e->is_device && !e->dev) {
      void *d = NULL;
      if (hb_malloc(&d, e->size) == HB_OK) e->dev = (uint8_t *)d;
    }
    p = e->dev;
  }
  pthread_mutex_unlock(&g_lock);
  return p;
}

int htp_ops_amd_buffer_write(int fd, size_t offset, const void *src, size_t bytes) {
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  int rc = -1;
  if (e && offset <= e->size && bytes <= e->size - offset && (src || bytes == 0)) {
    if (e->is_device) {
      rc = hb_memcpy_h2d(e->dev + offset, src, bytes, NULL) == HB_OK ? 0 : -5;
    } else {
      memcpy(e->host + offset, src, bytes);
      rc = 0;
    }
    stale_range_locked(fd, (size_t)offset, bytes);
  }
  pthread_mutex_unlock(&g_lock);
  return rc;
}

int htp_ops_amd_buffer_read(int fd, size_t offset, void *dst, size_t bytes) {
  pthread_mutex_lock(&g_lock);
  reg_entry *e = find_fd_locked(fd);
  int rc = -1;
  if (e && offset <= e->size && bytes <= e->size - offset && (dst || bytes == 0)) {
    if (e->is_device) {
      rc = hb_memcpy_d2h(dst, e->dev + offset, bytes, NULL) == HB_OK ? 0 : -5;
    } else {
      memcpy(dst, e->host + offset, bytes);
      rc = 0;
    }
  }
  pthread_mutex_unlock(&g_lock);
  return rc;
}

int htp_ops_amd_invalidate_weights(int fd) { return htp_weight_cache_drop_fd(fd); }

/* ---- prepacked weight cache ------------------------------------------------ */

int htp_weight_cache_enabled(void) {
  const char *v = getenv("HTP_OPS_AMD_WEIGHT_CACHE");
  return !(v && v[0] == '0');
}

int htp_weight_cache_drop_fd(int fd) {
  pthread_mutex_lock(&g_lock);
  const size_t before = g_cache_count;
  drop_cache_fd_locked(fd);
  const int dropped = (int)(before - g_cache_count);
  pthread_mutex_unlock(&g_lock);
  return dropped;
}

static size_t packed_bytes(int kind, const htp_view *src, int k, int n) {
  if (kind == HTP_WEIGHT_QK0_RAW) return src->bytes;
  return kind == HTP_WEIGHT_W8A8 ? hb_w8a8_packed_bytes(k, n) : hb_f16_packed_bytes(k, n);
}

/* ggml type of a quantized-weight cache kind, 0 for the others. */
static int qk0_type(int kind) {
  switch (kind) {
    case HTP_WEIGHT_Q4_0: return HB_GGML_Q4_0;
    case HTP_WEIGHT_Q8_0: return HB_GGML_Q8_0;
    case HTP_WEIGHT_IQ4_NL: return HB_GGML_IQ4_NL;
    default: return 0;
  }
}

int htp_weight_cache_peek(int kind, const htp_view *src, int k, int n, uint64_t sig) {
  if (!htp_weight_cache_enabled()) return 0;
  int found = 0;
  pthread_mutex_lock(&g_lock);
  for (size_t i = 0; i < g_cache_count && !found; ++i) {
    const cache_entry *c = &g_cache[i];
    found = c->kind == kind && c->fd == src->fd && c->offset == src->offset && c->bytes == src->bytes &&
            c->k == k && c->n == n && c->sig == sig && c->generation == src->generation;
  }
  pthread_mutex_unlock(&g_lock);
  return found;
}

int htp_weight_cache_get(int kind, const htp_view *src, int k, int n, uint64_t sig, void **packed, int *built,
                         hb_stream s) {
  *packed = NULL;
  *built = 0;
  const int use_cache = htp_weight_cache_enabled();
  pthread_mutex_lock(&g_lock);
  cache_entry *hit = NULL;
  for (size_t i = 0; i < g_cache_count; ++i) {
    cache_entry *c = &g_cache[i];
    if (c->kind == kind && c->fd == src->fd && c->offset == src->offset && c->bytes == src->bytes && c->k == k &&
        c->n == n) {
      hit = c;
      break;
    }
  }
  if (hit && use_cache && hit->sig == sig && hit->generation == src->generation) {
    *packed = hit->packed;
    pthread_mutex_unlock(&g_lock);
    return 0;
  }
  if (hit) {
    hb_free(hit->packed);
    *hit = g_cache[--g_cache_count];
  }
  pthread_mutex_unlock(&g_lock);

  /* Build: bring the source bytes to an aligned device buffer, then prepack. */
  int rc = 0;
  const uint8_t *dsrc = src->dev;
  void *tmp = NULL;
  if (!src->is_device) {
    rc = hb_memcpy_h2d(src->dev, src->host, src->bytes, s);
    if (rc) return -5;
  }
  if (((uintptr_t)dsrc & 15u) != 0) {
    if (hb_malloc(&tmp, src->bytes) != HB_OK) return -5;
    if (hb_memcpy_d2d(tmp, dsrc, src->bytes, s) != HB_OK) {
      hb_free(tmp);
      return -5;
    }
    dsrc = (const uint8_t *)tmp;
  }
  void *img = NULL;
  if (hb_malloc(&img, packed_bytes(kind, src, k, n)) != HB_OK) {
    hb_free(tmp);
    return -5;
  }
  if (kind == HTP_WEIGHT_W8A8)
    rc = hb_w8a8_prepack(img, dsrc, k, n, s);
  else if (kind == HTP_WEIGHT_QK0_RAW)
    rc = hb_memcpy_d2d(img, dsrc, src->bytes, s);
  else if (qk0_type(kind))
    rc = hb_qk0_prepack((uint16_t *)img, dsrc, k, n, qk0_type(kind), s);
  else
    rc = hb_f16_prepack((uint16_t *)img, (const uint16_t *)dsrc, k, n, s);
  if (rc == HB_OK) rc = hb_stream_sync(s);
  hb_free(tmp);
  if (rc != HB_OK) {
    hb_free(img);
    return rc == HB_E_INVAL ? -10 : -5;
  }
  pthread_mutex_lock(&g_lock);
  if (g_cache_count == g_cache_cap) {
    size_t cap = g_cache_cap ? g_cache_cap * 2 : 32;
    cache_entry *grown = (cache_entry *)realloc(g_cache, cap * sizeof(cache_entry));
    if (!grown) {
      pthread_mutex_unlock(&g_lock);
      hb_free(img);
      return -5;
    }
    g_cache = grown;
    g_cache_cap = cap;
  }
  cache_entry c = {kind, src->fd, src->offset, src->bytes, k, n, sig, src->generation, img};
  g_cache[g_cache_count++] = c;
  pthread_mutex_unlock(&g_lock);
  *packed = img;
  *built = 1;
  return 0;
}
