/*
 * Request executor for opcodes 1, 15, 16 and 19.
 *
 * Validation order and return codes follow the reference dispatcher
 * (reference src/dsp/op_executor.cc:274-540) and its kernels' argument checks
 * (reference src/dsp/ops/linear_w8a8.c:337-338, src/dsp/ops/mat_mul.c:939-955):
 * every check that can fail does so before any GPU work is queued.  Compute
 * runs on the library stream; host-resident tensors are staged through their
 * device mirrors, HBM-resident tensors are used in place, and outputs are
 * host-visible when the call returns.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include "host_internal.h"
#include "htp_ops/executor.h"
#include "htp_ops/op_reg.h"

/* Envelope of opcode 15.  The reference accepts m <= 4096 and k <= 6144
 * (reference src/dsp/op_executor.cc:320); this library extends both (the
 * int32 accumulator stays exact while 255*128*k < 2^31, i.e. k < 65793). */
#define W8A8_MAX_M 65536
#define W8A8_MAX_K 32768
#define W8A8_MAX_N 65536

#define QTIMER_HZ 19200000.0

static pthread_mutex_t g_exec_lock = PTHREAD_MUTEX_INITIALIZER;
/* Device scratch slots: 0 W8A8 workspace (opcode 19: a realigned weight; QKV:
 * a realigned bias), 1 raw accumulators, a realigned bias or the QKV GEMM
 * output, 2 realigned activations, 3 realigned output, 4 F16 split-K partials
 * or opcode-19 group-norm partials, 5 / 6 realigned QKV q_norm / k_norm, 7 a
 * realigned rotary table, 8-10 realigned QKV outputs.  A slot is allocated on
 * first use. */
enum { kScratchSlots = 11 };
static void *g_scratch[kScratchSlots];
static size_t g_scratch_size[kScratchSlots];
static __thread int t_device_ready = 0;

int htp_executor_ensure_device(void) {
  if (t_device_ready) return 0;
  const int rc = hb_init(htp_backend_device());
  if (rc != HB_OK) return rc;
  t_device_ready = 1;
  return 0;
}

hb_stream htp_executor_stream(void) { return hb_default_stream(); }

void *htp_executor_scratch(int slot, size_t bytes) {
  if (slot < 0 || slot >= kScratchSlots) return NULL;
  if (bytes == 0) bytes = 256;
  if (g_scratch_size[slot] < bytes) {
    /* queued (deferred) work may still use the old buffer */
    if (g_scratch[slot] && hb_stream_sync(htp_executor_stream()) != HB_OK) return NULL;
    if (g_scratch[slot]) hb_free(g_scratch[slot]);
    g_scratch[slot] = NULL;
    g_scratch_size[slot] = 0;
    const size_t grown = bytes + bytes / 4;
    if (hb_malloc(&g_scratch[slot], grown) != HB_OK) return NULL;
    g_scratch_size[slot] = grown;
  }
  return g_scratch[slot];
}

static double now_seconds(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

static int checked_mul(size_t a, size_t b, size_t *out) {
  if (a != 0 && b > SIZE_MAX / a) return 0;
  *out = a * b;
  return 1;
}

static inline uint64_t rotl64(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }

/* Hash of every byte of a host buffer: four independent 64-bit
 * multiply-rotate lanes over 32-byte blocks, then the tail bytes (about
 * 10 GB/s on one core). */
static uint64_t content_hash(const uint8_t *p, size_t n) {
  const uint64_t k1 = 0x9e3779b97f4a7c15ull, k2 = 0xc2b2ae3d27d4eb4full;
  uint64_t lane[4] = {k1, k2, k1 ^ 0x5555555555555555ull, k2 ^ 0xaaaaaaaaaaaaaaaaull};
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    uint64_t w[4];
    memcpy(w, p + i, sizeof(w));
    for (int j = 0; j < 4; ++j) lane[j] = rotl64(lane[j] ^ (w[j] * k2), 29) * k1;
  }
  uint64_t h = (uint64_t)n * k2;
  for (int j = 0; j < 4; ++j) h = rotl64(h ^ lane[j], 31) * k1;
  for (; i < n; ++i) h = (h ^ p[i]) * 1099511628211ull;
  return h ^ (h >> 32);
}

/* Hash of every byte of a large host buffer: content_hash of each 1 MiB
 * chunk, combined in chunk order, the chunks shared out over up to 8 threads
 * (the caller's among them).  The signature is the same whatever the thread
 * count or whether a thread could be started: a share that finds no thread
 * is hashed by the caller. */
#define HASH_CHUNK ((size_t)1 << 20)
#define HASH_MAX_THREADS 8

typedef struct {
  const uint8_t *p;
  size_t n, c0, c1;
  uint64_t *out;
} hash_share;

static void hash_chunks(const hash_share *sh) {
  for (size_t c = sh->c0; c < sh->c1; ++c) {
    const size_t off = c * HASH_CHUNK;
    sh->out[c] = content_hash(sh->p + off, sh->n - off < HASH_CHUNK ? sh->n - off : HASH_CHUNK);
  }
}

static void *hash_worker(void *arg) {
  hash_chunks((const hash_share *)arg);
  return NULL;
}

static uint64_t content_signature(const uint8_t *p, size_t n) {
  if (n < 4 * HASH_CHUNK) return content_hash(p, n);
  const uint64_t k1 = 0x9e3779b97f4a7c15ull, k2 = 0xc2b2ae3d27d4eb4full;
  const size_t chunks = (n + HASH_CHUNK - 1) / HASH_CHUNK;
  uint64_t *hc = malloc(chunks * sizeof(uint64_t));
  uint64_t h = (uint64_t)n * k2;
  if (!hc) {
    for (size_t c = 0; c < chunks; ++c) {
      const size_t off = c * HASH_CHUNK;
      const uint64_t v = content_hash(p + off, n - off < HASH_CHUNK ? n - off : HASH_CHUNK);
      h = rotl64(h ^ (v + (uint64_t)c * k1), 27) * k1;
    }
    return h ^ (h >> 32);
  }
  long cpus = sysconf(_SC_NPROCESSORS_ONLN);
  size_t threads = cpus > 0 ? (size_t)cpus : 1;
  if (threads > HASH_MAX_THREADS) threads = HASH_MAX_THREADS;
  if (threads > chunks / 2) threads = chunks / 2;
  hash_share share[HASH_MAX_THREADS];
  pthread_t tid[HASH_MAX_THREADS];
  int started[HASH_MAX_THREADS] = {0};
  for (size_t t = 0; t < threads; ++t) {
    share[t] = (hash_share){p, n, chunks * t / threads, chunks * (t + 1) / threads, hc};
    if (t > 0) started[t] = pthread_create(&tid[t], NULL, hash_worker, &share[t]) == 0;
  }
  hash_chunks(&share[0]);
  for (size_t t = 1; t < threads; ++t) {
    if (started[t]) pthread_join(tid[t], NULL);
    else hash_chunks(&share[t]);
  }
  for (size_t c = 0; c < chunks; ++c) h = rotl64(h ^ (hc[c] + (uint64_t)c * k1), 27) * k1;
  free(hc);
  return h ^ (h >> 32);
}

/* Signature of a host-resident weight's contents.  The reference reads the
 * constants from DDR on every call (reference src/dsp/ops/linear_w8a8.c:242-268),
 * so a caller may rewrite them in place between calls without a map "put";
 * by default every byte is hashed, so any rewrite rebuilds the prepacked
 * image.  HTP_OPS_AMD_WEIGHT_CACHE=sampled is for callers that always
 * "put" (or call htp_ops_amd_invalidate_weights) after writing: it hashes
 * the first 128 bytes (the W8A8 header), the last `tail` bytes in full (the
 * W8A8 scale, sum and smoothing sections) and 64 spaced 64-byte samples of
 * the rest.  HBM-resident weights change only through this library: a
 * library write marks the cached images whose byte range it overlaps stale,
 * and images of other ranges of the same fd stay valid. */
static uint64_t weight_signature(const htp_view *v, size_t tail) {
  if (v->is_device || !v->host) return 0;
  static int sampled = -1;
  if (sampled < 0) {
    const char *e = getenv("HTP_OPS_AMD_WEIGHT_CACHE");
    sampled = e && strcmp(e, "sampled") == 0;
  }
  if (!sampled || v->bytes <= 128 + tail + 64 * 64) return content_signature(v->host, v->bytes);
  uint64_t h = content_hash(v->host, 128) ^ rotl64(content_hash(v->host + v->bytes - tail, tail), 17);
  const size_t span = v->bytes - 128 - tail;
  for (int i = 0; i < 64; ++i) {
    const size_t off = 128 + span / 64 * (size_t)i;
    h ^= rotl64(content_hash(v->host + off, 64), i) + 0x9e3779b97f4a7c15ull * (uint64_t)(i + 1);
  }
  return h;
}

/* Resolves a tensor without touching the GPU; maps registry errors to the
 * opcode's "unmapped" code. */
static int resolve(const struct RpcmemBufAddr *a, size_t bytes, htp_view *v, int unmapped_code) {
  const int rc = htp_registry_host_view(a->fd, a->offset, bytes, v);
  if (rc == -1) return unmapped_code;
  if (rc != 0) return -5;
  return 0;
}

/* After validation: gives a host-resident view its device mirror. */
static int materialize(htp_view *v) {
  if (v->dev) return 0;
  return htp_registry_view(v->fd, (int64_t)v->offset, v->bytes, v) == 0 ? 0 : -5;
}

static int stage_in(const htp_view *v, hb_stream s) {
  if (v->is_device || v->bytes == 0) return 0;
  return hb_memcpy_h2d(v->dev, v->host, v->bytes, s) == HB_OK ? 0 : -5;
}

static int stage_out(const htp_view *v, hb_stream s) {
  if (v->is_device || v->bytes == 0) return 0;
  return hb_memcpy_d2h(v->host, v->dev, v->bytes, s) == HB_OK ? 0 : -5;
}

/* A device pointer with at least `align` alignment holding the view's bytes
 * (the view itself, or a copy in scratch slot `slot`). */
static const void *aligned_input(const htp_view *v, size_t align, int slot, hb_stream s) {
  if (((uintptr_t)v->dev % align) == 0) return v->dev;
  void *tmp = htp_executor_scratch(slot, v->bytes);
  if (!tmp || hb_memcpy_d2d(tmp, v->dev, v->bytes, s) != HB_OK) return NULL;
  return tmp;
}

typedef struct {
  hb_event e[5];
  int n;
} event_set;

/* Timing events are created once and reused (creating and destroying
 * events costs several microseconds per call).  Every op runs under
 * g_exec_lock; an op takes its events from the pool at g_event_next and
 * hands them back when it completes, or leaves them taken while its
 * completion is deferred (below). */
static hb_event *g_event_pool;
static int g_event_pool_n = 0, g_event_next = 0;

static int events_open(event_set *ev, int count) {
  ev->n = 0;
  if (g_event_next + count > g_event_pool_n) {
    const int want = g_event_next + count;
    hb_event *grown = (hb_event *)realloc(g_event_pool, (size_t)want * sizeof(hb_event));
    if (!grown) return -5;
    g_event_pool = grown;
    while (g_event_pool_n < want) {
      if (hb_event_create(&g_event_pool[g_event_pool_n]) != HB_OK) return -5;
      ++g_event_pool_n;
    }
  }
  for (int i = 0; i < count; ++i) ev->e[i] = g_event_pool[g_event_next + i];
  g_event_next += count;
  ev->n = count;
  return 0;
}

static void events_close(event_set *ev) {
  g_event_next -= ev->n;
  ev->n = 0;
}

static double event_ms(const event_set *ev, int a, int b) {
  float ms = 0.0f;
  if (hb_event_elapsed_ms(&ms, ev->e[a], ev->e[b]) != HB_OK) return 0.0;
  return (double)ms;
}

/* ---- deferred completion inside a mailbox message ----------------------------
 * The reference publishes a message's completion once, after flushing every
 * request's outputs (reference src/dsp/commu.c:250-263).  Inside a message,
 * a request whose tensors all live in HBM therefore does not wait for the
 * GPU: its return code is final once its work is queued (every argument
 * check runs before that), and its elapsed_us field is written when the
 * message is flushed, after one stream synchronisation.  A request with a
 * host-resident output (copied back to the host), a profile trailer or the
 * CPU-control planes still completes before it returns. */
enum { kMaxDeferred = 64 };
typedef struct {
  uint8_t *elapsed_dst; /* int32 elapsed_us field in the payload, or NULL */
  void *state;          /* the request's int32 return code, for a failed flush */
  event_set ev;
  int first, last;      /* events bracketing the timed GPU work */
  double extra_us;      /* host-side time added to elapsed_us (a prepack) */
} deferred_op;

static int g_in_message = 0;
static void *g_request_state = NULL;
static deferred_op g_deferred[kMaxDeferred];
static int g_deferred_n = 0;

static int flush_deferred_locked(void) {
  if (g_deferred_n == 0) return 0;
  const int rc = hb_stream_sync(htp_executor_stream());
  for (int i = 0; i < g_deferred_n; ++i) {
    deferred_op *d = &g_deferred[i];
    if (rc != HB_OK) {
      if (d->state) {
        const int32_t code = -5;
        memcpy(d->state, &code, sizeof(code));
      }
    } else if (d->elapsed_dst) {
      const int32_t us = (int32_t)(event_ms(&d->ev, d->first, d->last) * 1e3 + d->extra_us);
      memcpy(d->elapsed_dst, &us, sizeof(us));
    }
  }
  g_deferred_n = 0;
  g_event_next = 0;
  return rc == HB_OK ? 0 : -5;
}

/* Completes the queued work of one request: defers it when the message
 * allows, else synchronises, writes elapsed_us and hands the events back. */
static int complete(event_set *ev, int first, int last, uint8_t *elapsed_dst, double extra_us, int deferrable) {
  if (g_in_message && deferrable && g_deferred_n < kMaxDeferred) {
    deferred_op *d = &g_deferred[g_deferred_n++];
    d->elapsed_dst = elapsed_dst;
    d->state = g_request_state;
    d->ev = *ev;
    d->first = first;
    d->last = last;
    d->extra_us = extra_us;
    return 0; /* the events stay taken until the flush */
  }
  const int rc = hb_stream_sync(htp_executor_stream());
  if (rc == HB_OK && elapsed_dst) {
    const int32_t us = (int32_t)(event_ms(ev, first, last) * 1e3 + extra_us);
    memcpy(elapsed_dst, &us, sizeof(us));
  }
  events_close(ev);
  return rc == HB_OK ? 0 : -5;
}

void htp_executor_message_begin(void) {
  pthread_mutex_lock(&g_exec_lock);
  g_in_message = 1;
  pthread_mutex_unlock(&g_exec_lock);
}

int htp_executor_message_request(struct OpComputeRequest *req, size_t req_size, void *state) {
  pthread_mutex_lock(&g_exec_lock);
  g_request_state = state;
  pthread_mutex_unlock(&g_exec_lock);
  const int rc = execute_op_simple(req, req_size);
  pthread_mutex_lock(&g_exec_lock);
  g_request_state = NULL;
  pthread_mutex_unlock(&g_exec_lock);
  return rc;
}

int htp_executor_flush(void) {
  pthread_mutex_lock(&g_exec_lock);
  const int rc = flush_deferred_locked();
  pthread_mutex_unlock(&g_exec_lock);
  return rc;
}

int htp_executor_message_end(void) {
  pthread_mutex_lock(&g_exec_lock);
  const int rc = flush_deferred_locked();
  g_in_message = 0;
  pthread_mutex_unlock(&g_exec_lock);
  return rc;
}

/* ---- opcode 15 --------------------------------------------------------------- */

/* Rows per batch of the CPU-control variant, planned as the reference plans
 * its M chunks for its 8 MB VTCM (reference src/dsp/ops/linear_w8a8.c:338-390),
 * so a caller sees the same batch boundaries: with W8A8_CONTROL_WEIGHT_FIRST
 * and every weight resident beside one 64-row activation slab, the caller's
 * resident_batch_rows in 64-row slabs (at least one, at most what the VTCM
 * holds beside the weights); otherwise as many 64-row slabs as min(2 MB, the
 * VTCM left beside one weight slab) holds, at most 64.  Also returns the
 * resident weight columns (in 64s) the reference reports. */
static int cpu_batch_rows(int m, int k, int n, uint32_t flags, uint32_t resident_rows, uint32_t *weight_columns) {
  const size_t vtcm = (size_t)8 << 20, planes = (size_t)1 << 20, meta = 1024u + 4096u * 4u;
  const size_t slab = (size_t)k * 64u; /* one 64-column weight slab = one 64-row activation slab */
  const size_t all_weights = (size_t)k * (size_t)n;
  const long slabs_m = (m + 63) / 64;
  long slabs;
  size_t weight_area;
  if ((flags & W8A8_CONTROL_WEIGHT_FIRST) && all_weights + planes + meta + slab <= vtcm) {
    const long room = (long)((vtcm - planes - meta - all_weights) / slab);
    slabs = (long)(resident_rows / 64u);
    if (slabs > room) slabs = room;
    if (slabs > slabs_m) slabs = slabs_m;
    if (slabs < 1) slabs = 1;
    weight_area = all_weights;
  } else {
    size_t budget = vtcm > planes + meta + slab ? vtcm - planes - meta - slab : 0;
    if (budget > ((size_t)2 << 20)) budget = (size_t)2 << 20;
    slabs = (long)(budget / slab);
    if (slabs > 64) slabs = 64;
    if (slabs > slabs_m) slabs = slabs_m;
    if (slabs < 1) slabs = 1;
    const size_t used = (size_t)slabs * slab + planes + meta;
    weight_area = vtcm > used ? (vtcm - used) / slab * slab : slab;
  }
  *weight_columns = (uint32_t)(weight_area / slab);
  return (int)(slabs * 64);
}

/* Events that mark each CPU-control batch done (created once, reused under
 * the executor lock). */
static hb_event g_batch_events[W8A8_CPU_MAX_BATCHES];
static int g_batch_events_n = 0;

static int batch_events(int count) {
  while (g_batch_events_n < count) {
    if (hb_event_create(&g_batch_events[g_batch_events_n]) != HB_OK) return -5;
    ++g_batch_events_n;
  }
  return 0;
}

static int exec_w8a8(uint8_t *payload, size_t payload_size) {
  /* reference src/dsp/op_executor.cc:314-353 */
  if (payload_size != sizeof(struct NativeW8A8Params) && payload_size != sizeof(struct NativeW8A8ProfileParams) &&
      payload_size != sizeof(struct NativeW8A8CpuParams))
    return -1;
  struct NativeW8A8Params p;
  memcpy(&p, payload, sizeof(p));
  const int m = p.m, k = p.k, n = p.n;
  if (m < 1 || m > W8A8_MAX_M || k < 32 || k > W8A8_MAX_K || k % 32 || n < 64 || n > W8A8_MAX_N || n % 64)
    return -1;
  const int cpu_output = payload_size == sizeof(struct NativeW8A8CpuParams);
  const int profiled = payload_size == sizeof(struct NativeW8A8ProfileParams);
  if (cpu_output && m > 4096) return -1; /* W8A8CpuControl.scales holds 4096 rows */
  const size_t constants_size = 128u + (size_t)k * n + (size_t)n * 8u + (size_t)k * 4u;
  htp_view out, act, cst, ctl;
  int rc = resolve(&p.output, (size_t)m * n * 4u, &out, -2);
  if (!rc) rc = resolve(&p.activation, (size_t)m * k * 4u, &act, -2);
  if (!rc) rc = resolve(&p.constants, constants_size, &cst, -2);
  struct NativeW8A8CpuParams cp;
  if (!rc && cpu_output) {
    memcpy(&cp, payload, sizeof(cp));
    rc = resolve(&cp.control, sizeof(struct W8A8CpuControl), &ctl, -2);
  }
  if (rc) return rc;

  /* Header acceptance, reference src/dsp/op_executor.cc:331-335.  A device
   * blob whose prepacked image is cached passed this check when the image was
   * built and has not been written since (a library write that overlaps the
   * blob's bytes marks its image stale), so only a miss reads the header back
   * (a blocking copy). */
  const uint64_t cst_sig = weight_signature(&cst, (size_t)n * 8u + (size_t)k * 4u);
  if (!(cst.is_device && htp_weight_cache_peek(HTP_WEIGHT_W8A8, &cst, k, n, cst_sig))) {
    struct W8A8Header h;
    if (cst.is_device) {
      if (hb_memcpy_d2h(&h, cst.dev, sizeof(h), htp_executor_stream()) != HB_OK) return -5;
    } else {
      memcpy(&h, cst.host, sizeof(h));
    }
    const size_t scale_off = 128u + (size_t)k * n;
    if (h.magic != W8A8_BLOB_MAGIC || h.version != W8A8_BLOB_VERSION || h.k != (uint32_t)k ||
        h.n != (uint32_t)n || h.weight_offset != 128u || h.scale_offset != scale_off ||
        h.sum_offset != scale_off + (size_t)n * 4u || h.inverse_offset != (size_t)h.sum_offset + (size_t)n * 4u ||
        h.bytes != constants_size)
      return -3;
  }

  struct NativeW8A8Profile profile;
  memset(&profile, 0, sizeof(profile));
  if (profiled) {
    memcpy(&profile, payload + sizeof(struct NativeW8A8Params), sizeof(profile));
    if (profile.mode != 1 && profile.mode != 2 && profile.mode != 3) return -1;
    const uint32_t mode = profile.mode;
    memset(&profile, 0, sizeof(profile));
    profile.mode = mode;
  }

  const double t_setup = now_seconds();
  if (htp_executor_ensure_device() != 0) return -5;
  if (materialize(&out) || materialize(&act) || materialize(&cst) || (cpu_output && materialize(&ctl))) return -5;
  hb_stream s = htp_executor_stream();
  void *packed = NULL;
  int built = 0;
  const double t_w0 = now_seconds();
  rc = htp_weight_cache_get(HTP_WEIGHT_W8A8, &cst, k, n, cst_sig, &packed, &built, s);
  if (rc) return rc;
  const double t_w1 = now_seconds();
  if (stage_in(&act, s)) return -5;
  const float *x = (const float *)aligned_input(&act, 16, 2, s);
  if (!x) return -5;
  const size_t ws_bytes = hb_w8a8_linear_workspace_bytes(m, k, n);
  uint8_t *ws = (uint8_t *)htp_executor_scratch(0, ws_bytes);
  if (!ws) return -5;
  int8_t *q = (int8_t *)ws;
  const size_t q_bytes = ((size_t)(m + 15) / 16 * 16) * ((size_t)(k + 63) / 64 * 64);
  float *scales = (float *)(ws + (q_bytes + 255u) / 256u * 256u); /* layout of hb_w8a8_workspace_bytes, the prefix */
  const float *inv = (const float *)((const uint8_t *)packed + hb_w8a8_packed_offset(k, n, HB_W8A8_INV));
  /* The GEMM writes 16-byte vectors: a misaligned output is produced in scratch and copied. */
  float *y = ((uintptr_t)out.dev % 16u) == 0 ? (float *)out.dev : (float *)htp_executor_scratch(3, out.bytes);
  /* profile mode 2 runs the GEMM's epilogue as its own launch, so the MAC
   * and readout phases are timed apart (reference linear_w8a8.c:488-500) */
  const int split_readout = profiled && profile.mode == 2 && !cpu_output;
  void *raw = cpu_output || split_readout ? htp_executor_scratch(1, (size_t)m * n * 4u) : NULL;
  if (!y || ((cpu_output || split_readout) && !raw)) return -5;

  /* CPU-control variant: the control block as the caller left it (flags,
   * requested batch rows), the batch plan, and the block's diagnostics; a
   * host-resident block is updated in place, so the caller may poll
   * `produced` while the batches complete. */
  struct W8A8CpuControl *hc = NULL;
  int batch_rows = m, nbatch = 1;
  if (cpu_output) {
    if (ctl.is_device) {
      hc = (struct W8A8CpuControl *)malloc(sizeof(*hc));
      if (!hc || hb_memcpy_d2h(hc, ctl.dev, sizeof(*hc), s) != HB_OK) {
        free(hc);
        return -5;
      }
    } else {
      hc = (struct W8A8CpuControl *)ctl.host;
    }
    uint32_t weight_columns = 0;
    batch_rows = cpu_batch_rows(m, k, n, hc->flags, hc->resident_batch_rows, &weight_columns);
    nbatch = (m + batch_rows - 1) / batch_rows;
    if (batch_events(nbatch)) {
      if (ctl.is_device) free(hc);
      return -5;
    }
    __atomic_store_n(&hc->produced, 0u, __ATOMIC_RELEASE);
    hc->vtcm_bytes = 8u << 20; /* the budget the batches are planned for */
    hc->activation_rows = (uint32_t)batch_rows;
    hc->weight_columns = weight_columns;
    hc->weight_loads = built ? 1u : 0u;
    hc->weight_loaded_bytes = built ? (uint64_t)k * n : 0u;
  }

  event_set ev;
  if (events_open(&ev, 4)) {
    events_close(&ev);
    if (cpu_output && ctl.is_device) free(hc);
    return -5;
  }
  int hrc = hb_event_record(ev.e[0], s);
  /* A plain request runs through hb_w8a8_linear, which takes the one-launch
   * kernels that quantize their own rows where the shape allows (m == 1,
   * 2-4 rows, 5-128 rows with short K) and quantize + GEMM otherwise; all
   * its time is then reported as GEMM time.  A profiled or CPU-control
   * request keeps quantization as its own launch so its phases are timed
   * apart. */
  const int split = cpu_output || profiled;
  if (!hrc && split) hrc = hb_w8a8_quantize(q, scales, x, inv, m, k, s);
  /* the phase events only where phases are reported (each record is a host
   * call and a GPU packet: about 2 us per request at M=1) */
  if (!hrc && split) hrc = hb_event_record(ev.e[1], s);
  /* the row scales reach a host-resident control block with the first batch */
  if (!hrc && cpu_output && !ctl.is_device) hrc = hb_memcpy_d2h_async(hc->scales, scales, (size_t)m * 4u, s);
  if (!hrc && cpu_output) {
    /* batch b: its rows' accumulators, their byte planes in the output, and
     * (host-resident output) their copy to the host, then its event */
    const size_t kp = (size_t)(k + 63) / 64 * 64, row_bytes = (size_t)n * 4u;
    for (int b = 0; !hrc && b < nbatch; ++b) {
      const int m0 = b * batch_rows, rows = m - m0 < batch_rows ? m - m0 : batch_rows;
      int32_t *rb = (int32_t *)raw + (size_t)m0 * n;
      uint8_t *yb = (uint8_t *)y + (size_t)m0 * row_bytes, *ob = (uint8_t *)out.dev + (size_t)m0 * row_bytes;
      hrc = hb_w8a8_gemm(rb, n, q + (size_t)m0 * kp, scales + m0, packed, rows, k, n, HB_W8A8_EPI_RAW, s);
      if (!hrc) hrc = hb_w8a8_planes_from_raw(yb, rb, rows, n, s);
      if (!hrc && (void *)y != (void *)out.dev) hrc = hb_memcpy_d2d(ob, yb, (size_t)rows * row_bytes, s);
      if (!hrc && !out.is_device)
        hrc = hb_memcpy_d2h_async((uint8_t *)out.host + (size_t)m0 * row_bytes, ob, (size_t)rows * row_bytes, s);
      if (!hrc) hrc = hb_event_record(g_batch_events[b], s);
    }
  } else if (!hrc) {
    if (!split) hrc = hb_w8a8_linear(y, x, packed, m, k, n, HB_W8A8_EPI_SCALE, ws, ws_bytes, s);
    else if (split_readout) hrc = hb_w8a8_gemm(raw, n, q, scales, packed, m, k, n, HB_W8A8_EPI_RAW, s);
    else hrc = hb_w8a8_gemm(y, n, q, scales, packed, m, k, n, HB_W8A8_EPI_SCALE, s);
  }
  if (!hrc && split) hrc = hb_event_record(ev.e[2], s);
  if (!hrc && split_readout)
    hrc = hb_w8a8_readout(y, n, (const int32_t *)raw, scales, packed, m, k, n, HB_W8A8_EPI_SCALE, s);
  if (!hrc) hrc = hb_event_record(ev.e[3], s);
  if (!hrc && !cpu_output && (void *)y != (void *)out.dev) hrc = hb_memcpy_d2d(out.dev, y, out.bytes, s);
  if (!hrc && cpu_output && !ctl.is_device) {
    /* publish each batch as soon as it is done (reference
     * src/dsp/ops/linear_w8a8.c:512-526): the caller's CPU epilogue of
     * batch b overlaps the GPU's work on the batches after it */
    for (int b = 0; !hrc && b < nbatch; ++b) {
      if (hb_event_sync(g_batch_events[b]) != HB_OK) {
        hrc = -5;
        break;
      }
      const int m0 = b * batch_rows, rows = m - m0 < batch_rows ? m - m0 : batch_rows;
      hc->batches[b].m0 = m0;
      hc->batches[b].rows = rows;
      hc->batches[b].n0 = 0;
      hc->batches[b].columns = n / 64;
      __atomic_store_n(&hc->produced, (uint32_t)(b + 1), __ATOMIC_RELEASE);
    }
  }
  if (hrc) {
    events_close(&ev);
    if (cpu_output && ctl.is_device) free(hc);
    return hrc == HB_E_INVAL ? -10 : -5;
  }
  const double weight_s = built ? t_w1 - t_w0 : 0.0;
  if (!split && out.is_device) {
    htp_registry_touch(out.fd, out.offset, out.bytes);
    return complete(&ev, 0, 3, payload + offsetof(struct NativeW8A8Params, elapsed_us), weight_s * 1e6, 1);
  }
  if (hb_stream_sync(s) != HB_OK) {
    events_close(&ev);
    if (cpu_output && ctl.is_device) free(hc);
    return -5;
  }
  /* a plain request recorded only the bracketing events: all its time is GEMM
   * time; a CPU-control request's batches (GEMM, planes and copies) all count
   * as GEMM time */
  const double quant_ms = split ? event_ms(&ev, 0, 1) : 0.0;
  const double gemm_ms = split ? event_ms(&ev, 1, 2) : event_ms(&ev, 0, 3);
  const double out_ms = split ? event_ms(&ev, 2, 3) : 0.0;
  events_close(&ev);

  if (cpu_output && ctl.is_device) {
    /* an HBM-resident control block is written once, after every batch */
    int crc = hb_memcpy_d2h(hc->scales, scales, (size_t)m * 4u, s) != HB_OK;
    for (int b = 0; b < nbatch; ++b) {
      const int m0 = b * batch_rows;
      hc->batches[b].m0 = m0;
      hc->batches[b].rows = m - m0 < batch_rows ? m - m0 : batch_rows;
      hc->batches[b].n0 = 0;
      hc->batches[b].columns = n / 64;
    }
    hc->produced = (uint32_t)nbatch;
    if (!crc) crc = hb_memcpy_h2d(ctl.dev, hc, sizeof(*hc), s) != HB_OK;
    free(hc);
    if (crc) return -5;
  }
  /* (a CPU-control request copied its host-resident output batch by batch) */
  if (!cpu_output && stage_out(&out, s)) return -5;
  htp_registry_touch(out.fd, out.offset, out.bytes);

  const double total_us = (quant_ms + gemm_ms + out_ms) * 1e3 + weight_s * 1e6;
  p.elapsed_us = (int32_t)total_us;
  memcpy(payload + offsetof(struct NativeW8A8Params, elapsed_us), &p.elapsed_us, sizeof(int32_t));
  if (profiled) {
    profile.setup_ticks = (uint64_t)((t_w0 - t_setup) * QTIMER_HZ);
    profile.activation_ticks = (uint64_t)(quant_ms * 1e-3 * QTIMER_HZ);
    profile.weight_ticks = (uint64_t)(weight_s * QTIMER_HZ);
    profile.hmx_ticks = (uint64_t)(gemm_ms * 1e-3 * QTIMER_HZ);
    profile.output_ticks = (uint64_t)(out_ms * 1e-3 * QTIMER_HZ);
    if (profile.mode == 2) {
      /* the accumulating GEMM (int32 sums out) is the MAC phase; the launch
       * after it (the scale epilogue, or the byte planes of the CPU-control
       * variant) reads the sums out.  Both are HMX-phase time, as on the
       * reference, and no output phase remains. */
      profile.mac_ticks = profile.hmx_ticks;
      profile.readout_ticks = profile.output_ticks;
      profile.hmx_ticks += profile.output_ticks;
      profile.output_ticks = 0;
    } else if (profile.mode == 3) {
      /* reserved: low 16 bits = rows per workgroup tile, high 16 = columns,
       * of the GEMM kernel that ran (the choice hb_w8a8_gemm makes for this
       * shape); mac/readout = weight loads / bytes during this call. */
      int bm = 0, bn = 0;
      if (hb_w8a8_gemm_tile(m, k, n, &bm, &bn) == HB_E_INVAL) bm = bn = 0;
      profile.reserved = (uint32_t)bm | ((uint32_t)bn << 16);
      profile.mac_ticks = built ? 1u : 0u;
      profile.readout_ticks = built ? (uint64_t)k * n : 0u;
    }
    memcpy(payload + sizeof(struct NativeW8A8Params), &profile, sizeof(profile));
  }
  return 0;
}

/* ---- opcodes 16 and 1 -------------------------------------------------------- */

static uintptr_t primary_address(const htp_view *v) {
  return v->is_device ? (uintptr_t)v->dev : (uintptr_t)v->host;
}

/* Shared F16 compute after validation.  Returns 0 or a negative code.
 * qk0_type != 0 (opcodes 2/3/4): with m <= 16 the quantized super-blocks are
 * multiplied directly (in place when already device-resident and aligned,
 * else from a cached device copy); otherwise through their cached F16 image. */
static int run_f16(int kind, int qk0_type, htp_view *out, htp_view *act, htp_view *wgt, htp_view *bias, int m, int k,
                   int n, int channels, int mode, uint8_t *elapsed_dst) {
  if (htp_executor_ensure_device() != 0) return -5;
  if (materialize(out) || materialize(act) || materialize(wgt) || (bias && materialize(bias))) return -5;
  hb_stream s = htp_executor_stream();
  const int direct = qk0_type != 0 && m <= 16;
  void *packed = NULL;
  int built = 0;
  const double t_w0 = now_seconds();
  int rc = 0;
  if (direct && wgt->is_device && ((uintptr_t)wgt->dev & 15u) == 0)
    packed = wgt->dev;
  else
    rc = htp_weight_cache_get(direct ? HTP_WEIGHT_QK0_RAW : kind, wgt, k, n, weight_signature(wgt, 0), &packed, &built,
                              s);
  if (rc) return rc;
  const double t_w1 = now_seconds();
  if (stage_in(act, s)) return -5;
  const float *x = (const float *)aligned_input(act, 16, 2, s);
  if (!x) return -5;
  const float *b = NULL;
  if (bias) {
    if (stage_in(bias, s)) return -5;
    b = (const float *)aligned_input(bias, 4, 1, s);
    if (!b) return -5;
  }
  const size_t out_bytes = out->bytes;
  float *y = ((uintptr_t)out->dev % 4u) == 0 ? (float *)out->dev : (float *)htp_executor_scratch(3, out_bytes);
  if (!y) return -5;
  event_set ev;
  if (events_open(&ev, 2)) {
    events_close(&ev);
    return -5;
  }
  /* Few rows: the split-K path, with its partial sums in executor scratch. */
  const size_t ws_bytes = hb_f16_workspace_bytes(m, k, n);
  void *ws = ws_bytes ? htp_executor_scratch(4, ws_bytes) : NULL;
  if (ws_bytes && !ws) {
    events_close(&ev);
    return -5;
  }
  int hrc = hb_event_record(ev.e[0], s);
  if (!hrc)
    hrc = direct ? hb_qk0_gemm_ws(y, x, (const uint8_t *)packed, m, k, n, qk0_type, ws, ws_bytes, s)
                 : hb_f16_gemm_ws(y, x, (const uint16_t *)packed, b, m, k, n, channels, mode, ws, ws_bytes, s);
  if (!hrc) hrc = hb_event_record(ev.e[1], s);
  if (!hrc && (void *)y != (void *)out->dev) hrc = hb_memcpy_d2d(out->dev, y, out_bytes, s);
  if (hrc) {
    events_close(&ev);
    return hrc == HB_E_INVAL ? -11 : -5;
  }
  htp_registry_touch(out->fd, out->offset, out->bytes);
  const double extra_us = built ? (t_w1 - t_w0) * 1e6 : 0.0;
  if (complete(&ev, 0, 1, elapsed_dst, extra_us, out->is_device)) return -5;
  if (stage_out(out, s)) return -5;
  return 0;
}

static int exec_f16_epilogue(uint8_t *payload, size_t payload_size) {
  /* reference src/dsp/op_executor.cc:446-471, src/dsp/ops/mat_mul.c:937-955 */
  if (payload_size != sizeof(struct F16EpilogueParams)) return -1;
  struct F16EpilogueParams p;
  memcpy(&p, payload, sizeof(p));
  if (p.m <= 0 || p.k <= 0 || p.n <= 0 || p.k % 32 || p.n % 32 || p.channels <= 0 || p.channels > p.n ||
      p.mode < 0 || p.mode > 3 || (p.mode != 3 && p.channels != p.n))
    return -1;
  size_t out_size, act_size, weight_size;
  if (!checked_mul((size_t)p.m, (size_t)p.channels * sizeof(float), &out_size) ||
      !checked_mul((size_t)p.m, (size_t)p.k * sizeof(float), &act_size) ||
      !checked_mul((size_t)p.k, (size_t)p.n * 2u, &weight_size))
    return -1;
  htp_view out, act, wgt, bias;
  int rc = resolve(&p.output, out_size, &out, -1);
  if (!rc) rc = resolve(&p.activation, act_size, &act, -1);
  if (!rc) rc = resolve(&p.weight, weight_size, &wgt, -1);
  if (!rc && p.bias.fd >= 0) rc = resolve(&p.bias, (size_t)p.channels * sizeof(float), &bias, -1);
  if (rc) return rc;
  /* Kernel alignment contract: 128-byte aligned dst/activation/weight
   * (reference src/dsp/ops/mat_mul.c:947-949). */
  if ((primary_address(&out) | primary_address(&act) | primary_address(&wgt)) & 127u) return -12;
  return run_f16(HTP_WEIGHT_F16, 0, &out, &act, &wgt, p.bias.fd >= 0 ? &bias : NULL, p.m, p.k, p.n, p.channels,
                 p.mode, payload + offsetof(struct F16EpilogueParams, elapsed_us));
}

static int exec_matmul_params(const struct MatMulParams *p, uint8_t *elapsed_dst, uint64_t *act_hash,
                              uint64_t *out_hash) {
  /* reference src/dsp/op_executor.cc:473-540, src/dsp/ops/mat_mul.c:1046-1049 */
  const int m = p->m, k = p->k, n = p->n;
  const int dims_ok = m > 0 && k > 0 && n > 0;
  htp_view out, act, wgt;
  int rc = resolve(&p->output, dims_ok ? (size_t)m * n * 4u : 0, &out, -2);
  if (!rc) rc = resolve(&p->activation, dims_ok ? (size_t)m * k * 4u : 0, &act, -2);
  if (!rc) rc = resolve(&p->weight, dims_ok ? (size_t)k * n * 2u : 0, &wgt, -2);
  if (rc) return rc;
  if ((primary_address(&out) | primary_address(&act) | primary_address(&wgt)) & 127u) return -3;
  if (m == 0 || n == 0 || k == 0) return -10;
  if (!dims_ok || k % 32 || n % 32) return -11;
  if (act_hash) {
    *act_hash = 0;
    if (act.host) *act_hash = htp_fnv1a64(act.host, act.bytes);
  }
  rc = run_f16(HTP_WEIGHT_F16, 0, &out, &act, &wgt, NULL, m, k, n, n, 0, elapsed_dst);
  if (rc) return rc;
  if (out_hash) {
    *out_hash = 0;
    if (out.host) *out_hash = htp_fnv1a64(out.host, out.bytes);
  }
  return 0;
}

static int exec_matmul(uint8_t *payload, size_t payload_size) {
  if (payload_size < sizeof(struct MatMulParams)) return -1;
  struct MatMulParams p;
  memcpy(&p, payload, sizeof(p));
  uint8_t *elapsed_dst =
      payload_size >= sizeof(struct MatMulProfileParams) ? payload + offsetof(struct MatMulProfileParams, elapsed_us)
                                                         : NULL;
  return exec_matmul_params(&p, elapsed_dst, NULL, NULL);
}

/* Opcodes 2/3/4: Q4_0 / Q8_0 / IQ4_NL super-blocks.  m <= 16 multiplies the
 * blocks directly; larger m dequantizes them into the F16 image (once per
 * weight buffer, cached) and runs the F16 GEMM with mode 0 and no bias.  Reference src/dsp/op_executor.cc:771-800 (payload, buffer sizes
 * m*n*4, m*k*4, k*n/256*block) and src/dsp/ops/mat_mul.c:1601-1617 (-1 for
 * a missing buffer, a zero dimension, k or n not a multiple of 32, or an
 * output, activation or weight address not 128-byte aligned). */
static int exec_matmul_qk0(uint8_t *payload, size_t payload_size, int kind, int type) {
  if (payload_size < sizeof(struct MatMulParams)) return -1;
  struct MatMulParams p;
  memcpy(&p, payload, sizeof(p));
  const int m = p.m, k = p.k, n = p.n;
  if (m <= 0 || k <= 0 || n <= 0 || k % 32 || n % 32) return -1;
  size_t out_size, act_size;
  const size_t weight_size = hb_qk0_weight_bytes(k, n, type);
  if (!checked_mul((size_t)m, (size_t)n * sizeof(float), &out_size) ||
      !checked_mul((size_t)m, (size_t)k * sizeof(float), &act_size) || !weight_size)
    return -1;
  htp_view out, act, wgt;
  int rc = resolve(&p.output, out_size, &out, -1);
  if (!rc) rc = resolve(&p.activation, act_size, &act, -1);
  if (!rc) rc = resolve(&p.weight, weight_size, &wgt, -1);
  if (rc) return rc;
  if ((primary_address(&out) | primary_address(&act) | primary_address(&wgt)) & 127u) return -1;
  /* elapsed_us is not written for these opcodes, as in the reference */
  return run_f16(kind, type, &out, &act, &wgt, NULL, m, k, n, n, 0, NULL);
}

/* Direct (non-mailbox) opcode-1 entry used by htp_ops_mat_mul_permuted_w16a32[_trace]. */
int htp_exec_matmul_w16a32(const struct MatMulParams *p, int32_t *elapsed_us, uint64_t *act_hash,
                           uint64_t *out_hash) {
  pthread_mutex_lock(&g_exec_lock);
  const int saved = g_in_message; /* a direct call completes before it returns */
  g_in_message = 0;
  const int rc = exec_matmul_params(p, (uint8_t *)elapsed_us, act_hash, out_hash);
  g_in_message = saved;
  pthread_mutex_unlock(&g_exec_lock);
  return rc;
}

/* ---- opcodes 8/10/11/12 ------------------------------------------------------ */

/* One projection of a QKV request: the image or text half of the dual opcodes,
 * or the whole of opcodes 8 and 11. */
typedef struct {
  htp_view act, wgt, bias, q_norm, k_norm;
  int has_bias, tokens, out_offset, rope_offset;
} qkv_part;

static int qkv_resolve_part(qkv_part *p, const struct RpcmemBufAddr *act, const struct RpcmemBufAddr *wgt,
                            const struct RpcmemBufAddr *bias, int bias_required, const struct RpcmemBufAddr *q_norm,
                            const struct RpcmemBufAddr *k_norm, int tokens, int input_dim, size_t weight_bytes,
                            size_t bias_bytes, size_t norm_bytes) {
  size_t act_bytes;
  if (!checked_mul((size_t)tokens, (size_t)input_dim * sizeof(float), &act_bytes)) return -1;
  p->tokens = tokens;
  p->has_bias = bias_required || bias->fd >= 0;
  /* an unmapped buffer reaches the reference kernel as NULL, which it rejects */
  int rc = resolve(act, act_bytes, &p->act, -1);
  if (!rc) rc = resolve(wgt, weight_bytes, &p->wgt, -1);
  if (!rc && p->has_bias) rc = resolve(bias, bias_bytes, &p->bias, -1);
  if (!rc) rc = resolve(q_norm, norm_bytes, &p->q_norm, -1);
  if (!rc) rc = resolve(k_norm, norm_bytes, &p->k_norm, -1);
  if (rc) return rc;
  /* 128-byte activation and weight (reference src/dsp/ops/mat_mul.c:1385-1388) */
  if ((primary_address(&p->act) | primary_address(&p->wgt)) & 127u) return -1;
  return 0;
}

/* A device pointer to write an output view through: the view itself when
 * 16-byte aligned, else scratch slot `slot` (copied back by the caller). */
static void *qkv_output(const htp_view *v, int slot) {
  if (((uintptr_t)v->dev & 15u) == 0) return v->dev;
  return htp_executor_scratch(slot, v->bytes);
}

/* Validated request -> queued GEMM + post-processing for each part.
 * rope: pe view or NULL; rope_count the token bound of the rotation. */
static int run_qkv(htp_view out[3], qkv_part *parts, int n_parts, htp_view *pe, int rope_count, int input_dim,
                   int n_heads, int head_dim, int token_tiles, uint8_t *elapsed_dst) {
  if (htp_executor_ensure_device() != 0) return -5;
  for (int i = 0; i < 3; ++i)
    if (materialize(&out[i])) return -5;
  if (pe && materialize(pe)) return -5;
  for (int i = 0; i < n_parts; ++i) {
    qkv_part *p = &parts[i];
    if (materialize(&p->act) || materialize(&p->wgt) || materialize(&p->q_norm) || materialize(&p->k_norm) ||
        (p->has_bias && materialize(&p->bias)))
      return -5;
  }
  hb_stream s = htp_executor_stream();
  const int ncols = 3 * n_heads * head_dim;
  /* weights first: a build synchronises, which stays outside the timed region */
  void *packed[2] = {NULL, NULL};
  double extra_us = 0.0;
  for (int i = 0; i < n_parts; ++i) {
    int built = 0;
    const double t0 = now_seconds();
    const int rc = htp_weight_cache_get(HTP_WEIGHT_F16, &parts[i].wgt, input_dim, ncols,
                                        weight_signature(&parts[i].wgt, 0), &packed[i], &built, s);
    if (rc) return rc;
    if (built) extra_us += (now_seconds() - t0) * 1e6;
  }

  /* A part of 512 tokens or more runs the GEMM with the post-processing in
   * its epilogue (hb_qkv_gemm: its tiles then fill the CUs); a smaller one
   * the GEMM into scratch, then hb_qkv_post (same results either way). */
  int fused[2] = {0, 0};
  size_t ws_max = 0;
  for (int i = 0; i < n_parts; ++i) {
    fused[i] = parts[i].tokens >= 512 && (ncols / 3) % 128 == 0;
    const size_t b = fused[i] ? hb_qkv_gemm_workspace_bytes(parts[i].tokens, input_dim)
                              : hb_f16_workspace_bytes(parts[i].tokens, input_dim, ncols);
    ws_max = b > ws_max ? b : ws_max;
  }
  int raw_tokens = 0;
  for (int i = 0; i < n_parts; ++i)
    if (!fused[i] && parts[i].tokens > raw_tokens) raw_tokens = parts[i].tokens;
  float *raw = raw_tokens ? (float *)htp_executor_scratch(1, (size_t)raw_tokens * (size_t)ncols * sizeof(float))
                          : NULL;
  void *ws = ws_max ? htp_executor_scratch(4, ws_max) : NULL;
  uint16_t *dst[3];
  for (int i = 0; i < 3; ++i) dst[i] = (uint16_t *)qkv_output(&out[i], 8 + i);
  if ((raw_tokens && !raw) || (ws_max && !ws) || !dst[0] || !dst[1] || !dst[2]) return -5;
  const float *d_pe = NULL;
  if (pe) {
    if (stage_in(pe, s)) return -5;
    d_pe = (const float *)aligned_input(pe, 16, 7, s);
    if (!d_pe) return -5;
  }
  event_set ev;
  if (events_open(&ev, 2)) {
    events_close(&ev);
    return -5;
  }
  int hrc = 0;
  for (int i = 0; i < n_parts && !hrc; ++i) {
    qkv_part *p = &parts[i];
    if (stage_in(&p->act, s) || stage_in(&p->q_norm, s) || stage_in(&p->k_norm, s) ||
        (p->has_bias && stage_in(&p->bias, s))) {
      hrc = HB_E_HIP;
      break;
    }
    const float *x = (const float *)aligned_input(&p->act, 16, 2, s);
    const float *qn = (const float *)aligned_input(&p->q_norm, 4, 5, s);
    const float *kn = (const float *)aligned_input(&p->k_norm, 4, 6, s);
    const float *b = p->has_bias ? (const float *)aligned_input(&p->bias, 4, 0, s) : NULL;
    if (!x || !qn || !kn || (p->has_bias && !b)) {
      hrc = HB_E_HIP;
      break;
    }
    if (i == 0) hrc = hb_event_record(ev.e[0], s);
    if (!hrc && fused[i])
      hrc = hb_qkv_gemm(dst[0], dst[1], dst[2], x, (const uint16_t *)packed[i], b, qn, kn, d_pe, p->rope_offset,
                        rope_count, p->tokens, input_dim, n_heads, head_dim, token_tiles, p->out_offset, ws, ws_max,
                        s);
    if (!hrc && !fused[i])
      hrc = hb_f16_gemm_ws(raw, x, (const uint16_t *)packed[i], NULL, p->tokens, input_dim, ncols, ncols, 0, ws,
                           ws_max, s);
    if (!hrc && !fused[i])
      hrc = hb_qkv_post(dst[0], dst[1], dst[2], raw, b, qn, kn, d_pe, p->rope_offset, rope_count, p->tokens, n_heads,
                        head_dim, token_tiles, p->out_offset, s);
  }
  if (!hrc) hrc = hb_event_record(ev.e[1], s);
  for (int i = 0; i < 3 && !hrc; ++i)
    if ((void *)dst[i] != out[i].dev) hrc = hb_memcpy_d2d(out[i].dev, dst[i], out[i].bytes, s);
  if (hrc) {
    events_close(&ev);
    return hrc == HB_E_INVAL ? -1 : -5;
  }
  for (int i = 0; i < 3; ++i) htp_registry_touch(out[i].fd, out[i].offset, out[i].bytes);
  const int device_outputs = out[0].is_device && out[1].is_device && out[2].is_device;
  if (complete(&ev, 0, 1, elapsed_dst, extra_us, device_outputs)) return -5;
  for (int i = 0; i < 3; ++i)
    if (stage_out(&out[i], s)) return -5;
  return 0;
}

/* Output views of q / k_out / v: n_heads * token_tiles * head_dim * 32 fp16
 * each, 128-byte aligned (reference src/dsp/ops/mat_mul.c:1385-1388). */
static int qkv_resolve_outputs(htp_view out[3], const struct RpcmemBufAddr *q, const struct RpcmemBufAddr *k,
                               const struct RpcmemBufAddr *v, size_t bytes) {
  int rc = resolve(q, bytes, &out[0], -1);
  if (!rc) rc = resolve(k, bytes, &out[1], -1);
  if (!rc) rc = resolve(v, bytes, &out[2], -1);
  if (rc) return rc;
  if ((primary_address(&out[0]) | primary_address(&out[1]) | primary_address(&out[2])) & 127u) return -1;
  return 0;
}

/* Sizes shared by the four opcodes: output bytes for `token_tiles`, weight,
 * bias and norm bytes (reference src/dsp/op_executor.cc:244-272, :554-572). */
static int qkv_sizes(int token_tiles, int input_dim, int n_heads, int head_dim, size_t *qkv_bytes,
                     size_t *weight_bytes, size_t *bias_bytes, size_t *norm_bytes) {
  const size_t cols = (size_t)n_heads * (size_t)head_dim * 3u;
  if (!checked_mul((size_t)token_tiles * (size_t)n_heads, (size_t)head_dim / 32u * 1024u * 2u, qkv_bytes) ||
      !checked_mul((size_t)input_dim, cols * 2u, weight_bytes))
    return -1;
  *bias_bytes = cols * sizeof(float);
  *norm_bytes = (size_t)head_dim * sizeof(float);
  return 0;
}

/* Opcodes 8 and 11 (reference src/dsp/op_executor.cc:542-595, :645-705). */
static int exec_qkv_single(uint8_t *payload, size_t payload_size, int rope) {
  const size_t need = rope ? sizeof(struct QkvMulRmsPackedRopeParams) : sizeof(struct QkvMulRmsPackedParams);
  if (payload_size < need) return -1;
  struct QkvMulRmsPackedRopeParams p;
  memset(&p, 0, sizeof(p));
  if (rope) {
    memcpy(&p, payload, sizeof(p));
  } else {
    struct QkvMulRmsPackedParams b;
    memcpy(&b, payload, sizeof(b));
    p.q = b.q, p.k_out = b.k_out, p.v = b.v, p.activation = b.activation, p.weight = b.weight, p.bias = b.bias;
    p.q_norm = b.q_norm, p.k_norm = b.k_norm;
    p.tokens = b.tokens, p.input_dim = b.input_dim, p.n_heads = b.n_heads, p.head_dim = b.head_dim;
  }
  if (p.tokens <= 0 || p.input_dim <= 0 || !htp_packed_shape_supported(p.n_heads, p.n_heads, p.head_dim, 1) ||
      p.input_dim % 32 || (rope && (p.rope_token_offset < 0 || p.rope_token_count <= 0)))
    return -1;
  const int token_tiles = (p.tokens + 31) / 32;
  size_t qkv_bytes, weight_bytes, bias_bytes, norm_bytes, pe_bytes = 0;
  if (qkv_sizes(token_tiles, p.input_dim, p.n_heads, p.head_dim, &qkv_bytes, &weight_bytes, &bias_bytes,
                &norm_bytes) ||
      (rope && !checked_mul((size_t)p.rope_token_count, (size_t)p.head_dim / 2u * 4u * sizeof(float), &pe_bytes)))
    return -1;
  htp_view out[3], pe;
  qkv_part part;
  memset(&part, 0, sizeof(part));
  int rc = qkv_resolve_outputs(out, &p.q, &p.k_out, &p.v, qkv_bytes);
  if (!rc) rc = qkv_resolve_part(&part, &p.activation, &p.weight, &p.bias, !rope, &p.q_norm, &p.k_norm, p.tokens,
                                 p.input_dim, weight_bytes, bias_bytes, norm_bytes);
  if (rc) return rc;
  /* an unmapped rotary table leaves the rows unrotated (reference
   * src/dsp/ops/mat_mul.c:1212-1214 returns on a NULL table) */
  const int have_pe = rope && resolve(&p.rope_pe, pe_bytes, &pe, -1) == 0;
  part.rope_offset = p.rope_token_offset;
  uint8_t *elapsed = payload + (rope ? offsetof(struct QkvMulRmsPackedRopeParams, elapsed_us)
                                     : offsetof(struct QkvMulRmsPackedParams, elapsed_us));
  return run_qkv(out, &part, 1, have_pe ? &pe : NULL, p.rope_token_count, p.input_dim, p.n_heads, p.head_dim,
                 token_tiles, elapsed);
}

/* Opcodes 10 and 12: image tokens (a multiple of 32) then text tokens in one
 * packed output, each half with its own activation, weight, bias and norms
 * (reference src/dsp/op_executor.cc:597-643, :707-770, src/dsp/ops/mat_mul.c:1515-1583). */
static int exec_qkv_dual(uint8_t *payload, size_t payload_size, int rope) {
  const size_t need = rope ? sizeof(struct QkvMulRmsPackedDualRopeParams) : sizeof(struct QkvMulRmsPackedDualParams);
  if (payload_size < need) return -1;
  struct QkvMulRmsPackedDualRopeParams p;
  memset(&p, 0, sizeof(p));
  if (rope) {
    memcpy(&p, payload, sizeof(p));
  } else {
    /* the dual payload is the dual RoPE payload without rope_pe and the offsets */
    struct QkvMulRmsPackedDualParams b;
    memcpy(&b, payload, sizeof(b));
    memcpy(&p, &b, offsetof(struct QkvMulRmsPackedDualParams, image_tokens));
    p.image_tokens = b.image_tokens, p.text_tokens = b.text_tokens, p.input_dim = b.input_dim;
    p.n_heads = b.n_heads, p.head_dim = b.head_dim;
  }
  if (p.image_tokens <= 0 || p.text_tokens <= 0 || p.image_tokens % 32 || p.input_dim <= 0 || p.input_dim % 32 ||
      !htp_packed_shape_supported(p.n_heads, p.n_heads, p.head_dim, 1) ||
      p.text_tokens > INT32_MAX - p.image_tokens ||
      (rope && (p.image_rope_token_offset < 0 || p.text_rope_token_offset < 0)))
    return -1;
  const int combined = p.image_tokens + p.text_tokens;
  const int token_tiles = (combined + 31) / 32;
  size_t qkv_bytes, weight_bytes, bias_bytes, norm_bytes, pe_bytes = 0;
  if (qkv_sizes(token_tiles, p.input_dim, p.n_heads, p.head_dim, &qkv_bytes, &weight_bytes, &bias_bytes,
                &norm_bytes))
    return -1;
  if (rope) {
    const int64_t a = (int64_t)p.image_rope_token_offset + p.image_tokens;
    const int64_t b = (int64_t)p.text_rope_token_offset + p.text_tokens;
    if (!checked_mul((size_t)(a > b ? a : b), (size_t)p.head_dim / 2u * 4u * sizeof(float), &pe_bytes)) return -1;
  }
  htp_view out[3], pe;
  qkv_part parts[2];
  memset(parts, 0, sizeof(parts));
  int rc = qkv_resolve_outputs(out, &p.q, &p.k_out, &p.v, qkv_bytes);
  if (!rc) rc = qkv_resolve_part(&parts[0], &p.image_activation, &p.image_weight, &p.image_bias, 0, &p.image_q_norm,
                                 &p.image_k_norm, p.image_tokens, p.input_dim, weight_bytes, bias_bytes, norm_bytes);
  if (!rc) rc = qkv_resolve_part(&parts[1], &p.text_activation, &p.text_weight, &p.text_bias, 0, &p.text_q_norm,
                                 &p.text_k_norm, p.text_tokens, p.input_dim, weight_bytes, bias_bytes, norm_bytes);
  if (rc) return rc;
  const int have_pe = rope && resolve(&p.rope_pe, pe_bytes, &pe, -1) == 0;
  parts[0].out_offset = 0;
  parts[1].out_offset = p.image_tokens;
  parts[0].rope_offset = p.image_rope_token_offset;
  parts[1].rope_offset = p.text_rope_token_offset;
  uint8_t *elapsed = payload + (rope ? offsetof(struct QkvMulRmsPackedDualRopeParams, elapsed_us)
                                     : offsetof(struct QkvMulRmsPackedDualParams, elapsed_us));
  /* both halves rotate tokens below image_tokens + text_tokens */
  return run_qkv(out, parts, 2, have_pe ? &pe : NULL, combined, p.input_dim, p.n_heads, p.head_dim, token_tiles,
                 elapsed);
}

/* ---- opcode 19 ------------------------------------------------------------------- */

/* A device pointer with 4-byte alignment for an optional input view (NULL view: NULL). */
static const float *aux_input(const htp_view *v, int slot, hb_stream s, int *failed) {
  if (!v) return NULL;
  if (stage_in(v, s)) {
    *failed = 1;
    return NULL;
  }
  const float *p = (const float *)aligned_input(v, 4, slot, s);
  if (!p) *failed = 1;
  return p;
}

static int exec_model_aux(uint8_t *payload, size_t payload_size) {
  /* reference src/dsp/op_executor.cc:371-404, src/dsp/ops/mat_mul.c:2488-2501 */
  if (payload_size != sizeof(struct NativeAuxParams)) return -1;
  struct NativeAuxParams p;
  memcpy(&p, payload, sizeof(p));
  if (p.count <= 0 || p.mode < 0 || p.mode > 13 || p.width <= 0 || p.channels <= 0 || p.spatial <= 0 ||
      p.batch <= 0)
    return -1;
  const int64_t wsb = (int64_t)p.width * p.spatial * p.batch;
  const int has_w = p.weight.fd >= 0, has_b = p.bias.fd >= 0;
  if (p.mode == 8 && wsb != p.count) return -1;
  if (p.mode == 2 && (p.groups <= 0 || p.channels % p.groups)) return -1;
  /* Deviation: the reference does not check that a group norm's batch x
   * channels x spatial values lie inside `count` (its kernel would read past
   * the input); such a request is rejected here. */
  if (p.mode == 2 && (int64_t)p.batch * p.channels * p.spatial > p.count) return -1;
  if (p.mode == 12 && (wsb != p.count || has_w || has_b || p.channels < (int64_t)2 * p.width ||
                       (p.activation != 0 && p.activation != 1)))
    return -1;
  if (p.mode == 13 && (p.groups <= 0 || !has_w || has_b ||
                       ((int64_t)p.width + p.groups) * p.spatial * p.batch != p.count ||
                       (int64_t)p.groups * p.spatial * p.batch != p.other_count ||
                       p.channels < (int64_t)2 * p.width || (p.activation != 0 && p.activation != 1)))
    return -1;
  if ((p.mode == 9 || p.mode == 10) &&
      (wsb != p.count || !has_w || !has_b ||
       (p.other_count != p.width && p.other_count != (int64_t)p.width * p.batch) ||
       (p.mode == 9 && (!isfinite(p.eps) || p.eps < 0))))
    return -1;
  if (p.mode == 11 && (p.width % 2 || (int64_t)p.width * p.channels * p.spatial * p.batch != p.count || !has_w ||
                       has_b || (p.groups != 1 && p.groups != p.batch) ||
                       p.other_count != (int64_t)2 * p.width * p.spatial * p.groups))
    return -1;
  const int n = p.mode == 2 ? p.channels : p.mode == 9 ? p.other_count : p.mode == 10 ? p.count : p.width;
  if (p.mode <= 2 && has_w && p.other_count != n) return -1;
  if ((p.mode == 3 || p.mode == 4) && (p.other_count <= 0 || p.count % p.other_count || !has_w)) return -1;
  size_t input_bytes = (size_t)p.count * 4u;
  if (p.mode == 12 || p.mode == 13)
    input_bytes = ((size_t)p.spatial * (size_t)p.batch - 1u) * (size_t)p.channels * 4u + (size_t)2 * p.width * 4u;
  htp_view out, in, wgt, bias;
  int rc = resolve(&p.output, (size_t)p.count * 4u, &out, -1);
  if (!rc) rc = resolve(&p.input, input_bytes, &in, -1);
  if (!rc && has_w) rc = resolve(&p.weight, (size_t)p.other_count * 4u, &wgt, -1);
  if (!rc && has_b) rc = resolve(&p.bias, (size_t)n * 4u, &bias, -1);
  if (rc) return rc;
  /* The reference's worker pool refuses a call with no task (mat_mul.c:2491). */
  if ((p.mode <= 1 || p.mode == 9) && p.count / p.width == 0) return -40;
  if (htp_executor_ensure_device() != 0) return -5;
  if (materialize(&out) || materialize(&in) || (has_w && materialize(&wgt)) || (has_b && materialize(&bias)))
    return -5;
  hb_stream s = htp_executor_stream();
  int failed = 0;
  const float *x = aux_input(&in, 2, s, &failed);
  const float *w = aux_input(has_w ? &wgt : NULL, 0, s, &failed);
  const float *b = aux_input(has_b ? &bias : NULL, 1, s, &failed);
  if (failed) return -5;
  float *y = ((uintptr_t)out.dev % 4u) == 0 ? (float *)out.dev : (float *)htp_executor_scratch(3, out.bytes);
  if (!y) return -5;
  /* Values a mode does not write keep their contents: the norms cover whole
   * rows (modes 0/1) or groups (mode 2) only. */
  int64_t covered = p.count;
  if (p.mode <= 1) covered = (int64_t)(p.count / p.width) * p.width;
  if (p.mode == 2) covered = (int64_t)p.batch * p.spatial * p.channels;
  if (covered < p.count) {
    if (stage_in(&out, s)) return -5;
    if ((void *)y != (void *)out.dev && hb_memcpy_d2d(y, out.dev, out.bytes, s) != HB_OK) return -5;
  }
  event_set ev;
  if (events_open(&ev, 2)) {
    events_close(&ev);
    return -5;
  }
  /* Group norms over few long groups split each group: partial sums in scratch. */
  const size_t ws_bytes = hb_model_aux_workspace_bytes(p.mode, p.channels, p.spatial, p.groups, p.batch);
  void *ws = ws_bytes ? htp_executor_scratch(4, ws_bytes) : NULL;
  if (ws_bytes && !ws) {
    events_close(&ev);
    return -5;
  }
  int hrc = hb_event_record(ev.e[0], s);
  if (!hrc)
    hrc = hb_model_aux_ws(y, x, w, b, p.mode, p.count, p.width, p.channels, p.spatial, p.groups, p.batch,
                          p.other_count, p.activation, p.eps, ws, ws_bytes, s);
  if (!hrc) hrc = hb_event_record(ev.e[1], s);
  if (!hrc && (void *)y != (void *)out.dev) hrc = hb_memcpy_d2d(out.dev, y, out.bytes, s);
  if (hrc) {
    events_close(&ev);
    return hrc == HB_E_INVAL ? -1 : -5;
  }
  htp_registry_touch(out.fd, out.offset, out.bytes);
  if (complete(&ev, 0, 1, payload + offsetof(struct NativeAuxParams, elapsed_us), 0.0, out.is_device)) return -5;
  return stage_out(&out, s) ? -5 : 0;
}

/* ---- dispatcher ---------------------------------------------------------------- */

int execute_op_simple(struct OpComputeRequest *req, size_t req_size) {
  if (req == NULL || req_size < sizeof(struct OpComputeRequest)) return -1;
  const size_t payload_size = req_size - sizeof(struct OpComputeRequest);
  uint8_t *payload = (uint8_t *)req + sizeof(struct OpComputeRequest);
  uint32_t op;
  memcpy(&op, req, sizeof(op));
  int rc;
  pthread_mutex_lock(&g_exec_lock);
  switch (op) {
    case HTP_OPS_MAT_MUL_NATIVE_W8A8: rc = exec_w8a8(payload, payload_size); break;
    case HTP_OPS_MAT_MUL_F16_EPILOGUE: rc = exec_f16_epilogue(payload, payload_size); break;
    case HTP_OPS_MAT_MUL_PERMUTED_W16A32: rc = exec_matmul(payload, payload_size); break;
    case HTP_OPS_MAT_MUL_PERMUTED_W4D16A32:
      rc = exec_matmul_qk0(payload, payload_size, HTP_WEIGHT_Q4_0, HB_GGML_Q4_0);
      break;
    case HTP_OPS_MAT_MUL_PERMUTED_W8D16A32:
      rc = exec_matmul_qk0(payload, payload_size, HTP_WEIGHT_Q8_0, HB_GGML_Q8_0);
      break;
    case HTP_OPS_MAT_MUL_PERMUTED_W4D16A32_IQ4_NL:
      rc = exec_matmul_qk0(payload, payload_size, HTP_WEIGHT_IQ4_NL, HB_GGML_IQ4_NL);
      break;
    case HTP_OPS_MODEL_AUX_F32: rc = exec_model_aux(payload, payload_size); break;
    case HTP_OPS_QKV_MUL_RMS_PACKED_W16A32: rc = exec_qkv_single(payload, payload_size, 0); break;
    case HTP_OPS_QKV_MUL_RMS_PACKED_ROPE_W16A32: rc = exec_qkv_single(payload, payload_size, 1); break;
    case HTP_OPS_QKV_MUL_RMS_PACKED_DUAL_W16A32: rc = exec_qkv_dual(payload, payload_size, 0); break;
    case HTP_OPS_QKV_MUL_RMS_PACKED_DUAL_ROPE_W16A32: rc = exec_qkv_dual(payload, payload_size, 1); break;
    default: rc = HTP_OPS_E_UNSUPPORTED; break;
  }
  pthread_mutex_unlock(&g_exec_lock);
  return rc;
}

int htp_ops_execute_message(struct MessageHeader *msg, size_t capacity) {
  size_t total = 0;
  if (!message_header_validate_layout(msg, capacity, &total)) return -1;
  htp_channel_process(NULL, msg, capacity, 0);
  return 0;
}
