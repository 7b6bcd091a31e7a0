/*
 * CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this code; the product library (htp-ops-lib-sd.cpp_amd) never does.
 *
 * Build: gcc -std=c11 -O3 -march=native -ffp-contract=off -fno-fast-math -pthread
 *
 * Each function names the reference lines it restates.  Parity status of each
 * function (what pins it) is listed in tests/test_oracle.py and DESIGN.md.
 */
#define _GNU_SOURCE
#include "htp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* helpers                                                                   */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof(u));
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof(f));
  return f;
}

int oracle_num_threads(void) {
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n < 1 ? 1 : (int)n;
}

typedef void (*range_fn)(void *ctx, int begin, int end);

typedef struct {
  range_fn fn;
  void *ctx;
  int begin, end;
} range_job;

static void *range_thread(void *arg) {
  range_job *job = (range_job *)arg;
  job->fn(job->ctx, job->begin, job->end);
  return NULL;
}

/* Runs fn over [0, total) split into contiguous chunks on nthreads threads. */
static void parallel_for(int total, int nthreads, range_fn fn, void *ctx) {
  if (nthreads <= 0) nthreads = oracle_num_threads();
  if (nthreads > total) nthreads = total;
  if (nthreads <= 1) {
    if (total > 0) fn(ctx, 0, total);
    return;
  }
  pthread_t *threads = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
  range_job *jobs = (range_job *)malloc(sizeof(range_job) * (size_t)nthreads);
  for (int t = 0; t < nthreads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].begin = (int)((long long)total * t / nthreads);
    jobs[t].end = (int)((long long)total * (t + 1) / nthreads);
  }
  for (int t = 1; t < nthreads; ++t) pthread_create(&threads[t], NULL, range_thread, &jobs[t]);
  range_thread(&jobs[0]);
  for (int t = 1; t < nthreads; ++t) pthread_join(threads[t], NULL);
  free(jobs);
  free(threads);
}

/* ------------------------------------------------------------------------ */
/* binary16 conversion (IEEE 754-2008 binary16, round to nearest even)      */
/* Stands for the reference's fp32->fp16 activation conversion              */
/* (hvx_convert.h:5-12, mat_mul.c:114-148) and the HMX cvt.hf readout        */
/* (hmx_utils.h:34-40), both defined here as IEEE RNE.                       */
/* ------------------------------------------------------------------------ */

uint16_t oracle_f32_to_f16(float x) {
  const uint32_t u = f32_bits(x);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t absu = u & 0x7fffffffu;
  if (absu >= 0x7f800000u) { /* inf or nan */
    if (absu == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((absu >> 13) & 0x3ffu));
  }
  const int exp = (int)(absu >> 23) - 127;
  if (exp > 15) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  uint32_t mant = (absu & 0x7fffffu) | 0x800000u;  /* 24-bit significand */
  int shift;                                       /* bits dropped from the 24-bit significand */
  uint32_t biased;
  if (exp >= -14) { /* normal half */
    shift = 13;
    biased = (uint32_t)(exp + 15);
  } else { /* subnormal half (or underflow to zero) */
    if (absu == 0) return sign;
    shift = 13 + (-14 - exp);
    biased = 0;
    if (shift > 25) return sign; /* below half of the smallest subnormal */
  }
  uint32_t q = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  if (biased == 0) {
    /* q counts subnormal units; a carry into 0x400 yields the smallest normal */
    return (uint16_t)(sign | q);
  }
  /* q has the implicit bit at 0x400; a carry to 0x800 bumps the exponent */
  uint32_t e = biased;
  if (q & 0x800u) {
    q >>= 1;
    ++e;
  }
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (e << 10) | (q & 0x3ffu));
}

void oracle_f32_to_f16_array(uint16_t *dst, const float *src, size_t count) {
  for (size_t i = 0; i < count; ++i) dst[i] = oracle_f32_to_f16(src[i]);
}

void oracle_f16_to_f32_array(float *dst, const uint16_t *src, size_t count) {
  for (size_t i = 0; i < count; ++i) dst[i] = oracle_f16_to_f32(src[i]);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  if (e == 0) {
    if (m == 0) return bits_f32(sign);
    /* subnormal: value = m * 2^-24, exact in binary32 */
    float v = (float)m * 0x1p-24f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* ------------------------------------------------------------------------ */
/* W8A8 constants blob (reference include/op_reg.h:80-85,                  */
/* src/dsp/op_executor.cc:321-335; weight addressing                        */
/* src/dsp/ops/linear_w8a8.c:453,482,486-488 and                            */
/* tests/hmx-probe/study_dsp.c:82-84)                                       */
/* ------------------------------------------------------------------------ */

size_t oracle_w8a8_blob_bytes(int k, int n) {
  return 128u + (size_t)k * (size_t)n + (size_t)n * 8u + (size_t)k * 4u;
}

size_t oracle_w8a8_weight_offset(int k, int n_idx, int k_idx) {
  return 128u + (size_t)(n_idx / 64) * 64u * (size_t)k + (size_t)(k_idx / 32) * 2048u +
         (size_t)((n_idx % 64) / 32) * 1024u + (size_t)((k_idx % 32) / 4) * 128u + (size_t)(n_idx % 32) * 4u +
         (size_t)(k_idx % 4);
}

static void put_u32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }
static uint32_t get_u32(const uint8_t *p) {
  uint32_t v;
  memcpy(&v, p, 4);
  return v;
}

void oracle_w8a8_pack_blob(uint8_t *blob, const int8_t *w, const float *sw, const int32_t *sums,
                           const float *inv, int k, int n, uint64_t signature) {
  const size_t kn = (size_t)k * (size_t)n;
  memset(blob, 0, 128);
  put_u32(blob + 0, 0x38574d48u);
  put_u32(blob + 4, 1u);
  put_u32(blob + 8, (uint32_t)k);
  put_u32(blob + 12, (uint32_t)n);
  put_u32(blob + 16, 128u);
  put_u32(blob + 20, (uint32_t)(128u + kn));
  put_u32(blob + 24, (uint32_t)(128u + kn + 4u * (size_t)n));
  put_u32(blob + 28, (uint32_t)(128u + kn + 8u * (size_t)n));
  put_u32(blob + 32, (uint32_t)oracle_w8a8_blob_bytes(k, n));
  memcpy(blob + 40, &signature, 8);
  for (int c = 0; c < n; ++c)
    for (int r = 0; r < k; ++r) blob[oracle_w8a8_weight_offset(k, c, r)] = (uint8_t)w[(size_t)c * k + r];
  uint8_t *scale = blob + 128 + kn;
  uint8_t *sum = scale + 4u * (size_t)n;
  uint8_t *inverse = sum + 4u * (size_t)n;
  for (int c = 0; c < n; ++c) {
    memcpy(scale + 4u * (size_t)c, &sw[c], 4);
    int32_t s = 0;
    if (sums) {
      s = sums[c];
    } else {
      for (int r = 0; r < k; ++r) s += w[(size_t)c * k + r];
    }
    memcpy(sum + 4u * (size_t)c, &s, 4);
  }
  for (int r = 0; r < k; ++r) {
    const float one = 1.0f;
    memcpy(inverse + 4u * (size_t)r, inv ? &inv[r] : &one, 4);
  }
}

void oracle_w8a8_unpack_weights(int8_t *w, const uint8_t *blob, int k, int n) {
  for (int c = 0; c < n; ++c)
    for (int r = 0; r < k; ++r) w[(size_t)c * k + r] = (int8_t)blob[oracle_w8a8_weight_offset(k, c, r)];
}

/* Header acceptance of reference src/dsp/op_executor.cc:331-335; -3 on mismatch. */
int oracle_w8a8_check_header(const uint8_t *blob, int k, int n) {
  const size_t kn = (size_t)k * (size_t)n;
  const size_t scale = 128u + kn;
  if (get_u32(blob + 0) != 0x38574d48u || get_u32(blob + 4) != 1u || get_u32(blob + 8) != (uint32_t)k ||
      get_u32(blob + 12) != (uint32_t)n || get_u32(blob + 16) != 128u || get_u32(blob + 20) != scale ||
      get_u32(blob + 24) != scale + 4u * (size_t)n || get_u32(blob + 28) != get_u32(blob + 24) + 4u * (size_t)n ||
      get_u32(blob + 32) != oracle_w8a8_blob_bytes(k, n))
    return -3;
  return 0;
}

/* ------------------------------------------------------------------------ */
/* W8A8 activation quantization                                             */
/* ------------------------------------------------------------------------ */

/*
 * Clamp of v to [1, 255] done on the IEEE bit pattern as signed integers
 * (negative values and -NaN -> 1.0, +NaN and values above 255 -> 255.0),
 * then round-to-nearest-even of the significand by shifting
 * (reference src/dsp/ops/linear_w8a8.c:47-58).
 */
uint8_t oracle_w8a8_quantize_value(float v) {
  int32_t b = (int32_t)f32_bits(v);
  const int32_t lo = (int32_t)f32_bits(1.0f), hi = (int32_t)f32_bits(255.0f);
  if (b < lo) b = lo;
  if (b > hi) b = hi;
  const int32_t e = (int32_t)(((uint32_t)b >> 23) & 0xffu) - 127; /* 0..7 */
  const int32_t shift = 23 - e;                                   /* 16..23 */
  const int32_t mant = (b & 0x7fffff) | 0x800000;
  const int32_t whole = mant >> shift;
  const int32_t half = 1 << (shift - 1);
  return (uint8_t)((mant + (half - 1) + (whole & 1)) >> shift);
}

void oracle_w8a8_quantize_values(uint8_t *dst, const float *v, size_t count) {
  for (size_t i = 0; i < count; ++i) dst[i] = oracle_w8a8_quantize_value(v[i]);
}

typedef struct {
  uint8_t *u;
  float *s;
  const float *x;
  const float *inv;
  int k;
} quant_ctx;

/*
 * Per-token dynamic quantization, reference src/dsp/ops/linear_w8a8.c:
 *   t[k] = x[k]*inv[k]                              :83-87
 *   s    = fmaxf(max_k |t[k]| / 127, 1e-12f)         :34-40, :92-95, :102-105
 *   r    = 1/s                                      :106-109
 *   u[k] = rne(clamp(t[k]*r + 128, 1, 255))           :42-59, :110-118
 */
static void quant_rows(void *arg, int begin, int end) {
  quant_ctx *c = (quant_ctx *)arg;
  const int k = c->k;
  float *t = (float *)malloc(sizeof(float) * (size_t)k);
  for (int row = begin; row < end; ++row) {
    const float *x = c->x + (size_t)row * k;
    float amax = 0.0f;
    for (int i = 0; i < k; ++i) {
      t[i] = x[i] * c->inv[i];
      const float a = fabsf(t[i]);
      if (a > amax) amax = a;
    }
    const float s = fmaxf(amax / 127.0f, 1e-12f);
    const float r = 1.0f / s;
    c->s[row] = s;
    uint8_t *u = c->u + (size_t)row * k;
    for (int i = 0; i < k; ++i) {
      const float scaled = t[i] * r;
      const float v = scaled + 128.0f;
      u[i] = oracle_w8a8_quantize_value(v);
    }
  }
  free(t);
}

void oracle_w8a8_quantize(uint8_t *u, float *s, const float *x, const float *inv, int m, int k, int nthreads) {
  quant_ctx c = {u, s, x, inv, k};
  parallel_for(m, nthreads, quant_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* W8A8 integer accumulation: acc[m][n] = sum_k u[m][k] * W(n,k) (int32)     */
/* reference src/dsp/ops/linear_w8a8.c:478-502 (HMX u8 x s8 MAC), :130-138   */
/* ------------------------------------------------------------------------ */

typedef struct {
  int32_t *acc;
  const uint8_t *u;
  const int8_t *w; /* [n][k] */
  int k, n;
} acc_ctx;

static void acc_rows(void *arg, int begin, int end) {
  acc_ctx *c = (acc_ctx *)arg;
  const int k = c->k, n = c->n;
  const int nblock = 128;
  for (int n0 = 0; n0 < n; n0 += nblock) {
    const int n1 = n0 + nblock < n ? n0 + nblock : n;
    for (int row = begin; row < end; ++row) {
      const uint8_t *u = c->u + (size_t)row * k;
      int32_t *out = c->acc + (size_t)row * n;
      for (int col = n0; col < n1; ++col) {
        const int8_t *w = c->w + (size_t)col * k;
        int32_t sum = 0;
        for (int i = 0; i < k; ++i) sum += (int32_t)u[i] * (int32_t)w[i];
        out[col] = sum;
      }
    }
  }
}

void oracle_w8a8_accumulate(int32_t *acc, const uint8_t *u, const uint8_t *blob, int m, int k, int n,
                            int nthreads) {
  int8_t *w = (int8_t *)malloc((size_t)k * (size_t)n);
  oracle_w8a8_unpack_weights(w, blob, k, n);
  acc_ctx c = {acc, u, w, k, n};
  parallel_for(m, nthreads, acc_rows, &c);
  free(w);
}

/* ------------------------------------------------------------------------ */
/* W8A8 output: c = acc - (sums[n] << 7) (int32 wrap);                      */
/*              y = ((float)c * sw[n]) * s[m]                                */
/* reference src/dsp/ops/linear_w8a8.c:140-192                              */
/* ------------------------------------------------------------------------ */

typedef struct {
  float *y;
  const int32_t *acc;
  const float *s;
  const float *sw;
  const int32_t *sums;
  int n;
} out_ctx;

static void out_rows(void *arg, int begin, int end) {
  out_ctx *c = (out_ctx *)arg;
  for (int row = begin; row < end; ++row) {
    for (int col = 0; col < c->n; ++col) {
      const size_t i = (size_t)row * c->n + col;
      const int32_t corrected = (int32_t)((uint32_t)c->acc[i] - ((uint32_t)c->sums[col] << 7));
      const float value = (float)corrected;
      const float scaled = value * c->sw[col];
      c->y[i] = scaled * c->s[row];
    }
  }
}

void oracle_w8a8_output(float *y, const int32_t *acc, const float *s, const uint8_t *blob, int m, int k, int n,
                        int nthreads) {
  const size_t kn = (size_t)k * (size_t)n;
  float *sw = (float *)malloc(sizeof(float) * (size_t)n);
  int32_t *sums = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
  memcpy(sw, blob + 128 + kn, 4u * (size_t)n);
  memcpy(sums, blob + 128 + kn + 4u * (size_t)n, 4u * (size_t)n);
  out_ctx c = {y, acc, s, sw, sums, n};
  parallel_for(m, nthreads, out_rows, &c);
  free(sums);
  free(sw);
}

/* Whole opcode-15 computation on a blob; no envelope checks (K may exceed the
 * reference's 6144 limit, int32 stays exact up to K = 65535). */
void oracle_w8a8_linear(float *y, const float *x, const uint8_t *blob, int m, int k, int n, int nthreads) {
  const size_t kn = (size_t)k * (size_t)n;
  const float *inv_src = (const float *)(const void *)(blob + 128 + kn + 8u * (size_t)n);
  float *inv = (float *)malloc(sizeof(float) * (size_t)k);
  memcpy(inv, inv_src, 4u * (size_t)k);
  uint8_t *u = (uint8_t *)malloc((size_t)m * (size_t)k);
  float *s = (float *)malloc(sizeof(float) * (size_t)m);
  int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)m * (size_t)n);
  oracle_w8a8_quantize(u, s, x, inv, m, k, nthreads);
  oracle_w8a8_accumulate(acc, u, blob, m, k, n, nthreads);
  oracle_w8a8_output(y, acc, s, blob, m, k, n, nthreads);
  free(acc);
  free(s);
  free(u);
  free(inv);
}

/*
 * Raw-plane export of the CPU-control variant (reference
 * src/dsp/ops/linear_w8a8.c:209-227, byte order from :159-171): for every
 * 64-row tile and 32-column half, the four little-endian byte planes of the
 * raw accumulator (rows x 32 bytes each, plane 0 = low byte) are written as
 * one flat stream over the same rows x 128 bytes the f32 outputs occupy.
 */
void oracle_w8a8_planes(uint8_t *out, const int32_t *acc, int m, int n) {
  for (int tile = 0; tile * 64 < m; ++tile) {
    const int rows = m - tile * 64 < 64 ? m - tile * 64 : 64;
    for (int n0 = 0; n0 < n; n0 += 32) {
      for (int p = 0; p < 4; ++p) {
        for (int r = 0; r < rows; ++r) {
          for (int c = 0; c < 32; ++c) {
            const uint32_t v = (uint32_t)acc[(size_t)(tile * 64 + r) * n + n0 + c];
            const size_t flat = (size_t)p * rows * 32u + (size_t)r * 32u + (size_t)c;
            const size_t row = (size_t)tile * 64u + flat / 128u;
            out[(row * (size_t)n + (size_t)n0) * 4u + flat % 128u] = (uint8_t)(v >> (8 * p));
          }
        }
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Epilogue activations, reference src/dsp/ops/mat_mul.c:788-826             */
/* (mode 1: z*sigmoid(1.5957691216057308*(z + 0.044715*z^3)); mode 2:        */
/* z*sigmoid(1.702*z); sigmoid in the stable form e/(1+e) for negative       */
/* arguments and 1/(1+e) otherwise with e = 2^max(-|a|*log2(e), -126)).      */
/* The reference evaluates 2^x with a degree-6 polynomial and the reciprocal */
/* with Newton steps in QFloat; the oracle uses libm exp2f and IEEE division.*/
/* ------------------------------------------------------------------------ */

static float stable_sigmoid(float a) {
  const float absa = fabsf(a);
  float neg = absa * -1.4426950408889634f;
  if (neg < -126.0f) neg = -126.0f;
  const float e = exp2f(neg);
  const float denom = e + 1.0f;
  const float inv = 1.0f / denom;
  return a < 0.0f ? e * inv : inv;
}

float oracle_gelu_tanh(float z) {
  const float cubic = (z * z) * z;
  const float inner = z + cubic * 0.044715f;
  const float a = inner * 1.5957691216057308f;
  return z * stable_sigmoid(a);
}

float oracle_quick_gelu(float z) {
  const float a = z * 1.702f;
  return z * stable_sigmoid(a);
}

void oracle_gelu_tanh_inplace(float *y, size_t count) {
  for (size_t i = 0; i < count; ++i) y[i] = oracle_gelu_tanh(y[i]);
}

/* ------------------------------------------------------------------------ */
/* Opcode 19 model auxiliary ops, reference src/dsp/ops/mat_mul.c:2356-2486 */
/* (task decomposition :2489).  Row sums accumulate in double, as the       */
/* reference's cross-lane sum does (:2352-2355); every float step is one    */
/* IEEE operation in the reference's order.  Activation ids: 1 GELU-tanh,   */
/* 2 QuickGELU, 4 and 5 SiLU (x*sigmoid(x)).                                */
/* ------------------------------------------------------------------------ */

float oracle_silu(float z) { return z * stable_sigmoid(z); }

static float aux_activate(float v, int act) {
  if (act == 1) return oracle_gelu_tanh(v);
  if (act == 2) return oracle_quick_gelu(v);
  if (act == 4 || act == 5) return oracle_silu(v);
  return v;
}

int oracle_model_aux(float *y, const float *x, const float *w, const float *b, int mode, int count, int width,
                     int channels, int spatial, int groups, int batch, int other_count, int activation, float eps) {
  if (count <= 0 || width <= 0 || channels <= 0 || spatial <= 0 || batch <= 0) return -1;
  if (mode <= 2 || mode == 9) {
    int tasks, len;
    if (mode == 2) {
      if (groups <= 0 || channels % groups) return -1;
      tasks = groups * batch;
      len = spatial * (channels / groups);
    } else {
      tasks = count / width;
      len = width;
    }
    for (int task = 0; task < tasks; ++task) {
      const size_t offset = (size_t)task * (size_t)len;
      const float *xr = x + offset;
      float mean = 0.0f;
      if (mode != 1) {
        double sum = 0.0;
        for (int i = 0; i < len; ++i) sum += (double)xr[i];
        mean = (float)(sum / (double)len);
      }
      double sq = 0.0;
      for (int i = 0; i < len; ++i) {
        const double v = (double)(xr[i] - mean);
        sq += v * v;
      }
      const float inv = 1.0f / sqrtf((float)(sq / (double)len + (double)eps));
      const size_t pbase = (mode == 9 && other_count != width) ? (size_t)(task / spatial) * (size_t)width : 0;
      for (int i = 0; i < len; ++i) {
        float v = (xr[i] - mean) * inv;
        if (mode == 0 || mode == 1) {
          if (w) v = v * w[i];
          if (b) v = v + b[i];
        } else if (mode == 2) {
          const int ch = (int)(((offset + (size_t)i) / (size_t)spatial) % (size_t)channels);
          if (w) v = v * w[ch];
          if (b) v = v + b[ch];
        } else {
          v = v + v * w[pbase + (size_t)i];
          v = v + b[pbase + (size_t)i];
        }
        if (activation) v = aux_activate(v, 4);
        y[offset + (size_t)i] = v;
      }
    }
    return 0;
  }
  switch (mode) {
    case 3:
    case 4:
      if (!w || other_count <= 0) return -1;
      for (int64_t i = 0; i < count; ++i)
        y[i] = mode == 3 ? x[i] + w[i % other_count] : x[i] * w[i % other_count];
      return 0;
    case 5:
    case 6:
    case 7:
      for (int64_t i = 0; i < count; ++i) y[i] = aux_activate(x[i], mode == 5 ? 4 : mode == 6 ? 1 : 2);
      return 0;
    case 8:
      if ((int64_t)width * spatial * batch != count) return -1;
      for (int bt = 0; bt < batch; ++bt)
        for (int r = 0; r < width; ++r)
          for (int c = 0; c < spatial; ++c)
            y[((size_t)bt * spatial + c) * width + r] = x[((size_t)bt * width + r) * spatial + c];
      return 0;
    case 10:
      if (!w || !b) return -1;
      for (int64_t i = 0; i < count; ++i) {
        const int64_t channel = i % width, bt = i / ((int64_t)width * spatial);
        const int64_t pb = other_count == width ? 0 : bt;
        y[i] = x[i] * w[pb * width + channel] + b[i];
      }
      return 0;
    case 11: {
      if (!w || width % 2 || (groups != 1 && groups != batch)) return -1;
      for (int bt = 0; bt < batch; ++bt)
        for (int token = 0; token < spatial; ++token) {
          const float *pe = w + ((size_t)(groups == 1 ? 0 : bt) * spatial + token) * (size_t)width * 2;
          for (int head = 0; head < channels; ++head) {
            const float *xs = x + (((size_t)bt * spatial + token) * channels + head) * width;
            float *ys = y + (((size_t)bt * channels + head) * spatial + token) * width;
            for (int e = 0; e < width; e += 2) {
              const float *m = pe + 2 * e;
              const float x0 = xs[e], x1 = xs[e + 1];
              ys[e] = x0 * m[0] + x1 * m[1];
              ys[e + 1] = x1 * m[3] + x0 * m[2];
            }
          }
        }
      return 0;
    }
    case 12:
      if (channels < 2 * width) return -1;
      for (int64_t i = 0; i < count; ++i) {
        const int64_t column = i % width, row = i / width;
        const float *a = x + row * channels + column;
        const float gate = a[activation ? 0 : width], up = a[activation ? width : 0];
        y[i] = aux_activate(gate, 5) * up;
      }
      return 0;
    case 13:
      if (!w || groups <= 0 || channels < 2 * width) return -1;
      for (int64_t r = 0; r < (int64_t)spatial * batch; ++r) {
        float *dst = y + r * (width + groups);
        for (int i = 0; i < groups; ++i) dst[i] = w[r * groups + i];
        const float *xr = x + r * channels;
        for (int i = 0; i < width; ++i) {
          const float gate = xr[i + (activation ? 0 : width)], up = xr[i + (activation ? width : 0)];
          dst[groups + i] = aux_activate(gate, 5) * up;
        }
      }
      return 0;
    default:
      return -1;
  }
}

/* ------------------------------------------------------------------------ */
/* Packed F16 GEMM with epilogue (opcodes 1/16)                             */
/* layout: reference src/host/test.c:547-558 (writer);                      */
/* semantics: reference src/dsp/ops/mat_mul.c:937-1049                      */
/* ------------------------------------------------------------------------ */

size_t oracle_f16_permuted_index(int k_total, int k_idx, int n_idx) {
  return ((size_t)(n_idx / 32) * (size_t)(k_total / 32) + (size_t)(k_idx / 32)) * 1024u +
         (size_t)((k_idx % 32) / 2) * 64u + (size_t)(n_idx % 32) * 2u + (size_t)(k_idx % 2);
}

void oracle_f16_permute(uint16_t *permuted, const uint16_t *w_kn, int k, int n) {
  for (int r = 0; r < k; ++r)
    for (int c = 0; c < n; ++c) permuted[oracle_f16_permuted_index(k, r, c)] = w_kn[(size_t)r * n + c];
}

typedef struct {
  float *y;
  const float *x;
  const double *w; /* [n][k] */
  const float *bias;
  int m, k, n, channels, mode;
} f16_ctx;

/*
 * a = fp16(x); acc = sum_k a*W exactly (double); h = fp16(acc); v = (float)h
 * (mat_mul.c:114-148 conversion, :724-748 HMX core, :751-778 readout), then
 *   mode 0: v + bias                        (:864-882)
 *   mode 1/2: activation(v + bias)          (:864-882, :788-826)
 *   mode 3: yt[c][row] = v + bias, c < channels  (:830-862)
 */
static void f16_rows(void *arg, int begin, int end) {
  f16_ctx *c = (f16_ctx *)arg;
  const int k = c->k, n = c->n;
  double *a = (double *)malloc(sizeof(double) * (size_t)k);
  for (int row = begin; row < end; ++row) {
    for (int i = 0; i < k; ++i) a[i] = (double)oracle_f16_to_f32(oracle_f32_to_f16(c->x[(size_t)row * k + i]));
    const int cols = c->mode == 3 ? c->channels : n;
    for (int col = 0; col < cols; ++col) {
      const double *w = c->w + (size_t)col * k;
      double acc = 0.0;
      for (int i = 0; i < k; ++i) acc += a[i] * w[i];
      const float v = oracle_f16_to_f32(oracle_f32_to_f16((float)acc));
      float z = c->bias ? v + c->bias[col] : v;
      if (c->mode == 1) z = oracle_gelu_tanh(z);
      if (c->mode == 2) z = oracle_quick_gelu(z);
      if (c->mode == 3)
        c->y[(size_t)col * c->m + row] = z;
      else
        c->y[(size_t)row * n + col] = z;
    }
  }
  free(a);
}

void oracle_f16_gemm_epilogue(float *y, const float *x, const uint16_t *permuted, const float *bias, int m, int k,
                              int n, int channels, int mode, int nthreads) {
  double *w = (double *)malloc(sizeof(double) * (size_t)k * (size_t)n);
  for (int c = 0; c < n; ++c)
    for (int r = 0; r < k; ++r)
      w[(size_t)c * k + r] = (double)oracle_f16_to_f32(permuted[oracle_f16_permuted_index(k, r, c)]);
  f16_ctx ctx = {y, x, w, bias, m, k, n, channels, mode};
  parallel_for(m, nthreads, f16_rows, &ctx);
  free(w);
}

/* ------------------------------------------------------------------------ */
/* Fused QKV + RMS + RoPE packing (opcodes 8/10/11/12)                      */
/* post-processing of the F16 GEMM output: reference src/dsp/ops/mat_mul.c  */
/* :1051-1125 (packing), :1127-1231 (sum, rsqrt, RMS with bias, rotary),    */
/* :1233-1266 (casts), :1297-1371 (worker), :1373-1578 (driver)             */
/* ------------------------------------------------------------------------ */

/*
 * Halfword index of (token r of token tile tt, column c of the head) inside
 * one head's region:
 *   Q: row pairs interleaved per 32-column tile, wsf_to_vhf(row r+1, row r)
 *      (qkv_pack_q_tile :1051-1072), tiles [token tile][column tile];
 *   K: the row converted in natural column order (vdeal of wsf_to_vhf,
 *      :1233-1247), then scattered: word w (columns 2w, 2w+1) of a 64-column
 *      chunk of token r to byte 128*w + 4*r of the chunk's two tiles
 *      (qkv_pack_k_tile :1078-1101);
 *   V: row pairs interleaved per 32-column tile (vshuff of two rows,
 *      qkv_pack_v_tile :1103-1125), tiles [column tile][token tile]
 *      (worker :1359-1369).
 */
size_t oracle_qkv_index(int which, int token_tiles, int head_dim, int tt, int r, int c) {
  const size_t pair = (size_t)(r / 2) * 64u + (size_t)(c % 32) * 2u + (size_t)(r % 2);
  if (which == 0) return (size_t)tt * (size_t)head_dim * 32u + (size_t)(c / 32) * 1024u + pair;
  if (which == 1)
    return (size_t)tt * (size_t)head_dim * 32u + (size_t)(c / 64) * 2048u + (size_t)((c % 64) / 2) * 64u +
           (size_t)r * 2u + (size_t)(c % 2);
  return ((size_t)(c / 32) * (size_t)token_tiles + (size_t)tt) * 1024u + pair;
}

/* 1/sqrt(x): the 0x5f3759df start, then three Newton steps y*(1.5 - x/2*y*y),
 * each operation one IEEE rounding (qkv_rsqrt_vsf :1137-1165). */
float oracle_qkv_rsqrt(float x) {
  const float half = x * 0.5f;
  float y = bits_f32(0x5f3759dfu - (f32_bits(x) >> 1));
  for (int it = 0; it < 3; ++it) {
    const float y2 = y * y;
    const float corr = 1.5f - half * y2;
    y = y * corr;
  }
  return y;
}

/* RMS normalization of one row of a Q or K head with its bias
 * (qkv_rms_bias :1167-1208): v = x + b; the sum of squares in the order of
 * the 32-lane vector code (lane j adds v[64d+j]^2 then v[64d+32+j]^2 over the
 * 64-column chunks d, then lanes are summed by the shifted adds of
 * qkv_reduce_sum :1127-1135: lane i += lane i-s for s = 16, 8, 4, 2, 1, and
 * lane 31 is the sum); rsqrt(sum / hd + 1e-6); y = (v * inv) * gamma. */
static void qkv_rms_row(float *row, const float *x, const float *b, const float *gamma, int hd) {
  float lanes[32];
  for (int j = 0; j < 32; ++j) {
    float acc = 0.0f;
    for (int d = 0; d < hd / 64; ++d) {
      const float v0 = x[64 * d + j] + (b ? b[64 * d + j] : 0.0f);
      const float v1 = x[64 * d + 32 + j] + (b ? b[64 * d + 32 + j] : 0.0f);
      row[64 * d + j] = v0;
      row[64 * d + 32 + j] = v1;
      acc = acc + v0 * v0;
      acc = acc + v1 * v1;
    }
    lanes[j] = acc;
  }
  for (int s = 16; s >= 1; s /= 2) {
    float next[32];
    for (int i = 0; i < 32; ++i) next[i] = i >= s ? lanes[i] + lanes[i - s] : lanes[i];
    memcpy(lanes, next, sizeof(lanes));
  }
  const float inv = oracle_qkv_rsqrt(lanes[31] / (float)hd + 1.0e-6f);
  for (int c = 0; c < hd; ++c) row[c] = (row[c] * inv) * gamma[c];
}

void oracle_qkv_post(uint16_t *q, uint16_t *k, uint16_t *v, const float *raw, const float *bias, const float *q_norm,
                     const float *k_norm, const float *pe, int rope_token_offset, int rope_token_count, int tokens,
                     int n_heads, int head_dim, int output_token_tiles, int output_token_offset) {
  const int hd = head_dim, q_cols = n_heads * hd, n = 3 * q_cols;
  const size_t hte = (size_t)output_token_tiles * (size_t)(hd / 32) * 1024u;
  float *row = (float *)malloc(sizeof(float) * (size_t)hd);
  for (int t0 = 0; t0 < tokens; t0 += 32) {
    const int rows = tokens - t0 < 32 ? tokens - t0 : 32;
    const int tt = (output_token_offset + t0) / 32;
    for (int col0 = 0; col0 < n; col0 += hd) {
      const int which = col0 < q_cols ? 0 : col0 < 2 * q_cols ? 1 : 2;
      const int head = (col0 - which * q_cols) / hd;
      uint16_t *dst = (which == 0 ? q : which == 1 ? k : v) + (size_t)head * hte;
      const float *b = bias ? bias + col0 : NULL;
      for (int r = 0; r < 32; ++r) {
        if (r >= rows) {
          for (int c = 0; c < hd; ++c) dst[oracle_qkv_index(which, output_token_tiles, hd, tt, r, c)] = 0;
          continue;
        }
        const float *x = raw + (size_t)(t0 + r) * n + col0;
        if (which < 2) {
          qkv_rms_row(row, x, b, which == 0 ? q_norm : k_norm, hd);
          /* rotary (qkv_apply_rope :1210-1231): token = offset + row; rows at or
           * past the count are left as they are */
          const int token = rope_token_offset + t0 + r;
          if (pe && rope_token_offset >= 0 && rope_token_count > 0 && token < rope_token_count) {
            const float *tp = pe + (size_t)token * (size_t)(hd / 2) * 4u;
            for (int d = 0; d < hd / 2; ++d) {
              const float x0 = row[2 * d], x1 = row[2 * d + 1];
              const float *m = tp + (size_t)d * 4u;
              row[2 * d] = x0 * m[0] + x1 * m[1];
              row[2 * d + 1] = x0 * m[2] + x1 * m[3];
            }
          }
        } else {
          /* V: bias, then the cast (qkv_bias_cast :1249-1266) */
          for (int c = 0; c < hd; ++c) row[c] = x[c] + (b ? b[c] : 0.0f);
        }
        for (int c = 0; c < hd; ++c)
          dst[oracle_qkv_index(which, output_token_tiles, hd, tt, r, c)] = oracle_f32_to_f16(row[c]);
      }
    }
  }
  free(row);
}

/* ------------------------------------------------------------------------ */
/* Dequantizing GEMM (opcodes 2/3/4): Q4_0, Q8_0, IQ4_NL super-blocks        */
/* block formats: reference include/dsp/quants.h:16-31 (my_block_q4_0,      */
/* my_block_q8_0); dequantization: src/dsp/ops/mat_mul.c:330-429 (Q4_0,     */
/* IQ4_NL) and :431-530 (Q8_0); driver :1601-1720; executor                 */
/* src/dsp/op_executor.cc:771-800                                           */
/* ------------------------------------------------------------------------ */

/* ggml's IQ4_NL code book (reference mat_mul.c:34-37, ggml's published
 * kvalues_iq4nl). */
static const int8_t k_iq4nl_values[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                          1,    13,   25,  38,  53,  69,  89,  113};

size_t oracle_qk0_block_bytes(int type) {
  switch (type) {
    case ORACLE_GGML_Q4_0:
    case ORACLE_GGML_IQ4_NL: return 16u + 128u; /* 8 fp16 scales + 256 nibbles */
    case ORACLE_GGML_Q8_0: return 16u + 256u;   /* 8 fp16 scales + 256 int8 */
    default: return 0u;
  }
}

/*
 * Value j (0..255) of one super-block.  Super-block b holds positions
 * [256*b, 256*b + 256) of the permuted F16 image of opcode 1 (the driver
 * dequantizes n_cols*k consecutive values of a column chunk into the buffer
 * the F16 core reads, mat_mul.c:1700-1712).  Position j uses scale j/32
 * (vlut16 of the scale indices 0,2 / 1,3 per half, :338-346, :414-421).
 *   Q8_0: quant byte j sign-extended (vunpack keeps byte order, :505-511).
 *   Q4_0 / IQ4_NL: the four 64-lane vlut16 results are written in the order
 *     lo(low nibbles), hi(low nibbles), lo(high nibbles), hi(high nibbles)
 *     (:424-427); vlut16 sends the even bytes of its source to the lo vector
 *     and the odd bytes to the hi vector (the single-group path re-interleaves
 *     them with vshuff, :296-298), so lane i of result v reads byte 2*i+(v&1),
 *     its low nibble for v < 2 and its high nibble otherwise.  Q4_0 values are
 *     nibble-8 (:30-32), IQ4_NL values the code book above.
 * The product value*scale is exact in binary32 and rounded once to binary16
 * (RNE): parity unpinned against the qf16 multiply and conversion of the
 * reference (Q6_Vqf16_vmpy_VhfVhf, Q6_Vhf_equals_Vqf16).
 */
uint16_t oracle_qk0_value(const uint8_t *block, int j, int type) {
  const int g = j / 32;
  const uint16_t sbits = (uint16_t)(block[2 * g] | (block[2 * g + 1] << 8));
  const float scale = oracle_f16_to_f32(sbits);
  int q;
  if (type == ORACLE_GGML_Q8_0) {
    q = (int8_t)block[16 + j];
  } else {
    const int v = j / 64, lane = j % 64;
    const uint8_t byte = block[16 + 2 * lane + (v & 1)];
    const int nib = v < 2 ? (byte & 15) : (byte >> 4);
    q = type == ORACLE_GGML_IQ4_NL ? k_iq4nl_values[nib] : nib - 8;
  }
  return oracle_f32_to_f16((float)q * scale);
}

int oracle_qk0_dequant(uint16_t *permuted, const uint8_t *blocks, int k, int n, int type) {
  const size_t bb = oracle_qk0_block_bytes(type);
  if (!bb || k <= 0 || n <= 0 || k % 32 || n % 32) return -1;
  const size_t nblk = (size_t)k * (size_t)n / 256u;
  for (size_t b = 0; b < nblk; ++b)
    for (int j = 0; j < 256; ++j) permuted[b * 256u + (size_t)j] = oracle_qk0_value(blocks + b * bb, j, type);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Deterministic synthetic inputs: splitmix64, Box-Muller in double          */
/* ------------------------------------------------------------------------ */

uint64_t oracle_splitmix64(uint64_t *state) {
  uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static double unit_double(uint64_t *state) { return (double)(oracle_splitmix64(state) >> 11) * 0x1.0p-53; }

void oracle_fill_normal(float *dst, size_t count, float mean, float stddev, uint64_t seed) {
  uint64_t st = seed;
  for (size_t i = 0; i < count; i += 2) {
    double u1 = unit_double(&st);
    const double u2 = unit_double(&st);
    if (u1 < 0x1.0p-60) u1 = 0x1.0p-60;
    const double r = sqrt(-2.0 * log(u1));
    const double th = 6.283185307179586 * u2;
    dst[i] = (float)(mean + stddev * r * cos(th));
    if (i + 1 < count) dst[i + 1] = (float)(mean + stddev * r * sin(th));
  }
}

void oracle_fill_uniform(float *dst, size_t count, float lo, float hi, uint64_t seed) {
  uint64_t st = seed;
  for (size_t i = 0; i < count; ++i) dst[i] = (float)(lo + (hi - lo) * unit_double(&st));
}

void oracle_fill_int8(int8_t *dst, size_t count, int lo, int hi, uint64_t seed) {
  uint64_t st = seed;
  const uint64_t span = (uint64_t)(hi - lo + 1);
  const uint64_t limit = UINT64_MAX - UINT64_MAX % span; /* unbiased draw */
  for (size_t i = 0; i < count; ++i) {
    uint64_t v;
    do {
      v = oracle_splitmix64(&st);
    } while (v >= limit);
    dst[i] = (int8_t)(lo + (int)(v % span));
  }
}
