/*
 * Host weight packers (formats consumed by opcodes 15 and 1/16).
 *   W8A8 blob:   header / offsets reference include/op_reg.h:80-85 and
 *                src/dsp/op_executor.cc:321-335; W(n,k) deep tile address
 *                reference src/dsp/ops/linear_w8a8.c:453,482,486-488 and
 *                tests/hmx-probe/study_dsp.c:82-84.
 *   F16 permute: reference src/host/test.c:551-556.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "host_internal.h"
#include "htp_ops/op_reg.h"
#include "htp_ops/pack.h"

size_t htp_ops_w8a8_constants_bytes(int k, int n) {
  if (k <= 0 || n <= 0) return 0;
  return 128u + (size_t)k * (size_t)n + (size_t)n * 8u + (size_t)k * 4u;
}

uint64_t htp_ops_fnv1a64(const void *data, size_t bytes) { return htp_fnv1a64(data, bytes); }

int htp_ops_w8a8_pack_constants(uint8_t *blob, size_t blob_bytes, const int8_t *w, const float *sw,
                                const int32_t *sums, const float *inv, int k, int n, uint64_t signature) {
  if (!blob || !w || !sw || k < 32 || k % 32 || n < 64 || n % 64) return -1;
  const size_t need = htp_ops_w8a8_constants_bytes(k, n);
  if (blob_bytes < need) return -1;
  const size_t kn = (size_t)k * (size_t)n;
  struct W8A8Header h;
  memset(&h, 0, sizeof(h));
  h.magic = W8A8_BLOB_MAGIC;
  h.version = W8A8_BLOB_VERSION;
  h.k = (uint32_t)k;
  h.n = (uint32_t)n;
  h.weight_offset = 128u;
  h.scale_offset = (uint32_t)(128u + kn);
  h.sum_offset = (uint32_t)(h.scale_offset + 4u * (size_t)n);
  h.inverse_offset = (uint32_t)(h.sum_offset + 4u * (size_t)n);
  h.bytes = (uint32_t)need;
  h.original_f16_signature = signature;
  memcpy(blob, &h, sizeof(h));
  /* Deep tiles: per 64-column group, per 32-k block, two 32-column halves of
   * 8 k-quads x 32 columns x 4 bytes. */
  for (int g = 0; g < n / 64; ++g) {
    for (int kb = 0; kb < k / 32; ++kb) {
      uint8_t *tile = blob + 128u + (size_t)g * 64u * (size_t)k + (size_t)kb * 2048u;
      for (int half = 0; half < 2; ++half) {
        for (int quad = 0; quad < 8; ++quad) {
          for (int c = 0; c < 32; ++c) {
            const int col = g * 64 + half * 32 + c;
            const int8_t *src = w + (size_t)col * k + (size_t)kb * 32u + (size_t)quad * 4u;
            memcpy(tile + half * 1024 + quad * 128 + c * 4, src, 4);
          }
        }
      }
    }
  }
  uint8_t *scale = blob + h.scale_offset, *sum = blob + h.sum_offset, *inverse = blob + h.inverse_offset;
  memcpy(scale, sw, 4u * (size_t)n);
  for (int c = 0; c < n; ++c) {
    int32_t s = 0;
    if (sums) {
      s = sums[c];
    } else {
      for (int r = 0; r < k; ++r) s += w[(size_t)c * k + r];
    }
    memcpy(sum + 4u * (size_t)c, &s, 4);
  }
  for (int r = 0; r < k; ++r) {
    const float v = inv ? inv[r] : 1.0f;
    memcpy(inverse + 4u * (size_t)r, &v, 4);
  }
  return 0;
}

int htp_ops_w8a8_quantize_weights(int8_t *q, float *sw, const float *w, const float *inv, int k, int n) {
  if (!q || !sw || !w || k <= 0 || n <= 0) return -1;
  for (int c = 0; c < n; ++c) {
    const float *row = w + (size_t)c * k;
    float amax = 0.0f;
    for (int r = 0; r < k; ++r) {
      const float v = inv ? row[r] / inv[r] : row[r];
      const float a = fabsf(v);
      if (a > amax) amax = a;
    }
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    sw[c] = s;
    for (int r = 0; r < k; ++r) {
      const float v = inv ? row[r] / inv[r] : row[r];
      float t = rintf(v / s);
      if (t > 127.0f) t = 127.0f;
      if (t < -127.0f) t = -127.0f;
      q[(size_t)c * k + r] = (int8_t)t;
    }
  }
  return 0;
}

/* IEEE binary16 bits -> float (every half value is exactly representable). */
static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13); /* inf / nan (payload kept) */
  } else if (e != 0) {
    bits = sign | ((e + 112u) << 23) | (m << 13); /* normal: rebias 15 -> 127 */
  } else if (m == 0) {
    bits = sign; /* signed zero */
  } else {
    /* subnormal half: m * 2^-24, normalized as a float */
    uint32_t shift = 0, mm = m;
    while (!(mm & 0x400)) {
      mm <<= 1;
      ++shift;
    }
    bits = sign | ((113u - shift) << 23) | ((mm & 0x3ff) << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof(f));
  return f;
}

int htp_ops_w8a8_pack_f16(uint8_t *blob, size_t blob_bytes, const uint16_t *w_f16, const float *inv, int k, int n) {
  if (!blob || !w_f16 || k < 32 || k % 32 || n < 64 || n % 64) return -1;
  if (blob_bytes < htp_ops_w8a8_constants_bytes(k, n)) return -1;
  const size_t kn = (size_t)k * (size_t)n;
  float *w = (float *)malloc(kn * sizeof(float));
  int8_t *q = (int8_t *)malloc(kn);
  float *sw = (float *)malloc((size_t)n * sizeof(float));
  int rc = (w && q && sw) ? 0 : -1;
  if (!rc) {
    for (size_t i = 0; i < kn; ++i) w[i] = half_to_float(w_f16[i]);
    rc = htp_ops_w8a8_quantize_weights(q, sw, w, inv, k, n);
  }
  if (!rc)
    rc = htp_ops_w8a8_pack_constants(blob, blob_bytes, q, sw, NULL, inv, k, n, htp_fnv1a64(w_f16, kn * 2u));
  free(w);
  free(q);
  free(sw);
  return rc;
}

int htp_ops_f16_permute_weights(uint16_t *permuted, const uint16_t *w_kn, int k, int n) {
  if (!permuted || !w_kn || k < 32 || k % 32 || n < 32 || n % 32) return -1;
  for (int r = 0; r < k; ++r) {
    for (int c = 0; c < n; ++c) {
      const size_t tile = (size_t)(c / 32) * (size_t)(k / 32) + (size_t)(r / 32);
      permuted[tile * 1024u + (size_t)((r % 32) / 2) * 64u + (size_t)(c % 32) * 2u + (size_t)(r % 2)] =
          w_kn[(size_t)r * n + c];
    }
  }
  return 0;
}
