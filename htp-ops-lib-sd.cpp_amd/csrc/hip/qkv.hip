// Opcodes 8/10/11/12 (fused QKV projection + RMS norm + RoPE, packed outputs)
// on gfx950: the post-processing of a packed-F16 GEMM output held in HBM
// (the arithmetic and layouts are described in qkv_post.h).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

#include "hb_internal.h"
#include "qkv_post.h"

namespace {

template <int HD>
__global__ __launch_bounds__(kQkvThreads) void qkv_post(uint16_t *q, uint16_t *k, uint16_t *v, const float *raw,
                                                        const float *bias, const float *q_norm, const float *k_norm,
                                                        const float *pe, int rope_off, int rope_count, int tokens,
                                                        int n_heads, int token_tiles, int out_tile0) {
  __shared__ __attribute__((aligned(16))) uint16_t blk[HD * 32];
  const int t0 = blockIdx.x * 32, tt = out_tile0 + blockIdx.x;
  const int which = blockIdx.y / n_heads, head = blockIdx.y % n_heads;
  const int q_cols = n_heads * HD, ncols = 3 * q_cols, col0 = which * q_cols + head * HD;
  const size_t head_base = (size_t)head * (size_t)token_tiles * (HD / 32) * 1024;
  const float *src = raw + (size_t)t0 * (size_t)ncols + col0;
  const float *b = bias ? bias + col0 : nullptr;
  const int rows = min(32, tokens - t0);
  if (which == 0)
    qkv_block<HD, 0>(blk, q, src, ncols, b, q_norm, pe, rope_off, rope_count, rows, t0, tt, token_tiles, head_base);
  else if (which == 1)
    qkv_block<HD, 1>(blk, k, src, ncols, b, k_norm, pe, rope_off, rope_count, rows, t0, tt, token_tiles, head_base);
  else
    qkv_block<HD, 2>(blk, v, src, ncols, b, nullptr, nullptr, 0, 0, rows, t0, tt, token_tiles, head_base);
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

extern "C" {

int hb_qkv_post(uint16_t *d_q, uint16_t *d_k, uint16_t *d_v, const float *d_raw, const float *d_bias,
                const float *d_q_norm, const float *d_k_norm, const float *d_pe, int rope_offset, int rope_count,
                int tokens, int n_heads, int head_dim, int token_tiles, int out_offset, hb_stream s) {
  if (!d_q || !d_k || !d_v || !d_raw || !d_q_norm || !d_k_norm) return hb_invalid("hb_qkv_post null pointer");
  if (tokens <= 0 || n_heads <= 0 || (head_dim != 64 && head_dim != 128) || out_offset < 0 || out_offset % 32 ||
      out_offset / 32 + (tokens + 31) / 32 > token_tiles)
    return hb_invalid("hb_qkv_post shape");
  if (!aligned(d_q, 16) || !aligned(d_k, 16) || !aligned(d_v, 16) || !aligned(d_raw, 4) ||
      (d_pe && !aligned(d_pe, 16)))
    return hb_invalid("hb_qkv_post alignment");
  if (d_pe && (rope_offset < 0 || rope_count <= 0)) d_pe = nullptr;  // the reference skips the rotation
  hipStream_t st = hb_resolve_stream(s);
  const dim3 grid((tokens + 31) / 32, 3 * n_heads), block(kQkvThreads);
  if (head_dim == 64)
    hipLaunchKernelGGL(qkv_post<64>, grid, block, 0, st, d_q, d_k, d_v, d_raw, d_bias, d_q_norm, d_k_norm, d_pe,
                       rope_offset, rope_count, tokens, n_heads, token_tiles, out_offset / 32);
  else
    hipLaunchKernelGGL(qkv_post<128>, grid, block, 0, st, d_q, d_k, d_v, d_raw, d_bias, d_q_norm, d_k_norm, d_pe,
                       rope_offset, rope_count, tokens, n_heads, token_tiles, out_offset / 32);
  return hb_check_launch("qkv_post");
}

}  // extern "C"
