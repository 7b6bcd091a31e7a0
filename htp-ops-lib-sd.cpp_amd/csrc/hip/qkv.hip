// Opcodes 8/10/11/12 (fused QKV projection + RMS norm + RoPE, packed outputs)
// on gfx950: the post-processing of the packed-F16 GEMM's output.
//
// Semantics (reference src/dsp/ops/mat_mul.c): the GEMM output is the HMX
// fp16 readout (:1297-1330, transfer_output_chunk_fp16_to_fp32 :751-778), so
// its f32 values are fp16-exact.  Per 32-token tile and head:
//   Q, K  v = x + bias; sum of squares in the order of the 32-lane vector code
//         (lane j: v[64d+j]^2 then v[64d+32+j]^2 over the 64-column chunks d,
//         then the shifted lane adds of qkv_reduce_sum :1127-1135);
//         inv = rsqrt(sum/hd + 1e-6) by three Newton steps from 0x5f3759df
//         (:1137-1165); y = (v*inv)*gamma (:1167-1208); then the rotary
//         matrices of the token (:1210-1231) while token < rope_count;
//   V     y = x + bias (:1249-1266);
// each value rounded once to fp16 and placed in the packed layouts:
//   Q  row pairs interleaved per 32-column tile, tiles [token tile][column tile]
//      (:1051-1072);
//   K  per 64-column chunk of token r, word w (columns 2w, 2w+1) at byte
//      128w + 4r of the chunk's two tiles (the vscatter of :1078-1101);
//   V  row pairs interleaved per 32-column tile, tiles [column tile][token tile]
//      (:1103-1125, :1359-1369).
// Rows past the call's tokens inside its last tile are zeros.  Every float
// step is one IEEE binary32 operation (the reference computes them in QFloat).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

#include "hb_internal.h"

namespace {

constexpr int kQkvThreads = 256;  // 4 waves; a wave takes two rows at a time (one per 32 lanes)

__device__ inline float qkv_rsqrt(float x) {
  const float half = __fmul_rn(x, 0.5f);
  float y = __uint_as_float(0x5f3759dfu - (__float_as_uint(x) >> 1));
#pragma unroll
  for (int it = 0; it < 3; ++it) {
    const float y2 = __fmul_rn(y, y);
    const float corr = __fsub_rn(1.5f, __fmul_rn(half, y2));
    y = __fmul_rn(y, corr);
  }
  return y;
}

// LDS index of (row r, column c) inside one (token tile, head) block, in the
// order of the destination: Q and K blocks are contiguous, V's column tiles
// are copied to their own places.
template <int WHICH>
__device__ inline int block_index(int r, int c) {
  const int pair = (r >> 1) * 64 + (c & 31) * 2 + (r & 1);
  if (WHICH == 1) return (c >> 6) * 2048 + ((c & 63) >> 1) * 64 + r * 2 + (c & 1);
  return (c >> 5) * 1024 + pair;
}

// One workgroup per (32-token tile, head) of one of Q / K / V (WHICH 0 / 1 / 2).
// Every load of the tile (rows, bias, gamma, rotary matrices) is issued
// before the arithmetic: one round of 4 row pairs per wave keeps enough
// bytes in flight to stream from HBM.
template <int HD, int WHICH>
__device__ void qkv_block(uint16_t *__restrict__ dst, const float *__restrict__ raw, const float *__restrict__ bias,
                          const float *__restrict__ gamma, const float *__restrict__ pe, int rope_off, int rope_count,
                          int tokens, int ncols, int col0, int t0, int tt, int token_tiles, size_t head_base) {
  constexpr int CH = HD / 64;  // 64-column chunks; lane j holds columns 64d+j and 64d+32+j
  constexpr int E = 2 * CH;    // values per lane and row
  constexpr int PAIRS = 16 / (kQkvThreads / 64);
  constexpr bool ROPE_OK = WHICH < 2;
  __shared__ __attribute__((aligned(16))) uint16_t blk[HD * 32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, j = lane & 31;
  const int rows = min(32, tokens - t0);
  auto col = [&](int e) { return 64 * (e >> 1) + 32 * (e & 1) + j; };

  float v[PAIRS][E];
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    const int r = 2 * (wave + 4 * i) + half;
    const float *x = raw + (size_t)(t0 + r) * (size_t)ncols + col0;
#pragma unroll
    for (int e = 0; e < E; ++e) v[i][e] = r < rows ? x[col(e)] : 0.0f;
  }
  float b[E], g[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    b[e] = bias ? bias[col0 + col(e)] : 0.0f;
    g[e] = WHICH < 2 ? gamma[col(e)] : 0.0f;
  }
  // rotary matrices (x0, x1 -> m.x x0 + m.y x1, m.z x0 + m.w x1) of each row's token
  float4 m[ROPE_OK ? PAIRS : 1][ROPE_OK ? E : 1];
  bool rot[PAIRS];
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    const int r = 2 * (wave + 4 * i) + half;
    const int token = rope_off + t0 + r;
    rot[i] = ROPE_OK && pe && r < rows && token < rope_count;
    if (ROPE_OK) {
#pragma unroll
      for (int e = 0; e < E; ++e)
        m[i][e] = rot[i] ? *(const float4 *)(pe + ((size_t)token * (HD / 2) + (size_t)(col(e) >> 1)) * 4u)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    const int r = 2 * (wave + 4 * i) + half;
#pragma unroll
    for (int e = 0; e < E; ++e) v[i][e] = __fadd_rn(v[i][e], b[e]);
    if (WHICH < 2) {
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc = __fadd_rn(acc, __fmul_rn(v[i][e], v[i][e]));
      // lane i += lane i - s within the 32 lanes of the row, s = 16 .. 1
#pragma unroll
      for (int s = 16; s >= 1; s >>= 1) {
        const float o = __shfl(acc, (lane - s) & 63, 64);
        if (j >= s) acc = __fadd_rn(acc, o);
      }
      const float sum = __shfl(acc, half * 32 + 31, 64);
      const float inv = qkv_rsqrt(__fadd_rn(__fdiv_rn(sum, (float)HD), 1.0e-6f));
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] = __fmul_rn(__fmul_rn(v[i][e], inv), g[e]);
      if (pe) {
        // the pair of column c is c ^ 1, held by lane j ^ 1
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float other = __shfl(v[i][e], lane ^ 1, 64);
          if (rot[i]) {
            const bool odd = j & 1;
            const float x0 = odd ? other : v[i][e], x1 = odd ? v[i][e] : other;
            const float4 mm = m[i][ROPE_OK ? e : 0];
            v[i][e] = odd ? __fadd_rn(__fmul_rn(x0, mm.z), __fmul_rn(x1, mm.w))
                          : __fadd_rn(__fmul_rn(x0, mm.x), __fmul_rn(x1, mm.y));
          }
        }
      }
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
      blk[block_index<WHICH>(r, col(e))] = r < rows ? __half_as_ushort(__float2half_rn(v[i][e])) : (uint16_t)0;
  }
  __syncthreads();
  const uint4 *src = (const uint4 *)blk;
  if (WHICH < 2) {
    uint4 *out = (uint4 *)(dst + head_base + (size_t)tt * HD * 32);
    for (int i = threadIdx.x; i < HD * 32 / 8; i += kQkvThreads) out[i] = src[i];
  } else {
    for (int i = threadIdx.x; i < HD * 32 / 8; i += kQkvThreads) {
      const int ct = i / 128;  // 1024 halfwords = 128 uint4 per column tile
      uint4 *out = (uint4 *)(dst + head_base + ((size_t)ct * token_tiles + tt) * 1024);
      out[i % 128] = src[i];
    }
  }
}

template <int HD>
__global__ __launch_bounds__(kQkvThreads) void qkv_post(uint16_t *q, uint16_t *k, uint16_t *v, const float *raw,
                                                        const float *bias, const float *q_norm, const float *k_norm,
                                                        const float *pe, int rope_off, int rope_count, int tokens,
                                                        int n_heads, int token_tiles, int out_tile0) {
  const int t0 = blockIdx.x * 32, tt = out_tile0 + blockIdx.x;
  const int which = blockIdx.y / n_heads, head = blockIdx.y % n_heads;
  const int q_cols = n_heads * HD, ncols = 3 * q_cols, col0 = which * q_cols + head * HD;
  const size_t head_base = (size_t)head * (size_t)token_tiles * (HD / 32) * 1024;
  if (which == 0)
    qkv_block<HD, 0>(q, raw, bias, q_norm, pe, rope_off, rope_count, tokens, ncols, col0, t0, tt, token_tiles,
                     head_base);
  else if (which == 1)
    qkv_block<HD, 1>(k, raw, bias, k_norm, pe, rope_off, rope_count, tokens, ncols, col0, t0, tt, token_tiles,
                     head_base);
  else
    qkv_block<HD, 2>(v, raw, bias, nullptr, nullptr, 0, 0, tokens, ncols, col0, t0, tt, token_tiles, head_base);
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
