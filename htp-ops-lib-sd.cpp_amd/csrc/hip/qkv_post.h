// Packed Q / K / V post-processing of the fused QKV opcodes (8/10/11/12),
// shared by the standalone kernel (qkv.hip) and the GEMM with the
// post-processing in its epilogue (f16.hip).
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
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

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
// NH blocks side by side: heads h = 0 .. NH-1 of one 32-token tile, whose
// inputs are HD columns apart in src (and in bias); the NH heads' arithmetic
// is interleaved (independent chains), the rotary matrices are shared (they
// depend on the token and the column pair only).
// src: row 0, column 0 of head 0's input (f32, or fp16 holding the same
// fp16-exact values; rows src_stride elements apart);
// bias: head 0's first column (NULL: none); rows: valid rows (1..32);
// token0: the call's token index of row 0 (for the rotary matrices);
// blk: NH * HD * 32 halfwords of LDS, 16-byte aligned, for the packed blocks;
// head h's block goes to dst + head_base + h * head_stride.
template <int HD, int WHICH, int NH, typename T>
__device__ void qkv_blocks(uint16_t *__restrict__ blk, uint16_t *__restrict__ dst, const T *__restrict__ src,
                           int src_stride, const float *__restrict__ bias, const float *__restrict__ gamma,
                           const float *__restrict__ pe, int rope_off, int rope_count, int rows, int token0, int tt,
                           int token_tiles, size_t head_base, size_t head_stride) {
  constexpr int CH = HD / 64;  // 64-column chunks; lane j holds columns 64d+j and 64d+32+j
  constexpr int E = 2 * CH;    // values per lane and row
  constexpr int PAIRS = 16 / (kQkvThreads / 64);
  constexpr bool ROPE_OK = WHICH < 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, j = lane & 31;
  auto col = [&](int e) { return 64 * (e >> 1) + 32 * (e & 1) + j; };

  float v[NH][PAIRS][E];
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    const int r = 2 * (wave + 4 * i) + half;
    const T *x = src + (size_t)r * (size_t)src_stride;
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int e = 0; e < E; ++e) v[h][i][e] = r < rows ? (float)x[h * HD + col(e)] : 0.0f;
  }
  float b[NH][E], g[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
#pragma unroll
    for (int h = 0; h < NH; ++h) b[h][e] = bias ? bias[h * HD + col(e)] : 0.0f;
    g[e] = WHICH < 2 ? gamma[col(e)] : 0.0f;
  }
  // rotary matrices (x0, x1 -> m.x x0 + m.y x1, m.z x0 + m.w x1) of each row's token
  float4 m[ROPE_OK ? PAIRS : 1][ROPE_OK ? E : 1];
  bool rot[PAIRS];
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    const int r = 2 * (wave + 4 * i) + half;
    const int token = rope_off + token0 + r;
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
    for (int h = 0; h < NH; ++h) {
#pragma unroll
      for (int e = 0; e < E; ++e) v[h][i][e] = __fadd_rn(v[h][i][e], b[h][e]);
      if (WHICH < 2) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc = __fadd_rn(acc, __fmul_rn(v[h][i][e], v[h][i][e]));
        // lane i += lane i - s within the 32 lanes of the row, s = 16 .. 1
#pragma unroll
        for (int s = 16; s >= 1; s >>= 1) {
          const float o = __shfl(acc, (lane - s) & 63, 64);
          if (j >= s) acc = __fadd_rn(acc, o);
        }
        const float sum = __shfl(acc, half * 32 + 31, 64);
        const float inv = qkv_rsqrt(__fadd_rn(__fdiv_rn(sum, (float)HD), 1.0e-6f));
#pragma unroll
        for (int e = 0; e < E; ++e) v[h][i][e] = __fmul_rn(__fmul_rn(v[h][i][e], inv), g[e]);
        if (pe) {
          // the pair of column c is c ^ 1, held by lane j ^ 1
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float other = __shfl(v[h][i][e], lane ^ 1, 64);
            if (rot[i]) {
              const bool odd = j & 1;
              const float x0 = odd ? other : v[h][i][e], x1 = odd ? v[h][i][e] : other;
              const float4 mm = m[i][ROPE_OK ? e : 0];
              v[h][i][e] = odd ? __fadd_rn(__fmul_rn(x0, mm.z), __fmul_rn(x1, mm.w))
                               : __fadd_rn(__fmul_rn(x0, mm.x), __fmul_rn(x1, mm.y));
            }
          }
        }
      }
#pragma unroll
      for (int e = 0; e < E; ++e)
        blk[h * HD * 32 + block_index<WHICH>(r, col(e))] =
            r < rows ? __half_as_ushort(__float2half_rn(v[h][i][e])) : (uint16_t)0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const uint4 *packed = (const uint4 *)(blk + h * HD * 32);
    uint16_t *hdst = dst + head_base + (size_t)h * head_stride;
    if (WHICH < 2) {
      uint4 *out = (uint4 *)(hdst + (size_t)tt * HD * 32);
      for (int i = threadIdx.x; i < HD * 32 / 8; i += kQkvThreads) out[i] = packed[i];
    } else {
      for (int i = threadIdx.x; i < HD * 32 / 8; i += kQkvThreads) {
        const int ct = i / 128;  // 1024 halfwords = 128 uint4 per column tile
        uint4 *out = (uint4 *)(hdst + ((size_t)ct * token_tiles + tt) * 1024);
        out[i % 128] = packed[i];
      }
    }
  }
}

// One block (NH = 1).
template <int HD, int WHICH, typename T>
__device__ void qkv_block(uint16_t *__restrict__ blk, uint16_t *__restrict__ dst, const T *__restrict__ src,
                          int src_stride, const float *__restrict__ bias, const float *__restrict__ gamma,
                          const float *__restrict__ pe, int rope_off, int rope_count, int rows, int token0, int tt,
                          int token_tiles, size_t head_base) {
  qkv_blocks<HD, WHICH, 1, T>(blk, dst, src, src_stride, bias, gamma, pe, rope_off, rope_count, rows, token0, tt,
                              token_tiles, head_base, 0);
}

}  // namespace
