// Opcode 19 (model auxiliary f32 ops) on gfx950: the normalizations,
// modulation, activations, layout changes and gated MLP products that sit
// between the GEMMs of a DiT / text-encoder block.
//
// Semantics (reference src/dsp/ops/mat_mul.c:2356-2486, hvx_model_aux_f32
// :2488-2501; activation formulas :787-826):
//   modes 0/1/9  one row of `width` per task: mean (mode 1: 0), centered sum of
//                squares, inv = 1/sqrt(sumsq/width + eps), v = (x-mean)*inv, then
//                affine w[i]/b[i] (modes 0/1) or modulation v += v*w; v += b
//                (mode 9, per batch when other_count != width); optional SiLU
//   mode 2       group norm, one task per (batch, group) of spatial*channels/groups
//                contiguous values, per-channel affine
//   modes 3/4    x + w[i % other_count] / x * w[i % other_count]
//   modes 5/6/7  SiLU / GELU-tanh / QuickGELU
//   mode 8       per-batch transpose [width][spatial] -> [spatial][width]
//   mode 10      x[i] * w[batch-or-0][i % width] + b[i]
//   mode 11      rotary embedding with 2x2 matrices per (token, pair), written in
//                [batch][head][token][dim] order
//   modes 12/13  SiLU(gate) * up from [.., gate | up ..] rows (13 also copies
//                an attention row in front of each output row)
// Every float step is one IEEE binary32 operation in the reference's order;
// the row sums of the norms accumulate in double (the reference sums its 32
// lanes in double, mat_mul.c:2352-2355), so mean and inv match a double
// restatement except at rounding ties.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "hb_internal.h"

namespace {

constexpr int kAuxThreads = 256;

// x * sigmoid(z), with the stable sigmoid e/(1+e) for z < 0, e = 2^max(-|z|*log2(e), -126).
__device__ inline float times_sigmoid(float x, float z) {
  const float neg = fmaxf(__fmul_rn(fabsf(z), -1.4426950408889634f), -126.0f);
  const float e = exp2f(neg);
  const float inv = __fdiv_rn(1.0f, __fadd_rn(e, 1.0f));
  return __fmul_rn(x, z < 0.0f ? __fmul_rn(e, inv) : inv);
}

// Activation ids of the reference epilogue: 1 GELU-tanh, 2 QuickGELU, 4 and 5 SiLU.
__device__ inline float activate(float x, int act) {
  if (act == 1) {
    const float cubic = __fmul_rn(__fmul_rn(x, x), x);
    const float inner = __fadd_rn(x, __fmul_rn(cubic, 0.044715f));
    return times_sigmoid(x, __fmul_rn(inner, 1.5957691216057308f));
  }
  if (act == 2) return times_sigmoid(x, __fmul_rn(x, 1.702f));
  if (act == 4 || act == 5) return times_sigmoid(x, x);
  return x;
}

__device__ inline double block_sum(double v, double *red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();  // red may still be read from the previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < kAuxThreads / 64; ++w) t += red[w];
  return t;
}

// Modes 0, 1, 2, 9: one workgroup per task of `len` contiguous values.
template <int MODE>
__global__ __launch_bounds__(kAuxThreads) void aux_norm(float *__restrict__ y, const float *__restrict__ x,
                                                        const float *__restrict__ w, const float *__restrict__ b,
                                                        int len, int width, int channels, int spatial,
                                                        int other_count, float eps, int act) {
  __shared__ double red[kAuxThreads / 64];
  const size_t offset = (size_t)blockIdx.x * (size_t)len;
  const float *xr = x + offset;
  float *yr = y + offset;
  float mean = 0.0f;
  if (MODE != 1) {
    double s = 0.0;
    for (int i = threadIdx.x; i < len; i += kAuxThreads) s += (double)xr[i];
    mean = (float)(block_sum(s, red) / (double)len);
  }
  double q = 0.0;
  for (int i = threadIdx.x; i < len; i += kAuxThreads) {
    const double v = (double)__fsub_rn(xr[i], mean);
    q += v * v;
  }
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn((float)(block_sum(q, red) / (double)len + (double)eps)));
  // mode 9: per-batch parameters unless they are shared by all batches
  const size_t pbase = (MODE == 9 && other_count != width) ? (size_t)(blockIdx.x / spatial) * (size_t)width : 0;
  for (int i = threadIdx.x; i < len; i += kAuxThreads) {
    float v = __fmul_rn(__fsub_rn(xr[i], mean), inv);
    if (MODE == 0 || MODE == 1) {
      if (w) v = __fmul_rn(v, w[i]);
      if (b) v = __fadd_rn(v, b[i]);
    } else if (MODE == 2) {
      const int ch = (int)(((offset + (size_t)i) / (size_t)spatial) % (size_t)channels);
      if (w) v = __fmul_rn(v, w[ch]);
      if (b) v = __fadd_rn(v, b[ch]);
    } else {
      v = __fadd_rn(v, __fmul_rn(v, w[pbase + i]));
      v = __fadd_rn(v, b[pbase + i]);
    }
    if (act) v = activate(v, 4);
    yr[i] = v;
  }
}

// Modes 3, 4, 5, 6, 7, 10, 12: one thread per output value, grid-stride.
template <int MODE>
__global__ __launch_bounds__(kAuxThreads) void aux_elementwise(float *__restrict__ y, const float *__restrict__ x,
                                                               const float *__restrict__ w,
                                                               const float *__restrict__ b, int64_t count, int width,
                                                               int channels, int spatial, int other_count, int act) {
  const int64_t stride = (int64_t)gridDim.x * kAuxThreads;
  for (int64_t i = (int64_t)blockIdx.x * kAuxThreads + threadIdx.x; i < count; i += stride) {
    float v;
    if (MODE == 3) {
      v = __fadd_rn(x[i], w[i % other_count]);
    } else if (MODE == 4) {
      v = __fmul_rn(x[i], w[i % other_count]);
    } else if (MODE == 5 || MODE == 6 || MODE == 7) {
      v = activate(x[i], MODE == 5 ? 4 : MODE == 6 ? 1 : 2);
    } else if (MODE == 10) {
      const int64_t channel = i % width, batch = i / ((int64_t)width * spatial);
      const int64_t pb = other_count == width ? 0 : batch;
      v = __fadd_rn(__fmul_rn(x[i], w[pb * width + channel]), b[i]);
    } else {  // 12
      const int64_t column = i % width, row = i / width;
      const float *a = x + row * channels + column;
      const float gate = a[act ? 0 : width], up = a[act ? width : 0];
      v = __fmul_rn(activate(gate, 5), up);
    }
    y[i] = v;
  }
}

// Mode 8: x[batch][width][spatial] -> y[batch][spatial][width], 32 x 32 tiles through LDS.
__global__ __launch_bounds__(kAuxThreads) void aux_transpose(float *__restrict__ y, const float *__restrict__ x,
                                                             int width, int spatial) {
  __shared__ float tile[32][33];
  const int batch = blockIdx.z, r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  const float *xb = x + (size_t)batch * width * spatial;
  float *yb = y + (size_t)batch * width * spatial;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8)
    if (r0 + r < width && c0 + tx < spatial) tile[r][tx] = xb[(size_t)(r0 + r) * spatial + c0 + tx];
  __syncthreads();
  for (int c = ty; c < 32; c += 8)
    if (c0 + c < spatial && r0 + tx < width) yb[(size_t)(c0 + c) * width + r0 + tx] = tile[tx][c];
}

// Mode 11: one workgroup per (batch, token); threads over heads x pairs.
__global__ __launch_bounds__(kAuxThreads) void aux_rope(float *__restrict__ y, const float *__restrict__ x,
                                                        const float *__restrict__ pe, int dim, int heads,
                                                        int tokens, int groups) {
  const int task = blockIdx.x;
  const int token = task % tokens, batch = task / tokens;
  const float *m_base = pe + ((size_t)(groups == 1 ? 0 : batch) * tokens + token) * (size_t)dim * 2;
  const int pairs = dim / 2;
  for (int t = threadIdx.x; t < heads * pairs; t += kAuxThreads) {
    const int head = t / pairs, p = t % pairs;
    const float *m = m_base + 4 * p;
    const float *xs = x + (((size_t)batch * tokens + token) * heads + head) * dim + 2 * p;
    float *ys = y + (((size_t)batch * heads + head) * tokens + token) * dim + 2 * p;
    const float x0 = xs[0], x1 = xs[1];
    ys[0] = __fadd_rn(__fmul_rn(x0, m[0]), __fmul_rn(x1, m[1]));
    ys[1] = __fadd_rn(__fmul_rn(x1, m[3]), __fmul_rn(x0, m[2]));
  }
}

// Mode 13: output row r = [attention row r (groups values) | SiLU(gate) * up (width values)].
__global__ __launch_bounds__(kAuxThreads) void aux_swiglu_concat(float *__restrict__ y, const float *__restrict__ x,
                                                                 const float *__restrict__ attn, int width,
                                                                 int groups, int channels, int act) {
  const size_t r = blockIdx.x;
  float *dst = y + r * (size_t)(width + groups);
  const float *a = attn + r * (size_t)groups;
  for (int i = threadIdx.x; i < groups; i += kAuxThreads) dst[i] = a[i];
  const float *xr = x + r * (size_t)channels;
  for (int i = threadIdx.x; i < width; i += kAuxThreads) {
    const float gate = xr[i + (act ? 0 : width)], up = xr[i + (act ? width : 0)];
    dst[groups + i] = __fmul_rn(activate(gate, 5), up);
  }
}

int elementwise_grid(int64_t count) {
  const int64_t blocks = (count + kAuxThreads - 1) / kAuxThreads;
  return (int)(blocks < 65536 ? blocks : 65536);
}

}  // namespace

extern "C" int hb_model_aux(float *d_y, const float *d_x, const float *d_w, const float *d_b, int mode, int count,
                            int width, int channels, int spatial, int groups, int batch, int other_count,
                            int activation, float eps, hb_stream s) {
  if (!d_y || !d_x) return hb_invalid("hb_model_aux null pointer");
  if (count <= 0 || width <= 0 || channels <= 0 || spatial <= 0 || batch <= 0)
    return hb_invalid("hb_model_aux shape");
  hipStream_t st = hb_resolve_stream(s);
  const dim3 block(kAuxThreads);
  switch (mode) {
    case 0:
    case 1:
    case 9: {
      if (mode == 9 && (!d_w || !d_b)) return hb_invalid("hb_model_aux mode 9 parameters");
      const int rows = count / width;
      if (rows < 1) return hb_invalid("hb_model_aux rows");
      if (mode == 0)
        hipLaunchKernelGGL(aux_norm<0>, dim3(rows), block, 0, st, d_y, d_x, d_w, d_b, width, width, channels, spatial,
                           other_count, eps, activation);
      else if (mode == 1)
        hipLaunchKernelGGL(aux_norm<1>, dim3(rows), block, 0, st, d_y, d_x, d_w, d_b, width, width, channels, spatial,
                           other_count, eps, activation);
      else
        hipLaunchKernelGGL(aux_norm<9>, dim3(rows), block, 0, st, d_y, d_x, d_w, d_b, width, width, channels, spatial,
                           other_count, eps, activation);
      break;
    }
    case 2: {
      if (groups <= 0 || channels % groups) return hb_invalid("hb_model_aux groups");
      const int len = spatial * (channels / groups);
      hipLaunchKernelGGL(aux_norm<2>, dim3(groups * batch), block, 0, st, d_y, d_x, d_w, d_b, len, width, channels,
                         spatial, other_count, eps, activation);
      break;
    }
    case 3:
    case 4:
      if (!d_w || other_count <= 0) return hb_invalid("hb_model_aux broadcast operand");
      if (mode == 3)
        hipLaunchKernelGGL(aux_elementwise<3>, dim3(elementwise_grid(count)), block, 0, st, d_y, d_x, d_w, d_b,
                           (int64_t)count, width, channels, spatial, other_count, activation);
      else
        hipLaunchKernelGGL(aux_elementwise<4>, dim3(elementwise_grid(count)), block, 0, st, d_y, d_x, d_w, d_b,
                           (int64_t)count, width, channels, spatial, other_count, activation);
      break;
    case 5:
      hipLaunchKernelGGL(aux_elementwise<5>, dim3(elementwise_grid(count)), block, 0, st, d_y, d_x, d_w, d_b,
                         (int64_t)count, width, channels, spatial, other_count, activation);
      break;
    case 6:
      hipLaunchKernelGGL(aux_elementwise<6>, dim3(elementwise_grid(count)), block, 0, st, d_y, d_x, d_w, d_b,
                         (int64_t)count, width, channels, spatial, other_count, activation);
      break;
    case 7:
      hipLaunchKernelGGL(aux_elementwise<7>, dim3(elementwise_grid(count)), block, 0, st, d_y, d_x, d_w, d_b,
                         (int64_t)count, width, channels, spatial, other_count, activation);
      break;
    case 8: {
      if ((int64_t)width * spatial * batch != count) return hb_invalid("hb_model_aux transpose shape");
      const dim3 grid((spatial + 31) / 32, (width + 31) / 32, batch);
      hipLaunchKernelGGL(aux_transpose, grid, block, 0, st, d_y, d_x, width, spatial);
      break;
    }
    case 10:
      if (!d_w || !d_b) return hb_invalid("hb_model_aux mode 10 parameters");
      hipLaunchKernelGGL(aux_elementwise<10>, dim3(elementwise_grid(count)), block, 0, st, d_y, d_x, d_w, d_b,
                         (int64_t)count, width, channels, spatial, other_count, activation);
      break;
    case 11:
      if (!d_w || width % 2 || (groups != 1 && groups != batch)) return hb_invalid("hb_model_aux rope");
      hipLaunchKernelGGL(aux_rope, dim3(spatial * batch), block, 0, st, d_y, d_x, d_w, width, channels, spatial,
                         groups);
      break;
    case 12:
      if (channels < 2 * width) return hb_invalid("hb_model_aux gated width");
      hipLaunchKernelGGL(aux_elementwise<12>, dim3(elementwise_grid(count)), block, 0, st, d_y, d_x, d_w, d_b,
                         (int64_t)count, width, channels, spatial, other_count, activation);
      break;
    case 13:
      if (!d_w || groups <= 0 || channels < 2 * width) return hb_invalid("hb_model_aux concat");
      hipLaunchKernelGGL(aux_swiglu_concat, dim3(spatial * batch), block, 0, st, d_y, d_x, d_w, width, groups,
                         channels, activation);
      break;
    default:
      return hb_invalid("hb_model_aux mode");
  }
  return hb_check_launch("hb_model_aux");
}
