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

template <int T = kAuxThreads>
__device__ inline double block_sum(double v, double *red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();  // red may still be read from the previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < T / 64; ++w) t += red[w];
  return t;
}

// Affine / modulation step of the norms for element i of the task (MODE as in aux_norm).
// Mode 2: a task is one (batch, group) of channels/groups whole channels, so
// the channel of element i is pbase + i / spatial with pbase = (task % groups)
// * channels / groups (the reference's ((offset + i) / spatial) % channels).
template <int MODE>
__device__ inline float norm_affine(float v, int i, const float *w, const float *b, size_t pbase, int spatial) {
  if (MODE == 0 || MODE == 1) {
    if (w) v = __fmul_rn(v, w[i]);
    if (b) v = __fadd_rn(v, b[i]);
  } else if (MODE == 2) {
    const int ch = (int)pbase + (int)((unsigned)i / (unsigned)spatial);
    if (w) v = __fmul_rn(v, w[ch]);
    if (b) v = __fadd_rn(v, b[ch]);
  } else {
    v = __fadd_rn(v, __fmul_rn(v, w[pbase + i]));
    v = __fadd_rn(v, b[pbase + i]);
  }
  return v;
}

// Modes 0, 1, 2, 9 with the task held in registers: T threads x NV float4,
// len % 4 == 0 and 16-byte aligned rows; x is read once.
template <int MODE, int NV, int T>
__global__ __launch_bounds__(T) void aux_norm_reg(float *__restrict__ y, const float *__restrict__ x,
                                                  const float *__restrict__ w, const float *__restrict__ b, int len,
                                                  int width, int channels, int spatial, int groups, int other_count,
                                                  float eps, int act) {
  __shared__ double red[T / 64];
  const size_t offset = (size_t)blockIdx.x * (size_t)len;
  const float4 *xr = (const float4 *)(x + offset);
  const int nv4 = len / 4;
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = xr[min((int)threadIdx.x + j * T, nv4 - 1)];
  float mean = 0.0f;
  if (MODE != 1) {
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if ((int)threadIdx.x + j * T < nv4) s += (double)v[j].x + (double)v[j].y + (double)v[j].z + (double)v[j].w;
    mean = (float)(block_sum<T>(s, red) / (double)len);
  }
  double q = 0.0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if ((int)threadIdx.x + j * T < nv4) {
      const double d0 = __fsub_rn(v[j].x, mean), d1 = __fsub_rn(v[j].y, mean), d2 = __fsub_rn(v[j].z, mean),
                   d3 = __fsub_rn(v[j].w, mean);
      q += d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
    }
  }
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn((float)(block_sum<T>(q, red) / (double)len + (double)eps)));
  const size_t pbase = MODE == 9 ? (other_count != width ? (size_t)(blockIdx.x / spatial) * (size_t)width : 0)
                      : MODE == 2 ? (size_t)(blockIdx.x % groups) * (size_t)(channels / groups)
                                  : 0;
  float4 *yr = (float4 *)(y + offset);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = (int)threadIdx.x + j * T;
    if (idx < nv4) {
      float o[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      if (MODE == 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float t = norm_affine<MODE>(__fmul_rn(__fsub_rn(o[e], mean), inv), 4 * idx + e, w, b, pbase, spatial);
          o[e] = act ? activate(t, 4) : t;
        }
      } else {
        // the row's parameters are 16-byte aligned quads (width % 4 == 0)
        const float4 wv = w ? ((const float4 *)(w + pbase))[idx] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        const float4 bv = b ? ((const float4 *)(b + pbase))[idx] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float wq[4] = {wv.x, wv.y, wv.z, wv.w}, bq[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = __fmul_rn(__fsub_rn(o[e], mean), inv);
          if (MODE == 9) {
            t = __fadd_rn(t, __fmul_rn(t, wq[e]));
            t = __fadd_rn(t, bq[e]);
          } else {
            if (w) t = __fmul_rn(t, wq[e]);
            if (b) t = __fadd_rn(t, bq[e]);
          }
          o[e] = act ? activate(t, 4) : t;
        }
      }
      yr[idx] = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

// Modes 0, 1, 2, 9, any task length: one workgroup of T threads per task of
// `len` contiguous values, three passes (the later ones mostly from cache).
template <int MODE, int T>
__global__ __launch_bounds__(T) void aux_norm(float *__restrict__ y, const float *__restrict__ x,
                                              const float *__restrict__ w, const float *__restrict__ b, int len,
                                              int width, int channels, int spatial, int groups, int other_count,
                                              float eps, int act) {
  __shared__ double red[T / 64];
  const size_t offset = (size_t)blockIdx.x * (size_t)len;
  const float *xr = x + offset;
  float *yr = y + offset;
  float mean = 0.0f;
  if (MODE != 1) {
    double s = 0.0;
    for (int i = threadIdx.x; i < len; i += T) s += (double)xr[i];
    mean = (float)(block_sum<T>(s, red) / (double)len);
  }
  double q = 0.0;
  for (int i = threadIdx.x; i < len; i += T) {
    const double v = (double)__fsub_rn(xr[i], mean);
    q += v * v;
  }
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn((float)(block_sum<T>(q, red) / (double)len + (double)eps)));
  // mode 9: per-batch parameters unless they are shared by all batches; mode 2: the group's first channel
  const size_t pbase = MODE == 9 ? (other_count != width ? (size_t)(blockIdx.x / spatial) * (size_t)width : 0)
                      : MODE == 2 ? (size_t)(blockIdx.x % groups) * (size_t)(channels / groups)
                                  : 0;
  for (int i = threadIdx.x; i < len; i += T) {
    float v = __fmul_rn(__fsub_rn(xr[i], mean), inv);
    v = norm_affine<MODE>(v, i, w, b, pbase, spatial);
    if (act) v = activate(v, 4);
    yr[i] = v;
  }
}

// Group norm over few long groups: each group is split into `chunks` pieces
// of `chunk` values (a multiple of 4) handled by separate workgroups, in two
// launches.  The first reads x once for shifted sums per chunk: with s the
// group's first value and d = x - s (exact in double for floats within 2^29
// of each other, otherwise below 1e-16 relative), sum d and sum d^2.
// The second adds the chunk partials in chunk order (so every workgroup of a
// group derives the same mean and inv), takes the reference's float mean
// (float)(sum x / len) with sum x = sum d + len * s, and its centered sum of
// squares about that mean, sum (x - mean)^2 = sum d^2 - 2 e sum d + len e^2
// with e = mean - s (exact in double), then writes the output.  The
// reference's second pass rounds each x - mean to float before squaring;
// the two sums differ by about 1e-10 relative (1e-16 * len in the worst
// case, a shift far from every other value), so inv is the same float but
// at rounding ties.  Centering on a sample of the group keeps the
// cancellation bounded where |mean| >> standard deviation.
// ws: double sum[tasks][chunks], then double sq[tasks][chunks].
constexpr int kGnUnroll = 4;

__device__ inline void shifted_add(const float4 v, double shift, double &s, double &q) {
  const double d0 = (double)v.x - shift, d1 = (double)v.y - shift, d2 = (double)v.z - shift,
               d3 = (double)v.w - shift;
  s += (d0 + d1) + (d2 + d3);
  q = fma(d3, d3, fma(d2, d2, fma(d1, d1, fma(d0, d0, q))));
}

// n / d for quotients below 2^22: the float estimate n * (1/d) is within one
// of the quotient there (three roundings of 2^-24 each), and one step against
// the remainder makes it exact.
__device__ inline unsigned small_quotient(unsigned n, unsigned d, float rd) {
  int q = (int)__fmul_rn((float)n, rd);
  const int r = (int)n - q * (int)d;
  q += r < 0 ? -1 : (r >= (int)d ? 1 : 0);
  return (unsigned)q;
}

template <int PASS>
__global__ __launch_bounds__(kAuxThreads) void aux_group_norm_chunk(float *__restrict__ y, const float *__restrict__ x,
                                                                    const float *__restrict__ w,
                                                                    const float *__restrict__ b, double *ws, int len,
                                                                    int chunk, int chunks, int tasks, int channels,
                                                                    int spatial, int groups, float eps, int act) {
  __shared__ double red[kAuxThreads / 64];
  __shared__ float stats[2];
  constexpr int T = kAuxThreads;
  const int c = blockIdx.x, task = blockIdx.y;
  const size_t offset = (size_t)task * (size_t)len;
  const int v0 = c * (chunk / 4), v1 = min(c * chunk + chunk, len) / 4;  // the chunk's float4 range
  const float4 *xr = (const float4 *)(x + offset);
  double *sum = ws + (size_t)task * chunks, *sq = ws + (size_t)tasks * chunks + (size_t)task * chunks;
  const float shift = x[offset];
  if (PASS == 0) {
    double s = 0.0, q = 0.0;
    int i = v0 + (int)threadIdx.x;
    for (; i + (kGnUnroll - 1) * T < v1; i += kGnUnroll * T) {
      float4 v[kGnUnroll];
#pragma unroll
      for (int u = 0; u < kGnUnroll; ++u) v[u] = xr[i + u * T];
#pragma unroll
      for (int u = 0; u < kGnUnroll; ++u) shifted_add(v[u], (double)shift, s, q);
    }
    for (; i < v1; i += T) shifted_add(xr[i], (double)shift, s, q);
    s = block_sum(s, red);
    q = block_sum(q, red);
    if (threadIdx.x == 0) {
      sum[c] = s;
      sq[c] = q;
    }
    return;
  }
  if (threadIdx.x == 0) {
    double ts = 0.0, tq = 0.0;
    for (int k = 0; k < chunks; ++k) {
      ts += sum[k];
      tq += sq[k];
    }
    const double n = (double)len;
    const float mean = (float)((ts + n * (double)shift) / n);
    const double e = (double)mean - (double)shift;
    const double centered = (tq - 2.0 * e * ts) + n * e * e;
    stats[0] = mean;
    stats[1] = __fdiv_rn(1.0f, __fsqrt_rn((float)(centered / n + (double)eps)));
  }
  __syncthreads();
  const float mean = stats[0], inv = stats[1];
  const int cpg = channels / groups;
  const size_t pbase = (size_t)(task % groups) * (size_t)cpg;
  const float rsp = __fdiv_rn(1.0f, (float)spatial);
  const bool fast = cpg < (1 << 22);  // the channel within the group by small_quotient
  // spatial % 4 == 0: a quad lies in one channel, and a lane's channel changes
  // only every spatial / 4 quads, so its parameters stay in registers until then
  const bool quad_channel = spatial % 4 == 0 && fast;
  size_t held = ~(size_t)0;
  float hw = 1.0f, hb = 0.0f;
  float4 *yr = (float4 *)(y + offset);
  auto finish = [&](float4 v, int idx) {
    float o[4] = {v.x, v.y, v.z, v.w};
    if (quad_channel && (w || b)) {
      const size_t ch = pbase + small_quotient(4u * (unsigned)idx, (unsigned)spatial, rsp);
      if (ch != held) {
        held = ch;
        hw = w ? w[ch] : 1.0f;
        hb = b ? b[ch] : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = __fmul_rn(__fsub_rn(o[e], mean), inv);
        if (w) t = __fmul_rn(t, hw);
        if (b) t = __fadd_rn(t, hb);
        o[e] = act ? activate(t, 4) : t;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = __fmul_rn(__fsub_rn(o[e], mean), inv);
        if (w || b) {
          const unsigned i = 4u * (unsigned)idx + (unsigned)e;
          const size_t ch = pbase + (fast ? small_quotient(i, (unsigned)spatial, rsp) : i / (unsigned)spatial);
          if (w) t = __fmul_rn(t, w[ch]);
          if (b) t = __fadd_rn(t, b[ch]);
        }
        o[e] = act ? activate(t, 4) : t;
      }
    }
    __builtin_nontemporal_store(hb_f32x4{o[0], o[1], o[2], o[3]}, (hb_f32x4 *)(yr + idx));
  };
  int i = v0 + (int)threadIdx.x;
  for (; i + (kGnUnroll - 1) * T < v1; i += kGnUnroll * T) {
    float4 v[kGnUnroll];
#pragma unroll
    for (int u = 0; u < kGnUnroll; ++u) v[u] = xr[i + u * T];
#pragma unroll
    for (int u = 0; u < kGnUnroll; ++u) finish(v[u], i + u * T);
  }
  for (; i < v1; i += T) finish(xr[i], i);
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

// The same modes, four consecutive values per thread with 16-byte loads and
// stores (count % 4 == 0, x and y 16-byte aligned; mode 12 also needs width
// and channels divisible by 4 so each quad of gate and up values is contiguous).
template <int MODE>
__global__ __launch_bounds__(kAuxThreads) void aux_elementwise4(float *__restrict__ y, const float *__restrict__ x,
                                                                const float *__restrict__ w,
                                                                const float *__restrict__ b, int64_t count4,
                                                                int width, int channels, int spatial,
                                                                int other_count, int act) {
  const int64_t stride = (int64_t)gridDim.x * kAuxThreads;
  for (int64_t q = (int64_t)blockIdx.x * kAuxThreads + threadIdx.x; q < count4; q += stride) {
    const int64_t i0 = 4 * q;
    float o[4];
    if (MODE == 12) {
      const int64_t column = i0 % width, row = i0 / width;
      const float *a = x + row * channels + column;
      const float4 g = *(const float4 *)(a + (act ? 0 : width)), u = *(const float4 *)(a + (act ? width : 0));
      o[0] = __fmul_rn(activate(g.x, 5), u.x);
      o[1] = __fmul_rn(activate(g.y, 5), u.y);
      o[2] = __fmul_rn(activate(g.z, 5), u.z);
      o[3] = __fmul_rn(activate(g.w, 5), u.w);
    } else {
      const float4 xv = ((const float4 *)x)[q];
      const float xi[4] = {xv.x, xv.y, xv.z, xv.w};
      const float4 bv = MODE == 10 ? ((const float4 *)b)[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      const float bi[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t i = i0 + e;
        if (MODE == 3) {
          o[e] = __fadd_rn(xi[e], w[i % other_count]);
        } else if (MODE == 4) {
          o[e] = __fmul_rn(xi[e], w[i % other_count]);
        } else if (MODE == 5 || MODE == 6 || MODE == 7) {
          o[e] = activate(xi[e], MODE == 5 ? 4 : MODE == 6 ? 1 : 2);
        } else {  // 10
          const int64_t channel = i % width, batch = i / ((int64_t)width * spatial);
          const int64_t pb = other_count == width ? 0 : batch;
          o[e] = __fadd_rn(__fmul_rn(xi[e], w[pb * width + channel]), bi[e]);
        }
      }
    }
    ((float4 *)y)[q] = make_float4(o[0], o[1], o[2], o[3]);
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

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Register-resident tasks when they fit (256 threads up to 8192 values, 1024
// threads up to 65536), else the three-pass kernel; few long tasks (group
// norm) take 1024-thread workgroups.
template <int MODE>
void launch_norm(float *y, const float *x, const float *w, const float *b, int tasks, int len, int width,
                 int channels, int spatial, int groups, int other_count, float eps, int act, bool vec,
                 hipStream_t st) {
  const dim3 grid(tasks);
  const int nv4 = len / 4;
  // Rows of 513-2048 values: two waves per row, where the 256-thread form
  // leaves a quarter to a half of its lanes idle (4096 rows: LayerNorm +
  // modulation 10.9 -> 9.6 us at 1536 values and 13.2 -> 11.8 at 2048,
  // RMSNorm 10.0 -> 9.3 and 13.1 -> 11.8; from 3072 values the 256-thread
  // form is as fast or faster).
  if (vec && nv4 > 128 && nv4 <= 128 * 4) {
    if (nv4 <= 128 * 2)
      hipLaunchKernelGGL((aux_norm_reg<MODE, 2, 128>), grid, dim3(128), 0, st, y, x, w, b, len, width, channels,
                         spatial, groups, other_count, eps, act);
    else if (nv4 <= 128 * 3)
      hipLaunchKernelGGL((aux_norm_reg<MODE, 3, 128>), grid, dim3(128), 0, st, y, x, w, b, len, width, channels,
                         spatial, groups, other_count, eps, act);
    else
      hipLaunchKernelGGL((aux_norm_reg<MODE, 4, 128>), grid, dim3(128), 0, st, y, x, w, b, len, width, channels,
                         spatial, groups, other_count, eps, act);
    return;
  }
  if (vec && nv4 <= 256 * 1) {
    hipLaunchKernelGGL((aux_norm_reg<MODE, 1, 256>), grid, dim3(256), 0, st, y, x, w, b, len, width, channels,
                       spatial, groups, other_count, eps, act);
  } else if (vec && nv4 <= 256 * 2) {
    hipLaunchKernelGGL((aux_norm_reg<MODE, 2, 256>), grid, dim3(256), 0, st, y, x, w, b, len, width, channels,
                       spatial, groups, other_count, eps, act);
  } else if (vec && nv4 <= 256 * 4) {
    hipLaunchKernelGGL((aux_norm_reg<MODE, 4, 256>), grid, dim3(256), 0, st, y, x, w, b, len, width, channels,
                       spatial, groups, other_count, eps, act);
  } else if (vec && nv4 <= 256 * 8) {
    hipLaunchKernelGGL((aux_norm_reg<MODE, 8, 256>), grid, dim3(256), 0, st, y, x, w, b, len, width, channels,
                       spatial, groups, other_count, eps, act);
  } else if (vec && nv4 <= 1024 * 16) {
    hipLaunchKernelGGL((aux_norm_reg<MODE, 16, 1024>), grid, dim3(1024), 0, st, y, x, w, b, len, width, channels,
                       spatial, groups, other_count, eps, act);
  } else if (tasks < 1024) {
    hipLaunchKernelGGL((aux_norm<MODE, 1024>), grid, dim3(1024), 0, st, y, x, w, b, len, width, channels, spatial,
                       groups, other_count, eps, act);
  } else {
    hipLaunchKernelGGL((aux_norm<MODE, 256>), grid, dim3(256), 0, st, y, x, w, b, len, width, channels, spatial,
                       groups, other_count, eps, act);
  }
}

// Chunked group-norm plan: used when the groups alone would leave most CUs
// idle and the values divide into float4 quads; 0 chunks means "not chunked".
struct GroupPlan {
  int chunks, chunk;
};

GroupPlan group_plan(int tasks, int len) {
  GroupPlan p{0, 0};
  if (tasks >= 512 || len % 4 || len < 8192) return p;
  int chunks = (1024 + tasks - 1) / tasks;  // aim for about 1024 workgroups
  if (chunks > len / 4096) chunks = len / 4096;
  if (chunks < 2) return p;
  int chunk = (len + chunks - 1) / chunks;
  chunk = (chunk + 3) / 4 * 4;
  p.chunks = (len + chunk - 1) / chunk;
  p.chunk = chunk;
  return p;
}

int elementwise_grid(int64_t count) {
  const int64_t blocks = (count + kAuxThreads - 1) / kAuxThreads;
  return (int)(blocks < 65536 ? blocks : 65536);
}

template <int MODE>
void launch_elementwise(float *y, const float *x, const float *w, const float *b, int count, int width, int channels,
                        int spatial, int other_count, int act, hipStream_t st) {
  bool vec = count % 4 == 0 && aligned16(x) && aligned16(y) && (MODE != 10 || aligned16(b));
  if (MODE == 12) vec = vec && width % 4 == 0 && channels % 4 == 0;
  if (vec) {
    const int64_t count4 = count / 4;
    hipLaunchKernelGGL(aux_elementwise4<MODE>, dim3(elementwise_grid(count4)), dim3(kAuxThreads), 0, st, y, x, w, b,
                       count4, width, channels, spatial, other_count, act);
  } else {
    hipLaunchKernelGGL(aux_elementwise<MODE>, dim3(elementwise_grid(count)), dim3(kAuxThreads), 0, st, y, x, w, b,
                       (int64_t)count, width, channels, spatial, other_count, act);
  }
}

}  // namespace

extern "C" size_t hb_model_aux_workspace_bytes(int mode, int channels, int spatial, int groups, int batch) {
  if (mode != 2 || groups <= 0 || channels <= 0 || spatial <= 0 || batch <= 0 || channels % groups) return 0;
  const int64_t len64 = (int64_t)spatial * (channels / groups), tasks64 = (int64_t)groups * batch;
  if (len64 > INT32_MAX || tasks64 > INT32_MAX) return 0;
  const GroupPlan p = group_plan((int)tasks64, (int)len64);
  return p.chunks ? (size_t)tasks64 * (size_t)p.chunks * 2u * sizeof(double) : 0;
}

extern "C" int hb_model_aux_ws(float *d_y, const float *d_x, const float *d_w, const float *d_b, int mode, int count,
                               int width, int channels, int spatial, int groups, int batch, int other_count,
                               int activation, float eps, void *d_workspace, size_t workspace_bytes, hb_stream s) {
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
      const bool vec = width % 4 == 0 && aligned16(d_x) && aligned16(d_y) && aligned16(d_w) && aligned16(d_b);
      if (mode == 0)
        launch_norm<0>(d_y, d_x, d_w, d_b, rows, width, width, channels, spatial, 1, other_count, eps, activation,
                       vec, st);
      else if (mode == 1)
        launch_norm<1>(d_y, d_x, d_w, d_b, rows, width, width, channels, spatial, 1, other_count, eps, activation,
                       vec, st);
      else
        launch_norm<9>(d_y, d_x, d_w, d_b, rows, width, width, channels, spatial, 1, other_count, eps, activation,
                       vec, st);
      break;
    }
    case 2: {
      if (groups <= 0 || channels % groups) return hb_invalid("hb_model_aux groups");
      if ((int64_t)batch * channels * spatial > count) return hb_invalid("hb_model_aux group norm extent");
      const int len = spatial * (channels / groups);
      const bool vec = len % 4 == 0 && aligned16(d_x) && aligned16(d_y);
      const GroupPlan gp = group_plan(groups * batch, len);
      const size_t need = hb_model_aux_workspace_bytes(mode, channels, spatial, groups, batch);
      if (vec && gp.chunks && d_workspace && workspace_bytes >= need && ((uintptr_t)d_workspace & 7u) == 0) {
        const dim3 grid(gp.chunks, groups * batch);
        double *ws = (double *)d_workspace;
        hipLaunchKernelGGL(aux_group_norm_chunk<0>, grid, block, 0, st, d_y, d_x, d_w, d_b, ws, len, gp.chunk,
                           gp.chunks, groups * batch, channels, spatial, groups, eps, activation);
        hipLaunchKernelGGL(aux_group_norm_chunk<1>, grid, block, 0, st, d_y, d_x, d_w, d_b, ws, len, gp.chunk,
                           gp.chunks, groups * batch, channels, spatial, groups, eps, activation);
        break;
      }
      launch_norm<2>(d_y, d_x, d_w, d_b, groups * batch, len, width, channels, spatial, groups, other_count, eps,
                     activation, vec, st);
      break;
    }
    case 3:
    case 4:
      if (!d_w || other_count <= 0) return hb_invalid("hb_model_aux broadcast operand");
      if (mode == 3)
        launch_elementwise<3>(d_y, d_x, d_w, d_b, count, width, channels, spatial, other_count, activation, st);
      else
        launch_elementwise<4>(d_y, d_x, d_w, d_b, count, width, channels, spatial, other_count, activation, st);
      break;
    case 5:
      launch_elementwise<5>(d_y, d_x, d_w, d_b, count, width, channels, spatial, other_count, activation, st);
      break;
    case 6:
      launch_elementwise<6>(d_y, d_x, d_w, d_b, count, width, channels, spatial, other_count, activation, st);
      break;
    case 7:
      launch_elementwise<7>(d_y, d_x, d_w, d_b, count, width, channels, spatial, other_count, activation, st);
      break;
    case 8: {
      if ((int64_t)width * spatial * batch != count) return hb_invalid("hb_model_aux transpose shape");
      const dim3 grid((spatial + 31) / 32, (width + 31) / 32, batch);
      hipLaunchKernelGGL(aux_transpose, grid, block, 0, st, d_y, d_x, width, spatial);
      break;
    }
    case 10:
      if (!d_w || !d_b) return hb_invalid("hb_model_aux mode 10 parameters");
      launch_elementwise<10>(d_y, d_x, d_w, d_b, count, width, channels, spatial, other_count, activation, st);
      break;
    case 11:
      if (!d_w || width % 2 || (groups != 1 && groups != batch)) return hb_invalid("hb_model_aux rope");
      hipLaunchKernelGGL(aux_rope, dim3(spatial * batch), block, 0, st, d_y, d_x, d_w, width, channels, spatial,
                         groups);
      break;
    case 12:
      if (channels < 2 * width) return hb_invalid("hb_model_aux gated width");
      launch_elementwise<12>(d_y, d_x, d_w, d_b, count, width, channels, spatial, other_count, activation, st);
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

extern "C" int hb_model_aux(float *d_y, const float *d_x, const float *d_w, const float *d_b, int mode, int count,
                            int width, int channels, int spatial, int groups, int batch, int other_count,
                            int activation, float eps, hb_stream s) {
  return hb_model_aux_ws(d_y, d_x, d_w, d_b, mode, count, width, channels, spatial, groups, batch, other_count,
                         activation, eps, nullptr, 0, s);
}
