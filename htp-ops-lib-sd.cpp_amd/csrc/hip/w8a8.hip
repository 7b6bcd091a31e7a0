// W8A8 linear (opcode 15) on gfx950: weight prepack, per-token activation
// quantization and the INT8 MFMA GEMM with its fused output epilogue.
//
// Arithmetic contract (reference src/dsp/ops/linear_w8a8.c):
//   t = x*inv; s = max(max|t|/127, 1e-12); r = 1/s;                 :34-40, :83-109
//   u = rne(clamp(t*r + 128, 1, 255))  (clamp on IEEE bits)          :42-59
//   acc = sum_k u*W(n,k) (int32);  c = acc - (sums[n] << 7) (wrap)   :478-502, :159-171
//   y = ((float)c * sw[n]) * s[m]                                    :172-179
// Every float step is one IEEE RNE operation (no contraction).  The GEMM
// multiplies signed q = u - 128 by W and adds delta[n] = 128*(sum_k W - sums[n]),
// which equals acc - (sums << 7) modulo 2^32 for every input.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "hb_internal.h"

namespace {

constexpr int kKStep = 64;        // k per v_mfma_i32_16x16x64_i8
constexpr int kFragBytes = 1024;  // one 16 x 64 int8 operand tile, lane-ordered

size_t kp_of(int k) { return hb_round_up((size_t)k, 64); }
size_t mp_of(int m) { return hb_round_up((size_t)m, 16); }

// ---------------------------------------------------------------------------
// Prepack: constants blob -> MFMA tile image.
// ---------------------------------------------------------------------------

__device__ inline size_t blob_weight_offset(int k, int col, int kk) {
  // W(n,k) address in the blob (reference linear_w8a8.c:453,482,486-488;
  // tests/hmx-probe/study_dsp.c:82-84); kk is a multiple of 4.
  return 128u + (size_t)(col / 64) * 64u * (size_t)k + (size_t)(kk / 32) * 2048u +
         (size_t)((col % 64) / 32) * 1024u + (size_t)((kk % 32) / 4) * 128u + (size_t)(col % 32) * 4u;
}

__global__ __launch_bounds__(256) void w8a8_prepack_weights(uint4 *__restrict__ wpack,
                                                           const uint8_t *__restrict__ blob, int k, int n,
                                                           int kp) {
  const size_t slots = (size_t)n * (size_t)kp / 16u;
  const int kblocks = kp / kKStep;
  for (size_t slot = (size_t)blockIdx.x * blockDim.x + threadIdx.x; slot < slots;
       slot += (size_t)gridDim.x * blockDim.x) {
    const size_t blk = slot / 64u;
    const int lane = (int)(slot % 64u);
    const int nb = (int)(blk / (size_t)kblocks), kb = (int)(blk % (size_t)kblocks);
    const int col = nb * 16 + lane % 16;
    const int k0 = kb * kKStep + (lane / 16) * 16;
    uint32_t w[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int kk = k0 + g * 4;
      w[g] = kk < k ? *(const uint32_t *)(blob + blob_weight_offset(k, col, kk)) : 0u;
    }
    wpack[slot] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Column parameters: a workgroup per 64-column group, whose weights are one
// contiguous run of 64*k blob bytes (per 32 k, 2 KB: the two 32-column halves,
// each 8 rows of 4 k x 32 columns); its 16 waves take the 32-k blocks in turn
// and lane l sums column l of the group; the waves' sums are added in LDS
// (exact integer sums, so the split does not change them).  The grid's
// threads also copy the smoothing vector, zero-padded to kp.
__global__ __launch_bounds__(1024) void w8a8_prepack_columns(float *__restrict__ sw_out, int32_t *__restrict__ delta,
                                                            int32_t *__restrict__ wsum128,
                                                            float *__restrict__ inv_out,
                                                            const uint8_t *__restrict__ blob, int k, int n,
                                                            int kp) {
  __shared__ int32_t part[16][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t kn = (size_t)k * (size_t)n;
  const uint8_t *grp =
      blob + 128u + (size_t)blockIdx.x * 64u * (size_t)k + (size_t)(lane / 32) * 1024u + (size_t)(lane % 32) * 4u;
  int32_t sum = 0;
  for (int kb = wave; kb < k / 32; kb += 16) {
    const uint8_t *p = grp + (size_t)kb * 2048u;
    uint32_t w[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) w[r] = *(const uint32_t *)(p + r * 128);
#pragma unroll
    for (int r = 0; r < 8; ++r)
      sum += (int32_t)(int8_t)(w[r] & 0xffu) + (int32_t)(int8_t)((w[r] >> 8) & 0xffu) +
             (int32_t)(int8_t)((w[r] >> 16) & 0xffu) + (int32_t)(int8_t)(w[r] >> 24);
  }
  part[wave][lane] = sum;
  __syncthreads();
  if (wave == 0) {
    const int t = blockIdx.x * 64 + lane;
    uint32_t tot = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) tot += (uint32_t)part[w][lane];
    const float sw = *(const float *)(blob + 128u + kn + 4u * (size_t)t);
    const int32_t sums = *(const int32_t *)(blob + 128u + kn + 4u * (size_t)n + 4u * (size_t)t);
    sw_out[t] = sw;
    wsum128[t] = (int32_t)(tot << 7);
    delta[t] = (int32_t)((tot - (uint32_t)sums) << 7);
  }
  for (int t = blockIdx.x * 1024 + threadIdx.x; t < kp; t += gridDim.x * 1024)
    inv_out[t] = t < k ? *(const float *)(blob + 128u + kn + 8u * (size_t)n + 4u * (size_t)t) : 0.0f;
}

// ---------------------------------------------------------------------------
// Activation quantization: blocks of 8 or 16 rows (a wave per row) for many
// rows, a workgroup per row for few or long rows, a two-pass fallback for
// unaligned rows.
// ---------------------------------------------------------------------------

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// u = rne(clamp(v, 1, 255)) with the clamp on the IEEE bits as signed
// integers, returned as q = u - 128 in the low byte.
__device__ inline uint32_t quantize_byte(float t, float r) {
  const float v = __fadd_rn(__fmul_rn(t, r), 128.0f);
  int32_t b = __float_as_int(v);
  b = max(b, 0x3f800000);  // 1.0f
  b = min(b, 0x437f0000);  // 255.0f
  const int32_t u = (int32_t)rintf(__int_as_float(b));
  return (uint32_t)(u - 128) & 0xffu;
}

// Quantized activations use the weights' MFMA tile layout: 16 rows x 64 k
// per 1 KB block, element (m,k) at ((m/16)*(kp/64) + k/64)*1024 +
// ((m%16) + 16*((k%64)/16))*16 + k%16.  Returns the word holding k..k+3 (k%4 == 0).
__device__ inline uint32_t *q_word(int8_t *q, int kp, int row, int k) {
  const size_t off = ((size_t)(row / 16) * (size_t)(kp / kKStep) + (size_t)(k / kKStep)) * kFragBytes +
                     (size_t)((row % 16) + 16 * ((k % kKStep) / 16)) * 16u + (size_t)(k % 16);
  return (uint32_t *)(q + off);
}

// Any row length and 4-byte aligned pointers: two passes over the row
// (the second pass re-reads x from cache and recomputes the same t).
__global__ __launch_bounds__(256) void w8a8_quant_rows_any(int8_t *__restrict__ q, float *__restrict__ scales,
                                                          const float *__restrict__ x,
                                                          const float *__restrict__ inv, int m, int k, int kp) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  const float *xr = x + (size_t)row * k;
  float amax = 0.0f;
  for (int i = lane; i < k; i += 64) amax = fmaxf(amax, fabsf(__fmul_rn(xr[i], inv[i])));
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
  const float r = __fdiv_rn(1.0f, s);
  if (lane == 0) scales[row] = s;
  for (int i = 4 * lane; i < kp; i += 256) {
    uint32_t word = 0u;
    if (i < k) {
#pragma unroll
      for (int e = 0; e < 4; ++e) word |= quantize_byte(__fmul_rn(xr[i + e], inv[i + e]), r) << (8 * e);
    }
    *q_word(q, kp, row, i) = word;
  }
}

// Many rows: one workgroup per block of ROWS rows (8 or 16), one wave per
// row with its NV float4 per lane in registers.  The block's quantized bytes
// are assembled in LDS and written out as whole 128-byte lines (a tile holds
// 16 rows x 64 k; rows r..r+7 of one 16-k group are 128 contiguous bytes), so
// no output line is shared between workgroups.  Rows past m inside the block
// are written as zeros.
// INV_LDS (long rows): the smoothing vector is copied once per workgroup into
// LDS and read from there, so a wave holds only its row (NV float4) and two
// workgroups fit on a CU: one's stores overlap the other's loads.
template <int NV, int ROWS, int MINB = 1, bool INV_LDS = false>
__global__ __launch_bounds__(64 * ROWS, MINB) void w8a8_quant_block(int8_t *__restrict__ q, float *__restrict__ scales,
                                                              const float *__restrict__ x,
                                                              const float *__restrict__ inv, int m, int k, int kp) {
  static_assert(ROWS == 8 || ROWS == 16, "a block is half or all of a tile's rows");
  extern __shared__ uint4 stage[];  // ROWS * kp bytes: [tile][16-k group][row][16 bytes]
  __shared__ float4 ivs[INV_LDS ? 64 * NV : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * ROWS, row = row0 + wave;
  const bool live = row < m;
  const int nvec = k / 4;
  // x is read once (non-temporal loads keep it from displacing the smoothing
  // vector and the quantized output in the caches); inv is shared by all rows.
  const hb_f32x4 *xr = (const hb_f32x4 *)(x + (size_t)min(row, m - 1) * k);
  const float4 *iv = (const float4 *)inv;
  float4 a[NV], b[INV_LDS ? 1 : NV];
  if constexpr (INV_LDS) {
    // buffer loads of the row (32-bit offsets, not 64-bit addresses, per
    // load); offsets past the row's end read zeros
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)xr, 0, (uint32_t)nvec * 16u, 0x00020000);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const hb_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(lane + 64 * j) * 16u, 0, 2);
      a[j] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
    }
  } else {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int idx = min(lane + 64 * j, nvec - 1);
      const hb_f32x4 v = __builtin_nontemporal_load(xr + idx);
      a[j] = make_float4(v.x, v.y, v.z, v.w);
      b[j] = iv[idx];
    }
  }
  if constexpr (INV_LDS) {
    for (int v = tid; v < nvec; v += 64 * ROWS) ivs[v] = iv[v];
    __syncthreads();
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float4 bj = INV_LDS ? ivs[min(lane + 64 * j, nvec - 1)] : b[INV_LDS ? 0 : j];
    a[j] = make_float4(__fmul_rn(a[j].x, bj.x), __fmul_rn(a[j].y, bj.y), __fmul_rn(a[j].z, bj.z),
                       __fmul_rn(a[j].w, bj.w));
    if (lane + 64 * j < nvec)
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a[j].x), fabsf(a[j].y)), fmaxf(fabsf(a[j].z), fabsf(a[j].w))));
  }
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
  const float r = __fdiv_rn(1.0f, s);
  if (live && lane == 0) scales[row] = s;
  uint32_t *sw = (uint32_t *)stage;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = lane + 64 * j;
    if (idx < kp / 4) {
      const int kk = 4 * idx;
      const uint32_t word = (live && idx < nvec) ? (quantize_byte(a[j].x, r) | (quantize_byte(a[j].y, r) << 8) |
                                                    (quantize_byte(a[j].z, r) << 16) | (quantize_byte(a[j].w, r) << 24))
                                                 : 0u;
      sw[((kk / kKStep) * 4 * ROWS + ((kk % kKStep) / 16) * ROWS + wave) * 4 + (kk % 16) / 4] = word;
    }
  }
  __syncthreads();
  // rows row0..row0+ROWS-1 sit at row offset row0 % 16 of tile row row0 / 16
  int8_t *base = q + (size_t)(row0 / 16) * (size_t)kp * 16u + (size_t)(row0 % 16) * 16u;
  for (int v = tid; v < ROWS * kp / 16; v += 64 * ROWS) {
    const int tile = v / (4 * ROWS), g = (v / ROWS) % 4, rr = v % ROWS;
    *(uint4 *)(base + (size_t)tile * kFragBytes + (size_t)(g * 16 + rr) * 16u) = stage[v];
  }
}

// One 512-thread workgroup per row: for few rows (a single wave per row is
// latency bound there) and for rows longer than the register path holds.
// Loads are unconditional with the index clamped into the row, so they all
// issue before the first use; out-of-row values never reach the maximum.
constexpr int kRowThreads = 512;

template <int VX>
__global__ __launch_bounds__(kRowThreads) void w8a8_quant_rows_wg(int8_t *__restrict__ q, float *__restrict__ scales,
                                                                  const float *__restrict__ x,
                                                                  const float *__restrict__ inv, int k, int kp) {
  __shared__ float red[kRowThreads / 64];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float4 *xr = (const float4 *)(x + (size_t)row * k);
  const float4 *iv = (const float4 *)inv;
  const int nvec = k / 4;
  float4 a[VX], b[VX];
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    const int idx = min(tid + kRowThreads * j, nvec - 1);
    a[j] = xr[idx];
    b[j] = iv[idx];
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    a[j] = make_float4(__fmul_rn(a[j].x, b[j].x), __fmul_rn(a[j].y, b[j].y), __fmul_rn(a[j].z, b[j].z),
                       __fmul_rn(a[j].w, b[j].w));
    if (tid + kRowThreads * j < nvec)
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a[j].x), fabsf(a[j].y)), fmaxf(fabsf(a[j].z), fabsf(a[j].w))));
  }
  amax = wave_max(amax);
  if (lane == 0) red[wave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kRowThreads / 64; ++w) amax = fmaxf(amax, red[w]);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
  const float r = __fdiv_rn(1.0f, s);
  if (tid == 0) scales[row] = s;
  const int qvec = kp / 4;
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    const int idx = tid + kRowThreads * j;
    if (idx < nvec) {
      *q_word(q, kp, row, 4 * idx) = quantize_byte(a[j].x, r) | (quantize_byte(a[j].y, r) << 8) |
                                    (quantize_byte(a[j].z, r) << 16) | (quantize_byte(a[j].w, r) << 24);
    } else if (idx < qvec) {
      *q_word(q, kp, row, 4 * idx) = 0u;
    }
  }
}

// ---------------------------------------------------------------------------
// Output epilogue shared by both GEMM kernels.
// ---------------------------------------------------------------------------

__device__ inline float gelu_tanh(float z) {
  // z * sigmoid(1.5957691216057308*(z + 0.044715*z^3)), stable sigmoid
  // (reference src/dsp/ops/mat_mul.c:788-826, mode 1).  The exponential and
  // the reciprocal are the hardware's v_exp_f32 and v_rcp_f32 (each within
  // 1 ulp; the argument is at least -126, 1 + e lies in [1, 2]), about 3e-7
  // relative in all, inside the 1e-5 bound; IEEE division would cost a long
  // sequence per output element (the GELU GEMM at 4096x1536x6144 took 59.6
  // against 47.0 us).
  const float cubic = __fmul_rn(__fmul_rn(z, z), z);
  const float inner = __fadd_rn(z, __fmul_rn(cubic, 0.044715f));
  const float a = __fmul_rn(inner, 1.5957691216057308f);
  const float neg = fmaxf(__fmul_rn(fabsf(a), -1.4426950408889634f), -126.0f);
  const float e = __builtin_amdgcn_exp2f(neg);
  const float inv = __builtin_amdgcn_rcpf(__fadd_rn(e, 1.0f));
  const float sig = a < 0.0f ? __fmul_rn(e, inv) : inv;
  return __fmul_rn(z, sig);
}

// DPP row shifts (within 16-lane rows): lane i takes lane i - 8 / lane i + 8.
constexpr int kDppRowShr8 = 0x118, kDppRowShl8 = 0x108;

// Bits of one output element: int32 raw accumulator, or the scaled f32.
template <int EPI>
__device__ inline uint32_t epilogue_bits(int32_t acc, int32_t corr, float sw, float s) {
  const int32_t c = (int32_t)((uint32_t)acc + (uint32_t)corr);
  if (EPI == HB_W8A8_EPI_RAW) return (uint32_t)c;
  float v = __fmul_rn(__fmul_rn((float)c, sw), s);
  if (EPI == HB_W8A8_EPI_SCALE_GELU) v = gelu_tanh(v);
  return __float_as_uint(v);
}

template <int EPI>
__device__ inline void store_result(void *y, int ldy, int row, int col, int32_t acc, int32_t corr, float sw,
                                    float s) {
  const size_t idx = (size_t)row * (size_t)ldy + (size_t)col;
  __builtin_nontemporal_store(epilogue_bits<EPI>(acc, corr, sw, s), (uint32_t *)y + idx);
}

// ---------------------------------------------------------------------------
// Tiled GEMM: BM x BN output tile per workgroup of WM x WN waves, 64-k stages.
// Operands move global -> LDS by direct DMA (global_load_lds_dwordx4): one
// wave instruction fills one 1 KB, MFMA-lane-ordered 16 x 64 block (lane l's
// 16 bytes land at l*16), so the MFMA loop reads LDS conflict-free with
// ds_read_b128 at lane*16.  S stages form a ring: stage kt+S-1 is in flight
// while stage kt is multiplied; each wave waits only for its own DMA of stage
// kt (vmcnt), then one barrier publishes the stage to all waves.
// A = q int8 [mp][kp] row-major; B = packed tiles (see hb.h).
// ---------------------------------------------------------------------------

#include "hb_lds_ring.h"
static_assert(kFragBytes == kRingTileBytes, "operand tiles are the ring's tiles");

template <int BM, int BN, int WM, int WN, int S, int EPI>
__global__ __launch_bounds__(64 * WM *WN) void w8a8_gemm_tiles(void *__restrict__ y, int ldy,
                                                               const int8_t *__restrict__ q,
                                                               const float *__restrict__ scales,
                                                               const int8_t *__restrict__ wpack,
                                                               const float *__restrict__ sw,
                                                               const int32_t *__restrict__ corr, int m, int n,
                                                               int kp) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int ABLK = BM / 16, BBLK = BN / 16;
  constexpr int NB = ABLK + BBLK;
  constexpr int PW = (NB + NW - 1) / NW;  // DMA instructions per wave per stage (at most)
  constexpr int PW_LO = NB / NW;          // ... for waves at or above NB % NW
  static_assert(PW_LO >= 1, "every wave takes part in the DMA");
  constexpr int STAGE = (ABLK + BBLK) * kFragBytes;
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE];

  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kt_count = kp / kKStep;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;

  // DMA instruction i of this wave fills stage block b = i*NW + wave.
  const int8_t *src[PW];
  int stride[PW];
  const int nblocks = n / 16;
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int b = min(i * NW + wave, NB - 1);
    if (b < ABLK) {
      // A is tiled like B: block row mb is 1 KB per k-step, contiguous over k.
      const int mb = min(m0 / 16 + b, (m + 15) / 16 - 1);
      src[i] = q + (size_t)mb * kt_count * kFragBytes + lane * 16;
      stride[i] = kFragBytes;
    } else {
      const int nb = min(n0 / 16 + (b - ABLK), nblocks - 1);
      src[i] = wpack + (size_t)nb * kt_count * kFragBytes + lane * 16;
      stride[i] = kFragBytes;
    }
  }

  hb_i32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = hb_i32x4{0, 0, 0, 0};

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < kt_count) dma_stage<PW, NW, NB>(lds + (s % S) * STAGE, src, stride, s, wave, lane);
  for (int kt = 0; kt < kt_count; ++kt) {
    if (PW == PW_LO || wave < NB % NW)
      wait_stage<PW, S - 2>(kt_count - 1 - kt);
    else
      wait_stage<PW_LO, S - 2>(kt_count - 1 - kt);
    block_barrier();
    if (kt + S - 1 < kt_count)
      dma_stage<PW, NW, NB>(lds + ((kt + S - 1) % S) * STAGE, src, stride, kt + S - 1, wave, lane);
    const int8_t *base = lds + (kt % S) * STAGE;
    const int8_t *la = base + (wm * FM) * kFragBytes + lane * 16;
    const int8_t *lb = base + (ABLK + wn * FN) * kFragBytes + lane * 16;
    hb_i32x4 bf[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *(const hb_i32x4 *)(lb + j * kFragBytes);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const hb_i32x4 af = *(const hb_i32x4 *)(la + i * kFragBytes);
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue.  The lane holds rows 4*(lane/16)+r, column lane%16 of each
  // 16x16 accumulator block.  Each 16-row chunk of the wave tile is finished
  // in registers, staged in a wave-private padded LDS area, and written back
  // as 16-byte vectors running along the output rows.
  // All per-row and per-column parameters are requested together so the
  // epilogue pays one global-load latency, not one per 16-row chunk.
  const int row0 = m0 + wm * WTM;
  const int col0 = n0 + wn * WTN;
  int32_t cc[FN];
  float sc[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = min(col0 + j * 16 + (lane & 15), n - 1);
    cc[j] = corr[col];
    sc[j] = sw[col];
  }
  float sv[FM][4];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sv[i][r] = EPI == HB_W8A8_EPI_RAW ? 0.0f : scales[min(row0 + i * 16 + (lane >> 4) * 4 + r, m - 1)];
  block_barrier();  // every wave is done with the operand stages: LDS becomes staging
  constexpr int SROW = WTN + 4;  // padded staging row (32-bit words): row groups hit different banks
  static_assert(16 * SROW * 4 * NW <= S * STAGE, "staging must fit in the operand LDS");
  uint32_t *stg = (uint32_t *)lds + wave * 16 * SROW;
  constexpr int VPR = WTN / 4;  // 16-byte vectors per staged row
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        stg[((lane >> 4) * 4 + r) * SROW + j * 16 + (lane & 15)] =
            epilogue_bits<EPI>(acc[i][j][r], cc[j], sc[j], sv[i][r]);
#pragma unroll
    for (int v = lane; v < 16 * VPR; v += 64) {
      const int r = v / VPR, c4 = v % VPR;
      const int row = row0 + i * 16 + r, col = col0 + c4 * 4;
      if (row < m && col < n) {
        const hb_u32x4 val = *(const hb_u32x4 *)(stg + r * SROW + c4 * 4);
        __builtin_nontemporal_store(val, (hb_u32x4 *)((uint32_t *)y + (size_t)row * ldy + col));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming tiled GEMM (persistent): one workgroup per CU walks its share of
// BM x BN output tiles with one continuous operand ring, so the next tile's
// first k-steps are in flight while a tile finishes.
//
// Two kinds of waves, because a wave's loads and stores complete in issue
// order for its s_waitcnt count: a wave that has issued output stores cannot
// wait for a later DMA stage without also waiting for those stores.
//  - ND DMA waves issue every operand DMA (global_load_lds, 1 KB lane-ordered
//    blocks) and the tile parameters, wait for their own DMA only, and publish
//    each stage with the workgroup barrier.  They keep S - 3 stages in flight
//    while the compute waves work on the stage before, and do little else:
//    the scalar unit is shared by every wave of the CU.
//  - WM x WN compute waves never load from global memory.  Each step they
//    read the next step's fragments from LDS while the current step's MFMAs
//    run.  Operands are swapped in the MFMA (weights as src0), so a lane holds
//    4 consecutive output columns of one row.  Accumulators start at the
//    tile's column corrections.  At a tile's end the compute waves scale in
//    registers and store straight from the MFMA layout (16 rows x 64 bytes per
//    store; the two stores of a 32-column pair fill whole 128-byte lines),
//    without waiting: the stores drain during the next tile's main loop.  The
//    epilogue is VALU and LDS work on the waves that issue the MFMAs, so it
//    reads each parameter once (no LDS regroup, no per-piece re-reads).  The
//    stores are non-temporal, so the output does not evict the operands the
//    other CUs of the XCD still read from L2.
//  - The epilogue parameters of a tile (corr and sw of its BN columns, the row
//    scales of its BM rows) arrive in LDS by DMA with the tile's first k-step,
//    double-buffered by tile parity: DMA waves 0.. load corr then sw, one
//    kilobyte each (16 bytes per lane; two waves for 192-column tiles), DMA
//    wave d loads rows 64d..64d+63 of the scales (4 bytes per lane, rows past
//    m clamped).
//  - Stores are buffer stores bounded by the tile's valid rows; columns past
//    n get an out-of-range offset.
//  - The XCD that runs a workgroup (blockIdx % 8) owns a contiguous chunk of
//    the tiles in 4-row-block groups; its workgroups take consecutive tiles of
//    the chunk, so the A and B blocks they share stay in that XCD's L2.
// Requires gridDim.x % 8 == 0 and kp / 64 >= S - 1 (a tile's parameter
// buffer is rewritten only after the tile two before it has finished).
// ---------------------------------------------------------------------------

__device__ inline void grouped_tile(int p, int tiles_m, int tiles_n, int &tm, int &tn) {
  constexpr int G = 4;
  const int first_m = (p / (G * tiles_n)) * G;
  const int gsize = min(tiles_m - first_m, G);
  const int in_group = p % (G * tiles_n);
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// Operand and parameter DMA of the streaming kernel's DMA wave d (of ND):
// one stage per issue(), in step order across the workgroup's tiles.  TAG
// (the kernel's epilogue) gives each kernel instantiation its own type:
// hipcc's host pass drops the launch stub of a second kernel that shares
// this device-only type with another.
template <int BM, int BN, int ND, bool SCALES, int TAG>
struct StreamDma {
  static constexpr int ABLK = BM / 16, BBLK = BN / 16, NB = ABLK + BBLK, PW = NB / ND;
  // instruction i of wave d fills block i * ND + d: activation blocks for i < ABLK / ND
  // a tile's parameter buffer: [corr | sw] (BN*8 bytes in PCS one-kilobyte
  // chunks, the last one padded), then the BM row scales at PSC
  static constexpr int PCS = (BN * 8 + kFragBytes - 1) / kFragBytes, PSC = PCS * kFragBytes;
  static_assert(NB % ND == 0 && ABLK % ND == 0 && (!SCALES || BM / 64 <= ND) && PCS <= ND, "DMA split");
  uint32_t soff[PW];        // byte offset of each block's k-step 0 in its operand (uniform)
  const int8_t *pcs, *psc;  // this wave's corr|sw chunk (waves below PCS) and scale rows
  int tile, kt, slot;

  // Points the DMA at tile (tm, tn): operand blocks (clamped into A and B)
  // and this wave's parameter blocks.
  __device__ void point(int tm, int tn, const int8_t *q, const int8_t *wpack, const float *scales, const float *sw,
                        const int32_t *corr, int m, int n, int ktc, int d, int lane) {
    const int mblocks = (m + 15) / 16, nblocks = n / 16;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int b = i * ND + d;
      const int blk = i < ABLK / ND ? min(tm * ABLK + b, mblocks - 1) : min(tn * BBLK + (b - ABLK), nblocks - 1);
      soff[i] = (uint32_t)blk * (uint32_t)ktc * (uint32_t)kFragBytes;
    }
    // 16-byte piece c = 64d + lane of [corr | sw]: corr of columns 4c..4c+3
    // for c < BN/4, then sw; pieces past BN/2 (padding) repeat the last sw
    // piece.  n % 16 == 0, so a group of 4 columns lies wholly inside or
    // wholly past n (then clamped).
    const int c = min(64 * d + lane, BN / 2 - 1);
    const int col = min(tn * BN + 4 * (c < BN / 4 ? c : c - BN / 4), n - 4);
    pcs = c < BN / 4 ? (const int8_t *)(corr + col) : (const int8_t *)(sw + col);
    psc = SCALES ? (const int8_t *)(scales + min(tm * BM + 64 * d + lane, m - 1)) : nullptr;
  }

  // Issues the DMA of the next stage into ring slot `slot` (and, at a tile's
  // first k-step, the tile's parameters into buffer tile & 1).  Operand
  // blocks are buffer loads (ra: activations, rb: packed weights) whose block
  // offset is scalar and whose lane offset is one constant register, so the
  // issue costs no vector instructions on the SIMDs the MFMAs run on.
  __device__ void issue(int8_t *lds, int stage_bytes, int8_t *params, int pbuf, int ktc, int S, int d,
                        __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, uint32_t l16) {
    int8_t *dst = lds + slot * stage_bytes;
#pragma unroll
    for (int i = 0; i < PW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(i < ABLK / ND ? ra : rb, HB_LDS_PTR(dst + (i * ND + d) * kFragBytes), 16,
                                               l16, soff[i] + (uint32_t)kt * (uint32_t)kFragBytes, 0, 0);
    if (kt == 0) {
      int8_t *pb = params + (tile & 1) * pbuf;
      if (d < PCS) __builtin_amdgcn_global_load_lds(pcs, HB_LDS_PTR(pb + d * kFragBytes), 16, 0, 0);
      if (SCALES && d < BM / 64) __builtin_amdgcn_global_load_lds(psc, HB_LDS_PTR(pb + PSC + d * 256), 4, 0, 0);
    }
    if (++kt == ktc) kt = 0;
    if (++slot == S) slot = 0;
  }
};

__device__ inline __amdgpu_buffer_rsrc_t stream_out_rsrc(void *y, int ldy, int row0, int rows) {
  return __builtin_amdgcn_make_buffer_rsrc((uint32_t *)y + (size_t)row0 * ldy, 0,
                                           (uint32_t)rows * (uint32_t)ldy * 4u, 0x00020000);
}

template <int BM, int BN, int WM, int WN, int ND, int S, int EPI>
__global__ __launch_bounds__(64 * (WM * WN + ND), 1) void w8a8_gemm_stream(void *__restrict__ y, int ldy,
                                                                          const int8_t *__restrict__ q,
                                                                          const float *__restrict__ scales,
                                                                          const int8_t *__restrict__ wpack,
                                                                          const float *__restrict__ sw,
                                                                          const int32_t *__restrict__ corr, int m,
                                                                          int n, int kp, int tiles_m, int tiles_n,
                                                                          int stagger) {
  constexpr int NW = WM * WN;  // compute waves 0..NW-1; DMA waves NW..NW+ND-1
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int ABLK = BM / 16;
  constexpr int NB = ABLK + BN / 16;
  constexpr int STAGE = NB * kFragBytes;
  // parameters per tile: [corr | sw] (BN*8 bytes, padded to whole kilobytes), then the row scales
  static_assert(BM * 4 == kFragBytes, "one kilobyte of row scales");
  constexpr bool SCALES = EPI != HB_W8A8_EPI_RAW;
  constexpr int PSC = StreamDma<BM, BN, ND, SCALES, EPI>::PSC;
  constexpr int PBUF = PSC + kFragBytes;
#ifndef HB_STREAM_SPLIT
#define HB_STREAM_SPLIT 2
#endif
  // row blocks of a step multiplied before the step's barrier
  constexpr int SPLIT = HB_STREAM_SPLIT < FM ? HB_STREAM_SPLIT : FM;
  static_assert(FN % 2 == 0, "column blocks in pairs (32 columns, one 128-byte line)");
  using Dma = StreamDma<BM, BN, ND, SCALES, EPI>;
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE + 2 * PBUF];
  int8_t *params = lds + S * STAGE;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int ktc = kp / kKStep;

  // This workgroup's tiles: chunk [c0, c1) of the grouped order belongs to its XCD.
  const int total = tiles_m * tiles_n;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8, nslots = gridDim.x / 8;
  const int per = (total + 7) / 8;
  const int c0 = min(total, xcd * per), c1 = min(total, c0 + per);
  const int ntile = c0 + slot < c1 ? (c1 - c0 - slot + nslots - 1) / nslots : 0;
  if (ntile == 0) return;
  const int steps = ntile * ktc;
  // Workgroups of odd slot start `stagger` ticks of the 100 MHz real-time
  // counter late, so their tile ends, and the output store bursts that
  // follow, fall between those of the even slots.
  if (stagger > 0 && (slot & 1)) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < (uint64_t)stagger) __builtin_amdgcn_s_sleep(8);
  }

  if (wave >= NW) {
    // --------------------------------- DMA wave ---------------------------------
    // Stage g + 1 has landed once at most (S - 3) * PW of this wave's DMA
    // instructions are outstanding, while the S - 3 stages after it have
    // been issued: each has at least PW instructions (a tile's first stage
    // has the parameter DMA besides), so the count waits for stage g + 1 and
    // possibly a parameter load after it.  With fewer stages left: vmcnt(0).
    const int d = wave - NW;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)q, 0, (uint32_t)((m + 15) / 16) * (uint32_t)kp * 16u, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void *)wpack, 0, (uint32_t)n * (uint32_t)kp,
                                                                        0x00020000);
    Dma dma;
    dma.tile = -1;
    dma.kt = 0;
    dma.slot = 0;
#define STREAM_ISSUE()                                                                 \
  do {                                                                                 \
    if (dma.kt == 0) {                                                                 \
      int tm_, tn_;                                                                    \
      grouped_tile(c0 + slot + (++dma.tile) * nslots, tiles_m, tiles_n, tm_, tn_);     \
      dma.point(tm_, tn_, q, wpack, scales, sw, corr, m, n, ktc, d, lane);             \
    }                                                                                  \
    dma.issue(lds, STAGE, params, PBUF, ktc, S, d, ra, rb, (uint32_t)lane * 16u);      \
  } while (0)
    static_assert(S >= 4, "at least one stage in flight behind the awaited one");
    for (int st = 0; st < S - 1 && st < steps; ++st) STREAM_ISSUE();
    if (S - 1 <= steps) wait_vmcnt<(S - 2) * Dma::PW>(); else wait_vmcnt<0>();
    block_barrier();  // stage 0 published
    for (int g = 0; g < steps; ++g) {
      if (g + S - 2 < steps) wait_vmcnt<(S - 3) * Dma::PW>();
      else if (g + 1 < steps) wait_vmcnt<0>();
      block_barrier();  // stage g + 1 published; every compute wave is done with stage g - 1
      if (g + S - 1 < steps) STREAM_ISSUE();  // into the slot stage g - 1 held
    }
#undef STREAM_ISSUE
    return;
  }

  // ------------------------------- compute wave -------------------------------
  const int wm = wave / WN, wn = wave % WN;
  // A lane of the MFMA layout holds output row lane%16 and columns
  // 4*(lane/16)..+3 of each 16x16 block.  The accumulators of a tile start at
  // its column corrections (corr), so the epilogue has no correction to add
  // (32-bit wrapping sums: the same bits as adding it at the end).
  hb_i32x4 acc[FM][FN];
  hb_i32x4 fa[2][FM], fb[2][FN];
  const int aoff = (wm * FM) * kFragBytes + lane * 16, boff = (ABLK + wn * FN) * kFragBytes + lane * 16;
  const int lcol = wn * WTN + 4 * (lane >> 4);  // tile column of this lane in block 0
  const int scol = 16 * ((lane >> 3) & 1) + 4 * (lane >> 4);  // column in a 32-column pair after the DPP trade
  block_barrier();  // stage 0 (and tile 0's parameters) published
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const hb_i32x4 cc = *(const hb_i32x4 *)(params + (lcol + j * 16) * 4);
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[i][j] = cc;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = *(const hb_i32x4 *)(lds + aoff + i * kFragBytes);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[0][j] = *(const hb_i32x4 *)(lds + boff + j * kFragBytes);
  int r = 0, kt = 0, rd_slot = 1 % S;  // tile and k-step of the step; slot of the next fragments

  // One step g with fragments fa[P]/fb[P]; the next step's go to fa[1-P]/fb[1-P].
#define STREAM_MFMA(P, I0, I1)                                                                               \
  _Pragma("unroll") for (int i = (I0); i < (I1); ++i) _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = \
      __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[P][j], fa[P][i], acc[i][j], 0, 0, 0);
#define STREAM_STEP(P)                                                                                       \
  {                                                                                                          \
                                                                                                             \
    STREAM_MFMA(P, 0, SPLIT)                                                                                 \
    __builtin_amdgcn_sched_barrier(0);                                                                       \
    block_barrier();                                                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                                       \
    {                                                                                                        \
      /* unconditional (after the last step it reads a stale slot, unused): a branch here */                 \
      /* would make the compiler wait for these reads before the MFMAs below */                              \
      const int8_t *base = lds + rd_slot * STAGE;                                                            \
      if (++rd_slot == S) rd_slot = 0;                                                                       \
      _Pragma("unroll") for (int i = 0; i < FM; ++i) fa[1 - (P)][i] =                                        \
          *(const hb_i32x4 *)(base + aoff + i * kFragBytes);                                                 \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) fb[1 - (P)][j] =                                        \
          *(const hb_i32x4 *)(base + boff + j * kFragBytes);                                                 \
    }                                                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                                       \
    STREAM_MFMA(P, SPLIT, FM)                                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                                       \
    if (++kt == ktc) {                                                                                       \
      /* epilogue of tile r: parameters from LDS (they arrived with its first stage); each lane */            \
      /* stores its 4 columns of a row, 16 rows x 64 bytes per store, whole 128-byte lines per */             \
      /* column-block pair */                                                                                 \
      int tm, tn;                                                                                            \
      grouped_tile(c0 + slot + r * nslots, tiles_m, tiles_n, tm, tn);                                        \
      const int8_t *par = params + (r & 1) * PBUF;                                                           \
      const __amdgpu_buffer_rsrc_t rsrc = stream_out_rsrc(y, ldy, tm * BM, min(BM, m - tm * BM));            \
      float sv[FM];                                                                                          \
      _Pragma("unroll") for (int i = 0; i < FM; ++i) sv[i] =                                                 \
          SCALES ? *(const float *)(par + PSC + (wm * WTM + i * 16 + (lane & 15)) * 4) : 0.0f;               \
      /* each 16-row x 32-column piece leaves in two stores of 8 whole 128-byte lines: the upper */         \
      /* 8 lanes of every 16-lane row trade their block-0 values for block 1 of the lanes 8 below */        \
      /* (DPP), so a lane then holds row lane%8 (+8 in the second store) of the piece, columns */             \
      /* 16*(lane/8%2) + 4*(lane/16)..+3 of the pair */                                                      \
      _Pragma("unroll") for (int jp = 0; jp < FN / 2; ++jp) {                                                \
        const hb_f32x4 sc0 = *(const hb_f32x4 *)(par + BN * 4 + (lcol + jp * 32) * 4);                      \
        const hb_f32x4 sc1 = *(const hb_f32x4 *)(par + BN * 4 + (lcol + jp * 32 + 16) * 4);                 \
        const int pc = tn * BN + wn * WTN + jp * 32 + scol;                                                  \
        _Pragma("unroll") for (int i = 0; i < FM; ++i) {                                                     \
          hb_u32x4 o0, o1, lo, hi;                                                                           \
          _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                                    \
            o0[e] = epilogue_bits<EPI>(acc[i][2 * jp][e], 0, sc0[e], sv[i]);                                 \
            o1[e] = epilogue_bits<EPI>(acc[i][2 * jp + 1][e], 0, sc1[e], sv[i]);                             \
          }                                                                                                  \
          _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                                    \
            lo[e] = (uint32_t)__builtin_amdgcn_update_dpp((int)o0[e], (int)o1[e], kDppRowShr8, 0xf, 0xc, false); \
            hi[e] = (uint32_t)__builtin_amdgcn_update_dpp((int)o1[e], (int)o0[e], kDppRowShl8, 0xf, 0x3, false); \
          }                                                                                                  \
          const uint32_t r0 = (uint32_t)(wm * WTM + i * 16 + (lane & 7));                                    \
          const uint32_t off0 = pc < n ? (r0 * (uint32_t)ldy + (uint32_t)pc) * 4u : 0xfffffff0u;             \
          const uint32_t off1 = pc < n ? ((r0 + 8u) * (uint32_t)ldy + (uint32_t)pc) * 4u : 0xfffffff0u;      \
          __builtin_amdgcn_raw_buffer_store_b128(lo, rsrc, off0, 0, 2);                                      \
          __builtin_amdgcn_raw_buffer_store_b128(hi, rsrc, off1, 0, 2);                                      \
        }                                                                                                    \
      }                                                                                                      \
      /* the next tile's accumulators start at its corrections (its parameters arrived with the */           \
      /* stage published at this step's barrier; after the last tile they are unused) */                      \
      const int8_t *npar = params + ((r + 1) & 1) * PBUF;                                                    \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) {                                                       \
        const hb_i32x4 cc = *(const hb_i32x4 *)(npar + (lcol + j * 16) * 4);                                 \
        _Pragma("unroll") for (int i = 0; i < FM; ++i) acc[i][j] = cc;                                       \
      }                                                                                                      \
      kt = 0;                                                                                                \
      ++r;                                                                                                   \
    }                                                                                                        \
  }

  for (int g = 0; g < steps; g += 2) {
    STREAM_STEP(0)
    if (g + 1 < steps) STREAM_STEP(1)
  }
#undef STREAM_STEP
#undef STREAM_MFMA
}

// ---------------------------------------------------------------------------
// Small-M (decode) GEMM, m <= 16: one workgroup per 16-column block streams
// that block's packed weights once; WAVES waves split K, each keeping U
// one-kilobyte weight loads in flight.  Integer partial sums are combined in
// LDS, so the result is independent of the split.
// ---------------------------------------------------------------------------

template <int WAVES, int U, int EPI>
__global__ __launch_bounds__(64 * WAVES) void w8a8_gemm_decode(void *__restrict__ y, int ldy,
                                                               const int8_t *__restrict__ q,
                                                               const float *__restrict__ scales,
                                                               const int8_t *__restrict__ wpack,
                                                               const float *__restrict__ sw,
                                                               const int32_t *__restrict__ corr, int m, int n,
                                                               int kp, int rtiles) {
  __shared__ hb_i32x4 part[WAVES][64];
  // blockIdx.x -> (column block, 16-row tile).  With several row tiles, the
  // tiles of one column block go to one XCD (workgroups are handed to the 8
  // XCDs in turn) one after another, so they share that XCD's L2 copy of the
  // block's weights; the grid covers the column blocks rounded up to 8.
  int nb = blockIdx.x, rtile = 0;
  if (rtiles > 1) {
    const int slot = blockIdx.x / 8;
    nb = (slot / rtiles) * 8 + blockIdx.x % 8;
    rtile = slot % rtiles;
    if (nb >= n / 16) return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kt_count = kp / kKStep;
  const int8_t *wb = wpack + (size_t)nb * kt_count * kFragBytes + lane * 16;
  const int row0 = rtile * 16;
  const int arow = lane & 15;
  const bool has_row = row0 + arow < m;
  // tiled A: row tile rtile, lane-ordered 1 KB per k-step
  const int8_t *qa = q + (size_t)rtile * kt_count * kFragBytes + lane * 16;
  // Epilogue parameters are requested before the weight stream so their
  // latency is hidden behind it.
  const int col = nb * 16 + (lane & 15);
  const int32_t cc = corr[col];
  const float sc = sw[col];
  float sv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    sv[r] = EPI == HB_W8A8_EPI_RAW ? 0.0f : scales[min(row0 + (lane >> 4) * 4 + r, m - 1)];

  hb_i32x4 acc = {0, 0, 0, 0};
  for (int kt0 = wave * U; kt0 < kt_count; kt0 += WAVES * U) {
    hb_i32x4 b[U], a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = kt0 + u;
      const bool ok = kt < kt_count;
      b[u] = ok ? *(const hb_i32x4 *)(wb + (size_t)kt * kFragBytes) : hb_i32x4{0, 0, 0, 0};
      a[u] = (ok && has_row) ? *(const hb_i32x4 *)(qa + (size_t)kt * kFragBytes) : hb_i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u], acc, 0, 0, 0);
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  hb_i32x4 total = part[0][lane];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) {
    const hb_i32x4 p = part[w][lane];
    total = hb_i32x4{(int)((uint32_t)total[0] + (uint32_t)p[0]), (int)((uint32_t)total[1] + (uint32_t)p[1]),
                     (int)((uint32_t)total[2] + (uint32_t)p[2]), (int)((uint32_t)total[3] + (uint32_t)p[3])};
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = row0 + (lane >> 4) * 4 + r;
    if (row < m) store_result<EPI>(y, ldy, row, col, total[r], cc, sc, sv[r]);
  }
}

// ---------------------------------------------------------------------------
// Single-row decode with the quantization fused in (m == 1).  One workgroup
// per 16-column block.  Each workgroup first requests the activation row and
// the smoothing vector, then every packed weight tile of its block (wave w
// owns tiles [w*VW, w*VW + VW), held in registers), so the row's
// quantization runs while the weight stream is in flight; the quantized row
// goes to LDS in the A-operand order and the tiles are consumed by MFMA.
// The arithmetic is the quantization kernels' and the decode GEMM's, step for
// step, so results are identical to the two-kernel path.
// ---------------------------------------------------------------------------

template <int WAVES, int BPW, int VW, int MINW, bool BUF, int EPI>
__global__ __launch_bounds__(64 * WAVES, MINW) void w8a8_decode_fused(void *__restrict__ y, const float *__restrict__ x,
                                                                  const float *__restrict__ inv,
                                                                  const int8_t *__restrict__ wpack,
                                                                  const float *__restrict__ sw,
                                                                  const int32_t *__restrict__ corr, int k, int kp,
                                                                  int nblocks) {
  constexpr int T = 64 * WAVES;
  constexpr int WPB = WAVES / BPW;               // waves per column block
  static_assert(WPB * BPW == WAVES, "blocks must split the waves evenly");
  constexpr int VX = (VW + 4 * BPW - 1) / (4 * BPW);  // float4 of the row per thread: VX * 4 * T >= VW * WPB * 64
  __shared__ __attribute__((aligned(16))) int8_t qs[VW * WPB * kKStep];  // [kt][k/16 group][16 bytes]
  __shared__ float red[WAVES];
  __shared__ int32_t part[WAVES][16];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, tid = threadIdx.x;
  const int wib = wave % WPB;  // wave within its column block: tiles [wib*VW, wib*VW + VW)
  const int nb_raw = blockIdx.x * BPW + wave / WPB;
  const int nb = min(nb_raw, nblocks - 1);  // a missing last block repeats the previous one and stores nothing
  const int kc = kp / kKStep, nvec = k / 4;
  // 1. activation row, smoothing vector, column parameters and this wave's
  //    weight tiles are all requested before any of them is used.
  float4 a[VX], iv[VX];
  hb_i32x4 b[VW];
  const int col = nb * 16 + (lane & 15);
  const int32_t cc = corr[col];
  const float sc = sw[col];
  if constexpr (BUF) {
    // Buffer loads: one 32-bit offset register per stream; reads past the
    // row or past the weight image return zeros, tiles past the block's kc
    // are fetched but never multiplied (unconditional loads keep every
    // request in flight before the first wait).
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (uint32_t)nvec * 16u, 0x00020000);
    const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc((void *)inv, 0, (uint32_t)nvec * 16u, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)wpack, 0, (uint32_t)nblocks * (uint32_t)kc * kFragBytes, 0x00020000);
#pragma unroll
    for (int j = 0; j < VX; ++j) {
      const uint32_t off = (uint32_t)(tid + T * j) * 16u;
      const hb_u32x4 xv = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
      const hb_u32x4 iw = __builtin_amdgcn_raw_buffer_load_b128(ri, off, 0, 0);
      a[j] = make_float4(__uint_as_float(xv[0]), __uint_as_float(xv[1]), __uint_as_float(xv[2]), __uint_as_float(xv[3]));
      iv[j] = make_float4(__uint_as_float(iw[0]), __uint_as_float(iw[1]), __uint_as_float(iw[2]), __uint_as_float(iw[3]));
    }
    // every wave's row requests enter the memory pipeline before any weight
    // request (no wait for them): otherwise a late wave's share of the row
    // queues behind the other waves' weight tiles and holds up the
    // quantization, which needs the whole row.  Long rows (more than two
    // float4 per thread) are a large part of a workgroup's bytes: there the
    // weight stream is not held back for them.
    if constexpr (VX <= 2) {
      __builtin_amdgcn_sched_barrier(0);
      block_barrier();
    }
    const uint32_t wv = ((uint32_t)nb * (uint32_t)kc + (uint32_t)(wib * VW)) * kFragBytes + (uint32_t)lane * 16u;
#pragma unroll
    for (int i = 0; i < VW; ++i) {
      const hb_u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw, wv + i * kFragBytes, 0, 2);
      b[i] = hb_i32x4{(int)t[0], (int)t[1], (int)t[2], (int)t[3]};
    }
  } else {
    // Clamped pointer loads (weight images of 4 GiB and more): the extra
    // loads repeat the block's last tile and are never multiplied.
#pragma unroll
    for (int j = 0; j < VX; ++j) {
      const int v = min(tid + T * j, nvec - 1);
      a[j] = ((const float4 *)x)[v];
      iv[j] = ((const float4 *)inv)[v];
    }
    if constexpr (VX <= 2) {
      __builtin_amdgcn_sched_barrier(0);
      block_barrier();  // the row before the weights, as above
    }
    const int8_t *wb = wpack + (size_t)nb * kc * kFragBytes + lane * 16;
#pragma unroll
    for (int i = 0; i < VW; ++i)
      b[i] = __builtin_nontemporal_load((const hb_i32x4 *)(wb + (size_t)min(wib * VW + i, kc - 1) * kFragBytes));
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. row absmax of t = x * inv, then the quantized row into LDS
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    a[j] = make_float4(__fmul_rn(a[j].x, iv[j].x), __fmul_rn(a[j].y, iv[j].y), __fmul_rn(a[j].z, iv[j].z),
                       __fmul_rn(a[j].w, iv[j].w));
    if (tid + T * j < nvec)
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a[j].x), fabsf(a[j].y)), fmaxf(fabsf(a[j].z), fabsf(a[j].w))));
  }
  amax = wave_max(amax);
  if (lane == 0) red[wave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) amax = fmaxf(amax, red[w]);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
  const float r = __fdiv_rn(1.0f, s);
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    const int v = tid + T * j;
    if (v < kp / 4) {
      const uint32_t word = v < nvec ? (quantize_byte(a[j].x, r) | (quantize_byte(a[j].y, r) << 8) |
                                        (quantize_byte(a[j].z, r) << 16) | (quantize_byte(a[j].w, r) << 24))
                                     : 0u;
      *(uint32_t *)(qs + 4 * v) = word;  // byte k at k: [kt][group][16] is k's natural order for one row
    }
  }
  __syncthreads();
  // 3. MFMA: lanes of row 0 (lane % 16 == 0) carry the row, the others zeros;
  //    row 0 of the product lands in element 0 of lanes 0..15.
  const bool has_row = (lane & 15) == 0;
  hb_i32x4 acc = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const int kt = wib * VW + i;
    if (kt < kc) {
      const hb_i32x4 av = has_row ? *(const hb_i32x4 *)(qs + kt * kKStep + (lane >> 4) * 16) : hb_i32x4{0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[i], acc, 0, 0, 0);
    }
  }
  if (lane < 16) part[wave][lane] = acc[0];
  __syncthreads();
  if (wib != 0 || lane >= 16 || nb_raw >= nblocks) return;
  int32_t tot = part[wave][lane];
#pragma unroll
  for (int w = 1; w < WPB; ++w) tot = (int32_t)((uint32_t)tot + (uint32_t)part[wave + w][lane]);
  __builtin_nontemporal_store(epilogue_bits<EPI>(tot, cc, sc, s), (uint32_t *)y + col);
}

// ---------------------------------------------------------------------------
// Few-row GEMM on quantized rows (2 <= m <= 16, k <= 4096) in the shape of
// the one-row kernel: 16 waves, two 16-column blocks per workgroup, each
// wave's 8 weight tiles requested up front with buffer loads.  The A tiles
// (rows 0-15 of the quantized activations, 1 KB per k-step) are read once
// per workgroup into LDS, requested before the weights so waiting for them
// does not wait for the weight stream; rows past m are zeroed at the MFMA.
// ---------------------------------------------------------------------------

template <int EPI>
__global__ __launch_bounds__(1024) void w8a8_decode_q(void *__restrict__ y, int ldy, const int8_t *__restrict__ q,
                                                      const float *__restrict__ scales,
                                                      const int8_t *__restrict__ wpack,
                                                      const float *__restrict__ sw,
                                                      const int32_t *__restrict__ corr, int m, int kp, int nblocks) {
  constexpr int WAVES = 16, WPB = 8, VW = 8, KT = VW * WPB;  // k-steps served: 64 (k <= 4096)
  __shared__ __attribute__((aligned(16))) int8_t qs[KT * kFragBytes];  // reused for the wave sums
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wib = wave % WPB;
  const int nb_raw = blockIdx.x * 2 + wave / WPB;
  const int nb = min(nb_raw, nblocks - 1);
  const int kc = kp / kKStep;
  const int col = nb * 16 + (lane & 15);
  const int32_t cc = corr[col];
  const float sc = sw[col];
  float sv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) sv[r] = EPI == HB_W8A8_EPI_RAW ? 0.0f : scales[min((lane >> 4) * 4 + r, m - 1)];
  // 1. A tiles: wave w loads k-steps w, w+16, w+32, w+48 (past kc: zeros)
  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc((void *)q, 0, (uint32_t)kc * kFragBytes, 0x00020000);
  hb_u32x4 av[KT / WAVES];
#pragma unroll
  for (int j = 0; j < KT / WAVES; ++j)
    av[j] = __builtin_amdgcn_raw_buffer_load_b128(rq, (uint32_t)(wave + WAVES * j) * kFragBytes + lane * 16u, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  // 2. this wave's weight tiles (reads past the image return zeros; tiles
  //    past kc are fetched, never multiplied)
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void *)wpack, 0, (uint32_t)nblocks * (uint32_t)kc * kFragBytes, 0x00020000);
  const uint32_t wv = ((uint32_t)nb * (uint32_t)kc + (uint32_t)(wib * VW)) * kFragBytes + (uint32_t)lane * 16u;
  hb_i32x4 b[VW];
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const hb_u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw, wv + i * kFragBytes, 0, 2);
    b[i] = hb_i32x4{(int)t[0], (int)t[1], (int)t[2], (int)t[3]};
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < KT / WAVES; ++j) *(hb_u32x4 *)(qs + (wave + WAVES * j) * kFragBytes + lane * 16) = av[j];
  __syncthreads();
  // 3. MFMA: lane l carries A row l % 16 (zero past m)
  const bool has_row = (lane & 15) < m;
  hb_i32x4 acc = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const int kt = wib * VW + i;
    if (kt < kc) {
      const hb_i32x4 a = has_row ? *(const hb_i32x4 *)(qs + kt * kFragBytes + lane * 16) : hb_i32x4{0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[i], acc, 0, 0, 0);
    }
  }
  __syncthreads();  // every wave is done reading qs
  hb_i32x4 *part = (hb_i32x4 *)qs;  // [WAVES][64]
  part[wave * 64 + lane] = acc;
  __syncthreads();
  if (wib != 0 || nb_raw >= nblocks) return;
  hb_i32x4 total = part[wave * 64 + lane];
#pragma unroll
  for (int w = 1; w < WPB; ++w) {
    const hb_i32x4 p = part[(wave + w) * 64 + lane];
    total = hb_i32x4{(int)((uint32_t)total[0] + (uint32_t)p[0]), (int)((uint32_t)total[1] + (uint32_t)p[1]),
                     (int)((uint32_t)total[2] + (uint32_t)p[2]), (int)((uint32_t)total[3] + (uint32_t)p[3])};
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = (lane >> 4) * 4 + r;
    if (row < m) store_result<EPI>(y, ldy, row, col, total[r], cc, sc, sv[r]);
  }
}

// ---------------------------------------------------------------------------
// Single-row decode balanced over the CUs (m == 1, k <= 2048).  Workgroup g
// owns the 8-column half blocks [g*H, g*H + H) with H <= 7, which touch at
// most four 16-column blocks; with one workgroup per CU every CU streams the
// same number of weight bytes (n = 14336 on 256 CUs: 3.5 blocks each, where
// whole blocks per workgroup leave the busiest CU with 4).  Four waves per
// touched block split its k-tiles.  A lane whose half block lies outside the
// range gets an out-of-range buffer offset, so its loads return zeros without
// a memory request, and it stores nothing.  Quantization and arithmetic are
// those of w8a8_decode_fused, so results are identical.
// ---------------------------------------------------------------------------

template <int VW, int EPI>
__global__ __launch_bounds__(1024) void w8a8_decode_even(void *__restrict__ y, const float *__restrict__ x,
                                                         const float *__restrict__ inv,
                                                         const int8_t *__restrict__ wpack,
                                                         const float *__restrict__ sw,
                                                         const int32_t *__restrict__ corr, int k, int kp,
                                                         int nblocks, int hpw) {
  constexpr int WAVES = 16, SLOTS = 4, WPS = WAVES / SLOTS;
  constexpr int KQ = VW * WPS * kKStep;  // the longest row served
  static_assert(KQ <= 4 * 64 * WAVES, "one float4 of the row per thread");
  __shared__ __attribute__((aligned(16))) int8_t qs[KQ];
  __shared__ float red[WAVES];
  __shared__ int32_t part[WAVES][16];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, tid = threadIdx.x;
  const int slot = wave / WPS, wis = wave % WPS;
  const int h0 = blockIdx.x * hpw, h1 = min(h0 + hpw, 2 * nblocks);
  const int nb_raw = h0 / 2 + slot;
  const int nb = min(nb_raw, nblocks - 1);
  const int half = 2 * nb_raw + ((lane & 15) >> 3);  // this lane's column's half block
  const bool mine = half >= h0 && half < h1;         // implies nb_raw < nblocks
  const int kc = kp / kKStep, nvec = k / 4;
  const int col = nb * 16 + (lane & 15);
  const int32_t cc = corr[col];
  const float sc = sw[col];
  // 1. the row, the smoothing vector and this wave's weight tiles, all
  //    requested before any is used (tiles past kc are fetched, never used)
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (uint32_t)nvec * 16u, 0x00020000);
  const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc((void *)inv, 0, (uint32_t)nvec * 16u, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void *)wpack, 0, (uint32_t)nblocks * (uint32_t)kc * kFragBytes, 0x00020000);
  const hb_u32x4 xv = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)tid * 16u, 0, 0);
  const hb_u32x4 iw = __builtin_amdgcn_raw_buffer_load_b128(ri, (uint32_t)tid * 16u, 0, 0);
  // every wave's row requests ahead of all weight requests (as in w8a8_decode_fused)
  __builtin_amdgcn_sched_barrier(0);
  block_barrier();
  const uint32_t wv =
      mine ? ((uint32_t)nb * (uint32_t)kc + (uint32_t)(wis * VW)) * kFragBytes + (uint32_t)lane * 16u : 0x80000000u;
  hb_i32x4 b[VW];
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const hb_u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw, wv + i * kFragBytes, 0, 2);
    b[i] = hb_i32x4{(int)t[0], (int)t[1], (int)t[2], (int)t[3]};
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. row absmax of t = x * inv, then the quantized row into LDS
  const float4 a = make_float4(__fmul_rn(__uint_as_float(xv[0]), __uint_as_float(iw[0])),
                               __fmul_rn(__uint_as_float(xv[1]), __uint_as_float(iw[1])),
                               __fmul_rn(__uint_as_float(xv[2]), __uint_as_float(iw[2])),
                               __fmul_rn(__uint_as_float(xv[3]), __uint_as_float(iw[3])));
  float amax = tid < nvec ? fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))) : 0.0f;
  amax = wave_max(amax);
  if (lane == 0) red[wave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) amax = fmaxf(amax, red[w]);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
  const float r = __fdiv_rn(1.0f, s);
  if (tid < kp / 4) {
    const uint32_t word = tid < nvec ? (quantize_byte(a.x, r) | (quantize_byte(a.y, r) << 8) |
                                        (quantize_byte(a.z, r) << 16) | (quantize_byte(a.w, r) << 24))
                                     : 0u;
    *(uint32_t *)(qs + 4 * tid) = word;
  }
  __syncthreads();
  // 3. MFMA: lanes of row 0 (lane % 16 == 0) carry the row, the others zeros
  const bool has_row = (lane & 15) == 0;
  hb_i32x4 acc = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const int kt = wis * VW + i;
    if (kt < kc) {
      const hb_i32x4 av = has_row ? *(const hb_i32x4 *)(qs + kt * kKStep + (lane >> 4) * 16) : hb_i32x4{0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[i], acc, 0, 0, 0);
    }
  }
  if (lane < 16) part[wave][lane] = acc[0];
  __syncthreads();
  if (wis != 0 || lane >= 16 || !mine) return;
  int32_t tot = part[wave][lane];
#pragma unroll
  for (int w = 1; w < WPS; ++w) tot = (int32_t)((uint32_t)tot + (uint32_t)part[wave + w][lane]);
  __builtin_nontemporal_store(epilogue_bits<EPI>(tot, cc, sc, s), (uint32_t *)y + col);
}

// ---------------------------------------------------------------------------
// A few rows (2 <= m <= R <= 4, k <= 4096) with the quantization fused in:
// the 16-wave, two-block shape of w8a8_decode_fused.  Every workgroup
// quantizes all m rows itself (one workgroup reduction for all rows) before
// it streams its weight tiles; rows of the MFMA A operand past m are zero.
// ---------------------------------------------------------------------------

template <int R, int EPI>
__global__ __launch_bounds__(1024, 8) void w8a8_decode_rows(void *__restrict__ y, int ldy, const float *__restrict__ x,
                                                         const float *__restrict__ inv,
                                                         const int8_t *__restrict__ wpack,
                                                         const float *__restrict__ sw,
                                                         const int32_t *__restrict__ corr, int m, int k, int kp,
                                                         int nblocks) {
  constexpr int WAVES = 16, BPW = 2, VW = 8;
  constexpr int WPB = WAVES / BPW;
  constexpr int KQ = VW * WPB * kKStep;  // the longest row served (4096)
  static_assert(R >= 2 && R <= 4, "two to four rows");
  __shared__ __attribute__((aligned(16))) int8_t qs[R][KQ];
  __shared__ float red[R][WAVES];
  __shared__ float srow[R];
  __shared__ int32_t part[WAVES][R][16];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, tid = threadIdx.x;
  const int wib = wave % WPB;
  const int nb_raw = blockIdx.x * BPW + wave / WPB;
  const int nb = min(nb_raw, nblocks - 1);
  const int kc = kp / kKStep, nvec = k / 4;
  const int col = nb * 16 + (lane & 15);
  const int32_t cc = corr[col];
  const float sc = sw[col];
  // 1. the rows and the smoothing vector (a resource covering m rows; offsets
  //    past a row's end are pushed out of range and read as zeros)
  const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc((void *)inv, 0, (uint32_t)nvec * 16u, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (uint32_t)m * (uint32_t)nvec * 16u, 0x00020000);
  const bool in_row = tid < nvec;
  const hb_u32x4 ivb = __builtin_amdgcn_raw_buffer_load_b128(ri, (uint32_t)tid * 16u, 0, 0);
  hb_u32x4 xv[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    xv[r] = __builtin_amdgcn_raw_buffer_load_b128(
        rx, in_row ? ((uint32_t)r * (uint32_t)nvec + (uint32_t)tid) * 16u : 0x80000000u, 0, 0);
  // 2. every row's absmax in one workgroup reduction, then the rows quantized
  //    into LDS -- before the weight stream, whose registers it would compete
  //    for (a load issued after the weights could only be waited for behind them)
  float4 t[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    t[r] = make_float4(__fmul_rn(__uint_as_float(xv[r][0]), __uint_as_float(ivb[0])),
                       __fmul_rn(__uint_as_float(xv[r][1]), __uint_as_float(ivb[1])),
                       __fmul_rn(__uint_as_float(xv[r][2]), __uint_as_float(ivb[2])),
                       __fmul_rn(__uint_as_float(xv[r][3]), __uint_as_float(ivb[3])));
    float amax = in_row ? fmaxf(fmaxf(fabsf(t[r].x), fabsf(t[r].y)), fmaxf(fabsf(t[r].z), fabsf(t[r].w))) : 0.0f;
    amax = wave_max(amax);
    if (lane == 0) red[r][wave] = amax;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float a = red[r][0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) a = fmaxf(a, red[r][w]);
    const float sr = fmaxf(__fdiv_rn(a, 127.0f), 1e-12f);
    const float rcp = __fdiv_rn(1.0f, sr);
    if (tid == 0) srow[r] = sr;
    if (tid < kp / 4) {
      const uint32_t word = in_row ? (quantize_byte(t[r].x, rcp) | (quantize_byte(t[r].y, rcp) << 8) |
                                      (quantize_byte(t[r].z, rcp) << 16) | (quantize_byte(t[r].w, rcp) << 24))
                                   : 0u;
      *(uint32_t *)(&qs[r][4 * tid]) = word;
    }
  }
  // 3. the weight tiles (reads past the image return zeros and are never used)
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void *)wpack, 0, (uint32_t)nblocks * (uint32_t)kc * kFragBytes, 0x00020000);
  const uint32_t wv = ((uint32_t)nb * (uint32_t)kc + (uint32_t)(wib * VW)) * kFragBytes + (uint32_t)lane * 16u;
  hb_i32x4 b[VW];
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const hb_u32x4 tb = __builtin_amdgcn_raw_buffer_load_b128(rw, wv + i * kFragBytes, 0, 2);
    b[i] = hb_i32x4{(int)tb[0], (int)tb[1], (int)tb[2], (int)tb[3]};
  }
  __syncthreads();  // qs and srow complete
  // MFMA: lane l carries row l % 16 of the A operand (zero past R)
  const int arow = lane & 15;
  hb_i32x4 acc = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const int kt = wib * VW + i;
    if (kt < kc) {
      const hb_i32x4 av = arow < R ? *(const hb_i32x4 *)(&qs[arow][kt * kKStep + (lane >> 4) * 16])
                                   : hb_i32x4{0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[i], acc, 0, 0, 0);
    }
  }
  // element rr of lane l is row 4*(l/16) + rr, column l % 16
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int row = 4 * (lane >> 4) + rr;
    if (row < R) part[wave][row][lane & 15] = acc[rr];
  }
  __syncthreads();
  if (wib != 0 || nb_raw >= nblocks) return;
  for (int idx = lane; idx < R * 16; idx += 64) {
    const int row = idx / 16;  // idx % 16 == lane % 16: this lane's column
    if (row >= m) continue;
    int32_t tot = part[wave][row][lane & 15];
#pragma unroll
    for (int w = 1; w < WPB; ++w) tot = (int32_t)((uint32_t)tot + (uint32_t)part[wave + w][row][lane & 15]);
    __builtin_nontemporal_store(epilogue_bits<EPI>(tot, cc, sc, srow[row]),
                                (uint32_t *)y + (size_t)row * (size_t)ldy + col);
  }
}

// ---------------------------------------------------------------------------
// Small problems (m <= 128, k <= 1536) in one launch: a 16-wave workgroup per
// 16 rows x 16*CF columns quantizes its 16 rows itself (one wave per row,
// exactly the quantization kernels' arithmetic) into LDS, then multiplies the
// whole K with every wave's weight tiles requested up front, adds the waves'
// int32 sums in LDS and applies the epilogue.  The weights are the MFMA A
// operand, so a lane ends with 4 consecutive columns of one row and stores
// them as one 16-byte vector.
// ---------------------------------------------------------------------------

template <int CF, int KPW, int VX, int EPI>
__global__ __launch_bounds__(1024) void w8a8_small(void *__restrict__ y, const float *__restrict__ x,
                                                   const float *__restrict__ inv, const int8_t *__restrict__ wpack,
                                                   const float *__restrict__ sw, const int32_t *__restrict__ corr,
                                                   int m, int k, int n, int kp) {
  constexpr int WAVES = 16;
  __shared__ __attribute__((aligned(16))) int8_t qs[16][VX * 256];
  __shared__ float srow[16];
  __shared__ hb_i32x4 red[WAVES][CF][64];
  const int rt = blockIdx.x, g = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kc = kp / kKStep, nvec = k / 4;
  // 1. this wave's row (clamped; rows past m are quantized but never stored)
  const int qrow = min(rt * 16 + wave, m - 1);
  const float4 *xr = (const float4 *)(x + (size_t)qrow * k);
  float4 a[VX], iv[VX];
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    const int v = min(lane + 64 * j, nvec - 1);
    a[j] = xr[v];
    iv[j] = ((const float4 *)inv)[v];
  }
  // 2. the weight tiles of this wave's k-blocks (clamped; past kc never used)
  const int kb0 = wave * KPW;
  hb_i32x4 b[KPW][CF];
#pragma unroll
  for (int t = 0; t < KPW; ++t)
#pragma unroll
    for (int j = 0; j < CF; ++j)
      b[t][j] = __builtin_nontemporal_load(
          (const hb_i32x4 *)(wpack + ((size_t)(g * CF + j) * kc + min(kb0 + t, kc - 1)) * kFragBytes + lane * 16));
  // 3. quantize the row into LDS
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    a[j] = make_float4(__fmul_rn(a[j].x, iv[j].x), __fmul_rn(a[j].y, iv[j].y), __fmul_rn(a[j].z, iv[j].z),
                       __fmul_rn(a[j].w, iv[j].w));
    if (lane + 64 * j < nvec)
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a[j].x), fabsf(a[j].y)), fmaxf(fabsf(a[j].z), fabsf(a[j].w))));
  }
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
  const float r = __fdiv_rn(1.0f, s);
  if (lane == 0) srow[wave] = s;
#pragma unroll
  for (int j = 0; j < VX; ++j) {
    const int v = lane + 64 * j;
    if (v < kp / 4) {
      const uint32_t word = v < nvec ? (quantize_byte(a[j].x, r) | (quantize_byte(a[j].y, r) << 8) |
                                        (quantize_byte(a[j].z, r) << 16) | (quantize_byte(a[j].w, r) << 24))
                                     : 0u;
      *(uint32_t *)(&qs[wave][4 * v]) = word;
    }
  }
  __syncthreads();
  // 4. MFMA over this wave's k-blocks: weights as A (16 columns), rows as B
  hb_i32x4 acc[CF];
#pragma unroll
  for (int j = 0; j < CF; ++j) acc[j] = hb_i32x4{0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < KPW; ++t) {
    const int kt = kb0 + t;
    if (kt < kc) {
      const hb_i32x4 av = *(const hb_i32x4 *)(&qs[lane & 15][kt * kKStep + (lane >> 4) * 16]);
#pragma unroll
      for (int j = 0; j < CF; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[t][j], av, acc[j], 0, 0, 0);
    }
  }
#pragma unroll
  for (int j = 0; j < CF; ++j) red[wave][j][lane] = acc[j];
  __syncthreads();
  // 5. wave j < CF finishes column fragment j: lane l has row l % 16, columns
  //    4*(l/16) .. +3
  const int row = rt * 16 + (lane & 15);
  if (wave >= CF || row >= m) return;
  const int j = wave;
  hb_i32x4 tot = red[0][j][lane];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) {
    const hb_i32x4 p = red[w][j][lane];
    tot = hb_i32x4{(int)((uint32_t)tot[0] + (uint32_t)p[0]), (int)((uint32_t)tot[1] + (uint32_t)p[1]),
                   (int)((uint32_t)tot[2] + (uint32_t)p[2]), (int)((uint32_t)tot[3] + (uint32_t)p[3])};
  }
  const int col = (g * CF + j) * 16 + 4 * (lane >> 4);
  const float sv = srow[lane & 15];
  hb_u32x4 out;
#pragma unroll
  for (int q = 0; q < 4; ++q) out[q] = epilogue_bits<EPI>(tot[q], corr[col + q], sw[col + q], sv);
  __builtin_nontemporal_store(out, (hb_u32x4 *)((uint32_t *)y + (size_t)row * n + col));
}

// ---------------------------------------------------------------------------
// The GEMM epilogue as its own pass (profile mode 2): raw = sum_k u*W (the
// HB_W8A8_EPI_RAW output), c = raw - wsum128 + delta = raw - 128*sums
// (wrapping, the bits the fused kernels start their accumulators from), then
// epilogue_bits, so the values equal the fused epilogue's.  Four columns per
// thread, grid-stride over the m x n/4 quads.
// ---------------------------------------------------------------------------

template <int EPI>
__global__ __launch_bounds__(256) void w8a8_readout(float *__restrict__ y, int ldy, const int32_t *__restrict__ raw,
                                                    const float *__restrict__ scales, const float *__restrict__ sw,
                                                    const int32_t *__restrict__ delta,
                                                    const int32_t *__restrict__ wsum, int m, int n) {
  const int nq = n / 4;
  const size_t quads = (size_t)m * (size_t)nq;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < quads; i += (size_t)gridDim.x * 256) {
    const int row = (int)(i / nq), c0 = (int)(i % nq) * 4;
    const hb_i32x4 a = *(const hb_i32x4 *)(raw + (size_t)row * n + c0);
    const hb_i32x4 d = *(const hb_i32x4 *)(delta + c0), w = *(const hb_i32x4 *)(wsum + c0);
    const hb_f32x4 sc = *(const hb_f32x4 *)(sw + c0);
    const float s = scales[row];
    hb_u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = epilogue_bits<EPI>((int32_t)((uint32_t)a[e] - (uint32_t)w[e]), d[e], sc[e], s);
    __builtin_nontemporal_store(o, (hb_u32x4 *)(y + (size_t)row * ldy + c0));
  }
}

// ---------------------------------------------------------------------------
// Raw accumulator -> byte-plane export of the CPU-control variant.
// One thread per output byte position (row, 32-column half, byte in 128).
// ---------------------------------------------------------------------------

// Split-K GEMM for up to 256 rows: grid (tiles, splits), split s multiplies
// k-steps [s*kps, s*kps + kps) of its BM x BN tile with the tiled kernel's
// k loop and stores the plain int32 sums (no column correction) to slice s
// of the workspace ([mp][n] per slice; rows past m dropped by the buffer
// bound).  w8a8_splitk_readout adds the slices and applies the epilogue;
// 32-bit wrapping sums are exact in any order, so the result equals the
// one-pass GEMM bit for bit.
template <int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(64 * WM *WN) void w8a8_splitk_partial(int32_t *__restrict__ ws,
                                                                  const int8_t *__restrict__ q,
                                                                  const int8_t *__restrict__ wpack, int m, int n,
                                                                  int kp, int kps) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int ABLK = BM / 16, BBLK = BN / 16;
  constexpr int NB = ABLK + BBLK;
  constexpr int PW = (NB + NW - 1) / NW;
  constexpr int PW_LO = NB / NW;
  static_assert(PW_LO >= 1 && PW == PW_LO, "every wave issues the same DMA count");
  constexpr int STAGE = NB * kFragBytes;
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE];

  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
  int tm, tn;
  tile_coords_2d<BM, BN>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kt_count = kp / kKStep;
  const int kt0 = blockIdx.y * kps, steps = min(kps, kt_count - kt0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;
  const int8_t *src[PW];
  int stride[PW];
  const int nblocks = n / 16;
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int b = i * NW + wave;
    if (b < ABLK) {
      const int mb = min(m0 / 16 + b, (m + 15) / 16 - 1);
      src[i] = q + (size_t)mb * kt_count * kFragBytes + lane * 16;
    } else {
      const int nb = min(n0 / 16 + (b - ABLK), nblocks - 1);
      src[i] = wpack + (size_t)nb * kt_count * kFragBytes + lane * 16;
    }
    stride[i] = kFragBytes;
  }
  hb_i32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = hb_i32x4{0, 0, 0, 0};
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < steps) dma_stage<PW, NW, NB>(lds + (st % S) * STAGE, src, stride, kt0 + st, wave, lane);
  for (int kt = 0; kt < steps; ++kt) {
    wait_stage<PW, S - 2>(steps - 1 - kt);
    block_barrier();
    if (kt + S - 1 < steps)
      dma_stage<PW, NW, NB>(lds + ((kt + S - 1) % S) * STAGE, src, stride, kt0 + kt + S - 1, wave, lane);
    const int8_t *base = lds + (kt % S) * STAGE;
    const int8_t *la = base + (wm * FM) * kFragBytes + lane * 16;
    const int8_t *lb = base + (ABLK + wn * FN) * kFragBytes + lane * 16;
    hb_i32x4 bf[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *(const hb_i32x4 *)(lb + j * kFragBytes);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const hb_i32x4 af = *(const hb_i32x4 *)(la + i * kFragBytes);
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[j], acc[i][j], 0, 0, 0);
    }
  }
  // lane l holds rows 4*(l/16)+r, column l%16 of each 16x16 block
  const int mp = (m + 15) / 16 * 16;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(ws + (size_t)blockIdx.y * mp * n, 0,
                                                                      (uint32_t)m * (uint32_t)n * 4u, 0x00020000);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn * WTN + j * 16 + (lane & 15);
      if (col >= n) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * WTM + i * 16 + 4 * (lane >> 4) + r;
        __builtin_amdgcn_raw_buffer_store_b32((uint32_t)acc[i][j][r], rs, (uint32_t)(row * n + col) * 4u, 0, 0);
      }
    }
}

// The split-K slices added in slice order (32-bit wrapping), then the GEMM
// epilogue: corr is delta (scaled epilogues) or wsum128 (raw sums).  Four
// outputs per thread, 16-byte loads and stores.
template <int EPI>
__global__ __launch_bounds__(256) void w8a8_splitk_readout(void *__restrict__ y, int ldy,
                                                          const int32_t *__restrict__ part, int splits,
                                                          const float *__restrict__ scales,
                                                          const float *__restrict__ sw,
                                                          const int32_t *__restrict__ corr, int m, int n) {
  const size_t quads = (size_t)m * (size_t)(n / 4);
  const size_t slice = (size_t)((m + 15) / 16 * 16) * (size_t)n;
  for (size_t qd = (size_t)blockIdx.x * blockDim.x + threadIdx.x; qd < quads; qd += (size_t)gridDim.x * blockDim.x) {
    const int row = (int)(qd / (size_t)(n / 4)), col = (int)(qd % (size_t)(n / 4)) * 4;
    const int32_t *p = part + (size_t)row * n + col;
    hb_u32x4 sum = *(const hb_u32x4 *)p;
    for (int t = 1; t < splits; ++t) sum += *(const hb_u32x4 *)(p + (size_t)t * slice);
    const hb_i32x4 c = *(const hb_i32x4 *)(corr + col);
    const hb_f32x4 w = *(const hb_f32x4 *)(sw + col);
    const float sr = EPI == HB_W8A8_EPI_RAW ? 0.0f : scales[row];
    hb_u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = epilogue_bits<EPI>((int32_t)sum[e], c[e], w[e], sr);
    __builtin_nontemporal_store(o, (hb_u32x4 *)((uint32_t *)y + (size_t)row * ldy + col));
  }
}

__global__ __launch_bounds__(256) void w8a8_planes(uint8_t *__restrict__ out, const int32_t *__restrict__ raw, int m,
                                                  int n) {
  const size_t total = (size_t)m * (size_t)n * 4u;
  for (size_t pos = (size_t)blockIdx.x * blockDim.x + threadIdx.x; pos < total;
       pos += (size_t)gridDim.x * blockDim.x) {
    const size_t row = pos / ((size_t)n * 4u);
    const int byte_in_row = (int)(pos % ((size_t)n * 4u));
    const int n0 = (byte_in_row / 128) * 32;
    const int within = byte_in_row % 128;
    const int tile = (int)(row / 64u);
    const int rows = m - tile * 64 < 64 ? m - tile * 64 : 64;
    const size_t flat = (row - (size_t)tile * 64u) * 128u + (size_t)within;
    const int p = (int)(flat / ((size_t)rows * 32u));
    const size_t rem = flat % ((size_t)rows * 32u);
    const int r = (int)(rem / 32u), c = (int)(rem % 32u);
    const uint32_t v = (uint32_t)raw[(size_t)(tile * 64 + r) * n + n0 + c];
    out[pos] = (uint8_t)(v >> (8 * p));
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------

// Candidate tile shapes in order of preference when the cost model ties;
// occ = workgroups resident per CU (LDS / register bound).  Two resident
// workgroups let one's epilogue stores overlap the other's MFMA loop, which
// is why 128x192 leads (measured at 4096x1536x6144: 128x192 57 us,
// 128x128 62 us, 256x192 64 us, 256x256 73 us).
// eff = measured MAC throughput of a full round of that shape relative to
// 128x192 (LDS traffic per MAC grows as tiles shrink; 64x64 is an estimate);
// it carries the effect of occupancy, which the cost model (tiles on the
// busiest CU x tile work / eff) does not count separately.
struct TileShape {
  int bm, bn, occ, eff;
};
constexpr TileShape kTileShapes[] = {
    {128, 192, 2, 100}, {256, 192, 1, 90}, {128, 128, 2, 92}, {256, 256, 1, 100}, {64, 64, 4, 60}};
constexpr int kNumShapes = 5;
// Index kNumShapes selects the streaming kernel (w8a8_gemm_stream, 256 x 128
// tiles, one persistent workgroup per CU); index kNumShapes + 1 its 256 x 192
// form (5 stages of 28 KB), for shapes whose 192-column tiles fill whole
// rounds of CUs.  The GELU epilogue keeps the 128-column form (the wider one
// runs out of registers there).
constexpr int kStreamShape = kNumShapes, kStreamWideShape = kNumShapes + 1;
constexpr int kStreamBM = 256, kStreamBN = 128, kStreamStages = 6;
constexpr int kStreamWideBN = 192, kStreamWideStages = 5;

// -1: automatic.  Set by hb_w8a8_force_tile; HTP_OPS_AMD_W8A8_TILE gives
// the initial value.
std::atomic<int> g_forced_tile{-2};

int forced_tile_shape() {
  int forced = g_forced_tile.load(std::memory_order_relaxed);
  if (forced == -2) {
    const char *v = getenv("HTP_OPS_AMD_W8A8_TILE");
    forced = (v && *v) ? atoi(v) : -1;
    if (forced < -1 || forced > kStreamWideShape) forced = -1;
    int expected = -2;
    if (!g_forced_tile.compare_exchange_strong(expected, forced)) forced = expected;
  }
  return forced;
}

int compute_units() {
  static std::atomic<int> cus{0};
  int v = cus.load(std::memory_order_relaxed);
  if (v == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cus.store(v, std::memory_order_relaxed);
  }
  return v;
}

// Picks the kernel for m > 16.  The streaming kernel keeps one workgroup per
// CU for the whole launch, so it runs outright where its tiles spread evenly
// over the CUs: the 256x192 form where its tiles fill whole rounds, the
// 256x128 form where they fill whole rounds or one round of at least half of
// the CUs (fewer tiles leave most CUs idle).  Otherwise every candidate is
// costed as (tiles on the busiest CU) x (work per tile) / (relative
// efficiency), the streaming forms with efficiency 110 where their tiles
// occupy at least half of the CUs; ties go to the earlier tiled entry.
// Measured (GEMM alone, us, automatic / best forced, one box) on the shapes
// this rule changed: 256x1536x4608 13.65 -> 7.40 (64x64 tiles instead of 36
// streaming tiles), 512x4096x4096 24.4 -> 16.2, 1024x6144x1536 33.1 -> 19.9,
// 256x4096x14336 25.5 -> 23.0, 512x1536x6144 14.3 -> 11.5, 1024x4096x14336
// 69.2 -> 59.6 (streaming instead of 256x256 tiles, 1.75 rounds),
// 2048x4096x14336 136 -> 119, 2048x1536x4608 21.3 -> 19.8.
// The streaming kernel needs kp / 64 >= kStreamStages - 1 (its parameter
// double buffer).
bool stream_applies(int kp) { return kp / kKStep >= kStreamStages - 1; }
bool stream_wide_applies(int n, int kp) { return n % kStreamWideBN == 0 && kp / kKStep >= kStreamWideStages - 1; }
int stream_mode() {
  static const int mode = getenv("HTP_OPS_AMD_W8A8_STREAM") ? atoi(getenv("HTP_OPS_AMD_W8A8_STREAM")) : -1;
  return mode;
}

int pick_tile_shape(int m, int n, int kp) {
  const int forced = forced_tile_shape();
  if (forced == kStreamWideShape && stream_wide_applies(n, kp)) return kStreamWideShape;
  if (forced == kStreamShape && stream_applies(kp)) return kStreamShape;
  if (forced >= 0 && forced < kNumShapes && (kTileShapes[forced].bn != 192 || n % 192 == 0)) return forced;
  const long long cus = compute_units();
  const long long stream_tiles = (long long)((m + kStreamBM - 1) / kStreamBM) * ((n + kStreamBN - 1) / kStreamBN);
  const long long wide_tiles =
      (long long)((m + kStreamBM - 1) / kStreamBM) * ((n + kStreamWideBN - 1) / kStreamWideBN);
  const bool stream_ok = stream_mode() != 0 && stream_applies(kp) && (stream_mode() == 1 || 2 * stream_tiles >= cus);
  const bool wide_ok = stream_mode() != 0 && stream_wide_applies(n, kp) && 2 * wide_tiles >= cus;
  if (wide_ok && wide_tiles >= cus && wide_tiles % cus == 0) return kStreamWideShape;
  if (stream_ok && (stream_mode() == 1 || stream_tiles <= cus || stream_tiles % cus == 0)) return kStreamShape;
  int best = 0;
  long long best_cost = -1;
  for (int i = 0; i < kNumShapes + 2; ++i) {
    int bm, bn, eff;
    if (i < kNumShapes) {
      bm = kTileShapes[i].bm, bn = kTileShapes[i].bn, eff = kTileShapes[i].eff;
      if (bn == 192 && n % 192 != 0) continue;
    } else if (i == kStreamShape) {
      if (!stream_ok) continue;
      bm = kStreamBM, bn = kStreamBN, eff = 110;
    } else {
      if (!wide_ok) continue;
      bm = kStreamBM, bn = kStreamWideBN, eff = 110;
    }
    const long long tiles = (long long)((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    const long long cost = (tiles + cus - 1) / cus * bm * bn * 100 / eff;
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = i;
    }
  }
  return best;
}

// Start delay (ticks of the 100 MHz real-time counter) of the streaming
// kernel's odd-slot workgroups.  With two or more tiles per workgroup the
// delayed half reaches its tile ends while the other half multiplies, so the
// two halves' output store bursts no longer share the HBM write bandwidth.
// Measured (GEMM alone, us, one box; delay 0 / best):
//   256x192 tiles: 4096x1536x6144 (2 rounds) 46.9 / 42.7 at 5 us,
//   4096x2048x6144 54.7 / 51.3, 8192x1536x3072 46.9 / 42.6,
//   4096x1536x12288 (4 rounds) 90.5 / 81.5;
//   256x128 tiles: 4096x1536x4096 (2 rounds) 31.6 / 30.1 at 4 us;
// with one round every delay only adds (2048x4096x6144 43.7 -> 44.3 at 5 us,
// 2048x4096x4096 32.3 -> 33.5) and the 3-round GELU case gains under 1 us.
// HTP_OPS_AMD_W8A8_STAGGER=ticks overrides the choice (measurement hook).
int stream_stagger(int tiles, int grid, int bn) {
  const char *env = getenv("HTP_OPS_AMD_W8A8_STAGGER");
  if (env && *env && atoi(env) >= 0) return atoi(env);
  const int rounds = tiles % grid == 0 ? tiles / grid : 0;
  if (bn == kStreamWideBN) return rounds >= 2 ? 500 : 0;
  return rounds == 2 ? 400 : 0;
}

template <int EPI>
int launch_tiles(void *y, int ldy, const int8_t *q, const float *scales, const int8_t *wpack, const float *sw,
                 const int32_t *corr, int m, int n, int kp, hipStream_t st) {
  int shape = pick_tile_shape(m, n, kp);
  if (shape == kStreamWideShape) {
    if constexpr (EPI == HB_W8A8_EPI_SCALE_GELU) {
      shape = stream_applies(kp) ? kStreamShape : 0;
    } else {
      const int tiles_m = (m + kStreamBM - 1) / kStreamBM, tiles_n = (n + kStreamWideBN - 1) / kStreamWideBN;
      const int tiles = tiles_m * tiles_n;
      const int grid = std::min(compute_units(), (tiles + 7) / 8 * 8) / 8 * 8;
      if (grid < 8) return hb_invalid("w8a8_gemm_stream grid");
      hipLaunchKernelGGL((w8a8_gemm_stream<kStreamBM, kStreamWideBN, 4, 2, 4, kStreamWideStages, EPI>), dim3(grid),
                         dim3(768), 0, st, y, ldy, q, scales, wpack, sw, corr, m, n, kp, tiles_m, tiles_n,
                         stream_stagger(tiles, grid, kStreamWideBN));
      return hb_check_launch("w8a8_gemm_stream");
    }
  }
  if (shape == kStreamShape) {
    const int tiles_m = (m + kStreamBM - 1) / kStreamBM, tiles_n = (n + kStreamBN - 1) / kStreamBN;
    const int tiles = tiles_m * tiles_n;
    const int grid = std::min(compute_units(), (tiles + 7) / 8 * 8) / 8 * 8;
    if (grid < 8) return hb_invalid("w8a8_gemm_stream grid");
    hipLaunchKernelGGL((w8a8_gemm_stream<kStreamBM, kStreamBN, 4, 2, 4, kStreamStages, EPI>), dim3(grid), dim3(768),
                       0, st, y, ldy, q, scales, wpack, sw, corr, m, n, kp, tiles_m, tiles_n,
                       stream_stagger(tiles, grid, kStreamBN));
    return hb_check_launch("w8a8_gemm_stream");
  }
  const TileShape t = kTileShapes[shape];
  const int grid = ((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
  switch (shape) {
    case 0:
      hipLaunchKernelGGL((w8a8_gemm_tiles<128, 192, 2, 2, 4, EPI>), dim3(grid), dim3(256), 0, st, y, ldy, q, scales,
                         wpack, sw, corr, m, n, kp);
      break;
    case 1:
      hipLaunchKernelGGL((w8a8_gemm_tiles<256, 192, 2, 2, 4, EPI>), dim3(grid), dim3(256), 0, st, y, ldy, q, scales,
                         wpack, sw, corr, m, n, kp);
      break;
    case 2:
      hipLaunchKernelGGL((w8a8_gemm_tiles<128, 128, 2, 2, 4, EPI>), dim3(grid), dim3(256), 0, st, y, ldy, q, scales,
                         wpack, sw, corr, m, n, kp);
      break;
    case 3:
      hipLaunchKernelGGL((w8a8_gemm_tiles<256, 256, 2, 2, 4, EPI>), dim3(grid), dim3(256), 0, st, y, ldy, q, scales,
                         wpack, sw, corr, m, n, kp);
      break;
    default:
      hipLaunchKernelGGL((w8a8_gemm_tiles<64, 64, 2, 2, 4, EPI>), dim3(grid), dim3(256), 0, st, y, ldy, q, scales,
                         wpack, sw, corr, m, n, kp);
      break;
  }
  return hb_check_launch("w8a8_gemm_tiles");
}

template <int EPI>
int launch_decode(void *y, int ldy, const int8_t *q, const float *scales, const int8_t *wpack, const float *sw,
                  const int32_t *corr, int m, int n, int kp, hipStream_t st) {
  // Size the workgroup so every wave is resident in a single round
  // (about 16 waves per CU) with 8 one-kilobyte loads in flight each.
  const int nblocks = n / 16;
  // k <= 4096 with at least 3.5 column blocks per CU: two blocks per 16-wave
  // workgroup (16 x 4096 x 14336: 17.6 -> 15.1 us for the op).  With fewer
  // blocks its workgroups leave CUs idle (16 x 4096 x 4096: 7.7 -> 9.0 us).
  if (kp <= 64 * kKStep && 2 * nblocks >= 7 * compute_units()) {
    hipLaunchKernelGGL((w8a8_decode_q<EPI>), dim3((nblocks + 1) / 2), dim3(1024), 0, st, y, ldy, q, scales, wpack,
                       sw, corr, m, kp, nblocks);
  } else if (nblocks >= 512) {
    hipLaunchKernelGGL((w8a8_gemm_decode<4, 8, EPI>), dim3(nblocks), dim3(256), 0, st, y, ldy, q, scales, wpack, sw,
                       corr, m, n, kp, 1);
  } else if (nblocks >= 128) {
    hipLaunchKernelGGL((w8a8_gemm_decode<16, 8, EPI>), dim3(nblocks), dim3(1024), 0, st, y, ldy, q, scales, wpack,
                       sw, corr, m, n, kp, 1);
  } else {
    hipLaunchKernelGGL((w8a8_gemm_decode<16, 4, EPI>), dim3(nblocks), dim3(1024), 0, st, y, ldy, q, scales, wpack,
                       sw, corr, m, n, kp, 1);
  }
  return hb_check_launch("w8a8_gemm_decode");
}

template <int EPI>
int launch_gemm(void *y, int ldy, const int8_t *q, const float *scales, const int8_t *wpack, const float *sw,
                const int32_t *corr, int m, int n, int kp, hipStream_t st) {
  if (m <= 16) return launch_decode<EPI>(y, ldy, q, scales, wpack, sw, corr, m, n, kp, st);
  // 17-80 rows whose output holds at most one 64x64 tile per four CUs: the
  // decode kernel per 16-row tile and 16-column block spreads the weight
  // stream over the whole chip (op time 64 x 14336 x 4096: 53.6 -> 38.2 us;
  // 32 x 4096 x 4096: 15.6 -> 9.1; 77 x 4096 x 2048: 20.4 -> 15.2).  With
  // more row tiles the weight re-reads cost more than the tiles gain
  // (128 x 4096 x 4096: 20.6 -> 24.9 us), as with more output tiles
  // (100 x 1536 x 6144: 11.1 -> 19.4 us).
  const int rtiles = (m + 15) / 16;
  if (rtiles <= 5 && 4LL * ((m + 63) / 64) * (n / 64) <= compute_units()) {
    const int nb8 = (n / 16 + 7) / 8 * 8;
    hipLaunchKernelGGL((w8a8_gemm_decode<16, 8, EPI>), dim3(nb8 * rtiles), dim3(1024), 0, st, y, ldy, q, scales,
                       wpack, sw, corr, m, n, kp, rtiles);
    return hb_check_launch("w8a8_gemm_decode");
  }
  return launch_tiles<EPI>(y, ldy, q, scales, wpack, sw, corr, m, n, kp, st);
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Quantization runs one workgroup per row up to these row counts (rows of
// more than 2048 values up to the second): measured against the 8-row
// blocks, 77x4096 6.44 -> 3.39 us, 256x4096 7.36 -> 3.49, 512x1536 3.97 ->
// 3.27, 1024x4096 8.33 -> 6.87; the blocks lead from 1024x1536 (4.44
// against 4.60) and 2048x4096 (10.27 against 11.75).
constexpr int kWgRowsMax = 768, kWgRowsMaxLong = 1024;

template <int NV, int ROWS, int MINB = 1, bool INV_LDS = false>
void launch_quant_block(int8_t *d_q, float *d_scales, const float *d_x, const float *d_inv, int m, int k, int kp,
                        hipStream_t st) {
  const dim3 blocks((m + ROWS - 1) / ROWS), threads(64 * ROWS);
  hipLaunchKernelGGL((w8a8_quant_block<NV, ROWS, MINB, INV_LDS>), blocks, threads, (size_t)ROWS * (size_t)kp, st, d_q, d_scales, d_x,
                     d_inv, m, k, kp);
}

// Launches one configuration of w8a8_decode_fused if its waves cover kp.
template <int WAVES, int BPW, int VW, int MINW, bool BUF, int EPI>
bool launch_decode_cfg(void *y, const float *x, const float *inv, const int8_t *wpack, const float *sw,
                       const int32_t *corr, int k, int nblocks, int kp, hipStream_t st, size_t pad = 0) {
  constexpr int kCover = VW * (WAVES / BPW) * kKStep;
  if (kp > kCover) return false;
  hipLaunchKernelGGL((w8a8_decode_fused<WAVES, BPW, VW, MINW, BUF, EPI>), dim3((nblocks + BPW - 1) / BPW),
                     dim3(64 * WAVES), pad, st, y, x, inv, wpack, sw, corr, k, kp, nblocks);
  return true;
}

// Two shapes serve k <= 4096.  One column block per 8-wave workgroup (up to
// four resident per CU), or two blocks per 16-wave workgroup, which reads
// the activation row and smoothing vector once for both blocks (they are
// half as many bytes as the block's weights).  The second is used when it
// puts no more blocks on the busiest CU than the first (measured at k=4096,
// n=14336: 11.3 us against 12.0 us; n=12288: 11.1 us against 10.0 us).
template <int EPI>
int launch_decode_fused(void *y, const float *x, const float *inv, const int8_t *wpack, const float *sw,
                        const int32_t *corr, int k, int n, int kp, hipStream_t st) {
  const int nblocks = n / 16, kc = kp / kKStep, cus = compute_units();
  const bool buf = (size_t)nblocks * (size_t)kp * 16u < ((size_t)1 << 32);
  const int per_cu_one = (nblocks + cus - 1) / cus;
  const int per_cu_two = 2 * (((nblocks + 1) / 2 + cus - 1) / cus);
  bool done = false;
  // k <= 2048 with 2.5-3.5 blocks per CU: the half-block split, one
  // workgroup per CU (n = 9216, k = 2048: 6.2 against 7.5 us).  At k = 4096
  // it is slower than the shapes below (n = 14336: 11.8 against 11.4 us;
  // n = 12288: 11.2 against 10.1 us): its 16 tiles per wave take 96 VGPRs,
  // which leaves a CU one 16-wave workgroup where the shapes below keep 24-32
  // waves per CU in flight.
  const int halves = 2 * nblocks, hpw = (halves + cus - 1) / cus;
  if ((size_t)nblocks * (size_t)kp * 16u < ((size_t)1 << 31) && kc <= 32 && hpw >= 5 && hpw <= 7) {
    hipLaunchKernelGGL((w8a8_decode_even<8, EPI>), dim3((halves + hpw - 1) / hpw), dim3(1024), 0, st, y, x, inv,
                       wpack, sw, corr, k, kp, nblocks, hpw);
    return hb_check_launch("w8a8_decode_even");
  }
  if (buf && kc > 48 && nblocks >= cus && per_cu_two <= per_cu_one)
    done = launch_decode_cfg<16, 2, 8, 8, true, EPI>(y, x, inv, wpack, sw, corr, k, nblocks, kp, st);
  if (!done) done = launch_decode_cfg<8, 1, 8, 1, false, EPI>(y, x, inv, wpack, sw, corr, k, nblocks, kp, st);
  if (!done) done = launch_decode_cfg<8, 1, 16, 1, false, EPI>(y, x, inv, wpack, sw, corr, k, nblocks, kp, st);
  // 4096 < k <= 16384: 16 waves of 16 tiles rather than 8 of 32 (k = 14336,
  // n = 4096: 13.2 -> 12.9 us; k = 11008: 12.6 -> 11.7 us)
  if (!done) done = launch_decode_cfg<16, 1, 16, 1, false, EPI>(y, x, inv, wpack, sw, corr, k, nblocks, kp, st);
  if (!done) return hb_invalid("w8a8_decode_fused: k too large");
  return hb_check_launch("w8a8_decode_fused");
}

// One-launch small path (w8a8_small): 5 <= m <= 128, kp <= 1536, a weight
// image of at most 16 MB.  Column fragments per workgroup as for the F16
// small kernel: 4 while that leaves a workgroup per two CUs, 2 while one per
// CU, else 1.
template <int VX, int KPW, int EPI>
void launch_w8a8_small_v(int cf, void *y, const float *x, const float *inv, const int8_t *wpack, const float *sw,
                         const int32_t *corr, int m, int k, int n, int kp, hipStream_t st) {
  const dim3 block(1024);
  const int rt = (m + 15) / 16;
  if (cf == 4)
    hipLaunchKernelGGL((w8a8_small<4, KPW, VX, EPI>), dim3(rt, n / 64), block, 0, st, y, x, inv, wpack, sw, corr, m,
                       k, n, kp);
  else if (cf == 2)
    hipLaunchKernelGGL((w8a8_small<2, KPW, VX, EPI>), dim3(rt, n / 32), block, 0, st, y, x, inv, wpack, sw, corr, m,
                       k, n, kp);
  else
    hipLaunchKernelGGL((w8a8_small<1, KPW, VX, EPI>), dim3(rt, n / 16), block, 0, st, y, x, inv, wpack, sw, corr, m,
                       k, n, kp);
}

template <int EPI>
int launch_w8a8_small(void *y, const float *x, const float *inv, const int8_t *wpack, const float *sw,
                      const int32_t *corr, int m, int k, int n, int kp, hipStream_t st) {
  const long long rt = (m + 15) / 16;
  const int cus = compute_units();
  const int cf = (n % 64 == 0 && rt * (n / 64) >= cus / 2) ? 4 : (n % 32 == 0 && rt * (n / 32) >= cus) ? 2 : 1;
  if (kp <= 768)
    launch_w8a8_small_v<3, 1, EPI>(cf, y, x, inv, wpack, sw, corr, m, k, n, kp, st);
  else
    launch_w8a8_small_v<6, 2, EPI>(cf, y, x, inv, wpack, sw, corr, m, k, n, kp, st);
  return hb_check_launch("w8a8_small");
}

}  // namespace

extern "C" {

size_t hb_w8a8_packed_offset(int k, int n, int section) {
  if (k <= 0 || n <= 0) return 0;
  const size_t kp = kp_of(k);
  const size_t w = hb_round_up((size_t)n * kp, 256);
  const size_t vec = hb_round_up((size_t)n * 4u, 256);
  switch (section) {
    case HB_W8A8_WEIGHTS: return 0;
    case HB_W8A8_SW: return w;
    case HB_W8A8_DELTA: return w + vec;
    case HB_W8A8_WSUM128: return w + 2 * vec;
    case HB_W8A8_INV: return w + 3 * vec;
    default: return 0;
  }
}

size_t hb_w8a8_packed_bytes(int k, int n) {
  if (k <= 0 || n <= 0) return 0;
  return hb_w8a8_packed_offset(k, n, HB_W8A8_INV) + hb_round_up(kp_of(k) * 4u, 256);
}

int hb_w8a8_prepack(void *d_packed, const uint8_t *d_blob, int k, int n, hb_stream s) {
  if (d_packed == nullptr || d_blob == nullptr) return hb_invalid("hb_w8a8_prepack null pointer");
  // The blob stores weights in whole 64-column groups (reference op_executor.cc:320 requires n % 64 == 0).
  if (k < 32 || k % 32 || n < 64 || n % 64) return hb_invalid("hb_w8a8_prepack shape (k%32, n%64)");
  if (!aligned(d_blob, 4) || !aligned(d_packed, 256)) return hb_invalid("hb_w8a8_prepack alignment");
  hipStream_t st = hb_resolve_stream(s);
  const int kp = (int)kp_of(k);
  uint8_t *base = (uint8_t *)d_packed;
  const size_t slots = (size_t)n * kp / 16u;
  const int grid = (int)((slots + 255) / 256 < 65536 ? (slots + 255) / 256 : 65536);
  hipLaunchKernelGGL(w8a8_prepack_weights, dim3(grid), dim3(256), 0, st,
                     (uint4 *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WEIGHTS)), d_blob, k, n, kp);
  int rc = hb_check_launch("w8a8_prepack_weights");
  if (rc) return rc;
  hipLaunchKernelGGL(w8a8_prepack_columns, dim3(n / 64), dim3(1024), 0, st,
                     (float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_SW)),
                     (int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_DELTA)),
                     (int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WSUM128)),
                     (float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_INV)), d_blob, k, n, kp);
  return hb_check_launch("w8a8_prepack_columns");
}

size_t hb_w8a8_workspace_bytes(int m, int k) {
  if (m <= 0 || k <= 0) return 0;
  return hb_round_up(mp_of(m) * kp_of(k), 256) + hb_round_up(mp_of(m) * 4u, 256);
}

int hb_w8a8_quantize(int8_t *d_q, float *d_scales, const float *d_x, const float *d_inv, int m, int k,
                     hb_stream s) {
  if (!d_q || !d_scales || !d_x || !d_inv) return hb_invalid("hb_w8a8_quantize null pointer");
  if (m < 1 || k < 32 || k % 32) return hb_invalid("hb_w8a8_quantize shape");
  if (!aligned(d_x, 4) || !aligned(d_inv, 4) || !aligned(d_q, 16) || !aligned(d_scales, 4))
    return hb_invalid("hb_w8a8_quantize alignment");
  hipStream_t st = hb_resolve_stream(s);
  const int kp = (int)kp_of(k);
  const dim3 grid((m + 3) / 4), block(256);
  const bool vec = aligned(d_x, 16) && aligned(d_inv, 16);
  // Up to about a thousand rows, or rows longer than the block kernel holds:
  // a workgroup per row.
  if (vec && (m <= kWgRowsMax || (m <= kWgRowsMaxLong && k > 2048) || k > 256 * 24) && k <= kRowThreads * 4 * 16) {
    const dim3 rows(m), threads(kRowThreads);
    if (k <= kRowThreads * 4 * 1) {
      hipLaunchKernelGGL(w8a8_quant_rows_wg<1>, rows, threads, 0, st, d_q, d_scales, d_x, d_inv, k, kp);
    } else if (k <= kRowThreads * 4 * 2) {
      hipLaunchKernelGGL(w8a8_quant_rows_wg<2>, rows, threads, 0, st, d_q, d_scales, d_x, d_inv, k, kp);
    } else if (k <= kRowThreads * 4 * 4) {
      hipLaunchKernelGGL(w8a8_quant_rows_wg<4>, rows, threads, 0, st, d_q, d_scales, d_x, d_inv, k, kp);
    } else if (k <= kRowThreads * 4 * 8) {
      hipLaunchKernelGGL(w8a8_quant_rows_wg<8>, rows, threads, 0, st, d_q, d_scales, d_x, d_inv, k, kp);
    } else {
      hipLaunchKernelGGL(w8a8_quant_rows_wg<16>, rows, threads, 0, st, d_q, d_scales, d_x, d_inv, k, kp);
    }
  } else if (vec && k <= 256 * 24) {
    // 8-row blocks (a workgroup per 128-byte output line), 16-row blocks
    // (whole 1 KB tiles) for short rows when there are enough of them; the
    // staging buffer is ROWS x kp bytes of LDS (at most 48 KB).
    const bool whole_tiles = m >= 2048;
    if (k <= 256 * 2) {
      whole_tiles ? launch_quant_block<2, 16>(d_q, d_scales, d_x, d_inv, m, k, kp, st)
                  : launch_quant_block<2, 8>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
    } else if (k <= 256 * 4) {
      whole_tiles ? launch_quant_block<4, 16>(d_q, d_scales, d_x, d_inv, m, k, kp, st)
                  : launch_quant_block<4, 8>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
    } else if (k <= 256 * 6) {
      // from 2048 rows: 16-row blocks when they put exactly one on each CU
      // (4096 rows: 7.30 us against 7.84 for the form below), otherwise
      // 8-row blocks with the smoothing vector in LDS, two or more per CU
      // (2048 rows 6.08 -> 5.12 us, 8192 rows 14.27 -> 12.75 us at k=1536)
      if (whole_tiles && (m + 15) / 16 == compute_units())
        launch_quant_block<6, 16>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
      else if (whole_tiles)
        launch_quant_block<6, 8, 4, true>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
      else
        launch_quant_block<6, 8>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
    } else if (k <= 256 * 8) {
      launch_quant_block<8, 8>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
    } else if (k <= 256 * 12) {
      launch_quant_block<12, 8>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
    } else if (k <= 256 * 16) {
      launch_quant_block<16, 8>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
    } else {
      // rows of 4097-6144 values: the smoothing vector from LDS and 4 waves
      // per SIMD (two workgroups per CU; 4096x6144: 28.8 -> 25.0 us).  The
      // same form at 2049-4096 values measured 1 us slower than this one.
      launch_quant_block<24, 8, 4, true>(d_q, d_scales, d_x, d_inv, m, k, kp, st);
    }
  } else {
    hipLaunchKernelGGL(w8a8_quant_rows_any, grid, block, 0, st, d_q, d_scales, d_x, d_inv, m, k, kp);
  }
  return hb_check_launch("w8a8_quant_rows");
}

int hb_w8a8_gemm(void *d_y, int ldy, const int8_t *d_q, const float *d_scales, const void *d_packed, int m, int k,
                 int n, int epilogue, hb_stream s) {
  if (!d_y || !d_q || !d_packed || (epilogue != HB_W8A8_EPI_RAW && !d_scales))
    return hb_invalid("hb_w8a8_gemm null pointer");
  if (m < 1 || k < 32 || k % 32 || n < 16 || n % 16 || ldy < n || ldy % 4) return hb_invalid("hb_w8a8_gemm shape");
  // Output rows are written as 16-byte vectors.
  if (!aligned(d_y, 16) || !aligned(d_q, 16) || !aligned(d_packed, 256)) return hb_invalid("hb_w8a8_gemm alignment");
  hipStream_t st = hb_resolve_stream(s);
  const int kp = (int)kp_of(k);
  const uint8_t *base = (const uint8_t *)d_packed;
  const int8_t *wpack = (const int8_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WEIGHTS));
  const float *sw = (const float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_SW));
  const int32_t *delta = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_DELTA));
  const int32_t *wsum = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WSUM128));
  switch (epilogue) {
    case HB_W8A8_EPI_SCALE:
      return launch_gemm<HB_W8A8_EPI_SCALE>(d_y, ldy, d_q, d_scales, wpack, sw, delta, m, n, kp, st);
    case HB_W8A8_EPI_SCALE_GELU:
      return launch_gemm<HB_W8A8_EPI_SCALE_GELU>(d_y, ldy, d_q, d_scales, wpack, sw, delta, m, n, kp, st);
    case HB_W8A8_EPI_RAW:
      return launch_gemm<HB_W8A8_EPI_RAW>(d_y, ldy, d_q, d_scales, wpack, sw, wsum, m, n, kp, st);
    default: return hb_invalid("hb_w8a8_gemm epilogue");
  }
}

int hb_w8a8_gemm_choice(int m, int k, int n) {
  if (m < 1 || k < 32 || k % 32 || n < 16 || n % 16) return hb_invalid("hb_w8a8_gemm_choice shape");
  if (m <= 16) return HB_W8A8_CHOICE_DECODE;
  const int rtiles = (m + 15) / 16;
  if (rtiles <= 5 && 4LL * ((m + 63) / 64) * (n / 64) <= compute_units()) return HB_W8A8_CHOICE_DECODE_TILES;
  return pick_tile_shape(m, n, (int)kp_of(k));
}

int hb_w8a8_gemm_tile(int m, int k, int n, int *bm, int *bn) {
  const int choice = hb_w8a8_gemm_choice(m, k, n);
  if (choice == HB_E_INVAL || !bm || !bn) return HB_E_INVAL;
  if (choice == HB_W8A8_CHOICE_DECODE || choice == HB_W8A8_CHOICE_DECODE_TILES) {
    *bm = 16;  // one 16-row tile (m <= 16: all rows) per 16-column block
    *bn = 16;
  } else if (choice == kStreamShape || choice == kStreamWideShape) {
    *bm = kStreamBM;
    *bn = choice == kStreamWideShape ? kStreamWideBN : kStreamBN;
  } else {
    *bm = kTileShapes[choice].bm;
    *bn = kTileShapes[choice].bn;
  }
  return choice;
}

}  // extern "C"

namespace {

// Split-K path of hb_w8a8_linear for 33 to 256 rows with long rows and few
// 128 x 128 tiles: slices of the K loop on more CUs, their int32 sums in the
// workspace after q and the scales (at most kMaxW8a8Splits slices), then
// w8a8_splitk_readout.  It pays where the K loop is long: from 128 k-steps
// (K 8192), or 80 with more than 128 rows (77x10240x4096 38.0 -> 22.8 us,
// 128x10240x4096 39.1 -> 25.7, 256x10240x4096 41.5 -> 30.8, 256x5120x1280
// 19.7 -> 16.2); at 64 k-steps and below the one-pass GEMM leads (48, 77 and
// 256 rows at 4096x4096, 77x4096x14336, 128x4096x10240).  Slices: s k-steps
// at about 0.28 us each on a 128 x 128 tile against s slices of 8 * mp * n
// bytes written and read back at about 3 TB/s, least at
// s = sqrt(steps * 105000 / (mp * n)) (measured best: 6-8, 6 and 4 slices at
// the three K = 10240 shapes).
constexpr int kMaxW8a8Splits = 8;

// HTP_OPS_AMD_W8A8_SPLITK (measurement hook): unset or -1 automatic, 0 off,
// 2..8 that many slices wherever 33-256 rows allow a split.
int w8a8_splitk_mode() {
  static const int mode = getenv("HTP_OPS_AMD_W8A8_SPLITK") ? atoi(getenv("HTP_OPS_AMD_W8A8_SPLITK")) : -1;
  return mode;
}

int w8a8_splits(int m, int kp, int n) {
  const long long tiles = (long long)((m + 127) / 128) * ((n + 127) / 128);
  const int mode = w8a8_splitk_mode(), steps = kp / kKStep;
  if (m < 33 || m > 256 || n % 16 || mode == 0) return 0;
  int splits;
  if (mode >= 2) {
    splits = mode;
  } else {
    if (2 * tiles >= compute_units() || !(steps >= 128 || (steps >= 80 && m > 128))) return 0;
    splits = (int)std::lround(std::sqrt((double)steps * 105000.0 / ((double)mp_of(m) * (double)n)));
  }
  splits = std::min(std::min(splits, kMaxW8a8Splits), steps);
  return splits >= 2 ? splits : 0;
}

size_t w8a8_linear_workspace(int m, int k, int n) {
  const size_t base = hb_w8a8_workspace_bytes(m, k);
  if (!base || n < 16) return base;
  return base + (w8a8_splits(m, (int)kp_of(k), n) ? (size_t)kMaxW8a8Splits * mp_of(m) * (size_t)n * 4u : 0);
}

template <int EPI>
int launch_w8a8_splitk(float *y, const int8_t *q, const float *scales, const void *packed, int m, int k, int n,
                       int splits, int32_t *part, hipStream_t st) {
  const uint8_t *base = (const uint8_t *)packed;
  const int8_t *wpack = (const int8_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WEIGHTS));
  const float *sw = (const float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_SW));
  const int32_t *delta = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_DELTA));
  const int kp = (int)kp_of(k), steps = kp / kKStep;
  const int kps = (steps + splits - 1) / splits, used = (steps + kps - 1) / kps;
  const int tiles = ((m + 127) / 128) * ((n + 127) / 128);
  hipLaunchKernelGGL((w8a8_splitk_partial<128, 128, 2, 2, 4>), dim3(tiles, used), dim3(256), 0, st, part, q, wpack, m,
                     n, kp, kps);
  int rc = hb_check_launch("w8a8_splitk_partial");
  if (rc) return rc;
  const size_t quads = (size_t)m * (size_t)(n / 4);
  const int grid = (int)std::min<size_t>((quads + 255) / 256, 65536);
  hipLaunchKernelGGL((w8a8_splitk_readout<EPI>), dim3(grid), dim3(256), 0, st, y, n, part, used, scales, sw, delta,
                     m, n);
  return hb_check_launch("w8a8_splitk_readout");
}

}  // namespace

extern "C" {

size_t hb_w8a8_linear_workspace_bytes(int m, int k, int n) { return w8a8_linear_workspace(m, k, n); }

int hb_w8a8_linear(float *d_y, const float *d_x, const void *d_packed, int m, int k, int n, int epilogue,
                   void *d_workspace, size_t workspace_bytes, hb_stream s) {
  if (!d_workspace || workspace_bytes < hb_w8a8_workspace_bytes(m, k))
    return hb_invalid("hb_w8a8_linear workspace too small");
  if (!d_packed) return hb_invalid("hb_w8a8_linear packed weights");
  if (!aligned(d_workspace, 256)) return hb_invalid("hb_w8a8_linear workspace alignment");
  int8_t *q = (int8_t *)d_workspace;
  float *scales = (float *)((uint8_t *)d_workspace + hb_round_up(mp_of(m) * kp_of(k), 256));
  const float *inv = (const float *)((const uint8_t *)d_packed + hb_w8a8_packed_offset(k, n, HB_W8A8_INV));
  // One row: quantization fused into the weight-streaming kernel.
  const int kp = (int)kp_of(k);
  if (m == 1 && kp <= 32 * 512 && k >= 32 && k % 32 == 0 && n >= 16 && n % 16 == 0 && d_y && d_x &&
      aligned(d_x, 16) && (epilogue == HB_W8A8_EPI_SCALE || epilogue == HB_W8A8_EPI_SCALE_GELU)) {
    if (!aligned(d_packed, 256)) return hb_invalid("hb_w8a8_linear alignment");
    const uint8_t *base = (const uint8_t *)d_packed;
    const int8_t *wpack = (const int8_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WEIGHTS));
    const float *sw = (const float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_SW));
    const int32_t *delta = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_DELTA));
    hipStream_t st = hb_resolve_stream(s);
    return epilogue == HB_W8A8_EPI_SCALE
               ? launch_decode_fused<HB_W8A8_EPI_SCALE>(d_y, d_x, inv, wpack, sw, delta, k, n, kp, st)
               : launch_decode_fused<HB_W8A8_EPI_SCALE_GELU>(d_y, d_x, inv, wpack, sw, delta, k, n, kp, st);
  }
  // Small problems: one launch that quantizes its own rows.  Every 16-row
  // tile streams the whole weight matrix, so the path is taken while the
  // weight bytes summed over row tiles stay within 16 MB (77x768x3072:
  // 8.0 -> 6.1 us; 64x1536x6144, 38 MB over its 4 row tiles, is faster as
  // quantize + GEMM: 9.5 against 16.0 us).  HTP_OPS_AMD_W8A8_SMALL=0 turns
  // the path off, for comparisons.
  static const int small_on = getenv("HTP_OPS_AMD_W8A8_SMALL") ? atoi(getenv("HTP_OPS_AMD_W8A8_SMALL")) : 1;
  if (small_on && m >= 5 && m <= 128 && kp <= 1536 && k >= 32 && k % 32 == 0 && n >= 16 && n % 16 == 0 &&
      (size_t)((m + 15) / 16) * (size_t)n * (size_t)kp <= ((size_t)16 << 20) && d_y && d_x && aligned(d_x, 16) &&
      aligned(d_y, 16) &&
      aligned(d_packed, 256) && (epilogue == HB_W8A8_EPI_SCALE || epilogue == HB_W8A8_EPI_SCALE_GELU)) {
    const uint8_t *base = (const uint8_t *)d_packed;
    const int8_t *wpack = (const int8_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WEIGHTS));
    const float *sw = (const float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_SW));
    const int32_t *delta = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_DELTA));
    hipStream_t st = hb_resolve_stream(s);
    return epilogue == HB_W8A8_EPI_SCALE
               ? launch_w8a8_small<HB_W8A8_EPI_SCALE>(d_y, d_x, inv, wpack, sw, delta, m, k, n, kp, st)
               : launch_w8a8_small<HB_W8A8_EPI_SCALE_GELU>(d_y, d_x, inv, wpack, sw, delta, m, k, n, kp, st);
  }
  // Two to four rows: quantization fused into the weight stream as well.
  const int nblocks = n / 16;
  if (m >= 2 && m <= 4 && kp <= 8 * 8 * kKStep && k >= 32 && k % 32 == 0 && n >= 16 && n % 16 == 0 && d_y && d_x &&
      aligned(d_x, 16) && aligned(d_packed, 256) && (size_t)nblocks * (size_t)kp * 16u < ((size_t)1 << 32) &&
      (epilogue == HB_W8A8_EPI_SCALE || epilogue == HB_W8A8_EPI_SCALE_GELU)) {
    const uint8_t *base = (const uint8_t *)d_packed;
    const int8_t *wpack = (const int8_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WEIGHTS));
    const float *sw = (const float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_SW));
    const int32_t *delta = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_DELTA));
    hipStream_t st = hb_resolve_stream(s);
    const dim3 grid((nblocks + 1) / 2), block(1024);
    if (m == 2) {
      if (epilogue == HB_W8A8_EPI_SCALE)
        hipLaunchKernelGGL((w8a8_decode_rows<2, HB_W8A8_EPI_SCALE>), grid, block, 0, st, d_y, n, d_x, inv, wpack, sw,
                           delta, m, k, kp, nblocks);
      else
        hipLaunchKernelGGL((w8a8_decode_rows<2, HB_W8A8_EPI_SCALE_GELU>), grid, block, 0, st, d_y, n, d_x, inv,
                           wpack, sw, delta, m, k, kp, nblocks);
    } else {
      if (epilogue == HB_W8A8_EPI_SCALE)
        hipLaunchKernelGGL((w8a8_decode_rows<4, HB_W8A8_EPI_SCALE>), grid, block, 0, st, d_y, n, d_x, inv, wpack, sw,
                           delta, m, k, kp, nblocks);
      else
        hipLaunchKernelGGL((w8a8_decode_rows<4, HB_W8A8_EPI_SCALE_GELU>), grid, block, 0, st, d_y, n, d_x, inv,
                           wpack, sw, delta, m, k, kp, nblocks);
    }
    return hb_check_launch("w8a8_decode_rows");
  }
  int rc = hb_w8a8_quantize(q, scales, d_x, inv, m, k, s);
  if (rc) return rc;
  // 33-256 rows with few tiles: K split over the workspace's int32 slices,
  // when the caller's workspace holds them (hb_w8a8_linear_workspace_bytes)
  if (const int splits = w8a8_splits(m, kp, n)) {
    if (workspace_bytes >= w8a8_linear_workspace(m, k, n) && d_y && aligned(d_y, 16) && aligned(d_packed, 256) &&
        (epilogue == HB_W8A8_EPI_SCALE || epilogue == HB_W8A8_EPI_SCALE_GELU) &&
        (size_t)(n / 16) * (size_t)kp * 16u < ((size_t)1 << 32)) {
      int32_t *part = (int32_t *)((uint8_t *)d_workspace + hb_w8a8_workspace_bytes(m, k));
      hipStream_t st = hb_resolve_stream(s);
      return epilogue == HB_W8A8_EPI_SCALE
                 ? launch_w8a8_splitk<HB_W8A8_EPI_SCALE>(d_y, q, scales, d_packed, m, k, n, splits, part, st)
                 : launch_w8a8_splitk<HB_W8A8_EPI_SCALE_GELU>(d_y, q, scales, d_packed, m, k, n, splits, part, st);
    }
  }
  return hb_w8a8_gemm(d_y, n, q, scales, d_packed, m, k, n, epilogue, s);
}

// ---- no-allocation variant of hb_w8a8_linear ------------------------------------
// Its workspace is this file-scope device array (one copy per GPU, held until
// the process ends).  In host code the name `scratch` only stands in for the
// symbol: its device address on the current GPU comes from
// hipGetSymbolAddress, taken once per device (hb_init calls
// hb_w8a8_static_setup) and used wherever host code passes the memory on.

}  // extern "C"

namespace {
static __device__ __align__(256) uint8_t scratch[HB_W8A8_STATIC_SCRATCH_BYTES];
constexpr int kMaxStaticDevices = 16;
std::atomic<void *> g_scratch_ptr[kMaxStaticDevices];
}  // namespace

extern "C" {

int hb_w8a8_static_setup(int device) {
  if (device < 0 || device >= kMaxStaticDevices) return hb_invalid("hb_w8a8_static_setup device");
  if (g_scratch_ptr[device].load(std::memory_order_acquire) != nullptr) return HB_OK;
  int cur = -1;
  hipError_t err = hipGetDevice(&cur);
  if (err != hipSuccess) return hb_fail(err, "hipGetDevice");
  if (cur != device) return hb_invalid("hb_w8a8_static_setup: device is not current");
  void *ptr = nullptr;
  err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (err != hipSuccess) return hb_fail(err, "hipGetSymbolAddress(scratch)");
  if (ptr == nullptr || ((uintptr_t)ptr % 256) != 0) return hb_invalid("hb_w8a8_static_setup: scratch address");
  g_scratch_ptr[device].store(ptr, std::memory_order_release);
  return HB_OK;
}

int hb_w8a8_linear_noalloc(float *d_y, const float *d_x, const void *d_packed, int m, int k, int n, int epilogue,
                           hb_stream s) {
  if (m < 1 || k < 32 || k % 32) return hb_invalid("hb_w8a8_linear_noalloc shape");
  const size_t need = hb_w8a8_workspace_bytes(m, k);
  if (need > (size_t)HB_W8A8_STATIC_SCRATCH_BYTES)
    return hb_invalid("hb_w8a8_linear_noalloc: m x k needs more than the 32 MiB static workspace");
  int dev = -1;
  const hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hb_fail(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxStaticDevices) return hb_invalid("hb_w8a8_linear_noalloc device");
  void *ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {  // first call on a device that hb_init did not set up
    const int rc = hb_w8a8_static_setup(dev);
    if (rc != HB_OK) return rc;
    ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  }
  return hb_w8a8_linear(d_y, d_x, d_packed, m, k, n, epilogue, ptr, HB_W8A8_STATIC_SCRATCH_BYTES, s);
}

int hb_w8a8_force_tile(int index) {
  if (index < -1 || index > kStreamWideShape) return hb_invalid("hb_w8a8_force_tile index");
  forced_tile_shape();  // settle the environment default first
  return g_forced_tile.exchange(index);
}

int hb_w8a8_readout(float *d_y, int ldy, const int32_t *d_raw, const float *d_scales, const void *d_packed, int m,
                    int k, int n, int epilogue, hb_stream s) {
  if (!d_y || !d_raw || !d_scales || !d_packed) return hb_invalid("hb_w8a8_readout null pointer");
  if (m < 1 || k < 32 || k % 32 || n < 16 || n % 16 || ldy < n || ldy % 4) return hb_invalid("hb_w8a8_readout shape");
  if ((uintptr_t)d_y % 16 || (uintptr_t)d_raw % 16) return hb_invalid("hb_w8a8_readout alignment");
  const uint8_t *base = (const uint8_t *)d_packed;
  const float *sw = (const float *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_SW));
  const int32_t *delta = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_DELTA));
  const int32_t *wsum = (const int32_t *)(base + hb_w8a8_packed_offset(k, n, HB_W8A8_WSUM128));
  const size_t quads = (size_t)m * (size_t)(n / 4);
  const int grid = (int)std::min<size_t>((quads + 255) / 256, 65536);
  hipStream_t st = hb_resolve_stream(s);
  if (epilogue == HB_W8A8_EPI_SCALE)
    hipLaunchKernelGGL((w8a8_readout<HB_W8A8_EPI_SCALE>), dim3(grid), dim3(256), 0, st, d_y, ldy, d_raw, d_scales, sw,
                       delta, wsum, m, n);
  else if (epilogue == HB_W8A8_EPI_SCALE_GELU)
    hipLaunchKernelGGL((w8a8_readout<HB_W8A8_EPI_SCALE_GELU>), dim3(grid), dim3(256), 0, st, d_y, ldy, d_raw,
                       d_scales, sw, delta, wsum, m, n);
  else
    return hb_invalid("hb_w8a8_readout epilogue");
  return hb_check_launch("w8a8_readout");
}

int hb_w8a8_planes_from_raw(uint8_t *d_out, const int32_t *d_raw, int m, int n, hb_stream s) {
  if (!d_out || !d_raw) return hb_invalid("hb_w8a8_planes_from_raw null pointer");
  if (m < 1 || n < 32 || n % 32) return hb_invalid("hb_w8a8_planes_from_raw shape");
  const size_t total = (size_t)m * n * 4u;
  const int grid = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  hipLaunchKernelGGL(w8a8_planes, dim3(grid), dim3(256), 0, hb_resolve_stream(s), d_out, d_raw, m, n);
  return hb_check_launch("w8a8_planes");
}

}  // extern "C"
